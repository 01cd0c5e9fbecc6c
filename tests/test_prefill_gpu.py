"""Batched prefill on the GPU against the token-by-token path it replaces.

The reference feeds a prompt one decode step per token (feedToken, src/FullModel.cpp:1096-1108,
1162-1170), so the oracle for a prompt is the oracle's decode step run at each of its positions,
and for each prefill kernel the oracle's per-token op at each row: GEMV (MatVec.cpp:52-60, f64
accumulation), rms_norm (RmsNorm.cpp:194-216), rope_neox (Rope.cpp:48-51,191-203), swiglu
(Swiglu.cpp:56) and the cache attention (Attention.cpp:253-294).

Tolerances, mixed form |a - e| <= tol * (1 + |e|): the decode bar (GEMV, swiglu, rope 1e-3;
rms_norm 1e-5; logits 1e-3; greedy ids identical) and, for the split products, a bound 50x
tighter than what f16-rounded activations alone reach, which fails if the lo plane is dropped.
Split planes and cache rows are checked bit-for-bit where f16 rounding fixes them.
"""
import ctypes
import math

import numpy as np
import pytest

from conftest import close, worst

pytestmark = pytest.mark.gpu

_libm = ctypes.CDLL("libm.so.6")
_libm.powf.restype = ctypes.c_float
_libm.powf.argtypes = [ctypes.c_float, ctypes.c_float]


def dev(torch, array):
    return torch.from_numpy(np.ascontiguousarray(array)).cuda()


def host(t):
    return t.detach().cpu().numpy()


def stream(torch):
    return torch.cuda.current_stream().cuda_stream


def run(mh, torch, status):
    mh.check(status)
    torch.cuda.synchronize()


def planes(torch, shape):
    return (torch.zeros(shape, dtype=torch.int16, device="cuda"), torch.zeros(shape, dtype=torch.int16, device="cuda"))


def joined(hi, lo):
    """hi + lo as f64 from two uint16 planes (device tensors)."""
    h = host(hi).view(np.uint16).view(np.float16).astype(np.float64)
    l = host(lo).view(np.uint16).view(np.float16).astype(np.float64)
    return h + l


def split_np(x):
    """The split the kernels make: hi = x with its 13 low mantissa bits cleared (exact in f16 in
    f16's normal range), lo = f16(x - hi) rounded to nearest even."""
    x = np.ascontiguousarray(x, np.float32)
    hi32 = (x.view(np.uint32) & np.uint32(0xFFFFE000)).view(np.float32)
    return hi32.astype(np.float16).view(np.uint16), (x - hi32).astype(np.float16).view(np.uint16)


def rope_pow(theta_scale, head_dim):
    """theta_scale^j with the C library's powf, as the decoder computes its table."""
    return np.array([_libm.powf(theta_scale, float(j)) for j in range(head_dim // 2)], np.float32)


# ------------------------------------------------------------------------------------------------
# Split planes


def test_split_planes_are_f16_and_remainder(mh, gpu):
    torch = gpu
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.normal(0, 1, 4000), rng.normal(0, 300, 4000), [0.0, -0.0, 1e-8, 65000.0, -3.1415927]])
    x = np.resize(x.astype(np.float32), 8012)
    hi, lo = planes(torch, x.shape)
    xd = dev(torch, x)
    run(mh, torch, mh.load().muyo_split_f32_f16x2(xd.data_ptr(), x.size, hi.data_ptr(), lo.data_ptr(), stream(torch)))
    want_hi, want_lo = split_np(x)
    normal = np.abs(x) >= 2.0 ** -14  # below, hi itself is an f16 subnormal and rounds
    assert np.array_equal(host(hi).view(np.uint16)[normal], want_hi[normal])
    assert np.array_equal(host(lo).view(np.uint16)[normal], want_lo[normal])
    # hi + lo holds x to 2^-21 of its magnitude (f16 subnormals aside).
    err = np.abs(joined(hi, lo) - x.astype(np.float64))
    assert np.all(err <= np.abs(x) * 2.0 ** -21 + 2.0 ** -24)


def test_rms_norm_split_matches_oracle(mh, gpu, orc):
    torch = gpu
    for rows, cols, seed in ((1, 896, 3), (37, 896, 4), (5, 3584, 5), (9, 200, 6)):
        x = orc.normal_f32(rows * cols, seed).reshape(rows, cols) * 3
        w = orc.normal_f32(cols, seed + 100, 1.0, 0.1)
        hi, lo = planes(torch, (rows, cols))
        xd, wd = dev(torch, x), dev(torch, w)
        run(mh, torch, mh.load().muyo_rms_norm_split_f16x2(xd.data_ptr(), wd.data_ptr(), rows, cols, 1e-6,
                                                           hi.data_ptr(), lo.data_ptr(), stream(torch)))
        want = orc.rms_norm(x, w, 1e-6)
        assert close(joined(hi, lo), want, 1e-5) == 0, (rows, cols)
        assert worst(joined(hi, lo), want) < 1e-6


# ------------------------------------------------------------------------------------------------
# GEMMs

GEMM_SHAPES = [
    (1, 8, 8),          # one token, one 16-byte chunk of K
    (37, 100, 72),      # ragged rows, n not a multiple of 32, k not of 64
    (128, 128, 64),     # exactly one 128 x 128 tile
    (200, 1152, 896),   # 0.5B QKV
    (300, 896, 896),    # 0.5B o_proj
    (67, 896, 4864),    # 0.5B down: long K
    (640, 1152, 896),   # 45 tiles of 128 x 128: the 64-token tiles
]


def oracle_gemm(orc, w_bits, a):
    """Each row through the oracle's GEMV (f64 accumulation), as the token-by-token feed does."""
    return np.stack([orc.mat_vec_f16(w_bits, row, f64acc=True) for row in a])


@pytest.mark.parametrize("rows,n,k", GEMM_SHAPES)
def test_gemm_split_matches_per_token_gemv(mh, gpu, orc, rows, n, k):
    torch = gpu
    seed = rows * 7 + n * 3 + k
    a = orc.normal_f32(rows * k, seed).reshape(rows, k)
    w = orc.normal_f16(n * k, seed + 1, 0.0, 0.02).reshape(n, k)
    bias = orc.normal_f32(n, seed + 2, 0.0, 0.02)
    residual = orc.normal_f32(rows * n, seed + 3).reshape(rows, n)
    ahi, alo = split_np(a)
    out = torch.zeros((rows, n), dtype=torch.float32, device="cuda")
    lib = mh.load()
    keep = [dev(torch, ahi), dev(torch, alo), dev(torch, w), dev(torch, bias), dev(torch, residual)]
    args = tuple(t.data_ptr() for t in keep[:3])
    run(mh, torch, lib.muyo_gemm_split_f16(*args, keep[3].data_ptr(), None, out.data_ptr(), rows, n, k,
                                           stream(torch)))
    plain = oracle_gemm(orc, w, a)
    got = host(out)
    want = plain + bias
    assert close(got, want, 1e-3) == 0
    # Split precision: f16-rounded activations alone miss by ~1e-3 relative; the planes must do
    # 50x better than that.
    f16_only = oracle_gemm(orc, w, a.astype(np.float16).astype(np.float32)) + bias
    assert worst(got, want) * 50 < max(worst(f16_only, want), 1e-5) or worst(got, want) < 2e-7
    run(mh, torch, lib.muyo_gemm_split_f16(*args, None, keep[4].data_ptr(), out.data_ptr(), rows, n, k,
                                           stream(torch)))
    assert close(host(out), plain + residual, 1e-5) == 0


def test_gemm_split_integer_inputs_are_exact(mh, gpu):
    """Small integers are exact in f16 and their sums in f32: any index or layout slip shows."""
    torch = gpu
    rng = np.random.default_rng(9)
    rows, n, k = 150, 260, 136
    a = rng.integers(-8, 9, (rows, k)).astype(np.float32)
    w = rng.integers(-8, 9, (n, k)).astype(np.float16)
    ahi, alo = split_np(a)
    assert not alo.any()
    out = torch.zeros((rows, n), dtype=torch.float32, device="cuda")
    keep = [dev(torch, ahi), dev(torch, alo), dev(torch, w.view(np.uint16))]
    run(mh, torch, mh.load().muyo_gemm_split_f16(*(t.data_ptr() for t in keep), None, None, out.data_ptr(),
                                                 rows, n, k, stream(torch)))
    assert np.array_equal(host(out), a.astype(np.float64) @ w.astype(np.float64).T)


@pytest.mark.parametrize("rows,n,k", [(1990, 4600, 136), (1990, 16300, 72)])
def test_gemm_split_large_grids_integer_exact(mh, gpu, rows, n, k):
    """Integer inputs on the 128 x 128 and 128 x 256 tile kernels (576 and 1040 tiles, the second
    with token tiles fastest): a last token tile of 70 rows, a last weight tile of 120 or 172
    rows and a K tail inside the last K tile, whose lanes past the matrix read in-bounds rows."""
    torch = gpu
    rng = np.random.default_rng(rows + n + k)
    a = rng.integers(-8, 9, (rows, k)).astype(np.float32)
    w = rng.integers(-8, 9, (n, k)).astype(np.float16)
    ahi, alo = split_np(a)
    out = torch.zeros((rows, n), dtype=torch.float32, device="cuda")
    keep = [dev(torch, ahi), dev(torch, alo), dev(torch, w.view(np.uint16))]
    run(mh, torch, mh.load().muyo_gemm_split_f16(*(t.data_ptr() for t in keep), None, None, out.data_ptr(),
                                                 rows, n, k, stream(torch)))
    assert np.array_equal(host(out), a.astype(np.float64) @ w.astype(np.float64).T)


def test_gemm_swiglu_wide_tiles_integer_products(mh, gpu):
    """The 128 x 256 swiglu tiles (1040 of them) on integer inputs: both products exact, the
    swiglu of them to the planes' precision; ragged token and ffn tiles and a K tail."""
    torch = gpu
    rows, ffn, k = 1990, 8200, 40
    rng = np.random.default_rng(77)
    a = rng.integers(-2, 3, (rows, k)).astype(np.float32)
    wg = rng.integers(-2, 3, (ffn, k)).astype(np.float16)
    wu = rng.integers(-2, 3, (ffn, k)).astype(np.float16)
    ahi, alo = split_np(a)
    hhi, hlo = planes(torch, (rows, ffn))
    keep = [dev(torch, ahi), dev(torch, alo), dev(torch, wg.view(np.uint16)), dev(torch, wu.view(np.uint16))]
    run(mh, torch, mh.load().muyo_gemm_swiglu_split_f16(*(t.data_ptr() for t in keep), hhi.data_ptr(),
                                                        hlo.data_ptr(), rows, ffn, k, stream(torch)))
    g = a.astype(np.float64) @ wg.astype(np.float64).T
    u = a.astype(np.float64) @ wu.astype(np.float64).T
    want = g / (1.0 + np.exp(-g)) * u
    got = joined(hhi, hlo)
    assert np.abs(got - want).max() <= 1e-5 * (1.0 + np.abs(want)).max()


@pytest.mark.parametrize("rows,ffn,k", [(1, 8, 8), (45, 100, 72), (200, 4864, 896), (700, 4864, 896)])
def test_gemm_swiglu_matches_per_token_path(mh, gpu, orc, rows, ffn, k):
    torch = gpu
    seed = rows + ffn + k
    a = orc.normal_f32(rows * k, seed).reshape(rows, k)
    wg = orc.normal_f16(ffn * k, seed + 1, 0.0, 0.05).reshape(ffn, k)
    wu = orc.normal_f16(ffn * k, seed + 2, 0.0, 0.05).reshape(ffn, k)
    ahi, alo = split_np(a)
    hhi, hlo = planes(torch, (rows, ffn))
    keep = [dev(torch, ahi), dev(torch, alo), dev(torch, wg), dev(torch, wu)]
    run(mh, torch, mh.load().muyo_gemm_swiglu_split_f16(*(t.data_ptr() for t in keep), hhi.data_ptr(),
                                                        hlo.data_ptr(), rows, ffn, k, stream(torch)))
    want = orc.swiglu(oracle_gemm(orc, wg, a), oracle_gemm(orc, wu, a))
    got = joined(hhi, hlo)
    assert close(got, want, 1e-3) == 0
    assert worst(got, want) < 2e-5


def test_gemm_refusals(mh, gpu):
    lib = mh.load()
    fake = ctypes.c_void_p(256)
    assert lib.muyo_gemm_split_f16(None, fake, fake, None, None, fake, 1, 8, 8, 0) == mh.MUYO_E_NULL
    assert lib.muyo_gemm_split_f16(fake, fake, fake, None, None, fake, 1, 6, 8, 0) == mh.MUYO_E_CONTRACT
    assert lib.muyo_gemm_split_f16(fake, fake, fake, None, None, fake, 1, 8, 12, 0) == mh.MUYO_E_CONTRACT
    assert lib.muyo_gemm_split_f16(fake, fake, ctypes.c_void_p(258), None, None, fake, 1, 8, 8, 0) == mh.MUYO_E_CONTRACT
    assert lib.muyo_gemm_swiglu_split_f16(fake, fake, fake, fake, fake, fake, 0, 8, 8, 0) == mh.MUYO_E_CONTRACT


# ------------------------------------------------------------------------------------------------
# Rope + cache append, attention


@pytest.mark.parametrize("heads,kv_heads,head_dim,rows,pos0", [(14, 2, 64, 45, 0), (28, 4, 128, 33, 1990),
                                                                (4, 1, 64, 1, 7)])
def test_rope_split_append_matches_oracle(mh, gpu, orc, heads, kv_heads, head_dim, rows, pos0):
    torch = gpu
    max_seq = 2048
    width = (heads + 2 * kv_heads) * head_dim
    qkv = orc.normal_f32(rows * width, heads + rows).reshape(rows, width)
    theta_scale = np.float32(_libm.powf(np.float32(1e6), np.float32(-2.0 / head_dim)))
    table = dev(torch, rope_pow(theta_scale, head_dim))
    qhi, qlo = planes(torch, (rows, heads * head_dim))
    kc = torch.zeros((kv_heads, max_seq, head_dim), dtype=torch.int16, device="cuda")
    vc = torch.zeros_like(kc)
    qkv_d = dev(torch, qkv)
    run(mh, torch, mh.load().muyo_rope_split_append_f16kv(qkv_d.data_ptr(), rows, pos0, heads, kv_heads,
                                                          head_dim, max_seq, table.data_ptr(), qhi.data_ptr(),
                                                          qlo.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                                                          stream(torch)))
    qdim, kvdim = heads * head_dim, kv_heads * head_dim
    want_k = np.zeros((kv_heads, max_seq, head_dim), np.uint16)
    want_v = np.zeros_like(want_k)
    for m in range(rows):
        q = orc.rope_neox(qkv[m, :qdim].reshape(heads, head_dim), pos0 + m, float(theta_scale)).reshape(-1)
        assert close(joined(qhi[m], qlo[m]), q, 1e-3) == 0
        assert worst(joined(qhi[m], qlo[m]), q) < 1e-6, m
        k = orc.rope_neox(qkv[m, qdim:qdim + kvdim].reshape(kv_heads, head_dim), pos0 + m, float(theta_scale))
        want_k[:, pos0 + m] = orc.float_to_half(k)
        want_v[:, pos0 + m] = orc.float_to_half(qkv[m, qdim + kvdim:].reshape(kv_heads, head_dim))
    got_k = host(kc).view(np.uint16)
    # The cache rows outside pos0..pos0+rows stay untouched; inside, k is the f16 of the oracle's
    # f32 rope (last-bit rounding aside) and v is bit-exact.
    assert np.array_equal(host(vc).view(np.uint16), want_v)
    assert not got_k[:, :pos0].any() and not got_k[:, pos0 + rows:].any()
    want_f = orc.half_to_float(want_k)
    assert np.all(np.abs(orc.half_to_float(got_k) - want_f) <= np.abs(want_f) * 2.0 ** -10 + 2.0 ** -24)  # 1 ulp


def prefill_attention_case(mh, torch, orc, heads, kv_heads, head_dim, rows, pos0, max_seq, seed, check=None,
                           poison=False, split=False):
    q = orc.normal_f32(rows * heads * head_dim, seed).reshape(rows, heads * head_dim)
    kc = orc.normal_f16(kv_heads * max_seq * head_dim, seed + 1).reshape(kv_heads, max_seq, head_dim)
    vc = orc.normal_f16(kv_heads * max_seq * head_dim, seed + 2).reshape(kv_heads, max_seq, head_dim)
    if poison:
        # Cache rows past the last query's position hold NaN and infinity (fp16 bit patterns).
        last = pos0 + rows - 1
        kc[:, last + 1:] = 0x7E00
        vc[:, last + 1:, ::2] = 0x7C00
        vc[:, last + 1:, 1::2] = 0x7E00
    qhi, qlo = split_np(q)
    ohi, olo = planes(torch, (rows, heads * head_dim))
    scale = 1.0 / math.sqrt(head_dim)
    keep = [dev(torch, qhi), dev(torch, qlo), dev(torch, kc), dev(torch, vc)]
    lib = mh.load()
    if split:
        # The workspace starts as NaN: the merge must read only slots the chunks wrote.
        size = lib.muyo_prefill_attention_workspace_bytes(rows, heads, head_dim)
        ws = torch.full((size // 4,), float("nan"), dtype=torch.float32, device="cuda")
        run(mh, torch, lib.muyo_prefill_attention_f16kv_ws(*(t.data_ptr() for t in keep), ohi.data_ptr(),
                                                           olo.data_ptr(), rows, pos0, heads, kv_heads, head_dim,
                                                           max_seq, scale, ws.data_ptr(), size, stream(torch)))
    else:
        run(mh, torch, lib.muyo_prefill_attention_f16kv(*(t.data_ptr() for t in keep), ohi.data_ptr(),
                                                        olo.data_ptr(), rows, pos0, heads, kv_heads, head_dim,
                                                        max_seq, scale, stream(torch)))
    got = joined(ohi, olo)
    assert np.isfinite(got).all()
    for m in (range(rows) if check is None else check):
        want = orc.attention_f16kv(q[m], kc, vc, heads, kv_heads, head_dim, max_seq, pos0 + m, scale)
        assert close(got[m], want, 1e-3) == 0, m
        assert worst(got[m], want) < 2e-5, (m, worst(got[m], want))


@pytest.mark.parametrize("heads,kv_heads,head_dim,rows,pos0,max_seq", [
    (14, 2, 64, 1, 0, 64),        # one query at row 0: a single key
    (14, 2, 64, 70, 0, 128),      # three query tiles, ragged
    (14, 2, 64, 40, 1000, 2048),  # after an earlier prompt
    (28, 4, 128, 33, 2015, 2048), # 7B heads, ending at the last cache row
    (8, 1, 128, 64, 5, 100),      # a full group of 8, cache not a multiple of 32 keys
    (4, 4, 64, 31, 17, 48),       # no grouping
])
def test_prefill_attention_matches_per_token_attention(mh, gpu, orc, heads, kv_heads, head_dim, rows, pos0, max_seq):
    prefill_attention_case(mh, gpu, orc, heads, kv_heads, head_dim, rows, pos0, max_seq, heads + rows + pos0)


@pytest.mark.parametrize("heads,kv_heads,head_dim", [(14, 2, 64), (28, 4, 128)])
def test_prefill_attention_full_prompt(mh, gpu, orc, heads, kv_heads, head_dim):
    """2048 queries: the 0.5B shape's groups of 7 split over two workgroups per tile, the 7B shape's
    whole groups (its grid alone fills the chip); rows checked at tile edges and spread over the
    prompt."""
    rows = 2048
    check = [0, 1, 31, 32, 33, 500, 1023, 1024, 1537, 2015, 2016, 2046, 2047]
    prefill_attention_case(mh, gpu, orc, heads, kv_heads, head_dim, rows, 0, rows, 7 + heads, check)


@pytest.mark.parametrize("heads,kv_heads,head_dim,rows,pos0,max_seq", [
    (14, 2, 64, 5, 0, 64),        # one tile, keys 5..31 of it past the last query
    (14, 2, 64, 33, 30, 128),     # tiles 0..1, the last one mostly past the prompt
    (28, 4, 128, 40, 1000, 2048), # 7B heads after an earlier prompt
])
def test_prefill_attention_ignores_rows_past_the_prompt(mh, gpu, orc, heads, kv_heads, head_dim, rows, pos0,
                                                        max_seq):
    """The last key tile covers cache rows past the prompt's last position; NaN and infinity there
    must not reach any query's output (a weight of 0 times NaN is NaN)."""
    prefill_attention_case(mh, gpu, orc, heads, kv_heads, head_dim, rows, pos0, max_seq, 3 + rows, poison=True)


@pytest.mark.parametrize("heads,kv_heads,head_dim,rows,pos0,max_seq,check", [
    (14, 2, 64, 512, 0, 512, None),         # last tile exactly 16 key tiles: nothing split
    (14, 2, 64, 513, 0, 544, None),         # one query past it: a 16 + 1 split of the last tile
    (14, 2, 64, 600, 0, 640, None),         # tiles 16..18 in two chunks
    (14, 2, 64, 40, 1000, 2048, None),      # after an earlier prompt: every tile split in three
    (28, 4, 128, 33, 2015, 2048, None),     # 7B heads, ending at the last cache row: four chunks
    (8, 1, 128, 64, 1100, 1200, None),      # a full group of 8 over a ragged cache
    (4, 4, 64, 96, 8000, 8192, range(0, 96, 5)),  # 251+ key tiles: chunks of 32 key tiles, eight per tile
    (14, 2, 64, 2048, 0, 2048, [0, 31, 511, 512, 543, 544, 1000, 1535, 1536, 2046, 2047]),
    (28, 4, 128, 2048, 0, 2048, [0, 33, 512, 1023, 1024, 1500, 2015, 2016, 2047]),
    (14, 2, 64, 2100, 0, 2112, [0, 2047, 2048, 2099]),  # past the decoder's 2048-row passes: 170 items
    (14, 2, 64, 4160, 0, 4160, [0, 2047, 3000, 4159]),  # its chunks would be 564 work items: runs unsplit
])
def test_prefill_attention_key_chunks_match_per_token_attention(mh, gpu, orc, heads, kv_heads, head_dim, rows, pos0,
                                                               max_seq, check):
    """Query tiles split into key chunks, combined by the merge kernel, against the oracle's
    attention of each query."""
    prefill_attention_case(mh, gpu, orc, heads, kv_heads, head_dim, rows, pos0, max_seq, 11 + rows + pos0, check,
                           split=True)


@pytest.mark.parametrize("heads,kv_heads,head_dim,rows,pos0,max_seq", [
    (14, 2, 64, 600, 30, 1024),     # the split tiles' last key tile mostly past the prompt
    (28, 4, 128, 40, 1000, 2048),
])
def test_prefill_attention_key_chunks_ignore_rows_past_the_prompt(mh, gpu, orc, heads, kv_heads, head_dim, rows,
                                                                  pos0, max_seq):
    prefill_attention_case(mh, gpu, orc, heads, kv_heads, head_dim, rows, pos0, max_seq, 5 + rows, poison=True,
                           split=True)


def test_prefill_attention_refusals(mh, gpu):
    lib = mh.load()
    fake = ctypes.c_void_p(256)
    args = [fake] * 6
    assert lib.muyo_prefill_attention_f16kv(*args, 4, 0, 14, 2, 96, 64, 0.1, 0) == mh.MUYO_E_UNSUPPORTED
    assert lib.muyo_prefill_attention_f16kv(*args, 4, 0, 18, 2, 64, 64, 0.1, 0) == mh.MUYO_E_UNSUPPORTED
    assert lib.muyo_prefill_attention_f16kv(*args, 4, 62, 14, 2, 64, 64, 0.1, 0) == mh.MUYO_E_RANGE
    assert lib.muyo_prefill_attention_f16kv(*args, 4, -1, 14, 2, 64, 64, 0.1, 0) == mh.MUYO_E_RANGE


# ------------------------------------------------------------------------------------------------
# The decoder's prefill

SMALL = dict(layers=2, hidden=256, ffn=512, heads=4, kv_heads=2, head_dim=64, vocab=1000, max_seq=256)


def make_pair(mh, orc, shape, seed, kv_positions=0, kv_seed=7):
    dec = mh.Decoder(mh.qwen2_config(**shape))
    dec.fill_random(seed)
    model = orc.Model(**shape)
    model.fill_random(seed)
    if kv_positions:
        dec.fill_kv_random(kv_positions, kv_seed)
        model.fill_kv_random(kv_positions, kv_seed)
    return dec, model


def download(dec, kind, layer, like):
    out = np.empty_like(like)
    dec.download(kind, layer, out)
    return out


def prompt(orc, count, vocab, seed):
    return (orc.uniform_f32(count, seed) * 0.5 * vocab + 0.5 * vocab).astype(np.int32)


def check_against_oracle(dec, model, orc, shape, tokens, pos0):
    got = dec.prefill(tokens, pos0)
    for i, t in enumerate(tokens):
        want, logits, (top1, top2) = model.step(int(t), pos0 + i)
    gpu_logits = download(dec, "LOGITS", 0, np.empty(shape["vocab"], np.float32))
    assert close(gpu_logits, logits, 1e-3) == 0
    assert got == want, f"prefill {got} oracle {want} (margin {top1 - top2:.3g})"
    end = pos0 + len(tokens)
    for layer in range(shape["layers"]):
        for kind in ("KCACHE", "VCACHE"):
            ref = model.t[(kind, layer)]
            cache = download(dec, kind, layer, ref)
            assert np.array_equal(cache[:, :pos0], ref[:, :pos0])
            assert np.array_equal(cache[:, end:], ref[:, end:])
            diff = np.abs(orc.half_to_float(cache[:, pos0:end]) - orc.half_to_float(ref[:, pos0:end]))
            assert diff.max() <= 2e-3 * (1 + np.abs(orc.half_to_float(ref[:, pos0:end])).max()), (kind, layer)
    return got


def test_decoder_prefill_small_matches_oracle_steps(mh, gpu, orc):
    dec, model = make_pair(mh, orc, SMALL, seed=41, kv_positions=30, kv_seed=42)
    with dec:
        tokens = prompt(orc, 40, SMALL["vocab"], 43)
        nxt = check_against_oracle(dec, model, orc, SMALL, tokens, 30)
        # Generation continues from the prefilled cache as after 40 steps.
        ids = dec.generate(nxt, 70, 12)
    want, _ = model.greedy(nxt, 70, 12)
    assert ids == want


ODD = {
    "group8_hd128": dict(layers=1, hidden=512, ffn=1000, heads=8, kv_heads=1, head_dim=128, vocab=500, max_seq=300),
    "qdim1280_hd64": dict(layers=2, hidden=640, ffn=1792, heads=20, kv_heads=4, head_dim=64, vocab=700, max_seq=333),
}


@pytest.mark.parametrize("name", sorted(ODD))
def test_decoder_prefill_odd_shapes(mh, gpu, orc, name):
    shape = ODD[name]
    dec, model = make_pair(mh, orc, shape, seed=51)
    with dec:
        check_against_oracle(dec, model, orc, shape, prompt(orc, shape["max_seq"] - 5, shape["vocab"], 52), 0)


def test_decoder_prefill_after_long_cache(mh, gpu, orc):
    """A 100-token prompt appended at cache row 15000 of 16384 (o_proj per kv group at head_dim
    128): each query tile's 470-472 key tiles split into eight chunks and merged."""
    shape = dict(layers=1, hidden=512, ffn=512, heads=12, kv_heads=4, head_dim=128, vocab=300, max_seq=16384)
    dec, model = make_pair(mh, orc, shape, seed=53, kv_positions=15000, kv_seed=54)
    with dec:
        check_against_oracle(dec, model, orc, shape, prompt(orc, 100, shape["vocab"], 55), 15000)


def test_decoder_prefill_05b_prompt_then_greedy(mh, gpu, orc, capsys):
    """Qwen2.5-0.5B shape: a 96-token prompt from row 0, then 16 greedy tokens, against the oracle
    fed token by token."""
    orc.set_threads(16)
    shape = mh.QWEN25_05B
    dec, model = make_pair(mh, orc, shape, seed=2026)
    tokens = prompt(orc, 96, shape["vocab"], 2028)
    with dec:
        nxt = dec.prefill(tokens, 0)
        ids = dec.generate(nxt, 96, 16)
    margins = []
    for i, t in enumerate(tokens):
        want, _, (top1, top2) = model.step(int(t), i)
        margins.append(top1 - top2)
    rest, more = model.greedy(want, 96, 16)
    with capsys.disabled():
        print(f"\n[0.5b prefill 96] next {nxt} ids {ids[:6]}... min margin {min(margins + more):.3g}")
    assert nxt == want
    assert ids == rest


def test_decoder_prefill_equals_steps_on_gpu(mh, gpu, orc):
    """Prefill vs the decoder's own steps on the 0.5B shape after a 500-row cache: same logits,
    same cache rows, same continuation."""
    shape = mh.QWEN25_05B
    tokens = prompt(orc, 300, shape["vocab"], 61)
    with mh.Decoder(mh.qwen2_config(**shape)) as dec:
        dec.fill_random(60)
        dec.fill_kv_random(500, 62)
        nxt = dec.prefill(tokens, 500)
        logits_p = download(dec, "LOGITS", 0, np.empty(shape["vocab"], np.float32))
        cache_p = download(dec, "KCACHE", 23, np.empty((2, 2048, 64), np.uint16))
        ids_p = dec.generate(nxt, 800, 8)
        dec.fill_kv_random(500, 62)
        for i, t in enumerate(tokens):
            stepped = dec.step(int(t), 500 + i)
        logits_s = download(dec, "LOGITS", 0, np.empty(shape["vocab"], np.float32))
        cache_s = download(dec, "KCACHE", 23, np.empty((2, 2048, 64), np.uint16))
        ids_s = dec.generate(stepped, 800, 8)
    assert close(logits_p, logits_s, 1e-3) == 0
    assert nxt == stepped
    assert np.abs(orc.half_to_float(cache_p) - orc.half_to_float(cache_s)).max() <= 2e-3 * (
        1 + np.abs(orc.half_to_float(cache_s)).max())
    assert ids_p == ids_s


@pytest.mark.parametrize("count", [2048, 1990])
def test_decoder_prefill_7b_width_full_prompt_equals_steps(mh, gpu, orc, count):
    """The 7B widths over a 2048-token (and a 1990-token: ragged last token tiles) prompt, where
    q|k|v takes 128 x 128 tiles over two K halves, o_proj and down 128 x 256 tiles over two K
    halves and the gate+up 128 x 256 tiles: the same logits, cache rows and next token as the
    decoder's own steps."""
    shape = dict(mh.QWEN25_7B, layers=2)
    tokens = prompt(orc, count, shape["vocab"], 63)
    with mh.Decoder(mh.qwen2_config(**shape)) as dec:
        dec.fill_random(64)
        nxt = dec.prefill(tokens, 0)
        logits_p = download(dec, "LOGITS", 0, np.empty(shape["vocab"], np.float32))
        cache_p = download(dec, "VCACHE", 1, np.empty((4, 2048, 128), np.uint16))
        dec.fill_kv_random(0, 0)
        for i, t in enumerate(tokens):
            stepped = dec.step(int(t), i)
        logits_s = download(dec, "LOGITS", 0, np.empty(shape["vocab"], np.float32))
        cache_s = download(dec, "VCACHE", 1, np.empty((4, 2048, 128), np.uint16))
    assert close(logits_p, logits_s, 1e-3) == 0
    assert nxt == stepped
    assert np.abs(orc.half_to_float(cache_p) - orc.half_to_float(cache_s)).max() <= 2e-3 * (
        1 + np.abs(orc.half_to_float(cache_s)).max())


@pytest.mark.timeout(900)
def test_decoder_prefill_7b_width_1024_tokens_matches_oracle(mh, gpu, orc):
    """The 7B widths (hidden 3584, ffn 18944, 28/4 heads of 128) over a 1024-token prompt from row
    0, which takes the 128 x 256 gate+up tiles, against the oracle fed token by token: the last
    position's logits, the next token and every cache row (a small vocabulary keeps the oracle's
    LM head cheap; the projections are full width)."""
    orc.set_threads(16)
    shape = dict(mh.QWEN25_7B, layers=2, vocab=2000)
    dec, model = make_pair(mh, orc, shape, seed=90)
    with dec:
        check_against_oracle(dec, model, orc, shape, prompt(orc, 1024, shape["vocab"], 91), 0)


def test_decoder_prefill_in_passes(mh, gpu, orc):
    """A prompt longer than one pass (2048 rows) runs in two; the second pass attends to the first
    through the cache."""
    shape = dict(layers=2, hidden=256, ffn=512, heads=4, kv_heads=2, head_dim=64, vocab=1000, max_seq=2300)
    dec, model = make_pair(mh, orc, shape, seed=71)
    with dec:
        check_against_oracle(dec, model, orc, shape, prompt(orc, 2200, shape["vocab"], 72), 50)


def test_decoder_prefill_7b_shape_two_layers(mh, gpu, orc):
    orc.set_threads(16)
    shape = dict(mh.QWEN25_7B, layers=2)
    dec, model = make_pair(mh, orc, shape, seed=80, kv_positions=2000, kv_seed=81)
    with dec:
        check_against_oracle(dec, model, orc, shape, prompt(orc, 24, shape["vocab"], 82), 2000)


def test_decoder_prefill_samples_like_a_step(mh, gpu, orc):
    """With a sampler set, the prefill draws once from the last position's logits with the prompt
    as history, as runTurn's sampleNext does after the feed (src/FullModel.cpp:1162-1176)."""
    params = dict(temperature=0.8, top_k=40, top_p=0.9, repeat_penalty=1.3, repeat_last_n=64, seed=99)
    tokens = prompt(orc, 50, SMALL["vocab"], 91)
    with mh.Decoder(mh.qwen2_config(**SMALL)) as dec:
        dec.fill_random(90)
        dec.set_sampler(**params)
        got = dec.prefill(tokens, 0)
        dec.set_sampler()
        for i, t in enumerate(tokens[:-1]):
            dec.step(int(t), i)
        dec.set_sampler(**params)
        want = dec.step(int(tokens[-1]), len(tokens) - 1)
    assert got == want


def test_decoder_prefill_refusals(mh, gpu):
    with mh.Decoder(mh.qwen2_config(**SMALL)) as dec:
        lib = mh.load()
        toks = (ctypes.c_int32 * 4)(1, 2, 3, SMALL["vocab"])
        nxt = ctypes.c_int32()
        assert lib.muyo_decoder_prefill(dec.handle, toks, 0, 0, ctypes.byref(nxt)) == mh.MUYO_E_RANGE
        assert lib.muyo_decoder_prefill(dec.handle, toks, 4, 0, ctypes.byref(nxt)) == mh.MUYO_E_RANGE
        assert lib.muyo_decoder_prefill(dec.handle, toks, 3, SMALL["max_seq"] - 2, ctypes.byref(nxt)) == mh.MUYO_E_RANGE
        assert lib.muyo_decoder_prefill(dec.handle, toks, 3, -1, ctypes.byref(nxt)) == mh.MUYO_E_RANGE
        assert lib.muyo_decoder_prefill(dec.handle, None, 3, 0, ctypes.byref(nxt)) == mh.MUYO_E_NULL
