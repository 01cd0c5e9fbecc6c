"""Per-op parity on the GPU: each C-ABI launcher against the CPU oracle on the same inputs.

Tolerances (mixed form |a - e| <= tol * (1 + |e|), the reference's own): GEMV, add, swiglu and
rope 1e-3; rms_norm and softmax 1e-5; argmax, get_rows, copies and cache indexing bit-exact.
Inputs: the reference's known-answer tests (src/*.cpp) and the batched decode shapes, drawn from
the portable seeded generator.
"""
import math

import numpy as np
import pytest

from conftest import close, worst

pytestmark = pytest.mark.gpu

SEED = 20261201


def dev(torch, array):
    return torch.from_numpy(np.ascontiguousarray(array)).cuda()


def host(t):
    return t.detach().cpu().numpy()


def stream(torch):
    return torch.cuda.current_stream().cuda_stream


def run(mh, torch, status):
    mh.check(status)
    torch.cuda.synchronize()


# ------------------------------------------------------------------------------------------------
# GEMV


def gemv(mh, torch, w_bits, x, rows=None, bias=None, num_rows=1, dispatch=None):
    rows_total, cols = w_bits.shape
    rows = rows or rows_total
    a = dev(torch, w_bits)
    b = dev(torch, x.astype(np.float32))
    d = torch.full((rows_total,), float("nan"), dtype=torch.float32, device="cuda")
    f0 = dev(torch, bias.astype(np.float32)) if bias is not None else None
    pc = mh.mat_vec_push_constants(cols, rows, fusion_flags=mh.FUSION_BIAS0 if bias is not None else 0)
    spec = mh.MuyoMatVecSpec(32, num_rows, 1)
    gx, gy, gz = dispatch or ((rows + num_rows - 1) // num_rows, 1, 1)
    run(mh, torch, mh.load().muyo_mul_mat_vec_f16_f32_f32(
        mh.ref(pc), mh.ref(spec), a.data_ptr(), b.data_ptr(), d.data_ptr(), f0.data_ptr() if f0 is not None else None,
        None, gx, gy, gz, stream(torch)))
    return host(d)


def test_matvec_reference_known_answer(mh, gpu, orc):
    """src/MatVec.cpp:68-80,198-210: exact equality."""
    rows, cols = 128, 256
    c = np.arange(cols)
    w = np.tile(((c % 7) - 3).astype(np.float16), (rows, 1)).view(np.uint16)
    x = ((c % 5) - 2).astype(np.float32)
    y = gemv(mh, gpu, w, x)
    assert np.array_equal(y, orc.mat_vec_f16(w, x))


def test_matvec_seeded_matvec_shape(mh, gpu, orc):
    """128 x 256 fp16 N(0, 0.02) weights, x U[-1, 1], f32 accumulate."""
    w = orc.normal_f16(128 * 256, SEED, 0.0, 0.02).reshape(128, 256)
    x = orc.uniform_f32(256, SEED + 1)
    y = gemv(mh, gpu, w, x)
    assert close(y, orc.mat_vec_f16(w, x), 1e-3) == 0
    assert worst(y, orc.mat_vec_f16(w, x, f64acc=True)) < 1e-5


@pytest.mark.parametrize(
    "rows,cols,with_bias",
    [(1152, 896, True), (896, 896, False), (4864, 896, False), (896, 4864, False), (151936, 896, False),
     (4608, 3584, True), (3584, 18944, False)],
    ids=["qkv", "o_proj", "gate_up", "down", "lm_head", "7b_qkv", "7b_down"])
def test_matvec_decode_shapes(mh, gpu, orc, rows, cols, with_bias):
    w = orc.normal_f16(rows * cols, SEED + rows, 0.0, 0.02).reshape(rows, cols)
    x = orc.normal_f32(cols, SEED + cols)
    bias = orc.normal_f32(rows, SEED + 7, 0.0, 0.02) if with_bias else None
    y = gemv(mh, gpu, w, x, bias=bias)
    expect = orc.mat_vec_f16(w, x, f64acc=True) + (bias if with_bias else 0)
    assert close(y, expect, 1e-3) == 0
    assert worst(y, expect) < 2e-5


def test_matvec_generic_path_and_row_bounds(mh, gpu, orc):
    # ncols not a multiple of 8 takes the any-alignment kernel; NUM_ROWS 3 with strideD clipping.
    rows, cols = 50, 250
    w = orc.normal_f16(rows * cols, 3, 0.0, 0.1).reshape(rows, cols)
    x = orc.normal_f32(cols, 4)
    y = gemv(mh, gpu, w, x, num_rows=3, dispatch=(17, 1, 1))  # 51 rows dispatched, 50 bound
    assert close(y, orc.mat_vec_f16(w, x, f64acc=True), 1e-3) == 0
    # A dispatch covering fewer rows leaves the rest untouched.
    y2 = gemv(mh, gpu, w, x, dispatch=(20, 1, 1))
    assert close(y2[:20], orc.mat_vec_f16(w, x, f64acc=True)[:20], 1e-3) == 0
    assert np.isnan(y2[20:]).all()


def test_matvec_f32_gqa_score_and_value_gemvs(mh, gpu, orc):
    """The attention GEMVs of src/FullModel.cpp:793-812 (scores) and :825-844 (values) on an f32 cache, via batch/broadcast."""
    torch = gpu
    heads, kv, hd, max_seq, pos = 14, 2, 64, 2048, 300
    gqa = heads // kv
    kcache = orc.normal_f32(kv * max_seq * hd, 11).reshape(kv, max_seq, hd)
    q = orc.normal_f32(heads * hd, 12)
    scores = torch.full((heads * max_seq,), -1e30, dtype=torch.float32, device="cuda")
    pc = mh.mat_vec_push_constants(hd, max_seq, stride_a=hd, stride_b=hd, batch_stride_a=hd * max_seq,
                                   batch_stride_b=hd, batch_stride_d=max_seq, ne02=1, ne12=gqa, broadcast2=gqa,
                                   broadcast3=1)
    kd, qd = dev(torch, kcache), dev(torch, q)
    run(mh, torch, mh.load().muyo_mul_mat_vec_f32_f32_f32(mh.ref(pc), None, kd.data_ptr(), qd.data_ptr(),
                                                           scores.data_ptr(), None, None, pos + 1, heads, 1,
                                                           stream(torch)))
    s = host(scores).reshape(heads, max_seq)
    for h in range(heads):
        expect = orc.mat_vec_f32(kcache[h // gqa, : pos + 1], q[h * hd:(h + 1) * hd])
        assert close(s[h, : pos + 1], expect, 1e-3) == 0
        assert np.all(s[h, pos + 1:] == -1e30)
    # Values: vcache transposed [kv][hd][max_seq], the reduction over the whole row (Finding F11).
    vcache_t = orc.normal_f32(kv * hd * max_seq, 13).reshape(kv, hd, max_seq)
    vcache_t[:, :, pos + 1:] = 0
    probs = orc.soft_max(orc.normal_f32(heads * max_seq, 14).reshape(heads, max_seq), 1.0)
    out = torch.zeros(heads * hd, dtype=torch.float32, device="cuda")
    pcv = mh.mat_vec_push_constants(max_seq, hd, stride_a=max_seq, stride_b=max_seq, batch_stride_a=hd * max_seq,
                                    batch_stride_b=max_seq, batch_stride_d=hd, ne02=1, ne12=gqa, broadcast2=gqa,
                                    broadcast3=1)
    vd, pd = dev(torch, vcache_t), dev(torch, probs)
    run(mh, torch, mh.load().muyo_mul_mat_vec_f32_f32_f32(mh.ref(pcv), None, vd.data_ptr(), pd.data_ptr(),
                                                           out.data_ptr(), None, None, hd, heads, 1, stream(torch)))
    o = host(out).reshape(heads, hd)
    for h in range(heads):
        assert close(o[h], orc.mat_vec_f32(vcache_t[h // gqa], probs[h]), 1e-3) == 0


def test_matvec_contract_errors(mh, gpu):
    torch = gpu
    lib = mh.load()
    a = torch.zeros(64, dtype=torch.float16, device="cuda")
    b = torch.zeros(8, dtype=torch.float32, device="cuda")
    d = torch.zeros(8, dtype=torch.float32, device="cuda")
    pc = mh.mat_vec_push_constants(8, 8, fusion_flags=mh.FUSION_BIAS0)
    assert lib.muyo_mul_mat_vec_f16_f32_f32(mh.ref(pc), None, a.data_ptr(), b.data_ptr(), d.data_ptr(), None, None,
                                            8, 1, 1, 0) == mh.MUYO_E_NULL
    assert b"FUSE0" in lib.muyo_last_error()
    spec = mh.MuyoMatVecSpec(32, 1, 2)
    pc.fusionFlags = 0
    assert lib.muyo_mul_mat_vec_f16_f32_f32(mh.ref(pc), mh.ref(spec), a.data_ptr(), b.data_ptr(), d.data_ptr(), None,
                                            None, 8, 1, 1, 0) == mh.MUYO_E_UNSUPPORTED


# ------------------------------------------------------------------------------------------------
# rms_norm


def rms(mh, torch, x, w, eps, half_weight=False):
    rows, cols = x.shape
    xd = dev(torch, x)
    wd = dev(torch, w)
    d = torch.empty_like(xd)
    pc = mh.rows_push_constants(cols, rows, eps)
    fn = mh.load().muyo_rms_norm_f32_f16w if half_weight else mh.load().muyo_rms_norm_f32
    run(mh, torch, fn(mh.ref(pc), 1, xd.data_ptr(), wd.data_ptr(), d.data_ptr(), None, rows, 1, 1, stream(torch)))
    return host(d)


def test_rms_norm_reference_known_answer(mh, gpu, orc):
    """src/RmsNorm.cpp:41-72,194-216."""
    idx = np.arange(8 * 512).reshape(8, 512)
    x = ((idx % 13) - 6).astype(np.float32)
    w = (0.5 + 0.001 * (np.arange(512) % 11)).astype(np.float32)
    assert close(rms(mh, gpu, x, w, 1e-6), orc.rms_norm(x, w, 1e-6), 1e-5) == 0


def test_rms_norm_batched_decode_shape(mh, gpu, orc):
    """4096 rows x 896, eps 1e-6, fp16 weight N(1, 0.1)."""
    x = orc.normal_f32(4096 * 896, SEED + 2).reshape(4096, 896)
    w = orc.normal_f16(896, SEED + 3, 1.0, 0.1)
    y = rms(mh, gpu, x, w, 1e-6, half_weight=True)
    assert close(y, orc.rms_norm(x, w, 1e-6), 1e-5) == 0


@pytest.mark.parametrize("rows,cols,half", [(4096, 896, True), (33, 2048, False), (7, 1028, True), (5, 12, False)])
def test_rms_norm_dense_and_strided_rows_agree(mh, gpu, orc, rows, cols, half):
    """Dense rows take the streaming kernel; the same rows at a stride of cols + 4 take the general
    one. Both match the oracle, and each other bit for bit (the same sums in the same order)."""
    torch = gpu
    x = orc.normal_f32(rows * cols, SEED + cols).reshape(rows, cols)
    w = orc.normal_f16(cols, SEED + 1, 1.0, 0.1) if half else orc.normal_f32(cols, SEED + 1, 1.0, 0.1)
    dense = rms(mh, gpu, x, w, 1e-6, half_weight=half)
    padded = np.zeros((rows, cols + 4), np.float32)
    padded[:, :cols] = x
    xd = dev(torch, padded)
    wd = dev(torch, w)
    d = torch.empty(rows * cols, dtype=torch.float32, device="cuda")
    pc = mh.rows_push_constants(cols, rows, 1e-6)
    pc.nb01, pc.nb02, pc.nb03 = cols + 4, (cols + 4) * rows, (cols + 4) * rows
    fn = mh.load().muyo_rms_norm_f32_f16w if half else mh.load().muyo_rms_norm_f32
    run(mh, torch, fn(mh.ref(pc), 1, xd.data_ptr(), wd.data_ptr(), d.data_ptr(), None, rows, 1, 1, stream(torch)))
    strided = host(d).reshape(rows, cols)
    assert np.array_equal(dense, strided)
    assert close(dense, orc.rms_norm(x, w, 1e-6), 1e-5) == 0


def test_rms_norm_broadcast_and_offsets(mh, gpu, orc):
    """Weight shorter than the row (fastmod wrap) and a dispatch over (rows, channels)."""
    torch = gpu
    x = orc.normal_f32(6 * 96, 5).reshape(6, 96)
    w = orc.normal_f32(32, 6, 1.0, 0.1)
    pc = mh.rows_push_constants(96, 3, 1e-5, weight_length=32)
    pc.ne02, pc.nb02 = 2, 96 * 3
    xd, wd = dev(torch, x), dev(torch, w)
    d = torch.empty_like(xd)
    run(mh, torch, mh.load().muyo_rms_norm_f32(mh.ref(pc), 1, xd.data_ptr(), wd.data_ptr(), d.data_ptr(), None, 3, 2,
                                               1, stream(torch)))
    expect = orc.rms_norm(x, np.tile(w, 3), 1e-5)
    assert close(host(d), expect, 1e-5) == 0


# ------------------------------------------------------------------------------------------------
# softmax


def softmax(mh, torch, x, scale):
    rows, cols = x.shape
    xd = dev(torch, x)
    d = torch.empty_like(xd)
    pc = mh.soft_max_push_constants(rows, cols, scale)
    run(mh, torch, mh.load().muyo_soft_max_f32(mh.ref(pc), xd.data_ptr(), None, None, d.data_ptr(),
                                               *mh.row_dispatch(rows), stream(torch)))
    return host(d)


def test_soft_max_reference_known_answer(mh, gpu, orc):
    """src/SoftMax.cpp:42-55,164-191."""
    x = ((np.arange(64) % 9) - 4).astype(np.float32)[None, :]
    assert close(softmax(mh, gpu, x, 0.125), orc.soft_max(x, 0.125), 1e-5) == 0


def test_soft_max_batched_decode_shape(mh, gpu, orc):
    """4096 x 14 heads x 2048 scores N(0, 3)."""
    x = orc.normal_f32(4096 * 14 * 2048, SEED + 4, 0.0, 3.0).reshape(4096 * 14, 2048)
    y = softmax(mh, gpu, x, 1.0)
    assert close(y, orc.soft_max(x, 1.0), 1e-5) == 0


def test_soft_max_masked_tail_and_long_rows(mh, gpu, orc):
    x = orc.normal_f32(14 * 2048, 8, 0.0, 3.0).reshape(14, 2048)
    x[:, 700:] = -1e30
    y = softmax(mh, gpu, x, 0.125)
    assert close(y, orc.soft_max(x, 0.125), 1e-5) == 0 and np.all(y[:, 700:] == 0)
    long = orc.normal_f32(3 * 9000, 9).reshape(3, 9000)  # past the register cache: general path
    assert close(softmax(mh, gpu, long, 0.5), orc.soft_max(long, 0.5), 1e-5) == 0


# ------------------------------------------------------------------------------------------------
# argmax


def argmax(mh, torch, x):
    rows, cols = x.shape
    xd = dev(torch, x)
    d = torch.full((rows,), -7, dtype=torch.int32, device="cuda")
    pc = mh.argmax_push_constants(cols, rows)
    run(mh, torch, mh.load().muyo_argmax_f32(mh.ref(pc), xd.data_ptr(), d.data_ptr(), *mh.row_dispatch(rows),
                                             stream(torch)))
    return host(d)


def test_argmax_reference_known_answer_and_ties(mh, gpu, orc):
    logits = (-1.0 + 0.001 * np.arange(32)).astype(np.float32)
    logits[21] = 5.0
    assert argmax(mh, gpu, logits[None])[0] == 21
    tie = np.zeros((2, 151936), np.float32)
    tie[0, [5000, 70000, 151935]] = 2.0
    tie[1, [151935]] = 1.0
    tie[1, 3] = 1.0
    assert argmax(mh, gpu, tie).tolist() == [5000, 3]


@pytest.mark.parametrize("cols", [1, 3, 1021, 4096, 4099, 8191, 151936])
def test_argmax_ties_across_load_batches_and_tails(mh, gpu, orc, cols):
    """A thread keeps four float4 loads in flight, 256 float4 apart, then finishes the row one
    float4 and one scalar at a time. Equal maxima planted in every such position (each batch
    slot, the float4 tail, the scalar tail) must resolve to the lowest index, as the host scan's
    strict '>' does."""
    rng = np.random.default_rng(cols)
    rows = 8
    x = rng.normal(0.0, 1.0, (rows, cols)).astype(np.float32)
    n4 = cols // 4
    for r in range(rows):
        candidates = {c for c in (r, 4 * 256 + r, 2 * 4 * 256 + 3, 3 * 4 * 256 + 1, 4 * 4 * 256 + 2,
                                  4 * (n4 - 1), 4 * n4, cols - 1) if 0 <= c < cols}
        picks = sorted(candidates)[r % max(1, len(candidates)):] or sorted(candidates)
        x[r, picks] = 7.5
    want = orc.argmax_rows(x)
    assert np.array_equal(want, np.argmax(x, axis=1))
    assert np.array_equal(argmax(mh, gpu, x), want)


def test_argmax_batched_decode_shape(mh, gpu, orc):
    """4096 rows x 151936 logits N(0, 2): 256 rows against the oracle, all rows against torch.argmax."""
    torch = gpu
    rows, cols = 4096, 151936
    xd = torch.empty(rows * cols, dtype=torch.float32, device="cuda")
    mh.check(mh.load().muyo_fill_normal_f32(xd.data_ptr(), rows * cols, SEED + 5, 0.0, 2.0, stream(torch)))
    d = torch.empty(rows, dtype=torch.int32, device="cuda")
    pc = mh.argmax_push_constants(cols, rows)
    run(mh, torch, mh.load().muyo_argmax_f32(mh.ref(pc), xd.data_ptr(), d.data_ptr(), *mh.row_dispatch(rows),
                                             stream(torch)))
    got = host(d)
    sample = host(xd[: 256 * cols]).reshape(256, cols)
    assert np.array_equal(got[:256], orc.argmax_rows(sample))
    assert np.array_equal(got, host(torch.argmax(xd.view(rows, cols), dim=1).to(torch.int32)))


# ------------------------------------------------------------------------------------------------
# add, swiglu


def test_add_reference_known_answer(mh, gpu, orc):
    torch = gpu
    i = np.arange(1000, dtype=np.float32)
    a, b = 0.5 * i, 1.0 + 0.25 * i
    ad, bd = dev(torch, a), dev(torch, b)
    d = torch.empty_like(ad)
    pc = mh.add_push_constants(1000)
    run(mh, torch, mh.load().muyo_add_f32(mh.ref(pc), 1, ad.data_ptr(), bd.data_ptr(), d.data_ptr(), None,
                                          *mh.add_dispatch(1000), stream(torch)))
    assert np.array_equal(host(d), orc.add(a, b))


def test_add_batched_and_broadcast(mh, gpu, orc):
    torch = gpu
    n = 4096 * 896
    a = orc.normal_f32(n, SEED + 6)
    b = orc.normal_f32(n, SEED + 7)
    ad, bd = dev(torch, a), dev(torch, b)
    d = torch.empty_like(ad)
    pc = mh.add_push_constants(n, row=896)
    run(mh, torch, mh.load().muyo_add_f32(mh.ref(pc), 1, ad.data_ptr(), bd.data_ptr(), d.data_ptr(), None,
                                          *mh.add_dispatch(n), stream(torch)))
    assert np.array_equal(host(d), orc.add(a, b))
    # B is one row repeated over all rows (norepeat = 0 takes the modulo path).
    row = orc.normal_f32(896, 3)
    rd = dev(torch, row)
    pc.ne11, pc.nb11, pc.nb12, pc.nb13 = 1, 896, 896, 896
    run(mh, torch, mh.load().muyo_add_f32(mh.ref(pc), 0, ad.data_ptr(), rd.data_ptr(), d.data_ptr(), None,
                                          *mh.add_dispatch(n), stream(torch)))
    assert np.array_equal(host(d), orc.add(a, np.tile(row, 4096)))


def swiglu(mh, torch, g, u, row=None):
    gd, ud = dev(torch, g), dev(torch, u)
    d = torch.empty_like(gd)
    pc = mh.glu_push_constants(g.size, row)
    run(mh, torch, mh.load().muyo_swiglu_f32(mh.ref(pc), gd.data_ptr(), ud.data_ptr(), d.data_ptr(),
                                             *mh.add_dispatch(g.size), stream(torch)))
    return host(d)


def test_swiglu_reference_known_answer(mh, gpu, orc):
    i = np.arange(600)
    g = (0.01 * ((i % 17) - 8)).astype(np.float32)
    u = (0.5 + 0.01 * (i % 7)).astype(np.float32)
    assert close(swiglu(mh, gpu, g, u), orc.swiglu(g, u), 1e-5) == 0


def test_swiglu_batched_decode_shape(mh, gpu, orc):
    n = 4096 * 4864
    g = orc.normal_f32(n, SEED + 8)
    u = orc.normal_f32(n, SEED + 9)
    assert close(swiglu(mh, gpu, g, u, row=4864), orc.swiglu(g, u), 1e-3) == 0


def test_swiglu_rejects_wrong_fastdiv(mh, gpu):
    torch = gpu
    x = torch.zeros(600, dtype=torch.float32, device="cuda")
    pc = mh.glu_push_constants(600)
    pc.ne2_0mp = 0  # what a zero-initialised block would carry
    status = mh.load().muyo_swiglu_f32(mh.ref(pc), x.data_ptr(), x.data_ptr(), x.data_ptr(), 1, 2, 1, 0)
    assert status == mh.MUYO_E_CONTRACT


# ------------------------------------------------------------------------------------------------
# rope


def test_rope_reference_known_answer(mh, gpu, orc):
    """src/Rope.cpp:41-64,191-214: nDims 8, pos 3, base 1e4."""
    torch = gpu
    x = (np.arange(8) - 3).astype(np.float32)
    xd, pd = dev(torch, x), dev(torch, np.array([3], np.int32))
    d = torch.empty_like(xd)
    pc = mh.rope_push_constants(1, 8, 10000.0)
    run(mh, torch, mh.load().muyo_rope_neox_f32(mh.ref(pc), xd.data_ptr(), pd.data_ptr(), None, d.data_ptr(), None,
                                                1, 1, 1, stream(torch)))
    assert close(host(d), orc.rope_neox(x[None], 3, pc.thetaScale)[0], 1e-5) == 0


def test_rope_batched_decode_shape(mh, gpu, orc):
    """4096 tokens x (14 q + 2 k heads) x 64, theta 1e6, positions U[0, 2047] per token."""
    torch = gpu
    tokens, heads, hd = 4096, 16, 64
    x = orc.normal_f32(tokens * heads * hd, SEED + 10).reshape(tokens, heads, hd)
    pos = (np.floor((orc.uniform_f32(tokens, SEED + 11) + 1.0) * 1024.0)).astype(np.int32)
    assert pos.min() >= 0 and pos.max() <= 2047
    xd, pd = dev(torch, x), dev(torch, pos)
    d = torch.empty_like(xd)
    pc = mh.rope_push_constants(heads, hd, 1e6, tokens=tokens)
    run(mh, torch, mh.load().muyo_rope_neox_f32(mh.ref(pc), xd.data_ptr(), pd.data_ptr(), None, d.data_ptr(), None,
                                                heads * tokens, 1, 1, stream(torch)))
    got = host(d)
    bad = 0
    for t in range(tokens):  # every token
        bad += close(got[t], orc.rope_neox(x[t], int(pos[t]), pc.thetaScale), 1e-3)
    assert bad == 0


@pytest.mark.parametrize("tokens,heads,hd", [(37, 14, 64), (5, 28, 128), (9, 3, 64), (2, 1, 8), (3, 2, 24)])
def test_rope_streaming_and_general_paths_agree(mh, gpu, orc, tokens, heads, hd):
    """The launcher streams whole 16-byte-aligned rows four heads at a time (head counts that are
    no multiple of 4 included) and takes the element-wise kernel otherwise: here a destination
    offset of one float forces the latter. Both match the oracle on every row and each other bit
    for bit (they compute every angle with the same code)."""
    torch = gpu
    x = orc.normal_f32(tokens * heads * hd, SEED + 40 + hd).reshape(tokens, heads, hd)
    pos = (np.arange(tokens, dtype=np.int32) * 613 + 7) % 2048
    xd, pd = dev(torch, x), dev(torch, pos.astype(np.int32))
    lib = mh.load()
    fast = torch.empty_like(xd)
    pc = mh.rope_push_constants(heads, hd, 1e6, tokens=tokens)
    run(mh, torch, lib.muyo_rope_neox_f32(mh.ref(pc), xd.data_ptr(), pd.data_ptr(), None, fast.data_ptr(), None,
                                          heads * tokens, 1, 1, stream(torch)))
    slow = torch.zeros(tokens * heads * hd + 1, dtype=torch.float32, device="cuda")
    pc1 = mh.rope_push_constants(heads, hd, 1e6, tokens=tokens, destination_offset=1)
    run(mh, torch, lib.muyo_rope_neox_f32(mh.ref(pc1), xd.data_ptr(), pd.data_ptr(), None, slow.data_ptr(), None,
                                          heads * tokens, 1, 1, stream(torch)))
    got, ref = host(fast), host(slow)[1:].reshape(tokens, heads, hd)
    assert np.array_equal(got, ref)
    for t in range(tokens):
        assert close(got[t], orc.rope_neox(x[t], int(pos[t]), pc.thetaScale), 1e-3) == 0, t


def test_rope_into_key_cache_row(mh, gpu, orc):
    """k_rope of src/FullModel.cpp:771-784: rows strided by hd*max_seq, dOffset = pos*hd; bit-exact slots."""
    torch = gpu
    kv, hd, max_seq, pos = 2, 64, 2048, 1234
    k = orc.normal_f32(kv * hd, 21)
    cache = torch.zeros(kv * max_seq * hd, dtype=torch.float32, device="cuda")
    kd, pd = dev(torch, k), dev(torch, np.array([pos], np.int32))
    pc = mh.rope_push_constants(kv, hd, 1e6, output_row_stride=hd * max_seq, destination_offset=pos * hd)
    run(mh, torch, mh.load().muyo_rope_neox_f32(mh.ref(pc), kd.data_ptr(), pd.data_ptr(), None, cache.data_ptr(),
                                                None, kv, 1, 1, stream(torch)))
    c = host(cache).reshape(kv, max_seq, hd)
    assert close(c[:, pos], orc.rope_neox(k.reshape(kv, hd), pos, pc.thetaScale), 1e-3) == 0
    c[:, pos] = 0
    assert not c.any()


# ------------------------------------------------------------------------------------------------
# get_rows, cpy


def test_get_rows_reference_known_answer_f32(mh, gpu):
    torch = gpu
    vocab, dim = 1024, 512
    t = np.arange(vocab)[:, None]
    table = ((((t % 5) - 2) + 0.001 * np.arange(dim)[None, :]).astype(np.float32))
    td, idx = dev(torch, table), dev(torch, np.array([7], np.int32))
    d = torch.empty(dim, dtype=torch.float32, device="cuda")
    pc = mh.get_rows_push_constants(dim, vocab)
    run(mh, torch, mh.load().muyo_get_rows_f32(mh.ref(pc), td.data_ptr(), idx.data_ptr(), d.data_ptr(), 1, 1, 1,
                                               stream(torch)))
    assert np.array_equal(host(d), table[7])


def test_get_rows_f16_embedding(mh, gpu, orc):
    torch = gpu
    vocab, dim = 151936, 896
    table = torch.empty(vocab * dim, dtype=torch.float16, device="cuda")
    mh.check(mh.load().muyo_fill_normal_f16(table.data_ptr(), vocab * dim, 77, 0.0, 0.02, stream(torch)))
    tokens = np.array([0, 1, 151935, 9707, 1879, -1, 151936], np.int32)
    idx = dev(torch, tokens)
    d = torch.full((len(tokens) * dim,), float("nan"), dtype=torch.float32, device="cuda")
    pc = mh.get_rows_push_constants(dim, vocab, count=len(tokens))
    run(mh, torch, mh.load().muyo_get_rows_f16_f32(mh.ref(pc), table.data_ptr(), idx.data_ptr(), d.data_ptr(),
                                                   (dim + 511) // 512, len(tokens), 1, stream(torch)))
    got = host(d).reshape(len(tokens), dim)
    bits = host(table.view(torch.int16)).view(np.uint16).reshape(vocab, dim)
    for i, tok in enumerate(tokens[:5]):
        assert np.array_equal(got[i], orc.get_rows_f16(bits, int(tok)))
    assert not got[5:].any()  # out-of-range ids give zero rows


def test_cpy_value_column_append(mh, gpu):
    """CopyValueColumnExecute (src/FullModel.cpp:376-420): v[kvh][c] -> vcache[kvh][c][pos], bit-exact.

    That fill encodes ne11 in ne1_0mp; the shader divides by what the words encode, so this runs."""
    torch = gpu
    kv, hd, max_seq = 2, 64, 2048
    for pos in (0, 5, 2047):
        v = np.arange(kv * hd, dtype=np.float32) + 0.5
        cache = torch.zeros(kv * hd * max_seq, dtype=torch.float32, device="cuda")
        vd = dev(torch, v)
        pc = mh.value_column_push_constants(kv * hd, hd, max_seq, pos)
        run(mh, torch, mh.load().muyo_cpy_f32_f32(mh.ref(pc), vd.data_ptr(), cache.data_ptr(), 1, 1, 1,
                                                  stream(torch)))
        c = host(cache).reshape(kv, hd, max_seq)
        assert np.array_equal(c[:, :, pos], v.reshape(kv, hd))
        c[:, :, pos] = 0
        assert not c.any()
    # A zeroed block's words encode no divisor: rejected, not scattered to row 0.
    pc.ne1_0mp = 0
    assert mh.load().muyo_cpy_f32_f32(mh.ref(pc), vd.data_ptr(), cache.data_ptr(), 1, 1, 1, 0) == mh.MUYO_E_CONTRACT


def _shader_fastdiv(n, mp, shift):
    """fastdiv of utils.glsl:13-18 in 32-bit arithmetic."""
    return ((((n * mp) >> 32) + n) & 0xFFFFFFFF) >> shift


def _shader_unary_idx(idx, ne, nb, mps, ls):
    """src0_idx/dst_idx of generic_unary_head.glsl:34-55 with explicit magic words."""
    i3 = _shader_fastdiv(idx, mps[0], ls & 0x3F)
    o3 = i3 * ne[2] * ne[1] * ne[0]
    i2 = _shader_fastdiv(idx - o3, mps[1], (ls >> 8) & 0x3F)
    o2 = i2 * ne[1] * ne[0]
    i1 = _shader_fastdiv(idx - o3 - o2, mps[2], (ls >> 16) & 0x3F)
    i0 = idx - o3 - o2 - i1 * ne[0]
    return i3 * nb[3] + i2 * nb[2] + i1 * nb[1] + i0 * nb[0]


def test_cpy_kv_cache_fill_and_shader_index_math(mh, gpu):
    """src/KvCache.cpp:196-217 (ne10 in ne1_0mp, [channels][positions], nb11 = 1) and a 3-D
    transposing copy, both against the shader's fastdiv index arithmetic evaluated on the host."""
    torch = gpu
    cases = []
    pc = mh.LlamaCopyPushConstants()
    pc.ne, pc.ne00, pc.ne01, pc.ne02, pc.ne03, pc.nb00 = 16, 16, 1, 1, 1, 1
    pc.ne10, pc.ne11, pc.ne12, pc.ne13, pc.nb10, pc.nb11 = 16, 4, 1, 1, 4, 1
    pc.misalignOffsets = 3  # position
    cases.append((pc, 16 * 4 + 8))
    q = mh.LlamaCopyPushConstants()  # [3][5][7] -> its transpose [7][5][3]
    q.ne, q.ne00, q.ne01, q.ne02, q.ne03 = 105, 7, 5, 3, 1
    q.nb00, q.nb01, q.nb02, q.nb03 = 1, 7, 35, 105
    q.ne10, q.ne11, q.ne12, q.ne13 = 7, 5, 3, 1
    q.nb10, q.nb11, q.nb12, q.nb13 = 15, 3, 1, 105
    cases.append((q, 128))
    for pc, size in cases:
        for side in (0, 1):
            ne = [getattr(pc, f"ne{side}{k}") for k in range(3)]
            mp012, l012 = mh.init_fastdiv(ne[0] * ne[1] * ne[2])
            mp01, l01 = mh.init_fastdiv(ne[0] * ne[1])
            mp0, l0 = mh.init_fastdiv(ne[0])
            setattr(pc, f"ne{side}_012mp", mp012)
            setattr(pc, f"ne{side}_01mp", mp01)
            setattr(pc, f"ne{side}_0mp", mp0)
            setattr(pc, f"ne{side}_Ls", l012 | (l01 << 8) | (l0 << 16))
        a = np.arange(pc.ne, dtype=np.float32) + 1.0
        ad = dev(torch, a)
        d = torch.zeros(size, dtype=torch.float32, device="cuda")
        run(mh, torch, mh.load().muyo_cpy_f32_f32(mh.ref(pc), ad.data_ptr(), d.data_ptr(), 1, 1, 1, stream(torch)))
        expect = np.zeros(size, np.float32)
        aoff, doff = pc.misalignOffsets >> 16, pc.misalignOffsets & 0xFFFF
        for i in range(pc.ne):
            s = _shader_unary_idx(i, [pc.ne00, pc.ne01, pc.ne02], [pc.nb00, pc.nb01, pc.nb02, pc.nb03],
                                  [pc.ne0_012mp, pc.ne0_01mp, pc.ne0_0mp], pc.ne0_Ls)
            t = _shader_unary_idx(i, [pc.ne10, pc.ne11, pc.ne12], [pc.nb10, pc.nb11, pc.nb12, pc.nb13],
                                  [pc.ne1_012mp, pc.ne1_01mp, pc.ne1_0mp], pc.ne1_Ls)
            expect[doff + t] = a[aoff + s]
        assert np.array_equal(host(d), expect)


# ------------------------------------------------------------------------------------------------
# fp16 KV cache: rope + append, attention


# Keys go to the 16 chunks in blocks of 32 (head_dim 64) or 16 (head_dim 128) consecutive rows,
# round-robin. Positions cover one key, block edges, the edges of a full lap of the chunks (512 or
# 256 rows), several rounds per lane (caches past one round's 4096 or 2048 rows) and the last row.
ATTN_CASES = [("0.5b", 2048, (0, 1, 31, 32, 63, 64, 255, 256, 257, 511, 512, 513, 1000, 1023, 1024, 1025, 2047)),
              ("7b", 2048, (0, 15, 16, 17, 255, 256, 257, 511, 512, 513, 2040, 2047)),
              ("0.5b", 8192, (4095, 8191)),
              ("7b", 8192, (5000, 8191))]


def attention_workspace(mh, torch, heads, kv, hd, max_seq):
    """A byte tensor of the size muyo_attention_decode_f16kv asks for (caller-owned partials)."""
    nbytes = mh.load().muyo_attention_decode_f16kv_workspace_bytes(heads, kv, hd, max_seq)
    assert nbytes > 0
    return torch.empty(nbytes, dtype=torch.uint8, device="cuda")


@pytest.mark.parametrize("shape,max_seq,positions", ATTN_CASES)
def test_rope_append_and_attention_f16kv(mh, gpu, orc, shape, max_seq, positions):
    torch = gpu
    heads, kv, hd = (14, 2, 64) if shape == "0.5b" else (28, 4, 128)
    ts = mh.theta_scale(1e6, hd)
    scale = 1.0 / math.sqrt(hd)
    kc = torch.empty(kv * max_seq * hd, dtype=torch.float16, device="cuda")
    vc = torch.empty_like(kc)
    mh.check(mh.load().muyo_fill_normal_f16(kc.data_ptr(), kc.numel(), 31, 0.0, 1.0, stream(torch)))
    mh.check(mh.load().muyo_fill_normal_f16(vc.data_ptr(), vc.numel(), 32, 0.0, 1.0, stream(torch)))
    for pos in positions:
        q = orc.normal_f32(heads * hd, 100 + pos)
        k = orc.normal_f32(kv * hd, 200 + pos)
        v = orc.normal_f32(kv * hd, 300 + pos)
        qd, kd, vd = dev(torch, q), dev(torch, k), dev(torch, v)
        pd = dev(torch, np.array([pos], np.int32))
        qr = torch.empty_like(qd)
        out = torch.empty_like(qd)
        lib = mh.load()
        mh.check(lib.muyo_rope_append_f16kv(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), qr.data_ptr(), kc.data_ptr(),
                                            vc.data_ptr(), pd.data_ptr(), heads, kv, hd, max_seq, ts, stream(torch)))
        ws = attention_workspace(mh, torch, heads, kv, hd, max_seq)
        run(mh, torch, lib.muyo_attention_decode_f16kv(qr.data_ptr(), kc.data_ptr(), vc.data_ptr(), out.data_ptr(),
                                                       pd.data_ptr(), heads, kv, hd, max_seq, scale, ws.data_ptr(),
                                                       ws.numel(), stream(torch)))
        kbits = host(kc.view(torch.int16)).view(np.uint16).reshape(kv, max_seq, hd)
        vbits = host(vc.view(torch.int16)).view(np.uint16).reshape(kv, max_seq, hd)
        # Appended rows: k roped, v as is, rounded to fp16 (bit-exact slots).
        k_expect = orc.rope_neox(k.reshape(kv, hd), pos, ts)
        assert close(orc.half_to_float(kbits[:, pos]), k_expect, 1e-3) == 0
        assert np.array_equal(vbits[:, pos], orc.float_to_half(v.reshape(kv, hd)))
        q_expect = orc.rope_neox(q.reshape(heads, hd), pos, ts).reshape(-1)
        assert close(host(qr), q_expect, 1e-3) == 0
        expect = orc.attention_f16kv(host(qr), kbits, vbits, heads, kv, hd, max_seq, pos, scale)
        assert close(host(out), expect, 1e-3) == 0, f"pos {pos}"
        assert worst(host(out), expect) < 1e-5


@pytest.mark.parametrize("shape", ["0.5b", "7b"])
def test_attention_ignores_rows_past_the_position(mh, gpu, orc, shape):
    """The first round of K/V rows is requested before the position is read, so it covers rows past
    the position too; those rows (here NaN and infinity) must not reach the output."""
    torch = gpu
    heads, kv, hd = (14, 2, 64) if shape == "0.5b" else (28, 4, 128)
    max_seq = 2048
    scale = 1.0 / math.sqrt(hd)
    lib = mh.load()
    for pos in (0, 5, 40, 700, 2046):
        kc = torch.empty(kv * max_seq * hd, dtype=torch.float16, device="cuda")
        vc = torch.empty_like(kc)
        mh.check(lib.muyo_fill_normal_f16(kc.data_ptr(), kc.numel(), 41, 0.0, 1.0, stream(torch)))
        mh.check(lib.muyo_fill_normal_f16(vc.data_ptr(), vc.numel(), 42, 0.0, 1.0, stream(torch)))
        kc.view(kv, max_seq, hd)[:, pos + 1:] = float("nan")
        vc.view(kv, max_seq, hd)[:, pos + 1:, ::2] = float("inf")
        vc.view(kv, max_seq, hd)[:, pos + 1:, 1::2] = float("nan")
        q = orc.normal_f32(heads * hd, 500 + pos)
        qd = dev(torch, q)
        pd = dev(torch, np.array([pos], np.int32))
        out = torch.empty_like(qd)
        ws = attention_workspace(mh, torch, heads, kv, hd, max_seq)
        run(mh, torch, lib.muyo_attention_decode_f16kv(qd.data_ptr(), kc.data_ptr(), vc.data_ptr(), out.data_ptr(),
                                                       pd.data_ptr(), heads, kv, hd, max_seq, scale, ws.data_ptr(),
                                                       ws.numel(), stream(torch)))
        kbits = host(kc.view(torch.int16)).view(np.uint16).reshape(kv, max_seq, hd)
        vbits = host(vc.view(torch.int16)).view(np.uint16).reshape(kv, max_seq, hd)
        expect = orc.attention_f16kv(q, kbits, vbits, heads, kv, hd, max_seq, pos, scale)
        got = host(out)
        assert np.isfinite(got).all(), f"pos {pos}"
        assert close(got, expect, 1e-3) == 0, f"pos {pos}"


def test_attention_workspace_sizes_and_refusals(mh, gpu, orc):
    """The workspace grows with the cache's chunk count and the group; a short workspace, a null one
    and unsupported shapes are refused before anything is launched. A small cache and then a
    larger one through workspaces of their own sizes both match the oracle."""
    torch = gpu
    lib = mh.load()
    small = lib.muyo_attention_decode_f16kv_workspace_bytes(14, 2, 64, 64)
    large = lib.muyo_attention_decode_f16kv_workspace_bytes(14, 2, 64, 4096)
    assert 0 < small < large == 2 * 16 * 7 * (2 + 64) * 4
    assert lib.muyo_attention_decode_f16kv_workspace_bytes(14, 3, 64, 64) == 0
    assert lib.muyo_attention_decode_f16kv_workspace_bytes(14, 2, 96, 64) == 0
    heads, kv, hd = 14, 2, 64
    scale = 1.0 / math.sqrt(hd)
    for max_seq, pos in ((64, 40), (4096, 3000)):
        kc = torch.empty(kv * max_seq * hd, dtype=torch.float16, device="cuda")
        vc = torch.empty_like(kc)
        mh.check(lib.muyo_fill_normal_f16(kc.data_ptr(), kc.numel(), 61, 0.0, 1.0, stream(torch)))
        mh.check(lib.muyo_fill_normal_f16(vc.data_ptr(), vc.numel(), 62, 0.0, 1.0, stream(torch)))
        q = orc.normal_f32(heads * hd, 600 + pos)
        qd = dev(torch, q)
        pd = dev(torch, np.array([pos], np.int32))
        out = torch.empty_like(qd)
        ws = attention_workspace(mh, torch, heads, kv, hd, max_seq)
        short = lib.muyo_attention_decode_f16kv(qd.data_ptr(), kc.data_ptr(), vc.data_ptr(), out.data_ptr(),
                                                pd.data_ptr(), heads, kv, hd, max_seq, scale, ws.data_ptr(),
                                                ws.numel() - 4, stream(torch))
        assert short == mh.MUYO_E_CONTRACT
        assert lib.muyo_attention_decode_f16kv(qd.data_ptr(), kc.data_ptr(), vc.data_ptr(), out.data_ptr(),
                                               pd.data_ptr(), heads, kv, hd, max_seq, scale, None, 0,
                                               stream(torch)) == mh.MUYO_E_CONTRACT
        run(mh, torch, lib.muyo_attention_decode_f16kv(qd.data_ptr(), kc.data_ptr(), vc.data_ptr(), out.data_ptr(),
                                                       pd.data_ptr(), heads, kv, hd, max_seq, scale, ws.data_ptr(),
                                                       ws.numel(), stream(torch)))
        kbits = host(kc.view(torch.int16)).view(np.uint16).reshape(kv, max_seq, hd)
        vbits = host(vc.view(torch.int16)).view(np.uint16).reshape(kv, max_seq, hd)
        expect = orc.attention_f16kv(q, kbits, vbits, heads, kv, hd, max_seq, pos, scale)
        assert close(host(out), expect, 1e-3) == 0, f"max_seq {max_seq}"


# ------------------------------------------------------------------------------------------------
# synthetic-input generator: device bits == oracle bits


def test_generator_matches_oracle_bits(mh, gpu, orc):
    torch = gpu
    n = 1_000_003
    h = torch.empty(n, dtype=torch.float16, device="cuda")
    f = torch.empty(n, dtype=torch.float32, device="cuda")
    u = torch.empty(n, dtype=torch.float32, device="cuda")
    lib = mh.load()
    mh.check(lib.muyo_fill_normal_f16(h.data_ptr(), n, 5, 0.0, 0.02, stream(torch)))
    mh.check(lib.muyo_fill_normal_f32(f.data_ptr(), n, 6, 1.0, 0.1, stream(torch)))
    run(mh, torch, lib.muyo_fill_uniform_f32(u.data_ptr(), n, 7, stream(torch)))
    assert np.array_equal(host(h.view(torch.int16)).view(np.uint16), orc.normal_f16(n, 5, 0.0, 0.02))
    assert np.array_equal(host(f), orc.normal_f32(n, 6, 1.0, 0.1))
    assert np.array_equal(host(u), orc.uniform_f32(n, 7))
    assert mh.tensor_seed(1, "FFN_UP", 3) == orc.tensor_seed(1, "FFN_UP", 3)


# ------------------------------------------------------------------------------------------------
# the reference's node self-tests (RunX), through the C ABI and the muyo_llm CLI


@pytest.mark.parametrize("mode", ["--add", "--matvec", "--rmsnorm", "--rope", "--swiglu", "--getrows", "--argmax",
                                  "--softmax", "--attention", "--kvcache"])
def test_reference_self_tests(mh, gpu, mode):
    assert mh.load().muyo_self_test(mode.encode()) == 0


def test_self_test_cli_smoke(mh, gpu):
    import pathlib
    import subprocess

    cli = pathlib.Path(mh.__file__).resolve().parent / "muyo_llm"
    done = subprocess.run([str(cli), "--smoke"], capture_output=True, text=True, timeout=120)
    assert done.returncode == 0, done.stdout + done.stderr
    assert done.stdout.count("OK:") == 10
    assert mh.load().muyo_self_test(b"--nope") == mh.MUYO_E_RANGE
