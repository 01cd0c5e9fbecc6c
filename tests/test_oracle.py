"""Pins of the CPU oracle (CPU only).

Each oracle function is checked against something other than its own formula: the reference's
known-answer tests (src/*.cpp self-tests, transcribed), closed forms and invariants, float64
library routines (numpy, torch) and exhaustive/brute-force evaluation on small inputs.
"""
import math

import numpy as np
import pytest
import torch

from conftest import close, worst


# ------------------------------------------------------------------------------------------------
# binary16


def test_half_to_float_exhaustive(orc):
    bits = np.arange(65536, dtype=np.uint16)
    ours = orc.half_to_float(bits)
    lib = bits.view(np.float16).astype(np.float32)
    same = (ours.view(np.uint32) == lib.view(np.uint32)) | (np.isnan(ours) & np.isnan(lib))
    assert same.all()


def test_float_to_half_matches_numpy_rne(orc):
    rng = np.random.default_rng(7)
    patterns = rng.integers(0, 2**32, size=400_000, dtype=np.uint64).astype(np.uint32)
    values = patterns.view(np.float32)
    # Add every half value, the midpoints between neighbours (ties), and the overflow edge.
    halves = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float64)
    mids = ((halves[:-1] + halves[1:]) / 2).astype(np.float32)
    edges = np.array([65504, 65519.99, 65520, 65536, 2**-24, 2**-25, 3 * 2**-26, 1e-8, -0.0], np.float32)
    values = np.concatenate([values, halves.astype(np.float32), mids, -mids, edges])
    ours = orc.float_to_half(values)
    lib = values.astype(np.float16).view(np.uint16)
    nan = np.isnan(values)
    assert (ours[~nan] == lib[~nan]).all()
    assert ((ours[nan] & 0x7C00) == 0x7C00).all() and ((ours[nan] & 0x3FF) != 0).all()


# ------------------------------------------------------------------------------------------------
# generator


def test_generator_is_deterministic_and_seeded(orc):
    a = orc.normal_f32(10_000, 42)
    b = orc.normal_f32(10_000, 42)
    c = orc.normal_f32(10_000, 43)
    assert np.array_equal(a, b)
    assert not np.array_equal(a, c)


def test_generator_irwin_hall_moments(orc):
    n = 2_000_000
    x = orc.normal_f32(n, 1234).astype(np.float64)
    # Irwin-Hall(12) - 6: mean 0, variance 1, excess kurtosis -0.1, support [-6, 6].
    assert abs(x.mean()) < 5 / math.sqrt(n)
    assert abs(x.var() - 1.0) < 0.005
    kurt = ((x - x.mean()) ** 4).mean() / x.var() ** 2 - 3.0
    assert abs(kurt + 0.1) < 0.02
    assert np.abs(x).max() <= 6.0


def test_generator_f16_is_rounded_f32(orc):
    f = orc.normal_f32(50_000, 9, 0.0, 0.02)
    h = orc.normal_f16(50_000, 9, 0.0, 0.02)
    assert np.array_equal(h, f.astype(np.float16).view(np.uint16))


def test_uniform_range(orc):
    u = orc.uniform_f32(1_000_000, 5)
    assert u.min() >= -1.0 and u.max() < 1.0
    assert abs(u.mean()) < 0.005
    # Exactly k * 2^-23 - 1 for an integer k.
    k = (u.astype(np.float64) + 1.0) * 2**23
    assert np.array_equal(k, np.round(k))


def test_mix64_known_value(orc):
    # SplitMix64's first output from state 0 (Steele et al. reference sequence).
    assert orc.mix64(0) == 0xE220A8397B1DCDAF


# ------------------------------------------------------------------------------------------------
# GEMV


def test_mat_vec_reference_known_answer(orc):
    """src/MatVec.cpp:68-80,198-210: W = half((c%7)-3), x = (c%5)-2, exact."""
    rows, cols = 128, 256
    c = np.arange(cols)
    w = np.tile(((c % 7) - 3).astype(np.float16), (rows, 1))
    x = ((c % 5) - 2).astype(np.float32)
    y = orc.mat_vec_f16(w.view(np.uint16), x)
    exact = sum(int((k % 7) - 3) * int((k % 5) - 2) for k in range(cols))
    assert np.all(y == exact)


def test_mat_vec_matches_float64_matmul(orc):
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((300, 896)) * 0.02).astype(np.float16)
    x = rng.uniform(-1, 1, 896).astype(np.float32)
    expect = w.astype(np.float64) @ x.astype(np.float64)
    assert close(orc.mat_vec_f16(w.view(np.uint16), x), expect, 1e-5) == 0
    assert worst(orc.mat_vec_f16(w.view(np.uint16), x, f64acc=True), expect) < 1e-7
    wf = rng.standard_normal((64, 100)).astype(np.float32)
    assert close(orc.mat_vec_f32(wf, x[:100]), wf.astype(np.float64) @ x[:100], 1e-5) == 0


def test_mat_vec_detects_transposed_operand(orc):
    rng = np.random.default_rng(4)
    w = rng.standard_normal((64, 64)).astype(np.float16)
    x = rng.standard_normal(64).astype(np.float32)
    y = orc.mat_vec_f16(w.view(np.uint16), x)
    assert close(y, w.astype(np.float64).T @ x, 1e-3) > 0


# ------------------------------------------------------------------------------------------------
# rms_norm


def _rms_kat():
    rows, cols = 8, 512
    idx = np.arange(rows * cols).reshape(rows, cols)
    x = ((idx % 13) - 6).astype(np.float32)
    w = (0.5 + 0.001 * (np.arange(cols) % 11)).astype(np.float32)
    return x, w


def test_rms_norm_reference_known_answer(orc):
    """src/RmsNorm.cpp:60-72,194-216 inputs, checked with torch's float64 rms_norm."""
    x, w = _rms_kat()
    y = orc.rms_norm(x, w, 1e-6)
    lib = torch.nn.functional.rms_norm(torch.from_numpy(x).double(), (512,), torch.from_numpy(w).double(), eps=1e-6)
    assert close(y, lib.numpy(), 1e-6) == 0


def test_rms_norm_closed_forms(orc):
    # A constant row c: y = c / sqrt(c^2 + eps) * w. With c = 1e-3 and eps = 1e-6, 1/sqrt(2).
    x = np.full((1, 896), 1e-3, np.float32)
    y = orc.rms_norm(x, None, 1e-6)
    assert np.allclose(y, 1e-3 / math.sqrt(2e-6), rtol=1e-6)
    # Scale invariance away from eps, and unit RMS with w = 1.
    rng = np.random.default_rng(0)
    x = rng.standard_normal((16, 896)).astype(np.float32)
    y1 = orc.rms_norm(x, np.ones(896, np.float32), 0.0)
    y2 = orc.rms_norm(4.0 * x, np.ones(896, np.float32), 0.0)
    assert np.allclose(y1, y2, rtol=1e-6, atol=1e-7)
    assert np.allclose((y1.astype(np.float64) ** 2).mean(axis=1), 1.0, rtol=1e-5)


def test_rms_norm_f16_weight(orc):
    rng = np.random.default_rng(1)
    x = rng.standard_normal((32, 896)).astype(np.float32)
    w16 = (1.0 + 0.1 * rng.standard_normal(896)).astype(np.float16)
    y = orc.rms_norm(x, w16.view(np.uint16), 1e-6)
    lib = torch.nn.functional.rms_norm(torch.from_numpy(x).double(), (896,), torch.from_numpy(w16.astype(np.float64)),
                                       eps=1e-6)
    assert close(y, lib.numpy(), 1e-6) == 0


# ------------------------------------------------------------------------------------------------
# softmax


def test_soft_max_reference_known_answer(orc):
    """src/SoftMax.cpp:49-53,164-191: 64 columns, x = (c%9)-4, scale 1/8."""
    x = ((np.arange(64) % 9) - 4).astype(np.float32)[None, :]
    y = orc.soft_max(x, 0.125)
    lib = torch.softmax(torch.from_numpy(x).double() * 0.125, dim=-1).numpy()
    assert close(y, lib, 1e-6) == 0


def test_soft_max_invariants(orc):
    rng = np.random.default_rng(2)
    x = (3.0 * rng.standard_normal((14, 2048))).astype(np.float32)
    y = orc.soft_max(x, 1.0)
    assert np.allclose(y.astype(np.float64).sum(axis=1), 1.0, atol=1e-5)
    lib = torch.softmax(torch.from_numpy(x).double(), dim=-1).numpy()
    assert close(y, lib, 1e-6) == 0
    uniform = orc.soft_max(np.full((1, 100), 7.0, np.float32), 0.5)
    assert np.allclose(uniform, 0.01, rtol=1e-6)
    # A -1e30 masked tail contributes exactly zero (src/FullModel.cpp:63-66).
    masked = np.concatenate([x[:1, :10], np.full((1, 50), -1e30, np.float32)], axis=1)
    ym = orc.soft_max(masked, 0.125)
    assert np.all(ym[0, 10:] == 0.0)
    assert close(ym[0, :10], torch.softmax(torch.from_numpy(x[0, :10]).double() * 0.125, 0).numpy(), 1e-6) == 0


# ------------------------------------------------------------------------------------------------
# argmax


def test_argmax_reference_known_answer(orc):
    """src/Argmax.cpp:51-56,146: 32 logits -1 + 0.001i with [21] = 5 -> 21."""
    logits = (-1.0 + 0.001 * np.arange(32)).astype(np.float32)
    logits[21] = 5.0
    assert orc.argmax(logits) == 21


def test_argmax_ties_lowest_and_numpy(orc):
    x = np.zeros(1000, np.float32)
    x[[17, 400, 999]] = 3.0
    assert orc.argmax(x) == 17
    rng = np.random.default_rng(11)
    rows = rng.standard_normal((50, 151936)).astype(np.float32)
    assert np.array_equal(orc.argmax_rows(rows), np.argmax(rows, axis=1))


# ------------------------------------------------------------------------------------------------
# add, swiglu


def test_add_reference_known_answer_and_bit_exact(orc):
    """src/ElementwiseAdd.cpp:95-99,204-215: A = 0.5i, B = 1 + 0.25i, exact."""
    i = np.arange(1000, dtype=np.float32)
    d = orc.add(0.5 * i, 1.0 + 0.25 * i)
    assert np.array_equal(d, (1.0 + 0.75 * i).astype(np.float32))
    rng = np.random.default_rng(5)
    a = rng.standard_normal(10_000).astype(np.float32)
    b = rng.standard_normal(10_000).astype(np.float32)
    assert np.array_equal(orc.add(a, b), a + b)


def test_swiglu_reference_known_answer(orc):
    """src/Swiglu.cpp:61-67,185-196: gate 0.01((i%17)-8), up 0.5 + 0.01(i%7)."""
    i = np.arange(600)
    g = (0.01 * ((i % 17) - 8)).astype(np.float32)
    u = (0.5 + 0.01 * (i % 7)).astype(np.float32)
    d = orc.swiglu(g, u)
    lib = (torch.nn.functional.silu(torch.from_numpy(g).double()) * torch.from_numpy(u).double()).numpy()
    assert close(d, lib, 1e-6) == 0
    assert orc.swiglu(np.zeros(4, np.float32), np.ones(4, np.float32)).tolist() == [0.0] * 4
    big = orc.swiglu(np.array([30.0], np.float32), np.array([2.0], np.float32))
    assert abs(big[0] - 60.0) < 1e-5


# ------------------------------------------------------------------------------------------------
# rope


def _rope_complex(x, pos, theta_scale):
    """NeoX rope as a complex rotation (x_j + i x_{j+h}) * e^{i pos theta_scale^j}, float64."""
    x = np.asarray(x, np.float64)
    h = x.shape[-1] // 2
    j = np.arange(h)
    theta = pos * np.power(np.float64(theta_scale), j)
    z = (x[..., :h] + 1j * x[..., h:]) * np.exp(1j * theta)
    return np.concatenate([z.real, z.imag], axis=-1)


def test_rope_reference_known_answer(orc):
    """src/Rope.cpp:55-64,191-214: nDims 8, pos 3, base 1e4, x = c - 3."""
    ts = np.float32(10000.0) ** (np.float32(-2.0) / np.float32(8))
    x = (np.arange(8) - 3).astype(np.float32)[None, :]
    y = orc.rope_neox(x, 3, float(ts))
    assert close(y, _rope_complex(x, 3, float(ts)), 1e-5) == 0


def test_rope_invariants(orc):
    rng = np.random.default_rng(6)
    ts = float(np.float32(1e6) ** (np.float32(-2.0) / np.float32(64)))
    x = rng.standard_normal((16, 64)).astype(np.float32)
    assert np.array_equal(orc.rope_neox(x, 0, ts), x)  # pos 0 is the identity
    for pos in (1, 777, 2047):
        y = orc.rope_neox(x, pos, ts)
        assert close(y, _rope_complex(x, pos, ts), 1e-3) == 0
        # Each (j, j + 32) pair keeps its norm.
        n0 = x[:, :32] ** 2 + x[:, 32:] ** 2
        n1 = y[:, :32].astype(np.float64) ** 2 + y[:, 32:].astype(np.float64) ** 2
        assert np.allclose(n0, n1, rtol=1e-5, atol=1e-6)
    # Partial rotation copies the channels past n_dims.
    yp = orc.rope_neox(x, 5, ts, n_dims=32)
    assert np.array_equal(yp[:, 32:], x[:, 32:])


# ------------------------------------------------------------------------------------------------
# get_rows


def test_get_rows_known_answer(orc):
    """src/GetRows.cpp:49-56,179-182 pattern (token 7, ((t%5)-2) + 0.001c), stored as fp16."""
    vocab, dim = 1024, 512
    t = np.arange(vocab)[:, None]
    c = np.arange(dim)[None, :]
    table = (((t % 5) - 2) + 0.001 * c).astype(np.float16)
    row = orc.get_rows_f16(table.view(np.uint16), 7)
    assert np.array_equal(row, table[7].astype(np.float32))


# ------------------------------------------------------------------------------------------------
# attention over fp16 caches


def _sdpa(q, k, v, heads, kv_heads, scale):
    """torch's float64 attention with GQA (head h reads kv head h // group)."""
    qt = torch.from_numpy(np.asarray(q, np.float64)).reshape(1, heads, 1, -1)
    kt = torch.from_numpy(np.asarray(k, np.float64))[None]
    vt = torch.from_numpy(np.asarray(v, np.float64))[None]
    out = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, scale=scale, enable_gqa=True)
    return out.reshape(-1).numpy()


def test_attention_reference_known_answer(orc):
    """src/Attention.cpp:79-105,253-294: head_dim 8, 16 keys of small integers."""
    hd, keys = 8, 16
    d = np.arange(hd)
    q = ((d % 5) - 2).astype(np.float32)
    kk = np.array([[((j + e) % 3) - 1 for e in range(hd)] for j in range(keys)], np.float16)
    vv = np.array([[((j * 2 + e) % 7) - 3 for e in range(hd)] for j in range(keys)], np.float16)
    max_seq = 20
    kc = np.zeros((1, max_seq, hd), np.float16)
    vc = np.zeros((1, max_seq, hd), np.float16)
    kc[0, :keys] = kk
    vc[0, :keys] = vv
    out = orc.attention_f16kv(q, kc.view(np.uint16), vc.view(np.uint16), 1, 1, hd, max_seq, keys - 1, 1 / math.sqrt(hd))
    lib = _sdpa(q, kk[None].astype(np.float64), vv[None].astype(np.float64), 1, 1, 1 / math.sqrt(hd))
    assert close(out, lib, 1e-6) == 0


def test_attention_gqa_and_closed_forms(orc):
    rng = np.random.default_rng(8)
    heads, kv, hd, max_seq, pos = 14, 2, 64, 64, 40
    q = rng.standard_normal(heads * hd).astype(np.float32)
    kc = rng.standard_normal((kv, max_seq, hd)).astype(np.float16)
    vc = rng.standard_normal((kv, max_seq, hd)).astype(np.float16)
    out = orc.attention_f16kv(q, kc.view(np.uint16), vc.view(np.uint16), heads, kv, hd, max_seq, pos, 0.125)
    lib = _sdpa(q, kc[:, : pos + 1].astype(np.float64), vc[:, : pos + 1].astype(np.float64), heads, kv, 0.125)
    assert close(out, lib, 1e-6) == 0
    # q = 0: uniform weights, the output is the mean of the value rows 0..pos.
    out0 = orc.attention_f16kv(np.zeros(heads * hd, np.float32), kc.view(np.uint16), vc.view(np.uint16), heads, kv,
                               hd, max_seq, pos, 0.125)
    mean = vc[:, : pos + 1].astype(np.float64).mean(axis=1)
    assert np.allclose(out0.reshape(heads, hd), np.repeat(mean, heads // kv, axis=0), atol=1e-6)
    # One key: the output is that value row.
    out1 = orc.attention_f16kv(q, kc.view(np.uint16), vc.view(np.uint16), heads, kv, hd, max_seq, 0, 0.125)
    assert np.allclose(out1.reshape(heads, hd), np.repeat(vc[:, 0].astype(np.float32), heads // kv, axis=0))


def test_kv_cache_reference_known_answer(orc):
    """src/KvCache.cpp:94-100,356-400: kvDim 16, query (d%5)-2, keys/values per token, rope base 1e4."""
    kvdim, max_seq = 16, 4
    ts = float(np.float32(10000.0) ** (np.float32(-2.0) / np.float32(kvdim)))
    query = ((np.arange(kvdim) % 5) - 2).astype(np.float32)
    kc = np.zeros((1, max_seq, kvdim), np.float16)
    vc = np.zeros((1, max_seq, kvdim), np.float16)
    keys, values = [], []
    for token in range(2):
        d = np.arange(kvdim)
        key = (((token * 3 + d) % 5) - 2).astype(np.float32)
        value = (((token + d) % 5) - 2).astype(np.float32)
        keys.append(_rope_complex(key, token, ts))
        values.append(value)
        kc[0, token] = orc.rope_neox(key[None], token, ts)[0].astype(np.float16)
        vc[0, token] = value.astype(np.float16)
        out = orc.attention_f16kv(query, kc.view(np.uint16), vc.view(np.uint16), 1, 1, kvdim, max_seq, token,
                                  1 / math.sqrt(kvdim))
        lib = _sdpa(query, np.array(keys)[None], np.array(values, np.float64)[None], 1, 1, 1 / math.sqrt(kvdim))
        # The cache stores fp16 keys; the reference stored f32 (tolerance 1e-4 there, 1e-3 here).
        assert close(out, lib, 1e-3) == 0


# ------------------------------------------------------------------------------------------------
# decode layer and step


def _torch_layer(m, layer, x, pos):
    """Independent float64 composition with torch library ops, for the oracle's decode layer."""
    f64 = torch.float64

    def t(name):
        arr = m.t[(name, layer)]
        if arr.dtype == np.uint16:
            return torch.from_numpy(arr.view(np.float16).astype(np.float64))
        return torch.from_numpy(arr.astype(np.float64))

    hd, heads, kv = m.head_dim, m.heads, m.kv_heads
    qdim, kvdim = heads * hd, kv * hd
    xt = torch.from_numpy(np.asarray(x, np.float64))
    xn = torch.nn.functional.rms_norm(xt, (m.hidden,), t("ATTN_NORM"), eps=m.eps)
    qkv = torch.nn.functional.linear(xn, t("ATTN_QKV"), t("ATTN_QKV_B"))
    q, k, v = qkv[:qdim], qkv[qdim: qdim + kvdim], qkv[qdim + kvdim:]
    ts = float(np.float32(m.rope_base) ** (np.float32(-2.0) / np.float32(hd)))
    qr = torch.from_numpy(_rope_complex(q.numpy().reshape(heads, hd), pos, ts))
    kr = torch.from_numpy(_rope_complex(k.numpy().reshape(kv, hd), pos, ts))
    kc = torch.from_numpy(m.t[("KCACHE", layer)].view(np.float16).astype(np.float64)).clone()
    vc = torch.from_numpy(m.t[("VCACHE", layer)].view(np.float16).astype(np.float64)).clone()
    kc[:, pos] = kr.to(torch.float16).to(f64)
    vc[:, pos] = v.reshape(kv, hd).to(torch.float16).to(f64)
    att = torch.nn.functional.scaled_dot_product_attention(
        qr.reshape(1, heads, 1, hd), kc[None, :, : pos + 1], vc[None, :, : pos + 1], scale=1 / math.sqrt(hd),
        enable_gqa=True).reshape(qdim)
    x1 = xt + torch.nn.functional.linear(att, t("ATTN_OUTPUT"))
    xn2 = torch.nn.functional.rms_norm(x1, (m.hidden,), t("FFN_NORM"), eps=m.eps)
    act = torch.nn.functional.silu(torch.nn.functional.linear(xn2, t("FFN_GATE"))) * torch.nn.functional.linear(
        xn2, t("FFN_UP"))
    return (x1 + torch.nn.functional.linear(act, t("FFN_DOWN"))).numpy()


SMALL = dict(layers=2, hidden=128, ffn=256, heads=4, kv_heads=2, head_dim=32, vocab=500, max_seq=64)


def test_decode_layer_matches_torch_float64(orc):
    m = orc.Model(**SMALL)
    m.fill_random(21)
    m.fill_kv_random(10, 22)
    x = orc.normal_f32(SMALL["hidden"], 99)
    # Scale the weights up so every term matters at the tolerance.
    for key, arr in m.t.items():
        if key[0] in ("ATTN_QKV", "ATTN_OUTPUT", "FFN_GATE", "FFN_UP", "FFN_DOWN"):
            arr[...] = (arr.view(np.float16).astype(np.float32) * 10).astype(np.float16).view(np.uint16)
    expect = _torch_layer(m, 0, x, 10)
    out = m.layer(0, x, 10)
    assert worst(out, expect) < 1e-4


def test_decode_layer_identity_without_projections(orc):
    m = orc.Model(**SMALL)
    m.fill_random(5)
    m.t[("ATTN_OUTPUT", 0)][...] = 0
    m.t[("FFN_DOWN", 0)][...] = 0
    x = orc.normal_f32(SMALL["hidden"], 6)
    assert np.array_equal(m.layer(0, x, 3), x)


def test_decode_step_appends_cache_rows(orc):
    m = orc.Model(**SMALL)
    m.fill_random(31)
    m.step(17, 5)
    for layer in range(SMALL["layers"]):
        kc = m.t[("KCACHE", layer)]
        assert np.any(kc[:, 5] != 0) and np.all(kc[:, :5] == 0) and np.all(kc[:, 6:] == 0)


def test_decode_step_tied_head_and_greedy(orc):
    m = orc.Model(**SMALL)
    m.fill_random(41)
    best, logits, (top1, top2) = m.step(3, 0)
    assert best == int(np.argmax(logits)) and top1 == logits[best] and top1 >= top2
    # The head is the embedding: a logit equals the embedding row dotted with the final hidden.
    emb = m.t[("TOKEN_EMBD", 0)].view(np.float16).astype(np.float64)
    assert np.linalg.matrix_rank(emb[:10]) == 10
    ids, margins = m.greedy(3, 1, 4)
    assert len(ids) == 4 and all(0 <= i < SMALL["vocab"] for i in ids) and all(g >= 0 for g in margins)


def _torch_step(m, token, pos, final_norm=True, head="model"):
    """Independent float64 whole step for the oracle's decode step: embed, every layer through
    _torch_layer, output_norm, then the LM head (tools/reference_qwen2.py:160-166;
    src/FullModel.cpp:955-993: output.weight when the model has one, else the tied embedding).

    `final_norm=False` and `head="embedding"|"output"` plant the mistakes the pin must catch."""
    emb = m.t[("TOKEN_EMBD", 0)].view(np.float16).astype(np.float64)
    h = emb[token].copy()
    for layer in range(m.layers):
        h = _torch_layer(m, layer, h, pos)
    ht = torch.from_numpy(np.asarray(h, np.float64))
    if final_norm:
        w = torch.from_numpy(m.t[("OUTPUT_NORM", 0)].astype(np.float64))
        ht = torch.nn.functional.rms_norm(ht, (m.hidden,), w, eps=m.eps)
    if head == "model":
        head = "output" if m.untied_output else "embedding"
    table = m.t[("OUTPUT", 0)] if head == "output" else m.t[("TOKEN_EMBD", 0)]
    table = torch.from_numpy(table.view(np.float16).astype(np.float64))
    return torch.nn.functional.linear(ht, table).numpy()


def _scaled_model(orc, seed, untied):
    m = orc.Model(**SMALL, untied_output=untied)
    m.fill_random(seed)
    m.fill_kv_random(12, seed + 1)
    # Larger projections so every layer term, the final norm and the head all move the logits
    # well past the tolerance.
    for key, arr in m.t.items():
        if key[0] in ("ATTN_QKV", "ATTN_OUTPUT", "FFN_GATE", "FFN_UP", "FFN_DOWN", "TOKEN_EMBD", "OUTPUT"):
            arr[...] = (arr.view(np.float16).astype(np.float32) * 10).astype(np.float16).view(np.uint16)
    return m


@pytest.mark.parametrize("untied", [False, True])
def test_decode_step_logits_match_torch_float64(orc, untied):
    """oracle_decode_step's logits against the float64 composition, tied and untied heads; the
    same comparison must fail with the final norm dropped and with the other head table."""
    m = _scaled_model(orc, 51 + int(untied), untied)
    token, pos = 7, 12
    expect = _torch_step(m, token, pos)
    no_norm = _torch_step(m, token, pos, final_norm=False)
    other_head = _torch_step(m, token, pos, head="embedding") if untied else None
    best, logits, (top1, _) = m.step(token, pos)
    tol = 1e-4
    assert worst(logits, expect) < tol
    assert best == int(np.argmax(expect)) or expect[best] == expect.max()
    # Teeth: the planted mistakes each move the logits far past the tolerance.
    assert worst(logits, no_norm) > 100 * tol
    if other_head is not None:
        assert worst(logits, other_head) > 100 * tol
    # The tied model's head is the embedding; a layer norm weight in place of output_norm fails.
    if not untied:
        saved = m.t[("OUTPUT_NORM", 0)].copy()
        m.t[("OUTPUT_NORM", 0)][...] = m.t[("ATTN_NORM", 0)]
        wrong = _torch_step(m, token, pos)
        m.t[("OUTPUT_NORM", 0)][...] = saved
        assert worst(logits, wrong) > 100 * tol


def test_decode_step_two_positions_carry_the_cache(orc):
    """Two consecutive oracle steps: the second attends over the row the first appended, as the
    float64 composition does when fed the same cache."""
    m = _scaled_model(orc, 61, False)
    m.step(5, 12)  # appends row 12 in every layer
    expect = _torch_step(m, 9, 13)
    _, logits, _ = m.step(9, 13)
    assert worst(logits, expect) < 1e-4


@pytest.mark.parametrize("untied", [False, True])
def test_f32_reference_path_step_matches_float64(orc, untied):
    """oracle_decode_step_f32 (the reference's CPU path: f32 running sums in index order, the
    timed CPU baseline) against the float64 composition: logits within f32 summation error, the
    same greedy id, the same cache rows as the checker's step, and no dependence on the thread
    count (each sum is one thread's loop). Dropping the final norm moves it far outside."""
    m = _scaled_model(orc, 71 + int(untied), untied)
    twin = _scaled_model(orc, 71 + int(untied), untied)
    token, pos = 11, 12
    expect = _torch_step(m, token, pos)
    orc.set_threads(1)
    best, logits = m.step_f32(token, pos)
    tol = 1e-3
    assert worst(logits, expect) < tol
    assert best == int(np.argmax(logits)) and expect[best] >= np.sort(expect)[-2]
    assert worst(logits, _torch_step(m, token, pos, final_norm=False)) > 100 * tol
    twin.step(token, pos)
    for layer in range(SMALL["layers"]):
        for kind in ("KCACHE", "VCACHE"):
            got = orc.half_to_float(m.t[(kind, layer)][:, pos])
            ref = orc.half_to_float(twin.t[(kind, layer)][:, pos])
            assert np.max(np.abs(got - ref)) <= 2e-3 * (1 + np.abs(ref).max())
    orc.set_threads(4)
    again = _scaled_model(orc, 71 + int(untied), untied)
    best4, logits4 = again.step_f32(token, pos)
    orc.set_threads(1)
    assert best4 == best and np.array_equal(logits4, logits)
