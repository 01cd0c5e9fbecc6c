"""The persistent decode step (one cooperative launch per token, muyo_decoder_set_persistent)
against the CPU oracle and against the graph-replayed kernel sequence that computes the same step.

The bar is the decoder's: logits within 1e-3 (mixed form) of the oracle's, greedy ids identical,
the appended cache rows equal to the oracle's within fp16 rounding."""
import numpy as np
import pytest

from conftest import close, worst

pytestmark = pytest.mark.gpu

SMALL = dict(layers=2, hidden=256, ffn=512, heads=4, kv_heads=2, head_dim=64, vocab=1000, max_seq=256)
HD128 = dict(layers=1, hidden=512, ffn=1024, heads=8, kv_heads=1, head_dim=128, vocab=500, max_seq=300)


def make_pair(mh, orc, shape, seed, kv_positions=0, kv_seed=7):
    dec = mh.Decoder(mh.qwen2_config(**shape))
    dec.fill_random(seed)
    model = orc.Model(**shape)
    model.fill_random(seed)
    if kv_positions:
        dec.fill_kv_random(kv_positions, kv_seed)
        model.fill_kv_random(kv_positions, kv_seed)
    return dec, model


def logits_of(dec, vocab):
    out = np.empty(vocab, np.float32)
    dec.download("LOGITS", 0, out)
    return out


@pytest.mark.parametrize("shape", ["small", "hd128"])
def test_persistent_steps_match_oracle(mh, gpu, orc, capsys, shape):
    cfg = SMALL if shape == "small" else HD128
    start = 30 if shape == "small" else 290
    dec, model = make_pair(mh, orc, cfg, seed=11, kv_positions=start, kv_seed=12)
    with dec:
        dec.set_persistent(True)
        assert dec.persistent and dec.launches_per_step() == 1
        token = 17
        for i in range(6):
            pos = start + i
            with capsys.disabled():
                print(f"\n[persistent {shape}] step {i} pos {pos} token {token}", flush=True)
            got = dec.step(token, pos)
            want, logits, (top1, top2) = model.step(token, pos)
            gpu_logits = logits_of(dec, cfg["vocab"])
            assert close(gpu_logits, logits, 1e-3) == 0, f"step {i}: worst {worst(gpu_logits, logits):.3g}"
            assert got == want, f"step {i}: gpu {got} oracle {want} (margin {top1 - top2:.3g})"
            token = got
        for layer in range(cfg["layers"]):
            for kind in ("KCACHE", "VCACHE"):
                ref = model.t[(kind, layer)]
                cache = np.empty_like(ref)
                dec.download(kind, layer, cache)
                assert np.array_equal(cache[:, :start], ref[:, :start])
                assert np.array_equal(cache[:, start + 6:], ref[:, start + 6:])
                diff = np.abs(orc.half_to_float(cache[:, start:start + 6]) - orc.half_to_float(ref[:, start:start + 6]))
                assert diff.max() <= 2e-3 * (1 + np.abs(orc.half_to_float(ref[:, start:start + 6])).max())


def test_persistent_matches_graph_path(mh, gpu, orc):
    """generate() both ways from the same cache: the same greedy ids, close logits."""
    with mh.Decoder(mh.qwen2_config(**SMALL)) as dec:
        dec.fill_random(21)
        dec.fill_kv_random(10, 22)
        dec.set_persistent(True)
        fast = dec.generate(5, 10, 20)
        fast_logits = logits_of(dec, SMALL["vocab"])
        dec.fill_kv_random(10, 22)
        dec.set_persistent(False)
        assert dec.launches_per_step() > 1
        graph = dec.generate(5, 10, 20)
        graph_logits = logits_of(dec, SMALL["vocab"])
    assert fast == graph
    assert close(fast_logits, graph_logits, 1e-3) == 0


def test_persistent_refuses_unsupported_shapes(mh, gpu):
    wide = dict(layers=1, hidden=1536, ffn=8960, heads=12, kv_heads=2, head_dim=128, vocab=300, max_seq=40)
    with mh.Decoder(mh.qwen2_config(**wide)) as dec:
        assert not dec.persistent
        assert mh.load().muyo_decoder_set_persistent(dec.handle, 1) == mh.MUYO_E_UNSUPPORTED
        dec.set_persistent(False)


def test_persistent_05b_greedy_32_steps(mh, gpu, orc):
    """Qwen2.5-0.5B shape on the persistent step: 32 greedy ids equal to the oracle's from a cache
    pre-filled to row 1024."""
    orc.set_threads(16)
    shape = mh.QWEN25_05B
    dec, model = make_pair(mh, orc, shape, seed=2026, kv_positions=1024, kv_seed=2027)
    with dec:
        dec.set_persistent(True)
        ids = dec.generate(4321, 1024, 32)
    want, _ = model.greedy(4321, 1024, 32)
    assert ids == want


def test_persistent_arena_allocated_on_selection(mh, gpu, orc):
    """The step's own arena (the transposed FFN_DOWN of every layer, about 209 MB on the 0.5B shape)
    is allocated when the step is first selected, not at creation; weights written after selection
    reach the transposed copies."""
    torch = gpu
    shape = mh.QWEN25_05B
    down_t = shape["layers"] * (shape["ffn"] + 3) * shape["hidden"] * 2
    with mh.Decoder(mh.qwen2_config(**shape)) as dec:
        torch.cuda.synchronize()
        before, _ = torch.cuda.mem_get_info()
        dec.set_persistent(True)
        after, _ = torch.cuda.mem_get_info()
        assert before - after >= down_t, (before, after, down_t)
        dec.set_persistent(False)
        dec.set_persistent(True)  # the arena is kept, not allocated again
        assert torch.cuda.mem_get_info()[0] > after - down_t // 2
    dec, model = make_pair(mh, orc, SMALL, seed=5)
    with dec:
        dec.set_persistent(True)
        dec.fill_random(6)
        model.fill_random(6)
        dec.fill_kv_random(20, 7)
        model.fill_kv_random(20, 7)
        got = dec.step(9, 20)
        want, logits, _ = model.step(9, 20)
        assert close(logits_of(dec, SMALL["vocab"]), logits, 1e-3) == 0
        assert got == want
