"""Decode-step parity on the GPU: the fused, graph-replayed decoder against the CPU oracle.

Both sides draw every weight and the pre-filled KV cache from the same portable generator, so
they start from identical bits (checked). The bar: greedy token ids identical over 32 steps on
the Qwen2.5-0.5B shape, per-step logits within 1e-3 (mixed form), cache rows bit-exact in place.
"""
import numpy as np
import pytest

from conftest import close, worst

pytestmark = pytest.mark.gpu

SMALL = dict(layers=2, hidden=256, ffn=512, heads=4, kv_heads=2, head_dim=64, vocab=1000, max_seq=256)


def make_pair(mh, orc, shape, seed, kv_positions=0, kv_seed=7):
    cfg = mh.qwen2_config(**shape)
    dec = mh.Decoder(cfg)
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


def test_decoder_weights_match_oracle_bits(mh, gpu, orc):
    dec, model = make_pair(mh, orc, SMALL, seed=3, kv_positions=100, kv_seed=4)
    with dec:
        for (kind, layer), arr in model.t.items():
            assert np.array_equal(download(dec, kind, layer, arr), arr), (kind, layer)


@pytest.mark.parametrize("untied", [False, True], ids=["tied", "untied"])
def test_decoder_small_steps_match_oracle(mh, gpu, orc, untied):
    """12 steps fed back token by token. With the LM head tied to the embedding, a model this small
    maps a token back to itself (17 at every step); the untied head makes the ids change, so the
    token path (embedding row, rope position, cache rows of a new token) is exercised too."""
    shape = dict(SMALL, untied_output=untied)
    dec, model = make_pair(mh, orc, shape, seed=11, kv_positions=30, kv_seed=12)
    with dec:
        token = 17
        seen = []
        for i in range(12):
            pos = 30 + i
            got = dec.step(token, pos)
            want, logits, (top1, top2) = model.step(token, pos)
            gpu_logits = download(dec, "LOGITS", 0, np.empty(SMALL["vocab"], np.float32))
            assert close(gpu_logits, logits, 1e-3) == 0, f"step {i}"
            assert worst(gpu_logits, logits) < 1e-4
            assert got == want, f"step {i}: gpu {got} oracle {want} (margin {top1 - top2:.3g})"
            token = got
            seen.append(got)
        if untied:
            assert len(set(seen)) > 3, seen
        # The appended cache rows hold the same fp16 values (bit-exact up to last-bit rounding).
        for layer in range(SMALL["layers"]):
            for kind in ("KCACHE", "VCACHE"):
                ref = model.t[(kind, layer)]
                got_cache = download(dec, kind, layer, ref)
                assert np.array_equal(got_cache[:, :30], ref[:, :30])
                assert np.array_equal(got_cache[:, 42:], ref[:, 42:])
                diff = np.abs(orc.half_to_float(got_cache[:, 30:42]) - orc.half_to_float(ref[:, 30:42]))
                assert diff.max() <= 2e-3 * (1 + np.abs(orc.half_to_float(ref[:, 30:42])).max())


def test_fused_ffn_follows_new_down_weights(mh, gpu, orc):
    """On a decoder whose feed-forward block is one launch (hidden 256), that launch reads its own
    transposed copy of the down weights. New down weights, uploaded or written through the
    tensor's device pointer, are picked up by the next step: the logits follow the oracle on the
    new weights (std 0.05 instead of 0.02, far past the 1e-3 bar had the old copy been read)."""
    dec, model = make_pair(mh, orc, SMALL, seed=51, kv_positions=20, kv_seed=52)
    shape = (SMALL["hidden"], SMALL["ffn"])
    state = {"token": 5, "pos": 20}

    def check(label):
        for i in range(3):
            got = dec.step(state["token"], state["pos"])
            want, logits, _ = model.step(state["token"], state["pos"])
            gpu_logits = download(dec, "LOGITS", 0, np.empty(SMALL["vocab"], np.float32))
            assert close(gpu_logits, logits, 1e-3) == 0, f"{label} step {i}"
            assert got == want, f"{label} step {i}"
            state["token"], state["pos"] = got, state["pos"] + 1

    with dec:
        check("initial weights")
        new = orc.normal_f16(shape[0] * shape[1], 54, 0.0, 0.05).reshape(shape)
        model.t[("FFN_DOWN", 0)][...] = new
        dec.upload("FFN_DOWN", 0, np.ascontiguousarray(new))
        check("after an upload")
        ptr, nbytes = dec.tensor("FFN_DOWN", 0)
        assert mh.load().muyo_fill_normal_f16(ptr, nbytes // 2, 55, 0.0, 0.05, None) == 0
        gpu.cuda.synchronize()
        model.t[("FFN_DOWN", 0)][...] = orc.normal_f16(shape[0] * shape[1], 55, 0.0, 0.05).reshape(shape)
        check("after a write through the pointer")


# Shapes off the two Qwen sizes: a full GQA group of 8 with head_dim 128 (q dim 1024, merged in
# o_proj), q dims past 1024 (o_proj split by kv group: four groups of 5 heads at head_dim 64, two
# of 6 at 128), eight kv heads (more group parts than gate/up's prologue adds up: a separate merge
# kernel), odd cache lengths and rows at the end of the cache.
ODD_SHAPES = {
    "group8_hd128": (dict(layers=1, hidden=512, ffn=1024, heads=8, kv_heads=1, head_dim=128, vocab=500,
                          max_seq=300), 296),
    "qdim1280_hd64": (dict(layers=2, hidden=640, ffn=1792, heads=20, kv_heads=4, head_dim=64, vocab=700,
                           max_seq=333), 329),
    "hidden_1536_short_cache": (dict(layers=1, hidden=1536, ffn=8960, heads=12, kv_heads=2, head_dim=128,
                                     vocab=300, max_seq=40), 36),
    "kv8_merge_kernel": (dict(layers=2, hidden=512, ffn=1024, heads=16, kv_heads=8, head_dim=128, vocab=400,
                              max_seq=200), 150),
    # The grouped o_proj's rows per wave (ceil(hidden / (2 * CUs * 4 waves / kv heads)) on a
    # 256-CU part): 1, 4 and 8 rows, beside the 2 of qdim1280_hd64 and 7 of the 7B shape.
    "grouped_rows1": (dict(layers=1, hidden=512, ffn=768, heads=20, kv_heads=4, head_dim=64, vocab=300,
                           max_seq=96), 90),
    "grouped_rows4": (dict(layers=1, hidden=2048, ffn=1024, heads=32, kv_heads=4, head_dim=64, vocab=300,
                           max_seq=96), 64),
    "grouped_rows8": (dict(layers=1, hidden=4096, ffn=1024, heads=32, kv_heads=4, head_dim=128, vocab=300,
                           max_seq=64), 60),
    # Normed rows wider than one wave stages (3584 floats) with few enough units (2048 gate/up
    # rows, 2000 LM-head rows) for single-wave workgroups: those GEMVs keep 256-thread ones.
    "wide_rows_few_units": (dict(layers=1, hidden=3584, ffn=2048, heads=28, kv_heads=4, head_dim=128,
                                 vocab=2000, max_seq=64), 40),
    # Long caches: attention rounds past the first (which covers 2048 rows), 128 key blocks per
    # chunk merged in o_proj at head_dim 64, 64 per chunk over 16 chunks merged per kv group.
    "long_cache_32k_hd64": (dict(layers=1, hidden=256, ffn=512, heads=4, kv_heads=2, head_dim=64, vocab=300,
                                 max_seq=32768), 32760),
    "long_cache_16k_grouped_hd128": (dict(layers=1, hidden=512, ffn=512, heads=12, kv_heads=4, head_dim=128,
                                          vocab=300, max_seq=16384), 16000),
}


# Launches per greedy step: embed + LM head, and five kernels a layer (six with a merge kernel);
# with a hidden size of at most 1024 and o_proj not split by kv group, gate/up and down are one
# launch in every layer but the last.
ODD_LAUNCHES = {"group8_hd128": 2 + 5, "qdim1280_hd64": 2 + 5 * 2, "hidden_1536_short_cache": 2 + 5,
                "kv8_merge_kernel": 2 + 6 * 2 - 1, "grouped_rows1": 2 + 5, "grouped_rows4": 2 + 5,
                "grouped_rows8": 2 + 5, "wide_rows_few_units": 2 + 5, "long_cache_32k_hd64": 2 + 5,
                "long_cache_16k_grouped_hd128": 2 + 5}


@pytest.mark.parametrize("name", sorted(ODD_SHAPES))
def test_decoder_odd_shapes_match_oracle(mh, gpu, orc, name):
    shape, start = ODD_SHAPES[name]
    dec, model = make_pair(mh, orc, shape, seed=31, kv_positions=start, kv_seed=32)
    with dec:
        assert dec.launches_per_step() == ODD_LAUNCHES[name]
        token = 3
        for i in range(4):
            got = dec.step(token, start + i)
            want, logits, _ = model.step(token, start + i)
            gpu_logits = download(dec, "LOGITS", 0, np.empty(shape["vocab"], np.float32))
            assert close(gpu_logits, logits, 1e-3) == 0, f"{name} step {i}"
            assert got == want
            token = got


def test_decoder_graph_replay_matches_eager_steps(mh, gpu, orc):
    """generate() (one hipGraph launch per token, ids fed back on the device) == step-by-step, with
    an untied LM head so the ids change from step to step."""
    cfg = mh.qwen2_config(**SMALL, untied_output=True)
    with mh.Decoder(cfg) as dec:
        dec.fill_random(21)
        dec.fill_kv_random(10, 22)
        ids = dec.generate(5, 10, 20)
        dec.fill_kv_random(10, 22)
        again = dec.generate(5, 10, 20)
        dec.fill_kv_random(10, 22)
        token, stepped = 5, []
        for i in range(20):
            token = dec.step(token, 10 + i)
            stepped.append(token)
    assert ids == again == stepped
    assert len(set(ids)) > 1, ids


@pytest.mark.parametrize("position", [128, 1024, 2016])
def test_decoder_05b_greedy_32_steps(mh, gpu, orc, capsys, position):
    """Qwen2.5-0.5B shape, KV pre-filled to p, 32 greedy tokens from a seeded random id (p = 2016
    ends at cache row 2047, the last of a 2048-row cache)."""
    orc.set_threads(16)
    shape = mh.QWEN25_05B
    dec, model = make_pair(mh, orc, shape, seed=2026, kv_positions=position, kv_seed=2027)
    start = int(orc.uniform_f32(1, 99)[0] * 0.5 * shape["vocab"] + 0.5 * shape["vocab"])
    with dec:
        ids = dec.generate(start, position, 32)
    want, margins = model.greedy(start, position, 32)
    with capsys.disabled():
        print(f"\n[0.5b greedy p={position}] start {start} ids {ids[:8]}... min top1-top2 margin {min(margins):.3g}")
    assert ids == want


def test_decoder_05b_greedy_across_the_short_attention_grid(mh, gpu, orc, capsys):
    """Qwen2.5-0.5B shape from cache row 1000: 48 greedy tokens, the first 24 on the short
    attention grid (4 chunks while the position is below 1024), the rest on the long one (8
    chunks), replayed from the two graphs in turn, against the oracle."""
    orc.set_threads(16)
    shape = mh.QWEN25_05B
    position = 1000
    dec, model = make_pair(mh, orc, shape, seed=2031, kv_positions=position, kv_seed=2032)
    start = int(orc.uniform_f32(1, 98)[0] * 0.5 * shape["vocab"] + 0.5 * shape["vocab"])
    with dec:
        ids = dec.generate(start, position, 48)
    want, margins = model.greedy(start, position, 48)
    with capsys.disabled():
        print(f"\n[0.5b greedy p={position} across grids] ids {ids[20:28]}... min margin {min(margins):.3g}")
    assert ids == want


@pytest.mark.parametrize("position", [1024, 2047])
def test_decoder_05b_single_step_long_cache(mh, gpu, orc, position):
    orc.set_threads(16)
    shape = mh.QWEN25_05B
    dec, model = make_pair(mh, orc, shape, seed=7, kv_positions=position, kv_seed=8)
    with dec:
        got = dec.step(151643, position)
        want, logits, _ = model.step(151643, position)
        gpu_logits = download(dec, "LOGITS", 0, np.empty(shape["vocab"], np.float32))
    assert close(gpu_logits, logits, 1e-3) == 0
    assert got == want


def test_decoder_7b_shape_two_layers(mh, gpu, orc):
    """Qwen2.5-7B widths (hidden 3584, ffn 18944, 28/4 heads, head_dim 128, vocab 152064), 2 layers."""
    orc.set_threads(16)
    shape = dict(mh.QWEN25_7B, layers=2)
    dec, model = make_pair(mh, orc, shape, seed=70, kv_positions=2040, kv_seed=71)
    with dec:
        ids = dec.generate(1000, 2040, 8)
        gpu_logits = download(dec, "LOGITS", 0, np.empty(shape["vocab"], np.float32))
    token, want = 1000, []
    for i in range(8):
        token, logits, _ = model.step(token, 2040 + i)
        want.append(token)
    assert ids == want
    assert close(gpu_logits, logits, 1e-3) == 0  # the last step, at cache row 2047


@pytest.mark.timeout(900)
def test_decoder_7b_shape_full_depth(mh, gpu, orc, capsys):
    """Every layer of the Qwen2.5-7B shape (28 layers, a ~14.3 GB arena with tensors past 4 GiB),
    two greedy steps at cache rows 2046 and 2047 (the last of a 2048-row cache): ids equal and each
    step's logits within 1e-3 of the oracle's."""
    orc.set_threads(16)
    shape = mh.QWEN25_7B
    dec, model = make_pair(mh, orc, shape, seed=77, kv_positions=2046, kv_seed=78)
    token = 4242
    with dec:
        for pos in (2046, 2047):
            got = dec.step(token, pos)
            gpu_logits = download(dec, "LOGITS", 0, np.empty(shape["vocab"], np.float32))
            want, logits, (top1, top2) = model.step(token, pos)
            with capsys.disabled():
                print(f"\n[7b full depth p={pos}] token {token} -> gpu {got} oracle {want} "
                      f"worst {worst(gpu_logits, logits):.2e} margin {top1 - top2:.3g}", flush=True)
            assert close(gpu_logits, logits, 1e-3) == 0, f"p={pos}"
            assert got == want, f"p={pos}"
            token = got


def test_decoder_rejects_out_of_range(mh, gpu):
    cfg = mh.qwen2_config(**SMALL)
    with mh.Decoder(cfg) as dec:
        lib = mh.load()
        assert lib.muyo_decoder_generate_async(dec.handle, SMALL["vocab"], 0, 1, 0) == mh.MUYO_E_RANGE
        assert lib.muyo_decoder_generate_async(dec.handle, 0, SMALL["max_seq"] - 2, 3, 0) == mh.MUYO_E_RANGE
        assert lib.muyo_decoder_generate_async(dec.handle, 0, -1, 1, 0) == mh.MUYO_E_RANGE
        # Gate/up and down in one launch in every layer but the last (hidden 256).
        assert dec.launches_per_step() == 2 + 5 * SMALL["layers"] - (SMALL["layers"] - 1)
