"""The device sampler (muyo_sample_f32) against the sampler oracle, which restates
src/Sampler.cpp:10-100 and is itself pinned to the reference's Sampler.cpp (tests/test_sampler.py).

Same logits, history, parameters and seed: the token ids must be identical draw after draw, and the
logits the call leaves behind (penalised, divided by the temperature, in place as the reference
leaves its mapped logits) bit-identical. A draw could in principle differ where a cumulative
weight sits within a double rounding of the target, since the device's exp is not glibc's; no
case here comes near one.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


class DeviceSampler:
    def __init__(self, mh, torch, vocab, **params):
        self.mh, self.torch, self.vocab = mh, torch, vocab
        self.params = mh.sampler_params(**params)
        lib = mh.load()
        self.lib = lib
        self.state = torch.empty(lib.muyo_sampler_state_bytes(), dtype=torch.uint8, device="cuda")
        ws = lib.muyo_sample_workspace_bytes(vocab, mh.ref(self.params))
        assert ws > 0
        self.ws = torch.zeros(ws, dtype=torch.uint8, device="cuda")  # zero before the first use
        self.token = torch.empty(1, dtype=torch.int32, device="cuda")
        self.stream = torch.cuda.current_stream().cuda_stream
        mh.check(lib.muyo_sampler_seed(self.state.data_ptr(), self.params.seed, self.stream))

    def sample(self, logits: np.ndarray, history) -> tuple[int, np.ndarray]:
        torch = self.torch
        d = torch.from_numpy(logits.copy()).cuda()
        hist = torch.tensor(np.asarray(history, np.int32), dtype=torch.int32, device="cuda")
        self.mh.check(self.lib.muyo_sample_f32(d.data_ptr(), self.vocab, hist.data_ptr() if len(history) else None,
                                               len(history), self.mh.ref(self.params), self.state.data_ptr(),
                                               self.ws.data_ptr(), self.token.data_ptr(), self.stream))
        torch.cuda.synchronize()
        return int(self.token.item()), d.cpu().numpy()


CASES = [
    # vocab, temperature, top_k, top_p, penalty, last_n, std
    (1000, 0.8, 40, 0.95, 1.0, 64, 1.0),
    (1000, 1.0, 40, 0.95, 1.3, 64, 1.0),
    (1000, 0.7, 5, 1.0, 0.9, -1, 2.0),
    (1000, 1.5, 0, 0.9, 1.1, 0, 1.0),
    (1000, 0.0, 40, 0.95, 1.2, 16, 1.0),
    (7, 1.0, 100, 0.5, 1.0, 64, 0.5),
    (1, 1.0, 40, 0.95, 1.0, 64, 1.0),
    (4096, 1.0, 1024, 0.99, 1.05, 300, 1.0),
    (4097, 1.0, 1024, 1.0, 1.0, 64, 0.3),
    (151936, 0.9, 40, 0.95, 1.1, 64, 2.0),
    (151936, 1.2, 1024, 0.8, 1.0, 64, 1.5),
    (152064, 1.0, 1, 0.95, 1.0, 64, 1.0),
    (151936, 0.0, 40, 0.95, 1.3, -1, 1.0),
    (4097, 1.0, 256, 0.9, 1.0, 64, 1.0),     # empty slices: the collection takes every key and overflows
    (20000, 1.0, 256, 0.95, 1.2, 64, 1.0),   # k at the number of slice maxima
    (20000, 1.0, 257, 0.95, 1.0, 64, 1.0),   # one past: selection rounds only
    (600000, 0.9, 40, 0.95, 1.2, 64, 1.0),   # slices past the LDS counts: the separate penalty kernel
]


@pytest.mark.parametrize("case", CASES, ids=[f"v{c[0]}_t{c[1]}_k{c[2]}_p{c[3]}_r{c[4]}_n{c[5]}" for c in CASES])
def test_device_sampler_matches_oracle(mh, gpu, orc, case):
    vocab, temperature, top_k, top_p, penalty, last_n, std = case
    params = dict(temperature=temperature, top_k=top_k, top_p=top_p, repeat_penalty=penalty, repeat_last_n=last_n,
                  seed=vocab * 7 + 3)
    dev = DeviceSampler(mh, gpu, vocab, **params)
    ref = orc.Sampler(**params)
    rng = np.random.default_rng(vocab + 1)
    history = list(rng.integers(-2, vocab + 2, size=300))
    history += history[:40]
    for step in range(40):  # 40 draws: the engine twists once at the first draw
        logits = (rng.standard_normal(vocab) * std).astype(np.float32)
        got, after = dev.sample(logits, history)
        expect = logits.copy()
        want = ref.sample(expect, history)
        assert got == want, f"step {step}"
        assert np.array_equal(after, expect), f"step {step}: in-place logits differ"
        history.append(got)


def test_engine_stream_over_several_twists(mh, gpu, orc):
    """Two equal logits at temperature 1 and top-p 1: token 1 iff the draw u > 1/2, so 1000 draws
    (three twists of the 312-word state) trace the engine's stream against std::mt19937_64."""
    params = dict(temperature=1.0, top_k=2, top_p=1.0, repeat_penalty=1.0, seed=5489)
    dev = DeviceSampler(mh, gpu, 2, **params)
    got = [dev.sample(np.zeros(2, np.float32), [])[0] for _ in range(1000)]
    u = orc.mt64_uniform(5489, 1000)
    assert got == [int(2.0 * x > 1.0) for x in u]


def test_ties_go_to_the_lower_index(mh, gpu, orc):
    vocab = 50000
    logits = np.zeros(vocab, np.float32)
    logits[[40000, 7, 31337]] = 5.0  # three-way tie for the top; top-k 1 must pick index 7
    dev = DeviceSampler(mh, gpu, vocab, temperature=1.0, top_k=1, seed=1)
    assert dev.sample(logits, [])[0] == 7
    dev = DeviceSampler(mh, gpu, vocab, temperature=0.0, repeat_penalty=1.1, seed=1)
    assert dev.sample(logits, [5])[0] == 7


@pytest.mark.parametrize("tied", [151936, 5000])
def test_ties_at_the_top_overflow_the_collection(mh, gpu, orc, tied):
    """More than 4096 keys at the collection threshold (all logits equal, or 5000 tied at the top):
    the collection overflows and the final workgroup selects from every logit itself, still
    matching the oracle."""
    vocab = 151936
    params = dict(temperature=1.0, top_k=40, top_p=0.95, repeat_penalty=1.0, seed=3)
    dev = DeviceSampler(mh, gpu, vocab, **params)
    ref = orc.Sampler(**params)
    rng = np.random.default_rng(tied)
    logits = (rng.standard_normal(vocab) * 0.5 - 10.0).astype(np.float32)
    logits[rng.permutation(vocab)[:tied]] = 2.0
    for step in range(6):
        got, after = dev.sample(logits, [])
        expect = logits.copy()
        assert got == ref.sample(expect, []), f"step {step}"
        assert np.array_equal(after, expect)


def test_unsupported_configurations_are_refused(mh, gpu):
    lib = mh.load()
    state = gpu.empty(lib.muyo_sampler_state_bytes(), dtype=gpu.uint8, device="cuda")
    logits = gpu.zeros(151936, dtype=gpu.float32, device="cuda")
    token = gpu.empty(1, dtype=gpu.int32, device="cuda")
    for top_k in (0, 1025):
        p = mh.sampler_params(temperature=1.0, top_k=top_k)
        ws = gpu.zeros(1 << 20, dtype=gpu.uint8, device="cuda")
        status = lib.muyo_sample_f32(logits.data_ptr(), 151936, None, 0, mh.ref(p), state.data_ptr(), ws.data_ptr(),
                                     token.data_ptr(), 0)
        assert status == mh.MUYO_E_UNSUPPORTED, top_k
    p = mh.sampler_params(temperature=1.0)
    assert lib.muyo_sample_f32(None, 10, None, 0, mh.ref(p), state.data_ptr(), state.data_ptr(), token.data_ptr(),
                               0) == mh.MUYO_E_NULL


# ------------------------------------------------------------------------------------------------
# The decoder's sampling mode: Sampler::Sample after every step, on the device.

SAMPLE_SHAPE = dict(layers=2, hidden=256, ffn=512, heads=4, kv_heads=2, head_dim=64, vocab=5000, max_seq=256)
DECODER_PARAMS = [
    dict(temperature=0.8, top_k=40, top_p=0.95, repeat_penalty=1.1, repeat_last_n=64, seed=42),
    dict(temperature=1.3, top_k=1024, top_p=0.9, repeat_penalty=1.0, repeat_last_n=64, seed=7),
    dict(temperature=0.0, top_k=40, top_p=0.95, repeat_penalty=1.3, repeat_last_n=-1, seed=0),
]


def sampled_steps(mh, orc, shape, params, start, steps, seed):
    """Steps one at a time; each step's token against the oracle sampler fed that step's raw
    logits and the same history (prompt, then every token embedded since)."""
    rng = np.random.default_rng(seed)
    prompt = [int(t) for t in rng.integers(0, shape["vocab"], size=start)]
    with mh.Decoder(mh.qwen2_config(**shape)) as dec:
        dec.fill_random(seed)
        dec.fill_kv_random(start, seed + 1)
        dec.set_history(prompt)
        dec.set_sampler(**params)
        ref = orc.Sampler(**params)
        history, token, got_ids, want_ids = list(prompt), int(rng.integers(0, shape["vocab"])), [], []
        for i in range(steps):
            got = dec.step(token, start + i)
            logits = np.empty(shape["vocab"], np.float32)
            dec.download("LOGITS", 0, logits)
            history.append(token)
            want = ref.sample(logits, history)
            got_ids.append(got)
            want_ids.append(want)
            token = got
        return got_ids, want_ids


@pytest.mark.parametrize("params", DECODER_PARAMS, ids=["t0.8_k40_pen", "t1.3_k1024", "greedy_pen_all"])
def test_decoder_sampling_matches_oracle(mh, gpu, orc, params):
    got, want = sampled_steps(mh, orc, SAMPLE_SHAPE, params, start=60, steps=24, seed=5)
    assert got == want
    if params["temperature"] > 0:
        assert len(set(got)) > 1  # the draws are not degenerate


def test_decoder_05b_sampling_32_steps(mh, gpu, orc):
    """Qwen2.5-0.5B shape, cache pre-filled to 1024, 32 sampled tokens with the reference's usual
    sampling settings plus a penalty."""
    params = dict(temperature=0.7, top_k=40, top_p=0.95, repeat_penalty=1.1, repeat_last_n=64, seed=2026)
    got, want = sampled_steps(mh, orc, mh.QWEN25_05B, params, start=1024, steps=32, seed=2027)
    assert got == want


def test_decoder_sampling_graph_replay_matches_steps(mh, gpu, orc):
    """generate() (graph replay, the sampled token fed back on the device) == one step at a time,
    from the same seed and history."""
    params = dict(temperature=1.0, top_k=50, top_p=0.9, repeat_penalty=1.2, repeat_last_n=32, seed=9)
    prompt = list(range(3, 43))
    with mh.Decoder(mh.qwen2_config(**SAMPLE_SHAPE)) as dec:
        dec.fill_random(21)
        dec.fill_kv_random(40, 22)
        dec.set_history(prompt)
        dec.set_sampler(**params)
        ids = dec.generate(5, 40, 20)
        launches = dec.launches_per_step()
        dec.set_history(prompt)
        dec.set_sampler(**params)
        token, stepped = 5, []
        for i in range(20):
            token = dec.step(token, 40 + i)
            stepped.append(token)
        dec.set_sampler()
        greedy_launches = dec.launches_per_step()
    assert ids == stepped
    # Scale (with the penalty's counts and the slice maxima), the collection (5000 > 4096 keys)
    # and the final draw.
    assert launches == greedy_launches + 3
