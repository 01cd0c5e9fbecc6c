"""The sampler oracle (oracle/sampler.cpp, restating src/Sampler.cpp:10-100), pinned on the CPU.

Pins, strongest first:
- the reference's own Sampler.cpp, compiled from the reference tree into oracle/_ref, drawing
  identical ids from identical logits, histories, parameters and seeds (skipped where the
  reference tree was absent when the oracle was built);
- the C++ standard's known answer for std::mt19937_64 ([rand.predef]: the 10000th output of a
  default-seeded engine is 9981545732273789042);
- closed forms: temperature <= 0 and top-k 1 are the greedy argmax; a top-p below the largest
  weight keeps one token; a token seen d times in the window is penalised d times in a row.
"""
import numpy as np
import pytest

import oracle

REF = oracle.Sampler.REF_PATH.exists()


def test_mt19937_64_known_answer():
    out = oracle.mt64_outputs(5489, 10000)
    assert int(out[-1]) == 9981545732273789042


def test_uniform_draws_in_unit_interval():
    u = oracle.mt64_uniform(7, 20000)
    assert u.min() >= 0.0 and u.max() < 1.0
    assert abs(u.mean() - 0.5) < 0.01


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
    (151936, 0.9, 40, 0.95, 1.1, 64, 2.0),
    (151936, 1.2, 1024, 0.8, 1.0, 64, 1.5),
]


@pytest.mark.skipif(not REF, reason="oracle/_ref/libref_sampler.so was not built (reference tree absent)")
@pytest.mark.parametrize("case", CASES, ids=[f"v{c[0]}_t{c[1]}_k{c[2]}_p{c[3]}_r{c[4]}_n{c[5]}" for c in CASES])
def test_restatement_matches_reference_sampler(case):
    vocab, temperature, top_k, top_p, penalty, last_n, std = case
    ours = oracle.Sampler(temperature, top_k, top_p, penalty, last_n, seed=vocab + 11)
    theirs = oracle.Sampler(temperature, top_k, top_p, penalty, last_n, seed=vocab + 11, ref=True)
    rng = np.random.default_rng(vocab)
    history = list(rng.integers(-2, vocab + 2, size=40))  # out-of-range ids are skipped by both
    history += history[:10]  # duplicates: penalised once per occurrence
    for step in range(25):
        logits = (rng.standard_normal(vocab) * std).astype(np.float32)
        a, b = logits.copy(), logits.copy()
        got, want = ours.sample(a, history), theirs.sample(b, history)
        assert got == want, f"step {step}"
        assert np.array_equal(a, b), f"step {step}: in-place logits differ"
        history.append(got)


def test_greedy_and_top1_are_argmax():
    rng = np.random.default_rng(3)
    logits = rng.standard_normal(5000).astype(np.float32)
    logits[1234] = logits[4321] = 9.0  # a tie: the lower index wins
    for temperature, top_k in ((0.0, 40), (-1.0, 40), (0.7, 1)):
        s = oracle.Sampler(temperature, top_k, 0.95, 1.0, 64, seed=5)
        assert [s.sample(logits.copy(), []) for _ in range(5)] == [1234] * 5


def test_tiny_top_p_keeps_the_top_token():
    rng = np.random.default_rng(4)
    logits = rng.standard_normal(3000).astype(np.float32)
    s = oracle.Sampler(1.0, 100, 1e-9, 1.0, 64, seed=9)
    assert {s.sample(logits.copy(), []) for _ in range(20)} == {int(np.argmax(logits))}


def test_penalty_applies_once_per_occurrence():
    # Token 0 leads by a factor 1.5^2 < 3 < 1.5^3: two occurrences keep it on top, three do not.
    logits = np.array([3.0, 1.0], np.float32)
    for times, want in ((2, 0), (3, 1)):
        s = oracle.Sampler(0.0, 40, 0.95, 1.5, 64, seed=0)
        a = logits.copy()
        assert s.sample(a, [0] * times) == want
        v = np.float32(3.0)
        for _ in range(times):
            v = np.float32(v / np.float32(1.5))
        assert a[0] == v
    # Negative logits are multiplied; a window of 0 applies nothing; a negative window, all.
    for last_n, expect in ((0, -2.0), (1, -3.0), (-1, -4.5)):
        s = oracle.Sampler(0.0, 40, 0.95, 1.5, last_n, seed=0)
        a = np.array([-2.0, 5.0], np.float32)
        s.sample(a, [0, 1, 0])
        assert a[0] == np.float32(expect), last_n


def test_draw_frequencies_follow_the_kept_weights():
    # Three tokens at logits log(1), log(2), log(3), top-p 1: frequencies 1/6, 2/6, 3/6.
    logits = np.log(np.array([1.0, 2.0, 3.0], np.float32)).astype(np.float32)
    s = oracle.Sampler(1.0, 3, 1.0, 1.0, 64, seed=2024)
    counts = np.bincount([s.sample(logits.copy(), []) for _ in range(30000)], minlength=3) / 30000
    assert np.allclose(counts, [1 / 6, 2 / 6, 3 / 6], atol=0.01)
