"""Pins of the oracle's sample() restatement (model/generate.go:147-262),
its nucleus variant (model/qwen/generate.go:94-181) and of the Philox draws
the device sampler uses, on the CPU.

- kthLargest and the near-greedy sample: the reference's own known answers
  (tests/golden/reference_known_answers.json, from model/generate_test.go).
- The distribution sample() leaves is checked against the mathematics with
  independent numpy code: with top-k the support is every index whose scaled
  logit reaches the k-th largest (np.sort), weights exp(scaled - max) in f64;
  with top-p the support is the longest run, in order of (p descending,
  index descending), whose sum stays within 1.5 * top_p (the set the
  reference's remove-the-smallest loop leaves), renormalised; the token is
  the first index whose cumulative probability exceeds the draw
  (np.searchsorted).
- Philox4x32-10 against the Random123 known-answer vectors.
- The nucleus restatement of model/qwen/generate.go's sampleLogits: closed
  forms (p = (0.5, 0.3, 0.2) at several top_p, where the two rules differ),
  equal probabilities taken by ascending index, and the distribution against
  independent numpy code (descending order by np.lexsort, the cut by
  np.searchsorted on np.cumsum), up to the Qwen vocabulary.
"""
import numpy as np
import pytest

import oracle as orc


def test_kth_largest_known_answers(known_answers):
    ka = known_answers["kth_largest"]
    for c in ka["cases"]:
        assert orc.kth_largest(np.array(ka["data"], np.float32), c["k"]) == c["want"]


def test_sample_near_greedy_known_answer(known_answers):
    ka = known_answers["sample_near_greedy"]
    for r in (0.0, 0.3, 0.999999):
        tok, probs = orc.sample(np.array(ka["logits"], np.float32), ka["temperature"], ka["top_k"], ka["top_p"], r)
        assert tok == ka["want"]
        assert probs[ka["want"]] == pytest.approx(1.0)


def _expected(logits, T, K, P):
    scaled = (logits.astype(np.float32) / np.float32(T)).astype(np.float32)
    n = scaled.size
    keep = np.ones(n, bool)
    if 0 < K < n:
        thr = np.sort(scaled)[::-1][K - 1]
        keep = scaled >= thr
    mx = scaled[keep].max()
    w = np.where(keep, np.exp((scaled - mx).astype(np.float64)), 0.0)
    p = w / w.sum()
    if 0 < P < 1:
        pos = np.nonzero(p > 0)[0]
        order = pos[np.lexsort((-pos, -p[pos]))]
        csum = np.cumsum(p[order])
        L = int(np.sum(csum <= np.float64(np.float32(P)) * 1.5))
        q = np.zeros(n)
        q[order[:L]] = p[order[:L]]
        # when even the largest probability exceeds the limit the loop
        # removes them all and the renormalisation is 0/0 (NaN everywhere)
        with np.errstate(invalid="ignore"):
            p = q / q.sum()
    return p


def _choice(p, r):
    """First index whose cumulative probability exceeds r, else n - 1."""
    if np.isnan(p).any():
        return p.size - 1
    return min(int(np.searchsorted(np.cumsum(p), r, side="right")), p.size - 1)


@pytest.mark.parametrize("n,T,K,P", [(1000, 0.8, 40, 0.0), (1000, 1.0, 0, 0.0), (1000, 0.7, 100, 0.9),
                                     (1000, 1.3, 50, 0.3), (1000, 4.0, 200, 0.4), (500, 0.5, 1, 0.0),
                                     (300, 2.0, 299, 0.5)])
def test_sample_distribution_and_choice(n, T, K, P):
    rng = np.random.default_rng(n + K)
    logits = (rng.standard_normal(n) * 3).astype(np.float32)
    want = _expected(logits, T, K, P)
    for r in rng.random(8):
        tok, probs = orc.sample(logits, T, K, P, float(r))
        assert np.array_equal(probs > 0, want > 0)
        np.testing.assert_allclose(probs, want, rtol=0, atol=1e-12, equal_nan=True)
        assert tok == _choice(want, r)


def test_sample_top_k_ties_keep_every_equal_value():
    logits = np.array([3, 1, 3, 2, 3, 0, 2], np.float32)
    _, probs = orc.sample(logits, 1.0, 2, 0.0, 0.5)
    # the 2nd largest is 3 (three of them): all three stay, nothing else
    assert np.array_equal(np.nonzero(probs)[0], [0, 2, 4])
    assert np.allclose(probs[[0, 2, 4]], 1 / 3)


def test_philox_known_answers():
    # Random123 kat_vectors, philox4x32_10
    assert orc.philox4x32_10([0, 0, 0, 0], [0, 0]) == [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]
    assert orc.philox4x32_10([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2) == [0x408F276D, 0x41C83B0E, 0xA20BC7C6,
                                                                       0x6D5451FD]
    assert orc.philox4x32_10([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0]) == [
        0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]
    u = [orc.philox_uniform(7, s, r) for s in range(4) for r in range(4)]
    assert all(0.0 <= v < 1.0 for v in u) and len(set(u)) == 16


# ---------------------------------------------------------------- Qwen sampleLogits

def _expected_nucleus(logits, T, K, P):
    """The support and weights of model/qwen/generate.go's nucleus cut from
    independent numpy code: the descending-probability order (ties by
    ascending index, np.lexsort), the shortest prefix whose cumulative sum
    reaches top_p (np.searchsorted on np.cumsum), renormalised."""
    scaled = (logits.astype(np.float32) / np.float32(T)).astype(np.float32)
    n = scaled.size
    keep = np.ones(n, bool)
    if 0 < K < n:
        thr = np.sort(scaled)[::-1][K - 1]
        keep = scaled >= thr
    mx = scaled[keep].max()
    w = np.where(keep, np.exp((scaled - mx).astype(np.float64)), 0.0)
    p = w / w.sum()
    if 0 < P < 1:
        order = np.lexsort((np.arange(n), -p))
        csum = np.cumsum(p[order])
        cut = min(int(np.searchsorted(csum, np.float64(np.float32(P)), side="left")) + 1, n)
        q = np.zeros(n)
        q[order[:cut]] = p[order[:cut]]
        p = q / q.sum()
    return p


def test_nucleus_closed_forms():
    # p = (0.5, 0.3, 0.2): a top_p of 0.6 keeps the two largest (0.5 < 0.6 <=
    # 0.8), renormalised to (5/8, 3/8); 0.45 keeps the largest alone
    logits = np.log(np.array([0.5, 0.3, 0.2])).astype(np.float32)
    tok, probs = orc.sample_nucleus(logits, 1.0, 0, 0.6, 0.7)
    np.testing.assert_allclose(probs, [0.625, 0.375, 0.0], rtol=0, atol=1e-7)
    assert tok == 1
    assert orc.sample_nucleus(logits, 1.0, 0, 0.6, 0.6)[0] == 0
    tok, probs = orc.sample_nucleus(logits, 1.0, 0, 0.45, 0.99)
    assert tok == 0 and probs[0] == 1.0 and probs[1] == probs[2] == 0.0
    # where sample()'s remove-the-smallest rule empties the set (every
    # probability above 1.5 * 0.3), the nucleus keeps the largest
    assert np.isnan(orc.sample(logits, 1.0, 0, 0.3, 0.5)[1]).all()
    assert orc.sample_nucleus(logits, 1.0, 0, 0.3, 0.5)[1][0] == 1.0


def test_nucleus_equal_probabilities_by_index():
    # four equal probabilities, top_p 0.5: two kept, the lower indices first
    tok, probs = orc.sample_nucleus(np.zeros(4, np.float32), 1.0, 0, 0.5, 0.9)
    np.testing.assert_allclose(probs, [0.5, 0.5, 0.0, 0.0])
    assert tok == 1


@pytest.mark.parametrize("n,T,K,P", [(1000, 0.8, 40, 0.0), (1000, 1.0, 0, 0.0), (1000, 0.7, 100, 0.9),
                                     (1000, 1.3, 50, 0.3), (1000, 4.0, 200, 0.4), (500, 0.5, 1, 0.0),
                                     (300, 2.0, 299, 0.5), (2000, 1.0, 0, 0.8), (151936, 0.7, 20, 0.8)])
def test_nucleus_distribution_and_choice(n, T, K, P):
    rng = np.random.default_rng(3 * n + K)
    logits = (rng.standard_normal(n) * 3).astype(np.float32)
    want = _expected_nucleus(logits, T, K, P)
    for r in rng.random(6):
        tok, probs = orc.sample_nucleus(logits, T, K, P, float(r))
        assert np.array_equal(probs > 0, want > 0)
        np.testing.assert_allclose(probs, want, rtol=0, atol=1e-12)
        assert tok == _choice(want, r)
