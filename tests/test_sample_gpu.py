"""GPU parity of gorch_hip_sample (sample(), model/generate.go:147-243)
against the oracle's restatement, given the same uniform draws.

The final distribution must have the oracle's support exactly and agree
within 1e-12 (f64 sums in a different order); the chosen token must be the
oracle's for every draw (draws are random, none lands within rounding of a
cumulative boundary at these sizes). Covers top-k only, neither, top-k with
top-p (including the case where the top-p loop removes every token: NaN
distribution, last index), ties at the top-k threshold, vocabularies up to
Qwen's 151,936, and the argument errors.
"""
import numpy as np
import pytest
import torch

import oracle as orc

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


CASES = [(50257, 0.8, 40, 0.0), (50257, 1.0, 0, 0.0), (1000, 0.7, 100, 0.9), (1000, 1.3, 50, 0.3),
         (4096, 4.0, 200, 0.4), (151936, 0.9, 64, 0.95), (151936, 1.0, 0, 0.0), (7, 1.0, 3, 0.0), (1, 1.0, 0, 0.0)]


@pytest.mark.parametrize("n,T,K,P", CASES)
def test_sample_matches_oracle(gpu, n, T, K, P):
    rng = np.random.default_rng(n + K + int(P * 10))
    rows = 3
    logits = (rng.standard_normal((rows, n)) * 3).astype(np.float32)
    u = rng.random(rows)
    out = torch.empty(rows, dtype=torch.int32, device="cuda")
    probs = torch.empty((rows, n), dtype=torch.float64, device="cuda")
    gpu.sample(dev(logits), T, K, P, dev(u), out, probs)
    got_tok, got_p = host(out), host(probs)
    for r in range(rows):
        tok, want = orc.sample(logits[r], T, K, P, float(u[r]))
        assert np.array_equal(got_p[r] > 0, want > 0)
        np.testing.assert_allclose(got_p[r], want, rtol=0, atol=1e-12, equal_nan=True)
        assert got_tok[r] == tok


def test_sample_ties_at_top_k_threshold(gpu):
    # integer-valued logits: many equal values at the k-th largest
    rng = np.random.default_rng(3)
    logits = rng.integers(0, 6, size=(4, 2000)).astype(np.float32)
    u = rng.random(4)
    out = torch.empty(4, dtype=torch.int32, device="cuda")
    probs = torch.empty((4, 2000), dtype=torch.float64, device="cuda")
    for K, P in ((10, 0.0), (700, 0.0), (700, 0.5)):
        gpu.sample(dev(logits), 1.0, K, P, dev(u), out, probs)
        got_tok, got_p = host(out), host(probs)
        for r in range(4):
            tok, want = orc.sample(logits[r], 1.0, K, P, float(u[r]))
            np.testing.assert_allclose(got_p[r], want, rtol=0, atol=1e-12, equal_nan=True)
            assert got_tok[r] == tok


def test_sample_argument_errors(gpu):
    x = torch.zeros((1, 10), device="cuda")
    u = torch.zeros(1, dtype=torch.float64, device="cuda")
    out = torch.empty(1, dtype=torch.int32, device="cuda")
    with pytest.raises(gpu.HipError) as e:
        gpu.sample(x, 0.0, 0, 0.0, u, out)
    assert e.value.rc == 2  # GORCH_HIP_EINVAL
    with pytest.raises(gpu.HipError) as e:
        gpu.sample(x, 1.0, 0, 0.5, u, out)  # top-p needs 1 <= top_k <= 4096
    assert e.value.rc == 1  # GORCH_HIP_EUNSUPPORTED


# ------------------------------------------------------------ sampleLogits (Qwen)

NUCLEUS = [(151936, 0.7, 20, 0.8), (151936, 0.9, 4096, 0.95), (151936, 1.0, 0, 0.0), (1000, 0.7, 100, 0.9),
           (1000, 1.3, 50, 0.3), (4096, 4.0, 200, 0.4), (500, 0.5, 1, 0.5), (7, 1.0, 3, 0.99)]


@pytest.mark.parametrize("n,T,K,P", NUCLEUS)
def test_sample_nucleus_matches_oracle(gpu, n, T, K, P):
    """gorch_hip_sample_nucleus against the oracle's sampleLogits
    (model/qwen/generate.go:94-181) with the same draws: support exact,
    probabilities within 1e-12, the same token."""
    rng = np.random.default_rng(2 * n + K + int(P * 100))
    rows = 3
    logits = (rng.standard_normal((rows, n)) * 3).astype(np.float32)
    u = rng.random(rows)
    out = torch.empty(rows, dtype=torch.int32, device="cuda")
    probs = torch.empty((rows, n), dtype=torch.float64, device="cuda")
    gpu.sample_nucleus(dev(logits), T, K, P, dev(u), out, probs)
    got_tok, got_p = host(out), host(probs)
    for r in range(rows):
        tok, want = orc.sample_nucleus(logits[r], T, K, P, float(u[r]))
        assert np.array_equal(got_p[r] > 0, want > 0)
        np.testing.assert_allclose(got_p[r], want, rtol=0, atol=1e-12)
        assert got_tok[r] == tok


def test_sample_nucleus_ties_by_index(gpu):
    """Equal probabilities in the nucleus: the lower indices are kept first
    (integer logits, many ties at the top-k threshold and in the cut)."""
    rng = np.random.default_rng(5)
    logits = rng.integers(0, 6, size=(4, 2000)).astype(np.float32)
    u = rng.random(4)
    out = torch.empty(4, dtype=torch.int32, device="cuda")
    probs = torch.empty((4, 2000), dtype=torch.float64, device="cuda")
    for K, P in ((10, 0.5), (700, 0.3), (700, 0.9)):
        gpu.sample_nucleus(dev(logits), 1.0, K, P, dev(u), out, probs)
        got_tok, got_p = host(out), host(probs)
        for r in range(4):
            tok, want = orc.sample_nucleus(logits[r], 1.0, K, P, float(u[r]))
            np.testing.assert_allclose(got_p[r], want, rtol=0, atol=1e-12)
            assert got_tok[r] == tok


@pytest.mark.parametrize("v2,nucleus", [(1.4099166, False), (1.4099166, True), (1.5, False), (1.5, True)])
def test_sample_scaled_ties_below_raw_threshold(gpu, v2, nucleus):
    """Two logits one float apart whose values divided by the temperature
    (0.7) are equal: the top_k-th largest scaled value is reached by both,
    so both stay (the reference's kthLargest counts the scaled values). With
    1.4099166 both sit in one histogram bin of the top-k candidate pass;
    with 1.5 (a bin's lowest value) the lower one sits in the bin below."""
    v2 = np.float32(v2)
    v1 = np.nextafter(v2, np.float32(0))
    T = np.float32(0.7)
    assert v1 / T == v2 / T and v1 < v2
    rng = np.random.default_rng(8)
    n = 3000
    logits = (rng.standard_normal((2, n)) * 0.3).astype(np.float32)
    logits[:, 100:105] = [2.5, 2.6, 2.7, 2.8, 2.9]
    logits[:, 700] = v2
    logits[:, 1700] = v1
    K = 6  # v2 is the 6th largest logit, v1 the 7th: both kept
    u = np.array([0.3, 0.97])
    out = torch.empty(2, dtype=torch.int32, device="cuda")
    probs = torch.empty((2, n), dtype=torch.float64, device="cuda")
    (gpu.sample_nucleus if nucleus else gpu.sample)(dev(logits), float(T), K, 0.0, dev(u), out, probs)
    got_tok, got_p = host(out), host(probs)
    for r in range(2):
        tok, want = (orc.sample_nucleus if nucleus else orc.sample)(logits[r], float(T), K, 0.0, float(u[r]))
        assert np.count_nonzero(want) == 7
        assert np.array_equal(got_p[r] > 0, want > 0)
        np.testing.assert_allclose(got_p[r], want, rtol=0, atol=1e-12)
        assert got_tok[r] == tok


@pytest.mark.parametrize("nucleus", [False, True])
def test_sample_nan_logit(gpu, nucleus):
    """A NaN logit is never below the top-k threshold (the reference's
    `scaled[i] < threshold` is false for it), so the f64 sum is NaN, every
    probability NaN and the draw falls through to the last index, on the
    device as in the oracle."""
    rng = np.random.default_rng(9)
    n = 5000
    logits = (rng.standard_normal((2, n)) * 2).astype(np.float32)
    logits[0, 17] = np.nan
    logits[1, 4321] = np.nan
    u = np.array([0.1, 0.8])
    out = torch.empty(2, dtype=torch.int32, device="cuda")
    probs = torch.empty((2, n), dtype=torch.float64, device="cuda")
    for K, P in ((40, 0.0), (40, 0.9), (0, 0.0)):
        (gpu.sample_nucleus if nucleus else gpu.sample)(dev(logits), 0.8, K, P, dev(u), out, probs)
        got_tok, got_p = host(out), host(probs)
        for r in range(2):
            tok, want = (orc.sample_nucleus if nucleus else orc.sample)(logits[r], 0.8, K, P, float(u[r]))
            assert got_tok[r] == tok == n - 1
            assert np.isnan(want).all() and np.isnan(got_p[r]).all()


WS_CASES = [(1, 50257, 0.8, 40, 0.0, "normal"), (1, 50257, 0.8, 40, 0.95, "normal"),
            (3, 151936, 0.7, 20, 0.8, "normal"), (16, 50257, 1.3, 1, 0.0, "normal"),
            (16, 8192, 1.0, 4096, 0.5, "normal"), (2, 20000, 1.0, 300, 0.0, "ties"),
            (2, 20000, 1.0, 10, 0.9, "ties"), (2, 9000, 0.8, 40, 0.9, "nan"), (2, 12000, 0.9, 50, 0.0, "zeros"),
            (2, 8192, 0.7, 6, 0.0, "below")]


@pytest.mark.parametrize("nucleus", [False, True])
@pytest.mark.parametrize("rows,n,T,K,P,kind", WS_CASES)
def test_sample_workspace_matches_one_block(gpu, rows, n, T, K, P, kind, nucleus):
    """gorch_hip_sample_with_workspace runs the top-k candidate search's two
    row passes over many blocks per row: its tokens and final distributions
    must equal the one-block kernel's bit for bit, including the rows that
    fall back to the full path (more than 4096 keys tied into the threshold
    bin, a NaN, a scaled tie below the bin), and every call must leave the
    workspace zero (three calls in a row on one workspace)."""
    rng = np.random.default_rng(n + K + rows)
    if kind == "ties":       # 5,000 copies of each of 0..3: the top bin holds more than 4096 keys
        logits = rng.integers(0, 4, size=(rows, n)).astype(np.float32)
    else:
        logits = (rng.standard_normal((rows, n)) * 3).astype(np.float32)
    if kind == "nan":
        logits[:, 1234] = np.nan
    if kind == "zeros":      # +0 and -0 compare equal; the keys must treat them as one value
        logits[:, ::3] = 0.0
        logits[:, 1::7] = -0.0
        logits *= (rng.random((rows, n)) < 0.999)
    if kind == "below":      # two logits one float apart, equal after division by T = 0.7
        logits = (rng.standard_normal((rows, n)) * 0.3).astype(np.float32)
        logits[:, 100:105] = [2.5, 2.6, 2.7, 2.8, 2.9]
        logits[:, 700] = np.float32(1.5)
        logits[:, 1700] = np.nextafter(np.float32(1.5), np.float32(0))
    u = rng.random(rows)
    lg, ud = dev(logits), dev(u)
    out0 = torch.empty(rows, dtype=torch.int32, device="cuda")
    p0 = torch.empty((rows, n), dtype=torch.float64, device="cuda")
    (gpu.sample_nucleus if nucleus else gpu.sample)(lg, T, K, P, ud, out0, p0)
    want_tok, want_p = host(out0), host(p0)
    ws = gpu.sample_workspace(rows)
    out1 = torch.empty(rows, dtype=torch.int32, device="cuda")
    p1 = torch.empty((rows, n), dtype=torch.float64, device="cuda")
    for _ in range(3):
        out1.fill_(-1)
        gpu.sample_with_workspace(lg, T, K, P, ud, out1, ws, p1, nucleus=nucleus)
        assert np.array_equal(host(out1), want_tok)
        assert np.array_equal(host(p1).view(np.uint64), want_p.view(np.uint64))
        assert not bool(ws.any())


@pytest.mark.parametrize("nucleus", [False, True])
def test_sample_tokens_without_probs(gpu, nucleus):
    """Without a distribution to write, up to 64 kept candidates finish in
    one wave (f64 sums across the wave, no barrier): its tokens must be the
    ones the block path (distribution written) chooses, over 64 rows of
    draws for top-k 1..64 with and without top-p, and the oracle's."""
    rng = np.random.default_rng(21)
    rows, n, T = 64, 20000, 0.9
    logits = (rng.standard_normal((rows, n)) * 2).astype(np.float32)
    lg = dev(logits)
    f = gpu.sample_nucleus if nucleus else gpu.sample
    ref = orc.sample_nucleus if nucleus else orc.sample
    probs = torch.empty((rows, n), dtype=torch.float64, device="cuda")
    for K, P in ((1, 0.0), (20, 0.8), (40, 0.95), (64, 0.5), (64, 0.0)):
        u = rng.random(rows)
        ud = dev(u)
        block = torch.empty(rows, dtype=torch.int32, device="cuda")
        wave = torch.empty(rows, dtype=torch.int32, device="cuda")
        f(lg, T, K, P, ud, block, probs)
        f(lg, T, K, P, ud, wave, None)
        got = host(wave)
        assert np.array_equal(host(block), got)
        for r in range(0, rows, 8):
            tok, _ = ref(logits[r], T, K, P, float(u[r]))
            assert got[r] == tok
