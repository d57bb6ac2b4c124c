"""Device sampling (llambda_hip_sampler_*) against the oracle's restatement of
sample-token-id-from-logits (llambda.lisp:1272-1317): the token is identical
for every case with top-k (the reference's serial sums over the survivors
are reproduced in order); without top-k, wherever the random value (and, with
top-p, the cut's running sum) is not within the rounding of the reference's
serial cumulative sums (n * 2^-24)."""
import numpy as np
import pytest

import oracle
from llambda_amd.sampling import HipSampler, SamplingError

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def sampler(hip):
    s = HipSampler(128256)
    yield s
    s.close()


def test_reference_sampling_kats_on_device(sampler, kats):
    k = kats["sampling"]
    for logits, kw, roll, want in k["tokens"]:
        assert sampler.sample(logits, random_value=roll, **dict(kw)) == want, (logits, kw)
    for logits, kw1, kw2, roll in k["same"]:
        assert sampler.sample(logits, random_value=roll, **kw1) == \
            sampler.sample(logits, random_value=roll, **kw2)


def _head_like(rng, n):
    # logits of an output head: N(0, 3) with a few large values
    x = (rng.normal(size=n) * 3).astype(np.float32)
    x[rng.integers(0, n, size=20)] += np.float32(8.0)
    return x


@pytest.mark.parametrize("top_k,top_p,temperature", [(40, 0.9, 1.0), (40, 1.0, 1.0),
                                                     (1, 0.9, 1.0), (1000, 0.5, 0.7),
                                                     (40, 0.95, 1.3), (7, 0.3, 2.0),
                                                     (1024, 0.9, 1.0), (1500, 0.8, 1.0),
                                                     (4096, 0.99, 1.0)])
def test_full_vocab_matches_oracle(sampler, top_k, top_p, temperature):
    rng = np.random.default_rng(top_k * 7 + int(top_p * 100))
    n = 128256
    for trial in range(6):
        x = _head_like(rng, n)
        hist = rng.integers(0, n, size=int(rng.integers(0, 30))).tolist()
        hist += hist[:3]  # repeats
        roll = float(np.float32(rng.random()))
        kw = dict(history=hist, repetition_penalty=1.15, top_k=top_k, top_p=top_p,
                  temperature=temperature, random_value=roll)
        got = sampler.sample(x, **kw)
        want = oracle.sample_token(x, **kw)
        assert got == want, (trial, got, want)


def test_long_histories(sampler):
    # up to 128 distinct history tokens travel in the launch's arguments,
    # longer histories through a device buffer: both sides of the threshold,
    # with the penalised tokens among the top candidates
    rng = np.random.default_rng(77)
    n = 128256
    for distinct in (127, 128, 129, 1000):
        x = _head_like(rng, n)
        top = np.argsort(-x)[:200]
        hist = rng.choice(n, size=distinct, replace=False)
        hist[:50] = top[:50]
        hist = rng.permutation(hist).tolist()
        hist += hist[:5]  # repeats do not count
        for roll in (0.05, 0.5, 0.95):
            kw = dict(history=hist, repetition_penalty=1.3, top_k=40, top_p=0.9,
                      temperature=1.0, random_value=roll)
            assert sampler.sample(x, **kw) == oracle.sample_token(x, **kw), (distinct, roll)


def test_ties_at_the_cutoff(sampler):
    rng = np.random.default_rng(5)
    n = 50000
    x = rng.integers(-5, 6, size=n).astype(np.float32)  # thousands of ties
    for k in (1, 3, 40):
        for roll in (0.0, 0.3, 0.999):
            x2 = x.copy()
            x2[:500] = np.float32(9.0)  # 500 tied maxima: every one survives top-k
            kw = dict(top_k=k, top_p=0.9, temperature=1.0, random_value=roll)
            assert sampler.sample(x2, **kw) == oracle.sample_token(x2, **kw)
    # more tied survivors than the device path holds
    with pytest.raises(SamplingError, match="tie"):
        sampler.sample(np.zeros(n, dtype=np.float32), top_k=5, top_p=0.9, random_value=0.5)


def test_ties_within_the_slices(sampler):
    """Ties at the top-k cutoff that every row slice can still pass on in
    full (at most 64 candidates a slice), and a cutoff at zero where -0.0 and
    +0.0 tie (the reference keeps every logit >= the k-th largest)."""
    rng = np.random.default_rng(11)
    n = 128256
    for trial in range(4):
        x = (rng.standard_normal(n) * 2.0).astype(np.float32)
        top = np.float32(x.max() + 1.0)
        spots = rng.choice(n, size=20, replace=False)  # spread over the slices
        x[spots] = top
        for k in (5, 20, 25):
            roll = float(np.float32(rng.random()))
            kw = dict(top_k=k, top_p=0.9, temperature=1.0, random_value=roll)
            assert sampler.sample(x, **kw) == oracle.sample_token(x, **kw), (trial, k)
    x = -np.abs(rng.standard_normal(n)).astype(np.float32) - 1.0
    zeros = rng.choice(n, size=12, replace=False)
    x[zeros[:6]] = np.float32(0.0)
    x[zeros[6:]] = np.float32(-0.0)
    for k in (3, 6, 12):
        for roll in (0.1, 0.6, 0.95):
            kw = dict(top_k=k, top_p=1.0, temperature=1.0, random_value=roll)
            assert sampler.sample(x, **kw) == oracle.sample_token(x, **kw), (k, roll)


def test_without_top_k(sampler):
    rng = np.random.default_rng(6)
    n = 128256
    for trial in range(8):
        x = _head_like(rng, n)
        roll = float(np.float32(rng.random()))
        got = sampler.sample(x, top_k=0, top_p=1.0, random_value=roll)
        want = oracle.sample_token(x, top_k=0, top_p=1.0, random_value=roll)
        if got != want:
            # only where the roll is within the rounding of a cumulative sum:
            # a serial fp32 sum over n terms is within n * 2^-24 of the exact one
            p = np.exp(x.astype(np.float64) - x.max())
            c = np.cumsum(p / p.sum())
            tol = n * 2.0 ** -24
            a, b = min(got, want), max(got, want)
            # every cumulative between the two draws lies within the window
            assert c[a] >= roll - tol and c[b - 1] <= roll + tol, (trial, got, want)


def _penalised32(x, hist, penalty):
    """apply-repetition-penalty (llambda.lisp:1036-1086) in float32, as the
    device computes it."""
    y = np.asarray(x, dtype=np.float32).copy()
    pen = np.float32(penalty)
    for t in set(hist):
        if y[t] > 0:
            y[t] = y[t] / pen
        elif y[t] < 0:
            y[t] = y[t] * pen
    return y


def _top_p_allowed_draws(x, hist, penalty, top_p, temperature, roll):
    """The tokens a top-p-only draw may return when the running sums are
    formed in another order than the reference's serial fp32 sums (each
    within n * 2^-24 of the exact one, n the row length): for every rank
    that may be the first whose running sum reaches p (its exact sum within
    the window of p), the row masked below that rank's value (ties kept), and
    for each such row the draws whose exact cumulative meets the roll within
    the window.  The oracle's own draw on each masked row is always among
    them."""
    n = x.size
    tol = n * 2.0 ** -24
    y = _penalised32(x, hist, penalty)
    order = np.argsort(-y, kind="stable")  # -0 and +0 compare equal: index order
    y64 = y.astype(np.float64)
    e = np.exp(y64[order] / temperature - y64[order[0]] / temperature)
    c = np.cumsum(e) / e.sum()
    prev = np.concatenate(([0.0], c[:-1]))
    cuts = np.nonzero((c >= top_p - tol) & (prev <= top_p + tol))[0]
    allowed = set()
    for r in cuts:
        keep = y >= y[order[r]]
        q = np.where(keep, np.exp(y64 / temperature - y64.max() / temperature), 0.0)
        cq = np.cumsum(q) / q.sum()
        pq = np.concatenate(([0.0], cq[:-1]))
        hits = np.nonzero(keep & (cq >= roll - tol) & (pq <= roll + tol))[0]
        allowed.update(int(i) for i in hits)
        masked = np.where(keep, y, np.float32(-1.0e30)).astype(np.float32)
        allowed.add(int(oracle.sample_token(masked, top_k=0, top_p=1.0, temperature=temperature,
                                            random_value=roll)))
    return allowed


@pytest.mark.parametrize("n", [1000, 20000])
def test_top_p_without_top_k(sampler, n):
    # the device ranks the whole row (stable radix sort) and sums in a fixed
    # tree order; it matches the oracle except where the reference's serial
    # running sums meet p, or the roll, within their rounding
    rng = np.random.default_rng(n)
    checked = 0
    for trial in range(12):
        x = _head_like(rng, n)
        if trial % 3 == 0:
            x[rng.integers(0, n, size=50)] = x.max()  # ties at the top
        top_p = (0.5, 0.9, 0.99)[trial % 3]
        temperature = (1.0, 0.7, 1.6)[(trial // 3) % 3]
        hist = rng.integers(0, n, size=20).tolist()
        roll = float(np.float32(rng.random()))
        kw = dict(history=hist, repetition_penalty=1.15, top_k=0, top_p=top_p,
                  temperature=temperature, random_value=roll)
        got = sampler.sample(x, **kw)
        want = oracle.sample_token(x, **kw)
        if got == want:
            checked += 1
        else:
            allowed = _top_p_allowed_draws(x, hist, 1.15, top_p, temperature, roll)
            assert want in allowed, (trial, want, sorted(allowed)[:20])
            assert got in allowed, (trial, got, want, sorted(allowed)[:20])
    assert checked >= 9


def test_top_p_without_top_k_largest_row(hip):
    # the longest row the device sampler takes, nearly in descending order so
    # that the reference's insertion sort (the oracle's) stays linear; a few
    # swapped neighbours and equal values exercise the stable ranking
    n = 262144
    rng = np.random.default_rng(21)
    x = np.sort(rng.normal(size=n).astype(np.float32) * 4)[::-1].copy()
    x[100:140] = x[100]  # equal values
    for i in rng.integers(0, 5000, size=30):
        x[i], x[i + 1] = x[i + 1], x[i]
    s = HipSampler(n)
    exact = 0
    cases = [(0.5, 0.3), (0.9, 0.8), (0.97, 0.01), (0.6, 0.5), (0.75, 0.9), (0.8, 0.2),
             (0.95, 0.65), (0.99, 0.45)]
    try:
        for top_p, roll in cases:
            kw = dict(top_k=0, top_p=top_p, temperature=1.0, random_value=roll)
            got, want = s.sample(x, **kw), oracle.sample_token(x, **kw)
            if got == want:
                exact += 1
            else:
                allowed = _top_p_allowed_draws(x, [], 1.15, top_p, 1.0, roll)
                assert got in allowed and want in allowed, (top_p, got, want)
    finally:
        s.close()
    # the top of this row holds ranks of a few percent each, far above the
    # window n * 2^-24 (1.6%): most draws are exact
    assert exact >= 6, exact


def test_signed_zero_ties_in_one_slice(sampler):
    """k +0 logits and one -0 in the same row slice with the cutoff at zero:
    the reference compares floats (-0 = +0) and keeps all of them."""
    n = 128256
    for zero_at, roll in ((40, 0.9), (5, 0.1), (5, 0.9), (25, 0.6)):
        x = np.full(n, np.float32(-3.0))
        x[[10, 20, 30]] = np.float32(0.0)
        x[zero_at] = np.float32(-0.0)
        kw = dict(top_k=3, top_p=1.0, temperature=1.0, random_value=roll)
        want = oracle.sample_token(x, **kw)
        assert sampler.sample(x, **kw) == want, (zero_at, roll, want)
    x = np.full(n, np.float32(-3.0))
    x[[10, 20, 30]] = np.float32(0.0)
    x[40] = np.float32(-0.0)
    assert oracle.sample_token(x, top_k=3, top_p=1.0, temperature=1.0, random_value=0.9) == 40


def test_errors(sampler):
    x = np.array([3.0, np.nan, 1.0], dtype=np.float32)
    with pytest.raises(SamplingError, match="NaN"):
        sampler.sample(x, top_k=2, top_p=1.0, random_value=0.5)
    with pytest.raises(SamplingError, match="RANDOM-VALUE"):
        sampler.sample([1.0, 2.0], random_value=1.0)
    with pytest.raises(SamplingError, match="TOP-P"):
        sampler.sample([1.0, 2.0], top_p=0.0, random_value=0.5)
    with pytest.raises(SamplingError, match="out of bounds"):
        sampler.sample([1.0, 2.0], history=[2], random_value=0.5)
    with pytest.raises(SamplingError, match="PENALTY"):
        sampler.sample([1.0, 2.0], history=[1], repetition_penalty=0.0, random_value=0.5)
