"""Oracle of the output head's selection and the sampling draw
(oracle/sampler_oracle.py): against the reference's own host sampler
(core/sampler.cpp, compiled into oracle/_ref) and closed forms."""
import numpy as np
import pytest

from oracle import sampler_oracle as so


def random_case(rng):
    n = int(rng.integers(1, 257))
    ids = rng.choice(200000, n, replace=False).astype(np.int32)
    vals = (rng.standard_normal(n) * rng.choice([0.5, 3, 10])).astype(np.float32)
    if rng.random() < 0.3:
        vals[rng.integers(0, n, 5)] = vals[0]  # equal values: the lower id wins
    hist = [int(t) for t in rng.choice(np.concatenate([ids, rng.integers(0, 200000, 50)]), int(rng.integers(0, 300)))]
    params = dict(temperature=float(rng.choice([0.0, 0.3, 0.8, 1.5])), top_k=int(rng.choice([1, 5, 40, 256])),
                  top_p=float(rng.choice([1.0, 0.95, 0.5, 0.05])), repeat=float(rng.choice([1.0, 1.1, 1.5])),
                  freq=float(rng.choice([0.0, 0.2])), present=float(rng.choice([0.0, 0.5])),
                  last_n=int(rng.choice([0, 16, 64, 256])))
    return ids, vals, hist, params


def test_sampler_vs_reference(ref):
    """2000 random candidate sets (ties, penalties, top-k, top-p, temperatures):
    the restatement picks the reference sampler's token for the same u."""
    rng = np.random.default_rng(0)
    for trial in range(2000):
        ids, vals, hist, p = random_case(rng)
        tok, u = ref.sample_candidates(ids, vals, hist, seed=trial + 1, skip=trial % 7, **p)
        assert so.sample_candidates(ids, vals, hist, u, **p) == tok, (trial, p)


def test_sampler_closed_forms():
    ids = np.array([7, 3, 9, 1], np.int32)
    vals = np.array([1.0, 2.0, 2.0, -1.0], np.float32)
    # greedy: the largest value, the lower id among equals
    assert so.sample_candidates(ids, vals, [], 0.5, temperature=0.0) == 3
    # u = 0 picks the first candidate of the order; u just below 1 the last kept one
    assert so.sample_candidates(ids, vals, [], 0.0, temperature=1.0, top_k=4, top_p=1.0) == 3
    assert so.sample_candidates(ids, vals, [], 0.9999999, temperature=1.0, top_k=4, top_p=1.0) == 1
    # top_p below the first probability keeps one candidate
    assert so.sample_candidates(ids, vals, [], 0.9999999, temperature=1.0, top_k=4, top_p=0.01) == 3
    # a repeat penalty of 2 on token 3 (value 2 -> 1): token 9 leads
    assert so.sample_candidates(ids, vals, [3], 0.5, temperature=0.0, repeat=2.0, last_n=8) == 9
    # a negative logit is multiplied: token 1 (-1 -> -2) with a present penalty
    v = so.penalised(ids, vals, [1], 2.0, 0.0, 0.5, 8)
    assert v[3] == np.float32(-2.5)


def test_sampler_frequencies_follow_softmax():
    """Over a fine grid of u the picks reproduce the temperature softmax of the
    top-k candidates (the draw inverts the cumulative distribution)."""
    rng = np.random.default_rng(1)
    ids = np.arange(10, dtype=np.int32)
    vals = rng.standard_normal(10).astype(np.float32)
    T, k = 0.7, 6
    picks = [so.sample_candidates(ids, vals, [], u, temperature=T, top_k=k, top_p=1.0)
             for u in (np.arange(20000) + 0.5) / 20000]
    top = np.argsort(-vals)[:k]
    p = np.exp(vals[top].astype(np.float64) / T)
    p /= p.sum()
    freq = np.array([picks.count(int(t)) for t in top]) / len(picks)
    assert np.abs(freq - p).max() < 1e-3


@pytest.mark.parametrize("n,kk", [(1, 1), (100, 40), (5000, 256), (40000, 7)])
def test_top_k_select(n, kk):
    rng = np.random.default_rng(n)
    v = rng.standard_normal(n).astype(np.float32)
    v[rng.integers(0, n, n // 10 + 1)] = v[0]  # many equal values
    got = so.top_k_select(v, kk)
    # brute force: repeatedly take the largest value, lowest index
    left = list(range(n))
    want = []
    for _ in range(kk):
        b = min(left, key=lambda i: (-float(v[i]), i))
        want.append(b)
        left.remove(b)
    assert list(got) == want
