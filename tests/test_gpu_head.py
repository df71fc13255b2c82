"""The output head and the device draw on the GPU against the oracle:
top-k selection exact (ids and values, the sampler's order), the draw
(Sampler::sample_candidates restated, pinned on the reference's own sampler)
the same token, head logits within 1e-3 of the final norm + the CPU GEMV,
the Q8_0 embedding row bit-exact."""
import ctypes

import numpy as np
import pytest
import torch

from desireeia_amd import _lib, ops, synth
from oracle import sampler_oracle as so

pytestmark = pytest.mark.gpu
TOL = 1e-3


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@pytest.mark.parametrize("n,kk", [(1, 1), (4096, 40), (4097, 256), (32000, 1), (32000, 104), (128256, 40),
                                  (262144, 256), (150000, 3)])
def test_topk_exact(gpu, n, kk):
    print(f"topk n={n} kk={kk}", flush=True)
    rng = np.random.default_rng(n + kk)
    v = (rng.standard_normal(n) * 4).astype(np.float32)
    v[rng.integers(0, n, n // 8 + 1)] = v[n // 2]  # many equal values
    v[rng.integers(0, n, 3)] = -np.inf
    if n > 10:
        v[5], v[6] = np.float32(0.0), np.float32(-0.0)
        v[7] = v.max()  # an equal maximum at a low index
    ids, vals = ops.topk(torch.from_numpy(v).to(gpu), kk)
    want = so.top_k_select(v, kk)
    assert np.array_equal(ids.cpu().numpy(), want.astype(np.int32))
    assert np.array_equal(vals.cpu().numpy(), v[want])


def sample_args(kk, temperature, top_k, top_p, repeat, freq, present, last_n, u, append=0, slot=0):
    a = _lib.CudaSampleArgs()
    a.temperature, a.top_k, a.top_p = temperature, top_k, top_p
    a.penalty_repeat, a.penalty_freq, a.penalty_present, a.penalty_last_n = repeat, freq, present, last_n
    a.kk, a.logit_scale, a.u, a.append_input, a.slot = kk, 0.0, u, append, slot
    return a


def test_sample_vs_oracle(gpu):
    """400 random candidate sets with every parameter kind: the device draw is
    the oracle's (u from the reference generator's draw). Cases whose u lies
    within 1e-5 of a boundary of the cumulative distribution (where an ulp of
    expf could move the pick) are counted and must be rare."""
    rng = np.random.default_rng(3)
    smp = ops.DeviceSampler(gpu)
    borderline = 0
    for trial in range(400):
        n = int(rng.integers(1, 257))
        ids = rng.choice(200000, n, replace=False).astype(np.int32)
        vals = (rng.standard_normal(n) * rng.choice([0.5, 3, 10])).astype(np.float32)
        if rng.random() < 0.3:
            vals[rng.integers(0, n, 5)] = vals[0]
        hist = [int(t) for t in rng.choice(np.concatenate([ids, rng.integers(0, 200000, 50)]),
                                            int(rng.integers(0, 300)))]
        p = dict(temperature=float(rng.choice([0.0, 0.3, 0.8, 1.5])), top_k=int(rng.choice([1, 5, 40, 256])),
                 top_p=float(rng.choice([1.0, 0.95, 0.5, 0.05])), repeat=float(rng.choice([1.0, 1.1, 1.5])),
                 freq=float(rng.choice([0.0, 0.2])), present=float(rng.choice([0.0, 0.5])),
                 last_n=int(rng.choice([0, 16, 64, 256])))
        u = float(np.float32(rng.random()))
        want = so.sample_candidates(ids, vals, hist, u, **p)
        if (so.sample_candidates(ids, vals, hist, min(u + 1e-5, 0.99999994), **p) != want or
                so.sample_candidates(ids, vals, hist, max(u - 1e-5, 0.0), **p) != want):
            borderline += 1
            continue
        smp.reset(hist)
        a = sample_args(n, p["temperature"], p["top_k"], p["top_p"], p["repeat"], p["freq"], p["present"],
                        p["last_n"], u, slot=trial % 4)
        smp.sample(torch.from_numpy(ids).to(gpu), torch.from_numpy(vals).to(gpu), a)
        st = smp.read()
        assert st.tok == want, (trial, p)
        assert st.ring[trial % 4] == want
    print(f"  borderline cases skipped: {borderline}", flush=True)
    assert borderline < 20


def test_sample_history_append(gpu):
    """Two consecutive draws: the second appends the first's token to the
    history before its penalties (append_input), as the pipelined decode does."""
    ids = np.array([10, 20, 30], np.int32)
    vals = np.array([3.0, 2.9, 1.0], np.float32)
    smp = ops.DeviceSampler(gpu, hist=[5, 6])
    a = sample_args(3, 0.0, 40, 1.0, 2.0, 0.0, 0.0, 64, 0.5)
    smp.sample(torch.from_numpy(ids).to(gpu), torch.from_numpy(vals).to(gpu), a)
    assert smp.read().tok == 10
    a.append_input = 1  # token 10 enters the history: its logit 3.0 -> 1.5, token 20 wins
    smp.sample(torch.from_numpy(ids).to(gpu), torch.from_numpy(vals).to(gpu), a)
    st = smp.read()
    assert st.tok == 20 and st.len == 3 and list(st.hist[:3]) == [5, 6, 10]
    assert so.sample_candidates(ids, vals, [5, 6, 10], 0.5, temperature=0.0, repeat=2.0, last_n=64) == 20


@pytest.mark.parametrize("qtype,rows", [(synth.Q6_K, 32000), (synth.Q8_0, 32000), (synth.Q4_K, 4096)])
def test_head_logits(gpu, orc, qtype, rows):
    E = 4096
    print(f"head type={qtype} rows={rows}", flush=True)
    w = synth.gen_weights(qtype, rows, E, seed=rows + qtype)
    m = ops.QuantMatrix.from_gguf(qtype, w, rows, E, device=gpu)
    rng = np.random.default_rng(rows)
    x = (rng.standard_normal(E) * 3).astype(np.float32)
    nw = (1 + 0.05 * rng.standard_normal(E)).astype(np.float32)
    y = ops.head_logits(m, torch.from_numpy(x).to(gpu), torch.from_numpy(nw).to(gpu), 1e-5).cpu().numpy()
    want = orc.matmul(qtype, w, rows, E, orc.rms_norm(x, nw, 1e-5))
    e = rel(y, want)
    print(f"  rel err {e:.3e}", flush=True)
    assert e <= TOL


def test_embed_q8_0(gpu, orc):
    rows, E = 1000, 4096
    w = synth.gen_weights(synth.Q8_0, rows, E, seed=5)
    m = ops.QuantMatrix.from_gguf(synth.Q8_0, w, rows, E, device=gpu)
    for t, mul in ((0, 0.0), (999, 0.0), (417, 64.0 ** 0.5)):
        tok = torch.tensor([t], dtype=torch.int32, device=gpu)
        x = ops.embed_q8_0(m, tok, mul).cpu().numpy()
        want = orc.dequantize_row(synth.Q8_0, np.ascontiguousarray(w[t]), E)
        if mul:
            want = (want * np.float32(mul)).astype(np.float32)
        assert np.array_equal(x, want)
