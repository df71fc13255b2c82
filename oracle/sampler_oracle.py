"""CPU restatement of the host sampler's draw over candidates and of the
head's top-k selection - test infrastructure only.

sample_candidates follows Sampler::sample_candidates (src/core/sampler.cpp
:298-322) and Sampler::finish_ (:202-253) of the reference, in float32 in
the same order of operations; the generator's uniform number is an input
(`u`, the value Sampler::draw_uniform returns, sampler.h:131), and the draw
is r = u * cum (uniform_real_distribution(0, cum) over the same canonical
number). min-p and DRY are host-only extras (Sampler::host_only) and are not
part of the device draw, so they are not restated. top_k_select is the order
every reference top-k uses (backend_cuda.cu:3438-3497, sampler.cpp:313-316):
larger value first, lower id on equal values.

Pinned by tests/test_oracle_head.py: the compiled reference sampler
(oracle/_ref, dqr_sample_candidates) on random candidate sets with every
parameter kind, and closed forms (greedy is the argmax with the lowest id;
u = 0 picks the first candidate; top_p below the first probability keeps one;
pick frequencies over a grid of u follow the softmax)."""
import numpy as np

f32 = np.float32


def top_k_select(values, kk):
    """Indices of the kk largest values, largest first, lower index on ties."""
    v = np.asarray(values, np.float32)
    order = np.lexsort((np.arange(v.size), -v.astype(np.float64)))
    return order[:kk]


def penalised(ids, vals, hist, repeat, freq, present, last_n):
    vals = np.asarray(vals, np.float32).copy()
    if last_n > 0 and (repeat != 1.0 or freq != 0.0 or present != 0.0):
        look = min(last_n, len(hist))
        counts = {}
        for t in hist[len(hist) - look:]:
            counts[int(t)] = counts.get(int(t), 0) + 1
        for j, i in enumerate(ids):
            c = counts.get(int(i))
            if c is None:
                continue
            lg = vals[j]
            lg = f32(lg * f32(repeat)) if lg <= 0 else f32(lg / f32(repeat))
            lg = f32(lg - f32(f32(c) * f32(freq) + f32(present)))
            vals[j] = lg
    return vals


def sample_candidates(ids, vals, hist, u, temperature=0.0, top_k=40, top_p=0.95, repeat=1.0, freq=0.0, present=0.0,
                      last_n=64):
    ids = np.asarray(ids, np.int64)
    n = ids.size
    if n == 0:
        return -1
    v = penalised(ids, vals, list(hist), repeat, freq, present, last_n)
    order = sorted(range(n), key=lambda j: (-float(v[j]), int(ids[j])))
    if temperature <= 0.0:
        return int(ids[order[0]])
    k = min(top_k, n)
    order = order[:k]
    inv_t = f32(f32(1.0) / f32(temperature))
    max_l = f32(v[order[0]] * inv_t)
    probs = np.zeros(k, np.float32)
    s = f32(0.0)
    for i in range(k):
        p = f32(np.exp(f32(f32(v[order[i]] * inv_t) - max_l)))
        probs[i] = p
        s = f32(s + p)
    if s <= 0:
        return int(ids[order[0]])
    for i in range(k):
        probs[i] = f32(probs[i] / s)
    keep = k
    if top_p < 1.0:
        cum = f32(0.0)
        for i in range(k):
            cum = f32(cum + probs[i])
            if cum >= f32(top_p):
                keep = i + 1
                break
        keep = max(keep, 1)
    cum = f32(0.0)
    for i in range(keep):
        cum = f32(cum + probs[i])
    if cum <= 0:
        return int(ids[order[0]])
    r = f32(f32(f32(u) * cum) + f32(0.0))
    acc = f32(0.0)
    for i in range(keep):
        acc = f32(acc + probs[i])
        if r <= acc:
            return int(ids[order[i]])
    return int(ids[order[keep - 1]])
