"""fp16 <-> fp32 of the oracle (reference quant/quant.h:285-323), pinned
exhaustively against numpy's IEEE conversion and the compiled reference."""
import numpy as np


def test_fp16_to_fp32_exhaustive_vs_numpy(orc):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ours = np.array([orc.fp16_to_fp32(int(v)) for v in h], dtype=np.float32)
    npy = h.view(np.float16).astype(np.float32)
    nan = np.isnan(npy)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), npy[~nan].view(np.uint32))


def test_fp16_to_fp32_exhaustive_vs_reference(orc, ref):
    for v in range(65536):
        a = np.float32(orc.fp16_to_fp32(v)).view(np.uint32)
        b = np.float32(ref.fp16_to_fp32(v)).view(np.uint32)
        assert a == b, hex(v)


def _samples():
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32)
    specials = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, 1e-8, 6.1035156e-05, 5.9604645e-08,
                         2.9802322e-08, 2.9802326e-08, np.inf, -np.inf], dtype=np.float32)
    # exact ties between two halves: midpoints of consecutive fp16 values
    h = np.arange(0x0001, 0x7BFF, 97, dtype=np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).view(np.float16).astype(np.float64)
    ties = ((lo + hi) / 2).astype(np.float32)
    return np.concatenate([bits.view(np.float32), specials, ties, -ties])


def test_fp32_to_fp16_rne_vs_numpy(orc):
    xs = _samples()
    xs = xs[~np.isnan(xs)]
    with np.errstate(over="ignore"):
        npy = xs.astype(np.float16).view(np.uint16)
    ours = np.array([orc.fp32_to_fp16(float(x)) for x in xs], dtype=np.uint16)
    assert np.array_equal(ours, npy)


def test_fp32_to_fp16_vs_reference(orc, ref):
    for x in _samples()[::7]:
        assert orc.fp32_to_fp16(float(x)) == ref.fp32_to_fp16(float(x)), x
