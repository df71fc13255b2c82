"""Activation quantizers of the oracle (reference core/quant.cpp:15-50,
core/matmul.cpp:1660-1778, kv/kv_quant.cpp:31-56): closed-form known answers
and bit-exact agreement with the compiled reference."""
import os

import numpy as np

from desireeia_amd import synth


def test_zero_block(orc):
    q, d, isum, fsum = orc.quantize_q8_1(np.zeros(64, np.float32))
    assert np.all(q == 0) and np.all(d == 0) and np.all(isum == 0) and np.all(fsum == 0)
    q, d, s = orc.quantize_q8k_rep(np.zeros(256, np.float32))
    assert np.all(q == 0) and np.all(d == 0)


def test_amax_maps_to_127_and_ties_round_to_even(orc):
    # amax = 127 -> d = 1, id = 1: x*id is exact, so the rounding is visible
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    x[1:9] = [2.5, 3.5, -2.5, -3.5, 0.5, -0.5, 1.5, 126.5]
    q, d, isum, fsum = orc.quantize_q8_1(x)
    assert d[0] == 1.0
    assert list(q[:9]) == [127, 2, 4, -2, -4, 0, 0, 2, 126]
    assert isum[0] == int(q.astype(np.int32).sum())
    assert fsum[0] == np.float32(sum(np.float32(v) for v in x))


def test_q8k_rep_uses_127_over_amax(orc):
    """quantize_act_q8k_rep multiplies by id = 127/amax, not 1/(amax/127)
    (core/matmul.cpp:1683). Build blocks whose values sit on a rounding
    boundary where the two reciprocals round differently, and check the
    oracle takes the reference's branch."""
    rng = np.random.default_rng(5)
    found = 0
    for _ in range(400):
        amax = np.float32(rng.uniform(1.0, 4.0))
        id_a = np.float32(np.float32(127.0) / amax)
        id_b = np.float32(np.float32(1.0) / np.float32(amax / np.float32(127.0)))
        if id_a == id_b:
            continue
        k = int(rng.integers(1, 120))
        x0 = np.float32((k + 0.5) / float(id_a))
        for nudge in range(-3, 4):
            xv = np.nextafter(x0, np.float32(np.inf) if nudge > 0 else np.float32(-np.inf), dtype=np.float32)
            xv = x0 if nudge == 0 else xv
            for _ in range(abs(nudge) - 1):
                xv = np.nextafter(xv, np.float32(np.inf) if nudge > 0 else np.float32(-np.inf), dtype=np.float32)
            qa, qb = np.rint(xv * id_a), np.rint(xv * id_b)
            if qa != qb and abs(xv) < amax:
                x = np.zeros(256, np.float32)
                x[0] = amax
                x[1] = xv
                q, d, sums = orc.quantize_q8k_rep(x)
                assert q[1] == qa and q[0] == 127
                found += 1
                break
    assert found > 0


def _inputs():
    rng = np.random.default_rng(9)
    x = rng.standard_normal(4096).astype(np.float32)
    x[::97] *= 40.0  # outliers
    x[512:544] = 0.0  # an all-zero block
    return x


def test_q8_0_bitexact_vs_reference(orc, ref):
    x = _inputs()
    q, d, isum, fsum = orc.quantize_q8_1(x)
    rq, rd = ref.quantize_q8_0(x)
    assert np.array_equal(q, rq)
    assert np.array_equal(d.view(np.uint32), rd.view(np.uint32))


def test_q8k_rep_bitexact_vs_reference(orc, ref):
    x = _inputs()
    q, d, s = orc.quantize_q8k_rep(x)
    rq, rd, rs = ref.quantize_q8k_rep(x)
    assert np.array_equal(q, rq)
    assert np.array_equal(d.view(np.uint32), rd.view(np.uint32))
    assert np.array_equal(s, rs)


def test_kv_quantize_bitexact_vs_reference_and_roundtrip(orc, ref):
    x = synth.gen_act(512, seed=4)
    a = orc.kv_quantize_row(x)
    assert np.array_equal(a, ref.kv_quantize_row(x))
    # LE/tests/selftest.cpp:1931-1960: round trip rel-RMS < 1% at dim 512
    y = orc.dequantize_row(synth.Q8_0, a, 512)
    assert np.sqrt(np.mean((y - x) ** 2)) / np.sqrt(np.mean(x ** 2)) < 0.01


def _tiny_block_input():
    """Blocks whose maximum spans the range where id = 1/d or 127/amax
    overflows: 1e-30 (finite id), 1e-36, 3e-37 (just above 127/FLT_MAX),
    1e-38, 1e-40 (subnormal maximum), 1e-44 (d rounds to 0), mixed signs and
    an exact zero in each block."""
    rng = np.random.default_rng(11)
    scales = [1e-30, 1e-36, 3e-37, 1e-38, 1e-40, 1e-44, 1.0, 1e-39]
    x = np.concatenate([(rng.standard_normal(256) * s).astype(np.float32) for s in scales])
    x[5::256] = 0.0
    return x, scales


def test_tiny_blocks_saturate(orc, ref):
    """Where the block maximum is at least 127/FLT_MAX the oracle is the
    reference bit for bit. Below it id overflows to inf and the reference's
    conversion of +-inf/NaN is not defined by its source: compiled here, its
    per-256 AVX2 quantizer writes -128 in every slot and its per-32 ones 0
    (lrintf's overflow value truncated to int32). The oracle, like the GPU
    kernels, saturates instead: sign(x) * 127, 0 for x = 0, with d = amax / 127
    kept."""
    x, scales = _tiny_block_input()
    for kind in ("q8k", "q8_0", "kv"):
        for b, s in enumerate(scales):
            xb = x[256 * b:256 * (b + 1)]
            if kind == "q8k":
                q, d, isum = orc.quantize_q8k_rep(xb)
                rq, rd, _ = ref.quantize_q8k_rep(xb)
            elif kind == "q8_0":
                q, d, isum, _ = orc.quantize_q8_1(xb)
                rq, rd = ref.quantize_q8_0(xb)
            else:
                q = orc.kv_quantize_row(xb).reshape(-1, 34)[:, 2:].view(np.int8).reshape(-1)
                rq = ref.kv_quantize_row(xb).reshape(-1, 34)[:, 2:].view(np.int8).reshape(-1)
            if kind != "kv":
                assert np.array_equal(d.view(np.uint32), rd.view(np.uint32))
            blk = 256 if kind == "q8k" else 32
            for j in range(0, 256, blk):
                xs, qs, rqs = xb[j:j + blk], q[j:j + blk], rq[j:j + blk]
                amax = np.float32(np.abs(xs).max())
                dd = np.float32(amax / np.float32(127))
                with np.errstate(over="ignore", divide="ignore"):
                    idv = np.float32(127) / amax if kind == "q8k" else np.float32(1) / dd
                if dd == 0:
                    assert not qs.any() and not rqs.any()
                elif np.isfinite(idv):
                    assert np.array_equal(qs, rqs)
                else:
                    assert np.array_equal(qs, (np.sign(xs) * 127).astype(np.int8))
                    assert (rqs == (-128 if kind == "q8k" else 0)).all()  # the reference's overflow


def _run_chunks(fn, lo, hi, n=16):
    """fn over [lo, hi) in n chunks on threads (ctypes releases the GIL)."""
    from concurrent.futures import ThreadPoolExecutor
    edges = np.linspace(lo, hi, n + 1).astype(np.uint64)
    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        return sum(ex.map(lambda i: int(fn(int(edges[i]), int(edges[i + 1]))), range(n)))


def test_quantizer_identities_exhaustive(orc):
    """The float identities the GPU quantizers use in place of a division and
    a clamped conversion hold for every input (oracle dqo_check_*):
    amax / 127 as a double product, rint as the low byte of p + 1.5 * 2^23,
    and |x * id| <= 127 without a clamp wherever id is finite."""
    import ctypes
    L = orc.L
    for nm in ("dqo_check_div127", "dqo_check_rint_byte", "dqo_check_id_bound"):
        getattr(L, nm).restype = ctypes.c_uint64
        getattr(L, nm).argtypes = [ctypes.c_uint32, ctypes.c_uint32]
    pos_end = 0x7F800000  # +inf: every finite non-negative float below it
    assert _run_chunks(L.dqo_check_div127, 0, pos_end) == 0
    assert _run_chunks(L.dqo_check_id_bound, 1, pos_end) == 0
    m128 = 0x43000001  # bits of 128.0f, plus one
    assert _run_chunks(L.dqo_check_rint_byte, 0, m128) == 0
    assert _run_chunks(L.dqo_check_rint_byte, 0x80000000, 0x80000000 + m128) == 0
