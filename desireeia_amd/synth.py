"""Seeded synthetic GGUF weights and activations (numpy only).

Generates raw GGUF block bytes for Q4_0, Q8_0, Q4_K and Q6_K with the value
distributions the benchmark configurations name, so tests and benchmarks feed
identical bytes to the HIP path and to the CPU checker:

  Q8_0  qs uniform in [-127, 127], d = fp16(|N(0, 0.02)| / 127)
  Q4_0  nibbles uniform in [0, 15], d = fp16(|N(0, 0.02)| / 8)
  Q4_K  nibbles uniform, 6-bit scales/mins uniform in [0, 63],
        d, dmin = fp16(|N(0, 0.01)|)
  Q6_K  6-bit quants uniform, int8 scales uniform in [-128, 127],
        d = fp16(|N(0, 0.01)|)

Block layouts are the GGUF ones (reference quant/quant.h:41-187).
"""
import numpy as np

Q4_0, Q8_0, Q8_1, Q4_K, Q6_K = 2, 8, 9, 12, 14          # GGUF type ids
FMT_Q8_0, FMT_Q4_0, FMT_Q4_K, FMT_Q6_K = 0, 1, 5, 7     # device format ids

BLOCK = {Q4_0: (32, 18), Q8_0: (32, 34), Q8_1: (32, 36), Q4_K: (256, 144), Q6_K: (256, 210)}
FMT_OF_TYPE = {Q8_0: FMT_Q8_0, Q4_0: FMT_Q4_0, Q4_K: FMT_Q4_K, Q6_K: FMT_Q6_K}
TYPE_OF_FMT = {v: k for k, v in FMT_OF_TYPE.items()}
NAME = {Q4_0: "Q4_0", Q8_0: "Q8_0", Q8_1: "Q8_1", Q4_K: "Q4_K", Q6_K: "Q6_K"}


def row_bytes(qtype, cols):
    qk, sz = BLOCK[qtype]
    assert cols % qk == 0
    return cols // qk * sz


def _fp16_bits(v):
    return np.asarray(v, dtype=np.float32).astype(np.float16).view(np.uint16)


def pack_scales_min_k4(sc, mn):
    """Eight 6-bit scales and mins -> the 12 bytes of a Q4_K block.
    Vectorised over leading dims; inverse of get_scale_min_k4
    (reference quant/quant.cpp:22-29, :287-293)."""
    sc = np.asarray(sc, dtype=np.uint8)
    mn = np.asarray(mn, dtype=np.uint8)
    out = np.zeros(sc.shape[:-1] + (12,), dtype=np.uint8)
    for i in range(4):
        out[..., i] = (sc[..., i] & 63) | ((sc[..., i + 4] >> 4) << 6)
        out[..., i + 4] = (mn[..., i] & 63) | ((mn[..., i + 4] >> 4) << 6)
        out[..., i + 8] = (sc[..., i + 4] & 0xF) | ((mn[..., i + 4] & 0xF) << 4)
    return out


def gen_weights(qtype, rows, cols, seed):
    """rows x cols matrix as GGUF bytes, shape [rows, row_bytes] uint8."""
    rng = np.random.default_rng(seed)
    qk, sz = BLOCK[qtype]
    nb = rows * cols // qk
    blk = np.zeros((nb, sz), dtype=np.uint8)
    if qtype == Q8_0:
        d = _fp16_bits(np.abs(rng.normal(0.0, 0.02, nb)) / 127.0)
        blk[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
        blk[:, 2:34] = rng.integers(-127, 128, (nb, 32), dtype=np.int16).astype(np.int8).view(np.uint8)
    elif qtype == Q4_0:
        d = _fp16_bits(np.abs(rng.normal(0.0, 0.02, nb)) / 8.0)
        blk[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
        blk[:, 2:18] = rng.integers(0, 256, (nb, 16), dtype=np.uint16).astype(np.uint8)
    elif qtype == Q4_K:
        d = _fp16_bits(np.abs(rng.normal(0.0, 0.01, nb)))
        dmin = _fp16_bits(np.abs(rng.normal(0.0, 0.01, nb)))
        blk[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
        blk[:, 2:4] = dmin.view(np.uint8).reshape(nb, 2)
        sc = rng.integers(0, 64, (nb, 8), dtype=np.uint8)
        mn = rng.integers(0, 64, (nb, 8), dtype=np.uint8)
        blk[:, 4:16] = pack_scales_min_k4(sc, mn)
        blk[:, 16:144] = rng.integers(0, 256, (nb, 128), dtype=np.uint16).astype(np.uint8)
    elif qtype == Q6_K:
        blk[:, 0:192] = rng.integers(0, 256, (nb, 192), dtype=np.uint16).astype(np.uint8)
        blk[:, 192:208] = rng.integers(-128, 128, (nb, 16), dtype=np.int16).astype(np.int8).view(np.uint8)
        d = _fp16_bits(np.abs(rng.normal(0.0, 0.01, nb)))
        blk[:, 208:210] = d.view(np.uint8).reshape(nb, 2)
    else:
        raise ValueError(f"unsupported type {qtype}")
    return blk.reshape(rows, row_bytes(qtype, cols))


def gen_act(shape, seed, scale=1.0):
    """fp32 activations drawn from N(0, scale^2)."""
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(shape) * scale).astype(np.float32)


def lcg_floats(seed, n):
    """The reference self-test generator (LE/tests/selftest.cpp:528-532):
    rng = rng*1664525 + 1013904223 (mod 2^32); x = (rng & 0xFFFF)/32767.5 - 1."""
    out = np.empty(n, dtype=np.float32)
    r = seed & 0xFFFFFFFF
    for i in range(n):
        r = (r * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = np.float32(np.float32(r & 0xFFFF) / np.float32(32767.5)) - np.float32(1.0)
    return out
