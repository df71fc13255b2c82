"""Prefill GEMM on the GPU against the oracle's i8_gemm semantics (reference
core/matmul.cpp:806-845, core/i8gemm_impl.h:326-419): norm-wise relative error
<= 4e-3 (the MFMA GEMM tolerance). The full config-3 shapes are checked on
row/token sub-blocks against the oracle's GEMM itself, and in every output
(overall and per workgroup tile) against the fp64 product of the oracle's
operands."""
import ctypes

import numpy as np
import pytest
import torch

from desireeia_amd import _lib, ops, synth

pytestmark = pytest.mark.gpu
TOL = 4e-3


def rel(a, b):
    return float(np.linalg.norm(a.astype(np.float64) - b) / max(np.linalg.norm(b), 1e-30))


@pytest.mark.parametrize("qtype,rows,cols,n_tok", [
    (synth.Q4_K, 14336, 4096, 512),   # config 3 up/gate
    (synth.Q6_K, 4096, 14336, 512),   # config 3 down
    (synth.Q8_0, 14336, 4096, 512),   # the same shape in the formats of Q8_0 / Q4_0 models
    (synth.Q4_0, 4096, 14336, 512),
])
def test_gemm_config3(gpu, orc, qtype, rows, cols, n_tok):
    print(f"gemm type={qtype} rows={rows} cols={cols} n_tok={n_tok}", flush=True)
    w = synth.gen_weights(qtype, rows, cols, seed=rows + 7)
    x = synth.gen_act((n_tok, cols), seed=cols + 9)
    m = ops.QuantMatrix.from_gguf(qtype, w, rows, cols)
    y = ops.gemm(m, torch.from_numpy(x).to(gpu)).cpu().numpy()
    errs = []
    for (r0, r1, t0, t1) in [(0, 160, 0, 40), (rows // 2 - 37, rows // 2 + 91, 200, 260), (rows - 130, rows, n_tok - 70, n_tok)]:
        want = orc.gemm(qtype, w, rows, cols, x, n_tok, r0, r1, t0, t1)[t0:t1, r0:r1]
        e = rel(y[t0:t1, r0:r1], want)
        errs.append(e)
        assert e <= TOL, (r0, t0, e)
    print("  rel errs", ["%.2e" % e for e in errs])


def f64_product(orc, qtype, w, rows, cols, x, dev):
    """Every output of the prefill product in fp64 on the device, from the
    oracle's operands: y = (a q)(dx q_x)^T - m sx^T, with the weight integers,
    per-16 scales and Q4_K offsets of unpack_row and the per-32 activation
    integers, scales and exact block sums of the oracle's quantizer
    (test_oracle_gemm.py pins this form against the oracle's fp64 GEMM and the
    bit-exact dequantizer). Returns [n_tok][rows] float64 on the device."""
    q, a, m = orc.gemm_operands(qtype, w, rows, cols)
    n_tok = x.shape[0]
    xq = np.empty((n_tok, cols), np.int8)
    dx = np.empty((n_tok, cols // 32), np.float32)
    sx = np.empty((n_tok, cols // 32), np.float32)
    for t in range(n_tok):
        xq[t], dx[t], _, sx[t] = orc.quantize_q8_1(x[t])
    f64 = torch.float64
    wa = torch.from_numpy(q).to(dev, f64) * torch.from_numpy(a).to(dev, f64).repeat_interleave(16, dim=1)
    xqt = (torch.from_numpy(xq).to(dev, f64) * torch.from_numpy(dx).to(dev, f64).repeat_interleave(32, dim=1)).t()
    yt = torch.mm(wa, xqt.contiguous())  # [rows][n_tok]
    del wa
    if qtype == synth.Q4_K:
        mt = torch.from_numpy(np.ascontiguousarray(m[:, ::2])).to(dev, f64)
        yt -= torch.mm(mt, torch.from_numpy(sx).to(dev, f64).t().contiguous())
    return yt.t()


@pytest.mark.parametrize("qtype,rows,cols", [
    (synth.Q4_K, 14336, 4096),   # config 3 up/gate
    (synth.Q6_K, 4096, 14336),   # config 3 down
    (synth.Q8_0, 14336, 4096),
    (synth.Q4_0, 4096, 14336),
])
def test_gemm_config3_every_output(gpu, orc, qtype, rows, cols):
    """All n_tok x rows outputs of the config-3 products against the fp64
    product of the oracle's operands: norm-wise within the GEMM bound overall
    and within every 128-token x 256-row tile (a misplaced or skipped
    workgroup tile fails on its own)."""
    n_tok = 512
    print(f"gemm every output type={qtype} {n_tok}x{cols} . {cols}x{rows}", flush=True)
    w = synth.gen_weights(qtype, rows, cols, seed=rows + 11)
    x = synth.gen_act((n_tok, cols), seed=cols + 13)
    m = ops.QuantMatrix.from_gguf(qtype, w, rows, cols)
    y = ops.gemm(m, torch.from_numpy(x).to(gpu)).double()
    want = f64_product(orc, qtype, w, rows, cols, x, gpu)
    assert torch.isfinite(y).all()
    e = float(torch.linalg.norm(y - want) / torch.linalg.norm(want))
    tiles = (y - want).reshape(n_tok // 128, 128, rows // 256, 256).square().sum(dim=(1, 3)).sqrt() / \
        want.reshape(n_tok // 128, 128, rows // 256, 256).square().sum(dim=(1, 3)).sqrt()
    worst = float(tiles.max())
    print(f"  rel err {e:.2e}, worst 128x256 tile {worst:.2e} of {tiles.numel()}", flush=True)
    assert e <= TOL
    assert worst <= TOL


@pytest.mark.parametrize("qtype,rows,cols,n_tok", [
    (synth.Q4_K, 129, 512, 130),      # ragged tiles in both M and N
    (synth.Q6_K, 100, 768, 7),        # a single partial M tile
    (synth.Q4_K, 64, 256, 4),         # K = one super-block, min columns padded
    (synth.Q6_K, 300, 2048, 33),
    (synth.Q8_0, 300, 1024, 33),      # Q8_0: per-32 scales, four sub-planes
    (synth.Q8_0, 129, 512, 2),        # Q8_0 takes the i8_gemm path from 2 tokens
    (synth.Q4_0, 129, 512, 130),      # Q4_0: nibbles - 8
    (synth.Q4_0, 64, 256, 4),
])
def test_gemm_ragged(gpu, orc, qtype, rows, cols, n_tok):
    print(f"gemm ragged type={qtype} rows={rows} cols={cols} n_tok={n_tok}", flush=True)
    w = synth.gen_weights(qtype, rows, cols, seed=rows * 5 + cols)
    x = synth.gen_act((n_tok, cols), seed=n_tok)
    m = ops.QuantMatrix.from_gguf(qtype, w, rows, cols)
    y = ops.gemm(m, torch.from_numpy(x).to(gpu)).cpu().numpy()
    want = orc.gemm(qtype, w, rows, cols, x, n_tok)
    e = rel(y, want)
    print(f"  rel err {e:.2e}")
    assert e <= TOL


def test_gemm_deterministic(gpu):
    w = synth.gen_weights(synth.Q6_K, 4096, 14336, seed=1)
    x = torch.from_numpy(synth.gen_act((64, 14336), seed=2)).to(gpu)
    m = ops.QuantMatrix.from_gguf(synth.Q6_K, w, 4096, 14336)
    a = ops.gemm(m, x).cpu().numpy()
    b = ops.gemm(m, x).cpu().numpy()
    assert np.array_equal(a, b)


def test_gemm_unsupported(gpu):
    lib = _lib.load()
    import ctypes
    n = ctypes.c_size_t(0)
    assert lib.dq_gemm_workspace_bytes(synth.FMT_Q8_0, 64, 320, 16, ctypes.byref(n)) == -2  # K % 256
    assert lib.dq_gemm_workspace_bytes(synth.FMT_Q4_K, 64, 100, 16, ctypes.byref(n)) == -2
    assert lib.dq_gemm_workspace_bytes(99, 64, 4096, 16, ctypes.byref(n)) == -2  # unknown format


@pytest.mark.parametrize("scale", [3000.0, 1e-4])
@pytest.mark.parametrize("qtype", [synth.Q4_K, synth.Q6_K])
def test_gemm_activation_range(gpu, orc, qtype, scale):
    """Activations far from N(0,1): the fp16 operands are range-scaled per token
    by a power of two (block sums of 32 values of 3000 would overflow fp16;
    1e-4 would fall into its subnormals). Rows mix both ranges."""
    rows, cols, n_tok = 96, 1024, 12
    w = synth.gen_weights(qtype, rows, cols, seed=31)
    x = synth.gen_act((n_tok, cols), seed=32)
    x[: n_tok // 2] *= scale
    m = ops.QuantMatrix.from_gguf(qtype, w, rows, cols)
    y = ops.gemm(m, torch.from_numpy(x).to(gpu)).cpu().numpy()
    want = orc.gemm(qtype, w, rows, cols, x, n_tok)
    assert np.isfinite(y).all()
    for t in range(n_tok):  # per token: each row's own magnitude
        assert rel(y[t], want[t]) <= TOL, t


def _f16_act_ref(fmt, x):
    """The GEMM's activation workspace rebuilt in numpy from its definition:
    per token the power-of-two range scale s = 2^(15 - E) with 32 max|x| =
    m 2^E (frexp), per 32-block the reference quantizer (d = amax/127, id =
    1/d, q = rint(x id) clamped to +-127) written as fp16((q d) s) in the
    format's K order, and for Q4_K the sequential float block sums as
    fp16(sum s) in [cols/256][n_tok][8]. Returns (act [n_tok][cols], minp, s)."""
    n_tok, cols = x.shape
    f32 = np.float32
    r = np.abs(x).max(axis=1)
    s = np.empty(n_tok, f32)
    for t in range(n_tok):
        E = int(np.frexp(f32(32.0) * r[t])[1]) if r[t] > 0 else 0
        s[t] = np.ldexp(f32(1.0), 15 - min(max(E, -100), 115))
    blk = x.reshape(n_tok, cols // 32, 32)
    amax = np.abs(blk).max(axis=2)
    d = np.divide(amax, f32(127.0), out=np.zeros_like(amax), where=amax > 0).astype(f32)
    idv = np.divide(f32(1.0), d, out=np.zeros_like(d), where=d > 0).astype(f32)
    # through int32, as the kernel does: a negative value that rounds to zero gives +0
    q = np.clip(np.rint(blk * idv[..., None]), -127, 127).astype(np.int32).astype(f32)
    h = ((q * d[..., None]) * s[:, None, None]).astype(np.float16)  # [n_tok][nb][32]
    nb = cols // 32
    col = np.empty((nb, 32), np.int64)
    for b in range(nb):
        for e in range(32):
            if fmt == synth.Q4_K:
                kk, hf, bo, hi = (e % 16) // 4, e // 16, e % 4, b % 2
                col[b, e] = 64 * (b // 2) + 16 * kk + 8 * hf + 4 * (bo & 1) + (bo >> 1) + 2 * hi
            elif fmt == synth.Q6_K:
                sb, pos0 = b // 8, 32 * (b % 8)
                n, qq, k = pos0 // 128, (pos0 % 128) // 32, e // 16
                col[b, e] = sb * 256 + (2 * n + k) * 64 + qq * 16 + e % 16
            else:
                col[b, e] = 32 * b + e
    act = np.zeros((n_tok, cols), np.float16)
    act[:, col.reshape(-1)] = h.reshape(n_tok, -1)
    minp = None
    if fmt == synth.Q4_K:
        fs = np.cumsum(blk, axis=2, dtype=f32)[..., -1]  # sequential float sums
        minp = (fs * s[:, None]).astype(np.float16).reshape(n_tok, cols // 256, 8).transpose(1, 0, 2)
    return act, minp, s


@pytest.mark.parametrize("qtype,cols,n_tok", [(synth.Q4_K, 4096, 512), (synth.Q4_K, 256, 3), (synth.Q4_K, 14336, 7),
                                              (synth.Q6_K, 14336, 5), (synth.Q8_0, 4096, 9), (synth.Q4_0, 512, 2)])
def test_gemm_activation_layout(gpu, qtype, cols, n_tok):
    """dq_quantize_act_f16 writes exactly the fp16 activation, block sums and
    row scales of its definition (bit-exact), including zero blocks, a zero
    row and rows far from N(0,1)."""
    print(f"gemm act layout type={qtype} cols={cols} n_tok={n_tok}", flush=True)
    lib = _lib.load()
    x = synth.gen_act((n_tok, cols), seed=cols + n_tok).astype(np.float32)
    x[0, 32:96] = 0.0                        # two zero blocks
    if n_tok > 2:
        x[1] *= np.float32(3e4)
        x[2] = 0.0                           # a zero row
    m = ops.QuantMatrix.from_gguf(qtype, synth.gen_weights(qtype, 1, cols, seed=1), 1, cols)
    n = ctypes.c_size_t()
    _lib.check(lib.dq_gemm_workspace_bytes(m.fmt, 1, cols, n_tok, ctypes.byref(n)), "dq_gemm_workspace_bytes")
    work = torch.zeros(n.value, dtype=torch.uint8, device=gpu)
    xd = torch.from_numpy(x).to(gpu)
    _lib.check(lib.dq_quantize_act_f16(m.fmt, ops._ptr(xd), cols, n_tok, ops._ptr(work), ops._stream()),
               "dq_quantize_act_f16")
    w = work.cpu().numpy()
    lda = cols + 64
    a256 = lambda b: (b + 255) // 256 * 256
    act_b = a256(n_tok * lda * 2)
    got = w[:n_tok * lda * 2].view(np.float16).reshape(n_tok, lda)[:, :cols]
    want, minp, s = _f16_act_ref(qtype, x)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
    off = act_b
    if minp is not None:
        gm = w[off:off + minp.size * 2].view(np.float16).reshape(minp.shape)
        assert np.array_equal(gm.view(np.uint16), minp.view(np.uint16))
        off += a256(n_tok * (cols // 32) * 2)
    gs = w[off:off + 4 * n_tok].view(np.float32)
    assert np.array_equal(gs, s)
    gi = w[off + a256(4 * n_tok):off + a256(4 * n_tok) + 4 * n_tok].view(np.float32)
    assert np.array_equal(gi, (np.float32(1.0) / s).astype(np.float32))


@pytest.mark.parametrize("qtype,n,n_tok", [(synth.Q4_K, 4096, 512), (synth.Q6_K, 4096, 512),
                                           (synth.Q8_0, 2048, 64), (synth.Q6_K, 4096, 16)])
def test_gemm_in_place(gpu, qtype, n, n_tok):
    """y may overlap x: an in-place product (y written over x) and one whose y
    starts inside x equal the out-of-place product bit for bit, whichever plan
    (K split or not) the shape takes."""
    print(f"gemm in place type={qtype} n={n} n_tok={n_tok}", flush=True)
    w = synth.gen_weights(qtype, n, n, seed=n + n_tok)
    x = torch.from_numpy(synth.gen_act((n_tok, n), seed=n_tok + 3)).to(gpu)
    m = ops.QuantMatrix.from_gguf(qtype, w, n, n)
    want = ops.gemm(m, x.clone())
    buf = x.clone()
    got = ops.gemm(m, buf, out=buf)
    assert got.data_ptr() == buf.data_ptr()
    assert torch.equal(got, want)
    # y begins half a row into x
    big = torch.zeros(n_tok * n + n // 2, dtype=torch.float32, device=gpu)
    big[:n_tok * n] = x.reshape(-1)
    xv = big[:n_tok * n].view(n_tok, n)
    yv = big[n // 2:].view(n_tok, n)
    ops.gemm(m, xv, out=yv)
    assert torch.equal(yv, want)


@pytest.mark.parametrize("qtype,rows,cols,n_tok", [
    (synth.Q4_K, 14336, 4096, 512),   # config 3 shapes: 4x1 tiles
    (synth.Q6_K, 4096, 14336, 512),   # 2x2 tiles with the K split
    (synth.Q8_0, 14336, 4096, 512),
    (synth.Q4_0, 4096, 14336, 512),
    (synth.Q4_K, 300, 512, 37),       # ragged: rows past the matrix in the last tile
    (synth.Q6_K, 1000, 768, 130),
    (synth.Q8_0, 65, 256, 8),
    (synth.Q4_0, 513, 1024, 300),
])
def test_gemm_tiles_match_rows(gpu, qtype, rows, cols, n_tok):
    """The tile copy (dq_gemm_tiles_pack, DQ_FMT_GEMM_TILES) gives exactly the
    packed rows' result: the same bytes reach the same LDS slots."""
    print(f"gemm tiles type={qtype} rows={rows} cols={cols} n_tok={n_tok}", flush=True)
    w = synth.gen_weights(qtype, rows, cols, seed=rows + cols)
    x = torch.from_numpy(synth.gen_act((n_tok, cols), seed=n_tok)).to(gpu)
    m = ops.QuantMatrix.from_gguf(qtype, w, rows, cols)
    t = ops.GemmTiles(m)
    a = ops.gemm(m, x).cpu().numpy()
    b = ops.gemm(t, x).cpu().numpy()
    assert np.array_equal(a, b)


def test_gemm_tiles_sizes(gpu):
    lib = _lib.load()
    n = ctypes.c_size_t(0)
    # whole 256-row tiles: 300 rows of Q4_K at 512 columns = 2 tiles x 4 slices x 2 stages x 9 KB
    assert lib.dq_gemm_tiles_bytes(synth.FMT_Q4_K, 300, 512, ctypes.byref(n)) == 0
    assert n.value == 2 * 4 * 2 * (2 * 4096 + 1024)
    assert lib.dq_gemm_tiles_bytes(synth.FMT_Q6_K, 256, 768, ctypes.byref(n)) == 0
    assert n.value == 4 * 6 * (3 * 2048 + 768)
    assert lib.dq_gemm_tiles_bytes(synth.FMT_Q4_K, 300, 500, ctypes.byref(n)) == -2
    assert lib.dq_gemm_tiles_bytes(9, 300, 512, ctypes.byref(n)) == -2
