"""dq_gemv_group_fused: the per-256 GEMV group whose kernel forms its own
activation (RMSNorm, or act(gate) * up) and quantizes it in-kernel. Its
outputs must equal those of the separate quantizer followed by the grouped
GEMV (dq_norm_quant / dq_silu_quant + dq_gemv_group), bit for bit, and the
oracle's (rms_norm or the activation, quantize_q8k_rep, matmul) within the
GEMV tolerance 1e-3. Shapes: the config-4 layer's Q/K/V (Q4_K + Q6_K in one
flat launch), gate+up (the persistent form), down (K split), and ragged and
wider cases (K split from 4097 columns)."""
import ctypes

import numpy as np
import pytest
import torch

from desireeia_amd import _lib, ops, synth

pytestmark = pytest.mark.gpu
TOL = 1e-3
EPS = 1e-5


def rel(a, b):
    return float(np.linalg.norm(a.astype(np.float64) - b) / max(np.linalg.norm(b), 1e-30))


def mats_of(fmts, rows, cols, seed):
    ws, ms = [], []
    for j, (qt, r) in enumerate(zip(fmts, rows)):
        w = synth.gen_weights(qt, r, cols, seed=seed + j)
        ws.append(w)
        ms.append(ops.QuantMatrix.from_gguf(qt, w, r, cols))
    return ws, ms


# Up to 4096 columns both paths sum a row's items in the same order (one
# item per lane), so the outputs are bit-identical; wider rows run here with
# the K split and in the separate path's grid without it, so only the float
# summation order differs (~1e-7).
@pytest.mark.parametrize("fmts,rows,cols", [
    ((synth.Q4_K, synth.Q4_K, synth.Q6_K), (4096, 1024, 1024), 4096),   # config 4 Q/K/V: flat, mixed formats
    ((synth.Q4_K, synth.Q4_K), (14336, 14336), 4096),                    # config 4 gate/up: persistent form
    ((synth.Q6_K, synth.Q4_K, synth.Q6_K), (7, 33, 130), 256),           # ragged rows, one 256-block per row
    ((synth.Q4_K, synth.Q6_K), (1000, 77), 5120),                        # K split, 80 items
    ((synth.Q6_K,), (3000,), 8192),
    ((synth.Q4_K, synth.Q6_K), (2048, 1024), 8192),
])
def test_fused_norm_group(gpu, orc, fmts, rows, cols):
    print(f"fused norm fmts={fmts} rows={rows} cols={cols}", flush=True)
    lib = _lib.load()
    rng = np.random.default_rng(cols + len(rows))
    x = (rng.standard_normal(cols) * 3).astype(np.float32)
    nw = (1 + 0.05 * rng.standard_normal(cols)).astype(np.float32)
    res = [(rng.standard_normal(r) * 10).astype(np.float32) for r in rows]
    ws, ms = mats_of(fmts, rows, cols, seed=200)
    xd, wd = torch.from_numpy(x).to(gpu), torch.from_numpy(nw).to(gpu)
    rd = [torch.from_numpy(r).to(gpu) for r in res]
    # the residual on the first matrix only (the epilogue's add is per job)
    resid = [rd[0]] + [None] * (len(ms) - 1)
    ys = ops.gemv_group_fused(ms, ops.FUSE_NORM, xd, wd, EPS, residuals=resid)
    # the separate path: norm_quant, then the grouped GEMV
    act = ops.empty_act((cols,), ops.ACT_Q8K_REP, gpu)
    _lib.check(lib.dq_norm_quant(ops._ptr(xd), None, None, ops._ptr(wd), cols, ctypes.c_float(EPS),
                                 ops._ptr(act.q), ops._ptr(act.scale), ops._ptr(act.isum), ops._stream()))
    want_dev = ops.gemv_group(ms, act, residuals=resid)
    torch.cuda.synchronize()
    y_norm = orc.rms_norm(x, nw, EPS)
    for j, (qt, r) in enumerate(zip(fmts, rows)):
        a, b = ys[j].cpu().numpy(), want_dev[j].cpu().numpy()
        if cols <= 4096:
            assert np.array_equal(a, b), f"job {j}: fused differs from norm_quant + gemv ({rel(a, b):.3e})"
        else:
            assert rel(a, b) <= 1e-6, f"job {j}: fused vs norm_quant + gemv {rel(a, b):.3e}"
        want = orc.matmul(qt, ws[j], r, cols, y_norm) + (res[0] if j == 0 else 0)
        e = rel(a, want)
        print(f"  job {j}: rel err vs oracle {e:.3e}")
        assert e <= TOL


@pytest.mark.parametrize("qtype,rows,cols", [
    (synth.Q6_K, 4096, 14336),   # config 4 down
    (synth.Q4_K, 4096, 14336),
    (synth.Q4_K, 77, 11008),     # ragged rows, 44 items per K quarter (the last 40)
])
def test_fused_silu_down(gpu, orc, qtype, rows, cols):
    print(f"fused silu type={qtype} rows={rows} cols={cols}", flush=True)
    lib = _lib.load()
    rng = np.random.default_rng(rows + cols)
    g = (rng.standard_normal(cols) * 4).astype(np.float32)
    u = (rng.standard_normal(cols) * 4).astype(np.float32)
    res = (rng.standard_normal(rows) * 10).astype(np.float32)
    ws, ms = mats_of((qtype,), (rows,), cols, seed=300)
    gd, ud, rd = (torch.from_numpy(v).to(gpu) for v in (g, u, res))
    (y,) = ops.gemv_group_fused(ms, ops.FUSE_SILU, gd, ud, residuals=[rd])
    act = ops.empty_act((cols,), ops.ACT_Q8K_REP, gpu)
    _lib.check(lib.dq_silu_quant(ops._ptr(gd), ops._ptr(ud), cols, ops._ptr(act.q), ops._ptr(act.scale),
                                 ops._ptr(act.isum), ops._stream()))
    (want_dev,) = ops.gemv_group(ms, act, residuals=[rd])
    torch.cuda.synchronize()
    a = y.cpu().numpy()
    assert np.array_equal(a, want_dev.cpu().numpy())
    h = np.array([orc.L.dqo_silu(float(v)) for v in g], np.float32) * u
    e = rel(a, orc.matmul(qtype, ws[0], rows, cols, h) + res)
    print(f"  rel err vs oracle {e:.3e}")
    assert e <= TOL


def test_fused_geglu_down(gpu, orc):
    """GEGLU (geglu_inplace's exp polynomial): the activation the kernel forms
    equals the oracle's value by value, so the output equals the GEMV of the
    oracle's activation quantized on the device."""
    rows, cols = 4096, 14336
    rng = np.random.default_rng(9)
    g = (rng.standard_normal(cols) * 3).astype(np.float32)
    u = (rng.standard_normal(cols) * 3).astype(np.float32)
    ws, ms = mats_of((synth.Q6_K,), (rows,), cols, seed=400)
    gd, ud = torch.from_numpy(g).to(gpu), torch.from_numpy(u).to(gpu)
    (y,) = ops.gemv_group_fused(ms, ops.FUSE_GEGLU, gd, ud)
    h = np.array([orc.L.dqo_geglu(float(v)) for v in g], np.float32) * u
    hd = torch.from_numpy(h).to(gpu)
    act = ops.quantize_act(hd, ops.ACT_Q8K_REP)
    want_dev = ops.gemv(ms[0], act)
    torch.cuda.synchronize()
    a = y.cpu().numpy()
    assert np.array_equal(a, want_dev.cpu().numpy())
    assert rel(a, orc.matmul(synth.Q6_K, ws[0], rows, cols, h)) <= TOL


@pytest.mark.parametrize("qtype,glu", [(synth.Q4_K, "silu"), (synth.Q6_K, "geglu"), (synth.Q4_K, "geglu")])
def test_fused_norm_glu_pair(gpu, orc, qtype, glu):
    """Gate and up paired in one kernel (DQ_FUSE_NORM_SILU / _GEGLU): the
    output is act(gate) * up of exactly the unpaired launch's gate and up."""
    rows, cols = 14336, 4096
    print(f"fused glu pair type={qtype} act={glu}", flush=True)
    rng = np.random.default_rng(21)
    x = (rng.standard_normal(cols) * 3).astype(np.float32)
    nw = (1 + 0.05 * rng.standard_normal(cols)).astype(np.float32)
    ws, ms = mats_of((qtype, qtype), (rows, rows), cols, seed=500)
    xd, wd = torch.from_numpy(x).to(gpu), torch.from_numpy(nw).to(gpu)
    kind = ops.FUSE_NORM_SILU if glu == "silu" else ops.FUSE_NORM_GEGLU
    h = torch.empty(rows, device=gpu)
    ops.gemv_group_fused(ms, kind, xd, wd, EPS, outs=[h, torch.empty(rows, device=gpu)])
    gate, up = ops.gemv_group_fused(ms, ops.FUSE_NORM, xd, wd, EPS)
    if glu == "silu":
        want = torch.empty(rows, device=gpu)
        lib = _lib.load()
        _lib.check(lib.dq_silu_mul(ops._ptr(gate), ops._ptr(up), rows, ops._ptr(want), ops._stream()))
        torch.cuda.synchronize()
        want = want.cpu().numpy()
    else:
        torch.cuda.synchronize()
        g = gate.cpu().numpy()
        want = np.array([orc.L.dqo_geglu(float(v)) for v in g], np.float32) * up.cpu().numpy()
    assert np.array_equal(h.cpu().numpy(), want)
    # and the oracle's gate / up within the GEMV tolerance
    y_norm = orc.rms_norm(x, nw, EPS)
    assert rel(gate.cpu().numpy(), orc.matmul(qtype, ws[0], rows, cols, y_norm)) <= TOL
    assert rel(up.cpu().numpy(), orc.matmul(qtype, ws[1], rows, cols, y_norm)) <= TOL


def test_fused_unsupported(gpu):
    lib = _lib.load()
    x = torch.zeros(32768, device=gpu)
    m = ops.QuantMatrix.from_gguf(synth.Q8_0, synth.gen_weights(synth.Q8_0, 4, 4096, 1), 4, 4096)
    jobs = (_lib.GemvJob * 1)()
    y = torch.empty(4, device=gpu)
    jobs[0].fmt, jobs[0].d_w, jobs[0].rows, jobs[0].d_y = m.fmt, m.buf.data_ptr(), 4, y.data_ptr()
    # a per-32 format, more than 16384 columns, an unknown kind: nothing launched
    assert lib.dq_gemv_group_fused(jobs, 1, 4096, ops.FUSE_NORM, ops._ptr(x), ops._ptr(x), 1e-5,
                                   ops._stream()) == -2
    jobs[0].fmt = synth.FMT_Q4_K
    assert lib.dq_gemv_group_fused(jobs, 1, 16640, ops.FUSE_NORM, ops._ptr(x), ops._ptr(x), 1e-5,
                                   ops._stream()) == -2
    assert lib.dq_gemv_group_fused(jobs, 1, 4096, 7, ops._ptr(x), ops._ptr(x), 0.0, ops._stream()) == -2
    # the paired form takes exactly two jobs of one format and equal rows
    assert lib.dq_gemv_group_fused(jobs, 1, 4096, ops.FUSE_NORM_SILU, ops._ptr(x), ops._ptr(x), 1e-5,
                                   ops._stream()) == -2
    # a group whose weights the K-split grid cannot keep in flight at once
    # (the caller then quantizes separately): refused before any launch
    # (valid buffers all the same: zero weights of the full size)
    wz = torch.zeros(11008 * (8192 // 256) * 144, dtype=torch.uint8, device=gpu)
    yz = torch.empty(11008, device=gpu)
    big = (_lib.GemvJob * 2)()
    for j in range(2):
        big[j].fmt, big[j].d_w, big[j].rows, big[j].d_y = synth.FMT_Q4_K, wz.data_ptr(), 11008, yz.data_ptr()
    assert lib.dq_gemv_group_fused(big, 2, 8192, ops.FUSE_NORM, ops._ptr(x), ops._ptr(x), 1e-5,
                                   ops._stream()) == -2
