"""Prefill GEMM on the GPU against the oracle's i8_gemm semantics (reference
core/matmul.cpp:806-845, core/i8gemm_impl.h:326-419): norm-wise relative error
<= 4e-3 (the MFMA GEMM tolerance). The full config-3 shapes are checked on
row/token sub-blocks that cover the first, middle and last tiles."""
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
