"""Batch-1 decode GEMV on the GPU against the oracle (reference CPU GEMV
semantics, activation quantized the same way): norm-wise relative error
<= 1e-3 (the fp32-accumulated GEMV tolerance), at the benchmark shapes and at
ragged edge shapes."""
import numpy as np
import pytest
import torch

from desireeia_amd import _lib, ops, synth

pytestmark = pytest.mark.gpu
TOL = 1e-3

CASES = [
    (synth.Q8_0, 4096, 4096),      # config 1
    (synth.Q4_0, 14336, 4096),     # config 2 up/gate
    (synth.Q4_0, 4096, 14336),     # config 2 down
    (synth.Q4_K, 14336, 4096),
    (synth.Q4_K, 4096, 14336),
    (synth.Q6_K, 1024, 4096),      # config 4 wv
    (synth.Q6_K, 4096, 14336),     # config 4 down
    (synth.Q8_0, 5, 64),           # ragged: rows not a multiple of the rows per wave
    (synth.Q4_0, 3, 128),
    (synth.Q4_K, 7, 256),
    (synth.Q6_K, 9, 768),
    (synth.Q4_K, 1, 32768),        # 8 items per lane
    (synth.Q8_0, 333, 4160),       # items not a multiple of 64
]


def rel(a, b):
    return float(np.linalg.norm(a.astype(np.float64) - b) / max(np.linalg.norm(b), 1e-30))


@pytest.mark.parametrize("qtype,rows,cols", CASES)
def test_gemv_vs_oracle(gpu, orc, qtype, rows, cols):
    print(f"gemv type={qtype} rows={rows} cols={cols}", flush=True)
    w = synth.gen_weights(qtype, rows, cols, seed=rows * 3 + cols)
    x = synth.gen_act(cols, seed=cols + 1)
    m = ops.QuantMatrix.from_gguf(qtype, w, rows, cols)
    y = ops.matmul(m, torch.from_numpy(x).to(gpu)).cpu().numpy()
    want = orc.matmul(qtype, w, rows, cols, x)
    e = rel(y, want)
    print(f"  rel err {e:.3e}")
    assert e <= TOL
    # per-row: no row may be wrong even if the norm hides it
    scale = np.abs(want).max()
    assert np.max(np.abs(y - want)) <= 1e-3 * scale


def test_gemv_repeat_and_two_sizes(gpu, orc):
    """Two matrices of different shape in a row give the same answers as alone."""
    outs = []
    for rows, cols in [(4096, 14336), (64, 512), (4096, 14336)]:
        w = synth.gen_weights(synth.Q4_K, rows, cols, seed=5)
        x = synth.gen_act(cols, seed=6)
        m = ops.QuantMatrix.from_gguf(synth.Q4_K, w, rows, cols)
        outs.append(ops.matmul(m, torch.from_numpy(x).to(gpu)).cpu().numpy())
    assert np.array_equal(outs[0], outs[2])


def test_gemv_unsupported_shapes(gpu):
    lib = _lib.load()
    assert lib.dq_gemv(synth.FMT_Q4_K, None, 4, 100, None, None, None, None, None) == -2
    assert lib.dq_gemv(synth.FMT_Q8_0, None, 4, 96, None, None, None, None, None) == -2
    assert lib.dq_gemv(9, None, 4, 256, None, None, None, None, None) == -2
    assert lib.dq_gemv(synth.FMT_Q8_0, None, 0, 256, None, None, None, None, None) == 0


def test_gemv_add_residual(gpu, orc):
    """dq_gemv_add: y = W x + res, the residual adds of the decoder layer."""
    for qtype, rows, cols in ((synth.Q4_K, 4096, 4096), (synth.Q6_K, 4096, 14336)):
        w = synth.gen_weights(qtype, rows, cols, seed=rows + cols)
        x = synth.gen_act(cols, seed=3)
        res = np.random.default_rng(4).standard_normal(rows).astype(np.float32) * 100
        m = ops.QuantMatrix.from_gguf(qtype, w, rows, cols)
        act = ops.quantize_act(torch.from_numpy(x).to(gpu), ops.act_kind_for(m.fmt))
        rd = torch.from_numpy(res).to(gpu)
        y = torch.empty(rows, dtype=torch.float32, device=gpu)
        lib = _lib.load()
        _lib.check(lib.dq_gemv_add(m.fmt, ops._ptr(m.buf), rows, cols, ops._ptr(act.q), ops._ptr(act.scale),
                                   ops._ptr(act.isum), ops._ptr(rd), ops._ptr(y), ops._stream()))
        plain = ops.gemv(m, act)
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().numpy(), plain.cpu().numpy() + res)
        want = orc.matmul(qtype, w, rows, cols, x) + res
        assert rel(y.cpu().numpy(), want) <= TOL


@pytest.mark.parametrize("fmts,rows,cols", [
    ((synth.Q4_K, synth.Q4_K, synth.Q6_K), (4096, 1024, 1024), 4096),   # config 4 Q/K/V (V in Q6_K)
    ((synth.Q4_K, synth.Q4_K), (14336, 14336), 4096),                    # config 4 gate/up
    ((synth.Q8_0, synth.Q4_0, synth.Q8_0, synth.Q4_0), (5, 64, 129, 3), 256),  # ragged, per-32 kind
    ((synth.Q6_K,), (7,), 768),
    ((synth.Q6_K, synth.Q4_K, synth.Q6_K, synth.Q4_K), (7, 33, 130, 5), 256),  # mixed per-256 kinds, one launch
    ((synth.Q4_K, synth.Q6_K), (1000, 77), 2048),
    ((synth.Q6_K, synth.Q4_K), (300, 2000), 8192),      # beyond one item per lane: a launch per format
])
def test_gemv_group_matches_single(gpu, orc, fmts, rows, cols):
    """The grouped GEMV (matmul_fused_pq semantics) gives every matrix exactly
    the result of its own launch, and the oracle's within the tolerance."""
    print(f"gemv_group fmts={fmts} rows={rows} cols={cols}", flush=True)
    x = torch.from_numpy(synth.gen_act(cols, seed=cols)).to(gpu)
    mats, ws = [], []
    for j, (qt, r) in enumerate(zip(fmts, rows)):
        w = synth.gen_weights(qt, r, cols, seed=100 + j)
        ws.append(w)
        mats.append(ops.QuantMatrix.from_gguf(qt, w, r, cols))
    act = ops.quantize_act(x, ops.act_kind_for(mats[0].fmt))
    ys = ops.gemv_group(mats, act)
    xn = x.cpu().numpy()
    for j, m in enumerate(mats):
        alone = ops.gemv(m, act).cpu().numpy()
        got = ys[j].cpu().numpy()
        assert np.array_equal(got, alone)
        want = orc.matmul(fmts[j], ws[j], rows[j], cols, xn)
        assert rel(got, want) <= TOL


def test_gemv_group_residual_and_errors(gpu, orc):
    cols = 512
    x = torch.from_numpy(synth.gen_act(cols, seed=3)).to(gpu)
    a = ops.QuantMatrix.from_gguf(synth.Q4_K, synth.gen_weights(synth.Q4_K, 40, cols, seed=1), 40, cols)
    b = ops.QuantMatrix.from_gguf(synth.Q4_0, synth.gen_weights(synth.Q4_0, 40, cols, seed=2), 40, cols)
    res = torch.randn(40, device=gpu)
    act = ops.quantize_act(x, ops.ACT_Q8K_REP)
    (y,) = ops.gemv_group([a], act, residuals=[res])
    torch.testing.assert_close(y, ops.gemv(a, act) + res, rtol=0, atol=0)
    # mixing the per-32 and per-256 activation kinds is not covered: nothing runs
    sentinel = torch.full((40,), 7.0, device=gpu)
    with pytest.raises(_lib.DqError, match="NOT_SUPPORTED"):
        ops.gemv_group([a, b], act, outs=[sentinel, sentinel.clone()])
    assert bool((sentinel == 7.0).all())
    with pytest.raises(_lib.DqError, match="NOT_SUPPORTED"):
        ops.gemv_group([a] * 5, act)


# 5120 and 8192 columns: the per-256 kind without a K split in 8-wave
# workgroups (4096 < cols <= 8192), e.g. hidden sizes 5120 and 8192
@pytest.mark.parametrize("qtype,rows,cols", [(synth.Q4_K, 14336, 4096), (synth.Q4_K, 4096, 14336),
                                             (synth.Q6_K, 4096, 14336), (synth.Q8_0, 4096, 4096),
                                             (synth.Q4_0, 333, 4160), (synth.Q4_K, 5, 49152),
                                             (synth.Q4_K, 1000, 5120), (synth.Q6_K, 513, 8192),
                                             (synth.Q8_0, 700, 5120), (synth.Q4_0, 300, 8192)])
def test_gemv_f32_matches_quantize_then_gemv(gpu, qtype, rows, cols):
    """dq_gemv_f32 (activation quantized in-kernel) is bit-identical to
    dq_quantize_act + dq_gemv."""
    print(f"gemv_f32 type={qtype} {rows}x{cols}", flush=True)
    w = synth.gen_weights(qtype, rows, cols, seed=rows + cols + 1)
    x = torch.from_numpy(synth.gen_act(cols, seed=cols + 2)).to(gpu)
    m = ops.QuantMatrix.from_gguf(qtype, w, rows, cols)
    fused = ops.matmul(m, x)
    two = ops.gemv(m, ops.quantize_act(x, ops.act_kind_for(m.fmt)))
    assert torch.equal(fused, two)


def _edge_activation(cols, seed):
    """Per 256-column chunk: all zeros; amax 127 with exact .5 ties (id = 1,
    so rint must round half to even); magnitudes near 1e30 and 1e-30; one
    lone nonzero; magnitudes near 1e-38 (id overflows to inf: the saturating
    branch); subnormals of mixed sign with exact zeros (subnormal maximum);
    otherwise N(0,1)."""
    x = synth.gen_act(cols, seed=seed).astype(np.float32)
    ties = np.arange(-60, 60, dtype=np.float32) + 0.5
    tiny = np.random.default_rng(seed + 1).integers(-4000, 4001, 256).astype(np.int32)
    for c in range(cols // 256):
        sl = slice(256 * c, 256 * c + 256)
        kind = c % 7
        if kind == 0:
            x[sl] = 0.0
        elif kind == 1:
            v = np.resize(ties, 256)
            v[::32] = 127.0  # every 32-block has amax 127
            x[sl] = v
        elif kind == 2:
            x[sl] *= np.float32(1e30)
        elif kind == 3:
            x[sl] *= np.float32(1e-30)
        elif kind == 4:
            x[sl] = 0.0
            x[256 * c + 77] = -3.25
        elif kind == 5:
            x[sl] *= np.float32(1e-38)
        else:
            # k * 2^-149: subnormals (|k| <= 4000), some exactly zero
            x[sl] = (tiny.astype(np.float64) * 2.0 ** -149).astype(np.float32)
    return x


@pytest.mark.parametrize("qtype,rows,cols", [(synth.Q4_K, 1000, 4096), (synth.Q4_K, 256, 14336),
                                             (synth.Q8_0, 700, 4096), (synth.Q4_0, 300, 14336),
                                             (synth.Q6_K, 513, 14336), (synth.Q4_K, 1000, 5120),
                                             (synth.Q6_K, 513, 8192)])
def test_gemv_f32_quantizer_edges(gpu, qtype, rows, cols):
    """The in-kernel quantizer of dq_gemv_f32 gives the same integers and
    scales as dq_quantize_act on zero blocks, .5 ties, extreme magnitudes and
    sparse blocks (bit-identical GEMV outputs)."""
    print(f"gemv_f32 edges type={qtype} {rows}x{cols}", flush=True)
    w = synth.gen_weights(qtype, rows, cols, seed=rows + 7)
    x = torch.from_numpy(_edge_activation(cols, seed=cols)).to(gpu)
    m = ops.QuantMatrix.from_gguf(qtype, w, rows, cols)
    fused = ops.matmul(m, x)
    two = ops.gemv(m, ops.quantize_act(x, ops.act_kind_for(m.fmt)))
    assert torch.equal(fused, two)


def test_gemv_group_f32_mixed_kinds(gpu, orc):
    """The fp32 group form mixes the per-32 and per-256 kinds (each launch
    quantizes for its own format) and keeps residuals; too wide: -2."""
    cols = 1024
    x = torch.from_numpy(synth.gen_act(cols, seed=8)).to(gpu)
    specs = [(synth.Q4_K, 300), (synth.Q8_0, 100), (synth.Q6_K, 64), (synth.Q4_0, 7)]
    mats = [ops.QuantMatrix.from_gguf(qt, synth.gen_weights(qt, r, cols, seed=r), r, cols) for qt, r in specs]
    res = [torch.randn(m.rows, device=gpu) for m in mats]
    ys = ops.matmul_group(mats, x, residuals=res)
    for m, y, r in zip(mats, ys, res):
        assert torch.equal(y, ops.matmul(m, x) + r)
    wide = ops.QuantMatrix.from_gguf(synth.Q4_K, synth.gen_weights(synth.Q4_K, 2, 65536, seed=1), 2, 65536)
    with pytest.raises(_lib.DqError, match="NOT_SUPPORTED"):
        ops.matmul(wide, torch.zeros(65536, device=gpu))


@pytest.mark.parametrize("cols", [5120, 8192])
def test_gemv_group_f32_wide_matches_quantize_then_group(gpu, cols):
    """The grouped fp32 form at 4096 < cols <= 8192 (8-wave workgroups, no K
    split, one quantization pass): bit-identical to dq_quantize_act +
    dq_gemv_group on normal and edge activations."""
    print(f"gemv_group_f32 cols={cols}", flush=True)
    specs = [(synth.Q4_K, 1024), (synth.Q4_K, 256), (synth.Q6_K, 300)]
    mats = [ops.QuantMatrix.from_gguf(qt, synth.gen_weights(qt, r, cols, seed=r + cols), r, cols) for qt, r in specs]
    for x in (synth.gen_act(cols, seed=cols), _edge_activation(cols, seed=cols + 1)):
        xd = torch.from_numpy(x).to(gpu)
        fused = ops.matmul_group(mats, xd)
        two = ops.gemv_group(mats, ops.quantize_act(xd, ops.ACT_Q8K_REP))
        for a, b in zip(fused, two):
            assert torch.equal(a, b)
