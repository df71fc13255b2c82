"""GPU dequantization, weight packing and activation quantization against the
oracle: bit-exact (integers, scales, sums and dequantized floats)."""
import numpy as np
import pytest
import torch

from desireeia_amd import _lib, ops, synth

pytestmark = pytest.mark.gpu

TYPES = [synth.Q4_0, synth.Q8_0, synth.Q8_1, synth.Q4_K, synth.Q6_K]


def _raw(qtype, n, seed):
    if qtype == synth.Q8_1:
        b = synth.gen_weights(synth.Q8_0, 1, n, seed).reshape(-1, 34)
        hs = np.zeros((b.shape[0], 2), np.uint8)
        return np.concatenate([b[:, :2], hs, b[:, 2:]], axis=1).reshape(-1)
    return synth.gen_weights(qtype, 1, n, seed).reshape(-1)


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("n", [256, 4096 * 64])
def test_dequantize_row_bitexact(gpu, orc, qtype, n):
    print(f"dequantize_row type={qtype} n={n}", flush=True)
    raw = _raw(qtype, n, seed=qtype * 100 + n % 97)
    y = ops.dequantize_row(qtype, torch.from_numpy(raw).to(gpu), n).cpu().numpy()
    want = orc.dequantize_row(qtype, raw, n)
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))


def test_dequantize_row_errors(gpu):
    lib = _lib.load()
    assert lib.dq_dequantize_row(3, None, None, 32, None) == -2      # Q4_1: not on this path
    assert lib.dq_dequantize_row(synth.Q4_K, None, None, 100, None) == -1
    assert lib.dq_dequantize_row(synth.Q8_0, None, None, 0, None) == 0


@pytest.mark.parametrize("qtype", [synth.Q8_0, synth.Q4_0, synth.Q4_K, synth.Q6_K])
@pytest.mark.parametrize("shape", [(5, 256), (64, 4096), (33, 14336)])
def test_pack_then_dequantize_bitexact(gpu, orc, qtype, shape):
    rows, cols = shape
    print(f"pack type={qtype} shape={shape}", flush=True)
    w = synth.gen_weights(qtype, rows, cols, seed=rows + cols)
    m = ops.QuantMatrix.from_gguf(qtype, w, rows, cols)
    y = m.dequantize().cpu().numpy().reshape(-1)
    want = orc.dequantize_row(qtype, w.reshape(-1), rows * cols)
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))


def _check_act(orc, x, kind, a):
    q = a.q.cpu().numpy().reshape(-1)
    s = a.scale.cpu().numpy().reshape(-1)
    isum = a.isum.cpu().numpy().reshape(-1)
    fsum = a.fsum.cpu().numpy().reshape(-1)
    cols = x.shape[-1]
    for t, xt in enumerate(x.reshape(-1, cols)):
        sl = slice(t * cols, (t + 1) * cols)
        bl = slice(t * cols // 32, (t + 1) * cols // 32)
        if kind == ops.ACT_Q8_0:
            oq, od, oi, of = orc.quantize_q8_1(xt)
            assert np.array_equal(fsum[bl].view(np.uint32), of.view(np.uint32))
        else:
            oq, od, oi = orc.quantize_q8k_rep(xt)
        assert np.array_equal(q[sl], oq)
        assert np.array_equal(s[bl].view(np.uint32), od.view(np.uint32))
        assert np.array_equal(isum[bl], oi)


@pytest.mark.parametrize("kind", [ops.ACT_Q8_0, ops.ACT_Q8K_REP])
@pytest.mark.parametrize("shape", [(4096,), (14336,), (7, 4096), (512, 4096)])
def test_quantize_act_bitexact(gpu, orc, kind, shape):
    print(f"quantize_act kind={kind} shape={shape}", flush=True)
    x = synth.gen_act(shape, seed=sum(shape) + kind)
    x.reshape(-1)[::101] *= 30.0
    x.reshape(-1)[:32] = 0.0
    a = ops.quantize_act(torch.from_numpy(x).to(gpu), kind)
    _check_act(orc, x, kind, a)


def test_quantize_q8_1_blocks(gpu, orc):
    x = synth.gen_act(4096, seed=3)
    blk = ops.quantize_q8_1_blocks(torch.from_numpy(x).to(gpu)).cpu().numpy().reshape(-1, 36)
    q, d, isum, _ = orc.quantize_q8_1(x)
    assert np.array_equal(blk[:, 4:].view(np.int8).reshape(-1), q)
    dh = blk[:, 0:2].copy().view(np.float16).reshape(-1)
    assert np.array_equal(dh.view(np.uint16), d.astype(np.float16).view(np.uint16))
    sh = blk[:, 2:4].copy().view(np.float16).reshape(-1)
    assert np.array_equal(sh.view(np.uint16), (d * isum.astype(np.float32)).astype(np.float16).view(np.uint16))
    # its dequantization is the q8_0 one
    y = orc.dequantize_row(synth.Q8_1, blk.reshape(-1), 4096)
    assert np.allclose(y, x, atol=np.abs(x).max() / 127)


@pytest.mark.parametrize("kind", [ops.ACT_Q8_0, ops.ACT_Q8K_REP])
def test_quantize_act_tiny_blocks(gpu, orc, kind):
    """Blocks whose maximum is near or below 127/FLT_MAX (id overflows to
    inf), subnormal and flushed-to-zero scales: the oracle's saturating
    conversion, bit for bit."""
    rng = np.random.default_rng(12)
    scales = [1e-30, 1e-36, 3e-37, 1e-38, 1e-40, 1e-44, 1.0, 1e-39]
    x = np.concatenate([(rng.standard_normal(256) * s).astype(np.float32) for s in scales])
    x[5::256] = 0.0
    a = ops.quantize_act(torch.from_numpy(x).to(gpu), kind)
    _check_act(orc, x, kind, a)
