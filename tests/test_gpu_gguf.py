"""GGUF file -> device: matrices read with the library's GGUF reader and
uploaded (GgufFile.matrix through dq_weights_pack; dq_gguf_upload through
the engine's cuda_upload_weights) give the oracle's GEMV and bit-exact
dequantization."""
import ctypes

import numpy as np
import pytest
import torch

import gguf_writer as gw
from desireeia_amd import _lib, gguf, ops, synth

pytestmark = pytest.mark.gpu

SHAPES = [("blk.0.attn_q.weight", synth.Q4_K, 512, 4096), ("blk.0.attn_v.weight", synth.Q6_K, 256, 4096),
          ("blk.0.ffn_down.weight", synth.Q8_0, 384, 1024), ("output.weight", synth.Q4_0, 333, 2048)]


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    tensors, want = [], {}
    for i, (name, qt, rows, cols) in enumerate(SHAPES):
        w = synth.gen_weights(qt, rows, cols, seed=100 + i)
        want[name] = (qt, rows, cols, w)
        tensors.append((name, qt, [cols, rows], w.tobytes()))
    p = tmp_path_factory.mktemp("gguf") / "m.gguf"
    gw.write_gguf(str(p), [("general.architecture", gw.STRING, "llama"),
                           ("general.alignment", gw.U32, 64)], tensors, version=3, alignment=64)
    return str(p), want


def test_matrix_from_gguf(gpu, orc, model):
    path, want = model
    with gguf.GgufFile(path) as f:
        for name, (qt, rows, cols, w) in want.items():
            print(f"gguf matrix {name} type={qt} {rows}x{cols}", flush=True)
            m = f.matrix(name)
            assert (m.rows, m.cols) == (rows, cols)
            deq = m.dequantize().cpu().numpy().reshape(-1)
            ref = orc.dequantize_row(qt, w.reshape(-1), rows * cols)
            assert np.array_equal(deq.view(np.uint32), ref.view(np.uint32))
            x = synth.gen_act(cols, seed=cols + 1)
            y = ops.matmul(m, torch.from_numpy(x).to(gpu)).cpu().numpy()
            yr = orc.matmul(qt, w, rows, cols, x)
            assert np.linalg.norm(y - yr) / np.linalg.norm(yr) <= 1e-3


def test_engine_upload_from_gguf(gpu, orc, model):
    """dq_gguf_upload -> matmul_kquant_cuda_resident / matmul_q8_0_cuda_resident
    (host x and y, as the engine calls them) -> cuda_free_device."""
    path, want = model
    lib = _lib.load()
    P = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    with gguf.GgufFile(path) as f:
        for name, (qt, rows, cols, w) in want.items():
            print(f"gguf upload {name} type={qt} {rows}x{cols}", flush=True)
            fmt, r, c, qs, sc = f.upload(name)
            assert (fmt, r, c) == (synth.FMT_OF_TYPE[qt], rows, cols) and qs
            x = synth.gen_act(cols, seed=cols + 2)
            y = np.zeros(rows, np.float32)
            if qt == synth.Q8_0:
                assert sc
                rc = lib.matmul_q8_0_cuda_resident(qs, sc, rows, cols, P(x), P(y))
            else:
                assert sc is None
                rc = lib.matmul_kquant_cuda_resident(fmt, qs, rows, cols, P(x), P(y))
            assert rc == 0
            yr = orc.matmul(qt, w, rows, cols, x)
            assert np.linalg.norm(y - yr) / np.linalg.norm(yr) <= 1e-3
            lib.cuda_free_device(sc)
            lib.cuda_free_device(qs)
        with pytest.raises(_lib.DqError, match="NOT_SUPPORTED"):
            f.upload("nope")
