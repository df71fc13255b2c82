"""The engine-layer argument structs of include/desireeia_hip.h have the
reference's field order (core/engine.h:536, :598-603, :675-691, :698-751,
:764-796), and
the ctypes mirrors used by the tests agree with the C compiler's layout
(no GPU needed: a C program prints sizeof/offsetof)."""
import os
import subprocess
import tempfile

import pytest

from desireeia_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
STRUCTS = [_lib.CudaKQuantJob, _lib.CudaQ80Job, _lib.CudaQkvAttnArgs, _lib.CudaLayerArgs,
           _lib.CudaLayerBatchArgs, _lib.CudaSampleArgs, _lib.SampleState, _lib.GemvJob, _lib.MoeDesc]
C_NAME = {"GemvJob": "dq_gemv_job_t", "MoeDesc": "dq_moe_t", "SampleState": "dq_sample_state_t"}


@pytest.fixture(scope="module")
def c_layout():
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "desireeia_hip.h"', 'int main(void) {']
    for st in STRUCTS:
        cn = C_NAME.get(st.__name__, st.__name__)
        lines.append(f'printf("{st.__name__} size %zu\\n", sizeof({cn}));')
        for f, _ in st._fields_:
            lines.append(f'printf("{st.__name__} {f} %zu\\n", offsetof({cn}, {f}));')
    lines.append("return 0; }")
    with tempfile.TemporaryDirectory() as d:
        src, exe = os.path.join(d, "l.c"), os.path.join(d, "l")
        open(src, "w").write("\n".join(lines))
        subprocess.run(["gcc", "-std=c11", "-I", os.path.join(ROOT, "include"), src, "-o", exe], check=True)
        out = subprocess.run([exe], capture_output=True, text=True, check=True).stdout
    table = {}
    for line in out.splitlines():
        s, f, v = line.split()
        table[(s, f)] = int(v)
    return table


@pytest.mark.parametrize("st", STRUCTS, ids=lambda s: s.__name__)
def test_ctypes_matches_c_layout(c_layout, st):
    import ctypes
    assert ctypes.sizeof(st) == c_layout[(st.__name__, "size")]
    for f, _ in st._fields_:
        assert getattr(st, f).offset == c_layout[(st.__name__, f)], f


def test_reference_field_order():
    """Field order of the two big argument blocks, as core/engine.h declares them."""
    qkv = [f for f, _ in _lib.CudaQkvAttnArgs._fields_]
    assert qkv[:8] == ["wq_qs", "wq_scale", "wk_qs", "wk_scale", "wv_qs", "wv_scale", "wo_qs", "wo_scale"]
    assert qkv[-3:] == ["kv_layer_off", "cc_start", "pos"]
    lay = [f for f, _ in _lib.CudaLayerArgs._fields_]
    i = lay.index
    assert i("x") < i("rope_cache") < i("x_out") < i("n_embd") < i("rms_eps") < i("fmt_q") < i("upload_x")
    assert lay[-4:] == ["x_from_token", "embd_qs", "embd_scale", "embd_mul"]
    assert len(lay) == 62
    bat = [f for f, _ in _lib.CudaLayerBatchArgs._fields_]
    j = bat.index
    # core/engine.h:764-796
    assert bat[:2] == ["wq_qs", "wq_scale"] and bat[25:27] == ["x", "x_out"]
    assert j("x_out") < j("x_out_row0") < j("rope_caches") < j("host_kcache") < j("n_embd") < j("kv_layer_off")
    assert j("kv_layer_off") < j("pos0") < j("n_tok") < j("n_swa") < j("x_row0") < j("n_total") < j("rms_eps")
    assert bat[-5:] == ["upload_x", "download_x", "upload_rope", "prepare_weights", "rope_slot"]
    assert len(bat) == 61
