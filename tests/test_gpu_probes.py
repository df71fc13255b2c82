"""The measurement probes of the library (no counterpart in the reference):
the streaming read and the LDS read probe run, consume their input without
writing the sink, and refuse invalid arguments before any launch."""
import pytest
import torch

import bench
from desireeia_amd import _lib, ops

pytestmark = pytest.mark.gpu
NEVER = 0x9E3779B9


def test_stream_read(gpu):
    lib = _lib.load()
    src = torch.randint(0, 255, (1 << 20,), dtype=torch.uint8, device=gpu)
    sink = torch.zeros(1, dtype=torch.int32, device=gpu)
    for wpc, depth in ((1, 4), (4, 8), (8, 16)):
        assert lib.dq_stream_read(ops._ptr(src), src.numel(), wpc, depth, ops._ptr(sink), NEVER, ops._stream()) == 0
    torch.cuda.synchronize()
    assert int(sink.item()) == 0
    assert lib.dq_stream_read(ops._ptr(src), src.numel(), 6, 4, ops._ptr(sink), NEVER, ops._stream()) == -2
    assert lib.dq_stream_read(ops._ptr(src), src.numel(), 4, 5, ops._ptr(sink), NEVER, ops._stream()) == -2
    assert lib.dq_stream_read(None, src.numel(), 4, 4, ops._ptr(sink), NEVER, ops._stream()) == -1


def test_lds_read_probe(gpu):
    lib = _lib.load()
    sink = torch.zeros(1, dtype=torch.int32, device=gpu)
    pats = bench.lds_probe_patterns()
    assert len(pats) == 39
    for name, offs in pats:
        assert len(offs) == 64 and all(0 <= o <= 65536 - 16 and o % 16 == 0 for o in offs), name
    # a few of them, and offsets outside the buffer (wrapped into it)
    for offs in [pats[0][1], pats[-1][1], [16 * l - 4096 for l in range(64)], [1 << 30] * 64]:
        d = torch.tensor(offs, dtype=torch.int32, device=gpu)
        assert lib.dq_lds_read_probe(ops._ptr(d), 64, 8, 0, ops._ptr(sink), NEVER, ops._stream()) == 0
    torch.cuda.synchronize()
    assert int(sink.item()) == 0
    d = torch.zeros(64, dtype=torch.int32, device=gpu)
    assert lib.dq_lds_read_probe(ops._ptr(d), 64, 0, 0, ops._ptr(sink), NEVER, ops._stream()) == -1
    assert lib.dq_lds_read_probe(None, 64, 8, 0, ops._ptr(sink), NEVER, ops._stream()) == -1
    assert lib.dq_lds_read_probe(ops._ptr(d), (1 << 20) + 1, 8, 0, ops._ptr(sink), NEVER, ops._stream()) == -1
