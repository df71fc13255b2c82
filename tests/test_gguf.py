"""GGUF reader (dq_gguf_* over the C ABI; host only, no GPU) against the CPU
restatement of the engine's reader (oracle/gguf_oracle.py), the engine's own
round-trip self-test files, and malformed inputs."""
import ctypes
import os
import struct

import numpy as np
import pytest

import gguf_writer as gw
from desireeia_amd import _lib, gguf, synth
from oracle import gguf_oracle as go

OK, INVALID_ARG, NOT_SUPPORTED, IO = 0, -1, -2, -3


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_row_size_table(lib):
    """dq_row_size and the oracle's table against the block layouts of
    quant/quant.h (the static_asserts, restated here as formulas)."""
    half, QK_K = 2, 256
    blocks = {  # type id: (block size, bytes)
        0: (1, 4), 1: (1, 2), 30: (1, 2), 24: (1, 1), 25: (1, 2), 26: (1, 4), 27: (1, 8), 28: (1, 8),
        2: (32, half + 16), 3: (32, 2 * half + 16), 6: (32, half + 4 + 16), 7: (32, 2 * half + 4 + 16),
        8: (32, half + 32), 9: (32, 2 * half + 32), 20: (32, half + 16), 39: (32, 1 + 16),
        40: (64, 64 // 16 + 32), 41: (128, half + 128 // 8), 42: (64, half + 64 // 4),
        10: (QK_K, 2 * half + QK_K // 16 + QK_K // 4), 11: (QK_K, half + QK_K // 4 + QK_K // 8 + 12),
        12: (QK_K, 2 * half + 12 + QK_K // 2), 13: (QK_K, 2 * half + 12 + QK_K // 2 + QK_K // 8),
        14: (QK_K, half + QK_K // 16 + 3 * QK_K // 4), 15: (QK_K, 4 + QK_K + QK_K // 16 * 2),
        16: (QK_K, half + QK_K // 8 * 2), 17: (QK_K, half + QK_K // 8 * 2 + QK_K // 32),
        22: (QK_K, half + QK_K // 4 + QK_K // 16), 18: (QK_K, half + 3 * (QK_K // 8)),
        21: (QK_K, half + 13 * (QK_K // 32) + QK_K // 64), 19: (QK_K, half + QK_K // 8 + QK_K // 16),
        29: (QK_K, QK_K // 8 + QK_K // 16 + QK_K // 32), 23: (QK_K, half + 2 + QK_K // 64 + QK_K // 2),
        34: (QK_K, half + QK_K // 64 + (QK_K - 4 * QK_K // 64) // 5), 35: (QK_K, half + QK_K // 4),
    }
    assert blocks == go.TYPE_TRAITS
    for t, (blck, nb) in blocks.items():
        for ne0 in (1, 31, 32, 33, 255, 256, 4096, 4097):
            want = -(-ne0 // blck) * nb
            assert lib.dq_row_size(t, ne0) == want == go.row_size(t, ne0), (t, ne0)
    for t in (4, 5, 31, 99, -1):
        assert lib.dq_row_size(t, 256) == 0
    for qt in (synth.Q8_0, synth.Q4_0, synth.Q4_K, synth.Q6_K):
        assert lib.dq_row_size(qt, 4096) == synth.row_bytes(qt, 4096)
        assert lib.dq_fmt_of_gguf_type(qt) == synth.FMT_OF_TYPE[qt]
    assert lib.dq_fmt_of_gguf_type(13) == -1 and lib.dq_fmt_of_gguf_type(0) == -1


def _kv_all_kinds(alignment_kv=None):
    kv = [
        ("general.architecture", gw.STRING, "llama"),
        ("general.name", gw.STRING, "tést \U0001F600"),
        ("llama.block_count", gw.U32, 32),
        ("llama.context_length", gw.U64, 1 << 40),
        ("llama.expert_count", gw.I32, -5),
        ("x.i64", gw.I64, -(1 << 62)),
        ("x.u8", gw.U8, 200), ("x.i8", gw.I8, -100), ("x.u16", gw.U16, 65000), ("x.i16", gw.I16, -30000),
        ("x.bool", gw.BOOL, 1),
        ("llama.rope.freq_base", gw.F32, 500000.0),
        ("x.f64", gw.F64, 3.141592653589793),
        ("x.flags", gw.ARRAY, (gw.U8, [1, 0, 1, 1])),
        ("x.i8arr", gw.ARRAY, (gw.I8, [-1, 2, -3])),
        ("x.i16arr", gw.ARRAY, (gw.I16, [-1000, 1000])),
        ("x.u32arr", gw.ARRAY, (gw.U32, [7, 8, 4000000000])),
        ("x.i32arr", gw.ARRAY, (gw.I32, [-7, 8])),
        ("x.boolarr", gw.ARRAY, (gw.BOOL, [0, 1, 1])),
        ("x.f32arr", gw.ARRAY, (gw.F32, [0.5, -2.25])),
        ("x.long", gw.ARRAY, (gw.U8, [3] * 5000)),
        ("x.nested", gw.ARRAY, (gw.ARRAY, [(gw.U16, [1, 2]), (gw.STRING, ["a", "bc"])])),
        ("x.strarr", gw.ARRAY, (gw.STRING, ["alpha", "", "gamma"])),
        ("tokenizer.ggml.model", gw.STRING, "gpt2"),
        ("tokenizer.ggml.tokens", gw.ARRAY, (gw.STRING, ["<s>", "</s>", "a"])),
        ("tokenizer.ggml.scores", gw.ARRAY, (gw.F32, [0.0, -1.0, -2.5])),
        ("tokenizer.ggml.token_type", gw.ARRAY, (gw.I32, [3, 3, 1])),
        ("tokenizer.ggml.bos_token_id", gw.U32, 0),
    ]
    if alignment_kv is not None:
        kv.append(alignment_kv)
    return kv


def _tensors():
    rng = np.random.default_rng(3)
    out = [("f32", 0, [16, 3], rng.standard_normal(48).astype(np.float32).tobytes()),
           ("f16", 1, [64], rng.standard_normal(64).astype(np.float16).tobytes())]
    for name, qt, cols, rows in (("q4_0", synth.Q4_0, 64, 5), ("q8_0", synth.Q8_0, 96, 2),
                                 ("q4_k", synth.Q4_K, 256, 3), ("q6_k", synth.Q6_K, 512, 2)):
        out.append((name, qt, [cols, rows], synth.gen_weights(qt, rows, cols, seed=cols).tobytes()))
    out.append(("q5_k", 13, [256, 1], bytes(range(176))))
    out.append(("odd", 0, [3, 2, 2], bytes(48)))          # 3-d: rows = 2*2
    out.append(("unknown", 77, [10], b"\1" * 10))          # a type without a row size
    return out


def _compare(lib, path, data):
    info = go.read(data)
    with gguf.GgufFile(path) as f:
        assert info is not None
        assert f.version == info["version"]
        assert f.data_offset == info["data_start"]
        assert f.n_tensors == len(info["tensors"])
        for name, t, dims, off in info["tensors"]:
            ti = f.tensor(name)
            assert (ti.name, ti.type, ti.dims) == (name, t, dims)
            assert ti.offset == info["data_start"] + off
            want = go.read_tensor_raw(data, info, name)
            if want is None:
                assert ti.nbytes == 0
                with pytest.raises(_lib.DqError, match="NOT_SUPPORTED"):
                    f.read_tensor_raw(name)
                continue
            raw, ty, ne0, rows = f.read_tensor_raw(name)
            assert raw.tobytes() == want[0] and (ty, ne0, rows) == want[1:]
            assert ti.nbytes == len(want[0])
        for k, v in info["kv_string"].items():
            assert f.get(k) == v
        for k, v in info["kv_int"].items():
            t = f.value_type(k)
            mask = 0xFFFFFFFF if t == gw.I32 else (1 << 64) - 1
            assert f.get(k) & mask == v, k
        for k, v in info["kv_float"].items():
            assert f.get(k) == v
        for k, v in info["kv_arr"].items():
            assert [x & 0xFFFFFFFF for x in f.get(k)] == v, k
        for k, v in info["vocab"].items():
            assert f.get("tokenizer.ggml." + k) == v
    return info


@pytest.mark.parametrize("version", [1, 2, 3])
@pytest.mark.parametrize("alignment,kv", [(32, None), (64, ("general.alignment", gw.U32, 64)),
                                          (1, ("general.alignment", gw.U64, 1)),
                                          (32, ("general.alignment", gw.U32, 48)),   # not a power of two
                                          (32, ("general.alignment", gw.U16, 64))])  # a kind the engine skips
def test_reader_matches_oracle(tmp_path, lib, version, alignment, kv):
    data = gw.gguf_bytes(_kv_all_kinds(kv), _tensors(), version=version, alignment=alignment)
    p = tmp_path / "m.gguf"
    p.write_bytes(data)
    info = _compare(lib, str(p), data)
    if version < 2:
        assert info["data_start"] == 0  # absolute offsets
    with gguf.GgufFile(str(p)) as f:
        # independent of the oracle: every sized tensor reads back as exactly
        # the bytes the writer placed (at its own aligned data start)
        for name, ty, dims, blob in _tensors():
            if go.row_size(ty, dims[0]):
                assert f.read_tensor_raw(name)[0].tobytes() == blob, name
        # the superset the library keeps beyond the engine's maps
        assert f.get("x.u16") == 65000 and f.get("x.i16") == -30000 and f.get("x.i8") == -100
        assert f.get("x.f64") == 3.141592653589793 and f.get("llama.expert_count") == -5
        assert f.get("x.i64") == -(1 << 62) and f.get("x.strarr") == ["alpha", "", "gamma"]
        assert len(f.get("x.long")) == 5000 and f.get("missing", "d") == "d"
        assert f.get("llama.rope.freq_base") == 500000.0


def _encode_q8_0(x):
    """GGUF Q8_0 blocks: fp16 d = amax/127, int8 rint(x/d) (the reference's
    encoder of the self-test)."""
    out = bytearray()
    for b in range(len(x) // 32):
        v = x[32 * b:32 * b + 32].astype(np.float32)
        amax = float(np.max(np.abs(v)))
        d = np.float32(amax / 127.0)
        q = np.zeros(32, np.int8) if d == 0 else np.clip(np.rint(v / d), -127, 127).astype(np.int8)
        out += np.float16(d).tobytes() + q.tobytes()
    return bytes(out)


def test_engine_selftest_roundtrip_files(tmp_path, lib, orc):
    """Replays the engine's GGUF round-trip self-test (tests/selftest.cpp
    :333-440): version-1 header with 64-bit counts, one 1-d tensor "w" of
    2 blocks of LCG values (seed 12345), its ABSOLUTE offset pointing at the
    next 32-aligned position; reading it back gives the bytes written, and
    the decoded values meet the self-test's tolerances."""
    def lcg_values(n):
        rng, out = 12345, []
        for _ in range(n):
            rng = (rng * 1664525 + 1013904223) & 0xFFFFFFFF
            out.append((rng & 0xFFFF) / 32767.5 - 1.0)
        return np.array(out, dtype=np.float32)

    for tid, tol in ((0, 1e-6), (1, 1e-3), (8, 0.01)):
        blck = go.TYPE_TRAITS[tid][0]
        n = 2 * blck
        src = lcg_values(n)
        raw = (src.tobytes() if tid == 0 else src.astype(np.float16).tobytes() if tid == 1 else _encode_q8_0(src))
        head = b"GGUF" + struct.pack("<IQQ", 1, 1, 0) + struct.pack("<Q", 1) + b"w" + struct.pack("<IQI", 1, n, tid)
        off_pos = len(head)
        data_abs = off_pos + 8
        pad = (32 - data_abs % 32) % 32
        data_off = data_abs + pad
        blob = head + struct.pack("<Q", data_off) + b"\0" * pad + raw
        p = tmp_path / f"rt_{tid}.gguf"
        p.write_bytes(blob)
        with gguf.GgufFile(str(p)) as f:
            got, ty, ne0, rows = f.read_tensor_raw("w")
            assert got.tobytes() == raw and (ty, ne0, rows) == (tid, n, 1)
            assert f.tensor("w").offset == data_off
        vals = (np.frombuffer(raw, np.float32) if tid == 0 else np.frombuffer(raw, np.float16).astype(np.float32)
                if tid == 1 else orc.dequantize_row(synth.Q8_0, np.frombuffer(raw, np.uint8), n))
        assert float(np.max(np.abs(vals - src))) <= tol


def test_malformed_inputs(tmp_path, lib):
    h = ctypes.c_void_p()
    assert lib.dq_gguf_open(str(tmp_path / "absent.gguf").encode(), ctypes.byref(h)) == IO
    assert lib.dq_gguf_open(None, ctypes.byref(h)) == INVALID_ARG
    good = gw.gguf_bytes(_kv_all_kinds(("general.alignment", gw.U32, 64)), _tensors()[:5], version=3, alignment=64)
    cases = {
        "empty": b"",
        "magic": b"GGUX" + good[4:],
        "kv_count": good[:8] + struct.pack("<Q", 2) + struct.pack("<Q", 1 << 60) + good[24:],
        "tensor_count": good[:8] + struct.pack("<Q", 1 << 60) + good[16:],
        # an unknown value type (13) after a valid key
        "value_type": b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1) + b"k" + struct.pack("<I", 13),
    }
    for name, blob in cases.items():
        p = tmp_path / f"bad_{name}.gguf"
        p.write_bytes(blob)
        rc = lib.dq_gguf_open(str(p).encode(), ctypes.byref(h))
        assert rc in (IO, INVALID_ARG), name
        assert go.read(blob) is None, name
    # every prefix of a valid file: the library and the oracle agree on
    # whether it opens and on which tensors can be read
    p = tmp_path / "cut.gguf"
    for n in list(range(0, 200)) + list(range(200, len(good), 37)) + [len(good) - 1]:
        blob = good[:n]
        p.write_bytes(blob)
        info = go.read(blob)
        rc = lib.dq_gguf_open(str(p).encode(), ctypes.byref(h))
        if info is None:
            assert rc in (IO, INVALID_ARG), n
            continue
        assert rc == OK, n
        for name, _, _, _ in info["tensors"]:
            ok = go.read_tensor_raw(blob, info, name) is not None
            got = lib.dq_gguf_read_tensor_raw(h, name.encode(), None, 0, None, None, None)
            assert (got == OK) == ok, (n, name)
        lib.dq_gguf_close(h)


def test_lookup_errors(tmp_path, lib):
    data = gw.gguf_bytes(_kv_all_kinds(), _tensors(), version=3)
    p = tmp_path / "m.gguf"
    p.write_bytes(data)
    with gguf.GgufFile(str(p)) as f:
        h = f._h
        v = ctypes.c_int64()
        assert lib.dq_gguf_get_int(h, b"nope", ctypes.byref(v)) == NOT_SUPPORTED
        assert lib.dq_gguf_get_int(h, b"general.name", ctypes.byref(v)) == NOT_SUPPORTED  # a string
        assert lib.dq_gguf_get_int(h, b"llama.block_count", None) == INVALID_ARG
        assert lib.dq_gguf_find_tensor(h, b"nope") == -1
        assert lib.dq_gguf_read_tensor_raw(h, b"nope", None, 0, None, None, None) == NOT_SUPPORTED
        small = (ctypes.c_uint8 * 4)()
        assert lib.dq_gguf_read_tensor_raw(h, b"f32", small, 4, None, None, None) == INVALID_ARG
        t = _lib.GgufTensor()
        assert lib.dq_gguf_tensor_info(h, 10 ** 6, ctypes.byref(t)) == INVALID_ARG
        with pytest.raises(KeyError):
            f.tensor("nope")
        with pytest.raises(_lib.DqError, match="NOT_SUPPORTED"):
            f.matrix("q5_k")  # a type without device kernels
