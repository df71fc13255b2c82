"""GGUF model files through the library's reader (dq_gguf_* in
include/desireeia_hip.h): the engine's ModelReader interface for this path
(src/gguf/gguf_reader.cpp: open, read_tensor_raw) plus the upload of a
quantized matrix into the device layout (load_matrix ->
cuda_upload_weights, models/dense_forward.cpp:1628-1720).

    with GgufFile("model.gguf") as f:
        f.get("llama.block_count")
        raw, qtype, ne0, rows = f.read_tensor_raw("blk.0.ffn_up.weight")
        m = f.matrix("blk.0.ffn_up.weight")      # ops.QuantMatrix on the device
"""
import ctypes

import numpy as np

from . import _lib

# metadata value types (0-12) and the numpy dtype of the scalar kinds
VALUE_DTYPES = {0: np.uint8, 1: np.int8, 2: np.uint16, 3: np.int16, 4: np.uint32, 5: np.int32, 6: np.float32,
                7: np.uint8, 10: np.uint64, 11: np.int64, 12: np.float64}


class GgufTensorInfo:
    def __init__(self, t: _lib.GgufTensor):
        self.name = t.name.decode("utf-8", "surrogateescape")
        self.type = t.type
        self.dims = list(t.dims[:t.n_dims])
        self.offset = t.offset
        self.nbytes = t.nbytes
        self._data = t.data

    @property
    def ne0(self):
        return self.dims[0] if self.dims else 0

    @property
    def rows(self):
        r = 1
        for d in self.dims[1:]:
            r *= d
        return r

    def __repr__(self):
        return f"GgufTensorInfo({self.name!r}, type={self.type}, dims={self.dims}, nbytes={self.nbytes})"


class GgufFile:
    def __init__(self, path):
        self._lib = _lib.load()
        h = ctypes.c_void_p()
        _lib.check(self._lib.dq_gguf_open(str(path).encode(), ctypes.byref(h)), f"dq_gguf_open({path})")
        self._h = h
        self.path = str(path)

    # ---------------------------------------------------------------- life --
    def close(self):
        if self._h:
            self._lib.dq_gguf_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ------------------------------------------------------------- header --
    @property
    def version(self):
        return self._lib.dq_gguf_version(self._h)

    @property
    def data_offset(self):
        return self._lib.dq_gguf_data_offset(self._h)

    def keys(self):
        n = self._lib.dq_gguf_kv_count(self._h)
        return [self._lib.dq_gguf_kv_key(self._h, i).decode("utf-8", "surrogateescape") for i in range(n)]

    def value_type(self, key):
        return self._lib.dq_gguf_kv_type(self._h, key.encode())

    def get(self, key, default=None):
        """The value of a key: int, float, str, or a list for an array
        (numeric elements decoded, string elements as str)."""
        k = key.encode()
        t = self._lib.dq_gguf_kv_type(self._h, k)
        if t < 0:
            return default
        if t == 8:
            p, n = ctypes.c_void_p(), ctypes.c_uint64()
            _lib.check(self._lib.dq_gguf_get_str(self._h, k, ctypes.byref(p), ctypes.byref(n)), "dq_gguf_get_str")
            return ctypes.string_at(p, n.value).decode("utf-8", "surrogateescape")
        if t == 9:
            et, n, p = ctypes.c_int(), ctypes.c_uint64(), ctypes.c_void_p()
            _lib.check(self._lib.dq_gguf_get_array(self._h, k, ctypes.byref(et), ctypes.byref(n), ctypes.byref(p)),
                       "dq_gguf_get_array")
            return _decode_array(et.value, n.value, p.value)
        if t in (6, 12):
            v = ctypes.c_double()
            _lib.check(self._lib.dq_gguf_get_float(self._h, k, ctypes.byref(v)), "dq_gguf_get_float")
            return v.value
        v = ctypes.c_int64()
        _lib.check(self._lib.dq_gguf_get_int(self._h, k, ctypes.byref(v)), "dq_gguf_get_int")
        return v.value

    # ------------------------------------------------------------ tensors --
    @property
    def n_tensors(self):
        return self._lib.dq_gguf_n_tensors(self._h)

    def tensor(self, i_or_name):
        i = i_or_name if isinstance(i_or_name, int) else self._lib.dq_gguf_find_tensor(self._h, i_or_name.encode())
        if i < 0:
            raise KeyError(i_or_name)
        t = _lib.GgufTensor()
        _lib.check(self._lib.dq_gguf_tensor_info(self._h, i, ctypes.byref(t)), "dq_gguf_tensor_info")
        return GgufTensorInfo(t)

    def tensors(self):
        return [self.tensor(i) for i in range(self.n_tensors)]

    def read_tensor_raw(self, name):
        """ModelReader::read_tensor_raw: (bytes as uint8 array, type, ne0, rows)."""
        k = name.encode()
        ty, ne0, rows = ctypes.c_int(), ctypes.c_uint64(), ctypes.c_uint64()
        _lib.check(self._lib.dq_gguf_read_tensor_raw(self._h, k, None, 0, ctypes.byref(ty), ctypes.byref(ne0),
                                                     ctypes.byref(rows)), f"dq_gguf_read_tensor_raw({name})")
        nbytes = rows.value * self._lib.dq_row_size(ty.value, ne0.value)
        out = np.empty(nbytes, dtype=np.uint8)
        _lib.check(self._lib.dq_gguf_read_tensor_raw(self._h, k, out.ctypes.data, nbytes, None, None, None),
                   f"dq_gguf_read_tensor_raw({name})")
        return out, ty.value, ne0.value, rows.value

    def matrix(self, name, device="cuda"):
        """A Q8_0 / Q4_0 / Q4_K / Q6_K matrix packed into the device layout
        (ops.QuantMatrix)."""
        from . import ops
        raw, ty, ne0, rows = self.read_tensor_raw(name)
        if self._lib.dq_fmt_of_gguf_type(ty) < 0:
            raise _lib.DqError(f"{name}: NOT_SUPPORTED (tensor type {ty} has no device kernels)")
        return ops.QuantMatrix.from_gguf(ty, raw, rows, ne0, device=device)

    def upload(self, name):
        """dq_gguf_upload: the engine's (d_qs, d_scale) device pair straight from
        the map, with fmt, rows and cols (release with cuda_free_device)."""
        fmt, rows, cols = ctypes.c_int(), ctypes.c_uint64(), ctypes.c_uint64()
        qs, sc = ctypes.c_void_p(), ctypes.c_void_p()
        _lib.check(self._lib.dq_gguf_upload(self._h, name.encode(), ctypes.byref(fmt), ctypes.byref(rows),
                                            ctypes.byref(cols), ctypes.byref(qs), ctypes.byref(sc)),
                   f"dq_gguf_upload({name})")
        return fmt.value, rows.value, cols.value, qs.value, sc.value


def _decode_array(et, n, addr):
    if et in VALUE_DTYPES:
        dt = np.dtype(VALUE_DTYPES[et])
        if n == 0:
            return []
        buf = ctypes.string_at(addr, n * dt.itemsize)
        return np.frombuffer(buf, dtype=dt).tolist()
    if et == 8:
        out, p = [], addr
        for _ in range(n):
            ln = int.from_bytes(ctypes.string_at(p, 8), "little")
            out.append(ctypes.string_at(p + 8, ln).decode("utf-8", "surrogateescape"))
            p += 8 + ln
        return out
    raise ValueError(f"array of element type {et} (nested arrays are listed but not decoded)")
