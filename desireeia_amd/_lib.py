"""ctypes binding of libdesireeia_hip.so (the C ABI in include/desireeia_hip.h).

The library is built in-tree by desireeia_amd/build.py. There is no fallback:
if the library is missing, load() raises.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libdesireeia_hip.so")

c_int, c_size, c_i64, c_p, c_f = ctypes.c_int, ctypes.c_size_t, ctypes.c_int64, ctypes.c_void_p, ctypes.c_float
c_u32 = ctypes.c_uint32

# name -> (restype, argtypes)
SIGNATURES = {
    "dq_version": (c_int, []),
    "dq_device_count": (c_int, []),
    "dq_dequantize_row": (c_int, [c_int, c_p, c_p, c_i64, c_p]),
    "dq_weights_bytes": (c_int, [c_int, c_size, c_size, ctypes.POINTER(c_size)]),
    "dq_weights_pack": (c_int, [c_int, c_p, c_size, c_size, c_p, c_p]),
    "dq_weights_dequantize": (c_int, [c_int, c_p, c_size, c_size, c_p, c_p]),
    "dq_quantize_act": (c_int, [c_int, c_p, c_size, c_size, c_p, c_p, c_p, c_p, c_p]),
    "dq_quantize_q8_1_blocks": (c_int, [c_p, c_size, c_p, c_p]),
    "dq_gemv": (c_int, [c_int, c_p, c_size, c_size, c_p, c_p, c_p, c_p, c_p]),
    "dq_gemm_workspace_bytes": (c_int, [c_int, c_size, c_size, c_size, ctypes.POINTER(c_size)]),
    "dq_gemm": (c_int, [c_int, c_p, c_size, c_size, c_p, c_size, c_p, c_p, c_size, c_p]),
    "dq_quantize_act_f16": (c_int, [c_int, c_p, c_size, c_size, c_p, c_p]),
    "dq_gemm_f16act": (c_int, [c_int, c_p, c_size, c_size, c_p, c_size, c_p, c_p]),
    "dq_kv_write": (c_int, [c_p, c_p, c_u32, c_u32, c_p, c_p, c_u32, c_p, c_u32, c_p]),
    "dq_attn_workspace_bytes": (c_int, [c_u32, c_u32, c_u32, c_u32, ctypes.POINTER(c_size)]),
    "dq_attn_decode_q8": (c_int, [c_p, c_p, c_p, c_u32, c_u32, c_u32, c_u32, c_u32, c_p, c_u32, c_p, c_p, c_size,
                                  c_p]),
    "dq_attn_decode_q8_act": (c_int, [c_p, c_p, c_p, c_u32, c_u32, c_u32, c_u32, c_u32, c_p, c_u32, c_p, c_p, c_p,
                                      c_p, c_p, c_size, c_p]),
    "dq_gemv_add": (c_int, [c_int, c_p, c_size, c_size, c_p, c_p, c_p, c_p, c_p, c_p]),
    "dq_rope_cache": (c_int, [c_p, c_u32, c_u32, c_f]),
    "dq_norm_quant": (c_int, [c_p, c_p, c_p, c_p, c_size, c_f, c_p, c_p, c_p, c_p]),
    "dq_silu_quant": (c_int, [c_p, c_p, c_size, c_p, c_p, c_p, c_p]),
    "dq_rope_kv_write": (c_int, [c_p, c_p, c_p, c_p, c_u32, c_u32, c_u32, c_u32, c_p, c_p, c_u32, c_p, c_u32, c_p]),
    "dq_layer_workspace_bytes": (c_int, [c_p, c_u32, ctypes.POINTER(c_size)]),
    "dq_layer_decode": (c_int, [c_p, c_p, c_p, c_p, c_u32, c_p, c_u32, c_p, c_p, c_u32, c_p, c_size, c_p]),
}

_lib = None


class DqError(RuntimeError):
    pass


def load():
    """Loads the HIP library once; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise DqError(f"{LIB_PATH} is missing: run __graft_entry__.build() (or python desireeia_amd/build.py)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


STATUS = {0: "OK", -1: "INVALID_ARG", -2: "NOT_SUPPORTED", -3: "IO"}


def check(rc, what=""):
    if rc != 0:
        raise DqError(f"{what}: {STATUS.get(rc, rc)}")
    return rc
