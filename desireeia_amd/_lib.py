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
    "dq_stream_read": (c_int, [c_p, c_size, c_u32, c_u32, c_p, c_u32, c_p]),
    "dq_lds_read_probe": (c_int, [c_p, c_u32, c_u32, c_int, c_p, c_u32, c_p]),
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
    "dq_gemm_tiles_bytes": (c_int, [c_int, c_size, c_size, ctypes.POINTER(c_size)]),
    "dq_gemm_tiles_pack": (c_int, [c_int, c_p, c_size, c_size, c_p, c_p]),
    "dq_kv_write": (c_int, [c_p, c_p, c_u32, c_u32, c_p, c_p, c_u32, c_p, c_u32, c_p]),
    "dq_attn_workspace_bytes": (c_int, [c_u32, c_u32, c_u32, c_u32, ctypes.POINTER(c_size)]),
    "dq_attn_decode_q8": (c_int, [c_p, c_p, c_p, c_u32, c_u32, c_u32, c_u32, c_u32, c_p, c_u32, c_p, c_p, c_size,
                                  c_p]),
    "dq_attn_decode_q8_noalloc": (c_int, [c_p, c_p, c_p, c_u32, c_u32, c_u32, c_u32, c_u32, c_p, c_u32, c_p, c_p]),
    "dq_attn_decode_q8_act": (c_int, [c_p, c_p, c_p, c_u32, c_u32, c_u32, c_u32, c_u32, c_p, c_u32, c_p, c_p, c_p,
                                      c_p, c_p, c_size, c_p]),
    "dq_attn_rope_kv_decode": (c_int, [c_p, c_p, c_p, c_p, c_u32, c_p, c_p, c_u32, c_u32, c_u32, c_u32, c_u32, c_p,
                                       c_u32, c_p, c_p, c_p, c_p, c_p, c_size, c_p]),
    "dq_gemv_add": (c_int, [c_int, c_p, c_size, c_size, c_p, c_p, c_p, c_p, c_p, c_p]),
    "dq_gemv_group": (c_int, [c_p, c_size, c_size, c_p, c_p, c_p, c_p]),
    "dq_gemv_f32": (c_int, [c_int, c_p, c_size, c_size, c_p, c_p, c_p]),
    "dq_gemv_group_f32": (c_int, [c_p, c_size, c_size, c_p, c_p]),
    "dq_gemv_group_fused": (c_int, [c_p, c_size, c_size, c_int, c_p, c_p, c_f, c_p]),
    "dq_rope_cache": (c_int, [c_p, c_u32, c_u32, c_f]),
    "dq_norm_quant": (c_int, [c_p, c_p, c_p, c_p, c_size, c_f, c_p, c_p, c_p, c_p]),
    "dq_silu_quant": (c_int, [c_p, c_p, c_size, c_p, c_p, c_p, c_p]),
    "dq_rope_kv_write": (c_int, [c_p, c_p, c_p, c_p, c_u32, c_u32, c_u32, c_u32, c_p, c_p, c_u32, c_p, c_u32, c_p]),
    "dq_kv_write_batch": (c_int, [c_p, c_p, c_size, c_u32, c_u32, c_u32, c_p, c_p, c_u32, c_u32, c_p]),
    "dq_rope_kv_write_batch": (c_int, [c_p, c_p, c_p, c_size, c_size, c_p, c_u32, c_u32, c_u32, c_u32, c_u32, c_p,
                                       c_p, c_u32, c_u32, c_p]),
    "dq_attn_prefill_workspace_bytes": (c_int, [c_u32, c_u32, c_u32, c_u32, ctypes.POINTER(c_size)]),
    "dq_attn_prefill_q8": (c_int, [c_p, c_p, c_p, c_u32, c_u32, c_u32, c_u32, c_u32, c_u32, c_u32, c_u32, c_p,
                                   c_p, c_size, c_p]),
    "dq_layer_workspace_bytes": (c_int, [c_p, c_u32, ctypes.POINTER(c_size)]),
    "dq_layer_prefill_workspace_bytes": (c_int, [c_p, c_u32, ctypes.POINTER(c_size)]),
    "dq_rms_norm_rows": (c_int, [c_p, c_p, c_p, c_p, c_size, c_size, c_f, c_p, c_p]),
    "dq_head_workspace_bytes": (c_int, [c_int, c_size, c_size, ctypes.POINTER(c_size)]),
    "dq_head_logits": (c_int, [c_int, c_p, c_size, c_size, c_p, c_p, c_f, c_p, c_p, c_size, c_p]),
    "dq_topk_workspace_bytes": (c_int, [c_u32, c_u32, ctypes.POINTER(c_size)]),
    "dq_topk": (c_int, [c_p, c_u32, c_u32, c_p, c_p, c_p, c_size, c_p]),
    "dq_sample_reset": (c_int, [c_p, c_p, c_size, c_p]),
    "dq_sample_candidates": (c_int, [c_p, c_p, c_u32, c_p, c_p, c_p]),
    "dq_embed_q8_0": (c_int, [c_p, c_size, c_size, c_p, c_f, c_p, c_p]),
    "cuda_head_forward": (c_int, [c_int, c_p, c_p, c_p, c_size, c_f, c_size, c_p]),
    "cuda_head_forward_topk": (c_int, [c_int, c_p, c_p, c_p, c_size, c_f, c_size, c_u32, c_p, c_p]),
    "cuda_head_forward_sample": (c_int, [c_int, c_p, c_p, c_p, c_size, c_f, c_size, c_p]),
    "cuda_sample_wait": (c_int, [c_u32, c_p]),
    "cuda_sample_history": (c_int, [c_p, c_size]),
    "cuda_fetch_x": (c_int, [c_p, c_size]),
    "dq_layer_prefill": (c_int, [c_p, c_p, c_p, c_p, c_u32, c_u32, c_u32, c_p, c_p, c_u32, c_p, c_size, c_p]),
    "dq_layer_decode": (c_int, [c_p, c_p, c_p, c_p, c_u32, c_p, c_u32, c_p, c_p, c_u32, c_p, c_size, c_p]),
    "dq_silu_mul": (c_int, [c_p, c_p, c_size, c_p, c_p]),
    "dq_moe_route": (c_int, [c_p, c_u32, c_u32, c_u32, c_int, c_f, c_p, c_p, c_p]),
    "dq_moe_tiles_bytes": (c_int, [c_u32, c_size, c_size, ctypes.POINTER(c_size)]),
    "dq_moe_tiles_pack": (c_int, [c_p, c_u32, c_size, c_size, c_p, c_p]),
    "dq_moe_workspace_bytes": (c_int, [c_p, c_u32, ctypes.POINTER(c_size)]),
    "dq_moe_ffn": (c_int, [c_p, c_p, c_p, c_u32, c_p, c_p, c_size, c_p]),
    # GGUF files (host)
    "dq_row_size": (c_size, [c_int, c_i64]),
    "dq_fmt_of_gguf_type": (c_int, [c_int]),
    "dq_gguf_open": (c_int, [ctypes.c_char_p, c_p]),
    "dq_gguf_close": (None, [c_p]),
    "dq_gguf_version": (c_int, [c_p]),
    "dq_gguf_data_offset": (ctypes.c_uint64, [c_p]),
    "dq_gguf_kv_count": (c_i64, [c_p]),
    "dq_gguf_kv_key": (ctypes.c_char_p, [c_p, c_i64]),
    "dq_gguf_kv_type": (c_int, [c_p, ctypes.c_char_p]),
    "dq_gguf_get_int": (c_int, [c_p, ctypes.c_char_p, ctypes.POINTER(c_i64)]),
    "dq_gguf_get_float": (c_int, [c_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_double)]),
    "dq_gguf_get_str": (c_int, [c_p, ctypes.c_char_p, ctypes.POINTER(c_p), ctypes.POINTER(ctypes.c_uint64)]),
    "dq_gguf_get_array": (c_int, [c_p, ctypes.c_char_p, ctypes.POINTER(c_int), ctypes.POINTER(ctypes.c_uint64),
                                  ctypes.POINTER(c_p)]),
    "dq_gguf_n_tensors": (c_i64, [c_p]),
    "dq_gguf_find_tensor": (c_i64, [c_p, ctypes.c_char_p]),
    "dq_gguf_tensor_info": (c_int, [c_p, c_i64, c_p]),
    "dq_gguf_read_tensor_raw": (c_int, [c_p, ctypes.c_char_p, c_p, c_size, ctypes.POINTER(c_int),
                                        ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)]),
    "dq_gguf_upload": (c_int, [c_p, ctypes.c_char_p, ctypes.POINTER(c_int), ctypes.POINTER(ctypes.c_uint64),
                               ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(c_p), ctypes.POINTER(c_p)]),
    # engine layer (core/engine.h GPU block); struct arguments as void*
    "cuda_gpu_count": (ctypes.c_int32, []),
    "cuda_probe_gpu": (ctypes.c_bool, [ctypes.c_int32, c_p, c_size, c_p, c_p, c_p, c_p, c_p]),
    "matmul_q8_0_cuda_upload_weights": (ctypes.c_bool, [c_p, c_size, c_size, c_p, c_p]),
    "cuda_upload_weights": (ctypes.c_bool, [c_int, c_p, c_size, c_size, c_p, c_p]),
    "cuda_free_device": (None, [c_p]),
    "cuda_backend_shutdown": (None, []),
    "matmul_kquant_cuda_resident": (c_int, [c_int, c_p, c_size, c_size, c_p, c_p]),
    "matmul_kquant_cuda_resident_same_x": (c_int, [c_p, c_size, c_size, c_p]),
    "matmul_q8_0_cuda_resident": (c_int, [c_p, c_p, c_size, c_size, c_p, c_p]),
    "matmul_q8_0_cuda_resident_group": (c_int, [c_p, c_size, c_size, c_p]),
    "matmul_q8_0_cuda": (c_int, [c_p, c_size, c_size, c_p, c_p]),
    "matmul_kquant_cuda_batch": (c_int, [c_int, c_p, c_size, c_size, c_p, c_size, c_p]),
    "matmul_q8_0_cuda_ffn_gated": (c_int, [c_p, c_p, c_p, c_p, c_p, c_p, c_size, c_size, c_p, c_p, c_int]),
    "cuda_kv_cache_reserve": (ctypes.c_bool, [c_size]),
    "cuda_kv_cache_release": (None, []),
    "cuda_kv_cache_upload": (ctypes.c_bool, [c_p, c_p, c_size]),
    "cuda_kv_cache_download": (ctypes.c_bool, [c_p, c_p, c_size]),
    "cuda_kv_cache_write": (ctypes.c_bool, [c_size, c_p, c_p, c_size]),
    "cuda_kv_cache_read": (ctypes.c_bool, [c_size, c_p, c_p, c_size]),
    "cuda_kv_cache_move": (ctypes.c_bool, [c_size, c_size, c_size]),
    "cuda_set_attention_long": (None, [ctypes.c_bool]),
    "cuda_drop_graphs": (None, []),
    "cuda_attention_out": (c_int, [c_p, c_p, c_p, c_u32, c_u32, c_u32, c_u32, c_size, c_u32, c_u32, c_size, c_size,
                                   c_p, c_int, c_size]),
    "cuda_qkv_attention_out": (c_int, [c_p]),
    "cuda_layer_forward": (c_int, [c_p]),
    "cuda_attention_batch": (c_int, [c_p, c_p, c_u32, c_u32, c_u32, c_u32, c_u32, c_size, c_size, c_size, c_u32,
                                     c_u32]),
    "cuda_layer_forward_batch": (c_int, [c_p]),
    "cuda_prefill_chunk_tokens": (c_int, []),
}



class GgufTensor(ctypes.Structure):
    """dq_gguf_tensor_t"""
    _fields_ = [("name", ctypes.c_char_p), ("type", c_int), ("n_dims", c_int), ("dims", ctypes.c_uint64 * 4),
                ("offset", ctypes.c_uint64), ("nbytes", ctypes.c_uint64), ("data", c_p)]


class CudaKQuantJob(ctypes.Structure):
    """core/engine.h:536 (include/desireeia_hip.h)."""
    _fields_ = [("format", c_int), ("d_w", c_p), ("rows", c_size), ("y", c_p)]


class CudaQ80Job(ctypes.Structure):
    """core/engine.h:598-603."""
    _fields_ = [("d_qs", c_p), ("d_scale", c_p), ("rows", c_size), ("y", c_p)]


class CudaQkvAttnArgs(ctypes.Structure):
    """core/engine.h:675-691."""
    _fields_ = ([(n, c_p) for n in ("wq_qs", "wq_scale", "wk_qs", "wk_scale", "wv_qs", "wv_scale", "wo_qs",
                                    "wo_scale", "bq", "bk", "bv", "attn_in", "rope_cache", "proj", "host_k_row",
                                    "host_v_row")]
                + [("n_embd", c_size), ("q_dim", c_size), ("kv_dim", c_size)]
                + [(n, c_u32) for n in ("n_head", "n_head_kv", "heads_per_kv", "head_dim", "n_rot")]
                + [("kv_layer_off", c_size), ("cc_start", c_u32), ("pos", c_u32)])


class CudaLayerArgs(ctypes.Structure):
    """core/engine.h:698-751."""
    _fields_ = ([(n, c_p) for n in ("wq_qs", "wq_scale", "wk_qs", "wk_scale", "wv_qs", "wv_scale", "wo_qs",
                                    "wo_scale", "wgate_qs", "wgate_scale", "wup_qs", "wup_scale", "wdown_qs",
                                    "wdown_scale", "wag_qs", "wag_scale", "bq", "bk", "bv", "attn_norm_w",
                                    "ffn_norm_w", "q_norm_w", "k_norm_w", "post_attn_norm_w", "post_ffn_norm_w", "x",
                                    "rope_cache", "x_out")]
                + [(n, c_size) for n in ("n_embd", "q_dim", "kv_dim", "n_ff")]
                + [(n, c_u32) for n in ("n_head", "n_head_kv", "heads_per_kv", "head_dim", "n_rot")]
                + [("kv_layer_off", c_size), ("cc_start", c_u32), ("pos", c_u32), ("rms_eps", c_f),
                   ("act_gelu", c_int)]
                + [(n, c_int) for n in ("fmt_q", "fmt_k", "fmt_v", "fmt_o", "fmt_gate", "fmt_up", "fmt_down",
                                        "fmt_ag", "upload_x", "download_x", "upload_dyn")]
                + [("dyn_all", c_p), ("rope_all", c_p), ("n_slots", c_u32), ("rope_stride", c_u32),
                   ("layer_slot", c_u32), ("x_from_token", c_int), ("embd_qs", c_p), ("embd_scale", c_p),
                   ("embd_mul", c_f)])


class CudaLayerBatchArgs(ctypes.Structure):
    """core/engine.h:764-796."""
    _fields_ = ([(n, c_p) for n in ("wq_qs", "wq_scale", "wk_qs", "wk_scale", "wv_qs", "wv_scale", "wo_qs",
                                    "wo_scale", "wgate_qs", "wgate_scale", "wup_qs", "wup_scale", "wdown_qs",
                                    "wdown_scale", "wag_qs", "wag_scale", "bq", "bk", "bv", "attn_norm_w",
                                    "ffn_norm_w", "q_norm_w", "k_norm_w", "post_attn_norm_w", "post_ffn_norm_w", "x",
                                    "x_out")]
                + [("x_out_row0", c_u32), ("rope_caches", c_p), ("host_kcache", c_p), ("host_vcache", c_p)]
                + [(n, c_size) for n in ("n_embd", "q_dim", "kv_dim", "n_ff")]
                + [(n, c_u32) for n in ("n_head", "n_head_kv", "heads_per_kv", "head_dim", "n_rot")]
                + [("kv_layer_off", c_size)]
                + [(n, c_u32) for n in ("pos0", "n_tok", "n_swa", "x_row0", "n_total")]
                + [("rms_eps", c_f), ("act_gelu", c_int)]
                + [(n, c_int) for n in ("fmt_q", "fmt_k", "fmt_v", "fmt_o", "fmt_gate", "fmt_up", "fmt_down",
                                        "fmt_ag", "upload_x", "download_x", "upload_rope", "prepare_weights",
                                        "rope_slot")])


class CudaSampleArgs(ctypes.Structure):
    """core/engine.h:570-579."""
    _fields_ = [("temperature", c_f), ("top_k", ctypes.c_int32), ("top_p", c_f), ("penalty_repeat", c_f),
                ("penalty_freq", c_f), ("penalty_present", c_f), ("penalty_last_n", ctypes.c_int32), ("kk", c_u32),
                ("logit_scale", c_f), ("u", c_f), ("append_input", c_int), ("slot", c_u32)]


class SampleState(ctypes.Structure):
    """dq_sample_state_t."""
    _fields_ = [("tok", ctypes.c_int32), ("len", c_u32), ("wpos", c_u32), ("ring", ctypes.c_int32 * 4),
                ("hist", ctypes.c_int32 * 256)]


class MoeDesc(ctypes.Structure):
    """dq_moe_t of include/desireeia_hip.h."""
    _fields_ = [("n_expert", c_u32), ("n_expert_used", c_u32), ("n_embd", c_u32), ("n_ff", c_u32),
                ("norm_w", c_int), ("w_scale", c_f), ("fmt", c_int), ("wgate", c_p), ("wup", c_p), ("wdown", c_p)]


class GemvJob(ctypes.Structure):
    """dq_gemv_job_t of include/desireeia_hip.h."""
    _fields_ = [("fmt", c_int), ("d_w", c_p), ("rows", c_size), ("d_y", c_p), ("d_res", c_p)]


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
