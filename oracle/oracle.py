"""ctypes wrappers of the CPU checkers (numpy in, numpy out).

TEST INFRASTRUCTURE ONLY - imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product path.

  Oracle()  liboracle.so: the restatement in dq_oracle.c
  Ref()     _ref/libdesireeia_ref.so: the reference engine's own CPU operators
            compiled from /root/reference (Makefile target `ref`); None when
            it has not been built.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libdesireeia_ref.so")
REF_SRC = "/root/reference/src/DesireeIA.LocaleEngine"

Q4_0, Q8_0, Q8_1, Q4_K, Q6_K = 2, 8, 9, 12, 14

c_int, c_size, c_i64, c_p, c_f, c_u32 = (ctypes.c_int, ctypes.c_size_t, ctypes.c_int64, ctypes.c_void_p,
                                         ctypes.c_float, ctypes.c_uint32)


def build(ref=True):
    """Builds liboracle.so and, when the reference tree is present, _ref."""
    subprocess.run(["make", "-s", "-C", HERE, "all"], check=True)
    if ref and os.path.isdir(REF_SRC):
        subprocess.run(["make", "-s", "-j8", "-C", HERE, "ref"], check=True)


def _p(a):
    return a.ctypes.data_as(c_p) if a is not None else None


class LayerArgs(ctypes.Structure):
    _fields_ = [("n_embd", c_u32), ("n_head", c_u32), ("n_head_kv", c_u32), ("head_dim", c_u32), ("n_ff", c_u32),
                ("rms_eps", c_f), ("rope_theta", c_f),
                ("fmt_q", c_int), ("fmt_k", c_int), ("fmt_v", c_int), ("fmt_o", c_int), ("fmt_gate", c_int),
                ("fmt_up", c_int), ("fmt_down", c_int),
                ("wq", c_p), ("wk", c_p), ("wv", c_p), ("wo", c_p), ("wgate", c_p), ("wup", c_p), ("wdown", c_p),
                ("attn_norm", c_p), ("ffn_norm", c_p),
                ("bq", c_p), ("bk", c_p), ("bv", c_p), ("q_norm", c_p), ("k_norm", c_p), ("act_gelu", c_int),
                ("post_attn_norm", c_p), ("post_ffn_norm", c_p), ("wag", c_p), ("fmt_ag", c_int)]


class Oracle:
    def __init__(self, path=ORACLE_SO):
        if not os.path.exists(path):
            build(ref=False)
        L = ctypes.CDLL(path)
        self.L = L
        L.dqo_fp16_to_fp32.restype = c_f
        L.dqo_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        L.dqo_fp32_to_fp16.restype = ctypes.c_uint16
        L.dqo_fp32_to_fp16.argtypes = [c_f]
        L.dqo_dequantize_row.argtypes = [c_int, c_p, c_p, c_i64]
        L.dqo_get_scale_min_k4.argtypes = [c_int, c_p, c_p, c_p]
        L.dqo_pack_scales_min_k4.argtypes = [c_p, c_p, c_p]
        L.dqo_quantize_q8_0.argtypes = [c_p, c_size, c_p, c_p]
        L.dqo_quantize_q8_1.argtypes = [c_p, c_size, c_p, c_p, c_p, c_p]
        L.dqo_quantize_q8k_rep.argtypes = [c_p, c_size, c_p, c_p, c_p]
        L.dqo_kv_quantize_row.argtypes = [c_p, c_size, c_p]
        L.dqo_attn_gate_apply.argtypes = [c_p, c_p, c_u32, c_size]
        L.dqo_matmul.argtypes = [c_int, c_p, c_size, c_size, c_p, c_p, c_size, c_size]
        L.dqo_matmul_f64.argtypes = [c_int, c_p, c_size, c_size, c_p, c_p, c_size, c_size]
        L.dqo_matmul_pq.argtypes = [c_int, c_p, c_size, c_size, c_p, c_p, c_p, c_p, c_size, c_size]
        L.dqo_gemm.argtypes = [c_int, c_p, c_size, c_size, c_p, c_size, c_p, c_size, c_size, c_size, c_size]
        L.dqo_gemm_f64.argtypes = [c_int, c_p, c_size, c_size, c_p, c_size, c_p, c_size, c_size, c_size, c_size]
        L.dqo_gemm_operands.argtypes = [c_int, c_p, c_size, c_size, c_p, c_p, c_p]
        L.dqo_kv_dot_q8_0.restype = c_f
        L.dqo_kv_dot_q8_0.argtypes = [c_p, c_p, c_size]
        L.dqo_kv_axpy_q8_0.argtypes = [c_p, c_p, c_size, c_f]
        L.dqo_attn_decode_q8.argtypes = [c_p, c_p, c_p, c_u32, c_u32, c_u32, c_u32, c_u32, c_p]
        L.dqo_attn_decode_q8_f64.argtypes = [c_p, c_p, c_p, c_u32, c_u32, c_u32, c_u32, c_u32, c_p]
        L.dqo_attn_prefill_q8.argtypes = [c_p, c_p, c_u32, c_u32, c_u32, c_u32, c_u32, c_p, c_p, c_size, c_size,
                                          c_u32, c_u32, c_f]
        L.dqo_moe_route.restype = c_u32
        L.dqo_moe_route.argtypes = [c_p, c_u32, c_u32, c_int, c_f, c_p, c_p]
        L.dqo_rms_norm.argtypes = [c_p, c_p, c_p, c_size, c_f]
        L.dqo_rope_cache.argtypes = [c_p, c_size, c_u32, c_f]
        L.dqo_rope_neox.argtypes = [c_p, c_size, c_p]
        L.dqo_silu.restype = c_f
        L.dqo_silu.argtypes = [c_f]
        for fn in ("dqo_gelu_tanh", "dqo_exp_avx2", "dqo_geglu"):
            getattr(L, fn).restype = c_f
            getattr(L, fn).argtypes = [c_f]
        L.dqo_softmax.argtypes = [c_p, c_size]
        L.dqo_layer_decode.argtypes = [ctypes.POINTER(LayerArgs), c_p, c_p, c_u32, c_p, c_p, c_p, c_p, c_p, c_p]
        L.dqo_layer_prefill.argtypes = [ctypes.POINTER(LayerArgs), c_p, c_p, c_u32, c_u32, c_u32, c_p, c_p]
        L.dqo_moe_ffn.argtypes = [c_int, c_p, c_p, c_p, c_u32, c_u32, c_u32, c_p, c_p, c_u32, c_u32, c_int, c_p,
                                  c_u32, c_u32]

    # -- scalars / formats
    def fp16_to_fp32(self, h):
        return self.L.dqo_fp16_to_fp32(int(h))

    def fp32_to_fp16(self, f):
        return self.L.dqo_fp32_to_fp16(float(f))

    def dequantize_row(self, qtype, src, n):
        src = np.ascontiguousarray(src, dtype=np.uint8)
        y = np.empty(n, dtype=np.float32)
        rc = self.L.dqo_dequantize_row(qtype, _p(src), _p(y), n)
        if rc != 0:
            raise ValueError(f"dequantize_row rc={rc}")
        return y

    def get_scale_min_k4(self, j, q12):
        q12 = np.ascontiguousarray(q12, dtype=np.uint8)
        sc = np.zeros(1, np.uint8)
        mn = np.zeros(1, np.uint8)
        self.L.dqo_get_scale_min_k4(j, _p(q12), _p(sc), _p(mn))
        return int(sc[0]), int(mn[0])

    def pack_scales_min_k4(self, sc, mn):
        out = np.zeros(12, np.uint8)
        self.L.dqo_pack_scales_min_k4(_p(np.ascontiguousarray(sc, np.uint8)), _p(np.ascontiguousarray(mn, np.uint8)),
                                      _p(out))
        return out

    # -- activation quantizers
    def quantize_q8_1(self, x):
        x = np.ascontiguousarray(x, np.float32).reshape(-1)
        n = x.size
        q = np.empty(n, np.int8)
        d = np.empty(n // 32, np.float32)
        isum = np.empty(n // 32, np.int32)
        fsum = np.empty(n // 32, np.float32)
        self.L.dqo_quantize_q8_1(_p(x), n, _p(q), _p(d), _p(isum), _p(fsum))
        return q, d, isum, fsum

    def quantize_q8k_rep(self, x):
        x = np.ascontiguousarray(x, np.float32).reshape(-1)
        n = x.size
        q = np.empty(n, np.int8)
        d = np.empty(n // 32, np.float32)
        isum = np.empty(n // 32, np.int32)
        self.L.dqo_quantize_q8k_rep(_p(x), n, _p(q), _p(d), _p(isum))
        return q, d, isum

    def kv_quantize_row(self, x):
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty((x.size + 31) // 32 * 34, np.uint8)
        self.L.dqo_kv_quantize_row(_p(x), x.size, _p(out))
        return out

    # -- GEMV / GEMM

    def attn_gate_apply(self, ao, gate, n_head, hd):
        """Head h of ao times 1 / (1 + expf(-gate[h])) (dqo_attn_gate_apply)."""
        ao = np.ascontiguousarray(ao, np.float32).copy()
        gate = np.ascontiguousarray(gate, np.float32)
        self.L.dqo_attn_gate_apply(ao.ctypes.data, gate.ctypes.data, n_head, hd)
        return ao
    def matmul(self, qtype, w, rows, cols, x, row0=0, row1=0):
        w = np.ascontiguousarray(w, np.uint8)
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros(rows, np.float32)
        rc = self.L.dqo_matmul(qtype, _p(w), rows, cols, _p(x), _p(y), row0, row1)
        if rc != 0:
            raise ValueError(f"matmul rc={rc}")
        return y

    def matmul_f64(self, qtype, w, rows, cols, x, row0=0, row1=0):
        w = np.ascontiguousarray(w, np.uint8)
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros(rows, np.float64)
        rc = self.L.dqo_matmul_f64(qtype, _p(w), rows, cols, _p(x), _p(y), row0, row1)
        if rc != 0:
            raise ValueError(f"matmul_f64 rc={rc}")
        return y

    def gemm(self, qtype, w, rows, cols, x, n_tok, row0=0, row1=0, t0=0, t1=0, f64=False):
        w = np.ascontiguousarray(w, np.uint8)
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros((n_tok, rows), np.float64 if f64 else np.float32)
        fn = self.L.dqo_gemm_f64 if f64 else self.L.dqo_gemm
        rc = fn(qtype, _p(w), rows, cols, _p(x), n_tok, _p(y), row0, row1, t0, t1)
        if rc != 0:
            raise ValueError(f"gemm rc={rc}")
        return y

    # -- attention / router / glue
    def gemm_operands(self, qtype, w, rows, cols):
        """unpack_row of every row: int8 weights [rows][cols], scale and Q4_K
        offset of each 16 columns [rows][cols/16] (the prefill GEMM's weight
        operands; y = (a q) (dx q_x)^T - m sx^T)."""
        q = np.empty((rows, cols), np.int8)
        a = np.empty((rows, cols // 16), np.float32)
        m = np.empty((rows, cols // 16), np.float32)
        rc = self.L.dqo_gemm_operands(qtype, _p(np.ascontiguousarray(w)), rows, cols, _p(q), _p(a), _p(m))
        if rc != 0:
            raise ValueError(f"gemm_operands rc={rc}")
        return q, a, m

    def kv_dot(self, q, row, dim):
        return self.L.dqo_kv_dot_q8_0(_p(np.ascontiguousarray(q, np.float32)),
                                      _p(np.ascontiguousarray(row, np.uint8)), dim)

    def kv_axpy(self, y, row, dim, w):
        y = np.ascontiguousarray(y, np.float32).copy()
        self.L.dqo_kv_axpy_q8_0(_p(y), _p(np.ascontiguousarray(row, np.uint8)), dim, w)
        return y

    def attn_decode(self, q, kc, vc, n_head, n_head_kv, hd, cc_start, pos, f64=False):
        q = np.ascontiguousarray(q, np.float32)
        out = np.zeros(n_head * hd, np.float64 if f64 else np.float32)
        fn = self.L.dqo_attn_decode_q8_f64 if f64 else self.L.dqo_attn_decode_q8
        fn(_p(q), _p(np.ascontiguousarray(kc, np.uint8)), _p(np.ascontiguousarray(vc, np.uint8)),
           n_head, n_head_kv, hd, cc_start, pos, _p(out))
        return out

    def attn_prefill(self, q_all, kc, vc, n_tok, n_head, n_head_kv, hd, pos0, n_swa=0, q_dim=None, out=None):
        return _attn_prefill(self.L.dqo_attn_prefill_q8, q_all, kc, vc, n_tok, n_head, n_head_kv, hd, pos0, n_swa,
                             q_dim, out)

    def moe_route(self, logits, k, norm_w=True, w_scale=1.0):
        logits = np.ascontiguousarray(logits, np.float32)
        ids = np.zeros(max(k, 1), np.uint32)
        wts = np.zeros(max(k, 1), np.float32)
        n = self.L.dqo_moe_route(_p(logits), logits.size, k, int(norm_w), w_scale, _p(ids), _p(wts))
        return ids[:n].copy(), wts[:n].copy()

    def rms_norm(self, x, w, eps):
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty_like(x)
        self.L.dqo_rms_norm(_p(x), _p(np.ascontiguousarray(w, np.float32)), _p(y), x.size, eps)
        return y

    def rope_cache(self, n_rot, pos, theta):
        c = np.empty(n_rot, np.float32)
        self.L.dqo_rope_cache(_p(c), n_rot, pos, theta)
        return c

    def rope_neox(self, v, n_rot, cache):
        v = np.ascontiguousarray(v, np.float32).copy()
        self.L.dqo_rope_neox(_p(v), n_rot, _p(np.ascontiguousarray(cache, np.float32)))
        return v

    def softmax(self, s):
        s = np.ascontiguousarray(s, np.float32).copy()
        self.L.dqo_softmax(_p(s), s.size)
        return s

    def layer_prefill(self, args, kc, vc, pos0, x, n_swa=0):
        """x: [n_tok][n_embd]; kc/vc: writable uint8 numpy arrays (one layer)."""
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty_like(x)
        rc = self.L.dqo_layer_prefill(ctypes.byref(args), _p(kc), _p(vc), pos0, x.shape[0], n_swa, _p(x), _p(out))
        if rc != 0:
            raise ValueError(f"layer_prefill rc={rc}")
        return out

    def layer_decode(self, args, kc, vc, pos, x):
        """args: LayerArgs; kc/vc: writable uint8 numpy arrays (one layer)."""
        x = np.ascontiguousarray(x, np.float32)
        E = args.n_embd
        qd = args.n_head * args.head_dim
        kvd = args.n_head_kv * args.head_dim
        out = np.empty(E, np.float32)
        q = np.empty(qd, np.float32)
        k = np.empty(kvd, np.float32)
        v = np.empty(kvd, np.float32)
        ao = np.empty(qd, np.float32)
        rc = self.L.dqo_layer_decode(ctypes.byref(args), _p(kc), _p(vc), pos, _p(x), _p(out), _p(q), _p(k), _p(v),
                                     _p(ao))
        if rc != 0:
            raise ValueError(f"layer_decode rc={rc}")
        return out, q, k, v, ao

    def moe_ffn(self, qtype, wgate, wup, wdown, n_expert, n_embd, n_ff, x, logits, n_tok, k_used, norm_w=True,
                t0=0, t1=0):
        out = np.zeros((n_tok, n_embd), np.float32)
        rc = self.L.dqo_moe_ffn(qtype, _p(wgate), _p(wup), _p(wdown), n_expert, n_embd, n_ff,
                                _p(np.ascontiguousarray(x, np.float32)), _p(np.ascontiguousarray(logits, np.float32)),
                                n_tok, k_used, int(norm_w), _p(out), t0, t1)
        if rc != 0:
            raise ValueError(f"moe_ffn rc={rc}")
        return out


class Ref:
    """The reference engine's own CPU operators (oracle/_ref)."""

    def __init__(self, path=REF_SO):
        L = ctypes.CDLL(path)
        self.L = L
        L.dqr_set_threads.argtypes = [c_int]
        L.dqr_threads.restype = c_int
        L.dqr_i8_isa.restype = ctypes.c_char_p
        L.dqr_fp16_to_fp32.restype = c_f
        L.dqr_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        L.dqr_fp32_to_fp16.restype = ctypes.c_uint16
        L.dqr_fp32_to_fp16.argtypes = [c_f]
        L.dqr_dequantize_row.argtypes = [c_int, c_p, c_p, c_i64]
        L.dqr_quantize_q8_0.argtypes = [c_p, c_size, c_p, c_p]
        L.dqr_quantize_q8k_rep.argtypes = [c_p, c_size, c_p, c_p, c_p]
        L.dqr_matmul.argtypes = [c_int, c_p, c_size, c_size, c_p, c_p]
        L.dqr_matmul_batch.argtypes = [c_int, c_p, c_size, c_size, c_p, c_size, c_p]
        L.dqr_kv_quantize_row.argtypes = [c_p, c_size, c_p]
        L.dqr_kv_dot_q8_0.restype = c_f
        L.dqr_kv_dot_q8_0.argtypes = [c_p, c_p, c_size]
        L.dqr_kv_axpy_q8_0.argtypes = [c_p, c_p, c_size, c_f]
        L.dqr_moe_route.restype = c_u32
        L.dqr_moe_route.argtypes = [c_p, c_u32, c_u32, c_int, c_f, c_p, c_p]
        L.dqr_sample_candidates.restype = ctypes.c_int32
        L.dqr_sample_candidates.argtypes = [c_f, ctypes.c_int32, c_f, c_f, c_f, c_f, ctypes.c_int32, c_u32, c_u32, c_p,
                                            c_p, c_size, c_p, c_size, c_p]
        L.dqr_attn_decode_q8.argtypes = [c_p, c_p, c_p, c_u32, c_u32, c_u32, c_u32, c_u32, c_p]
        L.dqr_attention_prefill_q8.argtypes = [c_p, c_p, c_u32, c_u32, c_u32, c_u32, c_u32, c_p, c_p, c_size, c_size,
                                               c_u32, c_u32, c_f]

    @staticmethod
    def available():
        return os.path.exists(REF_SO)

    def set_threads(self, n):
        self.L.dqr_set_threads(n)

    def threads(self):
        return self.L.dqr_threads()

    def isa(self):
        return self.L.dqr_i8_isa().decode()

    def fp16_to_fp32(self, h):
        return self.L.dqr_fp16_to_fp32(int(h))

    def fp32_to_fp16(self, f):
        return self.L.dqr_fp32_to_fp16(float(f))

    def dequantize_row(self, qtype, src, n):
        src = np.ascontiguousarray(src, dtype=np.uint8)
        y = np.empty(n, dtype=np.float32)
        rc = self.L.dqr_dequantize_row(qtype, _p(src), _p(y), n)
        if rc != 0:
            raise ValueError(f"ref dequantize_row rc={rc}")
        return y

    def quantize_q8_0(self, x):
        x = np.ascontiguousarray(x, np.float32).reshape(-1)
        q = np.empty(x.size, np.int8)
        d = np.empty(x.size // 32, np.float32)
        self.L.dqr_quantize_q8_0(_p(x), x.size, _p(q), _p(d))
        return q, d

    def quantize_q8k_rep(self, x):
        x = np.ascontiguousarray(x, np.float32).reshape(-1)
        q = np.empty(x.size, np.int8)
        d = np.empty(x.size // 32, np.float32)
        s = np.empty(x.size // 32, np.int32)
        self.L.dqr_quantize_q8k_rep(_p(x), x.size, _p(q), _p(d), _p(s))
        return q, d, s

    def matmul(self, qtype, w, rows, cols, x):
        y = np.zeros(rows, np.float32)
        rc = self.L.dqr_matmul(qtype, _p(np.ascontiguousarray(w, np.uint8)), rows, cols,
                               _p(np.ascontiguousarray(x, np.float32)), _p(y))
        if rc != 0:
            raise ValueError(f"ref matmul rc={rc}")
        return y

    def matmul_batch(self, qtype, w, rows, cols, x, n_tok):
        y = np.zeros((n_tok, rows), np.float32)
        rc = self.L.dqr_matmul_batch(qtype, _p(np.ascontiguousarray(w, np.uint8)), rows, cols,
                                     _p(np.ascontiguousarray(x, np.float32)), n_tok, _p(y))
        if rc != 0:
            raise ValueError(f"ref matmul_batch rc={rc}")
        return y

    def kv_quantize_row(self, x):
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty((x.size + 31) // 32 * 34, np.uint8)
        self.L.dqr_kv_quantize_row(_p(x), x.size, _p(out))
        return out

    def kv_dot(self, q, row, dim):
        return self.L.dqr_kv_dot_q8_0(_p(np.ascontiguousarray(q, np.float32)),
                                      _p(np.ascontiguousarray(row, np.uint8)), dim)

    def kv_axpy(self, y, row, dim, w):
        y = np.ascontiguousarray(y, np.float32).copy()
        self.L.dqr_kv_axpy_q8_0(_p(y), _p(np.ascontiguousarray(row, np.uint8)), dim, w)
        return y

    def moe_route(self, logits, k, norm_w=True, w_scale=1.0):
        logits = np.ascontiguousarray(logits, np.float32)
        ids = np.zeros(max(k, 1, logits.size), np.uint32)
        wts = np.zeros(max(k, 1, logits.size), np.float32)
        n = self.L.dqr_moe_route(_p(logits), logits.size, k, int(norm_w), w_scale, _p(ids), _p(wts))
        return ids[:n].copy(), wts[:n].copy()


    def sample_candidates(self, ids, vals, hist, temperature=0.0, top_k=40, top_p=0.95, repeat=1.0, freq=0.0,
                          present=0.0, last_n=64, seed=1, skip=0):
        """The reference's Sampler::sample_candidates with a seeded generator:
        (token, u) where u is the uniform number the device draw is given."""
        return _ref_sample(self.L, ids, vals, list(hist), temperature, top_k, top_p, repeat, freq, present, last_n,
                           seed, skip)

    def attn_decode(self, q, kc, vc, n_head, n_head_kv, hd, cc_start, pos):
        """Decode attention composed from the reference's kv_dot_q8_0 /
        kv_axpy_q8_0 over heads on its thread pool (dense_forward.cpp:4014-4066)."""
        out = np.zeros(n_head * hd, np.float32)
        self.L.dqr_attn_decode_q8(_p(np.ascontiguousarray(q, np.float32)), _p(np.ascontiguousarray(kc, np.uint8)),
                                  _p(np.ascontiguousarray(vc, np.uint8)), n_head, n_head_kv, hd, cc_start, pos, _p(out))
        return out

    def attn_prefill(self, q_all, kc, vc, n_tok, n_head, n_head_kv, hd, pos0, n_swa=0, q_dim=None, out=None):
        return _attn_prefill(self.L.dqr_attention_prefill_q8, q_all, kc, vc, n_tok, n_head, n_head_kv, hd, pos0,
                             n_swa, q_dim, out)


def _ref_sample(L, ids, vals, hist, temperature, top_k, top_p, repeat, freq, present, last_n, seed, skip):
    ids = np.ascontiguousarray(ids, np.int32)
    vals = np.ascontiguousarray(vals, np.float32)
    nh = len(hist)
    h = np.ascontiguousarray(hist if nh else [0], np.int32)
    u = ctypes.c_float()
    tok = L.dqr_sample_candidates(temperature, top_k, top_p, repeat, freq, present, last_n, seed, skip, _p(ids),
                                  _p(vals), ids.size, _p(h), nh, ctypes.byref(u))
    return tok, u.value


def _attn_prefill(fn, q_all, kc, vc, n_tok, n_head, n_head_kv, hd, pos0, n_swa, q_dim, out):
    """q_all [n_tok][q_dim] -> out [n_tok][q_dim]; caches of one layer laid out
    [pos][kv head][hd/32 Q8_0 blocks]."""
    q_dim = q_dim or n_head * hd
    q_all = np.ascontiguousarray(q_all, np.float32).reshape(-1)
    out = np.zeros(n_tok * q_dim, np.float32) if out is None else np.ascontiguousarray(out, np.float32).copy()
    row_bytes = hd // 32 * 34
    rc = fn(_p(q_all), _p(out), n_tok, n_head, n_head // n_head_kv, hd, q_dim, _p(np.ascontiguousarray(kc, np.uint8)),
            _p(np.ascontiguousarray(vc, np.uint8)), row_bytes, n_head_kv * row_bytes, pos0, n_swa,
            float(np.float32(1.0) / np.sqrt(np.float32(hd))))
    if rc != 0:
        raise ValueError(f"attn_prefill rc={rc}")
    return out


_oracle = None
_ref = None


def oracle():
    global _oracle
    if _oracle is None:
        _oracle = Oracle()
    return _oracle


def ref():
    """The compiled reference, or None when oracle/_ref has not been built."""
    global _ref
    if _ref is None and Ref.available():
        _ref = Ref()
    return _ref
