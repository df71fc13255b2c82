"""Host-side mirror of the reference's operator interface for the quantized
path, over torch device tensors. torch only provides device memory and the
current stream; every computation is a call into libdesireeia_hip.so.

Names follow the reference operators (src/DesireeIA.LocaleEngine/):
  dequantize_row      quant/quant.cpp:912   desireeia_dequantize_row
  quantize_q8_0       core/quant.cpp:15     (per-32 activation quantizer)
  quantize_act_q8k_rep core/matmul.cpp:1660 (per-256, replicated per 32)
  matmul_q8_0/q4_0/q4_k/q6_k  core/matmul.cpp:294-417, :2008, :2569
"""
import ctypes

import torch

from . import _lib
from .synth import BLOCK, FMT_OF_TYPE, Q4_0, Q4_K, Q6_K, Q8_0, TYPE_OF_FMT

ACT_Q8_0, ACT_Q8K_REP = 0, 1


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _dev(t, device="cuda"):
    if isinstance(t, torch.Tensor):
        return t.to(device)
    return torch.from_numpy(t).to(device)


def dequantize_row(qtype, src, n):
    """GGUF blocks (uint8 device tensor) -> n fp32 values, bit-exact."""
    lib = _lib.load()
    out = torch.empty(n, dtype=torch.float32, device=src.device)
    _lib.check(lib.dq_dequantize_row(qtype, _ptr(src), _ptr(out), n, _stream()), "dq_dequantize_row")
    return out


class Activation:
    """Quantized activation triple (q int8, scale per 32, isum per 32, fsum per 32)."""

    def __init__(self, q, scale, isum, fsum, kind):
        self.q, self.scale, self.isum, self.fsum, self.kind = q, scale, isum, fsum, kind


def empty_act(shape, kind, device):
    """Preallocated activation buffers for quantize_act(out=...)."""
    nb = shape[-1] // 32
    q = torch.empty(shape, dtype=torch.int8, device=device)
    scale = torch.empty(tuple(shape[:-1]) + (nb,), dtype=torch.float32, device=device)
    isum = torch.empty(tuple(shape[:-1]) + (nb,), dtype=torch.int32, device=device)
    fsum = torch.empty(tuple(shape[:-1]) + (nb,), dtype=torch.float32, device=device)
    return Activation(q, scale, isum, fsum, kind)


def quantize_act(x, kind=ACT_Q8_0, out=None):
    """x: fp32 [n_tok, cols] or [cols] device tensor."""
    lib = _lib.load()
    x = x.contiguous()
    cols = x.shape[-1]
    n_tok = x.numel() // cols
    a = out if out is not None else empty_act(tuple(x.shape), kind, x.device)
    _lib.check(lib.dq_quantize_act(kind, _ptr(x), cols, n_tok, _ptr(a.q), _ptr(a.scale), _ptr(a.isum),
                                   _ptr(a.fsum), _stream()), "dq_quantize_act")
    a.kind = kind
    return a


def quantize_q8_0(x):
    return quantize_act(x, ACT_Q8_0)


def quantize_act_q8k_rep(x):
    return quantize_act(x, ACT_Q8K_REP)


def quantize_q8_1_blocks(x):
    """GGUF block_q8_1 bytes of a flat fp32 device tensor."""
    lib = _lib.load()
    x = x.contiguous()
    out = torch.empty(x.numel() // 32 * 36, dtype=torch.uint8, device=x.device)
    _lib.check(lib.dq_quantize_q8_1_blocks(_ptr(x), x.numel(), _ptr(out), _stream()), "dq_quantize_q8_1_blocks")
    return out


class QuantMatrix:
    """A rows x cols quantized matrix in the on-device layout (cuda_upload_weights)."""

    def __init__(self, fmt, rows, cols, buf):
        self.fmt, self.rows, self.cols, self.buf = fmt, rows, cols, buf

    @property
    def qtype(self):
        return TYPE_OF_FMT[self.fmt]

    @staticmethod
    def nbytes(fmt, rows, cols):
        lib = _lib.load()
        n = ctypes.c_size_t(0)
        _lib.check(lib.dq_weights_bytes(fmt, rows, cols, ctypes.byref(n)), "dq_weights_bytes")
        return n.value

    @classmethod
    def from_gguf(cls, qtype, gguf, rows, cols, device="cuda"):
        """gguf: GGUF row bytes (numpy or tensor, rows*row_bytes uint8)."""
        lib = _lib.load()
        fmt = FMT_OF_TYPE[qtype]
        src = _dev(gguf, device).reshape(-1).contiguous()
        buf = torch.empty(cls.nbytes(fmt, rows, cols), dtype=torch.uint8, device=device)
        _lib.check(lib.dq_weights_pack(fmt, _ptr(src), rows, cols, _ptr(buf), _stream()), "dq_weights_pack")
        return cls(fmt, rows, cols, buf)

    def clone(self):
        return QuantMatrix(self.fmt, self.rows, self.cols, self.buf.clone())

    def dequantize(self):
        lib = _lib.load()
        out = torch.empty(self.rows, self.cols, dtype=torch.float32, device=self.buf.device)
        _lib.check(lib.dq_weights_dequantize(self.fmt, _ptr(self.buf), self.rows, self.cols, _ptr(out), _stream()),
                   "dq_weights_dequantize")
        return out


def act_kind_for(fmt):
    """The activation quantizer of the reference CPU GEMV for this format."""
    return ACT_Q8_0 if fmt in (FMT_OF_TYPE[Q8_0], FMT_OF_TYPE[Q4_0]) else ACT_Q8K_REP


def gemv(mat, act, out=None):
    lib = _lib.load()
    y = out if out is not None else torch.empty(mat.rows, dtype=torch.float32, device=mat.buf.device)
    _lib.check(lib.dq_gemv(mat.fmt, _ptr(mat.buf), mat.rows, mat.cols, _ptr(act.q), _ptr(act.scale),
                           _ptr(act.isum), _ptr(y), _stream()), "dq_gemv")
    return y


def gemv_group(mats, act, outs=None, residuals=None):
    """Several matrices with the same cols reading one activation
    (matmul_fused_pq / matvec_shared_group): one launch per distinct format,
    Q4_K and Q6_K together in one where cols <= 4096."""
    lib = _lib.load()
    n = len(mats)
    ys = outs if outs is not None else [torch.empty(m.rows, dtype=torch.float32, device=m.buf.device) for m in mats]
    res = residuals if residuals is not None else [None] * n
    jobs = (_lib.GemvJob * max(n, 1))()
    for j, m in enumerate(mats):
        jobs[j].fmt, jobs[j].d_w, jobs[j].rows = m.fmt, m.buf.data_ptr(), m.rows
        jobs[j].d_y = ys[j].data_ptr()
        jobs[j].d_res = res[j].data_ptr() if res[j] is not None else None
    cols = mats[0].cols if n else 0
    _lib.check(lib.dq_gemv_group(jobs, n, cols, _ptr(act.q), _ptr(act.scale), _ptr(act.isum), _stream()),
               "dq_gemv_group")
    return ys


def matmul(mat, x, out=None):
    """y = W x with the semantics of the reference's matmul_<fmt> (batch 1):
    one launch, the activation quantized in-kernel (dq_gemv_f32)."""
    lib = _lib.load()
    x = x.contiguous()
    y = out if out is not None else torch.empty(mat.rows, dtype=torch.float32, device=mat.buf.device)
    _lib.check(lib.dq_gemv_f32(mat.fmt, _ptr(mat.buf), mat.rows, mat.cols, _ptr(x), _ptr(y), _stream()),
               "dq_gemv_f32")
    return y


def matmul_group(mats, x, outs=None, residuals=None):
    """Several matrices reading the fp32 activation x, any formats mixed
    (dq_gemv_group_f32): one launch per distinct format."""
    lib = _lib.load()
    x = x.contiguous()
    n = len(mats)
    ys = outs if outs is not None else [torch.empty(m.rows, dtype=torch.float32, device=m.buf.device) for m in mats]
    res = residuals if residuals is not None else [None] * n
    jobs = (_lib.GemvJob * max(n, 1))()
    for j, m in enumerate(mats):
        jobs[j].fmt, jobs[j].d_w, jobs[j].rows = m.fmt, m.buf.data_ptr(), m.rows
        jobs[j].d_y = ys[j].data_ptr()
        jobs[j].d_res = res[j].data_ptr() if res[j] is not None else None
    _lib.check(lib.dq_gemv_group_f32(jobs, n, mats[0].cols if n else 0, _ptr(x), _stream()), "dq_gemv_group_f32")
    return ys


FUSE_NORM, FUSE_SILU, FUSE_GEGLU, FUSE_NORM_SILU, FUSE_NORM_GEGLU = 1, 2, 3, 4, 5


def gemv_group_fused(mats, kind, a, b, eps=0.0, outs=None, residuals=None):
    """Grouped per-256 GEMV whose kernel forms its activation from fp32
    inputs (dq_gemv_group_fused): kind FUSE_NORM y = rms_norm(a) * b (b the
    norm weights), FUSE_SILU / FUSE_GEGLU y = act(a) * b (gate, up);
    FUSE_NORM_SILU / FUSE_NORM_GEGLU: mats = (gate, up), outs[0] receives
    act(gate) * up."""
    lib = _lib.load()
    a, b = a.contiguous(), b.contiguous()
    n = len(mats)
    ys = outs if outs is not None else [torch.empty(m.rows, dtype=torch.float32, device=m.buf.device) for m in mats]
    res = residuals if residuals is not None else [None] * n
    jobs = (_lib.GemvJob * max(n, 1))()
    for j, m in enumerate(mats):
        jobs[j].fmt, jobs[j].d_w, jobs[j].rows = m.fmt, m.buf.data_ptr(), m.rows
        jobs[j].d_y = ys[j].data_ptr()
        jobs[j].d_res = res[j].data_ptr() if res[j] is not None else None
    _lib.check(lib.dq_gemv_group_fused(jobs, n, mats[0].cols if n else 0, kind, _ptr(a), _ptr(b), eps, _stream()),
               "dq_gemv_group_fused")
    return ys


def gemm_workspace(mat, n_tok):
    lib = _lib.load()
    n = ctypes.c_size_t(0)
    _lib.check(lib.dq_gemm_workspace_bytes(mat.fmt, mat.rows, mat.cols, n_tok, ctypes.byref(n)), "dq_gemm_workspace_bytes")
    return torch.empty(max(n.value, 1), dtype=torch.uint8, device=mat.buf.device)


GEMM_TILES = 0x200


class GemmTiles:
    """The opt-in tile copy of a matrix for the prefill GEMM
    (dq_gemm_tiles_pack): each 64-row slice's bytes of one GEMM stage in one
    contiguous run. Passed to gemm() in place of the QuantMatrix; results are
    bit-identical. The packed matrix stays what the decode GEMV reads."""

    def __init__(self, mat):
        lib = _lib.load()
        n = ctypes.c_size_t(0)
        _lib.check(lib.dq_gemm_tiles_bytes(mat.fmt, mat.rows, mat.cols, ctypes.byref(n)), "dq_gemm_tiles_bytes")
        self.buf = torch.empty(n.value, dtype=torch.uint8, device=mat.buf.device)
        _lib.check(lib.dq_gemm_tiles_pack(mat.fmt, _ptr(mat.buf), mat.rows, mat.cols, _ptr(self.buf), _stream()),
                   "dq_gemm_tiles_pack")
        self.fmt = mat.fmt | GEMM_TILES
        self.rows, self.cols = mat.rows, mat.cols


def gemm(mat, x, out=None, work=None):
    """Y[n_tok][rows] = X W^T with the semantics of matmul_<fmt>_batch (n_tok >= 4),
    reference core/matmul.cpp:2090-2125."""
    lib = _lib.load()
    x = x.contiguous()
    n_tok = x.shape[0]
    y = out if out is not None else torch.empty(n_tok, mat.rows, dtype=torch.float32, device=x.device)
    wk = work if work is not None else gemm_workspace(mat, n_tok)
    _lib.check(lib.dq_gemm(mat.fmt, _ptr(mat.buf), mat.rows, mat.cols, _ptr(x), n_tok, _ptr(y), _ptr(wk),
                           wk.numel(), _stream()), "dq_gemm")
    return y


class KVCache:
    """Q8_0 K and V caches of one layer on the device, [n_ctx][n_head_kv][hd/32 x 34 B]
    (models/dense_forward.cpp:2425, :4038-4043)."""

    def __init__(self, n_ctx, n_head_kv, hd, device="cuda"):
        self.n_ctx, self.n_head_kv, self.hd = n_ctx, n_head_kv, hd
        self.pos_bytes = n_head_kv * hd // 32 * 34
        self.k = torch.zeros(n_ctx * self.pos_bytes, dtype=torch.uint8, device=device)
        self.v = torch.zeros(n_ctx * self.pos_bytes, dtype=torch.uint8, device=device)

    def write(self, k, v, pos):
        """Quantizes the rows k, v ([n_head_kv * hd] fp32) into position pos.
        pos: int, or an int32 device tensor read when the kernel runs."""
        lib = _lib.load()
        dpos = pos if isinstance(pos, torch.Tensor) else None
        _lib.check(lib.dq_kv_write(_ptr(k.contiguous()), _ptr(v.contiguous()), self.n_head_kv, self.hd,
                                   _ptr(self.k), _ptr(self.v), 0 if dpos is not None else int(pos), _ptr(dpos),
                                   self.n_ctx, _stream()), "dq_kv_write")


    def write_batch(self, k, v, pos0):
        """Quantizes the rows of k, v ([n_tok][n_head_kv * hd] fp32) into
        positions [pos0, pos0 + n_tok)."""
        lib = _lib.load()
        k, v = k.contiguous(), v.contiguous()
        _lib.check(lib.dq_kv_write_batch(_ptr(k), _ptr(v), k.shape[-1], k.shape[0], self.n_head_kv, self.hd,
                                         _ptr(self.k), _ptr(self.v), int(pos0), self.n_ctx, _stream()),
                   "dq_kv_write_batch")

    def rope_write_batch(self, q, k, v, rope, n_rot, pos0):
        """RoPE of q (in place, [n_tok][q_ld]) and k with the per-token table
        rope ([n_tok][n_rot] device floats, or None), then the K/V rows of the
        tokens into positions [pos0, pos0 + n_tok)."""
        lib = _lib.load()
        k, v = k.contiguous(), v.contiguous()
        n_head = q.shape[-1] // self.hd
        _lib.check(lib.dq_rope_kv_write_batch(_ptr(q), _ptr(k), _ptr(v), q.shape[-1], k.shape[-1], _ptr(rope),
                                              n_rot, q.shape[0], n_head, self.n_head_kv, self.hd, _ptr(self.k),
                                              _ptr(self.v), int(pos0), self.n_ctx, _stream()),
                   "dq_rope_kv_write_batch")


def attn_prefill_workspace(n_tok, n_head, n_head_kv, hd, device="cuda"):
    lib = _lib.load()
    n = ctypes.c_size_t(0)
    _lib.check(lib.dq_attn_prefill_workspace_bytes(n_tok, n_head, n_head_kv, hd, ctypes.byref(n)),
               "dq_attn_prefill_workspace_bytes")
    return torch.empty(max(n.value, 1), dtype=torch.uint8, device=device)


def attention_prefill(q, cache, n_head, pos0, n_swa=0, out=None, work=None, split=True):
    """Prefill attention of q [n_tok][q_dim] (token t at position pos0 + t)
    over the cache, causal (n_swa 0) or over a sliding window of n_swa.
    split=False runs without a workspace (no key split)."""
    lib = _lib.load()
    q = q.contiguous()
    n_tok, q_dim = q.shape
    o = out if out is not None else torch.zeros(n_tok, q_dim, dtype=torch.float32, device=q.device)
    wk = work if work is not None or not split else attn_prefill_workspace(n_tok, n_head, cache.n_head_kv, cache.hd,
                                                                             q.device)
    _lib.check(lib.dq_attn_prefill_q8(_ptr(q), _ptr(cache.k), _ptr(cache.v), n_tok, n_head, cache.n_head_kv,
                                      cache.hd, q_dim, int(pos0), int(n_swa), cache.n_ctx, _ptr(o), _ptr(wk),
                                      wk.numel() if wk is not None else 0, _stream()), "dq_attn_prefill_q8")
    return o


def head_logits(mat, x, norm_w, eps=1e-5, out=None):
    """Final RMSNorm of x [cols] (weight norm_w) and the head product: logits [rows]."""
    lib = _lib.load()
    n = ctypes.c_size_t(0)
    _lib.check(lib.dq_head_workspace_bytes(mat.fmt, mat.rows, mat.cols, ctypes.byref(n)), "dq_head_workspace_bytes")
    wk = torch.empty(n.value, dtype=torch.uint8, device=x.device)
    y = out if out is not None else torch.empty(mat.rows, dtype=torch.float32, device=x.device)
    _lib.check(lib.dq_head_logits(mat.fmt, _ptr(mat.buf), mat.rows, mat.cols, _ptr(x.contiguous()),
                                  _ptr(norm_w.contiguous()), ctypes.c_float(eps), _ptr(y), _ptr(wk), wk.numel(),
                                  _stream()), "dq_head_logits")
    return y


def topk(v, kk):
    """(ids int32 [kk], values [kk]): the kk largest of v, largest first, lower index on ties."""
    lib = _lib.load()
    n = ctypes.c_size_t(0)
    _lib.check(lib.dq_topk_workspace_bytes(v.numel(), kk, ctypes.byref(n)), "dq_topk_workspace_bytes")
    wk = torch.empty(n.value, dtype=torch.uint8, device=v.device)
    ids = torch.empty(kk, dtype=torch.int32, device=v.device)
    vals = torch.empty(kk, dtype=torch.float32, device=v.device)
    _lib.check(lib.dq_topk(_ptr(v.contiguous()), v.numel(), kk, _ptr(ids), _ptr(vals), _ptr(wk), wk.numel(),
                           _stream()), "dq_topk")
    return ids, vals


class DeviceSampler:
    """The draw of the pipelined decode on the device (dq_sample_candidates)
    with its state: last token, 256-token history ring, readback slots."""

    def __init__(self, device="cuda", hist=()):
        self.state = torch.zeros(ctypes.sizeof(_lib.SampleState), dtype=torch.uint8, device=device)
        self.reset(hist)

    def reset(self, hist):
        lib = _lib.load()
        h = (ctypes.c_int32 * max(len(hist), 1))(*hist)
        _lib.check(lib.dq_sample_reset(_ptr(self.state), h if len(hist) else None, len(hist), _stream()),
                   "dq_sample_reset")

    def sample(self, ids, vals, args):
        lib = _lib.load()
        _lib.check(lib.dq_sample_candidates(_ptr(vals.contiguous()), _ptr(ids.contiguous()), ids.numel(),
                                            ctypes.byref(args), _ptr(self.state), _stream()), "dq_sample_candidates")

    def read(self):
        st = _lib.SampleState.from_buffer_copy(bytes(self.state.cpu().numpy()))
        return st


def embed_q8_0(mat, tok, mul=0.0, out=None):
    """Row tok (int32 device tensor of one element) of a packed Q8_0 matrix, times mul when non-zero."""
    lib = _lib.load()
    y = out if out is not None else torch.empty(mat.cols, dtype=torch.float32, device=tok.device)
    _lib.check(lib.dq_embed_q8_0(_ptr(mat.buf), mat.rows, mat.cols, _ptr(tok), ctypes.c_float(mul), _ptr(y),
                                 _stream()), "dq_embed_q8_0")
    return y


def attn_workspace(n_head, n_head_kv, hd, n_ctx, device="cuda"):
    lib = _lib.load()
    n = ctypes.c_size_t(0)
    _lib.check(lib.dq_attn_workspace_bytes(n_head, n_head_kv, hd, n_ctx, ctypes.byref(n)), "dq_attn_workspace_bytes")
    return torch.empty(max(n.value, 1), dtype=torch.uint8, device=device)


def attention_decode(q, cache, n_head, pos, cc_start=0, out=None, work=None):
    """Decode attention of q [n_head * hd] over positions [cc_start, pos] of
    the cache; pos an int or an int32 device tensor."""
    lib = _lib.load()
    hd = cache.hd
    o = out if out is not None else torch.empty(n_head * hd, dtype=torch.float32, device=q.device)
    wk = work if work is not None else attn_workspace(n_head, cache.n_head_kv, hd, cache.n_ctx, q.device)
    dpos = pos if isinstance(pos, torch.Tensor) else None
    _lib.check(lib.dq_attn_decode_q8(_ptr(q.contiguous()), _ptr(cache.k), _ptr(cache.v), n_head, cache.n_head_kv,
                                     hd, cc_start, 0 if dpos is not None else int(pos), _ptr(dpos), cache.n_ctx,
                                     _ptr(o), _ptr(wk), wk.numel(), _stream()), "dq_attn_decode_q8")
    return o


class LayerDesc(ctypes.Structure):
    """dq_layer_t of include/desireeia_hip.h."""
    _fields_ = [("n_embd", ctypes.c_uint32), ("n_head", ctypes.c_uint32), ("n_head_kv", ctypes.c_uint32),
                ("head_dim", ctypes.c_uint32), ("n_rot", ctypes.c_uint32), ("n_ff", ctypes.c_uint32),
                ("rms_eps", ctypes.c_float),
                ("fmt_q", ctypes.c_int), ("fmt_k", ctypes.c_int), ("fmt_v", ctypes.c_int), ("fmt_o", ctypes.c_int),
                ("fmt_gate", ctypes.c_int), ("fmt_up", ctypes.c_int), ("fmt_down", ctypes.c_int),
                ("wq", ctypes.c_void_p), ("wk", ctypes.c_void_p), ("wv", ctypes.c_void_p), ("wo", ctypes.c_void_p),
                ("wgate", ctypes.c_void_p), ("wup", ctypes.c_void_p), ("wdown", ctypes.c_void_p),
                ("attn_norm", ctypes.c_void_p), ("ffn_norm", ctypes.c_void_p),
                ("bq", ctypes.c_void_p), ("bk", ctypes.c_void_p), ("bv", ctypes.c_void_p),
                ("q_norm", ctypes.c_void_p), ("k_norm", ctypes.c_void_p), ("act_gelu", ctypes.c_int),
                ("post_attn_norm", ctypes.c_void_p), ("post_ffn_norm", ctypes.c_void_p),
                ("wag", ctypes.c_void_p), ("fmt_ag", ctypes.c_int),
                ("tq", ctypes.c_void_p), ("tk", ctypes.c_void_p), ("tv", ctypes.c_void_p), ("to", ctypes.c_void_p),
                ("tgate", ctypes.c_void_p), ("tup", ctypes.c_void_p), ("tdown", ctypes.c_void_p),
                ("tag", ctypes.c_void_p)]


def rope_cache(n_rot, pos, theta):
    """Host cos/sin table of rope_cache_init (dq_rope_cache), as a CPU float tensor."""
    lib = _lib.load()
    out = torch.empty(n_rot, dtype=torch.float32)
    _lib.check(lib.dq_rope_cache(ctypes.c_void_p(out.data_ptr()), n_rot, pos, theta), "dq_rope_cache")
    return out


class DecoderLayer:
    """One decoder layer on the device (dq_layer_decode): packed weights,
    norm weights and its Q8_0 KV cache. mats: dict name -> QuantMatrix for
    q, k, v, o, gate, up, down."""

    NAMES = ("q", "k", "v", "o", "gate", "up", "down")

    def __init__(self, mats, attn_norm, ffn_norm, n_head, n_head_kv, head_dim, n_ctx, rms_eps=1e-5,
                 rope_theta=500000.0, n_rot=None, device="cuda", bias=None, qk_norm=None, act_gelu=False,
                 post_norms=None, attn_gate=None):
        """bias: optional (bq, bk, bv) float tensors; qk_norm: optional
        (q_norm, k_norm) [head_dim] weights (Qwen-style layers); act_gelu: a
        gated GELU FFN; post_norms: optional (post_attn_norm, post_ffn_norm)
        [n_embd] sandwich-norm weights; attn_gate: optional QuantMatrix
        [n_head][n_embd], the per-head attention output gate."""
        self.mats = mats
        self.attn_norm = attn_norm.to(device).float().contiguous()
        self.ffn_norm = ffn_norm.to(device).float().contiguous()
        self.n_embd = mats["q"].cols
        self.n_head, self.n_head_kv, self.head_dim = n_head, n_head_kv, head_dim
        self.n_ff = mats["up"].rows
        self.n_rot = n_rot or head_dim
        self.rope_theta = rope_theta
        d = LayerDesc(self.n_embd, n_head, n_head_kv, head_dim, self.n_rot, self.n_ff, rms_eps)
        for nm in self.NAMES:
            setattr(d, "fmt_" + nm, mats[nm].fmt)
            setattr(d, "w" + nm, mats[nm].buf.data_ptr())
        d.attn_norm = self.attn_norm.data_ptr()
        d.ffn_norm = self.ffn_norm.data_ptr()
        d.act_gelu = int(act_gelu)
        self.attn_gate = attn_gate
        if attn_gate is not None:
            d.wag, d.fmt_ag = attn_gate.buf.data_ptr(), attn_gate.fmt
        self.extras = {}
        for names, vals in ((("bq", "bk", "bv"), bias), (("q_norm", "k_norm"), qk_norm),
                            (("post_attn_norm", "post_ffn_norm"), post_norms)):
            for nm, t in zip(names, vals or ()):
                if t is not None:
                    self.extras[nm] = t.to(device).float().contiguous()
                    setattr(d, nm, self.extras[nm].data_ptr())
        self.desc = d
        self.cache = KVCache(n_ctx, n_head_kv, head_dim, device)
        lib = _lib.load()
        n = ctypes.c_size_t(0)
        _lib.check(lib.dq_layer_workspace_bytes(ctypes.byref(d), n_ctx, ctypes.byref(n)), "dq_layer_workspace_bytes")
        self.work = torch.empty(max(n.value, 1), dtype=torch.uint8, device=device)
        self.rope = torch.empty(self.n_rot, dtype=torch.float32, device=device)

    def use_gemm_tiles(self):
        """Gives the prefill layer tile copies of the matrices (GemmTiles):
        the weights are then held twice; the decode layer is unchanged."""
        self.tiles = {nm: GemmTiles(self.mats[nm]) for nm in self.NAMES}
        for nm in self.NAMES:
            setattr(self.desc, "t" + nm, self.tiles[nm].buf.data_ptr())
        if self.attn_gate is not None:
            self.tiles["ag"] = GemmTiles(self.attn_gate)
            self.desc.tag = self.tiles["ag"].buf.data_ptr()
        return self

    def set_rope(self, pos):
        self.rope.copy_(rope_cache(self.n_rot, pos, self.rope_theta))

    def decode(self, x, pos, out=None, rope_ready=False, cc_start=0):
        """x: device [n_embd]; pos: int (the RoPE table is rebuilt unless
        rope_ready) or an int32 device tensor (then the caller keeps
        self.rope in step with it)."""
        lib = _lib.load()
        y = out if out is not None else torch.empty_like(x)
        dpos = pos if isinstance(pos, torch.Tensor) else None
        if dpos is None and not rope_ready:
            self.set_rope(int(pos))
        _lib.check(lib.dq_layer_decode(ctypes.byref(self.desc), _ptr(x), _ptr(y), _ptr(self.rope),
                                       0 if dpos is not None else int(pos), _ptr(dpos), cc_start,
                                       _ptr(self.cache.k), _ptr(self.cache.v), self.cache.n_ctx, _ptr(self.work),
                                       self.work.numel(), _stream()), "dq_layer_decode")
        return y


    def prefill_workspace(self, n_tok):
        lib = _lib.load()
        n = ctypes.c_size_t(0)
        _lib.check(lib.dq_layer_prefill_workspace_bytes(ctypes.byref(self.desc), n_tok, ctypes.byref(n)),
                   "dq_layer_prefill_workspace_bytes")
        return torch.empty(max(n.value, 1), dtype=torch.uint8, device=self.attn_norm.device)

    def prefill(self, x, pos0, out=None, n_swa=0, work=None, rope=None):
        """x: device [n_tok][n_embd], the chunk's tokens at positions pos0..;
        the RoPE tables of the chunk are built here unless given ([n_tok][n_rot])."""
        lib = _lib.load()
        n_tok = x.shape[0]
        y = out if out is not None else torch.empty_like(x)
        if rope is None:
            rope = torch.stack([rope_cache(self.n_rot, pos0 + t, self.rope_theta) for t in range(n_tok)]).to(x.device)
        wk = work if work is not None else self.prefill_workspace(n_tok)
        _lib.check(lib.dq_layer_prefill(ctypes.byref(self.desc), _ptr(x), _ptr(y), _ptr(rope), int(pos0), n_tok,
                                        int(n_swa), _ptr(self.cache.k), _ptr(self.cache.v), self.cache.n_ctx,
                                        _ptr(wk), wk.numel(), _stream()), "dq_layer_prefill")
        return y


class MoeLayer:
    """Expert FFN of one MoE layer on the device (dq_moe_ffn): stacked Q4_K
    experts, gate/up [n_expert * n_ff][n_embd] and down [n_expert * n_embd][n_ff]
    (models/dense_forward.cpp:1524-1560, combined as at :4160-4181)."""

    FMT_Q4_K_TILES = 0x105

    def __init__(self, wgate, wup, wdown, n_expert, n_expert_used, norm_w=True, w_scale=1.0, tiled=True):
        """wgate/wup/wdown: QuantMatrix (stacked experts). tiled: the expert
        GEMMs read the expert-tile copies of the matrices (dq_moe_tiles_pack,
        contiguous weight DMA), and the layer keeps only those (the packed rows
        are freed once the caller drops its own references: keeping both would
        hold the experts' bytes twice); False: the packed rows themselves."""
        self.n_embd, self.n_ff = wgate.cols, wdown.cols
        bufs, fmt = [m.buf for m in (wgate, wup, wdown)], wgate.fmt
        if tiled:
            lib = _lib.load()
            bufs = []
            for m, rows in ((wgate, self.n_ff), (wup, self.n_ff), (wdown, self.n_embd)):
                n = ctypes.c_size_t(0)
                _lib.check(lib.dq_moe_tiles_bytes(n_expert, rows, m.cols, ctypes.byref(n)), "dq_moe_tiles_bytes")
                t = torch.empty(n.value, dtype=torch.uint8, device=m.buf.device)
                _lib.check(lib.dq_moe_tiles_pack(_ptr(m.buf), n_expert, rows, m.cols, _ptr(t), _stream()),
                           "dq_moe_tiles_pack")
                bufs.append(t)
            fmt = self.FMT_Q4_K_TILES
        self.bufs = bufs
        d = _lib.MoeDesc(n_expert, n_expert_used, self.n_embd, self.n_ff, int(norm_w), w_scale, fmt,
                         bufs[0].data_ptr(), bufs[1].data_ptr(), bufs[2].data_ptr())
        self.desc = d
        self._work = None

    def workspace(self, n_tok, device):
        lib = _lib.load()
        n = ctypes.c_size_t(0)
        _lib.check(lib.dq_moe_workspace_bytes(ctypes.byref(self.desc), n_tok, ctypes.byref(n)),
                   "dq_moe_workspace_bytes")
        if self._work is None or self._work.numel() < n.value:
            self._work = torch.empty(max(n.value, 1), dtype=torch.uint8, device=device)
        return self._work

    def __call__(self, x, logits, out=None):
        """x [n_tok][n_embd], logits [n_tok][n_expert] fp32 device tensors."""
        lib = _lib.load()
        x = x.contiguous()
        logits = logits.contiguous()
        n_tok = x.shape[0]
        y = out if out is not None else torch.empty(n_tok, self.n_embd, dtype=torch.float32, device=x.device)
        wk = self.workspace(n_tok, x.device)
        _lib.check(lib.dq_moe_ffn(ctypes.byref(self.desc), _ptr(x), _ptr(logits), n_tok, _ptr(y), _ptr(wk),
                                  wk.numel(), _stream()), "dq_moe_ffn")
        return y


def moe_route(logits, k, norm_w=True, w_scale=1.0):
    """Router (moe_route_ex, softmax gating) of logits [n_tok][n_expert]:
    ids int32 [n_tok][k], weights fp32 [n_tok][k]."""
    lib = _lib.load()
    logits = logits.contiguous()
    n_tok, n_exp = logits.shape
    ids = torch.empty(n_tok, k, dtype=torch.int32, device=logits.device)
    wts = torch.empty(n_tok, k, dtype=torch.float32, device=logits.device)
    _lib.check(lib.dq_moe_route(_ptr(logits), n_tok, n_exp, k, int(norm_w), w_scale, _ptr(ids), _ptr(wts), _stream()),
               "dq_moe_route")
    return ids, wts
