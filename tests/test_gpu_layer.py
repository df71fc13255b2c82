"""One Llama-style decoder layer on the GPU (dq_layer_decode) against the
oracle's composition of the reference layer (models/dense_forward.cpp
:3897-4257): layer output within 1e-3 norm-wise, the KV rows written at pos
within the Q8_0 step of the oracle's, and the fused pieces (norm+quantize,
silu+quantize, RoPE+KV write) bit-exact against the oracle on the same
inputs."""
import ctypes

import numpy as np
import pytest
import torch

from desireeia_amd import _lib, ops, synth

pytestmark = pytest.mark.gpu
TOL = 1e-3
Q4K, Q6K = synth.Q4_K, synth.Q6_K


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


class HostLayer:
    """The host side of a synthetic layer: weights, norms, the prior cache and
    the oracle's arguments, with the shape attributes the stage chains read
    (n_head, n_head_kv, mats[nm].fmt/rows/cols, cache.pos_bytes)."""

    def __init__(self, orc, E, n_head, n_kv, F, n_ctx, n_prior, seed, norm_scale=(1.0, 1.0), types=None,
                 qwen=False, gelu=False, sandwich=False, attn_gate=False, hd=128):
        from types import SimpleNamespace as NS

        from oracle.oracle import LayerArgs
        self.hd = self.head_dim = hd
        qd, kvd = n_head * hd, n_kv * hd
        # Q4_K_M mix: Q4_K everywhere but attn_v and ffn_down (Q6_K)
        shapes = {"q": (Q4K, qd, E), "k": (Q4K, kvd, E), "v": (Q6K, kvd, E), "o": (Q4K, E, qd),
                  "gate": (Q4K, F, E), "up": (Q4K, F, E), "down": (Q6K, E, F)}
        for nm, qt in (types or {}).items():
            shapes[nm] = (qt,) + shapes[nm][1:]
        if attn_gate:  # per-head attention output gate [n_head][n_embd], Q8_0
            shapes["ag"] = (synth.Q8_0, n_head, E)
        self.shapes = shapes
        gg = {nm: (qt, synth.gen_weights(qt, r, c, seed=seed + i)) for i, (nm, (qt, r, c)) in enumerate(shapes.items())}
        rng = np.random.default_rng(seed)
        self.attn_norm = (norm_scale[0] * (1 + 0.02 * rng.standard_normal(E))).astype(np.float32)
        self.ffn_norm = (norm_scale[1] * (1 + 0.02 * rng.standard_normal(E))).astype(np.float32)
        self.n_head, self.n_head_kv = n_head, n_kv
        self.mats = {nm: NS(fmt=synth.FMT_OF_TYPE[qt], rows=r, cols=c) for nm, (qt, r, c) in shapes.items()}
        pb = n_kv * hd // 32 * 34
        self.cache = NS(pos_bytes=pb)
        # prior cache: N(0,1) rows quantized (kv_quantize_row)
        self.kc = np.zeros(n_ctx * pb, np.uint8)
        self.vc = np.zeros(n_ctx * pb, np.uint8)
        if n_prior:
            self.kc[:n_prior * pb] = orc.kv_quantize_row(rng.standard_normal(n_prior * kvd).astype(np.float32))
            self.vc[:n_prior * pb] = orc.kv_quantize_row(rng.standard_normal(n_prior * kvd).astype(np.float32))
        self.args = LayerArgs(E, n_head, n_kv, hd, F, 1e-5, 500000.0,
                              *[shapes[nm][0] for nm in ("q", "k", "v", "o", "gate", "up", "down")])
        self.keep = {nm: np.ascontiguousarray(w) for nm, (qt, w) in gg.items()}
        self.keep["attn_norm"], self.keep["ffn_norm"] = self.attn_norm, self.ffn_norm
        for nm in ("q", "k", "v", "o", "gate", "up", "down"):
            setattr(self.args, "w" + nm, self.keep[nm].ctypes.data)
        self.args.attn_norm = self.attn_norm.ctypes.data
        self.args.ffn_norm = self.ffn_norm.ctypes.data
        if attn_gate:
            self.args.wag, self.args.fmt_ag = self.keep["ag"].ctypes.data, synth.Q8_0
        self.gelu = gelu
        self.args.act_gelu = int(gelu)
        self.post = {}
        if sandwich:  # Gemma-style post-norms of the attention and FFN outputs
            r3 = np.random.default_rng(seed + 9)
            self.post = {"post_attn_norm": (0.5 + 0.05 * r3.standard_normal(E)).astype(np.float32),
                         "post_ffn_norm": (0.8 + 0.05 * r3.standard_normal(E)).astype(np.float32)}
            for nm, v in self.post.items():
                setattr(self.args, nm, v.ctypes.data)
                self.keep[nm] = v
        # Qwen-style extras: Q/K/V biases and per-head QK-norm weights
        self.extras = {}
        if qwen:
            r2 = np.random.default_rng(seed + 7)
            self.extras = {"bq": r2.standard_normal(qd).astype(np.float32),
                           "bk": r2.standard_normal(kvd).astype(np.float32),
                           "bv": (0.5 * r2.standard_normal(kvd)).astype(np.float32),
                           "q_norm": (1 + 0.1 * r2.standard_normal(hd)).astype(np.float32),
                           "k_norm": (0.5 + 0.1 * r2.standard_normal(hd)).astype(np.float32)}
            for nm, v in self.extras.items():
                setattr(self.args, nm, v.ctypes.data)
                self.keep[nm] = v


def make_layer(gpu, orc, E, n_head, n_kv, F, n_ctx, n_prior, seed, norm_scale=(1.0, 1.0), types=None, qwen=False,
               gelu=False, sandwich=False, attn_gate=False, hd=128):
    h = HostLayer(orc, E, n_head, n_kv, F, n_ctx, n_prior, seed, norm_scale, types, qwen, gelu, sandwich, attn_gate, hd)
    mats = {nm: ops.QuantMatrix.from_gguf(qt, h.keep[nm], r, c, device=gpu) for nm, (qt, r, c) in h.shapes.items()}
    ex = {nm: torch.from_numpy(v) for nm, v in h.extras.items()}
    layer = ops.DecoderLayer(mats, torch.from_numpy(h.attn_norm), torch.from_numpy(h.ffn_norm), n_head, n_kv, hd,
                             n_ctx, device=gpu,
                             bias=(ex["bq"], ex["bk"], ex["bv"]) if ex else None,
                             qk_norm=(ex["q_norm"], ex["k_norm"]) if ex else None, act_gelu=gelu,
                             post_norms=(torch.from_numpy(h.post["post_attn_norm"]),
                                         torch.from_numpy(h.post["post_ffn_norm"])) if h.post else None,
                             attn_gate=mats.get("ag"))
    assert layer.cache.pos_bytes == h.cache.pos_bytes
    layer.cache.k.copy_(torch.from_numpy(h.kc))
    layer.cache.v.copy_(torch.from_numpy(h.vc))
    return layer, h.args, h.keep, h.kc, h.vc


def dequant_rows(orc, b, n):
    return orc.dequantize_row(synth.Q8_0, np.ascontiguousarray(b), n)


@pytest.mark.parametrize("E,n_head,n_kv,F,pos,qwen", [
    (4096, 32, 8, 14336, 4096, False),   # config 4: Llama-3-8B layer, 4096 prior tokens
    (512, 4, 2, 1024, 0, False),         # first token
    (512, 8, 2, 1536, 70, False),        # GQA 4, two tiles
    (512, 8, 2, 1536, 70, True),         # Qwen-style: Q/K/V biases, per-head QK-norm
    (4096, 32, 8, 14336, 4096, True),
    (512, 8, 2, 1536, 70, "gelu"),       # gated GELU FFN (geglu_inplace)
    (512, 8, 2, 1536, 70, "gelu32"),     # gated GELU with a Q8_0 down projection (the float form)
    (512, 8, 2, 1536, 70, "gemma"),      # Gemma-style: gated GELU and sandwich norms
    (4096, 32, 8, 14336, 4096, "gemma"),
    (512, 8, 2, 1536, 70, "gate"),       # per-head attention output gate
    (4096, 32, 8, 14336, 4096, "gate"),
])
def test_layer_vs_oracle(gpu, orc, E, n_head, n_kv, F, pos, qwen):
    print(f"layer E={E} heads={n_head}/{n_kv} F={F} pos={pos} qwen={qwen}", flush=True)
    n_ctx = pos + 2
    gelu = qwen in ("gelu", "gelu32", "gemma")
    types = {"down": synth.Q8_0} if qwen == "gelu32" else None
    layer, args, keep, kc, vc = make_layer(gpu, orc, E, n_head, n_kv, F, n_ctx, pos, seed=E + pos, qwen=qwen is True,
                                           gelu=gelu, types=types, sandwich=qwen == "gemma", attn_gate=qwen == "gate")
    x = np.random.default_rng(pos + 1).standard_normal(E).astype(np.float32)
    want, q, k, v, ao = orc.layer_decode(args, kc, vc, pos, x)
    got = layer.decode(torch.from_numpy(x).to(gpu), pos).cpu().numpy()
    e = rel(got, want)
    print(f"  layer rel err {e:.3e}", flush=True)
    assert e <= TOL
    # the K/V rows written at pos: the same Q8_0 rows up to GEMV rounding
    pb = layer.cache.pos_bytes
    kd = layer.cache.k.cpu().numpy()
    vd = layer.cache.v.cpu().numpy()
    kvd = n_kv * 128
    for dev, host in ((kd, kc), (vd, vc)):
        assert np.array_equal(dev[:pos * pb], host[:pos * pb])  # prior rows untouched
        a = dequant_rows(orc, dev[pos * pb:(pos + 1) * pb], kvd)
        b = dequant_rows(orc, host[pos * pb:(pos + 1) * pb], kvd)
        assert rel(a, b) <= TOL


@pytest.mark.parametrize("hd,E,n_head,n_kv,F,pos,kind", [
    (64, 1024, 16, 4, 2048, 300, None),     # 64-value heads, GQA 4
    (64, 1024, 16, 4, 2048, 300, "qwen"),   # with Q/K/V biases and per-head QK-norm of 64 values
    (64, 512, 8, 8, 1024, 0, None),         # MHA, first token
    (256, 1024, 8, 2, 2048, 300, None),     # 256-value heads, GQA 4
    (256, 1024, 8, 2, 2048, 300, "gemma"),  # with gated GELU and sandwich norms
    (256, 2048, 8, 4, 4096, 1000, "qwen"),
])
def test_layer_head_dims(gpu, orc, hd, E, n_head, n_kv, F, pos, kind):
    """Decoder layers with 64- and 256-value heads (the fused RoPE / K/V write
    / attention kernel at rows of 2 and 8 Q8_0 blocks, QK-norm over the head's
    values, RoPE pairs across lanes at 64) against the oracle's layer, which
    takes the head size as a parameter."""
    print(f"layer hd={hd} E={E} heads={n_head}/{n_kv} F={F} pos={pos} kind={kind}", flush=True)
    n_ctx = pos + 2
    layer, args, keep, kc, vc = make_layer(gpu, orc, E, n_head, n_kv, F, n_ctx, pos, seed=E + pos + hd,
                                           qwen=kind == "qwen", gelu=kind == "gemma", sandwich=kind == "gemma",
                                           hd=hd)
    x = np.random.default_rng(pos + 2).standard_normal(E).astype(np.float32)
    want = orc.layer_decode(args, kc, vc, pos, x)[0]
    got = layer.decode(torch.from_numpy(x).to(gpu), pos).cpu().numpy()
    e = rel(got, want)
    print(f"  layer rel err {e:.3e}", flush=True)
    assert e <= TOL
    pb = layer.cache.pos_bytes
    for dev, host in ((layer.cache.k.cpu().numpy(), kc), (layer.cache.v.cpu().numpy(), vc)):
        assert np.array_equal(dev[:pos * pb], host[:pos * pb])
        a = dequant_rows(orc, dev[pos * pb:(pos + 1) * pb], n_kv * hd)
        b = dequant_rows(orc, host[pos * pb:(pos + 1) * pb], n_kv * hd)
        assert rel(a, b) <= TOL


def test_layer_graph_replay(gpu, orc):
    """The layer captured once with a device-side position and replayed for
    consecutive tokens (position and RoPE table updated between replays)
    matches eager calls on an identical layer."""
    E, n_head, n_kv, F, n_ctx = 512, 8, 2, 1024, 40
    la, _, _, _, _ = make_layer(gpu, orc, E, n_head, n_kv, F, n_ctx, 20, seed=9)
    lb, _, _, _, _ = make_layer(gpu, orc, E, n_head, n_kv, F, n_ctx, 20, seed=9)
    dpos = torch.tensor([20], dtype=torch.int32, device=gpu)
    x = torch.from_numpy(np.random.default_rng(3).standard_normal(E).astype(np.float32)).to(gpu)
    y = torch.empty_like(x)
    la.set_rope(20)
    la.decode(x, dpos, out=y)  # warm-up (writes position 20, rewritten below)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        la.decode(x, dpos, out=y)
    for pos in range(20, 26):
        dpos.fill_(pos)
        la.set_rope(pos)
        g.replay()
        want = lb.decode(x, pos)
        torch.cuda.synchronize()
        e = rel(y.cpu().numpy(), want.cpu().numpy())
        print(f"  replay pos={pos}: rel {e:.3e}", flush=True)
        assert e <= 1e-6
    assert torch.equal(la.cache.k[:26 * la.cache.pos_bytes], lb.cache.k[:26 * lb.cache.pos_bytes])


def test_norm_quant_bit_exact(gpu, orc):
    lib = _lib.load()
    rng = np.random.default_rng(4)
    for n in (4096, 512, 14336):
        x = (rng.standard_normal(n) * 3).astype(np.float32)
        w = (1 + 0.02 * rng.standard_normal(n)).astype(np.float32)
        act = ops.empty_act((n,), ops.ACT_Q8K_REP, gpu)
        xd, wd = torch.from_numpy(x).to(gpu), torch.from_numpy(w).to(gpu)
        _lib.check(lib.dq_norm_quant(ops._ptr(xd), None, None, ops._ptr(wd), n, ctypes.c_float(1e-5),
                                     ops._ptr(act.q), ops._ptr(act.scale), ops._ptr(act.isum), ops._stream()))
        y = orc.rms_norm(x, w, 1e-5)
        q, d, isum = orc.quantize_q8k_rep(y)
        assert np.array_equal(act.q.cpu().numpy(), q)
        assert np.array_equal(act.scale.cpu().numpy(), d)
        assert np.array_equal(act.isum.cpu().numpy(), isum)


def test_silu_quant_bit_exact(gpu, orc):
    lib = _lib.load()
    rng = np.random.default_rng(5)
    n = 14336
    g = (rng.standard_normal(n) * 4).astype(np.float32)
    u = (rng.standard_normal(n) * 4).astype(np.float32)
    act = ops.empty_act((n,), ops.ACT_Q8K_REP, gpu)
    gd, ud = torch.from_numpy(g).to(gpu), torch.from_numpy(u).to(gpu)  # kept alive until the kernel has run
    _lib.check(lib.dq_silu_quant(ops._ptr(gd), ops._ptr(ud), n, ops._ptr(act.q), ops._ptr(act.scale),
                                 ops._ptr(act.isum), ops._stream()))
    torch.cuda.synchronize()
    h = np.array([orc.L.dqo_silu(float(a)) for a in g], np.float32) * u
    q, d, isum = orc.quantize_q8k_rep(h)
    qg = act.q.cpu().numpy()
    # expf may differ from the host's by one ulp: allow rare one-step flips
    assert np.mean(qg != q) < 1e-3 and np.abs(qg.astype(int) - q).max() <= 1
    assert np.allclose(act.scale.cpu().numpy(), d, rtol=1e-6)


@pytest.mark.parametrize("hd,n_rot", [(128, 128), (128, 64), (64, 64), (64, 32), (256, 256), (256, 64)])
def test_rope_kv_write_bit_exact(gpu, orc, hd, n_rot):
    """RoPE of q and k (full or partial rotation) and the new K/V rows,
    bit-exact against the oracle, at 64-, 128- and 256-value heads."""
    print(f"rope_kv_write hd={hd} n_rot={n_rot}", flush=True)
    n_head, n_kv, pos, n_ctx = 32, 8, 4096, 4097
    rng = np.random.default_rng(6)
    q = rng.standard_normal(n_head * hd).astype(np.float32)
    k = rng.standard_normal(n_kv * hd).astype(np.float32)
    v = rng.standard_normal(n_kv * hd).astype(np.float32)
    cache = ops.KVCache(n_ctx, n_kv, hd, device=gpu)
    rope = ops.rope_cache(n_rot, pos, 500000.0)
    qd = torch.from_numpy(q).to(gpu)
    kd, vd, rd = torch.from_numpy(k).to(gpu), torch.from_numpy(v).to(gpu), rope.to(gpu)
    lib = _lib.load()
    _lib.check(lib.dq_rope_kv_write(ops._ptr(qd), ops._ptr(kd), ops._ptr(vd), ops._ptr(rd), n_head, n_kv, hd, n_rot,
                                    ops._ptr(cache.k), ops._ptr(cache.v), pos, None, n_ctx, ops._stream()))
    torch.cuda.synchronize()
    c = orc.rope_cache(n_rot, pos, 500000.0)
    qr = np.concatenate([orc.rope_neox(q[h * hd:(h + 1) * hd], n_rot, c) for h in range(n_head)])
    kr = np.concatenate([orc.rope_neox(k[h * hd:(h + 1) * hd], n_rot, c) for h in range(n_kv)])
    assert np.array_equal(qd.cpu().numpy(), qr)
    pb = cache.pos_bytes
    assert np.array_equal(cache.k.cpu().numpy()[pos * pb:], orc.kv_quantize_row(kr))
    assert np.array_equal(cache.v.cpu().numpy()[pos * pb:], orc.kv_quantize_row(v))
