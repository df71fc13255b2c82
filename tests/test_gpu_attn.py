"""Q8_0 KV cache writes and decode attention on the GPU against the oracle
(reference kv/kv_quant.cpp and models/dense_forward.cpp:3956-4065).

KV rows: bit-exact. Attention output: norm-wise relative error <= 1e-3 against
the oracle's float path (the reference's own summation order) and against the
fp64 evaluation over the same dequantized rows."""
import numpy as np
import pytest
import torch

from desireeia_amd import _lib, ops

pytestmark = pytest.mark.gpu
TOL = 1e-3
HD = 128


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def host_cache(orc, n_pos, n_kv, seed, hd=HD):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((n_pos, n_kv, hd)).astype(np.float32)
    v = rng.standard_normal((n_pos, n_kv, hd)).astype(np.float32)
    return orc.kv_quantize_row(k.reshape(-1)), orc.kv_quantize_row(v.reshape(-1))


def device_cache(gpu, kc, vc, n_ctx, n_kv, hd=HD):
    c = ops.KVCache(n_ctx, n_kv, hd, device=gpu)
    c.k[:kc.size] = torch.from_numpy(kc).to(gpu)
    c.v[:vc.size] = torch.from_numpy(vc).to(gpu)
    return c


@pytest.mark.parametrize("n_kv,pos", [(8, 0), (8, 4096), (1, 77), (2, 1000)])
def test_kv_write_bit_exact(gpu, orc, n_kv, pos):
    print(f"kv_write n_kv={n_kv} pos={pos}", flush=True)
    n_ctx = pos + 3
    cache = ops.KVCache(n_ctx, n_kv, HD, device=gpu)
    rng = np.random.default_rng(pos + n_kv)
    k = (rng.standard_normal(n_kv * HD) * 3).astype(np.float32)
    v = rng.standard_normal(n_kv * HD).astype(np.float32)
    k[:32] = 0.0  # an all-zero block
    cache.write(torch.from_numpy(k).to(gpu), torch.from_numpy(v).to(gpu), pos)
    torch.cuda.synchronize()
    pb = cache.pos_bytes
    kc = cache.k.cpu().numpy()
    vc = cache.v.cpu().numpy()
    assert np.array_equal(kc[pos * pb:(pos + 1) * pb], orc.kv_quantize_row(k))
    assert np.array_equal(vc[pos * pb:(pos + 1) * pb], orc.kv_quantize_row(v))
    # nothing else written
    assert not kc[:pos * pb].any() and not kc[(pos + 1) * pb:].any()
    # device-side position
    dpos = torch.tensor([pos + 1], dtype=torch.int32, device=gpu)
    cache.write(torch.from_numpy(v).to(gpu), torch.from_numpy(k).to(gpu), dpos)
    torch.cuda.synchronize()
    assert np.array_equal(cache.k.cpu().numpy()[(pos + 1) * pb:(pos + 2) * pb], orc.kv_quantize_row(v))


CASES = [
    # n_head, n_kv, pos, cc_start
    (32, 8, 4096, 0),    # config 4: 4097 keys, GQA 4
    (32, 8, 0, 0),       # one key
    (32, 8, 63, 0),      # exactly one tile
    (32, 8, 64, 0),      # one tile + one
    (32, 8, 1000, 900),  # sliding window start
    (8, 8, 513, 0),      # MHA
    (16, 8, 2000, 0),    # GQA 2
    (64, 8, 3000, 0),    # GQA 8
    (32, 8, 20000, 0),   # long context: 313 tiles merged
]


@pytest.mark.parametrize("n_head,n_kv,pos,cc_start", CASES)
def test_attention_vs_oracle(gpu, orc, n_head, n_kv, pos, cc_start):
    print(f"attn n_head={n_head} n_kv={n_kv} pos={pos} cc_start={cc_start}", flush=True)
    kc, vc = host_cache(orc, pos + 1, n_kv, seed=pos + n_head)
    q = np.random.default_rng(pos + 7).standard_normal(n_head * HD).astype(np.float32)
    cache = device_cache(gpu, kc, vc, pos + 5, n_kv)
    out = ops.attention_decode(torch.from_numpy(q).to(gpu), cache, n_head, pos, cc_start).cpu().numpy()
    want = orc.attn_decode(q, kc, vc, n_head, n_kv, HD, cc_start, pos)
    e = rel(out, want)
    print(f"  rel err {e:.3e}", flush=True)
    assert e <= TOL
    if pos <= 4096:
        w64 = orc.attn_decode(q, kc, vc, n_head, n_kv, HD, cc_start, pos, f64=True)
        assert rel(out, w64) <= TOL
    # per head: no head may be wrong even if the norm hides it
    for h in range(n_head):
        assert rel(out[h * HD:(h + 1) * HD], want[h * HD:(h + 1) * HD]) <= 10 * TOL


HD_CASES = [
    # hd, n_head, n_kv, pos, cc_start
    (64, 16, 4, 1000, 0),     # GQA 4, 16 tiles
    (64, 32, 4, 4096, 0),     # GQA 8, 65 tiles
    (64, 8, 8, 70, 0),        # MHA, a partial second tile
    (64, 8, 1, 0, 0),         # one key, 8 heads on one KV head
    (256, 8, 2, 1000, 0),     # GQA 4
    (256, 16, 2, 4096, 100),  # GQA 8, window start
    (256, 4, 4, 63, 0),       # MHA, exactly one tile
    (256, 2, 1, 20000, 0),    # GQA 2, long context
]


@pytest.mark.parametrize("hd,n_head,n_kv,pos,cc_start", HD_CASES)
def test_attention_head_dims(gpu, orc, hd, n_head, n_kv, pos, cc_start):
    """Heads of 64 and 256 values (rows of 2 and 8 Q8_0 blocks): the same
    bound against the oracle and its fp64 evaluation, head by head."""
    print(f"attn hd={hd} n_head={n_head} n_kv={n_kv} pos={pos} cc_start={cc_start}", flush=True)
    kc, vc = host_cache(orc, pos + 1, n_kv, seed=pos + n_head + hd, hd=hd)
    q = np.random.default_rng(pos + hd).standard_normal(n_head * hd).astype(np.float32)
    cache = device_cache(gpu, kc, vc, pos + 5, n_kv, hd=hd)
    out = ops.attention_decode(torch.from_numpy(q).to(gpu), cache, n_head, pos, cc_start).cpu().numpy()
    want = orc.attn_decode(q, kc, vc, n_head, n_kv, hd, cc_start, pos)
    e = rel(out, want)
    print(f"  rel err {e:.3e}", flush=True)
    assert e <= TOL
    if pos <= 4096:
        assert rel(out, orc.attn_decode(q, kc, vc, n_head, n_kv, hd, cc_start, pos, f64=True)) <= TOL
    for h in range(n_head):
        assert rel(out[h * hd:(h + 1) * hd], want[h * hd:(h + 1) * hd]) <= 10 * TOL


def test_attention_device_pos_graph(gpu, orc):
    """Position in device memory, captured once in a HIP graph and replayed for
    successive positions: every replay matches the eager call and the oracle."""
    n_head, n_kv, n_ctx = 32, 8, 700
    kc, vc = host_cache(orc, n_ctx, n_kv, seed=11)
    cache = device_cache(gpu, kc, vc, n_ctx, n_kv)
    q = torch.from_numpy(np.random.default_rng(12).standard_normal(n_head * HD).astype(np.float32)).to(gpu)
    dpos = torch.zeros(1, dtype=torch.int32, device=gpu)
    work = ops.attn_workspace(n_head, n_kv, HD, n_ctx, gpu)
    out = torch.empty(n_head * HD, dtype=torch.float32, device=gpu)
    ops.attention_decode(q, cache, n_head, dpos, out=out, work=work)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ops.attention_decode(q, cache, n_head, dpos, out=out, work=work)
    qh = q.cpu().numpy()
    for pos in (5, 64, 300, 699, 128):
        dpos.fill_(pos)
        g.replay()
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        eager = ops.attention_decode(q, cache, n_head, pos).cpu().numpy()
        want = orc.attn_decode(qh, kc, vc, n_head, n_kv, HD, 0, pos)
        print(f"  replay pos={pos}: rel err {rel(got, want):.3e}", flush=True)
        assert rel(got, want) <= TOL
        assert rel(got, eager) <= 1e-6


def test_attention_unsupported(gpu):
    n = ctypes_size()
    lib = _lib.load()
    assert lib.dq_attn_workspace_bytes(32, 8, 96, 100, n) == -2   # hd 96
    assert lib.dq_attn_workspace_bytes(32, 8, 32, 100, n) == -2   # hd 32
    assert lib.dq_attn_workspace_bytes(6, 2, 64, 100, n) == -2    # 384 outputs: not whole 256-blocks
    assert lib.dq_attn_workspace_bytes(24, 8, 128, 100, n) == -2  # 3 heads per KV head
    assert lib.dq_attn_workspace_bytes(30, 8, 128, 100, n) == -2  # not a multiple


def ctypes_size():
    import ctypes
    return ctypes.byref(ctypes.c_size_t(0))


def test_attention_quantized_output(gpu, orc):
    """dq_attn_decode_q8_act: the merged output quantized per 256 values is
    bit-identical to the per-256 quantizer applied to the fp32 output, on
    repeated calls sharing one workspace."""
    import ctypes
    n_head, n_kv, pos = 32, 8, 1500
    kc, vc = host_cache(orc, pos + 1, n_kv, seed=21)
    cache = device_cache(gpu, kc, vc, pos + 1, n_kv)
    q = np.random.default_rng(22).standard_normal(n_head * HD).astype(np.float32)
    qd = torch.from_numpy(q).to(gpu)
    work = ops.attn_workspace(n_head, n_kv, HD, pos + 1, gpu)
    lib = _lib.load()
    for p in (pos, 100, pos):
        out = torch.empty(n_head * HD, dtype=torch.float32, device=gpu)
        act = ops.empty_act((n_head * HD,), ops.ACT_Q8K_REP, gpu)
        _lib.check(lib.dq_attn_decode_q8_act(ops._ptr(qd), ops._ptr(cache.k), ops._ptr(cache.v), n_head, n_kv, HD, 0,
                                             p, None, cache.n_ctx, ops._ptr(out), ops._ptr(act.q),
                                             ops._ptr(act.scale), ops._ptr(act.isum), ops._ptr(work), work.numel(),
                                             ops._stream()))
        torch.cuda.synchronize()
        o = out.cpu().numpy()
        assert rel(o, orc.attn_decode(q, kc, vc, n_head, n_kv, HD, 0, p)) <= TOL
        wq, wd, wi = orc.quantize_q8k_rep(o)
        assert np.array_equal(act.q.cpu().numpy(), wq)
        assert np.array_equal(act.scale.cpu().numpy(), wd)
        assert np.array_equal(act.isum.cpu().numpy(), wi)


@pytest.mark.parametrize("HD,n_head,n_kv,pos,rope,quant", [
    (128, 32, 8, 4096, True, True),    # config 4's step
    (128, 32, 8, 0, True, True),       # the first token: the new row is the only key
    (128, 32, 8, 64, True, False),     # the new row starts a tile
    (128, 16, 16, 300, False, True),   # MHA, no RoPE: quantization falls back to a separate pass
    (128, 64, 8, 1000, True, True),    # GQA 8
    (64, 16, 4, 500, True, True),      # 64-value heads: RoPE pairs in lanes j and j + 32
    (64, 8, 8, 0, True, False),
    (256, 8, 2, 129, True, True),      # 256-value heads: two RoPE pairs per lane
    (256, 16, 2, 64, True, True),
])
def test_attention_rope_kv_fused(gpu, orc, HD, n_head, n_kv, pos, rope, quant):
    """dq_attn_rope_kv_decode: RoPE of the raw q and k, the new K/V rows at pos
    (bit-exact: kv_quantize_row of the oracle's rotated k and of v), attention
    over [0, pos] within 1e-3, the per-256 quantization of the output
    bit-exact on the kernel's own float output; the prior rows untouched."""
    print(f"fused attn hd={HD} n_head={n_head} n_kv={n_kv} pos={pos} rope={rope} quant={quant}", flush=True)
    n_ctx = pos + 3
    kc, vc = host_cache(orc, pos, n_kv, seed=pos + 3, hd=HD)
    cache = device_cache(gpu, kc, vc, n_ctx, n_kv, hd=HD)
    rng = np.random.default_rng(pos + 4)
    q = rng.standard_normal(n_head * HD).astype(np.float32)
    k = rng.standard_normal(n_kv * HD).astype(np.float32)
    v = rng.standard_normal(n_kv * HD).astype(np.float32)
    table = orc.rope_cache(HD, pos, 500000.0)
    dq, dk, dv = (torch.from_numpy(a).to(gpu) for a in (q, k, v))
    drope = torch.from_numpy(table).to(gpu) if rope else None
    out = torch.empty(n_head * HD, dtype=torch.float32, device=gpu)
    act = ops.empty_act((n_head * HD,), ops.ACT_Q8K_REP, gpu) if quant else None
    work = ops.attn_workspace(n_head, n_kv, HD, n_ctx, gpu)
    lib = _lib.load()
    for _ in range(2):  # the same step twice on one workspace
        _lib.check(lib.dq_attn_rope_kv_decode(ops._ptr(dq), ops._ptr(dk), ops._ptr(dv), ops._ptr(drope), HD,
                                              ops._ptr(cache.k), ops._ptr(cache.v), n_head, n_kv, HD, 0, pos, None,
                                              n_ctx, ops._ptr(out), ops._ptr(act.q) if quant else None,
                                              ops._ptr(act.scale) if quant else None,
                                              ops._ptr(act.isum) if quant else None, ops._ptr(work), work.numel(),
                                              ops._stream()), "dq_attn_rope_kv_decode")
    torch.cuda.synchronize()
    qr, kr = q.copy(), k.copy()
    if rope:
        for h in range(n_head):
            qr[h * HD:(h + 1) * HD] = orc.rope_neox(qr[h * HD:(h + 1) * HD], HD, table)
        for h in range(n_kv):
            kr[h * HD:(h + 1) * HD] = orc.rope_neox(kr[h * HD:(h + 1) * HD], HD, table)
    pb = n_kv * HD // 32 * 34
    gk, gv = cache.k.cpu().numpy(), cache.v.cpu().numpy()
    assert np.array_equal(gk[pos * pb:(pos + 1) * pb], orc.kv_quantize_row(kr))
    assert np.array_equal(gv[pos * pb:(pos + 1) * pb], orc.kv_quantize_row(v))
    assert np.array_equal(gk[:pos * pb], kc) and np.array_equal(gv[:pos * pb], vc)
    o = out.cpu().numpy()
    want = orc.attn_decode(qr, gk, gv, n_head, n_kv, HD, 0, pos)
    assert rel(o, want) <= TOL
    if quant:
        wq, wd, wi = orc.quantize_q8k_rep(o)
        assert np.array_equal(act.q.cpu().numpy(), wq)
        assert np.array_equal(act.scale.cpu().numpy(), wd)
        assert np.array_equal(act.isum.cpu().numpy(), wi)


@pytest.mark.parametrize("fused,HD", [(True, 128), (False, 128), (True, 64), (True, 256)])
def test_attention_wide_value_range(gpu, orc, fused, HD):
    """Large query, key and value magnitudes (scores in the tens of thousands,
    one dominant position; the new row's V block scale ~1000x the others):
    the weight operand scale is the maximum over every row of the tile, so no
    fp16 operand overflows. Output finite and within 1e-3 of the oracle."""
    n_head, n_kv, pos = 8, 2, 70
    print(f"wide range fused={fused} hd={HD}", flush=True)
    n_ctx = pos + 2
    rng = np.random.default_rng(pos)
    kc, vc = (orc.kv_quantize_row(rng.standard_normal(pos * n_kv * HD).astype(np.float32)) for _ in range(2))
    cache = device_cache(gpu, kc, vc, n_ctx, n_kv, hd=HD)
    q = (300 * rng.standard_normal(n_head * HD)).astype(np.float32)
    k = (200 * rng.standard_normal(n_kv * HD)).astype(np.float32)
    v = (1000 * rng.standard_normal(n_kv * HD)).astype(np.float32)
    dq, dk, dv = (torch.from_numpy(a).to(gpu) for a in (q, k, v))
    out = torch.empty(n_head * HD, dtype=torch.float32, device=gpu)
    work = ops.attn_workspace(n_head, n_kv, HD, n_ctx, gpu)
    if fused:
        lib = _lib.load()
        _lib.check(lib.dq_attn_rope_kv_decode(ops._ptr(dq), ops._ptr(dk), ops._ptr(dv), None, HD, ops._ptr(cache.k),
                                              ops._ptr(cache.v), n_head, n_kv, HD, 0, pos, None, n_ctx, ops._ptr(out),
                                              None, None, None, ops._ptr(work), work.numel(), ops._stream()),
                   "dq_attn_rope_kv_decode")
    else:
        cache.write(dk, dv, pos)
        ops.attention_decode(dq, cache, n_head, pos, out=out, work=work)
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    assert np.isfinite(o).all()
    want = orc.attn_decode(q, cache.k.cpu().numpy(), cache.v.cpu().numpy(), n_head, n_kv, HD, 0, pos)
    e = rel(o, want)
    print(f"  rel err {e:.3e}", flush=True)
    assert e <= TOL


def test_attention_workspace_reuse(gpu, orc):
    """One workspace through calls of every size class (one tile, a partial
    last tile, tile boundaries, a long context, back to short): each output
    matches the oracle, so no call reads another call's records."""
    n_head, n_kv, n_ctx = 32, 8, 5000
    kc, vc = host_cache(orc, n_ctx, n_kv, seed=41)
    cache = device_cache(gpu, kc, vc, n_ctx, n_kv)
    work = ops.attn_workspace(n_head, n_kv, HD, n_ctx, gpu)
    out = torch.empty(n_head * HD, dtype=torch.float32, device=gpu)
    rng = np.random.default_rng(42)
    for pos in (4999, 0, 127, 128, 4095, 255, 1, 4999):
        q = rng.standard_normal(n_head * HD).astype(np.float32)
        ops.attention_decode(torch.from_numpy(q).to(gpu), cache, n_head, pos, out=out, work=work)
        torch.cuda.synchronize()
        e = rel(out.cpu().numpy(), orc.attn_decode(q, kc, vc, n_head, n_kv, HD, 0, pos))
        print(f"  pos={pos}: rel err {e:.3e}", flush=True)
        assert e <= TOL
