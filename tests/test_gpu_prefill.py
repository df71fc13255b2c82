"""The prompt side of the Q8_0 KV cache on the GPU against the oracle:
batched K/V row writes (bit-exact kv_quantize_row, kv/kv_quant.cpp:31-56),
batched RoPE + row writes (bit-exact against rope_neox_cached + kv_quantize_row,
models/dense_forward.cpp:668-680), and prefill attention (core/attn_cpu.cpp,
norm-wise relative error <= 1e-3 against the oracle, per head <= 1e-2)."""
import numpy as np
import pytest
import torch

from desireeia_amd import ops

pytestmark = pytest.mark.gpu
TOL = 1e-3


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def host_cache(orc, n_pos, n_kv, hd, seed, scale=1.0):
    rng = np.random.default_rng(seed)
    k = (rng.standard_normal((n_pos, n_kv * hd)) * scale).astype(np.float32)
    v = rng.standard_normal((n_pos, n_kv * hd)).astype(np.float32)
    return orc.kv_quantize_row(k.reshape(-1)), orc.kv_quantize_row(v.reshape(-1))


def device_cache(gpu, kc, vc, n_ctx, n_kv, hd):
    c = ops.KVCache(n_ctx, n_kv, hd, device=gpu)
    c.k[:kc.size] = torch.from_numpy(kc).to(gpu)
    c.v[:vc.size] = torch.from_numpy(vc).to(gpu)
    return c


@pytest.mark.parametrize("n_kv,hd,pos0,n_tok,pad", [(8, 128, 0, 1, 0), (8, 128, 100, 77, 0), (2, 64, 5, 300, 16),
                                                   (1, 256, 0, 9, 0)])
def test_kv_write_batch_bit_exact(gpu, orc, n_kv, hd, pos0, n_tok, pad):
    print(f"kv_write_batch n_kv={n_kv} hd={hd} pos0={pos0} n_tok={n_tok} pad={pad}", flush=True)
    kvd = n_kv * hd
    rng = np.random.default_rng(n_tok)
    k = (rng.standard_normal((n_tok, kvd + pad)) * 3).astype(np.float32)
    v = rng.standard_normal((n_tok, kvd + pad)).astype(np.float32)
    k[0, :32] = 0.0  # an all-zero block
    v[-1, 32:64] = 0.5  # ties
    n_ctx = pos0 + n_tok + 2
    cache = ops.KVCache(n_ctx, n_kv, hd, device=gpu)
    cache.write_batch(torch.from_numpy(k).to(gpu), torch.from_numpy(v).to(gpu), pos0)
    torch.cuda.synchronize()
    pb = cache.pos_bytes
    kc, vc = cache.k.cpu().numpy(), cache.v.cpu().numpy()
    want_k = orc.kv_quantize_row(np.ascontiguousarray(k[:, :kvd]).reshape(-1))
    want_v = orc.kv_quantize_row(np.ascontiguousarray(v[:, :kvd]).reshape(-1))
    assert np.array_equal(kc[pos0 * pb:(pos0 + n_tok) * pb], want_k)
    assert np.array_equal(vc[pos0 * pb:(pos0 + n_tok) * pb], want_v)
    assert not kc[:pos0 * pb].any() and not kc[(pos0 + n_tok) * pb:].any()


@pytest.mark.parametrize("n_head,n_kv,n_rot,pos0,n_tok", [(32, 8, 128, 0, 5), (8, 2, 64, 1000, 33),
                                                          (4, 4, 0, 7, 3)])
def test_rope_kv_write_batch(gpu, orc, n_head, n_kv, n_rot, pos0, n_tok):
    print(f"rope_kv_write_batch n_head={n_head} n_kv={n_kv} n_rot={n_rot} pos0={pos0} n_tok={n_tok}", flush=True)
    hd = 128
    rng = np.random.default_rng(n_head + n_tok)
    q = rng.standard_normal((n_tok, n_head * hd)).astype(np.float32)
    k = rng.standard_normal((n_tok, n_kv * hd)).astype(np.float32)
    v = rng.standard_normal((n_tok, n_kv * hd)).astype(np.float32)
    tabs = np.stack([orc.rope_cache(n_rot, pos0 + t, 500000.0) for t in range(n_tok)]) if n_rot else None
    cache = ops.KVCache(pos0 + n_tok, n_kv, hd, device=gpu)
    dq = torch.from_numpy(q).to(gpu)
    dtab = torch.from_numpy(np.ascontiguousarray(tabs)).to(gpu) if n_rot else None
    cache.rope_write_batch(dq, torch.from_numpy(k).to(gpu), torch.from_numpy(v).to(gpu), dtab, n_rot, pos0)
    torch.cuda.synchronize()
    wq, wk = q.copy(), k.copy()
    if n_rot:
        for t in range(n_tok):
            for h in range(n_head):
                wq[t, h * hd:(h + 1) * hd] = orc.rope_neox(wq[t, h * hd:(h + 1) * hd], n_rot, tabs[t])
            for h in range(n_kv):
                wk[t, h * hd:(h + 1) * hd] = orc.rope_neox(wk[t, h * hd:(h + 1) * hd], n_rot, tabs[t])
    assert np.array_equal(dq.cpu().numpy(), wq)
    pb = cache.pos_bytes
    assert np.array_equal(cache.k.cpu().numpy()[pos0 * pb:], orc.kv_quantize_row(wk.reshape(-1)))
    assert np.array_equal(cache.v.cpu().numpy()[pos0 * pb:], orc.kv_quantize_row(v.reshape(-1)))


CASES = [
    # n_head, n_kv, hd, pos0, n_tok, n_swa, q_pad
    (32, 8, 128, 0, 1, 0, 0),       # one token, one key
    (32, 8, 128, 0, 37, 0, 0),      # causal from 0, partial query block
    (32, 8, 128, 1000, 64, 0, 0),   # after a prompt already cached
    (32, 8, 128, 500, 100, 64, 0),  # sliding window
    (8, 8, 128, 100, 130, 0, 0),    # MHA: 130 rows, two query blocks
    (64, 8, 128, 200, 40, 0, 0),    # GQA 8
    (6, 2, 128, 50, 45, 0, 0),      # GQA 3: row blocks cut through tokens
    (8, 2, 64, 300, 50, 0, 0),      # hd 64
    (8, 2, 256, 300, 50, 0, 0),     # hd 256
    (32, 8, 128, 40, 20, 0, 32),    # padded q rows: padding untouched
    (4, 1, 128, 0, 200, 7, 0),      # window shorter than a key tile
]


@pytest.mark.parametrize("n_head,n_kv,hd,pos0,n_tok,n_swa,q_pad", CASES)
def test_attention_prefill_vs_oracle(gpu, orc, n_head, n_kv, hd, pos0, n_tok, n_swa, q_pad):
    print(f"attn_prefill n_head={n_head} n_kv={n_kv} hd={hd} pos0={pos0} n_tok={n_tok} n_swa={n_swa} "
          f"q_pad={q_pad}", flush=True)
    n_pos = pos0 + n_tok
    kc, vc = host_cache(orc, n_pos, n_kv, hd, seed=n_pos + n_head + hd)
    q_dim = n_head * hd + q_pad
    q = np.random.default_rng(n_tok + 3).standard_normal((n_tok, q_dim)).astype(np.float32)
    cache = device_cache(gpu, kc, vc, n_pos + 3, n_kv, hd)
    sentinel = torch.full((n_tok, q_dim), 7.0, dtype=torch.float32, device=gpu)
    out = ops.attention_prefill(torch.from_numpy(q).to(gpu), cache, n_head, pos0, n_swa, out=sentinel).cpu().numpy()
    want = orc.attn_prefill(q, kc, vc, n_tok, n_head, n_kv, hd, pos0, n_swa, q_dim=q_dim,
                            out=np.full(n_tok * q_dim, 7.0, np.float32)).reshape(n_tok, q_dim)
    e = rel(out, want)
    print(f"  rel err {e:.3e}", flush=True)
    assert e <= TOL
    for t in (0, n_tok // 2, n_tok - 1):
        for h in range(n_head):
            assert rel(out[t, h * hd:(h + 1) * hd], want[t, h * hd:(h + 1) * hd]) <= 10 * TOL
    if q_pad:
        assert np.all(out[:, n_head * hd:] == 7.0)


def test_attention_prefill_large(gpu, orc):
    """512 tokens after 3584 cached positions (4096 keys for the last token,
    the decoder-layer config's context): sampled tokens against the oracle and
    every 32nd against the decode kernel at the same position."""
    n_head, n_kv, hd, pos0, n_tok = 32, 8, 128, 3584, 512
    print(f"attn_prefill large pos0={pos0} n_tok={n_tok}", flush=True)
    kc, vc = host_cache(orc, pos0 + n_tok, n_kv, hd, seed=11)
    q = np.random.default_rng(12).standard_normal((n_tok, n_head * hd)).astype(np.float32)
    cache = device_cache(gpu, kc, vc, pos0 + n_tok, n_kv, hd)
    dq = torch.from_numpy(q).to(gpu)
    out = ops.attention_prefill(dq, cache, n_head, pos0).cpu().numpy()
    for t in (0, 1, 255, 511):
        want = orc.attn_prefill(q[t:t + 1], kc, vc, 1, n_head, n_kv, hd, pos0 + t)
        e = rel(out[t], want)
        print(f"  token {t}: rel err {e:.3e}", flush=True)
        assert e <= TOL
    for t in range(0, n_tok, 32):
        dec = ops.attention_decode(dq[t], cache, n_head, pos0 + t).cpu().numpy()
        assert rel(out[t], dec) <= TOL


def test_attention_prefill_large_values(gpu, orc):
    """K rows of magnitude ~1000 (large scores, sharp softmax) and a query
    scaled up: the hi/lo operand split keeps the scores near fp32."""
    n_head, n_kv, hd, pos0, n_tok = 8, 2, 128, 60, 40
    kc, vc = host_cache(orc, pos0 + n_tok, n_kv, hd, seed=5, scale=300.0)
    q = (np.random.default_rng(6).standard_normal((n_tok, n_head * hd)) * 4).astype(np.float32)
    cache = device_cache(gpu, kc, vc, pos0 + n_tok, n_kv, hd)
    out = ops.attention_prefill(torch.from_numpy(q).to(gpu), cache, n_head, pos0).cpu().numpy()
    want = orc.attn_prefill(q, kc, vc, n_tok, n_head, n_kv, hd, pos0).reshape(n_tok, -1)
    e = rel(out, want)
    print(f"  rel err {e:.3e}", flush=True)
    assert e <= TOL


def test_attention_prefill_unsupported(gpu):
    from desireeia_amd import _lib
    cache = ops.KVCache(16, 2, 96, device=gpu)
    q = torch.zeros(4, 4 * 96, device=gpu)
    with pytest.raises(_lib.DqError):
        ops.attention_prefill(q, cache, 4, 0)
    cache = ops.KVCache(16, 2, 128, device=gpu)
    q = torch.zeros(4, 4 * 128, device=gpu)
    with pytest.raises(_lib.DqError):
        ops.attention_prefill(q, cache, 4, 13)  # positions past the cache


@pytest.mark.parametrize("n_head,n_kv,hd,pos0,n_tok,n_swa", [
    (32, 8, 128, 4000, 100, 0),    # a follow-up prompt after a long context: 32 workgroups, 16 key splits
    (32, 8, 128, 3000, 50, 1024),  # the same over a sliding window
    (8, 2, 64, 2000, 30, 0),       # hd 64
    (8, 2, 256, 1500, 20, 0),      # hd 256
    (4, 4, 128, 700, 3, 0),        # three tokens
])
def test_attention_prefill_key_split(gpu, orc, n_head, n_kv, hd, pos0, n_tok, n_swa):
    """Key splits (small grids): the merged result equals the unsplit kernel's
    to float rounding, and the oracle within the attention tolerance."""
    print(f"attn_prefill split n_head={n_head} n_kv={n_kv} hd={hd} pos0={pos0} n_tok={n_tok} n_swa={n_swa}",
          flush=True)
    kc, vc = host_cache(orc, pos0 + n_tok, n_kv, hd, seed=pos0 + n_tok)
    q = np.random.default_rng(n_tok).standard_normal((n_tok, n_head * hd)).astype(np.float32)
    cache = device_cache(gpu, kc, vc, pos0 + n_tok, n_kv, hd)
    dq = torch.from_numpy(q).to(gpu)
    split = ops.attention_prefill(dq, cache, n_head, pos0, n_swa).cpu().numpy()
    whole = ops.attention_prefill(dq, cache, n_head, pos0, n_swa, split=False).cpu().numpy()
    e = rel(split, whole)
    print(f"  split vs unsplit: {e:.2e}", flush=True)
    assert e <= 1e-6
    for t in (0, n_tok - 1):
        want = orc.attn_prefill(q[t:t + 1], kc, vc, 1, n_head, n_kv, hd, pos0 + t, n_swa)
        assert rel(split[t], want) <= TOL
