"""The allocation-free decode attention (dq_attn_decode_q8_noalloc) against the
allocating entry point (dq_attn_decode_q8) it shares its kernels with:
bit-identical outputs on two calls in a row, the second smaller than the
first (fewer positions, a smaller cache, a window start), both within the
oracle's attention bound; an oversized shape is refused with nothing
written."""
import ctypes

import numpy as np
import pytest
import torch

from desireeia_amd import _lib, ops

pytestmark = pytest.mark.gpu
HD = 128


def _cache(gpu, orc, n_ctx, n_kv, seed):
    rng = np.random.default_rng(seed)
    c = ops.KVCache(n_ctx, n_kv, HD, device=gpu)
    kc = orc.kv_quantize_row(rng.standard_normal(n_ctx * n_kv * HD).astype(np.float32))
    vc = orc.kv_quantize_row(rng.standard_normal(n_ctx * n_kv * HD).astype(np.float32))
    c.k.copy_(torch.from_numpy(kc))
    c.v.copy_(torch.from_numpy(vc))
    return c, kc, vc


def _noalloc(lib, q, c, n_head, cc_start, pos, out):
    return lib.dq_attn_decode_q8_noalloc(ops._ptr(q), ops._ptr(c.k), ops._ptr(c.v), n_head, c.n_head_kv, HD,
                                         cc_start, pos, None, c.n_ctx, ops._ptr(out), ops._stream())


def test_noalloc_matches_allocating_entry_point(gpu, orc):
    lib = _lib.load()
    rng = np.random.default_rng(5)
    # first call: config 4's heads over 4097 positions; second: fewer heads,
    # a smaller cache and a window start
    for n_head, n_kv, n_ctx, pos, cc_start in ((32, 8, 4097, 4096, 0), (8, 2, 300, 170, 37)):
        print(f"noalloc attention heads={n_head}/{n_kv} n_ctx={n_ctx} pos={pos} cc_start={cc_start}", flush=True)
        c, kc, vc = _cache(gpu, orc, n_ctx, n_kv, seed=n_ctx)
        qn = (0.3 * rng.standard_normal(n_head * HD)).astype(np.float32)
        q = torch.from_numpy(qn).to(gpu)
        out = torch.full((n_head * HD,), float("nan"), device=gpu)
        _lib.check(_noalloc(lib, q, c, n_head, cc_start, pos, out), "dq_attn_decode_q8_noalloc")
        want = ops.attention_decode(q, c, n_head, pos, cc_start=cc_start)
        torch.cuda.synchronize()
        assert torch.equal(out, want)
        o = orc.attn_decode(qn, kc, vc, n_head, n_kv, HD, cc_start, pos)
        got = out.cpu().numpy()
        assert np.linalg.norm(got - o) / np.linalg.norm(o) <= 1e-3


def test_noalloc_rejects_oversized_shape(gpu):
    """The 16 MiB scratch covers the contexts whose records
    (dq_attn_workspace_bytes) fit in it, for 32 heads of 128; the first
    context past them is refused and nothing runs."""
    lib = _lib.load()

    def need(n_ctx):
        n = ctypes.c_size_t(0)
        _lib.check(lib.dq_attn_workspace_bytes(32, 8, HD, n_ctx, ctypes.byref(n)), "dq_attn_workspace_bytes")
        return n.value

    lo, hi = 1, 1 << 22  # need(lo) fits, need(hi) does not
    assert need(lo) <= 16 << 20 < need(hi)
    while hi - lo > 1:
        mid = (lo + hi) // 2
        lo, hi = (mid, hi) if need(mid) <= 16 << 20 else (lo, mid)
    big = hi
    print(f"noalloc: contexts up to {lo} positions fit the scratch", flush=True)
    assert lo >= 60000  # config 4's heads cover long contexts
    q = torch.zeros(32 * HD, device=gpu)
    kc = torch.zeros(8 * 136, dtype=torch.uint8, device=gpu)  # position 0's rows, were anything to run
    out = torch.full((32 * HD,), 7.0, device=gpu)
    rc = lib.dq_attn_decode_q8_noalloc(ops._ptr(q), ops._ptr(kc), ops._ptr(kc), 32, 8, HD, 0, 0, None, big,
                                       ops._ptr(out), ops._stream())
    assert rc == -2  # DQ_ERR_NOT_SUPPORTED
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())
