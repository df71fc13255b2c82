"""MoE on the GPU against the oracle: the router (ids exact, weights within
1e-6 - expf may differ in the last bit between libm and the device), and the
expert FFN (dq_moe_ffn) within 4e-3 norm-wise of the reference composition
(expert_ffn with matmul_q4_k semantics) at config 5's shape and at ragged
shapes: experts with no token, one token, more than 128 tokens."""
import numpy as np
import pytest
import torch

from desireeia_amd import _lib, ops, synth

pytestmark = pytest.mark.gpu
Q4K = synth.Q4_K
TOL = 4e-3
TOL_TOKEN = 1e-2  # per-token structural check (test_moe_ffn)


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@pytest.mark.parametrize("n_tok,n_exp,k", [(64, 8, 2), (1, 8, 2), (37, 64, 8), (300, 4, 1)])
def test_route(gpu, orc, n_tok, n_exp, k):
    lg = synth.gen_act((n_tok, n_exp), seed=n_tok + n_exp)
    ids, wts = ops.moe_route(torch.from_numpy(lg).to(gpu), k)
    ids, wts = ids.cpu().numpy(), wts.cpu().numpy()
    for t in range(n_tok):
        ri, rw = orc.moe_route(lg[t], k, True)
        assert np.array_equal(ids[t], ri.astype(np.int32))
        np.testing.assert_allclose(wts[t], rw, rtol=1e-6, atol=0)


def test_route_not_supported(gpu):
    lg = torch.zeros(4, 65, device=gpu)
    with pytest.raises(_lib.DqError, match="NOT_SUPPORTED"):
        ops.moe_route(lg, 2)


def make_moe(gpu, n_exp, E, F, seed):
    wg = synth.gen_weights(Q4K, n_exp * F, E, seed)
    wu = synth.gen_weights(Q4K, n_exp * F, E, seed + 1)
    wd = synth.gen_weights(Q4K, n_exp * E, F, seed + 2)
    mats = [ops.QuantMatrix.from_gguf(Q4K, w, r, c, device=gpu)
            for w, r, c in ((wg, n_exp * F, E), (wu, n_exp * F, E), (wd, n_exp * E, F))]
    return (wg, wu, wd), mats


def moe_oracle_all(orc, ws, n_exp, E, F, x, lg, n_tok, k, threads=8):
    """The oracle's expert FFN for every token, token ranges on host threads
    (the C oracle releases the interpreter lock)."""
    from concurrent.futures import ThreadPoolExecutor
    step = -(-n_tok // threads)
    ranges = [(t0, min(n_tok, t0 + step)) for t0 in range(0, n_tok, step)]
    with ThreadPoolExecutor(len(ranges)) as ex:
        parts = list(ex.map(lambda r: orc.moe_ffn(Q4K, *ws, n_exp, E, F, x, lg, n_tok, k, t0=r[0], t1=r[1]), ranges))
    out = np.zeros((n_tok, E), np.float32)
    for (t0, t1), p in zip(ranges, parts):
        out[t0:t1] = p[t0:t1]
    return out


@pytest.mark.parametrize("n_tok,n_exp,k,E,F,skew", [
    (64, 8, 2, 4096, 14336, False),   # config 5
    (5, 8, 2, 512, 768, False),       # most experts get no token
    (300, 4, 2, 256, 512, True),      # one expert gets > 128 tokens (several passes)
    (1, 2, 2, 256, 256, False),       # one token, every expert
    (4, 4, 2, 256, 16640, False),     # n_ff past 16384 (65 super-blocks over 8 uneven down splits)
    (3, 4, 2, 4352, 256, False),      # rows of 17 blocks: the activation rows' two-pass form
    (3, 4, 2, 256, 33280, False),     # 17 super-blocks per down split: SiLU's two-pass form
    (40, 6, 2, 512, 1024, False),     # routing segments of 8 lanes with 2 lanes unused
    (20, 64, 8, 512, 1024, False),    # 64 experts, top-8: one token per wave
])
def test_moe_ffn(gpu, orc, n_tok, n_exp, k, E, F, skew):
    print(f"moe n_tok={n_tok} experts={n_exp} k={k} E={E} F={F}", flush=True)
    ws, mats = make_moe(gpu, n_exp, E, F, seed=E + F)
    x = synth.gen_act((n_tok, E), seed=3)
    lg = synth.gen_act((n_tok, n_exp), seed=4)
    if skew:
        lg[:, 0] += 4.0  # expert 0 in nearly every token's top-k
    moe = ops.MoeLayer(*mats, n_expert=n_exp, n_expert_used=k)
    got = moe(torch.from_numpy(x).to(gpu), torch.from_numpy(lg).to(gpu)).cpu().numpy()
    # every token against the CPU oracle (token ranges on host threads: the
    # oracle re-streams two experts' 177 MB per token at the full shape)
    want = moe_oracle_all(orc, ws, n_exp, E, F, x, lg, n_tok, k)
    e = rel(got, want)
    per_tok = [rel(got[t], want[t]) for t in range(n_tok)]
    print(f"  rel err {e:.3e}, per token median {np.median(per_tok):.2e} worst {max(per_tok):.2e}", flush=True)
    assert e <= TOL
    # each token on its own within TOL_TOKEN: a per-256 rounding tie of the
    # FFN intermediate that falls differently on the GPU and the CPU moves one
    # token by up to ~6e-3 (see test_moe_activation_range); a token sent to a
    # wrong expert, or a misplaced expert tile, is off by O(1)
    assert max(per_tok) <= TOL_TOKEN
    # a second call on the same workspace gives the same bits
    again = moe(torch.from_numpy(x).to(gpu), torch.from_numpy(lg).to(gpu)).cpu().numpy()
    assert np.array_equal(got, again)


def test_moe_route_launch_forms_agree(gpu, orc):
    """Past 1024 tokens the routing and the lists run as two launches (one
    wave per token, then one workgroup) instead of one workgroup. A token's
    output does not depend on the other tokens of the call (its expert tiles
    add the same products in the same order), so the first 1000 of 1100
    tokens must equal a 1000-token call bit for bit; the whole call is held to
    the oracle at the product tolerance."""
    n_exp, k, E, F, n = 4, 2, 512, 1024, 1100
    ws, mats = make_moe(gpu, n_exp, E, F, seed=91)
    x = synth.gen_act((n, E), seed=13)
    lg = synth.gen_act((n, n_exp), seed=14)
    moe = ops.MoeLayer(*mats, n_expert=n_exp, n_expert_used=k)
    two = moe(torch.from_numpy(x).to(gpu), torch.from_numpy(lg).to(gpu)).cpu().numpy()
    one = moe(torch.from_numpy(x[:1000]).to(gpu), torch.from_numpy(lg[:1000]).to(gpu)).cpu().numpy()
    assert np.array_equal(two[:1000], one)
    want = moe_oracle_all(orc, ws, n_exp, E, F, x, lg, n, k)
    e = rel(two, want)
    print(f"  rel err {e:.3e}", flush=True)
    assert e <= TOL


def test_moe_not_supported(gpu):
    _, mats = make_moe(gpu, 2, 256, 256, seed=1)
    moe = ops.MoeLayer(*mats, n_expert=2, n_expert_used=3)
    with pytest.raises(_lib.DqError, match="NOT_SUPPORTED"):
        moe(torch.zeros(4, 256, device=gpu), torch.zeros(4, 2, device=gpu))


@pytest.mark.parametrize("scale", [5000.0, 1e-4])
def test_moe_activation_range(gpu, orc, scale):
    """Token activations far from N(0,1) stay finite (per-row power-of-two range
    scaling of the fp16 operands). Tolerance 1e-2 per token: at x * 5000 the
    FFN intermediate spans ~1e11, and the ~5e-4 difference of the fp16 gate/up
    GEMVs flips some of its per-256 integers at rounding ties before the down
    projection (any GEMV not bit-identical to the CPU one does the same);
    config 5's N(0,1) inputs are held to 4e-3 in test_moe_ffn."""
    n_exp, E, F, n_tok, k = 4, 512, 768, 6, 2
    ws, mats = make_moe(gpu, n_exp, E, F, seed=77)
    x = synth.gen_act((n_tok, E), seed=5) * scale
    lg = synth.gen_act((n_tok, n_exp), seed=6)
    moe = ops.MoeLayer(*mats, n_expert=n_exp, n_expert_used=k)
    got = moe(torch.from_numpy(x).to(gpu), torch.from_numpy(lg).to(gpu)).cpu().numpy()
    want = orc.moe_ffn(Q4K, *ws, n_exp, E, F, x, lg, n_tok, k)
    assert np.isfinite(got).all()
    errs = [rel(got[t], want[t]) for t in range(n_tok)]
    print("  per-token rel errs", ["%.2e" % e for e in errs], flush=True)
    assert max(errs) <= 1e-2


@pytest.mark.parametrize("n_tok,n_exp,k,E,F", [(64, 8, 2, 4096, 14336), (300, 4, 2, 256, 512), (5, 8, 2, 512, 768),
                                             (9, 3, 2, 512, 256)])
def test_moe_tiles_match_rows(gpu, n_tok, n_exp, k, E, F):
    """The expert-tile layout (dq_moe_tiles_pack, contiguous weight DMA) and
    the packed rows give bit-identical outputs."""
    print(f"moe tiles n_tok={n_tok} E={E} F={F}", flush=True)
    _, mats = make_moe(gpu, n_exp, E, F, seed=E + 3 * F)
    x = torch.from_numpy(synth.gen_act((n_tok, E), seed=11)).to(gpu)
    lg = torch.from_numpy(synth.gen_act((n_tok, n_exp), seed=12)).to(gpu)
    rows = ops.MoeLayer(*mats, n_expert=n_exp, n_expert_used=k, tiled=False)(x, lg)
    tiles = ops.MoeLayer(*mats, n_expert=n_exp, n_expert_used=k, tiled=True)(x, lg)
    assert torch.equal(rows, tiles)


def test_moe_tiles_errors(gpu):
    lib = _lib.load()
    import ctypes
    n = ctypes.c_size_t(0)
    assert lib.dq_moe_tiles_bytes(8, 14336, 4096, ctypes.byref(n)) == 0
    assert n.value == 8 * 112 * 16 * (2 * 128 * 64 + 128 * 16)
    assert lib.dq_moe_tiles_bytes(8, 14336, 4000, ctypes.byref(n)) == -2   # cols % 256
    assert lib.dq_moe_tiles_bytes(0, 14336, 4096, ctypes.byref(n)) == -2
    assert lib.dq_moe_tiles_pack(None, 2, 256, 256, None, None) == -1
