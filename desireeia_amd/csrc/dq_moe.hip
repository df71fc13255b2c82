// dq_moe.hip - MoE expert FFN on the device: routing, per-expert token lists,
// the expert GEMMs (gate/up, then down) on fp16 MFMA, SiLU and the weighted
// scatter back to the tokens.
//
// Semantics (reference models/dense_forward.cpp:1524-1560 expert_ffn, the
// combine at :4160-4181, models/moe_route.cpp:10-81): per token, softmax over
// the router logits (float max, double sum), the k largest probabilities
// (ties: lower expert index), renormalised by their float sum; per selected
// expert e, up = W_up[e] x and gate = W_gate[e] x with matmul_q4_k semantics
// (x quantized per 256: quantize_act_q8k_rep, core/matmul.cpp:1660-1778),
// h = silu(gate) * up, down = W_down[e] h (h quantized the same way), and
// out += w * down in slot order starting from zero.
//
// Design: the reference CPU path re-streams every expert's weights once per
// token. Here the tokens routed to an expert are gathered into one list, and
// each weight byte is read from HBM once for all of them:
//  * routing: one wave per token, lane = expert;
//  * lists: expert-major, ascending (token, slot) order (deterministic), by
//    wave ballots in one workgroup (the same workgroup as the routing, for
//    up to 1024 tokens);
//  * activation rows per (token, expert) pair, one workgroup per pair: the
//    per-256 integers and scale of the reference, entered into the MFMA as
//    fp16(q * d * s) (s a power-of-two range scale of the row, undone on the
//    output), plus the 8 block sums
//    fp16(d * isum_j * s) per super-block in a plane with the pairs
//    contiguous, which carry the Q4_K min term as one extra 16-wide MFMA
//    slice per super-block against fp16(-dmin * m_j);
//  * expert GEMM: a workgroup owns 128 weight rows of one expert and streams
//    their packed bytes once per 32 of the expert's tokens, a super-block per
//    K step through a 2-stage LDS ring with the activation rows (64
//    contiguous bytes per row and sub-plane per DMA), dequantizing to fp16 in
//    registers (magic-number conversion, d*sc folded in) for 32x32x16 MFMA
//    tiles. The fp16 roundings of the two operands move results by ~3e-4
//    relative. A K split (partials summed in a fixed order by the next
//    kernel) gives the short down projection enough waves to stream HBM;
//  * SiLU(gate) * up, its range scale and quantization in one kernel per
//    pair; the weighted scatter back to the tokens in slot order.
#include <math.h>

#include <type_traits>

#include "dq_common.h"
#include "dq_f16.h"

namespace {

constexpr int MOE_MAX_EXPERT = 64;
constexpr int MOE_MAX_K = 8;
constexpr int TT = 32;         // tokens per MFMA tile
constexpr int MAX_TILES = 1;   // token tiles per pass of a workgroup (32 pairs)
constexpr int ACH = 32;        // 16-byte chunks of a token's activation per main step (256 halfs)
constexpr int WAVES = 4;       // waves per workgroup, 32 weight rows each
constexpr int NSTAGE = 2;      // LDS ring stages (one step in flight while one computes)

// ---------------------------------------------------------------- routing --
// The route of one token in a segment of W lanes of a wave (W a power of two,
// n_exp <= W <= 64; lanes base .. base + W - 1), lane base + e = expert e
// holding logit lv: softmax (the max is order-independent; the double sum
// runs sequentially over the experts as the reference's loop does), k rounds
// of arg-max over the unused experts (lower index on ties) by a butterfly
// within the segment, renormalisation. The results do not depend on W. Lane
// e = 0 of a segment with write set writes the token's ids and weights (and
// the ids to s_ids when given). Every lane of the wave must call it.
__device__ __forceinline__ void route_token(float lv, int e, int base, int W, int n_exp, int k, int norm_w,
                                            float w_scale, bool write, int32_t* __restrict__ ids,
                                            float* __restrict__ wts, int32_t* s_ids) {
    const float v = e < n_exp ? lv : 0.0f;
    float m = __shfl(v, base, DQ_WAVE);
    for (int i = 1; i < n_exp; ++i) {
        const float o = __shfl(v, base + i, DQ_WAVE);
        m = (m < o) ? o : m;
    }
    const float ex = e < n_exp ? expf(v - m) : 0.0f;
    double sum = 0.0;
    for (int i = 0; i < n_exp; ++i) sum += (double)__shfl(ex, base + i, DQ_WAVE);
    float p = (float)((double)ex / sum);
    if (isnan(p)) p = 0.0f;
    float key = e < n_exp ? p : -2.0f;
    float w[MOE_MAX_K];
    int id[MOE_MAX_K];
    float wsum = 0.0f;
    for (int s = 0; s < k; ++s) {
        float bv = key;
        int bi = e;
        for (int off = W >> 1; off >= 1; off >>= 1) {
            const float ov = __shfl_xor(bv, off, DQ_WAVE);
            const int oi = __shfl_xor(bi, off, DQ_WAVE);
            if (ov > bv || (ov == bv && oi < bi)) {
                bv = ov;
                bi = oi;
            }
        }
        id[s] = bi;
        w[s] = __shfl(p, base + bi, DQ_WAVE);
        wsum += w[s];
        if (e == bi) key = -1.0f;
    }
    if (e == 0 && write) {
        for (int s = 0; s < k; ++s) {
            float ws = w[s];
            if (norm_w && wsum > 1e-9f) ws /= wsum;
            if (w_scale != 0.0f && w_scale != 1.0f) ws *= w_scale;
            ids[s] = id[s];
            wts[s] = ws;
            if (s_ids) s_ids[s] = id[s];
        }
    }
}

// One wave per token (the logit load unconditional, clamped).
__global__ __launch_bounds__(256) void moe_route_kernel(const float* __restrict__ logits, int n_tok, int n_exp,
                                                        int k, int norm_w, float w_scale, int32_t* __restrict__ ids,
                                                        float* __restrict__ wts) {
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= n_tok) return;  // uniform per wave
    const float lv = logits[(size_t)t * n_exp + (lane < n_exp ? lane : n_exp - 1)];
    route_token(lv, lane, 0, 64, n_exp, k, norm_w, w_scale, true, ids + (size_t)t * k, wts + (size_t)t * k, nullptr);
}

// Per-expert lists of the (token, slot) entries i = t*k + s, expert-major and
// in ascending i; slot_pos[i] = the entry's position in that order. One
// workgroup of NW waves takes the entries 64 NW at a time (wave w: entries
// 64w..64w+63 of the round); per expert a ballot gives each wave's count and
// each lane's rank among the earlier lanes of its wave. Pass 1 counts, pass 2
// places.
template <int NW>
__device__ __forceinline__ void build_lists(const int32_t* ids, int n_ent, int n_exp, int32_t* __restrict__ offsets,
                                            int32_t* __restrict__ pairs, int32_t* __restrict__ slot_pos,
                                            int (&wcnt)[NW][MOE_MAX_EXPERT], int (&base)[MOE_MAX_EXPERT + 1]) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint64_t lt = lane ? (~0ull >> (64 - lane)) : 0ull;  // lanes below this one
    // pass 1: per-expert totals, lane e of each wave accumulating expert e
    int mine = 0;
    for (int c0 = 0; c0 < n_ent; c0 += 64 * NW) {
        const int i = c0 + tid;
        const int id = i < n_ent ? ids[i] : -1;
        for (int e = 0; e < n_exp; ++e) {
            const int c = __popcll(__ballot(id == e));
            if (lane == e) mine += c;
        }
    }
    if (lane < n_exp) wcnt[wave][lane] = mine;
    __syncthreads();
    if (tid < n_exp) {
        int c = 0;
        for (int w = 0; w < NW; ++w) c += wcnt[w][tid];
        base[tid] = c;
    }
    __syncthreads();
    if (tid == 0) {
        int o = 0;
        for (int e = 0; e < n_exp; ++e) {
            const int c = base[e];
            base[e] = o;
            o += c;
        }
        base[n_exp] = o;
    }
    __syncthreads();
    if (tid <= n_exp) offsets[tid] = base[tid];
    // pass 2: positions
    for (int c0 = 0; c0 < n_ent; c0 += 64 * NW) {
        const int i = c0 + tid;
        const int id = i < n_ent ? ids[i] : -1;
        int rank = 0;
        for (int e = 0; e < n_exp; ++e) {
            const uint64_t m = __ballot(id == e);
            if (id == e) rank = __popcll(m & lt);
            if (lane == e) wcnt[wave][e] = __popcll(m);
        }
        __syncthreads();
        if (id >= 0) {
            int pos = base[id] + rank;
            for (int w = 0; w < wave; ++w) pos += wcnt[w][id];
            pairs[pos] = i;
            slot_pos[i] = pos;
        }
        __syncthreads();
        if (tid < n_exp) {
            int c = 0;
            for (int w = 0; w < NW; ++w) c += wcnt[w][tid];
            base[tid] += c;
        }
        __syncthreads();
    }
}

__global__ __launch_bounds__(256) void moe_lists_kernel(const int32_t* __restrict__ ids, int n_ent, int n_exp,
                                                        int32_t* __restrict__ offsets, int32_t* __restrict__ pairs,
                                                        int32_t* __restrict__ slot_pos) {
    __shared__ int wcnt[4][MOE_MAX_EXPERT];
    __shared__ int base[MOE_MAX_EXPERT + 1];
    build_lists<4>(ids, n_ent, n_exp, offsets, pairs, slot_pos, wcnt, base);
}

// Routing and lists in one workgroup, for up to RL_MAX_TOK tokens (one launch
// instead of two): a wave routes 64 / W tokens at once, one per segment of W
// lanes (W = n_exp rounded up to a power of two), the logit loads of
// RL_BATCH rounds in flight together, keeping the ids in LDS; then the lists
// as moe_lists_kernel builds them.
constexpr int RL_WAVES = 16, RL_MAX_TOK = 1024, RL_BATCH = 4;
__global__ __launch_bounds__(64 * RL_WAVES) void moe_route_lists_kernel(
    const float* __restrict__ logits, int n_tok, int n_exp, int k, int norm_w, float w_scale,
    int32_t* __restrict__ ids, float* __restrict__ wts, int32_t* __restrict__ offsets, int32_t* __restrict__ pairs,
    int32_t* __restrict__ slot_pos) {
    __shared__ int32_t s_ids[RL_MAX_TOK * MOE_MAX_K];
    __shared__ int wcnt[RL_WAVES][MOE_MAX_EXPERT];
    __shared__ int base[MOE_MAX_EXPERT + 1];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int W = 1;
    while (W < n_exp) W <<= 1;
    const int G = 64 / W, seg = lane / W, e = lane & (W - 1);
    const int le = e < n_exp ? e : n_exp - 1;
    const int per = RL_WAVES * G;  // tokens per round of the workgroup
    for (int r0 = 0; r0 < n_tok; r0 += per * RL_BATCH) {  // uniform
        float lv[RL_BATCH];
#pragma unroll
        for (int j = 0; j < RL_BATCH; ++j)
            lv[j] = logits[(size_t)min(r0 + j * per + wave * G + seg, n_tok - 1) * n_exp + le];
#pragma unroll
        for (int j = 0; j < RL_BATCH; ++j) {
            const int t0 = r0 + j * per + wave * G;  // the wave's first token this round
            if (t0 < n_tok) {                        // wave-uniform
                const int t = t0 + seg;
                const bool live = t < n_tok;
                const int tc = live ? t : 0;
                route_token(lv[j], e, seg * W, W, n_exp, k, norm_w, w_scale, live, ids + (size_t)tc * k,
                            wts + (size_t)tc * k, s_ids + tc * k);
            }
        }
    }
    __syncthreads();
    build_lists<RL_WAVES>(s_ids, n_tok * k, n_exp, offsets, pairs, slot_pos, wcnt, base);
}

// ------------------------------------------------------- activation rows --
// One 256-block b of activation row p (values v, 4 per lane): the per-256
// quantization d = amax/127, id = 127/amax, q = rint(v*id) (core/matmul.cpp
// :1681-1700), written as fp16(q*d*s) in columns 256b + 4 lane .. +3 of the
// row (stored in the order 0, 2, 1, 3), and the block sums fp16(d*isum_j*s), j = 0..7, at minp[b][p][j] (a
// plane with the pairs contiguous per super-block); s the row's range scale.
__device__ __forceinline__ void quant_256_block(const float (&v)[4], float sc, int lane, int b, int p, int n_rows,
                                                _Float16* row, _Float16* minp) {
    float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    amax = dq_wave_max(amax);
    const float d = amax > 0.0f ? amax / 127.0f : 0.0f;
    const float id = d > 0.0f ? 127.0f / amax : 0.0f;
    int isum = 0;
    uint32_t hb[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        int q = (int)rintf(v[i] * id);
        q = q > 127 ? 127 : (q < -127 ? -127 : q);
        isum += q;
        hb[i] = __builtin_bit_cast(uint16_t, (_Float16)(((float)q * d) * sc));
    }
    // columns in the order 0, 2, 1, 3 of each group of 4 (the expert GEMM's
    // order of a word's 4 weight bytes)
    *reinterpret_cast<dq_u32x2*>(row + 256 * b + 4 * lane) = dq_u32x2{hb[0] | (hb[2] << 16), hb[1] | (hb[3] << 16)};
    // 8 lanes hold one 32-block
#pragma unroll
    for (int off = 1; off < 8; off <<= 1) isum += __shfl_xor(isum, off, DQ_WAVE);
    if ((lane & 7) == 0) minp[((size_t)b * n_rows + p) * 8 + (lane >> 3)] = (_Float16)((d * (float)isum) * sc);
}

// The range scale of a workgroup's row segment from each wave's max |v|:
// row_scale_of of the 4 waves' maximum.
__device__ __forceinline__ float wg_range_scale(float mx, float (&wmax)[4], int lane, int wave) {
    mx = dq_wave_max(mx);
    if (lane == 0) wmax[wave] = mx;
    __syncthreads();
    return row_scale_of(fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3])));
}

__device__ __forceinline__ float amax4(const float (&h)[4]) {
    return fmaxf(fmaxf(fabsf(h[0]), fabsf(h[1])), fmaxf(fabsf(h[2]), fabsf(h[3])));
}

// Row p of A from token pairs[p] / k of x, one workgroup of 4 waves per pair:
// the row's range scale s = row_scale_of(max |x|) and the per-256
// quantization (quant_256_block); inv[p] = 1/s. Wave w takes the 256-blocks
// w, w + 4, ... REG (rows of up to 4 * ACT_RB blocks): all of a wave's loads
// are issued at once (unconditional, clamped to the row) and the values stay
// in registers from the maximum to the quantization; otherwise two passes
// (the second's loads hit L2).
constexpr int ACT_RB = 4;  // 256-blocks per wave held in registers
template <bool REG>
__global__ __launch_bounds__(256) void moe_act_kernel(const float* __restrict__ x, const int32_t* __restrict__ pairs,
                                                      int k, int n_rows, int K, _Float16* __restrict__ A,
                                                      _Float16* __restrict__ minp, float* __restrict__ inv) {
    __shared__ float wmax[4];
    const int p = blockIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nblk = K / 256;
    const float* xr = x + (size_t)(pairs[p] / k) * K;
    _Float16* row = A + (size_t)p * K;
    auto load = [&](int b, float (&v)[4]) {
        const float4 f = *reinterpret_cast<const float4*>(xr + 256 * b + 4 * lane);
        v[0] = f.x, v[1] = f.y, v[2] = f.z, v[3] = f.w;
    };
    float sc;
    if constexpr (REG) {
        float v[ACT_RB][4];
#pragma unroll
        for (int i = 0; i < ACT_RB; ++i) {
            const int b = wave + 4 * i;
            load(b < nblk ? b : 0, v[i]);  // blocks past the row: block 0 again, left out
        }
        float mx = 0.0f;
#pragma unroll
        for (int i = 0; i < ACT_RB; ++i)
            if (wave + 4 * i < nblk) mx = fmaxf(mx, amax4(v[i]));
        sc = wg_range_scale(mx, wmax, lane, wave);
#pragma unroll
        for (int i = 0; i < ACT_RB; ++i) {
            const int b = wave + 4 * i;
            if (b < nblk) quant_256_block(v[i], sc, lane, b, p, n_rows, row, minp);  // wave-uniform
        }
    } else {
        float mx = 0.0f;
        for (int b = wave; b < nblk; b += 4) {
            float v[4];
            load(b, v);
            mx = fmaxf(mx, amax4(v));
        }
        sc = wg_range_scale(mx, wmax, lane, wave);
        for (int b = wave; b < nblk; b += 4) {
            float v[4];
            load(b, v);
            quant_256_block(v, sc, lane, b, p, n_rows, row, minp);
        }
    }
    if (threadIdx.x == 0) inv[p] = 1.0f / sc;  // the output factor
}

// The down projection's activation of pair p over the K range of the down
// GEMM's split q (its super-blocks [q * sps, min((q + 1) * sps, F / 256))),
// one workgroup of 4 waves per (pair, split): h = silu(g) * u
// (models/dense_forward.cpp:53-55) with g, u the sums over the K splits of
// the gate and up outputs (split order 0, 1, ...), the range scale s of that
// range (row_scale_of its max |h|) and the per-256 quantization as
// moe_act_kernel writes it; inv[q * n_rows + p] = 1/s. A range scale per
// split is exact: the GEMM undoes each split's s on that split's partial
// (powers of two, fp16 and fp32 alike), and the per-256 integers and scales
// do not depend on s. Wave w takes the 256-blocks w, w + 4, ... of the range.
// REG (ranges of up to 4 * RB blocks): the wave's gate and up loads are all
// issued at once (unconditional, clamped to the range), h stays in registers
// from the maximum to the quantization, one memory round trip in all;
// otherwise a first pass finds the maximum and a second recomputes h (its
// loads hit L2) and quantizes it.
constexpr int SILU_RB = 4;  // 256-blocks per wave held in registers
template <bool REG>
__global__ __launch_bounds__(256) void moe_silu_act_kernel(const float* __restrict__ gate, const float* __restrict__ up,
                                                           int nsplit, size_t split_stride, int F, int n_rows,
                                                           int n_dsplit, int sps, _Float16* __restrict__ A,
                                                           _Float16* __restrict__ minp, float* __restrict__ inv) {
    __shared__ float wmax[4];
    const int p = blockIdx.x / n_dsplit, q = blockIdx.x % n_dsplit;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int b0 = q * sps, b1 = min(b0 + sps, F / 256);
    auto load = [&](int b, float4& g, float4& u) {
        const size_t o = (size_t)p * F + 256 * (size_t)b + 4 * lane;
        g = *reinterpret_cast<const float4*>(gate + o);
        u = *reinterpret_cast<const float4*>(up + o);
        for (int s = 1; s < nsplit; ++s) {
            const float4 g2 = *reinterpret_cast<const float4*>(gate + s * split_stride + o);
            const float4 u2 = *reinterpret_cast<const float4*>(up + s * split_stride + o);
            g.x += g2.x, g.y += g2.y, g.z += g2.z, g.w += g2.w;
            u.x += u2.x, u.y += u2.y, u.z += u2.z, u.w += u2.w;
        }
    };
    auto h_of = [](const float4& g, const float4& u, float (&h)[4]) {
        const float gv[4] = {g.x, g.y, g.z, g.w}, uv[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) h[i] = gv[i] / (1.0f + expf(-gv[i])) * uv[i];
    };
    _Float16* row = A + (size_t)p * F;
    float sc;
    if constexpr (REG) {
        // blocks past the range (or all of an empty one) load a block of the
        // row instead and are left out
        const int bx = min(b0, F / 256 - 1);
        float4 g[SILU_RB], u[SILU_RB];
#pragma unroll
        for (int i = 0; i < SILU_RB; ++i) {
            const int b = b0 + wave + 4 * i;
            load(b < b1 ? b : bx, g[i], u[i]);
        }
        float h[SILU_RB][4];
        float mx = 0.0f;
#pragma unroll
        for (int i = 0; i < SILU_RB; ++i) {
            h_of(g[i], u[i], h[i]);
            if (b0 + wave + 4 * i < b1) mx = fmaxf(mx, amax4(h[i]));
        }
        sc = wg_range_scale(mx, wmax, lane, wave);
#pragma unroll
        for (int i = 0; i < SILU_RB; ++i) {
            const int b = b0 + wave + 4 * i;
            if (b < b1) quant_256_block(h[i], sc, lane, b, p, n_rows, row, minp);  // wave-uniform
        }
    } else {
        float mx = 0.0f;
        for (int b = b0 + wave; b < b1; b += 4) {
            float4 g, u;
            float h[4];
            load(b, g, u);
            h_of(g, u, h);
            mx = fmaxf(mx, amax4(h));
        }
        sc = wg_range_scale(mx, wmax, lane, wave);
        for (int b = b0 + wave; b < b1; b += 4) {
            float4 g, u;
            float h[4];
            load(b, g, u);
            h_of(g, u, h);
            quant_256_block(h, sc, lane, b, p, n_rows, row, minp);
        }
    }
    if (threadIdx.x == 0) inv[(size_t)q * n_rows + p] = 1.0f / sc;
}

// ------------------------------------------------------------ expert GEMM --
struct MoeGemm {
    const uint8_t* w[2];  // stacked matrices ([n_exp * rows][K]): packed rows, or expert tiles (TILED)
    DqLayout L[2];
    float* y[2];          // outputs [nsplit][n_pairs][rows]
    const _Float16* A;    // activation rows [n_pairs][K]
    const _Float16* minp; // their block sums [K/256][n_pairs][8]
    const float* inv;     // 1/s of each pair's activation: [nsplit][n_pairs] (a range scale per split's K
                          // range, inv_stride = n_pairs) or [n_pairs] (one per row, inv_stride = 0)
    size_t inv_stride;
    const int32_t* offsets;
    int rows, K, n_pairs, nsplit, steps_per_split, main_steps;
    int n_exp, n_tiles;
};

// Weight bytes of one main step, a Q4_K super-block (K = 256, 4 items) of this
// lane's row: the 4 16-byte items of quant sub-plane h and the super-block
// header.
struct WRaw {
    dq_u32x4 q[4];
    dq_u32x4 hd;
};

// The 8 sub-block scales fp16(d * sc_j) of a main step's super-block header
// as pairs (sub-blocks 2t, 2t + 1 in pair t); zeros when !ok.
__device__ __forceinline__ void step_scales(const dq_u32x4& hd, bool ok, h2 (&a)[4]) {
    uint32_t lo, hi;
    q4k_sc_bytes(hd, lo, hi);
    const _Float16 d = ok ? __builtin_bit_cast(_Float16, (uint16_t)(hd.x & 0xFFFFu)) : (_Float16)0.0f;
    bytes8_times(lo, hi, d, a);
}

// B fragments of item t (= group g of the super-block) of a main step. Lane
// half h holds quant sub-plane h of the item w: bytes 0-15 of its 32 qs bytes
// (h = 0) or 16-31 (h = 1), i.e. positions 16h..16h+15 of sub-block 2t (low
// nibbles) and 2t+1 (high nibbles). Slice kk: kk/2 picks the sub-block,
// kk%2 the 8 positions 16h + 8(kk%2) + 0..7, taken from each word in the
// byte order 0, 2, 1, 3 (two nibbles per instruction); values q * (d*sc) in
// fp16, sc = (a.x, a.y) for the two sub-blocks. The activation fragment of
// the same slice holds the same positions in the same order (a_offset, and
// quant_256_block's column order).
// Per pair one shift, one v_and_or and one fma (nib_pair_fma, c = -16 a):
// needs |d * sc| <= 4094 (weights up to 61,410 in magnitude; the fp16 operand
// caps them at 65,504 in any form).
__device__ __forceinline__ void b_item(const dq_u32x4& w, h2 a, NibConst k, h8 (&bf)[4]) {
    const h2 m16 = {(_Float16)-16.0f, (_Float16)-16.0f};
    const h2 c = a * m16;  // exact: a power of two
    const h2 a0 = {a.x, a.x}, a1 = {a.y, a.y}, c0 = {c.x, c.x}, c1 = {c.y, c.y};
    const uint32_t x[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
        const uint32_t u = x[2 * (kk & 1)], v = x[2 * (kk & 1) + 1];
        uint32_t o[4];
        if (kk < 2) {  // low nibbles: bytes 0, 2 of a word at bits 6-9, 22-25 after << 6, bytes 1, 3 after >> 2
            o[0] = nib_pair_fma(u << 6, k, a0, c0);
            o[1] = nib_pair_fma(u >> 2, k, a0, c0);
            o[2] = nib_pair_fma(v << 6, k, a0, c0);
            o[3] = nib_pair_fma(v >> 2, k, a0, c0);
        } else {       // high nibbles: bytes 0, 2 after << 2, bytes 1, 3 after >> 6
            o[0] = nib_pair_fma(u << 2, k, a1, c1);
            o[1] = nib_pair_fma(u >> 6, k, a1, c1);
            o[2] = nib_pair_fma(v << 2, k, a1, c1);
            o[3] = nib_pair_fma(v >> 6, k, a1, c1);
        }
        bf[kk] = __builtin_bit_cast(h8, dq_u32x4{o[0], o[1], o[2], o[3]});
    }
}

// Column (in halfs) of the activation fragment of lane half h for item t,
// slice kk of main step st: sub-block 2t + kk/2, positions 16h + 8(kk%2)..+7.
__device__ __forceinline__ int a_offset(int st, int t, int kk, int h) {
    return 256 * st + 64 * t + 32 * (kk >> 1) + 16 * h + 8 * (kk & 1);
}


// s_waitcnt vmcnt(N), other counters untouched (gfx9 encoding: vmcnt in bits
// 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int N>
__device__ __forceinline__ void wait_vm() {
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// DMA of the activation rows of main step st for the pass starting at pair c
// into LDS stage `dst`: token m (0 .. 32*ntile-1) has 32 chunks of 16 bytes,
// chunk k stored at slot m*32 + (k ^ (m & 31)) (an XOR swizzle: the 32 tokens
// a fragment read spans fall into different bank groups). Slot s is written
// by lane s % 64 of the instruction covering it (global_load_lds writes lane
// i at base + 16 i), so each lane fetches the chunk that belongs there.
constexpr int A_LOADS = MAX_TILES * TT * ACH / (64 * WAVES);  // DMAs per thread per step
static_assert(A_LOADS >= 1, "activation DMA slots per thread");
constexpr int A_MAIN_BYTES = MAX_TILES * TT * ACH * 16;
constexpr int A_STAGE_BYTES = A_MAIN_BYTES + 64 * 16;  // + the min chunks (64 slots, 32 tokens twice)
// Per-thread sources of a pass's activation DMAs at main step 0 (a main step
// adds 256 halfs to each, and n_pairs * 8 halfs to the block-sum source),
// computed once per pass.
struct ASrc {
    const _Float16* a[A_LOADS];
    const _Float16* m;
};
__device__ __forceinline__ ASrc a_sources(const _Float16* A, const _Float16* minp, int K, int c, int p_end, int tid) {
    ASrc s;
    // the block sums of pair lane % 32 (contiguous over the pairs; wave 0
    // loads them, issue_a)
    s.m = minp + (size_t)min(c + (tid & 31), p_end - 1) * 8;
#pragma unroll
    for (int j = 0; j < A_LOADS; ++j) {
        const int slot = j * 64 * WAVES + tid;
        const int m = slot / ACH, kp = slot % ACH, k = kp ^ (m & 31);
        const int p = min(c + m, p_end - 1);
        s.a[j] = A + (size_t)p * K + 8 * k;
    }
    return s;
}
// Only the instructions that carry one of the pass's n_tok tokens are issued
// (instruction j of wave w holds tokens 8j + 2w and 8j + 2w + 1): an expert
// with 16 tokens reads half the tile. The slots of the tokens past n_tok keep
// stale bytes; they feed only MFMA output columns that are never stored.
// (The activation rows, re-read from L2 by every row tile of the expert, cost
// as much DMA as the weights at 32 rows: with them removed the weights stream
// at the device's plain read rate.)
// The block sums (one 1 KB instruction) are loaded by wave 0 alone: every
// wave waits for its own DMAs before the step's barrier.
__device__ __forceinline__ void issue_a(const ASrc& s, int n_pairs, int st, uint8_t* dst, int tid, int n_tok) {
    const int w2 = 2 * __builtin_amdgcn_readfirstlane(tid >> 6);
    if (w2 == 0)
        __builtin_amdgcn_global_load_lds(s.m + (size_t)st * n_pairs * 8, DQ_LDS_PTR(dst + A_MAIN_BYTES), 16, 0, 0);
#pragma unroll
    for (int j = 0; j < A_LOADS; ++j) {
        if (8 * j + w2 >= n_tok) break;  // wave-uniform
        uint8_t* base = dst + (size_t)(j * 64 * WAVES + (tid & ~63)) * 16;  // wave-uniform
        __builtin_amdgcn_global_load_lds(s.a[j] + 256 * (size_t)st, DQ_LDS_PTR(base), 16, 0, 0);
    }
}

// Weight tile of a main step in LDS: for the workgroup's 256 rows, the 64
// bytes of sub-plane 0 and of sub-plane 1 (4 items of 16 bytes each) and the
// 16-byte super-block header. The DMA reads each row-plane's 64 bytes with 4
// consecutive lanes (whole 64-byte pieces of one line per row: the pattern
// HBM streams at full rate; one lane per row, 16 bytes each, streams at less
// than half of it). Item t of row r sits in chunk slot t ^ ((r >> 2) & 3), so
// the fragment reads of 32 rows spread over the banks.
constexpr int WROWS = 32 * WAVES;                  // rows per workgroup
constexpr int WT_PLANE = WROWS * 64;               // bytes of one sub-plane tile
constexpr int WT_BYTES = 2 * WT_PLANE + WROWS * 16;
__device__ __forceinline__ void issue_w(const uint8_t* base, const DqLayout& L, size_t row0, int nrows, int st,
                                        uint8_t* dst, int tid) {
    const int wbase = tid & ~63;
#pragma unroll
    for (int pl = 0; pl < 2; ++pl) {
#pragma unroll
        for (int j = 0; j < WROWS * 4 / (64 * WAVES); ++j) {
            const int slot = j * 64 * WAVES + tid;
            const int r = slot >> 2, ts = slot & 3, t = ts ^ ((r >> 2) & 3);
            const size_t row = row0 + (size_t)min(r, nrows - 1);
            const uint8_t* src = base + L.q_off + (size_t)pl * L.p_stride + row * L.q_row + 64 * (size_t)st + 16 * t;
            uint8_t* d = dst + pl * WT_PLANE + (size_t)(j * 64 * WAVES + wbase) * 16;
            __builtin_amdgcn_global_load_lds(src, DQ_LDS_PTR(d), 16, 0, 0);
        }
    }
    // headers: WROWS slots, so waves w and w + WAVES/2 load the same block
    const int slot = tid % WROWS;
    const size_t row = row0 + (size_t)min(slot, nrows - 1);
    __builtin_amdgcn_global_load_lds(base + L.s_off + row * L.s_row + 16 * (size_t)st,
                                     DQ_LDS_PTR(dst + 2 * WT_PLANE + (size_t)((tid & ~63) % WROWS) * 16), 16, 0, 0);
}
static_assert(WROWS * 4 % (64 * WAVES) == 0 && 64 * WAVES == 2 * WROWS, "DMA slots per thread");

// Expert-tile layout (DQ_FMT_Q4_K_TILES): the weight tile of one main step
// stored as the LDS stage image, so the step's DMA reads one contiguous
// run (64 lanes x 16 consecutive bytes per instruction) instead of 4 lanes
// per 64-byte row piece. Chunk (e, x, sb) of expert e, row tile x (rows
// 128x .. +127, the last row repeated past the expert's end) and super-block
// sb sits at ((e * n_tiles + x) * nsb + sb) * WT_BYTES: the two sub-plane
// tiles [128 rows][4 slots][16 B] (slot t ^ ((r >> 2) & 3) holding item t)
// and the headers [128 rows][16 B].
constexpr int WT_SLOTS = WT_BYTES / 16;
constexpr int WT_TILE_LOADS = (WT_SLOTS + 64 * WAVES - 1) / (64 * WAVES);  // DMAs per thread per step
static_assert(WT_TILE_LOADS == 2 * WROWS * 4 / (64 * WAVES) + 1, "the same DMA count as the row layout");
__device__ __forceinline__ void issue_w_tiles(const uint8_t* chunk, uint8_t* dst, int tid) {
    const int wv = tid >> 6, lane = tid & 63;
#pragma unroll
    for (int j = 0; j < WT_TILE_LOADS; ++j) {
        // a wave past the last full span repeats the last 64 slots (same bytes)
        const int ws = min(j * 64 * WAVES + 64 * wv, WT_SLOTS - 64);  // wave-uniform
        __builtin_amdgcn_global_load_lds(chunk + 16 * (size_t)(ws + lane), DQ_LDS_PTR(dst + 16 * (size_t)ws), 16, 0,
                                         0);
    }
}

// One thread per 16-byte slot of the tile layout, copied from the packed
// rows (dq_weights_pack of the stacked matrix).
__global__ __launch_bounds__(256) void moe_tiles_pack_kernel(const uint8_t* __restrict__ src, DqLayout L, int rows,
                                                             int n_tiles, int nsb, size_t n_slots,
                                                             uint8_t* __restrict__ dst) {
    const size_t g = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (g >= n_slots) return;
    const size_t chunk = g / WT_SLOTS;
    const int c = (int)(g % WT_SLOTS);
    const int sb = (int)(chunk % nsb);
    const size_t et = chunk / nsb;
    const int x = (int)(et % n_tiles);
    const size_t e = et / n_tiles;
    const uint8_t* p;
    if (c < 2 * WROWS * 4) {
        const int pl = c / (WROWS * 4), rs = c % (WROWS * 4), r = rs / 4, t = (rs % 4) ^ ((r >> 2) & 3);
        const size_t row = e * rows + (size_t)min(WROWS * x + r, rows - 1);
        p = src + L.q_off + (size_t)pl * L.p_stride + row * L.q_row + 16 * (size_t)(4 * sb + t);
    } else {
        const int r = c - 2 * WROWS * 4;
        const size_t row = e * rows + (size_t)min(WROWS * x + r, rows - 1);
        p = src + L.s_off + row * L.s_row + 16 * (size_t)sb;
    }
    *reinterpret_cast<dq_u32x4*>(dst + 16 * g) = *reinterpret_cast<const dq_u32x4*>(p);
}

size_t tiles_bytes(size_t n_exp, size_t rows, size_t cols) {
    return n_exp * ((rows + WROWS - 1) / WROWS) * (cols / 256) * (size_t)WT_BYTES;
}

// The 16 MFMAs of a main step's 4 items, items alternating between two
// accumulators (two independent MFMA chains).
__device__ __forceinline__ void item_mfmas(const WRaw& wr, const h2 (&sa)[4], NibConst k, const h8 (&af)[4][4],
                                           f16v& acc, f16v& acc1) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        h8 bf[4];
        b_item(wr.q[t], sa[t], k, bf);
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            if (t & 1) acc1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[t][kk], bf[kk], acc1, 0, 0, 0);
            else acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[t][kk], bf[kk], acc, 0, 0, 0);
        }
    }
}

// Grid (one dimension): workgroup id -> expert id % n_exp, then the row tile,
// then the K split, then the matrix. Workgroups are dealt to the 8 XCDs
// round-robin, so with 8 (or a multiple of 8) experts each XCD serves whole
// experts: the activation rows an expert's tiles re-read every K step stay
// in that XCD's L2. Wave w of the workgroup owns rows 128x + 32w .. +31 of
// row tile x; lane l feeds row l % 32 with K values 8(l/32)..+7 of each
// 16-wide slice. The expert's pairs are taken 32 at a time (one 32-token MFMA
// tile). Per main step (one super-block) the weight tile and the activation
// rows go through a 2-stage LDS ring, the next step's DMAs in flight while
// this one computes. The kernel is bound by its VALU work (the weight
// conversion: one shift, one v_and_or and one fma per pair of weights), so
// the step body keeps everything else off the VALU: scales decoded four at a
// time, LDS addresses as immediates.
template <bool TILED>
__global__ __launch_bounds__(64 * WAVES) __attribute__((amdgpu_waves_per_eu(2, 2))) void moe_gemm_kernel(MoeGemm G) {
    __shared__ __align__(16) uint8_t aring[NSTAGE][A_STAGE_BYTES];
    __shared__ __align__(16) uint8_t wring[NSTAGE][WT_BYTES];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(tid >> 6));
    const int e = (int)(blockIdx.x % (unsigned)G.n_exp);
    int rest = (int)(blockIdx.x / (unsigned)G.n_exp);
    const int tile = rest % G.n_tiles;
    rest /= G.n_tiles;
    const int split = rest % G.nsplit, mat = rest / G.nsplit;
    const int p_begin = G.offsets[e], p_end = G.offsets[e + 1];
    if (p_begin >= p_end) return;  // no token routed to this expert (uniform)
    const int h = lane >> 5;
    const int r_wg = tile * WROWS;                       // first row of the workgroup (in the expert)
    const int nrows = min(WROWS, G.rows - r_wg);
    const int rl = 32 * wave + (lane & 31);              // this lane's row in the tile
    const int rloc = r_wg + rl;
    const bool row_ok = rloc < G.rows;
    const size_t row0 = (size_t)e * G.rows + r_wg;
    // TILED: the expert tile's first chunk (one per main step after it)
    const size_t chunk0 = ((size_t)e * G.n_tiles + tile) * (size_t)G.main_steps;
    const uint8_t* base = G.w[mat];
    const DqLayout L = G.L[mat];
    float* __restrict__ y = G.y[mat] + (size_t)split * G.n_pairs * G.rows;
    const float* __restrict__ inv_s = G.inv + (size_t)split * G.inv_stride;  // the split's factors
    const int s0 = split * G.steps_per_split;
    const int main_end = min(G.main_steps, s0 + G.steps_per_split);
    if (s0 >= main_end) return;  // uniform

    const NibConst nk = nib_const();
    for (int c = p_begin; c < p_end; c += TT) {
        f16v acc, acc1;
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] = acc1[r] = 0.0f;
        {
            const ASrc as = a_sources(G.A, G.minp, G.K, c, p_end, tid);
            const int n_tok = min(TT, p_end - c);  // the pass's tokens
            // prologue: the first step in flight
            issue_a(as, G.n_pairs, s0, aring[0], tid, n_tok);
            if constexpr (TILED) issue_w_tiles(base + (chunk0 + s0) * WT_BYTES, wring[0], tid);
            else issue_w(base, L, row0, nrows, s0, wring[0], tid);
            // one main step from ring stage S = (st - s0) % 2, a constant in
            // each of the two copies of the body (every LDS address is then a
            // register plus an immediate)
            auto step = [&](int st, auto stage_c) {
                constexpr int S = decltype(stage_c)::value;
                wait_vm<0>();      // this step's DMAs, the only ones outstanding, have landed
                dq_lds_barrier();  // ... in every wave; stage 1 - S is free
                if (st + 1 < main_end) {
                    issue_a(as, G.n_pairs, st + 1, aring[1 - S], tid, n_tok);
                    if constexpr (TILED) issue_w_tiles(base + (chunk0 + st + 1) * WT_BYTES, wring[1 - S], tid);
                    else issue_w(base, L, row0, nrows, st + 1, wring[1 - S], tid);
                }
                const uint8_t* ab = aring[S];
                const uint8_t* wb = wring[S];
                // every LDS read of the step first (one wait for all of them),
                // then the dequantization and the MFMAs
                WRaw wr;
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    wr.q[t] = *reinterpret_cast<const dq_u32x4*>(wb + h * WT_PLANE + rl * 64 +
                                                                 16 * (t ^ ((rl >> 2) & 3)));
                wr.hd = *reinterpret_cast<const dq_u32x4*>(wb + 2 * WT_PLANE + rl * 16);
                const int m = lane & 31;
                h8 af[4][4];
#pragma unroll
                for (int t = 0; t < 4; ++t)
#pragma unroll
                    for (int kk = 0; kk < 4; ++kk) {
                        const int k = a_offset(0, t, kk, h) / 8;  // chunk of the slice
                        af[t][kk] = *reinterpret_cast<const h8*>(ab + (size_t)(m * ACH + (k ^ (m & 31))) * 16);
                    }
                const h8 zero = {};
                const h8 am = h == 0 ? *reinterpret_cast<const h8*>(ab + A_MAIN_BYTES + m * 16) : zero;
                h2 sa[4];
                step_scales(wr.hd, row_ok, sa);
                item_mfmas(wr, sa, nk, af, acc, acc1);
                {   // the super-block's min term: one 16-wide slice, lanes of half 0
                    // carry its 8 sub-blocks (the min columns K + 8st + j
                    // against fp16(-dmin * m_j)), half 1 zeros
                    const h8 bm = h == 0 ? q4k_neg_mins(wr.hd, row_ok) : zero;
                    acc1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(am, bm, acc1, 0, 0, 0);
                }
            };
            for (int st = s0; st < main_end; st += 2) {
                step(st, std::integral_constant<int, 0>{});
                if (st + 1 < main_end) step(st + 1, std::integral_constant<int, 1>{});
            }
            __syncthreads();  // the ring is reused by the next pass
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] += acc1[r];
        // D of 32x32x16: lane l, register r -> weight row l % 32, token (r/4)*8 + (l/32)*4 + r%4.
        // The pairs' factors 1/s are loaded together first (clamped pairs: a
        // load inside the store's branch would be waited for one at a time).
        float inv[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) inv[r] = inv_s[min(c + (r >> 2) * 8 + h * 4 + (r & 3), p_end - 1)];
        if (row_ok) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int p = c + (r >> 2) * 8 + h * 4 + (r & 3);
                if (p < p_end) y[(size_t)p * G.rows + rloc] = acc[r] * inv[r];
            }
        }
    }
}

// ---------------------------------------------------------------- scatter --
// out[t][c] = sum over slots s (ascending, from zero) of wts[t*k+s] * down
// of that entry (its K-split partials summed in split order).
__global__ __launch_bounds__(256) void moe_scatter_kernel(const float* __restrict__ down, int nsplit,
                                                          size_t split_stride, const int32_t* __restrict__ slot_pos,
                                                          const float* __restrict__ wts, int k, int n_tok, int E,
                                                          float* __restrict__ out) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)n_tok * E) return;
    const int t = (int)(i / E), c = (int)(i % E);
    float o = 0.0f;
    for (int s = 0; s < k; ++s) {
        const size_t p = (size_t)slot_pos[(size_t)t * k + s];
        float v = down[p * E + c];
        for (int q = 1; q < nsplit; ++q) v += down[q * split_stride + p * E + c];
        o += wts[(size_t)t * k + s] * v;
    }
    out[i] = o;
}

// ------------------------------------------------------------- workspace --
struct MoeWs {
    int32_t *ids, *offsets, *pairs, *slot_pos;
    float *wts, *inv_in, *inv_h;
    _Float16 *a_in, *a_h, *min_in, *min_h;
    float *gate, *up, *down;
    size_t total;
};


int cus() {
    static int n = 0;
    if (!n) {
        int dev = 0, v = 0;
        n = (hipGetDevice(&dev) == hipSuccess &&
             hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
                ? v
                : 256;
    }
    return n;
}

// K splits: enough waves (>= 16 per CU) to stream the weights, a split
// covering at least 4 K steps.
int pick_split(int n_exp, int rows, int n_mat, int steps) {
    const long waves = (long)n_exp * ((rows + 31) / 32) * n_mat;
    int s = 1;
    while (s < 8 && waves * s < 16L * cus() && steps / (2 * s) >= 4) s *= 2;
    return s;
}

MoeWs carve(const dq_moe_t* m, uint32_t n_tok, int split_gu, int split_d, uint8_t* base) {
    const size_t n_ent = (size_t)n_tok * m->n_expert_used;
    const size_t E = m->n_embd, F = m->n_ff;
    MoeWs w{};
    size_t off = 0;
    auto take = [&](size_t bytes) {
        uint8_t* p = base ? base + off : nullptr;
        off += dq_align256(bytes);
        return p;
    };
    w.ids = (int32_t*)take(n_ent * 4);
    w.wts = (float*)take(n_ent * 4);
    w.offsets = (int32_t*)take((m->n_expert + 1) * 4);
    w.pairs = (int32_t*)take(n_ent * 4);
    w.slot_pos = (int32_t*)take(n_ent * 4);
    w.inv_in = (float*)take(n_ent * 4);
    w.inv_h = (float*)take((size_t)split_d * n_ent * 4);
    w.a_in = (_Float16*)take(n_ent * E * 2);
    w.min_in = (_Float16*)take(n_ent * (E / 32) * 2);
    w.gate = (float*)take((size_t)split_gu * n_ent * F * 4);
    w.up = (float*)take((size_t)split_gu * n_ent * F * 4);
    w.a_h = (_Float16*)take(n_ent * F * 2);
    w.min_h = (_Float16*)take(n_ent * (F / 32) * 2);
    w.down = (float*)take((size_t)split_d * n_ent * E * 4);
    w.total = off;
    return w;
}

bool moe_ok(const dq_moe_t* m) {
    if (!m || (m->fmt != DQ_FMT_Q4_K && m->fmt != DQ_FMT_Q4_K_TILES)) return false;
    if (m->n_expert == 0 || m->n_expert > MOE_MAX_EXPERT) return false;
    if (m->n_expert_used == 0 || m->n_expert_used > MOE_MAX_K || m->n_expert_used > m->n_expert) return false;
    if (m->n_embd == 0 || m->n_embd % 256 || m->n_ff == 0 || m->n_ff % 256) return false;
    if (m->n_embd > (1u << 20) || m->n_ff > (1u << 20)) return false;
    if ((size_t)m->n_expert * m->n_ff > 0x3FFFFFFF || (size_t)m->n_expert * m->n_embd > 0x3FFFFFFF) return false;
    return true;
}

void splits(const dq_moe_t* m, int* sgu, int* sd) {
    const int steps_gu = (int)m->n_embd / 256;
    const int steps_d = (int)m->n_ff / 256;
    *sgu = pick_split((int)m->n_expert, (int)m->n_ff, 2, steps_gu);
    *sd = pick_split((int)m->n_expert, (int)m->n_embd, 1, steps_d);
}

int launch_gemm(bool tiled, const uint8_t* w0, const uint8_t* w1, int n_mat, int n_exp, int rows, int K,
                const _Float16* A, const _Float16* minp, const float* inv, bool inv_per_split,
                const int32_t* offsets, int n_pairs, int nsplit, float* y0, float* y1, hipStream_t s) {
    MoeGemm G{};
    G.w[0] = w0;
    G.w[1] = w1 ? w1 : w0;
    if (!dq_layout(DQ_FMT_Q4_K, (size_t)n_exp * rows, K, &G.L[0])) return DQ_ERR_NOT_SUPPORTED;
    G.L[1] = G.L[0];
    G.y[0] = y0;
    G.y[1] = y1 ? y1 : y0;
    G.A = A;
    G.minp = minp;
    G.inv = inv;
    G.inv_stride = inv_per_split ? (size_t)n_pairs : 0;
    G.offsets = offsets;
    G.rows = rows;
    G.K = K;
    G.n_pairs = n_pairs;
    G.nsplit = nsplit;
    G.main_steps = K / 256;  // a super-block per main step
    G.steps_per_split = (G.main_steps + nsplit - 1) / nsplit;
    // every split owns at least one step (its partial is always written)
    if ((long)(nsplit - 1) * G.steps_per_split >= G.main_steps) return DQ_ERR_NOT_SUPPORTED;
    G.n_exp = n_exp;
    G.n_tiles = (rows + WROWS - 1) / WROWS;
    const long wgs = (long)G.n_tiles * n_exp * n_mat * nsplit;
    if (wgs > 0x7FFFFFFF) return DQ_ERR_NOT_SUPPORTED;
    if (tiled)
        moe_gemm_kernel<true><<<(unsigned)wgs, 64 * WAVES, 0, s>>>(G);
    else
        moe_gemm_kernel<false><<<(unsigned)wgs, 64 * WAVES, 0, s>>>(G);
    return dq_launch_status();
}

#define DQ_TRY(x)                      \
    do {                               \
        const int rc_ = (x);           \
        if (rc_ != DQ_OK) return rc_;  \
    } while (0)

}  // namespace

extern "C" {

int dq_moe_route(const float* d_logits, uint32_t n_tok, uint32_t n_expert, uint32_t k, int norm_w, float w_scale,
                 int32_t* d_ids, float* d_wts, void* stream) {
    if (n_expert == 0 || n_expert > MOE_MAX_EXPERT || k == 0 || k > MOE_MAX_K || k > n_expert)
        return DQ_ERR_NOT_SUPPORTED;
    if (n_tok == 0) return DQ_OK;
    if (!d_logits || !d_ids || !d_wts) return DQ_ERR_INVALID_ARG;
    if (n_tok > (1u << 24)) return DQ_ERR_NOT_SUPPORTED;
    moe_route_kernel<<<(n_tok + 3) / 4, 256, 0, (hipStream_t)stream>>>(d_logits, (int)n_tok, (int)n_expert, (int)k,
                                                                       norm_w, w_scale, d_ids, d_wts);
    return dq_launch_status();
}

int dq_moe_tiles_bytes(uint32_t n_expert, size_t rows, size_t cols, size_t* bytes) {
    if (!bytes) return DQ_ERR_INVALID_ARG;
    if (n_expert == 0 || rows == 0 || cols == 0 || cols % 256 || (size_t)n_expert * rows > 0x3FFFFFFF)
        return DQ_ERR_NOT_SUPPORTED;
    *bytes = tiles_bytes(n_expert, rows, cols);
    return DQ_OK;
}

int dq_moe_tiles_pack(const void* d_packed, uint32_t n_expert, size_t rows, size_t cols, void* d_tiles,
                      void* stream) {
    size_t bytes = 0;
    DQ_TRY(dq_moe_tiles_bytes(n_expert, rows, cols, &bytes));
    if (!d_packed || !d_tiles) return DQ_ERR_INVALID_ARG;
    DqLayout L;
    if (!dq_layout(DQ_FMT_Q4_K, (size_t)n_expert * rows, cols, &L)) return DQ_ERR_NOT_SUPPORTED;
    const size_t n_slots = bytes / 16;
    moe_tiles_pack_kernel<<<(unsigned)((n_slots + 255) / 256), 256, 0, (hipStream_t)stream>>>(
        (const uint8_t*)d_packed, L, (int)rows, (int)((rows + WROWS - 1) / WROWS), (int)(cols / 256), n_slots,
        (uint8_t*)d_tiles);
    return dq_launch_status();
}

int dq_moe_workspace_bytes(const dq_moe_t* m, uint32_t n_tok, size_t* bytes) {
    if (!bytes) return DQ_ERR_INVALID_ARG;
    if (!moe_ok(m) || n_tok > (1u << 16)) return DQ_ERR_NOT_SUPPORTED;
    int sgu, sd;
    splits(m, &sgu, &sd);
    *bytes = carve(m, n_tok, sgu, sd, nullptr).total;
    return DQ_OK;
}

int dq_moe_ffn(const dq_moe_t* m, const float* d_x, const float* d_logits, uint32_t n_tok, float* d_out,
               void* d_work, size_t work_bytes, void* stream) {
    if (!moe_ok(m) || n_tok > (1u << 16)) return DQ_ERR_NOT_SUPPORTED;
    if (n_tok == 0) return DQ_OK;
    if (!d_x || !d_logits || !d_out || !d_work || !m->wgate || !m->wup || !m->wdown) return DQ_ERR_INVALID_ARG;
    int sgu, sd;
    splits(m, &sgu, &sd);
    const MoeWs w = carve(m, n_tok, sgu, sd, (uint8_t*)d_work);
    if (work_bytes < w.total) return DQ_ERR_INVALID_ARG;
    const hipStream_t s = (hipStream_t)stream;
    const int k = (int)m->n_expert_used, n_exp = (int)m->n_expert;
    const int E = (int)m->n_embd, F = (int)m->n_ff;
    const int n_ent = (int)n_tok * k;
    // routing and the per-expert lists (one launch up to RL_MAX_TOK tokens)
    if (n_tok <= (uint32_t)RL_MAX_TOK) {
        moe_route_lists_kernel<<<1, 64 * RL_WAVES, 0, s>>>(d_logits, (int)n_tok, n_exp, k, m->norm_w, m->w_scale,
                                                           w.ids, w.wts, w.offsets, w.pairs, w.slot_pos);
        DQ_TRY(dq_launch_status());
    } else {
        moe_route_kernel<<<(n_tok + 3) / 4, 256, 0, s>>>(d_logits, (int)n_tok, n_exp, k, m->norm_w, m->w_scale,
                                                         w.ids, w.wts);
        DQ_TRY(dq_launch_status());
        moe_lists_kernel<<<1, 256, 0, s>>>(w.ids, n_ent, n_exp, w.offsets, w.pairs, w.slot_pos);
        DQ_TRY(dq_launch_status());
    }
    // activation rows of the pairs, each with its range scale
    if (E / 256 <= 4 * ACT_RB)
        moe_act_kernel<true><<<(unsigned)n_ent, 256, 0, s>>>(d_x, w.pairs, k, n_ent, E, w.a_in, w.min_in, w.inv_in);
    else
        moe_act_kernel<false><<<(unsigned)n_ent, 256, 0, s>>>(d_x, w.pairs, k, n_ent, E, w.a_in, w.min_in, w.inv_in);
    DQ_TRY(dq_launch_status());
    // gate and up of every pair (one launch, two matrices)
    const bool tiled = m->fmt == DQ_FMT_Q4_K_TILES;
    // (one range scale per activation row, whatever the K split)
    DQ_TRY(launch_gemm(tiled, (const uint8_t*)m->wgate, (const uint8_t*)m->wup, 2, n_exp, F, E, w.a_in, w.min_in,
                       w.inv_in, false, w.offsets, n_ent, sgu, w.gate, w.up, s));
    // h = silu(gate) * up, quantized for the down projection
    {
        const int sps = (F / 256 + sd - 1) / sd;  // the down GEMM's super-blocks per split (launch_gemm)
        const unsigned wgs = (unsigned)((size_t)n_ent * sd);
        if (sps <= 4 * SILU_RB)
            moe_silu_act_kernel<true><<<wgs, 256, 0, s>>>(w.gate, w.up, sgu, (size_t)n_ent * F, F, n_ent, sd, sps,
                                                          w.a_h, w.min_h, w.inv_h);
        else
            moe_silu_act_kernel<false><<<wgs, 256, 0, s>>>(w.gate, w.up, sgu, (size_t)n_ent * F, F, n_ent, sd, sps,
                                                           w.a_h, w.min_h, w.inv_h);
    }
    DQ_TRY(dq_launch_status());
    // (a range scale per down split)
    DQ_TRY(launch_gemm(tiled, (const uint8_t*)m->wdown, nullptr, 1, n_exp, E, F, w.a_h, w.min_h, w.inv_h, true,
                       w.offsets, n_ent, sd, w.down, nullptr, s));
    {
        const size_t n = (size_t)n_tok * E;
        moe_scatter_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(w.down, sd, (size_t)n_ent * E, w.slot_pos,
                                                                       w.wts, k, (int)n_tok, E, d_out);
        DQ_TRY(dq_launch_status());
    }
    return DQ_OK;
}

}  // extern "C"
