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
//  * lists: expert-major, ascending token order (deterministic);
//  * activation rows per (token, expert) pair: the per-256 integers and scale
//    of the reference, entered into the MFMA as fp16(q * d), plus K/32 "min
//    columns" fp16(d * isum_j) that carry the Q4_K min term (the weight side
//    of those columns is fp16(-dmin * m_j));
//  * expert GEMM: a wave owns 32 weight rows of one expert and streams their
//    packed bytes once (prefetched one K step ahead), dequantizing each 64-K
//    step to fp16 in registers (magic-number conversion, d*sc folded in) and
//    applying it to up to 128 of the expert's tokens as 32x32x16 MFMA tiles.
//    The fp16 roundings of the two operands move results by ~3e-4 relative.
//    A K split (partials summed in a fixed order by the next kernel) gives
//    the short down projection enough waves to stream HBM.
#include <math.h>

#include "dq_common.h"
#include "dq_f16.h"

namespace {

constexpr int MOE_MAX_EXPERT = 64;
constexpr int MOE_MAX_K = 8;
constexpr int TT = 32;         // tokens per MFMA tile
constexpr int MAX_TILES = 4;   // token tiles per pass of a wave (128 pairs)
constexpr int WAVES = 4;       // waves per workgroup, 32 weight rows each
constexpr int MIN_BLK = 64;    // min columns are padded to a multiple of this

// ---------------------------------------------------------------- routing --
// One wave per token, lane e = expert e. The max is order-independent; the
// double sum runs sequentially over the experts as the reference's loop does.
__global__ __launch_bounds__(256) void moe_route_kernel(const float* __restrict__ logits, int n_tok, int n_exp,
                                                        int k, int norm_w, float w_scale, int32_t* __restrict__ ids,
                                                        float* __restrict__ wts) {
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= n_tok) return;  // uniform per wave
    const float* lg = logits + (size_t)t * n_exp;
    const float v = lane < n_exp ? lg[lane] : 0.0f;
    float m = lg[0];
    for (int i = 1; i < n_exp; ++i) {
        const float o = __shfl(v, i, DQ_WAVE);
        m = (m < o) ? o : m;
    }
    const float e = lane < n_exp ? expf(v - m) : 0.0f;
    double sum = 0.0;
    for (int i = 0; i < n_exp; ++i) sum += (double)__shfl(e, i, DQ_WAVE);
    float p = (float)((double)e / sum);
    if (isnan(p)) p = 0.0f;
    // k rounds of argmax over the unused experts (ties: lower index)
    float key = lane < n_exp ? p : -2.0f;
    float w[MOE_MAX_K];
    int id[MOE_MAX_K];
    float wsum = 0.0f;
    for (int s = 0; s < k; ++s) {
        float bv = key;
        int bi = lane;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const float ov = __shfl_xor(bv, off, DQ_WAVE);
            const int oi = __shfl_xor(bi, off, DQ_WAVE);
            if (ov > bv || (ov == bv && oi < bi)) {
                bv = ov;
                bi = oi;
            }
        }
        id[s] = bi;
        w[s] = __shfl(p, bi, DQ_WAVE);
        wsum += w[s];
        if (lane == bi) key = -1.0f;
    }
    if (lane == 0) {
        for (int s = 0; s < k; ++s) {
            float ws = w[s];
            if (norm_w && wsum > 1e-9f) ws /= wsum;
            if (w_scale != 0.0f && w_scale != 1.0f) ws *= w_scale;
            ids[(size_t)t * k + s] = id[s];
            wts[(size_t)t * k + s] = ws;
        }
    }
}

// Per-expert lists of the (token, slot) entries i = t*k + s, expert-major and
// in ascending i; slot_pos[i] = the entry's position in that order. One thread
// per expert, one workgroup.
__global__ __launch_bounds__(64) void moe_lists_kernel(const int32_t* __restrict__ ids, int n_ent, int n_exp,
                                                       int32_t* __restrict__ offsets, int32_t* __restrict__ pairs,
                                                       int32_t* __restrict__ slot_pos) {
    __shared__ int cnt[MOE_MAX_EXPERT + 1];
    const int e = threadIdx.x;
    if (e < n_exp) {
        int c = 0;
        for (int i = 0; i < n_ent; ++i) c += ids[i] == e;
        cnt[e] = c;
    }
    __syncthreads();
    if (e == 0) {
        int o = 0;
        for (int i = 0; i < n_exp; ++i) {
            const int c = cnt[i];
            cnt[i] = o;
            o += c;
        }
        cnt[n_exp] = o;
    }
    __syncthreads();
    if (e < n_exp) offsets[e] = cnt[e];
    if (e == 0) offsets[n_exp] = cnt[n_exp];
    if (e < n_exp) {
        int o = cnt[e];
        for (int i = 0; i < n_ent; ++i)
            if (ids[i] == e) {
                pairs[o] = i;
                slot_pos[i] = o;
                ++o;
            }
    }
}

// ------------------------------------------------------- activation rows --
// Row p of A: the per-256 quantization of its source row (256 values per
// wave, 4 per lane): d = amax/127, id = 127/amax, q = rint(v*id) (core/matmul.cpp
// :1681-1700); columns [0, K) = fp16(q*d*s), min columns K + j =
// fp16(d*isum_j*s) for the 32-blocks j, zero up to lda; inv[p] = 1/s.
// The source row of p is pairs[p] / k (a token of x) when pairs is given,
// else p.
__global__ __launch_bounds__(256) void moe_act_kernel(const float* __restrict__ src,
                                                      const float* __restrict__ rscale,
                                                      const int32_t* __restrict__ pairs, int k, int n_rows, int K,
                                                      int lda, _Float16* __restrict__ A, float* __restrict__ inv) {
    const int lane = threadIdx.x & 63;
    const int nblk = K / 256;
    const long w = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (w >= (long)n_rows * nblk) return;  // uniform per wave
    const int p = (int)(w / nblk), b = (int)(w % nblk);
    const size_t srow = pairs ? (size_t)(pairs[p] / k) : (size_t)p;
    const float sc = rscale[srow];
    const int c0 = 256 * b + 4 * lane;
    const float4 f = *reinterpret_cast<const float4*>(src + srow * K + c0);
    const float v[4] = {f.x, f.y, f.z, f.w};
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
    _Float16* row = A + (size_t)p * lda;
    *reinterpret_cast<dq_u32x2*>(row + c0) = dq_u32x2{hb[0] | (hb[1] << 16), hb[2] | (hb[3] << 16)};
    // 8 lanes hold one 32-block
#pragma unroll
    for (int off = 1; off < 8; off <<= 1) isum += __shfl_xor(isum, off, DQ_WAVE);
    if ((lane & 7) == 0) row[K + 8 * b + (lane >> 3)] = (_Float16)((d * (float)isum) * sc);
    if (b == 0) {  // zero padding of the min columns, and the output factor
        for (int c = K + K / 32 + lane; c < lda; c += DQ_WAVE) row[c] = (_Float16)0.0f;
        if (lane == 0) inv[p] = 1.0f / sc;
    }
}

// h[p] = silu(g) * u (models/dense_forward.cpp:53-55) with g, u the sums over
// the K splits of the gate and up outputs of pair p (split order 0, 1, ...).
__global__ __launch_bounds__(256) void moe_silu_kernel(const float* __restrict__ gate, const float* __restrict__ up,
                                                       int nsplit, size_t split_stride, size_t n,
                                                       float* __restrict__ h) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    float g = gate[i], u = up[i];
    for (int s = 1; s < nsplit; ++s) {
        g += gate[s * split_stride + i];
        u += up[s * split_stride + i];
    }
    h[i] = g / (1.0f + expf(-g)) * u;
}

// ------------------------------------------------------------ expert GEMM --
struct MoeGemm {
    const uint8_t* w[2];  // packed stacked matrices ([n_exp * rows][K])
    DqLayout L[2];
    float* y[2];          // outputs [nsplit][n_pairs][rows]
    const _Float16* A;    // activation rows [n_pairs][lda]
    const float* inv;     // per pair: 1/s of its activation row
    const int32_t* offsets;
    int rows, K, lda, n_pairs, nsplit, steps_per_split, main_steps, total_steps;
};

// Weight bytes of one 64-K step (Q4_K item of 64 weights) for this lane's row:
// qs bytes 8h..8h+7 of both sub-planes and the super-block header.
struct WRaw {
    dq_u32x2 p0, p1;
    dq_u32x4 hd;
};

__device__ __forceinline__ void load_w(WRaw& r, const uint8_t* base, const DqLayout& L, size_t row, int st, int h,
                                       bool live) {
    if (live) {
        const uint8_t* q = base + L.q_off + row * L.q_row + 16 * (size_t)st + 8 * h;
        r.p0 = __builtin_nontemporal_load(reinterpret_cast<const dq_u32x2*>(q));
        r.p1 = __builtin_nontemporal_load(reinterpret_cast<const dq_u32x2*>(q + L.p_stride));
        r.hd = __builtin_nontemporal_load(
            reinterpret_cast<const dq_u32x4*>(base + L.s_off + row * L.s_row + 16 * (size_t)(st >> 2)));
    } else {
        r.p0 = r.p1 = dq_u32x2{0, 0};
        r.hd = dq_u32x4{0, 0, 0, 0};
    }
}

// B fragments of a main step: kk 0: P0 low nibbles (sub-block 2g, first 16),
// 1: P1 low (sub-block 2g, last 16), 2: P0 high (2g+1), 3: P1 high, times
// a = d * sc of the sub-block (fp16), for this lane's 8 K values 8h..8h+7.
__device__ __forceinline__ void b_main(const WRaw& r, int st, bool ok, h8 (&bf)[4]) {
    const int g = st & 3;
    const float d = dq_h2f((uint16_t)(r.hd.x & 0xFFFF));
    const _Float16 a0 = (_Float16)(ok ? d * (float)q4k_scale(2 * g, r.hd.y, r.hd.z, r.hd.w) : 0.0f);
    const _Float16 a1 = (_Float16)(ok ? d * (float)q4k_scale(2 * g + 1, r.hd.y, r.hd.z, r.hd.w) : 0.0f);
    const h2 bias = {(_Float16)1024.0f, (_Float16)1024.0f};
    const h2 v0 = {a0, a0}, v1 = {a1, a1};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
        const dq_u32x2 src = (kk & 1) ? r.p1 : r.p0;
        const uint32_t m0 = kk < 2 ? (src.x & 0x0F0F0F0Fu) : ((src.x >> 4) & 0x0F0F0F0Fu);
        const uint32_t m1 = kk < 2 ? (src.y & 0x0F0F0F0Fu) : ((src.y >> 4) & 0x0F0F0F0Fu);
        uint32_t t[4];
        bytes_to_h2(m0, bias, kk < 2 ? v0 : v1, &t[0]);
        bytes_to_h2(m1, bias, kk < 2 ? v0 : v1, &t[2]);
        bf[kk] = __builtin_bit_cast(h8, dq_u32x4{t[0], t[1], t[2], t[3]});
    }
}

// B fragments of min step e: column 64e + 16kk + 8h + i is 32-block j of the
// row, i.e. sub-block i of super-block sb = 8e + 2kk + h: fp16(-dmin * m_i).
__device__ __forceinline__ void b_min(const uint8_t* base, const DqLayout& L, size_t row, int e, int h, int nsb,
                                      bool ok, h8 (&bf)[4]) {
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
        const int sb = 8 * e + 2 * kk + h;
        _Float16 v[8];
        if (ok && sb < nsb) {
            const dq_u32x4 hd = *reinterpret_cast<const dq_u32x4*>(base + L.s_off + row * L.s_row + 16 * (size_t)sb);
            const float dmin = dq_h2f((uint16_t)(hd.x >> 16));
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = (_Float16)(-(dmin * (float)q4k_min(i, hd.y, hd.z, hd.w)));
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = (_Float16)0.0f;
        }
        bf[kk] = *reinterpret_cast<const h8*>(v);
    }
}

// Grid: x = 128-row tiles of one expert's rows, y = expert, z = matrix * nsplit
// + split. Wave w of the workgroup owns rows 128x + 32w .. +31; lane l feeds
// row l % 32 with K values 8(l/32)..+7 of each 16-wide slice.
__global__ __launch_bounds__(64 * WAVES) void moe_gemm_kernel(MoeGemm G) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int e = blockIdx.y;
    const int mat = blockIdx.z / G.nsplit, split = blockIdx.z % G.nsplit;
    const int p_begin = G.offsets[e], p_end = G.offsets[e + 1];
    if (p_begin >= p_end) return;  // no token routed to this expert
    const int h = lane >> 5;
    const int rloc = blockIdx.x * (32 * WAVES) + 32 * wave + (lane & 31);
    const bool row_ok = rloc < G.rows;
    const size_t row = (size_t)e * G.rows + (size_t)min(rloc, G.rows - 1);
    const uint8_t* base = G.w[mat];
    const DqLayout L = G.L[mat];
    float* __restrict__ y = G.y[mat] + (size_t)split * G.n_pairs * G.rows;
    const int s0 = split * G.steps_per_split;
    const int s1 = min(G.total_steps, s0 + G.steps_per_split);
    if (s0 >= s1) return;
    const int nsb = G.K / 256;

    for (int c = p_begin; c < p_end; c += TT * MAX_TILES) {
        const int ntile = min(MAX_TILES, (p_end - c + TT - 1) / TT);
        f16v acc[MAX_TILES];
#pragma unroll
        for (int tt = 0; tt < MAX_TILES; ++tt)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[tt][r] = 0.0f;
        // activation row of this lane's token in each tile (clamped to the list)
        const _Float16* arow[MAX_TILES];
#pragma unroll
        for (int tt = 0; tt < MAX_TILES; ++tt)
            arow[tt] = G.A + (size_t)min(c + tt * TT + (lane & 31), p_end - 1) * G.lda + 8 * h;

        WRaw cur, nxt;
        load_w(cur, base, L, row, min(s0, G.main_steps - 1), h, s0 < G.main_steps);
        for (int st = s0; st < s1; ++st) {
            const bool main = st < G.main_steps;
            // prefetch the next main step's weights while this one computes
            load_w(nxt, base, L, row, min(st + 1, G.main_steps - 1), h, st + 1 < min(s1, G.main_steps));
            h8 bf[4];
            if (main) b_main(cur, st, row_ok, bf);
            else b_min(base, L, row, st - G.main_steps, h, nsb, row_ok, bf);
#pragma unroll
            for (int tt = 0; tt < MAX_TILES; ++tt) {
                if (tt < ntile) {
                    const _Float16* ap = arow[tt] + 64 * (size_t)st;
                    h8 af[4];
#pragma unroll
                    for (int kk = 0; kk < 4; ++kk) af[kk] = *reinterpret_cast<const h8*>(ap + 16 * kk);
#pragma unroll
                    for (int kk = 0; kk < 4; ++kk)
                        acc[tt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[kk], bf[kk], acc[tt], 0, 0, 0);
                }
            }
            cur = nxt;
        }
        // D of 32x32x16: lane l, register r -> weight row l % 32, token (r/4)*8 + (l/32)*4 + r%4
        if (row_ok) {
#pragma unroll
            for (int tt = 0; tt < MAX_TILES; ++tt) {
                if (tt < ntile) {
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int p = c + tt * TT + (r >> 2) * 8 + h * 4 + (r & 3);
                        if (p < p_end) y[(size_t)p * G.rows + rloc] = acc[tt][r] * G.inv[p];
                    }
                }
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
    float *wts, *xscale, *hscale, *inv_in, *inv_h;
    _Float16 *a_in, *a_h;
    float *gate, *up, *h, *down;
    size_t total;
};

int min_cols(int K) { return (K / 32 + MIN_BLK - 1) / MIN_BLK * MIN_BLK; }

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
// covering at least 16 K steps.
int pick_split(int n_exp, int rows, int n_mat, int steps) {
    const long waves = (long)n_exp * ((rows + 31) / 32) * n_mat;
    int s = 1;
    while (s < 8 && waves * s < 16L * cus() && steps / (2 * s) >= 16) s *= 2;
    return s;
}

MoeWs carve(const dq_moe_t* m, uint32_t n_tok, int split_gu, int split_d, uint8_t* base) {
    const size_t n_ent = (size_t)n_tok * m->n_expert_used;
    const size_t E = m->n_embd, F = m->n_ff;
    const size_t lda_in = E + min_cols((int)E), lda_h = F + min_cols((int)F);
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
    w.xscale = (float*)take((size_t)n_tok * 4);
    w.hscale = (float*)take(n_ent * 4);
    w.inv_in = (float*)take(n_ent * 4);
    w.inv_h = (float*)take(n_ent * 4);
    w.a_in = (_Float16*)take(n_ent * lda_in * 2);
    w.gate = (float*)take((size_t)split_gu * n_ent * F * 4);
    w.up = (float*)take((size_t)split_gu * n_ent * F * 4);
    w.h = (float*)take(n_ent * F * 4);
    w.a_h = (_Float16*)take(n_ent * lda_h * 2);
    w.down = (float*)take((size_t)split_d * n_ent * E * 4);
    w.total = off;
    return w;
}

bool moe_ok(const dq_moe_t* m) {
    if (!m || m->fmt != DQ_FMT_Q4_K) return false;
    if (m->n_expert == 0 || m->n_expert > MOE_MAX_EXPERT) return false;
    if (m->n_expert_used == 0 || m->n_expert_used > MOE_MAX_K || m->n_expert_used > m->n_expert) return false;
    if (m->n_embd == 0 || m->n_embd % 256 || m->n_ff == 0 || m->n_ff % 256) return false;
    if (m->n_embd > (1u << 20) || m->n_ff > (1u << 20)) return false;
    if ((size_t)m->n_expert * m->n_ff > 0x3FFFFFFF || (size_t)m->n_expert * m->n_embd > 0x3FFFFFFF) return false;
    return true;
}

void splits(const dq_moe_t* m, int* sgu, int* sd) {
    const int steps_gu = (int)m->n_embd / 64 + min_cols((int)m->n_embd) / 64;
    const int steps_d = (int)m->n_ff / 64 + min_cols((int)m->n_ff) / 64;
    *sgu = pick_split((int)m->n_expert, (int)m->n_ff, 2, steps_gu);
    *sd = pick_split((int)m->n_expert, (int)m->n_embd, 1, steps_d);
}

int launch_gemm(const uint8_t* w0, const uint8_t* w1, int n_mat, int n_exp, int rows, int K, const _Float16* A,
                const float* inv, int lda, const int32_t* offsets, int n_pairs, int nsplit, float* y0, float* y1,
                hipStream_t s) {
    MoeGemm G{};
    G.w[0] = w0;
    G.w[1] = w1 ? w1 : w0;
    if (!dq_layout(DQ_FMT_Q4_K, (size_t)n_exp * rows, K, &G.L[0])) return DQ_ERR_NOT_SUPPORTED;
    G.L[1] = G.L[0];
    G.y[0] = y0;
    G.y[1] = y1 ? y1 : y0;
    G.A = A;
    G.inv = inv;
    G.offsets = offsets;
    G.rows = rows;
    G.K = K;
    G.lda = lda;
    G.n_pairs = n_pairs;
    G.nsplit = nsplit;
    G.main_steps = K / 64;
    G.total_steps = G.main_steps + min_cols(K) / 64;
    G.steps_per_split = (G.total_steps + nsplit - 1) / nsplit;
    const dim3 grid((unsigned)((rows + 32 * WAVES - 1) / (32 * WAVES)), (unsigned)n_exp, (unsigned)(n_mat * nsplit));
    moe_gemm_kernel<<<grid, 64 * WAVES, 0, s>>>(G);
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
    const int lda_in = E + min_cols(E), lda_h = F + min_cols(F);
    // routing and lists
    DQ_TRY(dq_moe_route(d_logits, n_tok, m->n_expert, m->n_expert_used, m->norm_w, m->w_scale, w.ids, w.wts, stream));
    moe_lists_kernel<<<1, 64, 0, s>>>(w.ids, n_ent, n_exp, w.offsets, w.pairs, w.slot_pos);
    DQ_TRY(dq_launch_status());
    // activation rows of the pairs (row scale per token)
    row_scale_kernel<<<n_tok, 256, 0, s>>>(d_x, E, w.xscale);
    DQ_TRY(dq_launch_status());
    {
        const long waves = (long)n_ent * (E / 256);
        moe_act_kernel<<<(unsigned)((waves + 3) / 4), 256, 0, s>>>(d_x, w.xscale, w.pairs, k, n_ent, E, lda_in,
                                                                   w.a_in, w.inv_in);
        DQ_TRY(dq_launch_status());
    }
    // gate and up of every pair (one launch, two matrices)
    DQ_TRY(launch_gemm((const uint8_t*)m->wgate, (const uint8_t*)m->wup, 2, n_exp, F, E, w.a_in, w.inv_in, lda_in,
                       w.offsets, n_ent, sgu, w.gate, w.up, s));
    // h = silu(gate) * up, quantized for the down projection
    {
        const size_t n = (size_t)n_ent * F;
        moe_silu_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(w.gate, w.up, sgu, n, n, w.h);
        DQ_TRY(dq_launch_status());
        row_scale_kernel<<<n_ent, 256, 0, s>>>(w.h, F, w.hscale);
        DQ_TRY(dq_launch_status());
        const long waves = (long)n_ent * (F / 256);
        moe_act_kernel<<<(unsigned)((waves + 3) / 4), 256, 0, s>>>(w.h, w.hscale, nullptr, k, n_ent, F, lda_h, w.a_h,
                                                                   w.inv_h);
        DQ_TRY(dq_launch_status());
    }
    DQ_TRY(launch_gemm((const uint8_t*)m->wdown, nullptr, 1, n_exp, E, F, w.a_h, w.inv_h, lda_h, w.offsets, n_ent,
                       sd, w.down, nullptr, s));
    {
        const size_t n = (size_t)n_tok * E;
        moe_scatter_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(w.down, sd, (size_t)n_ent * E, w.slot_pos,
                                                                       w.wts, k, (int)n_tok, E, d_out);
        DQ_TRY(dq_launch_status());
    }
    return DQ_OK;
}

}  // extern "C"
