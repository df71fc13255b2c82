// dq_prefill.hip - the prompt (prefill) side of the Q8_0 KV cache: the K/V
// rows of a run of tokens written in one launch, optionally with their RoPE,
// and causal attention of every token of the run over the cache.
//
// Cache layout as in dq_attn.hip: [pos][kv_head][hd/32 Q8_0 blocks of 34 B].
//
// Attention (reference core/attn_cpu.cpp:128-390, the CPU definition of
// record; the GPU kernels it replaces are attention_prefill_*,
// cuda/backend_cuda.cu:7080-8290): row (token t, head h) at position
// pos0 + t attends to keys [lo, pos0 + t] of KV head h / hpk, lo = 0 or the
// sliding-window start; scores q.k / sqrt(hd), softmax, sum p v.
//
// Work split: a workgroup takes one KV head and 128 consecutive rows
// (row = token * hpk + head-in-group, so the query heads sharing a KV head
// share every K/V tile), four waves of 32 rows. Keys go in tiles of 32: the
// tile's raw Q8_0 rows are staged through LDS once per workgroup and turned
// into fp16 operands there; each wave then runs
//   S^T = K Q^T      (v_mfma_f32_32x32x16_f16, M = keys, N = its 32 rows)
//   online softmax   (one row per lane pair: lanes l and l + 32)
//   O^T += V^T P^T   (M = head dims, N = rows)
// so that a row's scores, running max/sum and output all sit in the two
// lanes of that row and no transpose is needed between the two products.
//
// Precision: every operand is split into fp16 hi + lo parts and each product
// runs as hi*hi + lo*hi + hi*lo (the lo*lo term is below 2^-22 relative), so
// the scores and the weighted sums carry ~22 bits. K and V values d*q (fp16
// d times an int8, at most 18 significant bits) split exactly. The query is
// scaled by 1/sqrt(hd) * log2(e) in fp32 first, so the softmax uses exp2.
// Range: the cached values and the scaled query must lie inside fp16
// (|x| < 65504), which Q8_0 rows of activations satisfy.
#include <cstdlib>
#include <mutex>

#include "dq_common.h"
#include "dq_f16.h"

namespace {

typedef _Float16 h4 __attribute__((ext_vector_type(4)));

constexpr int KT = 32;    // keys per tile
constexpr int NT = 256;   // threads per workgroup
constexpr int RPW = 32;   // rows per wave
constexpr int RPB = 128;  // rows per workgroup

struct PrefillArgs {
    const float* q;       // [n_tok][q_dim]
    float* out;           // [n_tok][q_dim]
    const uint8_t* kc;    // cache of the layer
    const uint8_t* vc;
    size_t pos_bytes;
    int q_dim, n_tok, hpk, n_kv, pos0, n_swa, n_qblk;
    float qscale;         // 1/sqrt(hd) * log2(e)
    int split;            // key splits per (KV head, row block); > 1: partial records
    float* part;          // [n_kv][n_rows][split][HD + 4]: O (unnormalised), max (log2 units), sum, pad
};

__device__ __forceinline__ int win_lo(int pos, int n_swa) {
    return (n_swa > 0 && pos + 1 > n_swa) ? pos + 1 - n_swa : 0;
}

__device__ __forceinline__ void split8(const float (&x)[8], h8& hi, h8& lo) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const _Float16 h = (_Float16)x[i];
        hi[i] = h;
        lo[i] = (_Float16)(x[i] - (float)h);
    }
}

// Column of actual key a (0..31) in the transposed V tile: the key order in
// which a lane's scores (S^T layout: keys 8*(r/4) + 4*(l/32) + r%4 of
// register r) are the B operand of the V product in register order, i.e.
// bits 2 and 3 of the key swapped.
__device__ __forceinline__ int vcol_group(int g) {  // g = a / 4
    return (g & 4) | ((g & 1) << 1) | ((g >> 1) & 1);
}

// Two waves per SIMD for HD <= 128 (the register budget fits without spills:
// the conversion and softmax VALU work of one workgroup overlaps the other's
// MFMAs); HD = 256 needs one.
template <int HD, bool SPLIT>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(HD <= 128 ? 2 : 1, 2))) void attn_prefill_kernel(
    PrefillArgs A) {
    constexpr int NB = HD / 32;          // Q8_0 blocks per row
    constexpr int RB = NB * DQ_SZ_Q8_0;  // row bytes
    constexpr int RBW = RB / 4;          // row dwords
    constexpr int NS = HD / 16;          // K steps of the score product
    constexpr int KROW = HD + 8;         // fp16 per K row in LDS (16-byte pad)
    constexpr int VROW = KT + 8;         // fp16 per transposed V row
    constexpr int PER = (KT * RBW + NT - 1) / NT;
    constexpr int UNITS = 2 * HD;        // conversion units of K (and of V) per tile
    static_assert(RB % 4 == 0, "rows must be whole dwords");

    __shared__ uint32_t rawk[KT * RBW], rawv[KT * RBW];
    __shared__ __attribute__((aligned(16))) _Float16 kh[KT * KROW], kl[KT * KROW];
    __shared__ __attribute__((aligned(16))) _Float16 vh[HD * VROW], vl[HD * VROW];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, half = lane >> 5;
    const int hkv = blockIdx.x % A.n_kv;
    const int sp = SPLIT ? (int)(blockIdx.x / A.n_kv) % A.split : 0;
    const int qb = A.n_qblk - 1 - (int)(blockIdx.x / A.n_kv / (SPLIT ? A.split : 1));  // longest rows first
    const int hpk = A.hpk;
    const int n_rows = A.n_tok * hpk;
    const int R0 = qb * RPB;
    const int p_first = A.pos0 + R0 / hpk;
    const int p_last = A.pos0 + min(R0 + RPB - 1, n_rows - 1) / hpk;
    const int k_begin = win_lo(p_first, A.n_swa);

    // this wave's rows and this lane's row (rows past the end are computed
    // on a clamped copy and not stored)
    const int wr0 = R0 + RPW * wave;
    const bool wave_live = wr0 < n_rows;
    const int w_pmax = A.pos0 + min(wr0 + RPW - 1, n_rows - 1) / hpk;
    const int w_lomin = win_lo(A.pos0 + min(wr0, n_rows - 1) / hpk, A.n_swa);
    const int row = wr0 + (lane & 31);
    const bool row_ok = row < n_rows;
    const int rc = min(row, n_rows - 1);
    const int t = rc / hpk, head = hkv * hpk + rc % hpk;
    const int pos = A.pos0 + t;
    const int lo = win_lo(pos, A.n_swa);

    // K/V rows of a tile into registers (positions clamped into
    // [k_begin, p_last]: rows outside are never read, in-tile keys past them
    // are masked)
    uint32_t rk[PER], rv[PER];
    auto load_tile = [&](int k0) {
#pragma unroll
        for (int it = 0; it < PER; ++it) {
            const int i = min(tid + it * NT, KT * RBW - 1);
            const int key = i / RBW, c = i - key * RBW;
            const int p = max(min(k0 + key, p_last), k_begin);
            const size_t off = (size_t)p * A.pos_bytes + (size_t)hkv * RB + 4 * c;
            rk[it] = *reinterpret_cast<const uint32_t*>(A.kc + off);
            rv[it] = *reinterpret_cast<const uint32_t*>(A.vc + off);
        }
    };
    int kt0 = k_begin & ~(KT - 1);
    int k_end = p_last;  // last key of this workgroup's range
    if constexpr (SPLIT) {
        // this split's contiguous share of the key tiles
        const int n_tiles = (p_last - kt0) / KT + 1;
        const int per = (n_tiles + A.split - 1) / A.split;
        const int first = kt0 + sp * per * KT;
        k_end = min(p_last, first + per * KT - 1);
        kt0 = first;
    }
    load_tile(kt0);

    // query fragments (B operand of S^T = K Q^T): dims 16s + 8*half + i
    h8 qh[NS], ql[NS];
    {
        const float* qp = A.q + (size_t)t * A.q_dim + (size_t)head * HD + 8 * half;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const float4 a = *reinterpret_cast<const float4*>(qp + 16 * s);
            const float4 b = *reinterpret_cast<const float4*>(qp + 16 * s + 4);
            const float x[8] = {a.x * A.qscale, a.y * A.qscale, a.z * A.qscale, a.w * A.qscale,
                                b.x * A.qscale, b.y * A.qscale, b.z * A.qscale, b.w * A.qscale};
            split8(x, qh[s], ql[s]);
        }
    }

    f16v o[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[b][r] = 0.0f;
    float m = -INFINITY, l = 0.0f;

    const uint8_t* rkb = reinterpret_cast<const uint8_t*>(rawk);
    const uint8_t* rvb = reinterpret_cast<const uint8_t*>(rawv);
    for (int k0 = kt0; k0 <= k_end; k0 += KT) {
#pragma unroll
        for (int it = 0; it < PER; ++it) {
            const int i = tid + it * NT;
            if (i < KT * RBW) {
                rawk[i] = rk[it];
                rawv[i] = rv[it];
            }
        }
        __syncthreads();
        // ---- raw Q8_0 -> fp16 hi/lo operands
        for (int u = tid; u < UNITS; u += NT) {
            {   // K: (key, 16 dims) -> kh/kl[key][dims]
                const int key = u / (HD / 16), part = u % (HD / 16);
                const int b = part >> 1, hf = part & 1;
                const uint8_t* bp = rkb + key * RB + b * DQ_SZ_Q8_0;
                const float d = dq_h2f(*reinterpret_cast<const uint16_t*>(bp));
                float x[16];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const uint16_t w = *reinterpret_cast<const uint16_t*>(bp + 2 + 16 * hf + 2 * j);
                    x[2 * j] = d * (float)(int8_t)(w & 0xFF);
                    x[2 * j + 1] = d * (float)(int8_t)(w >> 8);
                }
                h8 a0, a1, b0, b1;
                split8(reinterpret_cast<const float(&)[8]>(x[0]), a0, b0);
                split8(reinterpret_cast<const float(&)[8]>(x[8]), a1, b1);
                _Float16* dh = kh + key * KROW + 32 * b + 16 * hf;
                _Float16* dl = kl + key * KROW + 32 * b + 16 * hf;
                *reinterpret_cast<h8*>(dh) = a0;
                *reinterpret_cast<h8*>(dh + 8) = a1;
                *reinterpret_cast<h8*>(dl) = b0;
                *reinterpret_cast<h8*>(dl + 8) = b1;
            }
            {   // V: (4 keys, 4 dims) -> vh/vl[dim][permuted keys]
                const int g = u & 7, c = u >> 3;
                const int b = c >> 3, off = 4 * (c & 7);
                float x[4][4];  // [key][dim]
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) {
                    const uint8_t* bp = rvb + (4 * g + kk) * RB + b * DQ_SZ_Q8_0;
                    const float d = dq_h2f(*reinterpret_cast<const uint16_t*>(bp));
                    const uint16_t w0 = *reinterpret_cast<const uint16_t*>(bp + 2 + off);
                    const uint16_t w1 = *reinterpret_cast<const uint16_t*>(bp + 4 + off);
                    x[kk][0] = d * (float)(int8_t)(w0 & 0xFF);
                    x[kk][1] = d * (float)(int8_t)(w0 >> 8);
                    x[kk][2] = d * (float)(int8_t)(w1 & 0xFF);
                    x[kk][3] = d * (float)(int8_t)(w1 >> 8);
                }
                const int col = 4 * vcol_group(g);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    h4 hv, lv;
#pragma unroll
                    for (int kk = 0; kk < 4; ++kk) {
                        const _Float16 h = (_Float16)x[kk][j];
                        hv[kk] = h;
                        lv[kk] = (_Float16)(x[kk][j] - (float)h);
                    }
                    *reinterpret_cast<h4*>(vh + (4 * c + j) * VROW + col) = hv;
                    *reinterpret_cast<h4*>(vl + (4 * c + j) * VROW + col) = lv;
                }
            }
        }
        if (k0 + KT <= k_end) load_tile(k0 + KT);
        __syncthreads();
        if (!wave_live || k0 > w_pmax || k0 + KT - 1 < w_lomin) continue;  // uniform per wave

        // ---- scores S^T (lane: row lane%32, keys 8*(r/4) + 4*half + r%4)
        f16v st;
#pragma unroll
        for (int r = 0; r < 16; ++r) st[r] = 0.0f;
        {
            const _Float16* krh = kh + (lane & 31) * KROW + 8 * half;
            const _Float16* krl = kl + (lane & 31) * KROW + 8 * half;
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                const h8 ah = *reinterpret_cast<const h8*>(krh + 16 * s);
                const h8 al = *reinterpret_cast<const h8*>(krl + 16 * s);
                st = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, qh[s], st, 0, 0, 0);
                st = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, qh[s], st, 0, 0, 0);
                st = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, ql[s], st, 0, 0, 0);
            }
        }
        // ---- causal / window mask, online softmax
        float mt = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int key = k0 + 8 * (r >> 2) + 4 * half + (r & 3);
            const bool ok = key <= pos && key >= lo;
            st[r] = ok ? st[r] : -INFINITY;
            mt = fmaxf(mt, st[r]);
        }
        mt = fmaxf(mt, __shfl_xor(mt, 32, DQ_WAVE));
        const float mn = fmaxf(m, mt);
        const float corr = mn == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m - mn);
        float ps = 0.0f;
        float p[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            p[r] = st[r] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(st[r] - mn);
            ps += p[r];
        }
        l = l * corr + ps;
        m = mn;
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[b][r] *= corr;
        h8 ph[2], pl[2];
        split8(reinterpret_cast<const float(&)[8]>(p[0]), ph[0], pl[0]);
        split8(reinterpret_cast<const float(&)[8]>(p[8]), ph[1], pl[1]);
        // ---- O^T += V^T P^T (lane: row lane%32, dims 32b + 8*(r/4) + 4*half + r%4)
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const _Float16* vrh = vh + (32 * b + (lane & 31)) * VROW + 8 * half;
            const _Float16* vrl = vl + (32 * b + (lane & 31)) * VROW + 8 * half;
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                const h8 ah = *reinterpret_cast<const h8*>(vrh + 16 * s);
                const h8 al = *reinterpret_cast<const h8*>(vrl + 16 * s);
                o[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, ph[s], o[b], 0, 0, 0);
                o[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, ph[s], o[b], 0, 0, 0);
                o[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, pl[s], o[b], 0, 0, 0);
            }
        }
    }
    if (!wave_live) return;
    const float lt = l + __shfl_xor(l, 32, DQ_WAVE);
    if constexpr (SPLIT) {
        // partial record of this row and split: O, max, sum (a split with no
        // visible key leaves max = -inf, sum = 0)
        if (!row_ok) return;
        float* rec = A.part + (((size_t)hkv * n_rows + row) * A.split + sp) * (HD + 4);  // 16-byte aligned
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int g = 0; g < 4; ++g)
                *reinterpret_cast<float4*>(rec + 32 * b + 8 * g + 4 * half) =
                    make_float4(o[b][4 * g], o[b][4 * g + 1], o[b][4 * g + 2], o[b][4 * g + 3]);
        if (half == 0) {
            rec[HD] = m;
            rec[HD + 1] = lt;
        }
        return;
    }
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
    if (!row_ok) return;
    float* dst = A.out + (size_t)t * A.q_dim + (size_t)head * HD + 4 * half;
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int g = 0; g < 4; ++g)
            *reinterpret_cast<float4*>(dst + 32 * b + 8 * g) =
                make_float4(o[b][4 * g] * inv, o[b][4 * g + 1] * inv, o[b][4 * g + 2] * inv, o[b][4 * g + 3] * inv);
}

// Merge of the key splits: one wave per row combines its split records
// (max M = max m_s, O = sum O_s 2^(m_s - M) / sum l_s 2^(m_s - M)) and writes
// the row's output.
template <int HD>
__global__ __launch_bounds__(256) void attn_prefill_merge_kernel(PrefillArgs A) {
    constexpr int PER = HD / 64;  // dims per lane
    const int n_rows = A.n_tok * A.hpk;
    const int w = (int)(blockIdx.x * 4 + (threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    if (w >= n_rows * A.n_kv) return;  // uniform per wave
    const int hkv = w / n_rows, row = w % n_rows;
    const int t = row / A.hpk, head = hkv * A.hpk + row % A.hpk;
    const float* rec = A.part + ((size_t)hkv * n_rows + row) * A.split * (HD + 4);
    float M = -INFINITY;
    for (int s = 0; s < A.split; ++s) M = fmaxf(M, rec[s * (HD + 4) + HD]);
    float L = 0.0f, o[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) o[i] = 0.0f;
    for (int s = 0; s < A.split; ++s) {
        const float* r = rec + s * (HD + 4);
        const float ms = r[HD];
        const float f = ms == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ms - M);
        L += r[HD + 1] * f;
#pragma unroll
        for (int i = 0; i < PER; ++i) o[i] += r[lane + 64 * i] * f;
    }
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    float* dst = A.out + (size_t)t * A.q_dim + (size_t)head * HD;
#pragma unroll
    for (int i = 0; i < PER; ++i) dst[lane + 64 * i] = o[i] * inv;
}

// ------------------------------------------------------------ row writes --
// kv_quantize_batch_kernel (cuda/backend_cuda.cu:7028-7058) / write_kv_cache
// per position: kv_quantize_row (kv/kv_quant.cpp:31-56) of every token's K
// and V rows into positions pos0 + t. One lane per 32-value block: per block
// amax, d = amax/127, q = clamp(rint(x/d), -127, 127).
__device__ __forceinline__ void kv_block_store(const float* x, uint8_t* dst) {
    float xv[32];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 f = reinterpret_cast<const float4*>(x)[i];
        xv[4 * i] = f.x, xv[4 * i + 1] = f.y, xv[4 * i + 2] = f.z, xv[4 * i + 3] = f.w;
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(xv[i]));
    const float d = amax > 0.0f ? amax / 127.0f : 0.0f;
    const float id = d > 0.0f ? 1.0f / d : 0.0f;
    uint16_t* o = reinterpret_cast<uint16_t*>(dst);  // 34-byte blocks: 2-byte aligned
    o[0] = dq_f2h(d);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        int a = (int)rintf(xv[2 * i] * id), c = (int)rintf(xv[2 * i + 1] * id);
        a = a > 127 ? 127 : (a < -127 ? -127 : a);
        c = c > 127 ? 127 : (c < -127 ? -127 : c);
        o[1 + i] = (uint16_t)((a & 0xFF) | ((c & 0xFF) << 8));
    }
}

__global__ __launch_bounds__(256) void kv_write_batch_kernel(const float* __restrict__ k, const float* __restrict__ v,
                                                            size_t ld, int n_tok, int blocks_per_row,
                                                            uint8_t* __restrict__ kc, uint8_t* __restrict__ vc,
                                                            size_t pos_bytes, int pos0) {
    const int per_tok = 2 * blocks_per_row;
    const long gb = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (gb >= (long)n_tok * per_tok) return;
    const int t = (int)(gb / per_tok), b = (int)(gb % per_tok);
    const bool is_v = b >= blocks_per_row;
    const int bb = is_v ? b - blocks_per_row : b;
    const float* x = (is_v ? v : k) + (size_t)t * ld + (size_t)bb * 32;
    uint8_t* dst = (is_v ? vc : kc) + (size_t)(pos0 + t) * pos_bytes + (size_t)bb * DQ_SZ_Q8_0;
    kv_block_store(x, dst);
}

// The optional Q/K/V biases and per-head QK-norm, then RoPE of a run of tokens
// (models/dense_forward.cpp:668-680 per token, table row t =
// dq_rope_cache(pos0 + t)) on the query heads, in place, and on the
// key heads, whose rotated rows then go into the cache with the value rows
// (kv_quantize_row). HD-dim heads (64, 128, 256); grid (n_head + 2 n_kv,
// n_tok), 64 threads, thread j holds dims j + 64 i.
template <int HD>
__global__ __launch_bounds__(64) void rope_kv_batch_kernel(float* __restrict__ q, const float* __restrict__ k,
                                                           const float* __restrict__ v, size_t q_ld, size_t kv_ld,
                                                           const float* __restrict__ rope, int n_rot, int n_head,
                                                           int n_kv, uint8_t* __restrict__ kc,
                                                           uint8_t* __restrict__ vc, size_t pos_bytes, int pos0,
                                                           DqQkvPost post) {
    constexpr int QV = HD / 64;
    const int r = blockIdx.x, t = blockIdx.y, j = threadIdx.x;
    const int kind = r < n_head ? 0 : (r < n_head + n_kv ? 1 : 2);
    const int hh = kind == 0 ? r : (kind == 1 ? r - n_head : r - n_head - n_kv);
    float* qrow = q + (size_t)t * q_ld + (size_t)hh * HD;
    const float* src = kind == 0 ? qrow : (kind == 1 ? k : v) + (size_t)t * kv_ld + (size_t)hh * HD;
    float x[QV];
#pragma unroll
    for (int i = 0; i < QV; ++i) x[i] = src[j + 64 * i];
    dq_qkv_post<HD>(x, kind, hh, j, post);  // optional biases and QK-norm (:3318-3342)
    if (kind < 2 && rope) {
        const float* tab = rope + (size_t)t * n_rot;
        if (n_rot == HD) {
            dq_rope_head<HD>(x, tab, j);
        } else {
            __shared__ float rowb[HD];
#pragma unroll
            for (int i = 0; i < QV; ++i) rowb[j + 64 * i] = x[i];
            __syncthreads();
            const int hn = n_rot / 2;
            for (int jj = j; jj < hn; jj += 64) {
                const float c = tab[2 * jj], s = tab[2 * jj + 1];
                const float a = rowb[jj], b = rowb[jj + hn];
                rowb[jj] = a * c - b * s;
                rowb[jj + hn] = a * s + b * c;
            }
            __syncthreads();
#pragma unroll
            for (int i = 0; i < QV; ++i) x[i] = rowb[j + 64 * i];
        }
    }
    if (kind == 0) {
#pragma unroll
        for (int i = 0; i < QV; ++i) qrow[j + 64 * i] = x[i];
        return;
    }
    dq_q8_0_row<HD>(x, j, (kind == 1 ? kc : vc) + (size_t)(pos0 + t) * pos_bytes + (size_t)hh * (HD / 32) * DQ_SZ_Q8_0);
}

// Sandwich norm and residual of every row (models/dense_forward.cpp
// :4140-4147 and :4245-4255; batch :3546-3550, :3618-3626): out =
// rms_norm_vec(a, w) + b, the norm with squares in float summed in double,
// scale = 1/sqrtf(mean + eps), a * scale * w. One workgroup per row; out may
// alias b.
__global__ __launch_bounds__(256) void post_norm_add_kernel(const float* __restrict__ a, const float* __restrict__ w,
                                                           const float* b, int n, float eps, float* out) {
    __shared__ double part[4];
    const size_t row = (size_t)blockIdx.x * n;
    const int t = threadIdx.x;
    double acc = 0.0;
    for (int i = 4 * t; i < n; i += 1024) {
        const float4 x = *reinterpret_cast<const float4*>(a + row + i);
        const float s0 = x.x * x.x, s1 = x.y * x.y, s2 = x.z * x.z, s3 = x.w * x.w;
        acc += (double)s0;
        acc += (double)s1;
        acc += (double)s2;
        acc += (double)s3;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, DQ_WAVE);
    if ((t & 63) == 0) part[t >> 6] = acc;
    __syncthreads();
    const double sum = (part[0] + part[1]) + (part[2] + part[3]);
    const float sc = 1.0f / sqrtf((float)(sum / (double)n) + eps);
    for (int i = 4 * t; i < n; i += 1024) {
        const float4 x = *reinterpret_cast<const float4*>(a + row + i);
        const float4 ww = *reinterpret_cast<const float4*>(w + i);
        const float4 c = *reinterpret_cast<const float4*>(b + row + i);
        *reinterpret_cast<float4*>(out + row + i) = make_float4(x.x * sc * ww.x + c.x, x.y * sc * ww.y + c.y,
                                                                x.z * sc * ww.z + c.z, x.w * sc * ww.w + c.w);
    }
}

// rms_norm_vec (models/dense_forward.cpp:129-165) of every row of a
// [n_tok][n] array: squares in float summed in double, scale =
// 1/sqrtf(mean + eps), y = x * scale * w. With b: x = a + b first (the
// attention residual, :3549-3557), written to h. One workgroup per row.
__global__ __launch_bounds__(256) void rms_norm_rows_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                                           float* __restrict__ h, const float* __restrict__ w, int n,
                                                           float eps, float* __restrict__ y) {
    __shared__ double part[4];
    const size_t row = (size_t)blockIdx.x * n;
    const int t = threadIdx.x;
    double acc = 0.0;
    for (int i = 4 * t; i < n; i += 1024) {
        float4 x = *reinterpret_cast<const float4*>(a + row + i);
        if (b) {
            const float4 c = *reinterpret_cast<const float4*>(b + row + i);
            x = make_float4(x.x + c.x, x.y + c.y, x.z + c.z, x.w + c.w);
            if (h) *reinterpret_cast<float4*>(h + row + i) = x;
        }
        const float s0 = x.x * x.x, s1 = x.y * x.y, s2 = x.z * x.z, s3 = x.w * x.w;
        acc += (double)s0;
        acc += (double)s1;
        acc += (double)s2;
        acc += (double)s3;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, DQ_WAVE);
    if ((t & 63) == 0) part[t >> 6] = acc;
    __syncthreads();
    const double sum = (part[0] + part[1]) + (part[2] + part[3]);
    const float sc = 1.0f / sqrtf((float)(sum / (double)n) + eps);
    for (int i = 4 * t; i < n; i += 1024) {
        float4 x = *reinterpret_cast<const float4*>(a + row + i);
        if (b) {
            const float4 c = *reinterpret_cast<const float4*>(b + row + i);
            x = make_float4(x.x + c.x, x.y + c.y, x.z + c.z, x.w + c.w);
        }
        const float4 ww = *reinterpret_cast<const float4*>(w + i);
        *reinterpret_cast<float4*>(y + row + i) =
            make_float4(x.x * sc * ww.x, x.y * sc * ww.y, x.z * sc * ww.z, x.w * sc * ww.w);
    }
}

// out = a + b (the FFN residual, models/dense_forward.cpp:3616-3624), 4 per lane.
// The per-head attention output gate of a prompt chunk (DenseQuirks::attn_gate,
// models/dense_forward.cpp:3527-3536): row t, head h of the attention output
// [n_tok][q_dim] times 1 / (1 + exp(-g[t][h])). One workgroup per (token,
// head), a float4 of the head per thread.
__global__ __launch_bounds__(64) void attn_gate_rows_kernel(float* __restrict__ a, const float* __restrict__ g,
                                                             int n_head, int hd, size_t q_dim) {
    const int t = blockIdx.x / n_head, h = blockIdx.x % n_head;
    const float gv = 1.0f / (1.0f + expf(-g[(size_t)t * n_head + h]));
    float* row = a + (size_t)t * q_dim + (size_t)h * hd;
    for (int i = 4 * threadIdx.x; i < hd; i += 256) {
        float4 v = *reinterpret_cast<float4*>(row + i);
        v.x *= gv, v.y *= gv, v.z *= gv, v.w *= gv;
        *reinterpret_cast<float4*>(row + i) = v;
    }
}

__global__ __launch_bounds__(256) void add_kernel(const float* __restrict__ a, const float* __restrict__ b, size_t n4,
                                                 float* __restrict__ out) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) return;
    const float4 x = reinterpret_cast<const float4*>(a)[i];
    const float4 y = reinterpret_cast<const float4*>(b)[i];
    reinterpret_cast<float4*>(out)[i] = make_float4(x.x + y.x, x.y + y.y, x.z + y.z, x.w + y.w);
}

// ---------------------------------------------------------- layer prefill --
// Workspace of dq_layer_prefill: fp32 activations of the chunk, then one
// GEMM activation workspace per K-quant format (sized for the widest input).
struct PrefillWs {
    float *xn, *q, *k, *v, *attn, *h, *gate, *up, *down;
    float* ag;       // attention gate values [n_tok][n_head]
    uint8_t* gw[3];  // activation layouts: Q4_K, Q6_K, natural order (Q8_0 / Q4_0)
    uint8_t* aw;     // attention key-split records
    size_t gw_bytes, aw_bytes, total;
};

bool prefill_layer_ok(const dq_layer_t* L) {
    const int f[7] = {L->fmt_q, L->fmt_k, L->fmt_v, L->fmt_o, L->fmt_gate, L->fmt_up, L->fmt_down};
    for (int i = 0; i < 7; ++i)
        if (f[i] != DQ_FMT_Q4_K && f[i] != DQ_FMT_Q6_K && f[i] != DQ_FMT_Q8_0 && f[i] != DQ_FMT_Q4_0) return false;
    if (!dq_head_dim_supported(L->head_dim) || L->n_head_kv == 0 || L->n_head % L->n_head_kv) return false;
    if (L->n_embd % 256 || L->n_ff % 256 || ((size_t)L->n_head * L->head_dim) % 256) return false;
    if (L->n_rot == 0 || L->n_rot > L->head_dim || L->n_rot % 2) return false;
    if (L->wag && L->fmt_ag != DQ_FMT_Q4_K && L->fmt_ag != DQ_FMT_Q6_K && L->fmt_ag != DQ_FMT_Q8_0 &&
        L->fmt_ag != DQ_FMT_Q4_0)
        return false;
    return true;
}

PrefillWs prefill_carve(const dq_layer_t* L, uint32_t n_tok, uint8_t* base) {
    PrefillWs w{};
    const size_t E = L->n_embd, QD = (size_t)L->n_head * L->head_dim, KVD = (size_t)L->n_head_kv * L->head_dim;
    const size_t F = L->n_ff, T = n_tok;
    size_t off = 0;
    auto take = [&](size_t floats) {
        float* p = base ? reinterpret_cast<float*>(base + off) : nullptr;
        off += dq_align256(floats * 4);
        return p;
    };
    w.xn = take(T * E);
    w.q = take(T * QD);
    w.k = take(T * KVD);
    w.v = take(T * KVD);
    w.attn = take(T * QD);
    w.h = take(T * E);
    w.gate = take(T * F);
    w.up = take(T * F);
    w.down = take(T * E);
    w.ag = take(L->wag ? T * L->n_head : 0);
    size_t gb = 0;
    const size_t cols[3] = {E, QD, F};
    const int fmts[3] = {DQ_FMT_Q4_K, DQ_FMT_Q6_K, DQ_FMT_Q8_0};
    for (int f = 0; f < 3; ++f)
        for (size_t c : cols) {
            size_t b = 0;
            if (dq_gemm_workspace_bytes(fmts[f], 1, c, T, &b) == DQ_OK && b > gb) gb = b;
        }
    w.gw_bytes = dq_align256(gb);
    for (int f = 0; f < 3; ++f) {
        w.gw[f] = base ? base + off : nullptr;
        off += w.gw_bytes;
    }
    size_t ab = 0;
    (void)dq_attn_prefill_workspace_bytes(n_tok, L->n_head, L->n_head_kv, L->head_dim, &ab);
    w.aw = base ? base + off : nullptr;
    w.aw_bytes = ab;
    off += ab;
    w.total = off;
    return w;
}

template <int HD>
int launch_prefill(const PrefillArgs& a, int grid, hipStream_t s) {
    if (a.split > 1) {
        attn_prefill_kernel<HD, true><<<grid * a.split, NT, 0, s>>>(a);
        const int rows = a.n_tok * a.hpk * a.n_kv;
        attn_prefill_merge_kernel<HD><<<(rows + 3) / 4, 256, 0, s>>>(a);
    } else {
        attn_prefill_kernel<HD, false><<<grid, NT, 0, s>>>(a);
    }
    return dq_launch_status();
}

// Key splits for a grid of `blocks` workgroups over `tiles` key tiles of the
// longest rows: enough workgroups for two per CU, each split keeping at least
// 4 tiles (128 keys); at most 16.
int prefill_split(int blocks, int tiles, int cus) {
    int sp = 1;
    while (sp < 16 && blocks * sp < 2 * cus && tiles / (2 * sp) >= 4) sp *= 2;
    return sp;
}

int prefill_cus() {
    static int c = 0;
    if (!c) {
        int dev = 0, n = 0;
        c = (hipGetDevice(&dev) == hipSuccess &&
             hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
                ? n
                : 256;
    }
    return c;
}

// ------------------------------------------------------------ side streams --
// Products of one input that leave most of the GPU idle on their own (the K
// and V projections beside Q: 64 workgroups each at a 512-token chunk) run
// side by side: the first on the caller's stream, the others on side streams
// forked from it by an event and joined back before the next kernel, each
// planned for its share of the CUs. The side streams (default priority) and
// events are created once per device outside graph capture; a call under
// capture before they exist runs the products one after another. Under
// capture the fork and join become graph edges.
constexpr int SIDE_N = 3;
struct SideStreams {
    hipStream_t st[SIDE_N] = {};
    hipEvent_t fork = nullptr, join[SIDE_N] = {};
    bool ok = false;
};
constexpr int SIDE_DEVICES = 64;
SideStreams g_side[SIDE_DEVICES];
std::mutex g_side_mu;

SideStreams* side_streams(hipStream_t s) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= SIDE_DEVICES) return nullptr;
    std::lock_guard<std::mutex> lk(g_side_mu);
    SideStreams& g = g_side[dev];
    if (g.ok) return &g;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return nullptr;
    bool good = hipEventCreateWithFlags(&g.fork, hipEventDisableTiming) == hipSuccess;
    for (int i = 0; i < SIDE_N && good; ++i)
        good = hipStreamCreateWithFlags(&g.st[i], hipStreamNonBlocking) == hipSuccess &&
               hipEventCreateWithFlags(&g.join[i], hipEventDisableTiming) == hipSuccess;
    if (!good) {
        (void)hipGetLastError();
        for (int i = 0; i < SIDE_N; ++i) {
            if (g.st[i]) (void)hipStreamDestroy(g.st[i]);
            if (g.join[i]) (void)hipEventDestroy(g.join[i]);
            g.st[i] = nullptr;
            g.join[i] = nullptr;
        }
        if (g.fork) (void)hipEventDestroy(g.fork);
        g.fork = nullptr;
        return nullptr;
    }
    g.ok = true;
    return &g;
}

}  // namespace

extern "C" {

int dq_kv_write_batch(const float* d_k, const float* d_v, size_t ld, uint32_t n_tok, uint32_t n_head_kv, uint32_t hd,
                      void* d_kc, void* d_vc, uint32_t pos0, uint32_t n_ctx, void* stream) {
    if (!d_k || !d_v || !d_kc || !d_vc) return DQ_ERR_INVALID_ARG;
    if (hd == 0 || hd % 32 || n_head_kv == 0) return DQ_ERR_NOT_SUPPORTED;
    if (ld < (size_t)n_head_kv * hd || ld % 4) return DQ_ERR_INVALID_ARG;
    if (n_tok == 0) return DQ_OK;
    if ((uint64_t)pos0 + n_tok > n_ctx) return DQ_ERR_INVALID_ARG;
    const int bpr = (int)(n_head_kv * hd / 32);
    const uint64_t total = (uint64_t)n_tok * 2 * bpr;
    if (total > (1ull << 31)) return DQ_ERR_NOT_SUPPORTED;
    const size_t pos_bytes = (size_t)bpr * DQ_SZ_Q8_0;
    kv_write_batch_kernel<<<(unsigned)((total + 255) / 256), 256, 0, (hipStream_t)stream>>>(
        d_k, d_v, ld, (int)n_tok, bpr, (uint8_t*)d_kc, (uint8_t*)d_vc, pos_bytes, (int)pos0);
    return dq_launch_status();
}

int dq_rope_kv_write_batch(float* d_q, const float* d_k, const float* d_v, size_t q_ld, size_t kv_ld,
                           const float* d_rope, uint32_t n_rot, uint32_t n_tok, uint32_t n_head, uint32_t n_head_kv,
                           uint32_t hd, void* d_kc, void* d_vc, uint32_t pos0, uint32_t n_ctx, void* stream) {
    return dq_rope_kv_write_batch_post(d_q, d_k, d_v, q_ld, kv_ld, d_rope, n_rot, n_tok, n_head, n_head_kv, hd, d_kc,
                                       d_vc, pos0, n_ctx, DqQkvPost{}, stream);
}

}  // extern "C"

int dq_rope_kv_write_batch_post(float* d_q, const float* d_k, const float* d_v, size_t q_ld, size_t kv_ld,
                                const float* d_rope, uint32_t n_rot, uint32_t n_tok, uint32_t n_head,
                                uint32_t n_head_kv, uint32_t hd, void* d_kc, void* d_vc, uint32_t pos0,
                                uint32_t n_ctx, const DqQkvPost& post, void* stream) {
    if (!d_q || !d_k || !d_v || !d_kc || !d_vc) return DQ_ERR_INVALID_ARG;
    if (!dq_head_dim_supported(hd) || n_head_kv == 0) return DQ_ERR_NOT_SUPPORTED;
    if (d_rope && (n_rot == 0 || n_rot > hd || n_rot % 2)) return DQ_ERR_INVALID_ARG;
    if (q_ld < (size_t)n_head * hd || kv_ld < (size_t)n_head_kv * hd) return DQ_ERR_INVALID_ARG;
    if (n_tok == 0) return DQ_OK;
    if ((uint64_t)pos0 + n_tok > n_ctx || n_tok > 65535) return DQ_ERR_INVALID_ARG;
    const size_t pos_bytes = (size_t)n_head_kv * (hd / 32) * DQ_SZ_Q8_0;
    auto go = [&](auto kern) {
        kern<<<dim3(n_head + 2 * n_head_kv, n_tok), 64, 0, (hipStream_t)stream>>>(
            d_q, d_k, d_v, q_ld, kv_ld, d_rope, (int)n_rot, (int)n_head, (int)n_head_kv, (uint8_t*)d_kc,
            (uint8_t*)d_vc, pos_bytes, (int)pos0, post);
    };
    if (hd == 64)
        go(rope_kv_batch_kernel<64>);
    else if (hd == 128)
        go(rope_kv_batch_kernel<128>);
    else
        go(rope_kv_batch_kernel<256>);
    return dq_launch_status();
}

extern "C" {

// Key splits the grid of (n_tok, n_head, n_head_kv) could use at most, and
// the bytes of their partial records.
static int prefill_split_max(uint32_t n_tok, uint32_t n_head, uint32_t n_head_kv) {
    const uint64_t n_qblk = ((uint64_t)n_tok * (n_head / n_head_kv) + RPB - 1) / RPB;
    return prefill_split((int)(n_qblk * n_head_kv), 1 << 30, prefill_cus());
}

static size_t prefill_part_bytes(uint32_t n_tok, uint32_t n_head, uint32_t hd, int split) {
    return split > 1 ? dq_align256((size_t)n_tok * n_head * split * (hd + 4) * 4) : 0;
}

int dq_attn_prefill_workspace_bytes(uint32_t n_tok, uint32_t n_head, uint32_t n_head_kv, uint32_t hd,
                                    size_t* bytes) {
    if (!bytes) return DQ_ERR_INVALID_ARG;
    if (n_head_kv == 0 || n_head % n_head_kv) return DQ_ERR_NOT_SUPPORTED;
    if (hd != 64 && hd != 128 && hd != 256) return DQ_ERR_NOT_SUPPORTED;
    *bytes = prefill_part_bytes(n_tok, n_head, hd, prefill_split_max(n_tok, n_head, n_head_kv));
    return DQ_OK;
}

int dq_attn_prefill_q8(const float* d_q, const void* d_kc, const void* d_vc, uint32_t n_tok, uint32_t n_head,
                       uint32_t n_head_kv, uint32_t hd, uint32_t q_dim, uint32_t pos0, uint32_t n_swa,
                       uint32_t n_ctx, float* d_out, void* d_work, size_t work_bytes, void* stream) {
    if (!d_q || !d_kc || !d_vc || !d_out) return DQ_ERR_INVALID_ARG;
    if (n_head_kv == 0 || n_head % n_head_kv) return DQ_ERR_NOT_SUPPORTED;
    if (hd != 64 && hd != 128 && hd != 256) return DQ_ERR_NOT_SUPPORTED;
    if (q_dim < n_head * hd || q_dim % 4) return DQ_ERR_INVALID_ARG;
    if (((uintptr_t)d_kc | (uintptr_t)d_vc) & 3) return DQ_ERR_NOT_SUPPORTED;
    if (n_tok == 0) return DQ_OK;
    if ((uint64_t)pos0 + n_tok > n_ctx) return DQ_ERR_INVALID_ARG;
    const uint32_t hpk = n_head / n_head_kv;
    const uint64_t n_rows = (uint64_t)n_tok * hpk;
    const uint64_t n_qblk = (n_rows + RPB - 1) / RPB;
    if (n_qblk * n_head_kv * 16 > 0x7FFFFFFFull || n_rows > 0x7FFFFFFFull) return DQ_ERR_NOT_SUPPORTED;
    PrefillArgs a;
    a.q = d_q;
    a.out = d_out;
    a.kc = (const uint8_t*)d_kc;
    a.vc = (const uint8_t*)d_vc;
    a.pos_bytes = (size_t)n_head_kv * (hd / 32) * DQ_SZ_Q8_0;
    a.q_dim = (int)q_dim;
    a.n_tok = (int)n_tok;
    a.hpk = (int)hpk;
    a.n_kv = (int)n_head_kv;
    a.pos0 = (int)pos0;
    a.n_swa = (int)n_swa;
    a.n_qblk = (int)n_qblk;
    a.qscale = (1.0f / sqrtf((float)hd)) * 1.4426950408889634f;
    const int grid = (int)(n_qblk * n_head_kv);
    // key tiles of the longest rows (the last row block): the split is sized
    // so that a grid too small for the GPU spreads their keys over more
    // workgroups; it needs room for the partial records
    const uint32_t p_last = pos0 + n_tok - 1;
    const uint32_t p_first = pos0 + (uint32_t)(((n_qblk - 1) * RPB) / hpk);
    const uint32_t kb = (n_swa > 0 && p_first + 1 > n_swa) ? p_first + 1 - n_swa : 0;
    int split = prefill_split(grid, (int)((p_last - (kb & ~(uint32_t)(KT - 1))) / KT + 1), prefill_cus());
    while (split > 1 && (!d_work || work_bytes < prefill_part_bytes(n_tok, n_head, hd, split))) split /= 2;
    a.split = split;
    a.part = (float*)d_work;
    const hipStream_t s = (hipStream_t)stream;
    switch (hd) {
    case 64: return launch_prefill<64>(a, grid, s);
    case 128: return launch_prefill<128>(a, grid, s);
    default: return launch_prefill<256>(a, grid, s);
    }
}

int dq_rms_norm_rows(const float* d_a, const float* d_b, float* d_h, const float* d_w, size_t n, size_t rows,
                     float eps, float* d_y, void* stream) {
    if (!d_a || !d_w || !d_y) return DQ_ERR_INVALID_ARG;
    if (n == 0 || n % 4 || n > (1u << 30) || rows > 0x7FFFFFFF) return DQ_ERR_NOT_SUPPORTED;
    if (rows == 0) return DQ_OK;
    rms_norm_rows_kernel<<<(unsigned)rows, 256, 0, (hipStream_t)stream>>>(d_a, d_b, d_h, d_w, (int)n, eps, d_y);
    return dq_launch_status();
}

int dq_layer_prefill_workspace_bytes(const dq_layer_t* L, uint32_t n_tok, size_t* bytes) {
    if (!L || !bytes) return DQ_ERR_INVALID_ARG;
    if (!prefill_layer_ok(L)) return DQ_ERR_NOT_SUPPORTED;
    (void)side_streams(nullptr);  // set up here, outside any graph capture, when possible
    *bytes = prefill_carve(L, n_tok, nullptr).total;
    return DQ_OK;
}

#define DQP_TRY(x)                     \
    do {                               \
        const int rc_ = (x);           \
        if (rc_ != DQ_OK) return rc_;  \
    } while (0)

int dq_layer_prefill(const dq_layer_t* L, const float* d_x, float* d_x_out, const float* d_rope, uint32_t pos0,
                     uint32_t n_tok, uint32_t n_swa, void* d_kc, void* d_vc, uint32_t n_ctx, void* d_work,
                     size_t work_bytes, void* stream) {
    if (!L || !d_x || !d_x_out || !d_kc || !d_vc) return DQ_ERR_INVALID_ARG;
    if (!prefill_layer_ok(L)) return DQ_ERR_NOT_SUPPORTED;
    if (n_tok == 0) return DQ_OK;
    if ((uint64_t)pos0 + n_tok > n_ctx || n_tok > 65535) return DQ_ERR_INVALID_ARG;
    const PrefillWs w = prefill_carve(L, n_tok, (uint8_t*)d_work);
    if (!d_work || work_bytes < w.total) return DQ_ERR_INVALID_ARG;
    const hipStream_t s = (hipStream_t)stream;
    const size_t E = L->n_embd, QD = (size_t)L->n_head * L->head_dim, KVD = (size_t)L->n_head_kv * L->head_dim;
    const size_t F = L->n_ff, T = n_tok;
    // the activation layout a format's GEMM reads: Q4_K and Q6_K their own,
    // Q8_0 and Q4_0 the same natural order
    auto cls = [](int fmt) { return fmt == DQ_FMT_Q4_K ? 0 : (fmt == DQ_FMT_Q6_K ? 1 : 2); };
    auto gw = [&](int fmt) { return w.gw[cls(fmt)]; };
    // products of one input x [T][cols] with up to four matrices: one
    // activation quantization per distinct format class (with glu_gate, of
    // the gated FFN product act(glu_gate) * x). When the smallest product
    // would leave more than half the CUs idle on its own, they run side by
    // side (side_streams), each planned for its share of the CUs still free,
    // largest first: product 0 and its class's quantizer on the caller's
    // stream, then a fork; the other products of that class on side streams
    // of their own, another class's quantizer and products together on one
    // side stream.
    const float* glu_gate = nullptr;
    int glu_act = DQ_ACT_SILU;
    // with norm_w, x is first produced by the RMSNorm of norm_a (+ norm_b,
    // kept in norm_h) fused with the quantization (dq_norm_quant_f16)
    const float *norm_a = nullptr, *norm_b = nullptr, *norm_w = nullptr;
    float* norm_h = nullptr;
    auto products = [&](const float* x, size_t cols, int n, const int* fmt, const void* const* wm, const size_t* rows,
                        float* const* y, const void* const* tm) -> int {
        const int C = dq_gemm_cus();
        int budget[4] = {0, 0, 0, 0};
        SideStreams* ss = nullptr;
        if (n > 1) {
            size_t smallest = ~(size_t)0;
            for (int j = 0; j < n; ++j) {
                const size_t wg = dq_gemm_workgroups(fmt[j], rows[j], cols, T);
                if (wg < smallest) smallest = wg;
            }
            if (2 * smallest < (size_t)C) ss = side_streams(s);
        }
        if (ss) {
            int order[4] = {0, 1, 2, 3};
            for (int a = 1; a < n; ++a)  // by rows, largest first (stable)
                for (int b = a; b > 0 && rows[order[b]] > rows[order[b - 1]]; --b) {
                    const int t = order[b];
                    order[b] = order[b - 1];
                    order[b - 1] = t;
                }
            long rem_c = C;
            size_t rem_w = 0;
            for (int j = 0; j < n; ++j) rem_w += rows[j];
            for (int a = 0; a < n; ++a) {
                const int j = order[a];
                const long share = (long)((double)rem_c * (double)rows[j] / (double)rem_w);
                const int b = (int)(share > 8 ? share : 8);
                budget[j] = b;
                const long wg = (long)dq_gemm_workgroups(fmt[j], rows[j], cols, T, b);
                const long left = rem_c - (wg < b ? wg : b);
                rem_c = left > 8 ? left : 8;
                rem_w -= rows[j];
            }
        }
        // the stream of each product: -1 the caller's, else a side stream
        int lane[4] = {-1, -1, -1, -1}, n_side = 0, class_side[3] = {-1, -1, -1};
        const int c0 = cls(fmt[0]);
        if (ss) {
            for (int j = 1; j < n; ++j) {
                const int c = cls(fmt[j]);
                if (c == c0) {
                    if (n_side < SIDE_N) lane[j] = n_side++;
                } else if (class_side[c] >= 0) {
                    lane[j] = class_side[c];
                } else if (n_side < SIDE_N) {
                    lane[j] = class_side[c] = n_side++;
                }
            }
        }
        // a class's quantizer runs on the stream of its first product and
        // clears the outputs its K-split products add their partials into
        bool done[3] = {false, false, false}, zeroed[4] = {false, false, false, false};
        auto spans = [&](int j, unsigned classes) {
            DqZeroSpans z{};
            int k = 0;
            for (int i = j; i < n; ++i) {
                if (k == DqZeroSpans::N || !((classes >> cls(fmt[i])) & 1u) ||
                    !dq_gemm_adds_into_y(fmt[i], rows[i], cols, T, budget[i]) || !dq_zero_span_ok(y[i], rows[i] * T))
                    continue;
                z.p[k] = y[i];
                z.n[k++] = rows[i] * T;
                zeroed[i] = true;
            }
            return z;
        };
        auto quantize = [&](int j, hipStream_t qs) -> int {
            const int fi = cls(fmt[j]);
            const DqZeroSpans z = spans(j, 1u << fi);
            done[fi] = true;
            return dq_quantize_act_f16_zero(fmt[j], x, cols, T, gw(fmt[j]), z, qs, glu_gate, glu_act);
        };
        if (norm_w) {
            // the norm that produces x, fused with the quantization for
            // product 0's class and the first other class (x itself is
            // written only for a third class)
            int nf = 1, fq[2] = {fmt[0], 0};
            for (int j = 1; j < n && nf < 2; ++j)
                if (cls(fmt[j]) != cls(fmt[0])) fq[nf++] = fmt[j];
            void* outs[2] = {gw(fq[0]), nf > 1 ? gw(fq[1]) : nullptr};
            const unsigned classes = (1u << cls(fq[0])) | (nf > 1 ? 1u << cls(fq[1]) : 0u);
            bool third = false;
            for (int j = 0; j < n; ++j) third |= !((classes >> cls(fmt[j])) & 1u);
            const DqZeroSpans z = spans(0, classes);
            DQP_TRY(dq_norm_quant_f16(norm_a, norm_b, norm_h, norm_w, cols, T, L->rms_eps,
                                      third ? const_cast<float*>(x) : nullptr, nf, fq, outs, z, s));
            for (int k = 0; k < nf; ++k) done[cls(fq[k])] = true;
        } else {
            DQP_TRY(quantize(0, s));
        }
        // one fork after product 0's quantizer (a fork before it, letting
        // another class's quantizer run beside it, measured slower: the
        // replayed graph then ran that quantizer after product 0)
        if (n_side > 0) {
            if (hipEventRecord(ss->fork, s) != hipSuccess) return DQ_ERR_IO;
            for (int i = 0; i < n_side; ++i)
                if (hipStreamWaitEvent(ss->st[i], ss->fork, 0) != hipSuccess) return DQ_ERR_IO;
        }
        for (int j = 0; j < n; ++j) {
            const hipStream_t js = lane[j] < 0 ? s : ss->st[lane[j]];
            if (!done[cls(fmt[j])]) DQP_TRY(quantize(j, js));
            // the matrix's tile copy where the layer has one (same results)
            DQP_TRY(dq_gemm_f16act_zeroed(tm[j] ? (fmt[j] | DQ_FMT_GEMM_TILES) : fmt[j], tm[j] ? tm[j] : wm[j],
                                          rows[j], cols, gw(fmt[j]), T, y[j], zeroed[j], js, budget[j]));
        }
        for (int i = 0; i < n_side; ++i) {
            if (hipEventRecord(ss->join[i], ss->st[i]) != hipSuccess) return DQ_ERR_IO;
            if (hipStreamWaitEvent(s, ss->join[i], 0) != hipSuccess) return DQ_ERR_IO;
        }
        return DQ_OK;
    };
    // attention block (models/dense_forward.cpp:3264-3290, 3300-3362, 3430-3460)
    norm_a = d_x;
    norm_w = L->attn_norm;
    {
        // with the attention gate's matrix, which reads the same normalised
        // input (:3525-3526)
        const int f[4] = {L->fmt_q, L->fmt_k, L->fmt_v, L->fmt_ag};
        const void* m[4] = {L->wq, L->wk, L->wv, L->wag};
        const size_t r[4] = {QD, KVD, KVD, L->n_head};
        float* const y[4] = {w.q, w.k, w.v, w.ag};
        const void* t[4] = {L->tq, L->tk, L->tv, L->tag};
        DQP_TRY(products(w.xn, E, L->wag ? 4 : 3, f, m, r, y, t));
    }
    norm_w = nullptr;
    DQP_TRY(dq_rope_kv_write_batch_post(w.q, w.k, w.v, QD, KVD, d_rope, L->n_rot, n_tok, L->n_head, L->n_head_kv,
                                        L->head_dim, d_kc, d_vc, pos0, n_ctx, dq_layer_post(L), stream));
    DQP_TRY(dq_attn_prefill_q8(w.q, d_kc, d_vc, n_tok, L->n_head, L->n_head_kv, L->head_dim, (uint32_t)QD, pos0,
                               n_swa, n_ctx, w.attn, w.aw, w.aw_bytes, stream));
    if (L->wag) {  // the per-head output gate before the output projection
        attn_gate_rows_kernel<<<n_tok * L->n_head, 64, 0, s>>>(w.attn, w.ag, (int)L->n_head, (int)L->head_dim, QD);
        DQP_TRY(dq_launch_status());
    }
    {
        const int f[1] = {L->fmt_o};
        const void* m[1] = {L->wo};
        const size_t r[1] = {E};
        float* const y[1] = {w.down};
        const void* t[1] = {L->to};
        DQP_TRY(products(w.attn, QD, 1, f, m, r, y, t));
    }
    // residual + FFN norm (:3539-3560), gated FFN (:3600-3624)
    if (L->post_attn_norm) {  // sandwich norm of the projection before the residual
        DQP_TRY(dq_post_norm_add(w.down, L->post_attn_norm, d_x, w.h, E, n_tok, L->rms_eps, stream));
        norm_a = w.h;
    } else {  // the residual, kept in h, and the FFN norm of it
        norm_a = w.down;
        norm_b = d_x;
        norm_h = w.h;
    }
    norm_w = L->ffn_norm;
    {
        const int f[2] = {L->fmt_up, L->fmt_gate};
        const void* m[2] = {L->wup, L->wgate};
        const size_t r[2] = {F, F};
        float* const y[2] = {w.up, w.gate};
        const void* t[2] = {L->tup, L->tgate};
        DQP_TRY(products(w.xn, E, 2, f, m, r, y, t));
    }
    norm_w = nullptr;
    // the batch branch's activation, silu or gelu_tanh per element
    // (:3608-3609), formed by the down projection's quantizer as it reads
    // gate and up
    glu_gate = w.gate;
    glu_act = L->act_gelu ? DQ_ACT_GELU_TANH : DQ_ACT_SILU;
    {
        const int f[1] = {L->fmt_down};
        const void* m[1] = {L->wdown};
        const size_t r[1] = {E};
        float* const y[1] = {w.down};
        const void* t[1] = {L->tdown};
        DQP_TRY(products(w.up, F, 1, f, m, r, y, t));
    }
    const size_t ne4 = T * E / 4;
    if (L->post_ffn_norm)  // sandwich norm of the FFN output before the residual
        return dq_post_norm_add(w.down, L->post_ffn_norm, w.h, d_x_out, E, n_tok, L->rms_eps, stream);
    add_kernel<<<(unsigned)((ne4 + 255) / 256), 256, 0, s>>>(w.down, w.h, ne4, d_x_out);
    return dq_launch_status();
}

}  // extern "C"

int dq_post_norm_add(const float* d_a, const float* d_w, const float* d_b, float* d_out, size_t n, uint32_t rows,
                     float eps, void* stream) {
    if (!d_a || !d_w || !d_b || !d_out || n == 0 || n % 4) return DQ_ERR_INVALID_ARG;
    if (rows == 0) return DQ_OK;
    if (n > (1u << 26)) return DQ_ERR_NOT_SUPPORTED;
    post_norm_add_kernel<<<rows, 256, 0, (hipStream_t)stream>>>(d_a, d_w, d_b, (int)n, eps, d_out);
    return dq_launch_status();
}
