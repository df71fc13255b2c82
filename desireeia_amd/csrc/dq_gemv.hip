// dq_gemv.hip - batch-1 decode GEMV for Q8_0, Q4_0, Q4_K and Q6_K weights.
//
// HBM-bound design (gfx950, wave64):
//  * A row is cut into items of 64 weights (cols/64 per row); lane l of a wave
//    owns items l, l+64, ... of every row it visits. Items sit contiguously in
//    item-major planes (dq_common.h), so a wave's loads cover whole cache lines.
//  * The activation bytes of a lane's items (x int8, scale, sums) are loaded
//    into registers once per wave and reused for every row the wave visits;
//    only weights stream from HBM.
//  * Flat grid (the default where it fits): one wave, or one workgroup for a
//    K-split row, per group of R rows, sized so every wave of the launch is
//    resident at once (about 16 per CU). The activation registers are loaded
//    first, then every weight load of the group, so the whole matrix's loads
//    are in flight from the start and each row's arithmetic runs as soon as
//    its own weights land (rows are kept in order by scheduling barriers).
//  * Persistent grid (larger shapes): waves walk row groups with a two-deep
//    software pipeline, the loads of group k+1 issued before group k is
//    computed; past the last group the prefetch reads a cached dummy address
//    (no extra HBM traffic, static vmcnt accounting).
//  * Nibble/6-bit unpack and 6-bit scale decode in registers (one decode per
//    64 weights), v_dot4_i32_i8 dots, and row sums over the wave by DPP row
//    reductions and readlanes (no LDS round trips on the critical path).
//
// Semantics follow the reference CPU GEMVs (include/desireeia_hip.h): integer
// partial sums are exact; only the float summation order differs.
#include <cstdlib>
#include <type_traits>

#include "dq_common.h"
#include "dq_quant.h"

namespace {

__device__ __forceinline__ int dot16(const dq_u32x4& w, const dq_u32x4& x, int acc) {
    acc = dq_sdot4((int)w.x, (int)x.x, acc);
    acc = dq_sdot4((int)w.y, (int)x.y, acc);
    acc = dq_sdot4((int)w.z, (int)x.z, acc);
    acc = dq_sdot4((int)w.w, (int)x.w, acc);
    return acc;
}

__device__ __forceinline__ dq_u32x4 nib_lo(const dq_u32x4& v) { return v & 0x0F0F0F0Fu; }
__device__ __forceinline__ dq_u32x4 nib_hi(const dq_u32x4& v) { return (v >> 4) & 0x0F0F0F0Fu; }

__device__ __forceinline__ uint32_t ld_u32_nt(const uint8_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
}
__device__ __forceinline__ uint16_t ld_u16_nt(const uint8_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const uint16_t*>(p));
}

// ---------------------------------------------------------------- formats --
// X: activation registers of an item; W: its weight registers; load_w reads
// the item's 16-byte pieces from the quant sub-planes (ps apart) and its scales.

struct XItem {
    dq_u32x4 x[4];  // the 64 activation bytes the item multiplies
    float s0, s1;   // activation scales
    int i0, i1;     // activation integer sums
};

template <int FMT>
struct Fmt;

// Q8_0: item i = blocks 2i, 2i+1: 64 int8 (plane Q) + 2 fp16 scales (plane D).
template <>
struct Fmt<DQ_FMT_Q8_0> {
    struct W {
        dq_u32x4 q[4];
        uint32_t d;
    };
    __device__ static void load_x(XItem& X, int i, const int8_t* xq, const float* xs, const int32_t*) {
        const dq_u32x4* p = reinterpret_cast<const dq_u32x4*>(xq + 64 * (size_t)i);
        X.x[0] = p[0]; X.x[1] = p[1]; X.x[2] = p[2]; X.x[3] = p[3];
        X.s0 = xs[2 * i];
        X.s1 = xs[2 * i + 1];
    }
    __device__ static void load_w(W& w, const uint8_t* q, size_t ps, const uint8_t* d) {
        w.q[0] = dq_ld16_stream(q);
        w.q[1] = dq_ld16_stream(q + ps);
        w.q[2] = dq_ld16_stream(q + 2 * ps);
        w.q[3] = dq_ld16_stream(q + 3 * ps);
        w.d = ld_u32_nt(d);
    }
    __device__ static const uint8_t* aux(const uint8_t* base, const DqLayout& L, size_t r, int i) {
        return base + L.d_off + r * L.d_row + 4 * (size_t)i;
    }
    __device__ static float dot(const W& w, const XItem& X, int) {
        const int a = dot16(w.q[1], X.x[1], dot16(w.q[0], X.x[0], 0));
        const int b = dot16(w.q[3], X.x[3], dot16(w.q[2], X.x[2], 0));
        const float d0 = dq_h2f((uint16_t)(w.d & 0xFFFF)), d1 = dq_h2f((uint16_t)(w.d >> 16));
        return d0 * X.s0 * (float)a + d1 * X.s1 * (float)b;
    }
};

// Q4_0: item i = blocks 2i, 2i+1: 2 x 16 nibble bytes + 2 fp16 scales.
// sum (nib-8)*x = sum nib*x - 8*sum x.
template <>
struct Fmt<DQ_FMT_Q4_0> {
    struct W {
        dq_u32x4 q[2];
        uint32_t d;
    };
    __device__ static void load_x(XItem& X, int i, const int8_t* xq, const float* xs, const int32_t* xsum) {
        const dq_u32x4* p = reinterpret_cast<const dq_u32x4*>(xq + 64 * (size_t)i);
        X.x[0] = p[0]; X.x[1] = p[1]; X.x[2] = p[2]; X.x[3] = p[3];
        X.s0 = xs[2 * i];
        X.s1 = xs[2 * i + 1];
        X.i0 = xsum[2 * i];
        X.i1 = xsum[2 * i + 1];
    }
    __device__ static void load_w(W& w, const uint8_t* q, size_t ps, const uint8_t* d) {
        w.q[0] = dq_ld16_stream(q);
        w.q[1] = dq_ld16_stream(q + ps);
        w.d = ld_u32_nt(d);
    }
    __device__ static const uint8_t* aux(const uint8_t* base, const DqLayout& L, size_t r, int i) {
        return base + L.d_off + r * L.d_row + 4 * (size_t)i;
    }
    __device__ static float dot(const W& w, const XItem& X, int) {
        const int a = dot16(nib_hi(w.q[0]), X.x[1], dot16(nib_lo(w.q[0]), X.x[0], 0)) - 8 * X.i0;
        const int b = dot16(nib_hi(w.q[1]), X.x[3], dot16(nib_lo(w.q[1]), X.x[2], 0)) - 8 * X.i1;
        const float d0 = dq_h2f((uint16_t)(w.d & 0xFFFF)), d1 = dq_h2f((uint16_t)(w.d >> 16));
        return d0 * X.s0 * (float)a + d1 * X.s1 * (float)b;
    }
};

// Q4_K: item i = (s = i/4, g = i%4): qs bytes 32g..32g+31 of block s = sub-blocks
// 2g (low nibbles) and 2g+1 (high nibbles); header (d, dmin, 12 scale bytes)
// of block s from plane H.
template <>
struct Fmt<DQ_FMT_Q4_K> {
    struct W {
        dq_u32x4 qa, qb, h;
    };
    __device__ static void load_x(XItem& X, int i, const int8_t* xq, const float* xs, const int32_t* xsum) {
        const dq_u32x4* p = reinterpret_cast<const dq_u32x4*>(xq + 64 * (size_t)i);
        X.x[0] = p[0]; X.x[1] = p[1]; X.x[2] = p[2]; X.x[3] = p[3];
        X.s0 = xs[2 * i];  // the per-256 scale, replicated in every per-32 slot
        X.i0 = xsum[2 * i];
        X.i1 = xsum[2 * i + 1];
    }
    __device__ static void load_w(W& w, const uint8_t* q, size_t ps, const uint8_t* h) {
        w.qa = dq_ld16_stream(q);
        w.qb = dq_ld16_stream(q + ps);
        w.h = dq_ld16_stream(h);
    }
    __device__ static const uint8_t* aux(const uint8_t* base, const DqLayout& L, size_t r, int i) {
        return base + L.s_off + r * L.s_row + 16 * (size_t)(i >> 2);
    }
    __device__ static float dot(const W& w, const XItem& X, int i) {
        const int da = dot16(nib_lo(w.qb), X.x[1], dot16(nib_lo(w.qa), X.x[0], 0));
        const int db = dot16(nib_hi(w.qb), X.x[3], dot16(nib_hi(w.qa), X.x[2], 0));
        // 6-bit scale/min of sub-blocks j = 2g, 2g+1 (quant/quant.cpp:22-29);
        // scale bytes q[0..11] are header words h.y, h.z, h.w. Branch-free
        // (g differs between lanes): bytes 2(g&1), 2(g&1)+1 of each word, then
        //   j < 4:  sc = q[j] & 63,                     m = q[j+4] & 63
        //   j >= 4: sc = (q[j+4]&15) | ((q[j-4]>>6)<<4), m = (q[j+4]>>4) | ((q[j]>>6)<<4)
        const int g = i & 3;
        const int sh = 16 * (g & 1);
        const bool hi = g >= 2;
        const uint32_t b0a = (w.h.y >> sh) & 0xFF, b0b = (w.h.y >> (sh + 8)) & 0xFF;
        const uint32_t b1a = (w.h.z >> sh) & 0xFF, b1b = (w.h.z >> (sh + 8)) & 0xFF;
        const uint32_t b2a = (w.h.w >> sh) & 0xFF, b2b = (w.h.w >> (sh + 8)) & 0xFF;
        const int sca = (int)(hi ? ((b2a & 15) | ((b0a >> 6) << 4)) : (b0a & 63));
        const int scb = (int)(hi ? ((b2b & 15) | ((b0b >> 6) << 4)) : (b0b & 63));
        const int mna = (int)(hi ? ((b2a >> 4) | ((b1a >> 6) << 4)) : (b1a & 63));
        const int mnb = (int)(hi ? ((b2b >> 4) | ((b1b >> 6) << 4)) : (b1b & 63));
        const float d = dq_h2f((uint16_t)(w.h.x & 0xFFFF));
        const float dmin = dq_h2f((uint16_t)(w.h.x >> 16));
        const int isum = sca * da + scb * db;
        const int msum = mna * X.i0 + mnb * X.i1;
        return X.s0 * (d * (float)isum - dmin * (float)msum);
    }
};

// Q6_K: item i = (s = i/4, it = i%4 = 2n+k): 16 bytes of each of QA, QB, QH,
// 4 scales (plane S) and d (plane D); its 64 weights sit at positions
// 256s + 128n + 16k + 32*quarter + 0..15.
template <>
struct Fmt<DQ_FMT_Q6_K> {
    struct W {
        dq_u32x4 a, b, h;
        uint32_t sc;
        uint16_t d;
    };
    __device__ static void load_x(XItem& X, int i, const int8_t* xq, const float* xs, const int32_t*) {
        const int8_t* base = xq + 256 * (size_t)(i >> 2) + 128 * ((i >> 1) & 1) + 16 * (i & 1);
        X.x[0] = dq_ld16(base);
        X.x[1] = dq_ld16(base + 32);
        X.x[2] = dq_ld16(base + 64);
        X.x[3] = dq_ld16(base + 96);
        X.s0 = xs[8 * (i >> 2)];
    }
    __device__ static void load_w6(W& w, const uint8_t* q, size_t ps, const uint8_t* s, const uint8_t* d) {
        w.a = dq_ld16_stream(q);
        w.b = dq_ld16_stream(q + ps);
        w.h = dq_ld16_stream(q + 2 * ps);
        w.sc = ld_u32_nt(s);
        w.d = ld_u16_nt(d);
    }
    __device__ static int q6dot(uint32_t lo4, uint32_t hi2, uint32_t x, int acc) {
        return dq_sdot4(dq_sub32_bytes((lo4 & 0x0F0F0F0Fu) | ((hi2 & 0x03030303u) << 4)), (int)x, acc);
    }
    __device__ static float dot(const W& w, const XItem& X, int) {
        int d0 = 0, d1 = 0, d2 = 0, d3 = 0;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t a = w.a[t], b = w.b[t], h = w.h[t];
            d0 = q6dot(a, h, X.x[0][t], d0);
            d1 = q6dot(b, h >> 2, X.x[1][t], d1);
            d2 = q6dot(a >> 4, h >> 4, X.x[2][t], d2);
            d3 = q6dot(b >> 4, h >> 6, X.x[3][t], d3);
        }
        const int s0 = (int8_t)(w.sc & 0xFF), s1 = (int8_t)((w.sc >> 8) & 0xFF);
        const int s2 = (int8_t)((w.sc >> 16) & 0xFF), s3 = (int8_t)(w.sc >> 24);
        const int isum = s0 * d0 + s1 * d1 + s2 * d2 + s3 * d3;
        return dq_h2f(w.d) * X.s0 * (float)isum;
    }
};

// Up to DQ_GEMV_MAX_JOBS matrices that read the same activation (same cols,
// same format) run in one grid: their row groups are concatenated, job j
// owning groups [g0[j], g0[j+1]).
#define DQ_GEMV_MAX_JOBS 4
struct Jobs {
    const uint8_t* w[DQ_GEMV_MAX_JOBS];
    int fmt[DQ_GEMV_MAX_JOBS];  // the mixed-format launch picks each group's format by its job
    DqLayout L[DQ_GEMV_MAX_JOBS];
    float* y[DQ_GEMV_MAX_JOBS];
    const float* res[DQ_GEMV_MAX_JOBS];
    int rows[DQ_GEMV_MAX_JOBS];
    int g0[DQ_GEMV_MAX_JOBS + 1];
    int n;
};

// Job of global group g (g < g0[n]) and the group's index inside it.
__device__ __forceinline__ int job_of(const Jobs& J, int g, int* gl) {
    int j = 0;
#pragma unroll
    for (int k = 1; k < DQ_GEMV_MAX_JOBS; ++k)
        if (k < J.n && g >= J.g0[k]) j = k;
    *gl = g - J.g0[j];
    return j;
}

// Loads the weights of item i of row r (or, when `live` is false, reads a
// cached dummy location instead: the pipeline's prefetch past the last group).
template <int FMT>
__device__ __forceinline__ void load_item(typename Fmt<FMT>::W& w, const uint8_t* base, const DqLayout& L, size_t r,
                                          int i, bool live, const uint8_t* dummy) {
    const uint8_t* q = live ? base + L.q_off + r * L.q_row + 16 * (size_t)i : dummy;
    const size_t ps = live ? L.p_stride : 0;
    if constexpr (FMT == DQ_FMT_Q6_K) {
        const uint8_t* s = live ? base + L.s_off + r * L.s_row + 4 * (size_t)i : dummy;
        const uint8_t* d = live ? base + L.d_off + r * L.d_row + 2 * (size_t)(i >> 2) : dummy;
        Fmt<FMT>::load_w6(w, q, ps, s, d);
    } else {
        Fmt<FMT>::load_w(w, q, ps, live ? Fmt<FMT>::aux(base, L, r, i) : dummy);
    }
}

// Items of a wave: [i0, i1) of every row; lane owns i0 + lane + 64j.
template <int FMT, int R, int NIT>
__device__ __forceinline__ void load_group(typename Fmt<FMT>::W (&wr)[R][NIT], const Jobs& J, int g, int ngroups,
                                           int i0, int i1, int lane, const uint8_t* dummy) {
    const bool live = g < ngroups;
    int gl = 0;
    const int j = live ? job_of(J, g, &gl) : 0;
    const uint8_t* base = J.w[j];
    const int rows = J.rows[j];
#pragma unroll
    for (int rr = 0; rr < R; ++rr) {
        const size_t r = (size_t)min(gl * R + rr, rows - 1);
#pragma unroll
        for (int it = 0; it < NIT; ++it)
            load_item<FMT>(wr[rr][it], base, J.L[j], r, min(i0 + lane + DQ_WAVE * it, i1 - 1), live, dummy);
    }
}

// Row sums of group g. KS == 1: the wave owns whole rows and stores them.
// KS == 4: the 4 waves of the workgroup own a quarter of the items each; their
// partial sums meet in LDS (double-buffered by `buf`, one barrier per group)
// and wave 0 adds them in a fixed order.
template <int FMT, int R, int NIT, int KS>
__device__ __forceinline__ void compute_group(const typename Fmt<FMT>::W (&wr)[R][NIT], const XItem (&X)[NIT],
                                              const Jobs& J, int g, int i0, int i1, int lane, int ks,
                                              float (*part)[R][4], int buf, bool store = true) {
    float acc[R];
#pragma unroll
    for (int rr = 0; rr < R; ++rr) {
        float a = 0.0f;
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
            const int i = i0 + lane + DQ_WAVE * it;
            const float p = Fmt<FMT>::dot(wr[rr][it], X[it], i);
            a += i < i1 ? p : 0.0f;
        }
        // each row's sum over the wave (DPP row reductions + readlanes,
        // uniform) right after its dot products, so that only the last row's
        // reduction is left once the last weights land
        acc[rr] = dq_wave_sum_uniform(a);
        // row by row: the scheduler would otherwise sink every row's dot
        // products below the wait for the last row's weights
        __builtin_amdgcn_sched_barrier(0);
    }
    const float (&tot)[R] = acc;
    int gl = 0;
    const int j = job_of(J, g, &gl);
    float* __restrict__ y = J.y[j];
    const float* __restrict__ res = J.res[j];
    const int rows = J.rows[j];
    // lane rr stores row rr (vector stores)
    float mine = tot[0];
#pragma unroll
    for (int rr = 1; rr < R; ++rr) mine = lane == rr ? tot[rr] : mine;
    if constexpr (KS == 1) {
        if (store && lane < R) {
            const int r = gl * R + lane;
            if (r < rows) y[r] = res ? mine + res[r] : mine;
        }
    } else {
        if (lane < R) part[buf][lane][ks] = mine;
        __syncthreads();
        if (store && ks == 0 && lane < R) {
            const int r = gl * R + lane;
            if (r < rows) {
                const float v = ((part[buf][lane][0] + part[buf][lane][1]) + part[buf][lane][2]) + part[buf][lane][3];
                y[r] = res ? v + res[r] : v;
            }
        }
    }
}

// ----------------------------------------------------------------- kernel --

// Activation kind of a weight format's reference GEMV.
template <int FMT>
constexpr int act_kind_of() {
    return (FMT == DQ_FMT_Q8_0 || FMT == DQ_FMT_Q4_0) ? DQ_ACT_Q8_0 : DQ_ACT_Q8K_REP;
}

// XQ: the workgroup quantizes the fp32 activation xf itself into LDS (int8
// [cols], scale and int32 sum per 32, with the format's reference quantizer,
// bit-exact as dq_quantize_act) while its first weight loads are in flight.
template <int FMT>
__device__ __forceinline__ void quantize_to_lds(const float* __restrict__ xf, int cols, uint8_t* xl) {
    const int nblk = cols / 32;
    int8_t* lq = reinterpret_cast<int8_t*>(xl);
    float* ls = reinterpret_cast<float*>(xl + cols);
    int32_t* li = reinterpret_cast<int32_t*>(xl + cols + 4 * nblk);
    // per-256 groups of 8 lanes are aligned (nblk % 8 == 0 for the K-quants),
    // so a group is wholly inside or outside [0, nblk)
    for (int b = threadIdx.x; b < nblk; b += blockDim.x) {
        float v[32];
        dq_load32(xf + 32 * (size_t)b, v);
        uint32_t packed[8];
        float d, fs;
        int sum;
        dq_quant_block<act_kind_of<FMT>()>(v, packed, d, sum, fs);
        dq_u32x4* qo = reinterpret_cast<dq_u32x4*>(lq + 32 * b);
        qo[0] = dq_u32x4{packed[0], packed[1], packed[2], packed[3]};
        qo[1] = dq_u32x4{packed[4], packed[5], packed[6], packed[7]};
        ls[b] = d;
        li[b] = sum;
    }
}

// Grid: persistent 256-thread workgroups walking "units" u = blockIdx.x,
// blockIdx.x + gridDim.x, ... KS == 1: unit u = groups 4u..4u+3, one per wave.
// KS == 4: unit u = group u, shared by the 4 waves (K split in quarters).
// Groups are global over the jobs of J.
template <int FMT, int R, int NIT, int KS, bool XQ>
__global__ __launch_bounds__(256) void gemv_kernel(Jobs J, int items, const int8_t* __restrict__ xq,
                                                   const float* __restrict__ xs, const int32_t* __restrict__ xsum,
                                                   const float* __restrict__ xf) {
    using W = typename Fmt<FMT>::W;
    extern __shared__ __align__(16) uint8_t xl[];  // XQ: the quantized activation
    __shared__ float part[2][R][4];
    const int lane = threadIdx.x & (DQ_WAVE - 1);
    const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / DQ_WAVE));  // wave-uniform
    const int ks = KS == 1 ? 0 : wv;
    const int per = KS == 1 ? items : (items + 3) / 4;
    const int i0 = min(ks * per, items);
    const int i1 = min(i0 + per, items);
    const int ngroups = J.g0[J.n];
    const int stride = KS == 1 ? 4 * (int)gridDim.x : (int)gridDim.x;
    int g = KS == 1 ? 4 * (int)blockIdx.x + wv : (int)blockIdx.x;
    const bool active = g < ngroups && i0 < i1;  // uniform per wave (KS 1) / per workgroup (KS 4)
    if (!XQ && !active) return;
    const uint8_t* dummy = reinterpret_cast<const uint8_t*>(XQ ? (const void*)xf : (const void*)xq);

    W b0[R][NIT], b1[R][NIT];
    if (active) load_group<FMT, R, NIT>(b0, J, g, ngroups, i0, i1, lane, dummy);
    if constexpr (XQ) {
        const int cols = items * 64;
        quantize_to_lds<FMT>(xf, cols, xl);
        __syncthreads();
        if (!active) return;
        xq = reinterpret_cast<const int8_t*>(xl);
        xs = reinterpret_cast<const float*>(xl + cols);
        xsum = reinterpret_cast<const int32_t*>(xl + cols + 4 * (cols / 32));
    }
    XItem X[NIT];
#pragma unroll
    for (int j = 0; j < NIT; ++j) Fmt<FMT>::load_x(X[j], min(i0 + lane + DQ_WAVE * j, i1 - 1), xq, xs, xsum);

    // Two-deep pipeline, unrolled by two so the buffers never move.
    for (;;) {
        load_group<FMT, R, NIT>(b1, J, g + stride, ngroups, i0, i1, lane, dummy);
        compute_group<FMT, R, NIT, KS>(b0, X, J, g, i0, i1, lane, ks, part, 0);
        g += stride;
        if (g >= ngroups) break;
        load_group<FMT, R, NIT>(b0, J, g + stride, ngroups, i0, i1, lane, dummy);
        compute_group<FMT, R, NIT, KS>(b1, X, J, g, i0, i1, lane, ks, part, 1);
        g += stride;
        if (g >= ngroups) break;
    }
}

// In-kernel activation quantization of the flat grid, in two phases so that
// it overlaps the weight stream: xstage_load issues the fp32 loads BEFORE the
// weight loads (vector memory returns are counted in issue order, so loads
// issued after the weights could not be used before every weight byte had
// arrived); xstage_quant then quantizes into LDS while the weights are in
// flight. Loads are coalesced: round r of wave w (of nw) covers the 256
// columns c0 + 256*(w + r*nw) + [0, 256), lane l holding the 4 at +4l (one
// contiguous kilobyte per load instruction). A 32-block is 8 lanes, so block
// maxima and integer sums are DPP lane reductions; max and integer sums do
// not depend on order, so the integers and scales are bit-exact with the
// per-block quantizer (dq_quant_block). Columns past c1 load the last four
// (valid address) and are not stored; c0, c1 are multiples of 64 (whole
// 32-blocks of 8 lanes). Per-32 kind only (Q8_0, Q4_0); the per-256 kind
// takes xrow_quant.
template <int ROUNDS>
struct XStage {
    float4 v[ROUNDS];
};

template <int ROUNDS>
__device__ __forceinline__ void xstage_load(XStage<ROUNDS>& st, const float* __restrict__ xf, int c0, int c1, int w,
                                            int nw, int lane) {
#pragma unroll
    for (int r = 0; r < ROUNDS; ++r) {
        const int c = min(c0 + 256 * (w + r * nw) + 4 * lane, c1 - 4);
        st.v[r] = *reinterpret_cast<const float4*>(xf + c);
    }
}

// Maxima of |x| are taken on the bit patterns: non-negative floats order as
// their bits, so an unsigned max equals fmaxf on them (and needs no NaN
// canonicalization between DPP steps).
template <int CTRL>
__device__ __forceinline__ uint32_t umax_dpp(uint32_t v) {
    return max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ uint32_t max8_lanes(uint32_t v) {  // over the 8 lanes of an aligned group
    v = umax_dpp<0xB1>(v);          // quad_perm [1,0,3,2]
    v = umax_dpp<0x4E>(v);          // quad_perm [2,3,0,1]
    return umax_dpp<0x141>(v);      // row_half_mirror: the other quad of the 8
}
__device__ __forceinline__ int sum8_lanes(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);
    return v + __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);
}

// amax / 127 rounded to float, as the IEEE single division: the product in
// double is within 2^-52 (relative) of amax/127, and amax/127 is never within
// 2^-32 of a float rounding midpoint (a midpoint times 127 needs more than 24
// significant bits), so the final rounding is the division's. Checked
// exhaustively against amax / 127.0f over every positive float.
__device__ __forceinline__ float div127(float amax) {
    return (float)((double)amax * (1.0 / 127.0));
}

// Signed byte rint(p) for |p| <= 127.5 (round half to even): p + 1.5*2^23
// rounds p to an integer in the low mantissa bits (the sum's ulp is 1), whose
// low byte is rint(p) in two's complement. Checked exhaustively against
// rintf over every float of magnitude <= 128.
__device__ __forceinline__ uint32_t rint_bits(float p) {
    return __builtin_bit_cast(uint32_t, p + 12582912.0f);
}

// LDS image of columns [c0, c1): int8 q at xl + (c - c0), fp32 scale and
// int32 sum of 32-block k at xl + 32*nblk + 4k and xl + 36*nblk + 4k (nblk =
// the region's block capacity). Quantized values need no clamp: |x*id| <=
// 127 * (1 + 2^-23) by construction of id (1/d here, 127/amax per 256), so
// rint <= 127, except where id overflows to inf (handled on its own).
template <int FMT, int ROUNDS>
__device__ __forceinline__ void xstage_quant(const XStage<ROUNDS>& st, int c0, int c1, int w, int nw, int lane,
                                             int nblk, uint8_t* xl) {
    static_assert(act_kind_of<FMT>() != DQ_ACT_Q8K_REP, "per-256 activations use xrow_quant");
    float* ls = reinterpret_cast<float*>(xl + 32 * (size_t)nblk);
    int32_t* li = reinterpret_cast<int32_t*>(xl + 36 * (size_t)nblk);
    // A round wholly past the end is computed on its clamped loads and stores
    // nothing (c >= c1 in every lane). It is not skipped by a branch: the
    // compiler would sink that round's load into the branch, below the weight
    // loads, and its wait would then be for every weight byte.
#pragma unroll
    for (int r = 0; r < ROUNDS; ++r) {
        const int c = c0 + 256 * (w + r * nw) + 4 * lane;
        const float4 v = st.v[r];
        const float m4 = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
        const uint32_t am = max8_lanes(__builtin_bit_cast(uint32_t, m4));  // the 32-block's maximum
        const float amax = __builtin_bit_cast(float, am);
        const float d = amax > 0.0f ? div127(amax) : 0.0f;
        const float id = d > 0.0f ? 1.0f / d : 0.0f;  // core/quant.cpp:15-50
        // bytes rint(x * id) of the 4 columns, packed little-endian
        const uint32_t t0 = rint_bits(v.x * id), t1 = rint_bits(v.y * id);
        const uint32_t t2 = rint_bits(v.z * id), t3 = rint_bits(v.w * id);
        const uint32_t lo = __builtin_amdgcn_perm(t1, t0, 0x0C0C0400u);  // [t0.b0, t1.b0, 0, 0]
        const uint32_t hi = __builtin_amdgcn_perm(t3, t2, 0x0C0C0400u);  // [t2.b0, t3.b0, 0, 0]
        uint32_t packed = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
        if (__builtin_expect(!(id <= 3.40282347e38f), 0)) {
            // id = inf (d below 1 / FLT_MAX): x * id is +-inf or
            // NaN, converted with saturation and clamped as in dq_quant_block
            const float vv[4] = {v.x, v.y, v.z, v.w};
            packed = 0;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int iv = (int)rintf(vv[k] * id);
                packed |= (uint32_t)((iv > 127 ? 127 : (iv < -127 ? -127 : iv)) & 0xFF) << (8 * k);
            }
        }
        const int isum = sum8_lanes(dq_sdot4((int)packed, 0x01010101, 0));
        if (c < c1) {
            const int o = c - c0;
            *reinterpret_cast<uint32_t*>(xl + o) = packed;
            if ((lane & 7) == 0) {
                ls[o >> 5] = d;
                li[o >> 5] = isum;
            }
        }
    }
}

// Flat grid: one wave (KS == 1) or one workgroup (KS == 4, K split in
// quarters) per group of R rows, and every weight load of the group issued
// before any is used. No loop and no prefetch past the end: the grid holds
// all groups at once (about 16 waves per CU), which keeps the whole matrix's
// loads in flight from the start and ends every wave right after its only
// group. Groups are global over the jobs of J. One item per lane (NIT 1).
// XQ: XR quantization rounds per wave, enough for the activation (the host
// picks the smallest of its instantiations that covers it).
template <int FMT, int R, int KS, bool XQ, int XR>
__global__ __launch_bounds__(256) void gemv_flat_kernel(Jobs J, int items, int per, const int8_t* __restrict__ xq,
                                                        const float* __restrict__ xs,
                                                        const int32_t* __restrict__ xsum,
                                                        const float* __restrict__ xf) {
    using W = typename Fmt<FMT>::W;
    extern __shared__ __align__(16) uint8_t xl[];
    __shared__ float part[2][R][4];
    const int lane = threadIdx.x & (DQ_WAVE - 1);
    const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / DQ_WAVE));
    const int ks = KS == 1 ? 0 : wv;
    const int i0 = min(ks * per, items);
    const int i1 = min(i0 + per, items);
    const int ngroups = J.g0[J.n];
    const int g = KS == 1 ? 4 * (int)blockIdx.x + wv : (int)blockIdx.x;
    const bool live = g < ngroups;  // uniform per wave (KS 1) / per workgroup (KS 4)
    // KS 1 with XQ: every wave takes part in the shared quantization first
    if ((KS == 4 || !XQ) && !live) return;

    // A wave of a K split whose item range is empty (i0 == i1 == items) still
    // loads (clamped, valid) addresses; its terms are masked in compute_group.
    // XQ rounds: KS 1 - the 4 waves share the whole activation (cols <= 8192,
    // <= 8 rounds each); KS 4 - each wave its own K quarter (<= 4096 columns).
    const int xc0 = KS == 1 ? 0 : 64 * i0, xc1 = KS == 1 ? 64 * items : 64 * i1;
    const int xw = KS == 1 ? wv : 0, xnw = KS == 1 ? 4 : 1;
    XStage<XR> xst;
    if constexpr (XQ) xstage_load<XR>(xst, xf, xc0, xc1, xw, xnw, lane);  // xc1 >= 64: loads stay in x
    int xi = min(i0 + lane, i1 - 1);  // this lane's activation item (clamped)
    XItem X[1];
    // pre-quantized activation: its registers are loaded before the weights,
    // so each row's arithmetic can start when that row's weights land
    if constexpr (!XQ) Fmt<FMT>::load_x(X[0], xi, xq, xs, xsum);
    __builtin_amdgcn_sched_barrier(0);
    W w[R][1];
    load_group<FMT, R, 1>(w, J, min(g, ngroups - 1), ngroups, i0, i1, lane, nullptr);
    // keep the quantization's arithmetic below the weight loads: hoisted above
    // them, it would wait for its activation loads before the weights are issued
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (XQ) {
        const int nblk = KS == 1 ? 2 * items : 2 * per;
        // wave region (KS 4): 80 bytes per item (64 int8, 2 scales, 2 sums)
        uint8_t* reg = KS == 1 ? xl : xl + (size_t)ks * 80 * per;
        xstage_quant<FMT, XR>(xst, xc0, xc1, xw, xnw, lane, nblk, reg);
        if constexpr (KS == 1) {
            __syncthreads();
            if (!live) return;
        }
        xq = reinterpret_cast<const int8_t*>(reg);
        xs = reinterpret_cast<const float*>(reg + 32 * nblk);
        xsum = reinterpret_cast<const int32_t*>(reg + 36 * nblk);
        if constexpr (KS == 4) xi = max(0, min(lane, i1 - i0 - 1));  // relative to i0 (a multiple of 4 items)
        Fmt<FMT>::load_x(X[0], xi, xq, xs, xsum);
    }
    compute_group<FMT, R, 1, KS>(w, X, J, g, i0, i1, lane, ks, part, 0);
}

// Flat grid over jobs of two per-256 formats reading one pre-quantized
// activation (the decoder layer's Q/K in Q4_K and V in Q6_K): one launch for
// the whole group. A wave's group belongs to one job, so each wave runs the
// single-format body (activation registers, every weight load of the group,
// the rows' dot products) of its job's format; the arithmetic is that of the
// single-format flat kernel. One item per lane (no K split).
template <int FA, int FB, int R>
__global__ __launch_bounds__(256) void gemv_flat_mixed_kernel(Jobs J, int items, const int8_t* __restrict__ xq,
                                                              const float* __restrict__ xs,
                                                              const int32_t* __restrict__ xsum) {
    const int lane = threadIdx.x & (DQ_WAVE - 1);
    const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / DQ_WAVE));
    const int ngroups = J.g0[J.n];
    const int g = 4 * (int)blockIdx.x + wv;
    if (g >= ngroups) return;  // uniform per wave
    int gl = 0;
    const int j = job_of(J, g, &gl);
    const int xi = min(lane, items - 1);
    auto body = [&](auto fc) {
        constexpr int F = decltype(fc)::value;
        using W = typename Fmt<F>::W;
        XItem X[1];
        Fmt<F>::load_x(X[0], xi, xq, xs, xsum);
        __builtin_amdgcn_sched_barrier(0);
        W w[R][1];
        load_group<F, R, 1>(w, J, g, ngroups, 0, items, lane, nullptr);
        __builtin_amdgcn_sched_barrier(0);
        compute_group<F, R, 1, 1>(w, X, J, g, 0, items, lane, 0, nullptr, 0);
    };
    if (J.fmt[j] == FB)  // uniform per wave
        body(std::integral_constant<int, FB>{});
    else
        body(std::integral_constant<int, FA>{});
}

// Per-256 quantization of the 16-wave flat grid, one 256-column block per
// 16-lane row: lane j of row q of wave w holds columns 1024w + 256q + 64k +
// 4j + [0, 4), k = 0..3 (each load instruction reads four contiguous 256-byte
// runs). A block's maximum is a 4-step DPP reduction within the row, and one
// scale and one reciprocal serve the lane's 16 values, so a wave quantizes
// 1024 columns per pass (16 waves: cols <= 16384 in one pass). Same
// integers, scales and sums as dq_quant_block; same LDS image as
// xstage_quant.
struct XRow {
    float4 v[4];
};

__device__ __forceinline__ void xrow_load(XRow& st, const float* __restrict__ xf, int cols, int w, int lane) {
    const int base = 1024 * w + 256 * (lane >> 4) + 4 * (lane & 15);
#pragma unroll
    for (int k = 0; k < 4; ++k) st.v[k] = *reinterpret_cast<const float4*>(xf + min(base + 64 * k, cols - 4));
}

__device__ __forceinline__ void xrow_quant(const XRow& st, int cols, int w, int lane, int nblk, uint8_t* xl) {
    float* ls = reinterpret_cast<float*>(xl + 32 * (size_t)nblk);
    int32_t* li = reinterpret_cast<int32_t*>(xl + 36 * (size_t)nblk);
    float m = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k)
        m = fmaxf(m, fmaxf(fmaxf(fabsf(st.v[k].x), fabsf(st.v[k].y)), fmaxf(fabsf(st.v[k].z), fabsf(st.v[k].w))));
    uint32_t am = __builtin_bit_cast(uint32_t, m);
    am = umax_dpp<0xB1>(am);   // quad_perm [1,0,3,2]
    am = umax_dpp<0x4E>(am);   // quad_perm [2,3,0,1]
    am = umax_dpp<0x141>(am);  // row_half_mirror
    am = umax_dpp<0x140>(am);  // row_mirror: the block's maximum in all 16 lanes
    const float amax = __builtin_bit_cast(float, am);
    const float d = amax > 0.0f ? div127(amax) : 0.0f;
    const float id = d > 0.0f ? 127.0f / amax : 0.0f;  // core/matmul.cpp:1681-1700
    uint32_t packed[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float4 v = st.v[k];
        const uint32_t lo = __builtin_amdgcn_perm(rint_bits(v.y * id), rint_bits(v.x * id), 0x0C0C0400u);
        const uint32_t hi = __builtin_amdgcn_perm(rint_bits(v.w * id), rint_bits(v.z * id), 0x0C0C0400u);
        packed[k] = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
    }
    if (__builtin_expect(!(id <= 3.40282347e38f), 0)) {
        // id = inf (block maximum below 127 / FLT_MAX): saturating conversion
        // and clamp, as dq_quant_block
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float vv[4] = {st.v[k].x, st.v[k].y, st.v[k].z, st.v[k].w};
            packed[k] = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int iv = (int)rintf(vv[e] * id);
                packed[k] |= (uint32_t)((iv > 127 ? 127 : (iv < -127 ? -127 : iv)) & 0xFF) << (8 * e);
            }
        }
    }
    int isum[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) isum[k] = sum8_lanes(dq_sdot4((int)packed[k], 0x01010101, 0));
    const int o = 1024 * w + 256 * (lane >> 4) + 4 * (lane & 15);
    if (1024 * w + 256 * (lane >> 4) < cols) {  // the row's block lies inside the activation
#pragma unroll
        for (int k = 0; k < 4; ++k) *reinterpret_cast<uint32_t*>(xl + o + 64 * k) = packed[k];
        if ((lane & 7) == 0) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                ls[(o + 64 * k) >> 5] = d;
                li[(o + 64 * k) >> 5] = isum[k];
            }
        }
    }
}

// Flat grid for the fp32 activation with the per-256 quantizer: NW-wave
// workgroups, one quantization of the activation per workgroup. KS 1: NW
// (4 or 8) groups per workgroup, one per wave; KS 4: NW / 4 groups of 4
// waves (K quarters). The activation is quantized whole into LDS
// (xrow_quant: pass p of wave w takes columns [1024(w + NW p), +1024), XP
// passes, cols <= 1024 NW XP), its loads issued before the weights. A wave with no columns skips the arithmetic but still consumes
// its loads, so the compiler keeps them above the weight loads (a load used
// only inside the branch would be sunk into it, and its wait would then be
// for every weight byte). No wave leaves before the last barrier; a group
// past the end computes the clamped last group and stores nothing.
template <int FMT, int R, int KS, int NW = 16>
__global__ __launch_bounds__(NW * 64) void gemv_flat16_kernel(Jobs J, int items, int per, const float* __restrict__ xf) {
    static_assert(NW == 16 || NW == 8 || (NW == 4 && KS == 1), "waves per workgroup");
    constexpr int XP = (KS == 4 && NW == 8) ? 2 : 1;  // quantization passes per wave (cols <= 1024 NW XP)
    using W = typename Fmt<FMT>::W;
    constexpr int GPW = KS == 1 ? NW : NW / 4;  // groups per workgroup
    extern __shared__ __align__(16) uint8_t xl[];
    __shared__ float part[GPW][R][4];
    const int lane = threadIdx.x & (DQ_WAVE - 1);
    const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / DQ_WAVE));
    const int ks = KS == 1 ? 0 : (wv & 3);
    const int gi = KS == 1 ? wv : (wv >> 2);
    const int i0 = min(ks * per, items);
    const int i1 = min(i0 + per, items);
    const int ngroups = J.g0[J.n];
    const int g = GPW * (int)blockIdx.x + gi;
    const bool live = g < ngroups;
    const int cols = 64 * items;

    XRow xst[XP];
#pragma unroll
    for (int p = 0; p < XP; ++p) xrow_load(xst[p], xf, cols, wv + NW * p, lane);
    W w[R][1];
    load_group<FMT, R, 1>(w, J, min(g, ngroups - 1), ngroups, i0, i1, lane, nullptr);
    __builtin_amdgcn_sched_barrier(0);
    const int nblk = 2 * items;
#pragma unroll
    for (int p = 0; p < XP; ++p) {
        if (1024 * (wv + NW * p) < cols)
            xrow_quant(xst[p], cols, wv + NW * p, lane, nblk, xl);
        else
            asm volatile("" ::"v"(xst[p].v[0].x), "v"(xst[p].v[1].x), "v"(xst[p].v[2].x), "v"(xst[p].v[3].x));
    }
    __syncthreads();
    if (KS == 1 && !live) return;  // KS 1 has no barrier after this one
    XItem X[1];
    Fmt<FMT>::load_x(X[0], min(i0 + lane, i1 - 1), reinterpret_cast<const int8_t*>(xl),
                     reinterpret_cast<const float*>(xl + 32 * nblk), reinterpret_cast<const int32_t*>(xl + 36 * nblk));
    compute_group<FMT, R, 1, KS>(w, X, J, min(g, ngroups - 1), i0, i1, lane, ks,
                                 reinterpret_cast<float(*)[R][4]>(&part[gi][0][0]), 0, live);
}

// The decoder layer's per-256 GEMV groups with the activation formed in the
// kernel from fp32 inputs, so that no launch sits between the GEMV and the
// kernel that wrote those inputs:
//  * XS_NORM: y = h * (1/sqrtf(mean(h^2) + eps)) * w (the layer's RMSNorm:
//    squares in float, summed in double; models/dense_forward.cpp:129-165);
//  * XS_SILU / XS_GEGLU: y = act(gate) * up (dq_ffn_act);
// then the per-256 quantizer into LDS (xrow_quant), as gemv_flat16_kernel.
// Every workgroup forms and quantizes the whole activation (one or two
// passes of 1024 columns per wave, loads issued before the weights). Jobs
// may be Q4_K and Q6_K together (the Q/K/V group): each job's groups start
// at a multiple of the workgroup's GPW groups, so a workgroup runs one
// format and its barriers are uniform. The norm's double sum runs per lane,
// over the wave by xor shuffles and over the waves in order: another order
// than norm_quant_kernel's, so the scale can differ in the last bit of the
// double (not of the float, except within ~1e-13 relative of a float
// rounding boundary); act(gate) * up is value by value, bit-identical.
enum XSrcKind { XS_NORM = DQ_FUSE_NORM, XS_SILU = DQ_FUSE_SILU, XS_GEGLU = DQ_FUSE_GEGLU };
struct XSrc {
    const float* a;  // XS_NORM: h; else gate
    const float* b;  // XS_NORM: the norm weights; else up
    float eps;
};

template <int FA, int FB, int R, int KS, int NW, int XS>
__global__ __launch_bounds__(NW * 64) void gemv_src_kernel(Jobs J, int items, int per, XSrc S) {
    static_assert(NW == 16 || NW == 8 || (NW == 4 && KS == 1), "waves per workgroup");
    constexpr int XP = (KS == 4 && NW == 8) ? 2 : 1;  // passes per wave (cols <= 1024 NW XP)
    constexpr int GPW = KS == 1 ? NW : NW / 4;        // groups per workgroup
    extern __shared__ __align__(16) uint8_t xl[];
    __shared__ float part[GPW][R][4];
    __shared__ double red[NW];
    const int lane = threadIdx.x & (DQ_WAVE - 1);
    const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / DQ_WAVE));
    const int ks = KS == 1 ? 0 : (wv & 3);
    const int gi = KS == 1 ? wv : (wv >> 2);
    const int i0 = min(ks * per, items);
    const int i1 = min(i0 + per, items);
    const int ngroups = J.g0[J.n];
    const int g = GPW * (int)blockIdx.x + gi;
    const bool live = g < ngroups;
    const int cols = 64 * items;
    const int nblk = 2 * items;
    int gl0 = 0;
    const int j0 = job_of(J, min(GPW * (int)blockIdx.x, ngroups - 1), &gl0);  // workgroup-uniform

    auto body = [&](auto fc) {
        constexpr int F = decltype(fc)::value;
        using W = typename Fmt<F>::W;
        XRow xa[XP], xb[XP];
#pragma unroll
        for (int p = 0; p < XP; ++p) {
            xrow_load(xa[p], S.a, cols, wv + NW * p, lane);
            xrow_load(xb[p], S.b, cols, wv + NW * p, lane);
        }
        W w[R][1];
        load_group<F, R, 1>(w, J, min(g, ngroups - 1), ngroups, i0, i1, lane, nullptr);
        __builtin_amdgcn_sched_barrier(0);
        XRow y[XP];
        if constexpr (XS == XS_NORM) {
            double acc = 0.0;
#pragma unroll
            for (int p = 0; p < XP; ++p) {
                // a 256-block of the row lies wholly inside or outside the columns
                const bool in = 1024 * (wv + NW * p) + 256 * (lane >> 4) < cols;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float4 v = xa[p].v[k];
                    const float s0 = v.x * v.x, s1 = v.y * v.y, s2 = v.z * v.z, s3 = v.w * v.w;
                    acc += in ? (double)s0 : 0.0;
                    acc += in ? (double)s1 : 0.0;
                    acc += in ? (double)s2 : 0.0;
                    acc += in ? (double)s3 : 0.0;
                }
            }
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, DQ_WAVE);
            if (lane == 0) red[wv] = acc;
            __syncthreads();
            double t = 0.0;
#pragma unroll
            for (int i = 0; i < NW; ++i) t += red[i];
            const float sc = 1.0f / sqrtf((float)(t / (double)cols) + S.eps);
#pragma unroll
            for (int p = 0; p < XP; ++p)
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float4 v = xa[p].v[k], ww = xb[p].v[k];
                    y[p].v[k] = float4{v.x * sc * ww.x, v.y * sc * ww.y, v.z * sc * ww.z, v.w * sc * ww.w};
                }
        } else {
            constexpr int ACT = XS == XS_GEGLU ? DQ_ACT_GEGLU : DQ_ACT_SILU;
#pragma unroll
            for (int p = 0; p < XP; ++p)
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float4 gv = xa[p].v[k], uv = xb[p].v[k];
                    y[p].v[k] = float4{dq_ffn_act<ACT>(gv.x) * uv.x, dq_ffn_act<ACT>(gv.y) * uv.y,
                                       dq_ffn_act<ACT>(gv.z) * uv.z, dq_ffn_act<ACT>(gv.w) * uv.w};
                }
        }
#pragma unroll
        for (int p = 0; p < XP; ++p) {
            if (1024 * (wv + NW * p) < cols)
                xrow_quant(y[p], cols, wv + NW * p, lane, nblk, xl);
            else
                asm volatile("" ::"v"(y[p].v[0].x), "v"(y[p].v[1].x), "v"(y[p].v[2].x), "v"(y[p].v[3].x));
        }
        __syncthreads();
        if (KS == 1 && !live) return;  // KS 1 has no barrier after this one
        XItem X[1];
        Fmt<F>::load_x(X[0], min(i0 + lane, i1 - 1), reinterpret_cast<const int8_t*>(xl),
                       reinterpret_cast<const float*>(xl + 32 * nblk),
                       reinterpret_cast<const int32_t*>(xl + 36 * nblk));
        compute_group<F, R, 1, KS>(w, X, J, min(g, ngroups - 1), i0, i1, lane, ks,
                                   reinterpret_cast<float(*)[R][4]>(&part[gi][0][0]), 0, live);
    };
    if (FA == FB || J.fmt[j0] == FA)
        body(std::integral_constant<int, FA>{});
    else
        body(std::integral_constant<int, FB>{});
}

// Persistent form of gemv_src_kernel (the gate+up group, whose weights do not
// fit in flight at once): 4-wave workgroups walking units of 4 groups (one
// per wave, one item per lane: cols <= 4096, no K split) with gemv_kernel's
// two-deep pipeline, after forming and quantizing the activation once per
// workgroup (one pass of 1024 columns per wave).
// GLU >= 0 (DQ_ACT_SILU / DQ_ACT_GEGLU; R = 2): the paired gated FFN. Jobs
// 0 and 1 are gate and up with the same rows; group g is row g of both, whose
// sums (the same as the unpaired launch's) give y0[g] = act(gate) * up
// (dq_ffn_act, models/dense_forward.cpp:53-55, :107-126) in the epilogue, so
// the FFN's activation leaves the kernel as one fp32 vector.
template <int F, int R, int XS, int XP = 1, int GLU = -1>
__global__ __launch_bounds__(256) void gemv_src_persist_kernel(Jobs J, int items, XSrc S) {
    static_assert(GLU < 0 || R == 2, "a pair per group");
    using W = typename Fmt<F>::W;
    extern __shared__ __align__(16) uint8_t xl[];
    __shared__ double red[4];
    const int lane = threadIdx.x & (DQ_WAVE - 1);
    const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / DQ_WAVE));
    const int ngroups = J.g0[J.n];
    const int stride = 4 * (int)gridDim.x;
    int g = 4 * (int)blockIdx.x + wv;
    const bool active = g < ngroups;  // uniform per wave
    const int cols = 64 * items, nblk = 2 * items;
    const uint8_t* dummy = reinterpret_cast<const uint8_t*>(S.a);

    XRow xa[XP], xb[XP];
#pragma unroll
    for (int p = 0; p < XP; ++p) {
        xrow_load(xa[p], S.a, cols, wv + 4 * p, lane);
        xrow_load(xb[p], S.b, cols, wv + 4 * p, lane);
    }
    W b0[R][1], b1[R][1];
    // GLU: row g of gate (job 0) and of up (job 1); past the last group a
    // cached dummy location
    auto load_pair = [&](W(&w)[R][1], int gg) {
        const bool live = gg < ngroups;
        const int xi = min(lane, items - 1);
#pragma unroll
        for (int rr = 0; rr < 2; ++rr)
            load_item<F>(w[rr][0], J.w[rr], J.L[rr], (size_t)(live ? gg : 0), xi, live, dummy);
    };
    auto compute_pair = [&](const W(&w)[R][1], const XItem& Xi, int gg, int xi) {
        float a[2];
#pragma unroll
        for (int rr = 0; rr < 2; ++rr) {
            const float p = Fmt<F>::dot(w[rr][0], Xi, xi);
            a[rr] = dq_wave_sum_uniform(0.0f + (lane < items ? p : 0.0f));
            __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (GLU >= 0)
            if (lane == 0) J.y[0][gg] = dq_ffn_act<GLU>(a[0]) * a[1];
    };
    if constexpr (GLU >= 0)
        load_pair(b0, active ? g : ngroups);
    else
        load_group<F, R, 1>(b0, J, active ? g : ngroups, ngroups, 0, items, lane, dummy);
    __builtin_amdgcn_sched_barrier(0);
    XRow y[XP];
    if constexpr (XS == XS_NORM) {
        double acc = 0.0;
#pragma unroll
        for (int p = 0; p < XP; ++p) {
            const bool in = 1024 * (wv + 4 * p) + 256 * (lane >> 4) < cols;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float4 v = xa[p].v[k];
                const float s0 = v.x * v.x, s1 = v.y * v.y, s2 = v.z * v.z, s3 = v.w * v.w;
                acc += in ? (double)s0 : 0.0;
                acc += in ? (double)s1 : 0.0;
                acc += in ? (double)s2 : 0.0;
                acc += in ? (double)s3 : 0.0;
            }
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, DQ_WAVE);
        if (lane == 0) red[wv] = acc;
        __syncthreads();
        const double t = ((red[0] + red[1]) + red[2]) + red[3];
        const float sc = 1.0f / sqrtf((float)(t / (double)cols) + S.eps);
#pragma unroll
        for (int p = 0; p < XP; ++p)
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float4 v = xa[p].v[k], ww = xb[p].v[k];
                y[p].v[k] = float4{v.x * sc * ww.x, v.y * sc * ww.y, v.z * sc * ww.z, v.w * sc * ww.w};
            }
    } else {
        constexpr int ACT = XS == XS_GEGLU ? DQ_ACT_GEGLU : DQ_ACT_SILU;
#pragma unroll
        for (int p = 0; p < XP; ++p)
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float4 gv = xa[p].v[k], uv = xb[p].v[k];
                y[p].v[k] = float4{dq_ffn_act<ACT>(gv.x) * uv.x, dq_ffn_act<ACT>(gv.y) * uv.y,
                                   dq_ffn_act<ACT>(gv.z) * uv.z, dq_ffn_act<ACT>(gv.w) * uv.w};
            }
    }
#pragma unroll
    for (int p = 0; p < XP; ++p) {
        if (1024 * (wv + 4 * p) < cols)
            xrow_quant(y[p], cols, wv + 4 * p, lane, nblk, xl);
        else
            asm volatile("" ::"v"(y[p].v[0].x), "v"(y[p].v[1].x), "v"(y[p].v[2].x), "v"(y[p].v[3].x));
    }
    __syncthreads();
    if (!active) return;  // no barrier follows (no K split)
    XItem X[1];
    Fmt<F>::load_x(X[0], min(lane, items - 1), reinterpret_cast<const int8_t*>(xl),
                   reinterpret_cast<const float*>(xl + 32 * nblk), reinterpret_cast<const int32_t*>(xl + 36 * nblk));
    if constexpr (GLU >= 0) {
        const int xi = min(lane, items - 1);
        for (;;) {
            load_pair(b1, g + stride);
            compute_pair(b0, X[0], g, xi);
            g += stride;
            if (g >= ngroups) break;
            load_pair(b0, g + stride);
            compute_pair(b1, X[0], g, xi);
            g += stride;
            if (g >= ngroups) break;
        }
    } else {
        for (;;) {
            load_group<F, R, 1>(b1, J, g + stride, ngroups, 0, items, lane, dummy);
            compute_group<F, R, 1, 1>(b0, X, J, g, 0, items, lane, 0, nullptr, 0);
            g += stride;
            if (g >= ngroups) break;
            load_group<F, R, 1>(b0, J, g + stride, ngroups, 0, items, lane, dummy);
            compute_group<F, R, 1, 1>(b1, X, J, g, 0, items, lane, 0, nullptr, 1);
            g += stride;
            if (g >= ngroups) break;
        }
    }
}

int g_num_cus = 0;

int num_cus() {
    if (g_num_cus == 0) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
            g_num_cus = n;
        else
            g_num_cus = 256;
    }
    return g_num_cus;
}

int env_int(const char* name, int dflt) {
    const char* e = getenv(name);
    return e ? atoi(e) : dflt;
}

// Fills the group prefix of J for R rows per group.
void set_groups(Jobs& J, int R) {
    J.g0[0] = 0;
    for (int j = 0; j < J.n; ++j) J.g0[j + 1] = J.g0[j] + (J.rows[j] + R - 1) / R;
}

// LDS budget of the in-kernel quantized activation: within the 64 KB of
// dynamic LDS a launch gets by default (cols <= 49152).
constexpr size_t XQ_MAX_LDS = 60 * 1024;

// Bytes of the in-kernel quantized activation (XQ) in LDS.
size_t xq_lds_bytes(size_t cols) { return cols + 8 * (cols / 32); }

template <int FMT, int R, int NIT, int KS>
int launch(Jobs J, int items, const int8_t* xq, const float* xs, const int32_t* xsum, const float* xf,
           hipStream_t s) {
    static const int wpc = env_int("DQ_GEMV_WPC", 8);  // persistent waves per CU
    set_groups(J, R);
    const int ngroups = J.g0[J.n];
    const int units = KS == 1 ? (ngroups + 3) / 4 : ngroups;
    const int max_wg = max(1, num_cus() * wpc / 4);
    const int iters = (units + max_wg - 1) / max_wg;  // balance: every workgroup walks `iters` units
    const unsigned grid = (unsigned)((units + iters - 1) / iters);
    if (xf)
        gemv_kernel<FMT, R, NIT, KS, true><<<grid, 256, xq_lds_bytes((size_t)items * 64), s>>>(J, items, xq, xs,
                                                                                               xsum, xf);
    else
        gemv_kernel<FMT, R, NIT, KS, false><<<grid, 256, 0, s>>>(J, items, xq, xs, xsum, xf);
    return dq_launch_status();
}

// Quantization rounds per wave of the 4-wave flat grid: KS 1 - the 4 waves
// share the activation's 256-column chunks (2, 4 or 8 rounds: cols <= 8192);
// KS 4 - each wave its own K quarter (per <= 64 items: 16 rounds).
template <int KS>
int flat_xr(int items, int per) {
    if (KS == 4) return 16;
    const int rounds = ((items + 3) / 4 + 3) / 4;
    return rounds <= 2 ? 2 : rounds <= 4 ? 4 : 8;
}

// Calls f(std::integral_constant<int, XR>) for the 4-wave flat grid's XR.
template <int KS, class F>
auto with_flat_xr(int xr, F&& f) {
    if constexpr (KS == 4) {
        return f(std::integral_constant<int, 16>{});
    } else {
        if (xr == 2) return f(std::integral_constant<int, 2>{});
        if (xr == 4) return f(std::integral_constant<int, 4>{});
        return f(std::integral_constant<int, 8>{});
    }
}

// The in-kernel quantized (XQ) instantiations exist for the per-32 formats
// only: the per-256 formats take gemv_flat16_kernel with the fp32 activation.
template <int FMT>
constexpr bool flat_xq() { return act_kind_of<FMT>() != DQ_ACT_Q8K_REP; }

template <int FMT, int R, int KS>
int launch_flat_r(Jobs J, int items, int per, const int8_t* xq, const float* xs, const int32_t* xsum,
                  const float* xf, hipStream_t s) {
    set_groups(J, R);
    const int ngroups = J.g0[J.n];
    const unsigned grid = (unsigned)(KS == 1 ? (ngroups + 3) / 4 : ngroups);
    if (xf) {
        if constexpr (flat_xq<FMT>()) {
            const size_t lds = KS == 1 ? (size_t)80 * items : (size_t)4 * 80 * per;
            with_flat_xr<KS>(flat_xr<KS>(items, per), [&](auto xr) {
                gemv_flat_kernel<FMT, R, KS, true, decltype(xr)::value>
                    <<<grid, 256, lds, s>>>(J, items, per, xq, xs, xsum, xf);
                return 0;
            });
        } else {
            return DQ_ERR_NOT_SUPPORTED;
        }
    } else {
        gemv_flat_kernel<FMT, R, KS, false, 1><<<grid, 256, 0, s>>>(J, items, per, xq, xs, xsum, xf);
    }
    return dq_launch_status();
}

// Returned by launch_flat when the flat grid does not apply (no launch).
constexpr int NO_FLAT = 1;

// Groups of R rows over the jobs of J.
int count_groups(const Jobs& J, int R) {
    int n = 0;
    for (int j = 0; j < J.n; ++j) n += (J.rows[j] + R - 1) / R;
    return n;
}

// Waves of gemv_flat_mixed_kernel<FA, FB, R> one CU holds at once (cached).
template <int FA, int FB, int R>
int mixed_resident_waves() {
    static int c = 0;
    if (c == 0) {
        int nb = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &nb, reinterpret_cast<const void*>(&gemv_flat_mixed_kernel<FA, FB, R>), 256, 0) != hipSuccess ||
            nb <= 0)
            nb = 1;
        c = 4 * nb;
    }
    return c;
}

template <int FA, int FB, int R>
int launch_mixed_r(Jobs J, int items, const int8_t* xq, const float* xs, const int32_t* xsum, hipStream_t s) {
    set_groups(J, R);
    const unsigned grid = (unsigned)((J.g0[J.n] + 3) / 4);
    gemv_flat_mixed_kernel<FA, FB, R><<<grid, 256, 0, s>>>(J, items, xq, xs, xsum);
    return dq_launch_status();
}

// One launch for a group of Q4_K and Q6_K jobs on a pre-quantized per-256
// activation (cols <= 4096: one item per lane), with the fewest rows per
// group (1, 2, 4) whose waves are all resident at once; NO_FLAT otherwise.
int launch_mixed(const Jobs& J, int items, const int8_t* xq, const float* xs, const int32_t* xsum, hipStream_t s) {
    static const int on = env_int("DQ_GEMV_MIXED", 1);
    if (!on || items > DQ_WAVE) return NO_FLAT;
    const long cus = num_cus();
    static const int wpc = env_int("DQ_GEMV_FWPC", 16);
    auto fits = [&](int r, int resident) { return (long)count_groups(J, r) <= cus * min(wpc, resident); };
    constexpr int A = DQ_FMT_Q4_K, B = DQ_FMT_Q6_K;
    if (fits(1, mixed_resident_waves<A, B, 1>())) return launch_mixed_r<A, B, 1>(J, items, xq, xs, xsum, s);
    if (fits(2, mixed_resident_waves<A, B, 2>())) return launch_mixed_r<A, B, 2>(J, items, xq, xs, xsum, s);
    if (fits(4, mixed_resident_waves<A, B, 4>())) return launch_mixed_r<A, B, 4>(J, items, xq, xs, xsum, s);
    return NO_FLAT;
}

template <int FMT, int R, int KS, int NW>
int launch_flat16_r(Jobs J, int items, int per, const float* xf, hipStream_t s) {
    set_groups(J, R);
    constexpr int GPW = KS == 1 ? NW : NW / 4;
    const unsigned grid = (unsigned)((J.g0[J.n] + GPW - 1) / GPW);
    gemv_flat16_kernel<FMT, R, KS, NW><<<grid, NW * 64, (size_t)80 * items, s>>>(J, items, per, xf);
    return dq_launch_status();
}

// Workgroups of gemv_flat16_kernel<FMT, R, KS, NW> one CU holds at once (cached).
template <int FMT, int R, int KS, int NW>
int flat16_resident(size_t lds) {
    static int c = -1;
    if (c < 0) {
        int nb = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &nb, reinterpret_cast<const void*>(&gemv_flat16_kernel<FMT, R, KS, NW>), NW * 64, lds) != hipSuccess)
            nb = 0;
        c = nb;
    }
    return c;
}

template <int FMT, int KS, int NW>
int launch_flat16_fit(const Jobs& J, int items, int per, const float* xf, hipStream_t s) {
    const size_t lds = (size_t)80 * items;
    constexpr int GPW = KS == 1 ? NW : NW / 4;
    static const int rmin = env_int("DQ_GEMV_F16_RMIN", 1);  // smallest rows per group tried
    const long cus = num_cus();
    auto fits = [&](int r, int resident) {
        return r >= rmin && resident > 0 && (count_groups(J, r) + GPW - 1) / GPW <= cus * resident;
    };
    // K split (wide rows: every workgroup quantizes >= 32 KB of activation):
    // the most rows per group whose grid still covers every CU, so the fewest
    // workgroups repeat the quantization
    if constexpr (KS == 4) {
        auto covers = [&](int r) { return (count_groups(J, r) + GPW - 1) / GPW >= cus; };
        if (covers(4) && fits(4, flat16_resident<FMT, 4, KS, NW>(lds)))
            return launch_flat16_r<FMT, 4, KS, NW>(J, items, per, xf, s);
        if (covers(2) && fits(2, flat16_resident<FMT, 2, KS, NW>(lds)))
            return launch_flat16_r<FMT, 2, KS, NW>(J, items, per, xf, s);
    }
    if (fits(1, flat16_resident<FMT, 1, KS, NW>(lds))) return launch_flat16_r<FMT, 1, KS, NW>(J, items, per, xf, s);
    if (fits(2, flat16_resident<FMT, 2, KS, NW>(lds))) return launch_flat16_r<FMT, 2, KS, NW>(J, items, per, xf, s);
    if (fits(4, flat16_resident<FMT, 4, KS, NW>(lds))) return launch_flat16_r<FMT, 4, KS, NW>(J, items, per, xf, s);
    return NO_FLAT;
}

// 16-wave flat grid with the fewest rows per group (1, 2, 4) whose
// workgroups are all resident at once (K split: see launch_flat16_fit);
// NO_FLAT otherwise.
template <int FMT, int KS>
int launch_flat16(const Jobs& J, int items, int per, const float* xf, hipStream_t s) {
    if ((size_t)80 * items > XQ_MAX_LDS || items * 64 > 16384) return NO_FLAT;
    // Without a K split: the fewest waves whose one pass covers the columns
    // (4 waves: cols <= 4096; 8 waves: cols <= 8192). The barrier after the
    // quantization waits for the workgroup's slowest wave to issue its loads
    // under memory back-pressure, so smaller workgroups start their dot
    // products sooner; the quantization they repeat costs ~100 instructions
    // per wave pass (Q4_K 14336x4096 fp32 step: 16 waves 8.66 us, 8 waves
    // 8.16 us, 4 waves 7.96 us; pre-quantized GEMV 7.61 us).
    static const int nw = env_int("DQ_GEMV_F16_NW", 4);  // smallest waves per workgroup tried
    if constexpr (KS == 1) {
        if (nw <= 4 && items * 64 <= 4096) return launch_flat16_fit<FMT, KS, 4>(J, items, per, xf, s);
        if (nw <= 8) return launch_flat16_fit<FMT, KS, 8>(J, items, per, xf, s);
    } else {
        // K split: 8 waves (2 groups of 4 K quarters, two quantization
        // passes per wave) rather than 16 (Q4_K 4096x14336 fp32 step 9.48 ->
        // 8.96 us, Q6_K 12.58 -> 11.78 us)
        static const int nw4 = env_int("DQ_GEMV_F16_NW4", 8);
        if (nw4 == 8) return launch_flat16_fit<FMT, KS, 8>(J, items, per, xf, s);
    }
    return launch_flat16_fit<FMT, KS, 16>(J, items, per, xf, s);
}

// ---- gemv_src_kernel launches
// Group prefix of J for R rows per group, every job's groups rounded up to a
// multiple of gpw (a workgroup's groups then belong to one job).
void set_groups_aligned(Jobs& J, int R, int gpw) {
    J.g0[0] = 0;
    for (int j = 0; j < J.n; ++j) J.g0[j + 1] = J.g0[j] + ((J.rows[j] + R - 1) / R + gpw - 1) / gpw * gpw;
}

// Workgroups of gemv_src_kernel<...> one CU holds at once (cached).
template <int FA, int FB, int R, int KS, int NW, int XS>
int src_resident(size_t lds) {
    static int c = -1;
    if (c < 0) {
        int nb = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &nb, reinterpret_cast<const void*>(&gemv_src_kernel<FA, FB, R, KS, NW, XS>), NW * 64, lds) !=
            hipSuccess)
            nb = 0;
        c = nb;
    }
    return c;
}

template <int FA, int FB, int R, int KS, int NW, int XS>
int launch_src_r(Jobs J, int items, int per, const XSrc& S, hipStream_t s) {
    constexpr int GPW = KS == 1 ? NW : NW / 4;
    set_groups_aligned(J, R, GPW);
    const unsigned grid = (unsigned)(J.g0[J.n] / GPW);
    gemv_src_kernel<FA, FB, R, KS, NW, XS><<<grid, NW * 64, (size_t)80 * items, s>>>(J, items, per, S);
    return dq_launch_status();
}

// The fewest rows per group (K split: the most that still cover every CU,
// else the fewest that fit) whose workgroups are all resident at once, as
// launch_flat16_fit; NO_FLAT when none fits.
template <int FA, int FB, int KS, int NW, int XS>
int launch_src_fit(const Jobs& J, int items, int per, const XSrc& S, hipStream_t s) {
    const size_t lds = (size_t)80 * items;
    constexpr int GPW = KS == 1 ? NW : NW / 4;
    const long cus = num_cus();
    auto wgs = [&](int r) {
        Jobs t = J;
        set_groups_aligned(t, r, GPW);
        return (long)(t.g0[t.n] / GPW);
    };
    auto fits = [&](int r, int resident) { return resident > 0 && wgs(r) <= cus * resident; };
    if constexpr (KS == 4) {
        const int res4 = src_resident<FA, FB, 4, KS, NW, XS>(lds);
        if (wgs(4) >= cus && fits(4, res4)) return launch_src_r<FA, FB, 4, KS, NW, XS>(J, items, per, S, s);
        if (fits(2, src_resident<FA, FB, 2, KS, NW, XS>(lds)))
            return launch_src_r<FA, FB, 2, KS, NW, XS>(J, items, per, S, s);
        if (fits(4, res4)) return launch_src_r<FA, FB, 4, KS, NW, XS>(J, items, per, S, s);
    } else {
        if (fits(1, src_resident<FA, FB, 1, KS, NW, XS>(lds)))
            return launch_src_r<FA, FB, 1, KS, NW, XS>(J, items, per, S, s);
        if (fits(2, src_resident<FA, FB, 2, KS, NW, XS>(lds)))
            return launch_src_r<FA, FB, 2, KS, NW, XS>(J, items, per, S, s);
        if (fits(4, src_resident<FA, FB, 4, KS, NW, XS>(lds)))
            return launch_src_r<FA, FB, 4, KS, NW, XS>(J, items, per, S, s);
    }
    return NO_FLAT;
}

// The persistent form for one format (two rows per group, as gemv_kernel's
// grid: at most DQ_GEMV_WPC waves per CU, every workgroup walking the same
// number of units).
template <int F, int XS, int GLU = -1>
int launch_src_persist(Jobs J, size_t cols, const XSrc& S, hipStream_t s) {
    static const int wpc = env_int("DQ_GEMV_WPC", 8);
    constexpr int R = 2;
    if constexpr (GLU >= 0) {  // one group per pair of rows
        J.g0[0] = 0;
        J.g0[1] = J.g0[2] = J.rows[0];
    } else {
        set_groups(J, R);
    }
    const int units = (J.g0[J.n] + 3) / 4;
    const int max_wg = max(1, num_cus() * wpc / 4);
    const int iters = (units + max_wg - 1) / max_wg;
    const unsigned grid = (unsigned)((units + iters - 1) / iters);
    const int items = (int)(cols / 64);  // <= 64: one item per lane
    gemv_src_persist_kernel<F, R, XS, 1, GLU><<<grid, 256, (size_t)80 * items, s>>>(J, items, S);
    return dq_launch_status();
}

// Instantiated shapes (one item per lane): rows of <= 4096 columns without a
// K split (4-wave workgroups; the norm form of one format takes the
// persistent grid where the flat one does not fit), rows of 4097..16384
// columns with the K split (8 waves of two passes, else 16 waves of one).
template <int FA, int FB, int XS>
int launch_src(const Jobs& J, size_t cols, const XSrc& S, hipStream_t s) {
    const int items = (int)(cols / 64);
    if (cols <= 4096) {
        const int rc = launch_src_fit<FA, FB, 1, 4, XS>(J, items, items, S, s);
        if (rc != NO_FLAT) return rc;
        if constexpr (FA == FB) return launch_src_persist<FA, XS>(J, cols, S, s);
        return NO_FLAT;
    }
    if (cols > 16384) return NO_FLAT;
    const int per = (items + 15) / 16 * 4;  // whole 256-blocks per K quarter
    const int rc = launch_src_fit<FA, FB, 4, 8, XS>(J, items, per, S, s);
    if (rc != NO_FLAT) return rc;
    return launch_src_fit<FA, FB, 4, 16, XS>(J, items, per, S, s);
}

// Waves of gemv_flat_kernel<FMT, R, KS, XQ, XR> that one CU holds at once
// (its register and LDS needs; cached per instantiation; XR as flat_xr).
template <int FMT, int R, int KS>
int flat_resident_waves(bool xq, int xr, size_t lds) {
    static int cached[4] = {0, 0, 0, 0};
    const int slot = !xq ? 0 : xr == 2 ? 1 : xr == 4 ? 2 : 3;
    int& c = cached[slot];
    if (c == 0) {
        const void* k = reinterpret_cast<const void*>(&gemv_flat_kernel<FMT, R, KS, false, 1>);
        if constexpr (flat_xq<FMT>())
            if (xq)
                k = with_flat_xr<KS>(xr, [&](auto x) {
                    return reinterpret_cast<const void*>(&gemv_flat_kernel<FMT, R, KS, true, decltype(x)::value>);
                });
        int nb = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k, 256, lds) != hipSuccess || nb <= 0) nb = 1;
        c = 4 * nb;
    }
    return c;
}


// The flat grid with the fewest rows per group (1, 2, 4 or 8) whose waves all
// fit on the CUs at once, at most `wpc` per CU; NO_FLAT when one item per
// lane does not cover a wave's K range or no R fits (then the persistent grid
// runs).
template <int FMT, int KS>
int launch_flat(const Jobs& J, int items, int per, int nit, const int8_t* xq, const float* xs, const int32_t* xsum,
                const float* xf, hipStream_t s) {
    static const int on = env_int("DQ_GEMV_FLAT", 1);
    static const int wpc = env_int("DQ_GEMV_FWPC", 16);
    if (!on || nit != 1) return NO_FLAT;
    // fp32 activation with the per-256 quantizer (cross-row reductions and
    // two divisions per 256 columns, repeated by every workgroup): 16-wave
    // workgroups
    if constexpr (act_kind_of<FMT>() == DQ_ACT_Q8K_REP)
        if (xf) return launch_flat16<FMT, KS>(J, items, per, xf, s);
    const size_t lds = !xf ? 0 : KS == 1 ? (size_t)80 * items : (size_t)4 * 80 * per;
    if (lds > XQ_MAX_LDS) return NO_FLAT;
    const int gw = KS == 1 ? 1 : 4;  // waves per group
    const long cus = num_cus();
    const bool q = xf != nullptr;
    const int xr = flat_xr<KS>(items, per);
    auto fits = [&](int r, int resident) { return (long)count_groups(J, r) * gw <= cus * min(wpc, resident); };
    constexpr int WB = (int)sizeof(typename Fmt<FMT>::W);  // weight bytes per row per lane
    if (fits(1, flat_resident_waves<FMT, 1, KS>(q, xr, lds)))
        return launch_flat_r<FMT, 1, KS>(J, items, per, xq, xs, xsum, xf, s);
    if (fits(2, flat_resident_waves<FMT, 2, KS>(q, xr, lds)))
        return launch_flat_r<FMT, 2, KS>(J, items, per, xq, xs, xsum, xf, s);
    if (fits(4, flat_resident_waves<FMT, 4, KS>(q, xr, lds)))
        return launch_flat_r<FMT, 4, KS>(J, items, per, xq, xs, xsum, xf, s);
    if (8 * WB <= 400 && fits(8, flat_resident_waves<FMT, 8, KS>(q, xr, lds)))
        return launch_flat_r<FMT, 8, KS>(J, items, per, xq, xs, xsum, xf, s);
    return NO_FLAT;
}

// Persistent grid: two rows per group when one item per lane covers the K
// range, else one row with NIT items per lane. KS 1 has items <= 128 (NIT <= 2).
template <int FMT, int KS>
int launch_nit(int nit, const Jobs& J, int items, const int8_t* xq, const float* xs, const int32_t* xsum,
               const float* xf, hipStream_t s) {
    switch (nit) {
    case 1: return launch<FMT, 2, 1, KS>(J, items, xq, xs, xsum, xf, s);
    case 2: return launch<FMT, 1, 2, KS>(J, items, xq, xs, xsum, xf, s);
    }
    if constexpr (KS == 4) {
        if (nit == 3) return launch<FMT, 1, 3, KS>(J, items, xq, xs, xsum, xf, s);
        if (nit == 4) return launch<FMT, 1, 4, KS>(J, items, xq, xs, xsum, xf, s);
        if (nit <= 6) return launch<FMT, 1, 6, KS>(J, items, xq, xs, xsum, xf, s);
        if (nit <= 8) return launch<FMT, 1, 8, KS>(J, items, xq, xs, xsum, xf, s);
    }
    return DQ_ERR_NOT_SUPPORTED;
}

template <int FMT>
int launch_fmt(const Jobs& J, size_t cols, const int8_t* xq, const float* xs, const int32_t* xsum, const float* xf,
               hipStream_t s) {
    const int items = (int)(cols / 64);
    // K split: rows wider than 128 items are shared by the 4 waves of a workgroup
    const int ks = items > 2 * DQ_WAVE ? 4 : 1;
    const int per = ks == 1 ? items : (items + 3) / 4;
    const int nit = (per + DQ_WAVE - 1) / DQ_WAVE;
    if (nit > 8) return DQ_ERR_NOT_SUPPORTED;
    {   // flat grid first; a wave's K quarter holds whole 256-blocks (per-256 quantizer)
        const int fper = ks == 1 ? items : (act_kind_of<FMT>() == DQ_ACT_Q8K_REP ? (items + 15) / 16 * 4 : per);
        const int fnit = (fper + DQ_WAVE - 1) / DQ_WAVE;
        const int rc = ks == 1 ? launch_flat<FMT, 1>(J, items, fper, fnit, xq, xs, xsum, xf, s)
                               : launch_flat<FMT, 4>(J, items, fper, fnit, xq, xs, xsum, xf, s);
        if (rc != NO_FLAT) return rc;
    }
    return ks == 1 ? launch_nit<FMT, 1>(nit, J, items, xq, xs, xsum, xf, s)
                   : launch_nit<FMT, 4>(nit, J, items, xq, xs, xsum, xf, s);
}

int launch_jobs(int fmt, const Jobs& J, size_t cols, const int8_t* xq, const float* xs, const int32_t* xsum,
                const float* xf, hipStream_t s) {
    switch (fmt) {
    case DQ_FMT_Q8_0: return launch_fmt<DQ_FMT_Q8_0>(J, cols, xq, xs, xsum, xf, s);
    case DQ_FMT_Q4_0: return launch_fmt<DQ_FMT_Q4_0>(J, cols, xq, xs, xsum, xf, s);
    case DQ_FMT_Q4_K: return launch_fmt<DQ_FMT_Q4_K>(J, cols, xq, xs, xsum, xf, s);
    case DQ_FMT_Q6_K: return launch_fmt<DQ_FMT_Q6_K>(J, cols, xq, xs, xsum, xf, s);
    }
    return DQ_ERR_NOT_SUPPORTED;
}

bool per32_act(int fmt) { return fmt == DQ_FMT_Q8_0 || fmt == DQ_FMT_Q4_0; }
bool needs_sum(int fmt) { return fmt == DQ_FMT_Q4_0 || fmt == DQ_FMT_Q4_K; }

// Validates n jobs; writes the layouts. NOT_SUPPORTED for shapes/formats the
// kernels do not cover and for groups that mix the per-32 (Q8_0, Q4_0) and
// per-256 (Q4_K, Q6_K) activation kinds.
int check_jobs(const dq_gemv_job_t* jobs, size_t n, size_t cols, const int8_t* xq, const float* xs,
               const int32_t* xsum, const float* xf, DqLayout* L) {
    if (n == 0) return DQ_OK;
    if (!jobs) return DQ_ERR_INVALID_ARG;
    if (n > DQ_GEMV_MAX_JOBS) return DQ_ERR_NOT_SUPPORTED;
    for (size_t j = 0; j < n; ++j) {
        if (!dq_layout(jobs[j].fmt, jobs[j].rows, cols, &L[j])) return DQ_ERR_NOT_SUPPORTED;
        if (jobs[j].rows > 0x3FFFFFFF) return DQ_ERR_NOT_SUPPORTED;
        // one shared pre-quantized activation serves one activation kind;
        // with the fp32 activation every launch quantizes for its own format
        if (!xf && per32_act(jobs[j].fmt) != per32_act(jobs[0].fmt)) return DQ_ERR_NOT_SUPPORTED;
    }
    if (xf && xq_lds_bytes(cols) > XQ_MAX_LDS) return DQ_ERR_NOT_SUPPORTED;
    for (size_t j = 0; j < n; ++j) {
        if (jobs[j].rows == 0) continue;  // nothing to do: no pointer is read
        if (!jobs[j].d_w || !jobs[j].d_y) return DQ_ERR_INVALID_ARG;
        if (xf) continue;
        if (!xq || !xs) return DQ_ERR_INVALID_ARG;
        if (needs_sum(jobs[j].fmt) && !xsum) return DQ_ERR_INVALID_ARG;
    }
    return DQ_OK;
}

// One launch per distinct format, in job order of first appearance.
int run_jobs(const dq_gemv_job_t* jobs, size_t n, size_t cols, const int8_t* xq, const float* xs,
             const int32_t* xsum, const float* xf, hipStream_t s) {
    DqLayout L[DQ_GEMV_MAX_JOBS];
    const int rc = check_jobs(jobs, n, cols, xq, xs, xsum, xf, L);
    if (rc != DQ_OK || n == 0) return rc;
    {   // Q4_K and Q6_K jobs together on a pre-quantized activation: one launch
        bool q4 = false, q6 = false, other = false;
        for (size_t j = 0; j < n; ++j) {
            if (jobs[j].rows == 0) continue;
            q4 = q4 || jobs[j].fmt == DQ_FMT_Q4_K;
            q6 = q6 || jobs[j].fmt == DQ_FMT_Q6_K;
            other = other || (jobs[j].fmt != DQ_FMT_Q4_K && jobs[j].fmt != DQ_FMT_Q6_K);
        }
        if (!xf && q4 && q6 && !other) {
            Jobs J{};
            for (size_t j = 0; j < n; ++j) {
                if (jobs[j].rows == 0) continue;
                J.w[J.n] = (const uint8_t*)jobs[j].d_w;
                J.fmt[J.n] = jobs[j].fmt;
                J.L[J.n] = L[j];
                J.y[J.n] = jobs[j].d_y;
                J.res[J.n] = jobs[j].d_res;
                J.rows[J.n] = (int)jobs[j].rows;
                ++J.n;
            }
            const int r = launch_mixed(J, (int)(cols / 64), xq, xs, xsum, s);
            if (r != NO_FLAT) return r;
        }
    }
    bool done[DQ_GEMV_MAX_JOBS] = {};
    for (size_t a = 0; a < n; ++a) {
        if (done[a]) continue;
        Jobs J{};
        const int fmt = jobs[a].fmt;
        for (size_t j = a; j < n; ++j) {
            if (done[j] || jobs[j].fmt != fmt) continue;
            done[j] = true;
            if (jobs[j].rows == 0) continue;
            J.w[J.n] = (const uint8_t*)jobs[j].d_w;
            J.fmt[J.n] = fmt;
            J.L[J.n] = L[j];
            J.y[J.n] = jobs[j].d_y;
            J.res[J.n] = jobs[j].d_res;
            J.rows[J.n] = (int)jobs[j].rows;
            ++J.n;
        }
        if (J.n == 0) continue;
        const int r = launch_jobs(fmt, J, cols, xq, xs, xsum, xf, s);
        if (r != DQ_OK) return r;
    }
    return DQ_OK;
}

}  // namespace

extern "C" int dq_gemv(int fmt, const void* d_w, size_t rows, size_t cols, const int8_t* d_xq,
                       const float* d_xscale, const int32_t* d_xsum, float* d_y, void* stream) {
    const dq_gemv_job_t job = {fmt, d_w, rows, d_y, nullptr};
    return run_jobs(&job, 1, cols, d_xq, d_xscale, d_xsum, nullptr, (hipStream_t)stream);
}

extern "C" int dq_gemv_add(int fmt, const void* d_w, size_t rows, size_t cols, const int8_t* d_xq,
                           const float* d_xscale, const int32_t* d_xsum, const float* d_res, float* d_y,
                           void* stream) {
    if (!d_res) return DQ_ERR_INVALID_ARG;
    const dq_gemv_job_t job = {fmt, d_w, rows, d_y, d_res};
    return run_jobs(&job, 1, cols, d_xq, d_xscale, d_xsum, nullptr, (hipStream_t)stream);
}

extern "C" int dq_gemv_group(const dq_gemv_job_t* jobs, size_t n, size_t cols, const int8_t* d_xq,
                             const float* d_xscale, const int32_t* d_xsum, void* stream) {
    return run_jobs(jobs, n, cols, d_xq, d_xscale, d_xsum, nullptr, (hipStream_t)stream);
}

extern "C" int dq_gemv_f32(int fmt, const void* d_w, size_t rows, size_t cols, const float* d_x, float* d_y,
                           void* stream) {
    if (!d_x && rows) return DQ_ERR_INVALID_ARG;
    const dq_gemv_job_t job = {fmt, d_w, rows, d_y, nullptr};
    return run_jobs(&job, 1, cols, nullptr, nullptr, nullptr, d_x, (hipStream_t)stream);
}

extern "C" int dq_gemv_group_f32(const dq_gemv_job_t* jobs, size_t n, size_t cols, const float* d_x,
                                 void* stream) {
    bool any = false;
    for (size_t j = 0; jobs && j < n; ++j) any = any || jobs[j].rows;
    if (!d_x && any) return DQ_ERR_INVALID_ARG;
    return run_jobs(jobs, n, cols, nullptr, nullptr, nullptr, d_x, (hipStream_t)stream);
}

extern "C" int dq_gemv_group_fused(const dq_gemv_job_t* jobs, size_t n, size_t cols, int kind, const float* d_a,
                                   const float* d_b, float eps, void* stream) {
    if (kind < DQ_FUSE_NORM || kind > DQ_FUSE_NORM_GEGLU) return DQ_ERR_NOT_SUPPORTED;
    const bool glu = kind == DQ_FUSE_NORM_SILU || kind == DQ_FUSE_NORM_GEGLU;
    if (glu && (n != 2 || !jobs || jobs[0].fmt != jobs[1].fmt || jobs[0].rows != jobs[1].rows || jobs[0].d_res ||
                jobs[1].d_res || cols > 4096))
        return DQ_ERR_NOT_SUPPORTED;
    if (n == 0 || !jobs || n > DQ_GEMV_MAX_JOBS || cols % 256 || cols == 0) return DQ_ERR_NOT_SUPPORTED;
    if (!d_a || !d_b) return DQ_ERR_INVALID_ARG;
    DqLayout L[DQ_GEMV_MAX_JOBS];
    bool q4 = false, q6 = false;
    Jobs J{};
    for (size_t j = 0; j < n; ++j) {
        if (jobs[j].fmt != DQ_FMT_Q4_K && jobs[j].fmt != DQ_FMT_Q6_K) return DQ_ERR_NOT_SUPPORTED;
        if (!dq_layout(jobs[j].fmt, jobs[j].rows, cols, &L[j]) || jobs[j].rows > 0x3FFFFFFF)
            return DQ_ERR_NOT_SUPPORTED;
        if (jobs[j].rows == 0) continue;
        if (!jobs[j].d_w || !jobs[j].d_y) return DQ_ERR_INVALID_ARG;
        q4 = q4 || jobs[j].fmt == DQ_FMT_Q4_K;
        q6 = q6 || jobs[j].fmt == DQ_FMT_Q6_K;
        J.w[J.n] = (const uint8_t*)jobs[j].d_w;
        J.fmt[J.n] = jobs[j].fmt;
        J.L[J.n] = L[j];
        J.y[J.n] = jobs[j].d_y;
        J.res[J.n] = jobs[j].d_res;
        J.rows[J.n] = (int)jobs[j].rows;
        ++J.n;
    }
    if (J.n == 0) return DQ_OK;
    const XSrc S{d_a, d_b, eps};
    const hipStream_t s = (hipStream_t)stream;
    constexpr int A = DQ_FMT_Q4_K, B = DQ_FMT_Q6_K;
    int rc = NO_FLAT;
    if (glu) {
        // gate and up of one format, paired in the persistent kernel
        if (kind == DQ_FUSE_NORM_SILU)
            rc = q4 ? launch_src_persist<A, XS_NORM, DQ_ACT_SILU>(J, cols, S, s)
                    : launch_src_persist<B, XS_NORM, DQ_ACT_SILU>(J, cols, S, s);
        else
            rc = q4 ? launch_src_persist<A, XS_NORM, DQ_ACT_GEGLU>(J, cols, S, s)
                    : launch_src_persist<B, XS_NORM, DQ_ACT_GEGLU>(J, cols, S, s);
    } else if (kind == DQ_FUSE_NORM) {
        rc = q4 && q6 ? launch_src<A, B, XS_NORM>(J, cols, S, s)
                      : (q4 ? launch_src<A, A, XS_NORM>(J, cols, S, s) : launch_src<B, B, XS_NORM>(J, cols, S, s));
    } else if (!(q4 && q6)) {
        if (kind == DQ_FUSE_SILU)
            rc = q4 ? launch_src<A, A, XS_SILU>(J, cols, S, s) : launch_src<B, B, XS_SILU>(J, cols, S, s);
        else
            rc = q4 ? launch_src<A, A, XS_GEGLU>(J, cols, S, s) : launch_src<B, B, XS_GEGLU>(J, cols, S, s);
    }
    return rc == NO_FLAT ? DQ_ERR_NOT_SUPPORTED : rc;
}
