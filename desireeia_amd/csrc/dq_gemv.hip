// dq_gemv.hip - batch-1 decode GEMV for Q8_0, Q4_0, Q4_K and Q6_K weights.
//
// HBM-bound design (gfx950, wave64):
//  * A row is cut into "items" of 64 weights (cols/64 per row). Lane l of a
//    wave owns items l, l+64, l+128, ... of EVERY row it visits, so the 64
//    activation bytes of each owned item (plus its scales/sums) are loaded
//    into registers once per wave and reused for all its rows; only weights
//    stream from HBM.
//  * A wave computes R rows. All weight loads of the R rows (global_load
//    dwordx4, non-temporal) are issued before any arithmetic, so each wave
//    keeps R*NIT*(2..4) 16-byte loads in flight.
//  * Nibble/6-bit unpack and 6-bit scale decode happen in registers; dots are
//    v_dot4_i32_i8; a row's partials are combined with a wave reduction.
//
// Semantics follow the reference CPU GEMVs (see include/desireeia_hip.h):
// integer partial sums are exact; only the float summation order differs.
#include "dq_common.h"

#include <cstdlib>

namespace {

struct XItem {
    dq_u32x4 x[4];  // 64 activation bytes of the item
    float s0, s1;   // activation scales (per 32 / per 256)
    int i0, i1;     // activation integer sums
};

__device__ __forceinline__ int dot16(const dq_u32x4& w, const dq_u32x4& x, int acc) {
    acc = dq_sdot4((int)w.x, (int)x.x, acc);
    acc = dq_sdot4((int)w.y, (int)x.y, acc);
    acc = dq_sdot4((int)w.z, (int)x.z, acc);
    acc = dq_sdot4((int)w.w, (int)x.w, acc);
    return acc;
}

__device__ __forceinline__ dq_u32x4 nib_lo(const dq_u32x4& v) {
    return dq_u32x4{v.x & 0x0F0F0F0Fu, v.y & 0x0F0F0F0Fu, v.z & 0x0F0F0F0Fu, v.w & 0x0F0F0F0Fu};
}
__device__ __forceinline__ dq_u32x4 nib_hi(const dq_u32x4& v) {
    return dq_u32x4{(v.x >> 4) & 0x0F0F0F0Fu, (v.y >> 4) & 0x0F0F0F0Fu, (v.z >> 4) & 0x0F0F0F0Fu,
                    (v.w >> 4) & 0x0F0F0F0Fu};
}

// ---------------------------------------------------------------- formats --
// Each format: NW = 16-byte weight loads per item; load_x / load_w / dot.

template <int FMT>
struct Fmt;

// Q8_0: item = blocks 2i, 2i+1 (64 int8 in plane Q) + 2 fp16 scales (plane D).
template <>
struct Fmt<DQ_FMT_Q8_0> {
    static constexpr int NW = 4;
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
    __device__ static void load_w(W& w, const uint8_t* base, const DqLayout& L, size_t r, int i) {
        const uint8_t* q = base + L.q_off + r * L.q_row + 64 * (size_t)i;
        w.q[0] = dq_ld16_stream(q);
        w.q[1] = dq_ld16_stream(q + 16);
        w.q[2] = dq_ld16_stream(q + 32);
        w.q[3] = dq_ld16_stream(q + 48);
        w.d = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(base + L.d_off + r * L.d_row + 4 * (size_t)i));
    }
    __device__ static float dot(const W& w, const XItem& X) {
        const int a = dot16(w.q[1], X.x[1], dot16(w.q[0], X.x[0], 0));
        const int b = dot16(w.q[3], X.x[3], dot16(w.q[2], X.x[2], 0));
        const float d0 = dq_h2f((uint16_t)(w.d & 0xFFFF)), d1 = dq_h2f((uint16_t)(w.d >> 16));
        return d0 * X.s0 * (float)a + d1 * X.s1 * (float)b;
    }
};

// Q4_0: item = blocks 2i, 2i+1 (2 x 16 nibble bytes) + 2 fp16 scales.
// sum (nib-8)*x = sum nib*x - 8*sum x.
template <>
struct Fmt<DQ_FMT_Q4_0> {
    static constexpr int NW = 2;
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
    __device__ static void load_w(W& w, const uint8_t* base, const DqLayout& L, size_t r, int i) {
        const uint8_t* q = base + L.q_off + r * L.q_row + 32 * (size_t)i;
        w.q[0] = dq_ld16_stream(q);
        w.q[1] = dq_ld16_stream(q + 16);
        w.d = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(base + L.d_off + r * L.d_row + 4 * (size_t)i));
    }
    __device__ static float dot(const W& w, const XItem& X) {
        const int a = dot16(nib_hi(w.q[0]), X.x[1], dot16(nib_lo(w.q[0]), X.x[0], 0)) - 8 * X.i0;
        const int b = dot16(nib_hi(w.q[1]), X.x[3], dot16(nib_lo(w.q[1]), X.x[2], 0)) - 8 * X.i1;
        const float d0 = dq_h2f((uint16_t)(w.d & 0xFFFF)), d1 = dq_h2f((uint16_t)(w.d >> 16));
        return d0 * X.s0 * (float)a + d1 * X.s1 * (float)b;
    }
};

// Q4_K (native 144-byte blocks): item (s = i/4, g = i%4) = sub-blocks 2g
// (low nibbles) and 2g+1 (high nibbles) of super-block s; header = first 16
// bytes of the block (d, dmin, 12 scale bytes).
template <>
struct Fmt<DQ_FMT_Q4_K> {
    static constexpr int NW = 3;
    struct W {
        dq_u32x4 h, qa, qb;
    };
    __device__ static void load_x(XItem& X, int i, const int8_t* xq, const float* xs, const int32_t* xsum) {
        const dq_u32x4* p = reinterpret_cast<const dq_u32x4*>(xq + 64 * (size_t)i);
        X.x[0] = p[0]; X.x[1] = p[1]; X.x[2] = p[2]; X.x[3] = p[3];
        X.s0 = xs[2 * i];  // the per-256 scale, replicated in every per-32 slot
        X.i0 = xsum[2 * i];
        X.i1 = xsum[2 * i + 1];
    }
    __device__ static void load_w(W& w, const uint8_t* base, const DqLayout& L, size_t r, int i) {
        const uint8_t* blk = base + r * L.q_row + (size_t)(i >> 2) * DQ_SZ_Q4_K;
        w.h = dq_ld16_stream(blk);
        w.qa = dq_ld16_stream(blk + 16 + 32 * (i & 3));
        w.qb = dq_ld16_stream(blk + 32 + 32 * (i & 3));
    }
    __device__ static float dot(const W& w, const XItem& X, int g) {
        // low nibbles: sub-block 2g elements 0..31 (x bytes 0..31)
        const int da = dot16(nib_lo(w.qb), X.x[1], dot16(nib_lo(w.qa), X.x[0], 0));
        const int db = dot16(nib_hi(w.qb), X.x[3], dot16(nib_hi(w.qa), X.x[2], 0));
        // 6-bit scales/mins of sub-blocks j = 2g, 2g+1 (quant/quant.cpp:22-29)
        // scale bytes q[0..11] = header bytes 4..15 = words h.y, h.z, h.w
        const uint32_t w0 = w.h.y, w1 = w.h.z, w2 = w.h.w;
        int sca, mna, scb, mnb;
        if (g < 2) {
            // j = 2g, 2g+1 < 4: sc = q[j] & 63, m = q[j+4] & 63
            const int sh = 16 * g;
            sca = (w0 >> sh) & 63;
            scb = (w0 >> (sh + 8)) & 63;
            mna = (w1 >> sh) & 63;
            mnb = (w1 >> (sh + 8)) & 63;
        } else {
            // j >= 4: sc = (q[j+4]&15) | ((q[j-4]>>6)<<4), m = (q[j+4]>>4) | ((q[j]>>6)<<4)
            const int sh = 16 * (g - 2);  // byte index (j-4) within a word
            const uint32_t qa8 = (w2 >> sh) & 0xFF, qb8 = (w2 >> (sh + 8)) & 0xFF;       // q[j+4]
            const uint32_t la = (w0 >> sh) & 0xFF, lb = (w0 >> (sh + 8)) & 0xFF;         // q[j-4]
            const uint32_t ma = (w1 >> sh) & 0xFF, mb = (w1 >> (sh + 8)) & 0xFF;         // q[j]
            sca = (int)((qa8 & 0xF) | ((la >> 6) << 4));
            scb = (int)((qb8 & 0xF) | ((lb >> 6) << 4));
            mna = (int)((qa8 >> 4) | ((ma >> 6) << 4));
            mnb = (int)((qb8 >> 4) | ((mb >> 6) << 4));
        }
        const float d = dq_h2f((uint16_t)(w.h.x & 0xFFFF));
        const float dmin = dq_h2f((uint16_t)(w.h.x >> 16));
        const int isum = sca * da + scb * db;
        const int msum = mna * X.i0 + mnb * X.i1;
        return X.s0 * (d * (float)isum - dmin * (float)msum);
    }
};

// Q6_K (planes): item (s = i/4, n = (i/2)%2, k = i%2) = 48 bytes of plane Q,
// 4 scales of plane S, d of plane D. Activation bytes of the item:
// x[256s + 128n + 16k + 32*quarter + 0..15], quarter = 0..3.
template <>
struct Fmt<DQ_FMT_Q6_K> {
    static constexpr int NW = 3;
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
    __device__ static void load_w(W& w, const uint8_t* base, const DqLayout& L, size_t r, int i) {
        const uint8_t* q = base + L.q_off + r * L.q_row + 48 * (size_t)i;
        w.a = dq_ld16_stream(q);
        w.b = dq_ld16_stream(q + 16);
        w.h = dq_ld16_stream(q + 32);
        w.sc = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(base + L.s_off + r * L.s_row + 4 * (size_t)i));
        w.d = __builtin_nontemporal_load(reinterpret_cast<const uint16_t*>(base + L.d_off + r * L.d_row + 2 * (size_t)(i >> 2)));
    }
    __device__ static int q6dot(uint32_t lo4, uint32_t hi2, uint32_t x, int acc) {
        return dq_sdot4(dq_sub32_bytes((lo4 & 0x0F0F0F0Fu) | ((hi2 & 0x03030303u) << 4)), (int)x, acc);
    }
    __device__ static float dot(const W& w, const XItem& X) {
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

template <int FMT>
__device__ __forceinline__ float item_dot(const typename Fmt<FMT>::W& w, const XItem& X, int i) {
    if constexpr (FMT == DQ_FMT_Q4_K) return Fmt<FMT>::dot(w, X, i & 3);
    else return Fmt<FMT>::dot(w, X);
}

// ----------------------------------------------------------------- kernel --

template <int FMT, int R, int NIT>
__global__ __launch_bounds__(256) void gemv_kernel(const uint8_t* __restrict__ w, DqLayout L, int rows, int ipr,
                                                   const int8_t* __restrict__ xq, const float* __restrict__ xs,
                                                   const int32_t* __restrict__ xsum, float* __restrict__ y) {
    using F = Fmt<FMT>;
    const int lane = threadIdx.x & (DQ_WAVE - 1);
    const int wave = (int)((blockIdx.x * blockDim.x + threadIdx.x) / DQ_WAVE);
    const int r0 = wave * R;
    if (r0 >= rows) return;

    XItem X[NIT];
    bool on[NIT];
#pragma unroll
    for (int j = 0; j < NIT; ++j) {
        const int i = lane + DQ_WAVE * j;
        on[j] = i < ipr;
        F::load_x(X[j], on[j] ? i : ipr - 1, xq, xs, xsum);
    }

    typename F::W wr[R][NIT];
#pragma unroll
    for (int rr = 0; rr < R; ++rr) {
        const size_t r = (size_t)min(r0 + rr, rows - 1);
#pragma unroll
        for (int j = 0; j < NIT; ++j) {
            const int i = lane + DQ_WAVE * j;
            F::load_w(wr[rr][j], w, L, r, on[j] ? i : ipr - 1);
        }
    }

    float acc[R];
#pragma unroll
    for (int rr = 0; rr < R; ++rr) {
        float a = 0.0f;
#pragma unroll
        for (int j = 0; j < NIT; ++j) {
            const float p = item_dot<FMT>(wr[rr][j], X[j], lane + DQ_WAVE * j);
            a += on[j] ? p : 0.0f;
        }
        acc[rr] = a;
    }
#pragma unroll
    for (int rr = 0; rr < R; ++rr) {
        const float s = dq_wave_sum(acc[rr]);
        if (lane == rr && r0 + rr < rows) y[r0 + rr] = s;
    }
}

template <int FMT, int R>
int launch_r(const uint8_t* w, const DqLayout& L, int rows, int ipr, const int8_t* xq, const float* xs,
             const int32_t* xsum, float* y, hipStream_t s) {
    const int nit = (ipr + DQ_WAVE - 1) / DQ_WAVE;
    const int waves = (rows + R - 1) / R;
    const unsigned grid = (unsigned)((waves + 3) / 4);
    if (nit <= 1) gemv_kernel<FMT, R, 1><<<grid, 256, 0, s>>>(w, L, rows, ipr, xq, xs, xsum, y);
    else if (nit <= 2) gemv_kernel<FMT, R, 2><<<grid, 256, 0, s>>>(w, L, rows, ipr, xq, xs, xsum, y);
    else if (nit <= 4) gemv_kernel<FMT, R, 4><<<grid, 256, 0, s>>>(w, L, rows, ipr, xq, xs, xsum, y);
    else if (nit <= 8) gemv_kernel<FMT, R, 8><<<grid, 256, 0, s>>>(w, L, rows, ipr, xq, xs, xsum, y);
    else return DQ_ERR_NOT_SUPPORTED;
    return dq_launch_status();
}

// Rows per wave: enough loads in flight per wave, few enough registers.
int pick_r(int ipr) {
    static int forced = -1;
    if (forced < 0) {
        const char* e = getenv("DQ_GEMV_R");
        forced = e ? atoi(e) : 0;
    }
    if (forced == 1 || forced == 2 || forced == 4 || forced == 8) return forced;
    if (ipr <= 64) return 4;
    if (ipr <= 128) return 2;
    return 2;
}

template <int FMT>
int launch_fmt(const uint8_t* w, const DqLayout& L, int rows, int ipr, const int8_t* xq, const float* xs,
               const int32_t* xsum, float* y, hipStream_t s) {
    switch (pick_r(ipr)) {
    case 1: return launch_r<FMT, 1>(w, L, rows, ipr, xq, xs, xsum, y, s);
    case 2: return launch_r<FMT, 2>(w, L, rows, ipr, xq, xs, xsum, y, s);
    case 8: return launch_r<FMT, 8>(w, L, rows, ipr, xq, xs, xsum, y, s);
    default: return launch_r<FMT, 4>(w, L, rows, ipr, xq, xs, xsum, y, s);
    }
}

}  // namespace

extern "C" int dq_gemv(int fmt, const void* d_w, size_t rows, size_t cols, const int8_t* d_xq,
                       const float* d_xscale, const int32_t* d_xsum, float* d_y, void* stream) {
    DqLayout L;
    if (!dq_layout(fmt, rows, cols, &L)) return DQ_ERR_NOT_SUPPORTED;
    if (rows == 0) return DQ_OK;
    if (!d_w || !d_xq || !d_xscale || !d_y) return DQ_ERR_INVALID_ARG;
    if ((fmt == DQ_FMT_Q4_0 || fmt == DQ_FMT_Q4_K) && !d_xsum) return DQ_ERR_INVALID_ARG;
    if (rows > 0x7FFFFFFF) return DQ_ERR_NOT_SUPPORTED;
    const int ipr = (int)(cols / 64);
    const uint8_t* w = (const uint8_t*)d_w;
    hipStream_t s = (hipStream_t)stream;
    switch (fmt) {
    case DQ_FMT_Q8_0: return launch_fmt<DQ_FMT_Q8_0>(w, L, (int)rows, ipr, d_xq, d_xscale, d_xsum, d_y, s);
    case DQ_FMT_Q4_0: return launch_fmt<DQ_FMT_Q4_0>(w, L, (int)rows, ipr, d_xq, d_xscale, d_xsum, d_y, s);
    case DQ_FMT_Q4_K: return launch_fmt<DQ_FMT_Q4_K>(w, L, (int)rows, ipr, d_xq, d_xscale, d_xsum, d_y, s);
    case DQ_FMT_Q6_K: return launch_fmt<DQ_FMT_Q6_K>(w, L, (int)rows, ipr, d_xq, d_xscale, d_xsum, d_y, s);
    }
    return DQ_ERR_NOT_SUPPORTED;
}
