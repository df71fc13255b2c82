// dq_dequant.hip - GGUF block dequantization (bit-exact with the reference's
// dequantize_row_*) and the GGUF -> device layout conversion used at upload.
//
// Bit-exactness: fp16 -> fp32 is v_cvt_f32_f16 (exact); Q4_K's d1*q - m1 is a
// multiply then a subtract with two roundings, as quant/quant.cpp:269-270
// writes it - this file is compiled with -ffp-contract=off, so the compiler
// does not fuse them. Q6_K is (d*sc)*q (:532-535), Q4_0/Q8_0 one multiply.
#include "dq_common.h"

namespace {

__device__ __forceinline__ uint16_t rd16(const uint8_t* p) {
    return (uint16_t)(p[0] | ((uint16_t)p[1] << 8));
}

// quant/quant.cpp:22-29
__device__ __forceinline__ void scale_min_k4(int j, const uint8_t* q, int* sc, int* mn) {
    if (j < 4) {
        *sc = q[j] & 63;
        *mn = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *mn = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

// One lane per 32 outputs for every format.
__global__ __launch_bounds__(256) void dequant_q4_0_kernel(const uint8_t* __restrict__ x, float* __restrict__ y,
                                                           size_t nb) {
    const size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nb) return;
    const uint8_t* blk = x + b * DQ_SZ_Q4_0;
    const float d = dq_h2f(rd16(blk));
    float* o = y + b * 32;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const uint8_t v = blk[2 + j];
        o[j] = (float)((v & 0x0F) - 8) * d;
        o[j + 16] = (float)((v >> 4) - 8) * d;
    }
}

__global__ __launch_bounds__(256) void dequant_q8_kernel(const uint8_t* __restrict__ x, float* __restrict__ y,
                                                         size_t nb, int bsz, int qoff) {
    const size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nb) return;
    const uint8_t* blk = x + b * bsz;
    const float d = dq_h2f(rd16(blk));
    float* o = y + b * 32;
#pragma unroll
    for (int j = 0; j < 32; ++j) o[j] = (float)(int8_t)blk[qoff + j] * d;
}

__global__ __launch_bounds__(256) void dequant_q4_k_kernel(const uint8_t* __restrict__ x, float* __restrict__ y,
                                                           size_t n_sub) {
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n_sub) return;
    const size_t s = t / 8;
    const int j = (int)(t % 8);
    const uint8_t* blk = x + s * DQ_SZ_Q4_K;
    const float d = dq_h2f(rd16(blk));
    const float dmin = dq_h2f(rd16(blk + 2));
    int sc, mn;
    scale_min_k4(j, blk + 4, &sc, &mn);
    const float d1 = d * (float)sc;
    const float m1 = dmin * (float)mn;
    const uint8_t* q = blk + 16 + 32 * (j / 2);
    const int sh = 4 * (j & 1);
    float* o = y + t * 32;
#pragma unroll
    for (int l = 0; l < 32; ++l) o[l] = d1 * (float)((q[l] >> sh) & 0xF) - m1;
}

__global__ __launch_bounds__(256) void dequant_q6_k_kernel(const uint8_t* __restrict__ x, float* __restrict__ y,
                                                           size_t n_sub) {
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n_sub) return;
    const size_t s = t / 8;
    const int n = (int)((t % 8) / 4);   // 128-half
    const int qq = (int)(t % 4);        // quarter: outputs l + 32*qq
    const uint8_t* blk = x + s * DQ_SZ_Q6_K;
    const uint8_t* ql = blk + 64 * n + ((qq & 1) ? 32 : 0);
    const uint8_t* qh = blk + 128 + 32 * n;
    const int8_t* sc = (const int8_t*)(blk + 192 + 8 * n);
    const float d = dq_h2f(rd16(blk + 208));
    const int lsh = (qq >= 2) ? 4 : 0;
    const int hsh = 2 * qq;
    float* o = y + t * 32;
#pragma unroll
    for (int l = 0; l < 32; ++l) {
        const int q = (int)(((ql[l] >> lsh) & 0xF) | (((qh[l] >> hsh) & 3) << 4)) - 32;
        o[l] = d * (float)sc[l / 16 + 2 * qq] * (float)q;
    }
}

// ---------------------------------------------------------------- packing --
// Layouts: see dq_common.h. `ps` is the distance between quant sub-planes;
// PlaneRows maps a matrix-wide item index to its byte offset in a sub-plane
// (rows q_row bytes apart, ipr items per row).
struct PlaneRows {
    size_t ipr, q_row;
    __device__ size_t off(size_t item) const { return (item / ipr) * q_row + 16 * (item % ipr); }
};

__device__ __forceinline__ dq_u32x4 ld16_bytes(const uint8_t* src) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        w[i] = (uint32_t)src[4 * i] | ((uint32_t)src[4 * i + 1] << 8) | ((uint32_t)src[4 * i + 2] << 16) |
               ((uint32_t)src[4 * i + 3] << 24);
    return dq_u32x4{w[0], w[1], w[2], w[3]};
}

__global__ __launch_bounds__(256) void pack_q8_0_kernel(const uint8_t* __restrict__ x, uint8_t* __restrict__ qp,
                                                        size_t ps, PlaneRows pr, uint16_t* __restrict__ dp, size_t nb) {
    // one lane per block b: its halves go to sub-planes 2(b%2), 2(b%2)+1 of item b/2
    const size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nb) return;
    const uint8_t* blk = x + b * DQ_SZ_Q8_0;
    const size_t o = pr.off(b / 2), k = 2 * (b % 2);
    *reinterpret_cast<dq_u32x4*>(qp + k * ps + o) = ld16_bytes(blk + 2);
    *reinterpret_cast<dq_u32x4*>(qp + (k + 1) * ps + o) = ld16_bytes(blk + 18);
    dp[b] = rd16(blk);
}

__global__ __launch_bounds__(256) void pack_q4_0_kernel(const uint8_t* __restrict__ x, uint8_t* __restrict__ qp,
                                                        size_t ps, PlaneRows pr, uint16_t* __restrict__ dp, size_t nb) {
    const size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nb) return;
    const uint8_t* blk = x + b * DQ_SZ_Q4_0;
    *reinterpret_cast<dq_u32x4*>(qp + (b % 2) * ps + pr.off(b / 2)) = ld16_bytes(blk + 2);
    dp[b] = rd16(blk);
}

__global__ __launch_bounds__(256) void pack_q4_k_kernel(const uint8_t* __restrict__ x, uint8_t* __restrict__ qp,
                                                        size_t ps, PlaneRows pr, uint8_t* __restrict__ hp, size_t ns) {
    // one lane per 16-byte piece: 9 pieces per block (header + 8 qs pieces)
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= ns * 9) return;
    const size_t s = t / 9;
    const int p = (int)(t % 9);
    const dq_u32x4 v = ld16_bytes(x + s * DQ_SZ_Q4_K + 16 * p);
    if (p == 0) {
        *reinterpret_cast<dq_u32x4*>(hp + s * 16) = v;
    } else {
        const int q = p - 1, g = q / 2, k = q % 2;
        *reinterpret_cast<dq_u32x4*>(qp + (size_t)k * ps + pr.off(4 * s + g)) = v;
    }
}

__global__ __launch_bounds__(256) void pack_q6_k_kernel(const uint8_t* __restrict__ x, uint8_t* __restrict__ qp,
                                                        size_t ps, PlaneRows pr, uint8_t* __restrict__ sp,
                                                        uint16_t* __restrict__ dp, size_t ns) {
    // one lane per item t = 4s + it, it = 2n + k
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= ns * 4) return;
    const size_t s = t / 4;
    const int it = (int)(t % 4), n = it / 2, k = it % 2;
    const uint8_t* blk = x + s * DQ_SZ_Q6_K;
    const size_t o = pr.off(t);
    *reinterpret_cast<dq_u32x4*>(qp + o) = ld16_bytes(blk + 64 * n + 16 * k);
    *reinterpret_cast<dq_u32x4*>(qp + ps + o) = ld16_bytes(blk + 64 * n + 32 + 16 * k);
    *reinterpret_cast<dq_u32x4*>(qp + 2 * ps + o) = ld16_bytes(blk + 128 + 32 * n + 16 * k);
    for (int qq = 0; qq < 4; ++qq) sp[t * 4 + qq] = blk[192 + 8 * n + k + 2 * qq];
    if (it == 0) dp[s] = rd16(blk + 208);
}

// Dequantization from the device layout (same values as from GGUF blocks).
__global__ __launch_bounds__(256) void dequant_dev_q8_0_kernel(const uint8_t* __restrict__ qp, size_t ps,
                                                               PlaneRows pr, const uint16_t* __restrict__ dp,
                                                               float* __restrict__ y, size_t nb) {
    const size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nb) return;
    const float d = dq_h2f(dp[b]);
    const size_t o = pr.off(b / 2), k = 2 * (b % 2);
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        y[b * 32 + j] = (float)(int8_t)qp[k * ps + o + j] * d;
        y[b * 32 + 16 + j] = (float)(int8_t)qp[(k + 1) * ps + o + j] * d;
    }
}

__global__ __launch_bounds__(256) void dequant_dev_q4_0_kernel(const uint8_t* __restrict__ qp, size_t ps,
                                                               PlaneRows pr, const uint16_t* __restrict__ dp,
                                                               float* __restrict__ y, size_t nb) {
    const size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nb) return;
    const float d = dq_h2f(dp[b]);
    const uint8_t* q = qp + (b % 2) * ps + pr.off(b / 2);
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const uint8_t v = q[j];
        y[b * 32 + j] = (float)((v & 0x0F) - 8) * d;
        y[b * 32 + j + 16] = (float)((v >> 4) - 8) * d;
    }
}

__global__ __launch_bounds__(256) void dequant_dev_q4_k_kernel(const uint8_t* __restrict__ qp, size_t ps,
                                                               PlaneRows pr, const uint8_t* __restrict__ hp,
                                                               float* __restrict__ y, size_t n_sub) {
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n_sub) return;
    const size_t s = t / 8;
    const int j = (int)(t % 8), g = j / 2;
    const uint8_t* h = hp + s * 16;
    const float d = dq_h2f(rd16(h));
    const float dmin = dq_h2f(rd16(h + 2));
    int sc, mn;
    scale_min_k4(j, h + 4, &sc, &mn);
    const float d1 = d * (float)sc;
    const float m1 = dmin * (float)mn;
    const int sh = 4 * (j & 1);
    float* o = y + t * 32;
#pragma unroll
    for (int l = 0; l < 32; ++l) {
        const uint8_t v = qp[(size_t)(l / 16) * ps + pr.off(4 * s + g) + (l % 16)];
        o[l] = d1 * (float)((v >> sh) & 0xF) - m1;
    }
}

__global__ __launch_bounds__(256) void dequant_dev_q6_k_kernel(const uint8_t* __restrict__ qp, size_t ps,
                                                               PlaneRows pr, const int8_t* __restrict__ sp,
                                                               const uint16_t* __restrict__ dp,
                                                               float* __restrict__ y, size_t n_items) {
    // one lane per item (n,k): 64 outputs at 128n + 16k + {0..15} + 32*quarter
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n_items) return;
    const size_t s = t / 4;
    const int it = (int)(t % 4), n = it / 2, k = it % 2;
    const int8_t* sc = sp + t * 4;
    const float d = dq_h2f(dp[s]);
    float* o = y + s * 256 + 128 * n + 16 * k;
    const size_t qo = pr.off(t);
    for (int tt = 0; tt < 16; ++tt) {
        const uint8_t a = qp[qo + tt], b = qp[ps + qo + tt], h = qp[2 * ps + qo + tt];
        const int q1 = (int)((a & 0xF) | (((h >> 0) & 3) << 4)) - 32;
        const int q2 = (int)((b & 0xF) | (((h >> 2) & 3) << 4)) - 32;
        const int q3 = (int)((a >> 4) | (((h >> 4) & 3) << 4)) - 32;
        const int q4 = (int)((b >> 4) | (((h >> 6) & 3) << 4)) - 32;
        o[tt] = d * (float)sc[0] * (float)q1;
        o[tt + 32] = d * (float)sc[1] * (float)q2;
        o[tt + 64] = d * (float)sc[2] * (float)q3;
        o[tt + 96] = d * (float)sc[3] * (float)q4;
    }
}

inline unsigned grid_for(size_t n) { return (unsigned)((n + 255) / 256); }

}  // namespace

extern "C" int dq_dequantize_row(int type, const void* d_src, float* d_dst, int64_t n, void* stream) {
    if (n < 0) return DQ_ERR_INVALID_ARG;
    hipStream_t s = (hipStream_t)stream;
    const uint8_t* x = (const uint8_t*)d_src;
    switch (type) {
    case DQ_TYPE_Q4_0:
    case DQ_TYPE_Q8_0:
    case DQ_TYPE_Q8_1: {
        if (n % 32) return DQ_ERR_INVALID_ARG;
        if (n == 0) return DQ_OK;
        if (!d_src || !d_dst) return DQ_ERR_INVALID_ARG;
        const size_t nb = (size_t)n / 32;
        if (type == DQ_TYPE_Q4_0) dequant_q4_0_kernel<<<grid_for(nb), 256, 0, s>>>(x, d_dst, nb);
        else if (type == DQ_TYPE_Q8_0) dequant_q8_kernel<<<grid_for(nb), 256, 0, s>>>(x, d_dst, nb, DQ_SZ_Q8_0, 2);
        else dequant_q8_kernel<<<grid_for(nb), 256, 0, s>>>(x, d_dst, nb, DQ_SZ_Q8_1, 4);
        return dq_launch_status();
    }
    case DQ_TYPE_Q4_K:
    case DQ_TYPE_Q6_K: {
        if (n % 256) return DQ_ERR_INVALID_ARG;
        if (n == 0) return DQ_OK;
        if (!d_src || !d_dst) return DQ_ERR_INVALID_ARG;
        const size_t nsub = (size_t)n / 32;
        if (type == DQ_TYPE_Q4_K) dequant_q4_k_kernel<<<grid_for(nsub), 256, 0, s>>>(x, d_dst, nsub);
        else dequant_q6_k_kernel<<<grid_for(nsub), 256, 0, s>>>(x, d_dst, nsub);
        return dq_launch_status();
    }
    default:
        return DQ_ERR_NOT_SUPPORTED;
    }
}

extern "C" int dq_weights_bytes(int fmt, size_t rows, size_t cols, size_t* bytes) {
    DqLayout L;
    if (!bytes) return DQ_ERR_INVALID_ARG;
    if (!dq_layout(fmt, rows, cols, &L)) return DQ_ERR_NOT_SUPPORTED;
    *bytes = L.total;
    return DQ_OK;
}

extern "C" int dq_weights_pack(int fmt, const void* d_gguf, size_t rows, size_t cols, void* d_dev,
                               void* stream) {
    DqLayout L;
    if (!dq_layout(fmt, rows, cols, &L)) return DQ_ERR_NOT_SUPPORTED;
    if (!d_gguf || !d_dev) return DQ_ERR_INVALID_ARG;
    if (rows == 0) return DQ_OK;
    hipStream_t s = (hipStream_t)stream;
    const uint8_t* x = (const uint8_t*)d_gguf;
    uint8_t* base = (uint8_t*)d_dev;
    const PlaneRows pr{cols / 64, L.q_row};
    switch (fmt) {
    case DQ_FMT_Q8_0: {
        const size_t nb = rows * cols / 32;
        pack_q8_0_kernel<<<grid_for(nb), 256, 0, s>>>(x, base + L.q_off, L.p_stride, pr, (uint16_t*)(base + L.d_off), nb);
        break;
    }
    case DQ_FMT_Q4_0: {
        const size_t nb = rows * cols / 32;
        pack_q4_0_kernel<<<grid_for(nb), 256, 0, s>>>(x, base + L.q_off, L.p_stride, pr, (uint16_t*)(base + L.d_off), nb);
        break;
    }
    case DQ_FMT_Q4_K: {
        const size_t ns = rows * cols / 256;
        pack_q4_k_kernel<<<grid_for(ns * 9), 256, 0, s>>>(x, base + L.q_off, L.p_stride, pr, base + L.s_off, ns);
        break;
    }
    case DQ_FMT_Q6_K: {
        const size_t ns = rows * cols / 256;
        pack_q6_k_kernel<<<grid_for(ns * 4), 256, 0, s>>>(x, base + L.q_off, L.p_stride, pr, base + L.s_off,
                                                          (uint16_t*)(base + L.d_off), ns);
        break;
    }
    }
    return dq_launch_status();
}

extern "C" int dq_weights_dequantize(int fmt, const void* d_dev, size_t rows, size_t cols, float* d_out,
                                     void* stream) {
    DqLayout L;
    if (!dq_layout(fmt, rows, cols, &L)) return DQ_ERR_NOT_SUPPORTED;
    if (!d_dev || !d_out) return DQ_ERR_INVALID_ARG;
    if (rows == 0) return DQ_OK;
    hipStream_t s = (hipStream_t)stream;
    const uint8_t* base = (const uint8_t*)d_dev;
    const PlaneRows pr{cols / 64, L.q_row};
    switch (fmt) {
    case DQ_FMT_Q8_0: {
        const size_t nb = rows * cols / 32;
        dequant_dev_q8_0_kernel<<<grid_for(nb), 256, 0, s>>>(base + L.q_off, L.p_stride, pr,
                                                             (const uint16_t*)(base + L.d_off), d_out, nb);
        break;
    }
    case DQ_FMT_Q4_0: {
        const size_t nb = rows * cols / 32;
        dequant_dev_q4_0_kernel<<<grid_for(nb), 256, 0, s>>>(base + L.q_off, L.p_stride, pr,
                                                             (const uint16_t*)(base + L.d_off), d_out, nb);
        break;
    }
    case DQ_FMT_Q4_K: {
        const size_t nsub = rows * cols / 32;
        dequant_dev_q4_k_kernel<<<grid_for(nsub), 256, 0, s>>>(base + L.q_off, L.p_stride, pr, base + L.s_off, d_out,
                                                               nsub);
        break;
    }
    case DQ_FMT_Q6_K: {
        const size_t ni = rows * cols / 64;
        dequant_dev_q6_k_kernel<<<grid_for(ni), 256, 0, s>>>(base + L.q_off, L.p_stride, pr,
                                                             (const int8_t*)(base + L.s_off),
                                                             (const uint16_t*)(base + L.d_off), d_out, ni);
        break;
    }
    }
    return dq_launch_status();
}
