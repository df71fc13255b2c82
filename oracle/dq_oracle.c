/*
 * dq_oracle.c - CPU restatement of DesireeIA's quantized-weight compute path.
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT CODE: it is the checker the HIP library is
 * compared against, and the "port" CPU baseline bench.py may time. Nothing in
 * desireeia_amd/ links or calls it.
 *
 * Semantics follow the reference as compiled for x86-64 with AVX2 (the path
 * the engine actually runs on an x86 host): integer partial sums are exact, and
 * where the reference's float order is cheap to state (GEMM fma chain, KV dot,
 * RMS norm) it is stated exactly. Build with -ffp-contract=off so the only
 * fused multiply-adds are the explicit fmaf() calls, which mirror the explicit
 * _mm256_fmadd_ps of the reference. Reference paths below are relative to
 * src/DesireeIA.LocaleEngine/.
 */
#include "dq_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* fp16 <-> fp32: quant/quant.h:285-323 (desireeia_compute_fp16_to_fp32 /   */
/* desireeia_compute_fp32_to_fp16). Restated from IEEE-754 field arithmetic */
/* instead of the reference's magic-constant float tricks; results are the  */
/* same bits for every input (NaN: quiet bit set, payload kept, as the      */
/* reference's multiply by 2^-112 does on x86).                             */
/* ------------------------------------------------------------------------ */
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float dqo_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu;
    const uint32_t m = h & 0x3FFu;
    if (e == 0) {
        /* zero / subnormal: m * 2^-24, exact in fp32 */
        const float v = (float)m * 5.9604644775390625e-08f;
        return u2f(f2u(v) | sign);
    }
    if (e == 31) {
        return u2f(sign | 0x7F800000u | (m << 13) | (m ? 0x00400000u : 0u));
    }
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

uint16_t dqo_fp32_to_fp16(float f) {
    const uint32_t x = f2u(f);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax > 0x7F800000u) return sign | 0x7E00u;           /* NaN */
    if (ax >= 0x477FF000u) return sign | 0x7C00u;          /* >= 65520: inf */
    if (ax < 0x38800000u) {                                /* < 2^-14 */
        const float v = u2f(ax) * 16777216.0f;             /* exact scaling */
        return sign | (uint16_t)rintf(v);                  /* RNE */
    }
    uint32_t hbits = (((ax >> 23) - 112u) << 10) | ((ax >> 13) & 0x3FFu);
    const uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (hbits & 1u))) hbits++;
    return sign | (uint16_t)hbits;
}

/* ------------------------------------------------------------------------ */
/* Block layouts: quant/quant.h:41-46 (q4_0, 18 B), :98-103 (q8_0, 34 B),   */
/* :105-116 (q8_1, 36 B), :154-165 (q4_K, 144 B), :181-187 (q6_K, 210 B).   */
/* Accessed by byte offset (all little-endian fp16 fields).                 */
/* ------------------------------------------------------------------------ */
#define QK 32
#define QKK 256
#define SZ_Q4_0 18
#define SZ_Q8_0 34
#define SZ_Q8_1 36
#define SZ_Q4_K 144
#define SZ_Q6_K 210

static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* quant/quant.cpp:839-910 */
size_t dqo_type_size(int type) {
    switch (type) {
    case DQO_Q4_0: return SZ_Q4_0;
    case DQO_Q8_0: return SZ_Q8_0;
    case DQO_Q8_1: return SZ_Q8_1;
    case DQO_Q4_K: return SZ_Q4_K;
    case DQO_Q6_K: return SZ_Q6_K;
    default: return 0;
    }
}
int dqo_blck_size(int type) {
    return (type == DQO_Q4_K || type == DQO_Q6_K) ? QKK : QK;
}
size_t dqo_row_size(int type, int64_t n) {
    const int b = dqo_blck_size(type);
    return (size_t)((n / b + (n % b ? 1 : 0)) * (int64_t)dqo_type_size(type));
}

/* quant/quant.cpp:22-29 get_scale_min_k4 */
void dqo_get_scale_min_k4(int j, const uint8_t* q, uint8_t* sc, uint8_t* mn) {
    if (j < 4) {
        *sc = q[j] & 63;
        *mn = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *mn = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* quant/quant.cpp:287-293 pack_scales_min_k4 (inverse of the above) */
void dqo_pack_scales_min_k4(const uint8_t* sc, const uint8_t* mn, uint8_t* out) {
    for (int i = 0; i < 4; ++i) {
        out[i] = (uint8_t)((sc[i] & 63) | ((sc[i + 4] >> 4) << 6));
        out[i + 4] = (uint8_t)((mn[i] & 63) | ((mn[i + 4] >> 4) << 6));
        out[i + 8] = (uint8_t)((sc[i + 4] & 0xF) | ((mn[i + 4] & 0xF) << 4));
    }
}

/* quant/quant.cpp:62-75 */
static void deq_q4_0(const uint8_t* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n / QK; ++i) {
        const uint8_t* b = x + i * SZ_Q4_0;
        const float d = dqo_fp16_to_fp32(rd16(b));
        for (int j = 0; j < 16; ++j) {
            const int x0 = (b[2 + j] & 0x0F) - 8;
            const int x1 = (b[2 + j] >> 4) - 8;
            y[i * QK + j] = x0 * d;
            y[i * QK + j + 16] = x1 * d;
        }
    }
}

/* quant/quant.cpp:132-142 (Q8_0) and :179-189 (Q8_1, the s field unused) */
static void deq_q8(const uint8_t* x, float* y, int64_t n, int bsz, int qoff) {
    for (int64_t i = 0; i < n / QK; ++i) {
        const uint8_t* b = x + i * bsz;
        const float d = dqo_fp16_to_fp32(rd16(b));
        for (int j = 0; j < QK; ++j) y[i * QK + j] = (float)(int8_t)b[qoff + j] * d;
    }
}

/* quant/quant.cpp:255-273: y = d1*q - m1, a multiply and a subtract, two
 * roundings (the oracle is built with -ffp-contract=off). */
static void deq_q4_k(const uint8_t* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n / QKK; ++i) {
        const uint8_t* b = x + i * SZ_Q4_K;
        const float d = dqo_fp16_to_fp32(rd16(b));
        const float mn = dqo_fp16_to_fp32(rd16(b + 2));
        const uint8_t* scales = b + 4;
        const uint8_t* q = b + 16;
        int is = 0;
        for (int j = 0; j < QKK; j += 64) {
            uint8_t sc, m;
            dqo_get_scale_min_k4(is + 0, scales, &sc, &m);
            const float d1 = d * sc, m1 = mn * m;
            dqo_get_scale_min_k4(is + 1, scales, &sc, &m);
            const float d2 = d * sc, m2 = mn * m;
            for (int l = 0; l < 32; ++l) *y++ = d1 * (q[l] & 0xF) - m1;
            for (int l = 0; l < 32; ++l) *y++ = d2 * (q[l] >> 4) - m2;
            q += 32;
            is += 2;
        }
    }
}

/* quant/quant.cpp:517-543: y = (d*sc)*q, q = 6-bit value - 32 */
static void deq_q6_k(const uint8_t* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n / QKK; ++i) {
        const uint8_t* b = x + i * SZ_Q6_K;
        const uint8_t* ql = b;
        const uint8_t* qh = b + 128;
        const int8_t* sc = (const int8_t*)(b + 192);
        const float d = dqo_fp16_to_fp32(rd16(b + 208));
        for (int nn = 0; nn < QKK; nn += 128) {
            for (int l = 0; l < 32; ++l) {
                const int is = l / 16;
                const int q1 = (int)((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                const int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                const int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                const int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                y[l + 0] = d * sc[is + 0] * q1;
                y[l + 32] = d * sc[is + 2] * q2;
                y[l + 64] = d * sc[is + 4] * q3;
                y[l + 96] = d * sc[is + 6] * q4;
            }
            y += 128;
            ql += 64;
            qh += 32;
            sc += 8;
        }
    }
}

/* quant/quant.cpp:912-984 desireeia_dequantize_row (on-path types only) */
int dqo_dequantize_row(int type, const void* src, float* dst, int64_t n) {
    const uint8_t* x = (const uint8_t*)src;
    if (n < 0) return DQO_ERR_INVALID_ARG;
    switch (type) {
    case DQO_Q4_0: deq_q4_0(x, dst, n); return DQO_OK;
    case DQO_Q8_0: deq_q8(x, dst, n, SZ_Q8_0, 2); return DQO_OK;
    case DQO_Q8_1: deq_q8(x, dst, n, SZ_Q8_1, 4); return DQO_OK;
    case DQO_Q4_K: deq_q4_k(x, dst, n); return DQO_OK;
    case DQO_Q6_K: deq_q6_k(x, dst, n); return DQO_OK;
    default: return DQO_ERR_NOT_SUPPORTED;
    }
}

/* ------------------------------------------------------------------------ */
/* Activation quantizers                                                    */
/* ------------------------------------------------------------------------ */

/* x * id rounded to nearest-even and clamped to +-127. For every block
 * whose maximum |x| is at least 127 / FLT_MAX (about 3.7e-37) x * id is
 * finite and this is the reference's clamp(lrintf(x * id)). Below that
 * (and above the point where d rounds to 0) id overflows to inf and the
 * reference's conversion of +-inf / NaN is not defined by its source: its
 * AVX2 build packs the integer-indefinite value into -128 for every element
 * and its scalar path is undefined behaviour. Here, as on the GPU, the
 * conversion saturates: +-inf -> +-127, NaN (x = 0) -> 0. */
static inline long rint_sat127(float v) {
    if (v != v) return 0;
    if (v >= 127.0f) return 127;
    if (v <= -127.0f) return -127;
    return lrintf(v);
}

/* Per-32 recipe, core/quant.cpp:15-50 (quantize_q8_0): amax, d = amax/127,
 * id = 1/d, q = clamp(lrintf(x*id), +-127). */
void dqo_quantize_q8_0(const float* x, size_t n, int8_t* q, float* dout) {
    for (size_t b = 0; b < n / QK; ++b) {
        const float* p = x + b * QK;
        float vmax = 0.0f;
        for (int i = 0; i < QK; ++i) {
            const float a = fabsf(p[i]);
            vmax = (vmax < a) ? a : vmax; /* std::max(vmax, a) */
        }
        const float d = vmax > 0.0f ? vmax / 127.0f : 0.0f;
        const float id = d > 0.0f ? 1.0f / d : 0.0f;
        dout[b] = d;
        for (int i = 0; i < QK; ++i) {
            q[b * QK + i] = (int8_t)rint_sat127(p[i] * id);
        }
    }
}

/* Per-32 with sums: the integers of quantize_q8_0, the int32 sum of q
 * (backend_cuda.cu:187-214 keeps it for the GPU kernels) and the exact
 * sequential float sum of the 32 inputs (core/i8gemm_impl.h:50-82,
 * quantize_row_vec, used by the prefill GEMM's min term). */
void dqo_quantize_q8_1(const float* x, size_t n, int8_t* q, float* d,
                       int32_t* isum, float* fsum) {
    dqo_quantize_q8_0(x, n, q, d);
    for (size_t b = 0; b < n / QK; ++b) {
        int32_t s = 0;
        float fs = 0.0f;
        for (int i = 0; i < QK; ++i) {
            s += q[b * QK + i];
            fs += x[b * QK + i];
        }
        if (isum) isum[b] = s;
        if (fsum) fsum[b] = fs;
    }
}

/* Per-256 replicated, core/matmul.cpp:1660-1778 (quantize_act_q8k_rep):
 * d = amax/127 but id = 127/amax; the scale is replicated into the 8 per-32
 * slots and the per-32 int32 sums of q are kept. */
void dqo_quantize_q8k_rep(const float* x, size_t n, int8_t* q, float* d32, int32_t* isum32) {
    for (size_t s = 0; s < n / QKK; ++s) {
        const float* xs = x + s * QKK;
        float amax = 0.0f;
        for (int j = 0; j < QKK; ++j) {
            const float a = fabsf(xs[j]);
            amax = (amax < a) ? a : amax;
        }
        const float d = amax > 0.0f ? amax / 127.0f : 0.0f;
        const float id = d > 0.0f ? 127.0f / amax : 0.0f;
        for (int j = 0; j < QKK; ++j) {
            q[s * QKK + j] = (int8_t)rint_sat127(xs[j] * id);
        }
        for (int sb = 0; sb < 8; ++sb) {
            int32_t acc = 0;
            for (int j = 0; j < 32; ++j) acc += q[s * QKK + sb * 32 + j];
            d32[s * 8 + sb] = d;
            if (isum32) isum32[s * 8 + sb] = acc;
        }
    }
}

/* kv/kv_quant.cpp:31-56: the per-32 recipe with the scale stored as fp16. */
void dqo_kv_quantize_row(const float* x, size_t dim, uint8_t* out) {
    for (size_t b = 0; b < (dim + 31) / 32; ++b) {
        const size_t start = b * 32;
        const size_t len = (dim - start) < 32 ? (dim - start) : 32;
        float amax = 0.0f;
        for (size_t i = 0; i < len; ++i) {
            const float a = fabsf(x[start + i]);
            if (a > amax) amax = a;
        }
        const float d = amax > 0.0f ? amax / 127.0f : 0.0f;
        const float id = d > 0.0f ? 1.0f / d : 0.0f;
        uint8_t* blk = out + b * SZ_Q8_0;
        const uint16_t h = dqo_fp32_to_fp16(d);
        blk[0] = (uint8_t)(h & 0xFF);
        blk[1] = (uint8_t)(h >> 8);
        for (size_t i = 0; i < 32; ++i) {
            long v = 0;
            if (i < len) v = rint_sat127(x[start + i] * id);
            blk[2 + i] = (uint8_t)(int8_t)v;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* GEMV                                                                     */
/* ------------------------------------------------------------------------ */

/* Exact int dot of one 32-block of weights (already int) with x_q. */
static inline int32_t idot32(const int8_t* w, const int8_t* x) {
    int32_t s = 0;
    for (int j = 0; j < 32; ++j) s += (int32_t)w[j] * (int32_t)x[j];
    return s;
}

/* One Q4_K super-block dot (core/matmul.cpp:1833-1953, AVX2 branch):
 * min_acc -= dmin*m_j*dx*xsum_j for j = 0..7 (float, in order), isum =
 * sum_j sc_j*dot_j in int32, acc = d*dx*float(isum), returns acc + min_acc.
 * isum_out/msum_out receive the integer partials for the fp64 twin. */
static float q4k_super_dot(const uint8_t* blk, const int8_t* xq, const float* xscale,
                           const int32_t* xsum, int64_t* isum_out, int64_t* msum_out) {
    const float d = dqo_fp16_to_fp32(rd16(blk));
    const float dmin = dqo_fp16_to_fp32(rd16(blk + 2));
    const uint8_t* scales = blk + 4;
    const uint8_t* q = blk + 16;
    const float dx = xscale[0];
    float min_acc = 0.0f;
    uint8_t sc8[8];
    int64_t msum = 0;
    for (int i = 0; i < 8; ++i) {
        uint8_t sc, m;
        dqo_get_scale_min_k4(i, scales, &sc, &m);
        sc8[i] = sc;
        min_acc -= dmin * (float)m * dx * (float)xsum[i];
        msum += (int64_t)m * xsum[i];
    }
    int64_t isum = 0;
    for (int g = 0; g < 4; ++g) {
        int32_t da = 0, db = 0;
        for (int l = 0; l < 32; ++l) {
            da += (int32_t)(q[l] & 0x0F) * xq[g * 64 + l];
            db += (int32_t)(q[l] >> 4) * xq[g * 64 + 32 + l];
        }
        isum += (int64_t)sc8[2 * g] * da + (int64_t)sc8[2 * g + 1] * db;
        q += 32;
    }
    if (isum_out) *isum_out = isum;
    if (msum_out) *msum_out = msum;
    const float acc = d * dx * (float)isum;
    return acc + min_acc;
}

/* One Q6_K super-block integer dot (core/matmul.cpp:2287-2319 q6k_group128):
 * sum over the 16 groups of 16 of sc * sum (q6-32)*x_q. */
static int64_t q6k_super_isum(const uint8_t* blk, const int8_t* xq) {
    const uint8_t* ql = blk;
    const uint8_t* qh = blk + 128;
    const int8_t* sc = (const int8_t*)(blk + 192);
    int64_t isum = 0;
    for (int nn = 0; nn < 2; ++nn) {
        for (int qq = 0; qq < 4; ++qq) {
            for (int half = 0; half < 2; ++half) {
                int32_t dot = 0;
                for (int t = 0; t < 16; ++t) {
                    const int l = half * 16 + t;
                    int v;
                    switch (qq) {
                    case 0: v = (ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4); break;
                    case 1: v = (ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4); break;
                    case 2: v = (ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4); break;
                    default: v = (ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4); break;
                    }
                    dot += (v - 32) * (int32_t)xq[nn * 128 + qq * 32 + l];
                }
                isum += (int64_t)sc[qq * 2 + half] * dot;
            }
        }
        ql += 64;
        qh += 32;
        sc += 8;
    }
    return isum;
}

static void unpack_q4_0_block(const uint8_t* b, int8_t* w) {
    for (int j = 0; j < 16; ++j) {
        w[j] = (int8_t)((b[2 + j] & 0x0F) - 8);
        w[j + 16] = (int8_t)((b[2 + j] >> 4) - 8);
    }
}

/* GEMV on pre-quantized activations. Q8_0/Q4_0: core/matmul.cpp:294-417,
 * acc += wd*xs*float(dot) per 32-block. Q4_K: :1827-2021 (matmul_q4_k_core).
 * Q6_K: :2389-2578 (matmul_q6_k_core), acc += d*dx*float(isum) per 256. */
int dqo_matmul_pq(int type, const uint8_t* w, size_t rows, size_t cols,
                  const int8_t* xq, const float* d32, const int32_t* isum32,
                  float* y, size_t row0, size_t row1) {
    if (row1 == 0) row1 = rows;
    const size_t nb = cols / QK, ns = cols / QKK;
    switch (type) {
    case DQO_Q8_0:
    case DQO_Q4_0: {
        const size_t bsz = type == DQO_Q8_0 ? SZ_Q8_0 : SZ_Q4_0;
        for (size_t r = row0; r < row1; ++r) {
            const uint8_t* row = w + r * nb * bsz;
            float acc = 0.0f;
            for (size_t b = 0; b < nb; ++b) {
                const uint8_t* blk = row + b * bsz;
                const float wd = dqo_fp16_to_fp32(rd16(blk));
                int8_t wq[32];
                if (type == DQO_Q8_0) memcpy(wq, blk + 2, 32);
                else unpack_q4_0_block(blk, wq);
                const float dot = (float)idot32(wq, xq + b * QK);
                acc += wd * d32[b] * dot;
            }
            y[r] = acc;
        }
        return DQO_OK;
    }
    case DQO_Q4_K:
        for (size_t r = row0; r < row1; ++r) {
            const uint8_t* row = w + r * ns * SZ_Q4_K;
            float acc = 0.0f;
            for (size_t s = 0; s < ns; ++s)
                acc += q4k_super_dot(row + s * SZ_Q4_K, xq + s * QKK, d32 + s * 8,
                                     isum32 + s * 8, NULL, NULL);
            y[r] = acc;
        }
        return DQO_OK;
    case DQO_Q6_K:
        for (size_t r = row0; r < row1; ++r) {
            const uint8_t* row = w + r * ns * SZ_Q6_K;
            float acc = 0.0f;
            for (size_t s = 0; s < ns; ++s) {
                const uint8_t* blk = row + s * SZ_Q6_K;
                const float d = dqo_fp16_to_fp32(rd16(blk + 208));
                const float dx = d32[s * 8];
                acc += d * dx * (float)q6k_super_isum(blk, xq + s * QKK);
            }
            y[r] = acc;
        }
        return DQO_OK;
    default:
        return DQO_ERR_NOT_SUPPORTED;
    }
}

static int gemv_cols_ok(int type, size_t cols) {
    if (cols == 0) return 0;
    if (type == DQO_Q4_K || type == DQO_Q6_K) return cols % QKK == 0;
    return cols % QK == 0;
}

/* matmul_q8_0 / matmul_q4_0 quantize x per 32 (core/matmul.cpp:304,353);
 * matmul_q4_k / matmul_q6_k per 256 replicated (:2018, :2575). */
int dqo_matmul(int type, const uint8_t* w, size_t rows, size_t cols,
               const float* x, float* y, size_t row0, size_t row1) {
    if (!gemv_cols_ok(type, cols)) return DQO_ERR_NOT_SUPPORTED;
    const size_t nb = cols / QK;
    int8_t* xq = (int8_t*)malloc(cols);
    float* d32 = (float*)malloc(nb * sizeof(float));
    int32_t* is = (int32_t*)malloc(nb * sizeof(int32_t));
    if (type == DQO_Q8_0 || type == DQO_Q4_0) dqo_quantize_q8_0(x, cols, xq, d32);
    else dqo_quantize_q8k_rep(x, cols, xq, d32, is);
    const int rc = dqo_matmul_pq(type, w, rows, cols, xq, d32, is, y, row0, row1);
    free(xq);
    free(d32);
    free(is);
    return rc;
}

/* The same formula on the same integers, accumulated in double. */
int dqo_matmul_f64(int type, const uint8_t* w, size_t rows, size_t cols,
                   const float* x, double* y, size_t row0, size_t row1) {
    if (!gemv_cols_ok(type, cols)) return DQO_ERR_NOT_SUPPORTED;
    if (row1 == 0) row1 = rows;
    const size_t nb = cols / QK, ns = cols / QKK;
    int8_t* xq = (int8_t*)malloc(cols);
    float* d32 = (float*)malloc(nb * sizeof(float));
    int32_t* is = (int32_t*)malloc(nb * sizeof(int32_t));
    if (type == DQO_Q8_0 || type == DQO_Q4_0) dqo_quantize_q8_0(x, cols, xq, d32);
    else dqo_quantize_q8k_rep(x, cols, xq, d32, is);
    for (size_t r = row0; r < row1; ++r) {
        double acc = 0.0;
        if (type == DQO_Q8_0 || type == DQO_Q4_0) {
            const size_t bsz = type == DQO_Q8_0 ? SZ_Q8_0 : SZ_Q4_0;
            for (size_t b = 0; b < nb; ++b) {
                const uint8_t* blk = w + (r * nb + b) * bsz;
                int8_t wq[32];
                if (type == DQO_Q8_0) memcpy(wq, blk + 2, 32);
                else unpack_q4_0_block(blk, wq);
                acc += (double)dqo_fp16_to_fp32(rd16(blk)) * d32[b] * idot32(wq, xq + b * QK);
            }
        } else if (type == DQO_Q4_K) {
            for (size_t s = 0; s < ns; ++s) {
                const uint8_t* blk = w + (r * ns + s) * SZ_Q4_K;
                int64_t isum, msum;
                q4k_super_dot(blk, xq + s * QKK, d32 + s * 8, is + s * 8, &isum, &msum);
                acc += (double)d32[s * 8] * ((double)dqo_fp16_to_fp32(rd16(blk)) * (double)isum -
                                             (double)dqo_fp16_to_fp32(rd16(blk + 2)) * (double)msum);
            }
        } else {
            for (size_t s = 0; s < ns; ++s) {
                const uint8_t* blk = w + (r * ns + s) * SZ_Q6_K;
                acc += (double)dqo_fp16_to_fp32(rd16(blk + 208)) * d32[s * 8] *
                       (double)q6k_super_isum(blk, xq + s * QKK);
            }
        }
        y[r] = acc;
    }
    free(xq);
    free(d32);
    free(is);
    return DQO_OK;
}

/* ------------------------------------------------------------------------ */
/* Prefill GEMM: i8_gemm semantics (core/matmul.cpp:505-638 unpack_row,      */
/* :806-845 i8_gemm, core/i8gemm_impl.h:50-82 quantize_row_vec and :326-419 */
/* kernel4). Per row r, token t and 32-block b:                             */
/*   f = fma(float(I_b), a_rb*dx_tb, f)            (one half, Q8_0/Q4_0/Q4_K) */
/*   f = fma(float(I_bh), a_rbh*dx_tb, f), h=0,1    (Q6_K, per-16 scales)    */
/*   f = fma(-m_rb, sx_tb, f)                       (Q4_K min term)          */
/* where I is the exact integer dot of the unpacked weights with x_q.       */
/* Below 4 tokens (kI8MinTokens, :849) the per-token GEMV is used instead.  */
/* ------------------------------------------------------------------------ */
typedef struct {
    int8_t* q;  /* [cols] */
    float* a;   /* [2*nb] scale of each 16 */
    float* m;   /* [2*nb] offset of each 16 (Q4_K) */
} unpacked_row;

/* core/matmul.cpp:505-638 unpack_row */
static void unpack_row(int type, const uint8_t* row, size_t cols, unpacked_row* u) {
    const size_t nb = cols / QK;
    switch (type) {
    case DQO_Q8_0:
        for (size_t b = 0; b < nb; ++b) {
            const uint8_t* blk = row + b * SZ_Q8_0;
            memcpy(u->q + b * 32, blk + 2, 32);
            u->a[2 * b] = u->a[2 * b + 1] = dqo_fp16_to_fp32(rd16(blk));
        }
        break;
    case DQO_Q4_0:
        for (size_t b = 0; b < nb; ++b) {
            const uint8_t* blk = row + b * SZ_Q4_0;
            unpack_q4_0_block(blk, u->q + b * 32);
            u->a[2 * b] = u->a[2 * b + 1] = dqo_fp16_to_fp32(rd16(blk));
        }
        break;
    case DQO_Q4_K:
        for (size_t i = 0; i < cols / QKK; ++i) {
            const uint8_t* blk = row + i * SZ_Q4_K;
            const float d = dqo_fp16_to_fp32(rd16(blk));
            const float dmin = dqo_fp16_to_fp32(rd16(blk + 2));
            const uint8_t* ql = blk + 16;
            for (int j = 0; j < 4; ++j) {
                const size_t b0 = i * 8 + 2 * j, b1 = b0 + 1;
                uint8_t sc, mn;
                dqo_get_scale_min_k4(2 * j, blk + 4, &sc, &mn);
                u->a[2 * b0] = u->a[2 * b0 + 1] = d * sc;
                u->m[2 * b0] = u->m[2 * b0 + 1] = dmin * mn;
                dqo_get_scale_min_k4(2 * j + 1, blk + 4, &sc, &mn);
                u->a[2 * b1] = u->a[2 * b1 + 1] = d * sc;
                u->m[2 * b1] = u->m[2 * b1 + 1] = dmin * mn;
                for (int l = 0; l < 32; ++l) {
                    u->q[b0 * 32 + l] = (int8_t)(ql[l] & 0x0F);
                    u->q[b1 * 32 + l] = (int8_t)(ql[l] >> 4);
                }
                ql += 32;
            }
        }
        break;
    case DQO_Q6_K:
        for (size_t i = 0; i < cols / QKK; ++i) {
            const uint8_t* blk = row + i * SZ_Q6_K;
            const float d = dqo_fp16_to_fp32(rd16(blk + 208));
            const uint8_t* ql = blk;
            const uint8_t* qh = blk + 128;
            const int8_t* sc = (const int8_t*)(blk + 192);
            for (int n = 0; n < 2; ++n) {
                const size_t b = i * 8 + n * 4;
                for (int l = 0; l < 32; ++l) {
                    u->q[(b + 0) * 32 + l] = (int8_t)(((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32);
                    u->q[(b + 1) * 32 + l] = (int8_t)(((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32);
                    u->q[(b + 2) * 32 + l] = (int8_t)(((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32);
                    u->q[(b + 3) * 32 + l] = (int8_t)(((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32);
                }
                for (int k = 0; k < 8; ++k) u->a[2 * b + k] = d * sc[k];
                ql += 64;
                qh += 32;
                sc += 8;
            }
        }
        break;
    }
}

static int gemm_impl(int type, const uint8_t* w, size_t rows, size_t cols, const float* x,
                     size_t n_tok, float* yf, double* yd, size_t row0, size_t row1,
                     size_t t0, size_t t1) {
    if (!gemv_cols_ok(type, cols)) return DQO_ERR_NOT_SUPPORTED;
    if (type == DQO_Q8_1) return DQO_ERR_NOT_SUPPORTED;
    if (row1 == 0) row1 = rows;
    if (t1 == 0) t1 = n_tok;
    const size_t nb = cols / QK;
    const size_t row_bytes = dqo_row_size(type, (int64_t)cols);
    const size_t min_tok = type == DQO_Q8_0 ? 2 : 4; /* matmul_q8_0_batch uses i8_gemm from 2 */
    if (n_tok < min_tok) {
        /* per-token GEMV semantics */
        for (size_t t = t0; t < t1; ++t) {
            if (yf) {
                float* tmp = (float*)malloc(rows * sizeof(float));
                dqo_matmul(type, w, rows, cols, x + t * cols, tmp, row0, row1);
                for (size_t r = row0; r < row1; ++r) yf[t * rows + r] = tmp[r];
                free(tmp);
            } else {
                double* tmp = (double*)malloc(rows * sizeof(double));
                dqo_matmul_f64(type, w, rows, cols, x + t * cols, tmp, row0, row1);
                for (size_t r = row0; r < row1; ++r) yd[t * rows + r] = tmp[r];
                free(tmp);
            }
        }
        return DQO_OK;
    }
    const int has_m = type == DQO_Q4_K;
    const int split = type == DQO_Q6_K;
    /* activations of the requested tokens */
    const size_t nt = t1 - t0;
    int8_t* xq = (int8_t*)malloc(nt * cols);
    float* dx = (float*)malloc(nt * nb * sizeof(float));
    float* sx = (float*)malloc(nt * nb * sizeof(float));
    for (size_t t = 0; t < nt; ++t)
        dqo_quantize_q8_1(x + (t0 + t) * cols, cols, xq + t * cols, dx + t * nb, NULL, sx + t * nb);
    unpacked_row u;
    u.q = (int8_t*)malloc(cols);
    u.a = (float*)malloc(2 * nb * sizeof(float));
    u.m = (float*)malloc(2 * nb * sizeof(float));
    for (size_t r = row0; r < row1; ++r) {
        unpack_row(type, w + r * row_bytes, cols, &u);
        for (size_t t = 0; t < nt; ++t) {
            const int8_t* xt = xq + t * cols;
            float f = 0.0f;
            double fd = 0.0;
            for (size_t b = 0; b < nb; ++b) {
                const float dxb = dx[t * nb + b];
                if (split) {
                    int32_t lo = 0, hi = 0;
                    for (int j = 0; j < 16; ++j) {
                        lo += (int32_t)u.q[b * 32 + j] * xt[b * 32 + j];
                        hi += (int32_t)u.q[b * 32 + 16 + j] * xt[b * 32 + 16 + j];
                    }
                    f = fmaf((float)lo, u.a[2 * b] * dxb, f);
                    f = fmaf((float)hi, u.a[2 * b + 1] * dxb, f);
                    fd += (double)lo * u.a[2 * b] * dxb + (double)hi * u.a[2 * b + 1] * dxb;
                } else {
                    const int32_t I = idot32(u.q + b * 32, xt + b * 32);
                    f = fmaf((float)I, u.a[2 * b] * dxb, f);
                    fd += (double)I * u.a[2 * b] * dxb;
                }
                if (has_m) {
                    f = fmaf(-u.m[2 * b], sx[t * nb + b], f);
                    fd -= (double)u.m[2 * b] * sx[t * nb + b];
                }
            }
            if (yf) yf[(t0 + t) * rows + r] = f;
            else yd[(t0 + t) * rows + r] = fd;
        }
    }
    free(u.q);
    free(u.a);
    free(u.m);
    free(xq);
    free(dx);
    free(sx);
    return DQO_OK;
}

/* The weight side of the i8_gemm semantics above, as unpack_row gives it
 * (core/matmul.cpp:505-638): per row, the integer weights q[cols], the scale
 * a of each 16 columns and the Q4_K offset m of each 16 (0 for the other
 * types). With the per-32 activation integers and scales and the exact block
 * sums of dqo_quantize_q8_1, the product is
 *   y[t][r] = sum_k (a q)[r][k] (dx q_x)[t][k] - sum_b m[r][b] sx[t][b],
 * which a test can form in fp64 for every output of a full-size product. */
int dqo_gemm_operands(int type, const uint8_t* w, size_t rows, size_t cols, int8_t* q, float* a, float* m) {
    if (!gemv_cols_ok(type, cols) || type == DQO_Q8_1) return DQO_ERR_NOT_SUPPORTED;
    const size_t nb = cols / QK;
    const size_t row_bytes = dqo_row_size(type, (int64_t)cols);
    unpacked_row u;
    for (size_t r = 0; r < rows; ++r) {
        u.q = q + r * cols;
        u.a = a + r * 2 * nb;
        u.m = m + r * 2 * nb;
        memset(u.m, 0, 2 * nb * sizeof(float));
        unpack_row(type, w + r * row_bytes, cols, &u);
    }
    return DQO_OK;
}

int dqo_gemm(int type, const uint8_t* w, size_t rows, size_t cols, const float* x,
             size_t n_tok, float* y, size_t row0, size_t row1, size_t t0, size_t t1) {
    return gemm_impl(type, w, rows, cols, x, n_tok, y, NULL, row0, row1, t0, t1);
}

int dqo_gemm_f64(int type, const uint8_t* w, size_t rows, size_t cols, const float* x,
                 size_t n_tok, double* y, size_t row0, size_t row1, size_t t0, size_t t1) {
    return gemm_impl(type, w, rows, cols, x, n_tok, NULL, y, row0, row1, t0, t1);
}

/* ------------------------------------------------------------------------ */
/* Q8_0 KV cache and decode attention                                       */
/* ------------------------------------------------------------------------ */

/* kv/kv_quant.cpp:58-100, x86 branch: per 32-block, 8 lanes accumulate
 * fma(q, x) over the 4 chunks of 8, then (l, l+4), (0+2, 1+3), sum. */
float dqo_kv_dot_q8_0(const float* query, const uint8_t* row, size_t dim) {
    float acc = 0.0f;
    for (size_t b = 0; b < dim / 32; ++b) {
        const uint8_t* blk = row + b * SZ_Q8_0;
        const float d = dqo_fp16_to_fp32(rd16(blk));
        const int8_t* qs = (const int8_t*)(blk + 2);
        const float* qp = query + b * 32;
        float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int i = 0; i < 32; i += 8)
            for (int l = 0; l < 8; ++l) v[l] = fmaf((float)qs[i + l], qp[i + l], v[l]);
        float h[4];
        for (int l = 0; l < 4; ++l) h[l] = v[l] + v[l + 4];
        const float block_dot = (h[0] + h[2]) + (h[1] + h[3]);
        acc += d * block_dot;
    }
    return acc;
}

/* kv/kv_quant.cpp:102-140: y += (w*d)*q as one fma per element. */
void dqo_kv_axpy_q8_0(float* y, const uint8_t* row, size_t dim, float weight) {
    for (size_t b = 0; b < dim / 32; ++b) {
        const uint8_t* blk = row + b * SZ_Q8_0;
        const float scale = weight * dqo_fp16_to_fp32(rd16(blk));
        const int8_t* qs = (const int8_t*)(blk + 2);
        for (int i = 0; i < 32; ++i) y[b * 32 + i] = fmaf(scale, (float)qs[i], y[b * 32 + i]);
    }
}

/* models/dense_forward.cpp:805-821 softmax_inplace: float max, double sum */
void dqo_softmax(float* s, size_t n) {
    float m = -INFINITY;
    for (size_t i = 0; i < n; ++i) m = (m < s[i]) ? s[i] : m;
    double sum = 0.0;
    for (size_t i = 0; i < n; ++i) {
        s[i] = expf(s[i] - m);
        sum += (double)s[i];
    }
    for (size_t i = 0; i < n; ++i) s[i] /= (float)sum;
}

/* models/dense_forward.cpp:3956-4065 (quantized-KV branch, no ALiBi) */
void dqo_attn_decode_q8(const float* q, const uint8_t* kc, const uint8_t* vc,
                        uint32_t n_head, uint32_t n_head_kv, uint32_t hd,
                        uint32_t cc_start, uint32_t pos, float* out) {
    const size_t row_bytes = (size_t)hd / 32 * SZ_Q8_0;
    const size_t pos_bytes = (size_t)n_head_kv * row_bytes;
    const float inv_d = 1.0f / sqrtf((float)hd);
    const uint32_t hpk = n_head / n_head_kv;
    float* scores = (float*)malloc(((size_t)pos + 1) * sizeof(float));
    for (uint32_t h = 0; h < n_head; ++h) {
        const uint32_t hkv = h / hpk;
        const float* qh = q + (size_t)h * hd;
        float* oh = out + (size_t)h * hd;
        const uint8_t* kb = kc + (size_t)hkv * row_bytes;
        const uint8_t* vb = vc + (size_t)hkv * row_bytes;
        for (uint32_t cc = cc_start; cc <= pos; ++cc)
            scores[cc] = dqo_kv_dot_q8_0(qh, kb + (size_t)cc * pos_bytes, hd) * inv_d;
        dqo_softmax(scores + cc_start, (size_t)pos + 1 - cc_start);
        for (uint32_t d = 0; d < hd; ++d) oh[d] = 0.0f;
        for (uint32_t cc = cc_start; cc <= pos; ++cc)
            dqo_kv_axpy_q8_0(oh, vb + (size_t)cc * pos_bytes, hd, scores[cc]);
    }
    free(scores);
}

/* core/attn_cpu.cpp:128-390 (attention_prefill_cpu_q8), one row at a time:
 * row (token t, head h) sits at position pos0 + t and attends to the keys
 * [lo, pos] of KV head h / hpk, lo = pos + 1 - n_swa when n_swa > 0 and
 * pos + 1 > n_swa, else 0 (:165, :310-311). The query is multiplied by inv_d
 * first (:157); K and V rows are dequantized to float d * q (:96-104); the
 * scores are float dot products, the softmax subtracts the row maximum, and
 * the output is sum(p * v) * (1 / sum(p)) (:380-384). The reference tiles the
 * keys with an online maximum and a polynomial exp; results agree to float
 * rounding. Rows of other heads' columns of q_dim are left untouched. */
static void deq_kv_row(const uint8_t* row, uint32_t hd, float* out) {
    for (uint32_t b = 0; b < hd / 32; ++b) {
        const uint8_t* blk = row + (size_t)b * SZ_Q8_0;
        const float d = dqo_fp16_to_fp32(rd16(blk));
        for (int j = 0; j < 32; ++j) out[b * 32 + j] = d * (float)(int8_t)blk[2 + j];
    }
}

int dqo_attn_prefill_q8(const float* q_all, float* out, uint32_t n_tok, uint32_t n_head, uint32_t hpk,
                        uint32_t hd, uint32_t q_dim, const uint8_t* kbase, const uint8_t* vbase,
                        size_t row_bytes, size_t pos_bytes, uint32_t pos0, uint32_t n_swa, float inv_d) {
    if (hd == 0 || hd % 32 || hpk == 0 || n_head % hpk) return DQO_ERR_NOT_SUPPORTED;
    float* qs = (float*)malloc(hd * sizeof(float));
    float* row = (float*)malloc(hd * sizeof(float));
    float* o = (float*)malloc(hd * sizeof(float));
    float* s = (float*)malloc(((size_t)pos0 + n_tok) * sizeof(float));
    for (uint32_t t = 0; t < n_tok; ++t) {
        const uint32_t pos = pos0 + t;
        const uint32_t lo = (n_swa > 0 && pos + 1 > n_swa) ? pos + 1 - n_swa : 0;
        for (uint32_t h = 0; h < n_head; ++h) {
            const uint32_t hkv = h / hpk;
            const float* qh = q_all + (size_t)t * q_dim + (size_t)h * hd;
            for (uint32_t d = 0; d < hd; ++d) qs[d] = qh[d] * inv_d;
            float m = -INFINITY;
            for (uint32_t k = lo; k <= pos; ++k) {
                deq_kv_row(kbase + (size_t)k * pos_bytes + (size_t)hkv * row_bytes, hd, row);
                float a = 0.0f;
                for (uint32_t d = 0; d < hd; ++d) a += qs[d] * row[d];
                s[k] = a;
                m = a > m ? a : m;
            }
            float l = 0.0f;
            for (uint32_t k = lo; k <= pos; ++k) {
                s[k] = expf(s[k] - m);
                l += s[k];
            }
            for (uint32_t d = 0; d < hd; ++d) o[d] = 0.0f;
            for (uint32_t k = lo; k <= pos; ++k) {
                deq_kv_row(vbase + (size_t)k * pos_bytes + (size_t)hkv * row_bytes, hd, row);
                for (uint32_t d = 0; d < hd; ++d) o[d] += s[k] * row[d];
            }
            const float inv = l > 0.0f ? 1.0f / l : 0.0f;
            float* dst = out + (size_t)t * q_dim + (size_t)h * hd;
            for (uint32_t d = 0; d < hd; ++d) dst[d] = o[d] * inv;
        }
    }
    free(qs); free(row); free(o); free(s);
    return DQO_OK;
}

/* fp64 softmax attention over the dequantized K/V rows. */
void dqo_attn_decode_q8_f64(const float* q, const uint8_t* kc, const uint8_t* vc,
                            uint32_t n_head, uint32_t n_head_kv, uint32_t hd,
                            uint32_t cc_start, uint32_t pos, double* out) {
    const size_t row_bytes = (size_t)hd / 32 * SZ_Q8_0;
    const size_t pos_bytes = (size_t)n_head_kv * row_bytes;
    const uint32_t hpk = n_head / n_head_kv;
    const size_t np = (size_t)pos + 1;
    double* s = (double*)malloc(np * sizeof(double));
    float* row = (float*)malloc(hd * sizeof(float));
    for (uint32_t h = 0; h < n_head; ++h) {
        const uint32_t hkv = h / hpk;
        const float* qh = q + (size_t)h * hd;
        double m = -INFINITY;
        for (uint32_t cc = cc_start; cc <= pos; ++cc) {
            dqo_dequantize_row(DQO_Q8_0, kc + cc * pos_bytes + hkv * row_bytes, row, hd);
            double acc = 0.0;
            for (uint32_t d = 0; d < hd; ++d) acc += (double)qh[d] * row[d];
            s[cc] = acc / sqrt((double)hd);
            if (s[cc] > m) m = s[cc];
        }
        double sum = 0.0;
        for (uint32_t cc = cc_start; cc <= pos; ++cc) {
            s[cc] = exp(s[cc] - m);
            sum += s[cc];
        }
        for (uint32_t d = 0; d < hd; ++d) out[(size_t)h * hd + d] = 0.0;
        for (uint32_t cc = cc_start; cc <= pos; ++cc) {
            dqo_dequantize_row(DQO_Q8_0, vc + cc * pos_bytes + hkv * row_bytes, row, hd);
            for (uint32_t d = 0; d < hd; ++d) out[(size_t)h * hd + d] += s[cc] / sum * row[d];
        }
    }
    free(s);
    free(row);
}

/* ------------------------------------------------------------------------ */
/* MoE router: models/moe_route.cpp:10-75 (softmax gating, no bias)         */
/* ------------------------------------------------------------------------ */
uint32_t dqo_moe_route(const float* logits, uint32_t n, uint32_t k, int norm_w,
                       float w_scale, uint32_t* ids, float* wts) {
    if (n == 0) return 0;
    float* probs = (float*)malloc(n * sizeof(float));
    float m = logits[0];
    for (uint32_t i = 0; i < n; ++i) m = (m < logits[i]) ? logits[i] : m;
    double sum = 0.0;
    for (uint32_t i = 0; i < n; ++i) {
        probs[i] = expf(logits[i] - m);
        sum += probs[i];
    }
    for (uint32_t i = 0; i < n; ++i) probs[i] = (float)(probs[i] / sum);
    for (uint32_t i = 0; i < n; ++i)
        if (isnan(probs[i])) probs[i] = 0.0f;
    if (k > n) k = n;
    /* selection of the k largest, descending; ties keep the lower index */
    uint8_t* used = (uint8_t*)calloc(n, 1);
    float wsum = 0.0f;
    for (uint32_t s = 0; s < k; ++s) {
        uint32_t best = n;
        for (uint32_t i = 0; i < n; ++i) {
            if (used[i]) continue;
            if (best == n || probs[i] > probs[best]) best = i;
        }
        used[best] = 1;
        ids[s] = best;
        wts[s] = probs[best];
        wsum += probs[best];
    }
    if (norm_w && wsum > 1e-9f)
        for (uint32_t s = 0; s < k; ++s) wts[s] /= wsum;
    if (w_scale != 0.0f && w_scale != 1.0f)
        for (uint32_t s = 0; s < k; ++s) wts[s] *= w_scale;
    free(used);
    free(probs);
    return k;
}

/* ------------------------------------------------------------------------ */
/* Decoder-layer glue                                                       */
/* ------------------------------------------------------------------------ */

/* models/dense_forward.cpp:129-165 rms_norm_vec, AVX2 order: squares in
 * float, summed in double by two 4-lane accumulators, (0+1)+(2+3). */
void dqo_rms_norm(const float* x, const float* w, float* y, size_t n, float eps) {
    double s0[4] = {0, 0, 0, 0}, s1[4] = {0, 0, 0, 0};
    size_t i = 0;
    for (; i + 8 <= n; i += 8) {
        for (int l = 0; l < 4; ++l) {
            const float a = x[i + l] * x[i + l];
            const float b = x[i + 4 + l] * x[i + 4 + l];
            s0[l] += (double)a;
            s1[l] += (double)b;
        }
    }
    double t[4];
    for (int l = 0; l < 4; ++l) t[l] = s0[l] + s1[l];
    double sum = (t[0] + t[1]) + (t[2] + t[3]);
    for (; i < n; ++i) sum += (double)x[i] * x[i];
    const float scale = 1.0f / sqrtf((float)(sum / (double)n) + eps);
    for (size_t j = 0; j < n; ++j) y[j] = x[j] * scale * w[j];
}

/* models/dense_forward.cpp:631-657 rope_cache_init, no YaRN (ext_factor 0,
 * attn_factor 1, freq_scale 1). */
void dqo_rope_cache(float* cache, size_t n_rot, uint32_t pos, float theta_base) {
    const float theta_scale = powf(theta_base, -2.0f / (float)n_rot);
    float theta = (float)pos;
    for (size_t j = 0; j < n_rot / 2; ++j) {
        cache[2 * j + 0] = cosf(theta) * 1.0f;
        cache[2 * j + 1] = sinf(theta) * 1.0f;
        theta *= theta_scale;
    }
}

/* models/dense_forward.cpp:668-680 rope_neox_cached: pairs (j, j+n_rot/2) */
void dqo_rope_neox(float* v, size_t n_rot, const float* cache) {
    const size_t half = n_rot / 2;
    for (size_t j = 0; j < half; ++j) {
        const float c = cache[2 * j], s = cache[2 * j + 1];
        const float x0 = v[j], x1 = v[j + half];
        v[j] = x0 * c - x1 * s;
        v[j + half] = x0 * s + x1 * c;
    }
}

/* models/dense_forward.cpp:53-55 */
float dqo_silu(float v) { return v / (1.0f + expf(-v)); }

/* models/dense_forward.cpp:49-51 gelu_tanh (the batch branch's gated GELU,
 * :3608-3609, and the CPU fallback's scalar tail). */
float dqo_gelu_tanh(float v) {
    return 0.5f * v * (1.0f + tanhf(0.7978845608028654f * v * (1.0f + 0.044715f * v * v)));
}

/* :69-94 exp_ps_avx2, one lane: clamp to [-87, 87], t = x log2(e), k =
 * nearest integer of t (ties to even), r = t - k, 2^r by the degree-5
 * Horner polynomial (a multiply then an add per step), times 2^k built in
 * the exponent field. Separate multiplies and adds throughout (the
 * intrinsics are not contracted). */
float dqo_exp_avx2(float x) {
    x = x > -87.0f ? x : -87.0f; /* _mm256_max_ps(x, -87): NaN -> -87 */
    x = x < 87.0f ? x : 87.0f;
    const float t = x * 1.44269504088896341f;
    const float k = rintf(t);
    const float r = t - k;
    float p = 1.3327544e-3f;
    p = p * r + 9.6181292e-3f;
    p = p * r + 5.5504109e-2f;
    p = p * r + 2.4022651e-1f;
    p = p * r + 6.9314718e-1f;
    p = p * r + 1.0f;
    const int32_t bits = ((int32_t)k + 127) << 23;
    float pow2k;
    memcpy(&pow2k, &bits, 4);
    return p * pow2k;
}

/* :107-126 geglu_inplace, its 8-wide path (every n_ff here is a multiple of
 * 8): gelu(g) = g / (1 + exp(-2u)), u = (0.7978845608 g)(1 + 0.044715 g^2),
 * then times up. The decode branch's gated GELU (:4212-4213). */
float dqo_geglu(float g) {
    const float xx = g * g;
    const float u = (0.7978845608028654f * g) * (1.0f + 0.044715f * xx);
    const float e = dqo_exp_avx2(-2.0f * u);
    return g / (1.0f + e);
}

static size_t rb_of(int fmt, size_t cols) { return dqo_row_size(fmt, (int64_t)cols); }

/* After the Q/K/V products of one token (models/dense_forward.cpp
 * :3904-3931 decode, :3318-3342 batch): the optional biases (add_bias: y +=
 * b), then the optional per-head QK-norm (rms_norm_vec of each head of q and
 * of k with the head_dim weights q_norm / k_norm). */
static void qkv_post(const dqo_layer_t* L, float* q, float* k, float* v) {
    const size_t hd = L->head_dim, qd = (size_t)L->n_head * hd, kvd = (size_t)L->n_head_kv * hd;
    if (L->bq) for (size_t i = 0; i < qd; ++i) q[i] += L->bq[i];
    if (L->bk) for (size_t i = 0; i < kvd; ++i) k[i] += L->bk[i];
    if (L->bv) for (size_t i = 0; i < kvd; ++i) v[i] += L->bv[i];
    if (L->q_norm)
        for (uint32_t h = 0; h < L->n_head; ++h) dqo_rms_norm(q + h * hd, L->q_norm, q + h * hd, hd, L->rms_eps);
    if (L->k_norm)
        for (uint32_t h = 0; h < L->n_head_kv; ++h) dqo_rms_norm(k + h * hd, L->k_norm, k + h * hd, hd, L->rms_eps);
}

/* models/dense_forward.cpp:3897-4257, the Llama branch with the optional
 * Q/K/V biases and per-head QK-norm (Qwen-style layers); no sandwich norms,
 * gated SiLU FFN, Q8_0 KV. The K-quant matvecs quantize their input per 256
 * (matvec -> matmul_q4_k/q6_k, and quantize_shared_q8k for the shared Q/K/V
 * and gate/up inputs). */
/* The per-head output gate of one token (DenseQuirks::attn_gate,
 * models/dense_forward.cpp:4102-4114 and :3527-3536): g = 1 / (1 + exp(-x))
 * of the head's gate value, times every value of the head's output. */
void dqo_attn_gate_apply(float* ao, const float* gate, uint32_t n_head, size_t hd) {
    for (uint32_t h = 0; h < n_head; ++h) {
        const float g = 1.0f / (1.0f + expf(-gate[h]));
        for (size_t d = 0; d < hd; ++d) ao[h * hd + d] *= g;
    }
}

int dqo_layer_decode(const dqo_layer_t* L, uint8_t* kc, uint8_t* vc, uint32_t pos,
                     const float* x, float* x_out, float* q_out, float* k_out,
                     float* v_out, float* attn_out_opt) {
    const size_t E = L->n_embd, hd = L->head_dim;
    const size_t qd = (size_t)L->n_head * hd, kvd = (size_t)L->n_head_kv * hd, F = L->n_ff;
    float* attn_in = (float*)malloc(E * sizeof(float));
    float* q = (float*)malloc(qd * sizeof(float));
    float* k = (float*)malloc(kvd * sizeof(float));
    float* v = (float*)malloc(kvd * sizeof(float));
    float* ao = (float*)malloc(qd * sizeof(float));
    float* proj = (float*)malloc(E * sizeof(float));
    float* xnp = (float*)malloc(E * sizeof(float));
    float* up = (float*)malloc(F * sizeof(float));
    float* gate = (float*)malloc(F * sizeof(float));
    float* fout = (float*)malloc(E * sizeof(float));
    float* rope = (float*)malloc(hd * sizeof(float));
    int rc = DQO_OK;

    dqo_rms_norm(x, L->attn_norm, attn_in, E, L->rms_eps);
    rc |= dqo_matmul(L->fmt_q, L->wq, qd, E, attn_in, q, 0, 0);
    rc |= dqo_matmul(L->fmt_k, L->wk, kvd, E, attn_in, k, 0, 0);
    rc |= dqo_matmul(L->fmt_v, L->wv, kvd, E, attn_in, v, 0, 0);
    qkv_post(L, q, k, v);
    dqo_rope_cache(rope, hd, pos, L->rope_theta);
    for (uint32_t h = 0; h < L->n_head; ++h) dqo_rope_neox(q + h * hd, hd, rope);
    for (uint32_t h = 0; h < L->n_head_kv; ++h) dqo_rope_neox(k + h * hd, hd, rope);
    /* write_kv_cache (dense_forward.cpp:2552-2605): one Q8_0 row per kv head */
    const size_t row_bytes = hd / 32 * SZ_Q8_0;
    const size_t pos_bytes = (size_t)L->n_head_kv * row_bytes;
    for (uint32_t h = 0; h < L->n_head_kv; ++h) {
        dqo_kv_quantize_row(k + h * hd, hd, kc + (size_t)pos * pos_bytes + h * row_bytes);
        dqo_kv_quantize_row(v + h * hd, hd, vc + (size_t)pos * pos_bytes + h * row_bytes);
    }
    dqo_attn_decode_q8(q, kc, vc, L->n_head, L->n_head_kv, (uint32_t)hd, 0, pos, ao);
    if (L->wag) { /* :4102-4114: matvec of the same normalized input */
        float* gv = (float*)malloc(L->n_head * sizeof(float));
        rc |= dqo_matmul(L->fmt_ag, L->wag, L->n_head, E, attn_in, gv, 0, 0);
        dqo_attn_gate_apply(ao, gv, L->n_head, hd);
        free(gv);
    }
    rc |= dqo_matmul(L->fmt_o, L->wo, E, qd, ao, proj, 0, 0);
    if (L->post_attn_norm) dqo_rms_norm(proj, L->post_attn_norm, proj, E, L->rms_eps); /* :4140-4142 */
    for (size_t i = 0; i < E; ++i) proj[i] += x[i];
    dqo_rms_norm(proj, L->ffn_norm, xnp, E, L->rms_eps);
    rc |= dqo_matmul(L->fmt_up, L->wup, F, E, xnp, up, 0, 0);
    rc |= dqo_matmul(L->fmt_gate, L->wgate, F, E, xnp, gate, 0, 0);
    for (size_t i = 0; i < F; ++i) up[i] = (L->act_gelu ? dqo_geglu(gate[i]) : dqo_silu(gate[i])) * up[i];
    rc |= dqo_matmul(L->fmt_down, L->wdown, E, F, up, fout, 0, 0);
    if (L->post_ffn_norm) dqo_rms_norm(fout, L->post_ffn_norm, fout, E, L->rms_eps); /* :4245-4247 */
    for (size_t i = 0; i < E; ++i) x_out[i] = fout[i] + proj[i];

    if (q_out) memcpy(q_out, q, qd * sizeof(float));
    if (k_out) memcpy(k_out, k, kvd * sizeof(float));
    if (v_out) memcpy(v_out, v, kvd * sizeof(float));
    if (attn_out_opt) memcpy(attn_out_opt, ao, qd * sizeof(float));
    free(attn_in); free(q); free(k); free(v); free(ao); free(proj); free(xnp);
    free(up); free(gate); free(fout); free(rope);
    return rc ? DQO_ERR_NOT_SUPPORTED : DQO_OK;
}

/* The CPU batch branch of models/dense_forward.cpp for a prompt chunk of
 * n_tok tokens at positions pos0..: per token rms_norm (:3264-3273), Q/K/V
 * through matvec_batch (:3286-3290, matmul_q4_k_batch / matmul_q6_k_batch:
 * dqo_gemm), per token the optional biases and QK-norm (:3318-3342), RoPE
 * and KV rows (:3347-3362), attention over the
 * cache (:3449-3460, attention_prefill_cpu_q8), output projection, residual
 * and FFN norm (:3539-3560), up/gate, silu(gate) * up, down, residual
 * (:3600-3624). RoPE over the whole head (n_rot = head_dim). */
int dqo_layer_prefill(const dqo_layer_t* L, uint8_t* kc, uint8_t* vc, uint32_t pos0, uint32_t n_tok,
                      uint32_t n_swa, const float* x, float* x_out) {
    const size_t E = L->n_embd, hd = L->head_dim, T = n_tok;
    const size_t qd = (size_t)L->n_head * hd, kvd = (size_t)L->n_head_kv * hd, F = L->n_ff;
    float* xn = (float*)malloc(T * E * sizeof(float));
    float* q = (float*)malloc(T * qd * sizeof(float));
    float* k = (float*)malloc(T * kvd * sizeof(float));
    float* v = (float*)malloc(T * kvd * sizeof(float));
    float* ao = (float*)malloc(T * qd * sizeof(float));
    float* proj = (float*)malloc(T * E * sizeof(float));
    float* up = (float*)malloc(T * F * sizeof(float));
    float* gate = (float*)malloc(T * F * sizeof(float));
    float* fout = (float*)malloc(T * E * sizeof(float));
    float* rope = (float*)malloc(hd * sizeof(float));
    int rc = DQO_OK;
    for (size_t t = 0; t < T; ++t) dqo_rms_norm(x + t * E, L->attn_norm, xn + t * E, E, L->rms_eps);
    rc |= dqo_gemm(L->fmt_q, L->wq, qd, E, xn, T, q, 0, 0, 0, 0);
    rc |= dqo_gemm(L->fmt_k, L->wk, kvd, E, xn, T, k, 0, 0, 0, 0);
    rc |= dqo_gemm(L->fmt_v, L->wv, kvd, E, xn, T, v, 0, 0, 0, 0);
    const size_t row_bytes = hd / 32 * SZ_Q8_0;
    const size_t pos_bytes = (size_t)L->n_head_kv * row_bytes;
    for (size_t t = 0; t < T; ++t) {
        const uint32_t pos = pos0 + (uint32_t)t;
        qkv_post(L, q + t * qd, k + t * kvd, v + t * kvd);
        dqo_rope_cache(rope, hd, pos, L->rope_theta);
        for (uint32_t h = 0; h < L->n_head; ++h) dqo_rope_neox(q + t * qd + h * hd, hd, rope);
        for (uint32_t h = 0; h < L->n_head_kv; ++h) {
            dqo_rope_neox(k + t * kvd + h * hd, hd, rope);
            dqo_kv_quantize_row(k + t * kvd + h * hd, hd, kc + (size_t)pos * pos_bytes + h * row_bytes);
            dqo_kv_quantize_row(v + t * kvd + h * hd, hd, vc + (size_t)pos * pos_bytes + h * row_bytes);
        }
    }
    rc |= dqo_attn_prefill_q8(q, ao, n_tok, L->n_head, L->n_head / L->n_head_kv, (uint32_t)hd, (uint32_t)qd, kc, vc,
                              row_bytes, pos_bytes, pos0, n_swa, 1.0f / sqrtf((float)hd));
    if (L->wag) { /* :3522-3537: matvec_batch of the normalized inputs, per token */
        float* gv = (float*)malloc(T * L->n_head * sizeof(float));
        rc |= dqo_gemm(L->fmt_ag, L->wag, L->n_head, E, xn, T, gv, 0, 0, 0, 0);
        for (size_t t = 0; t < T; ++t) dqo_attn_gate_apply(ao + t * qd, gv + t * L->n_head, L->n_head, hd);
        free(gv);
    }
    rc |= dqo_gemm(L->fmt_o, L->wo, E, qd, ao, T, proj, 0, 0, 0, 0);
    if (L->post_attn_norm) /* :3546-3548 */
        for (size_t t = 0; t < T; ++t) dqo_rms_norm(proj + t * E, L->post_attn_norm, proj + t * E, E, L->rms_eps);
    for (size_t i = 0; i < T * E; ++i) proj[i] += x[i];
    for (size_t t = 0; t < T; ++t) dqo_rms_norm(proj + t * E, L->ffn_norm, xn + t * E, E, L->rms_eps);
    rc |= dqo_gemm(L->fmt_up, L->wup, F, E, xn, T, up, 0, 0, 0, 0);
    rc |= dqo_gemm(L->fmt_gate, L->wgate, F, E, xn, T, gate, 0, 0, 0, 0);
    for (size_t i = 0; i < T * F; ++i) up[i] = (L->act_gelu ? dqo_gelu_tanh(gate[i]) : dqo_silu(gate[i])) * up[i];
    rc |= dqo_gemm(L->fmt_down, L->wdown, E, F, up, T, fout, 0, 0, 0, 0);
    if (L->post_ffn_norm) /* :3618-3620 */
        for (size_t t = 0; t < T; ++t) dqo_rms_norm(fout + t * E, L->post_ffn_norm, fout + t * E, E, L->rms_eps);
    for (size_t i = 0; i < T * E; ++i) x_out[i] = fout[i] + proj[i];
    free(xn); free(q); free(k); free(v); free(ao); free(proj); free(up); free(gate); free(fout); free(rope);
    return rc ? DQO_ERR_NOT_SUPPORTED : DQO_OK;
}

/* models/dense_forward.cpp:1524-1560 expert_ffn (stacked experts, matvec_raw
 * -> matmul_q4_k per token) and the combine at :4160-4181. */
int dqo_moe_ffn(int fmt, const uint8_t* wgate, const uint8_t* wup, const uint8_t* wdown,
                uint32_t n_expert, uint32_t n_embd, uint32_t n_ff,
                const float* x, const float* logits, uint32_t n_tok, uint32_t k_used,
                int norm_w, float* out, uint32_t t0, uint32_t t1) {
    if (t1 == 0) t1 = n_tok;
    const size_t rb_gu = rb_of(fmt, n_embd), rb_d = rb_of(fmt, n_ff);
    float* up = (float*)malloc((size_t)n_ff * sizeof(float));
    float* gate = (float*)malloc((size_t)n_ff * sizeof(float));
    float* fo = (float*)malloc((size_t)n_embd * sizeof(float));
    uint32_t ids[64];
    float wts[64];
    int rc = DQO_OK;
    for (uint32_t t = t0; t < t1; ++t) {
        const float* xt = x + (size_t)t * n_embd;
        float* ot = out + (size_t)t * n_embd;
        const uint32_t k = dqo_moe_route(logits + (size_t)t * n_expert, n_expert, k_used, norm_w,
                                         1.0f, ids, wts);
        for (uint32_t i = 0; i < n_embd; ++i) ot[i] = 0.0f;
        for (uint32_t s = 0; s < k; ++s) {
            const size_t e = ids[s];
            rc |= dqo_matmul(fmt, wup + e * n_ff * rb_gu, n_ff, n_embd, xt, up, 0, 0);
            rc |= dqo_matmul(fmt, wgate + e * n_ff * rb_gu, n_ff, n_embd, xt, gate, 0, 0);
            for (uint32_t i = 0; i < n_ff; ++i) up[i] = dqo_silu(gate[i]) * up[i];
            rc |= dqo_matmul(fmt, wdown + e * n_embd * rb_d, n_embd, n_ff, up, fo, 0, 0);
            for (uint32_t i = 0; i < n_embd; ++i) ot[i] += wts[s] * fo[i];
        }
    }
    free(up);
    free(gate);
    free(fo);
    return rc ? DQO_ERR_NOT_SUPPORTED : DQO_OK;
}

/* ------------------------------------------------------------------------ */
/* Exhaustive identity checks (see dq_oracle.h)                             */
/* ------------------------------------------------------------------------ */
uint64_t dqo_check_div127(uint32_t lo, uint32_t hi) {
    uint64_t bad = 0;
    for (uint64_t u = lo; u < hi; ++u) {
        const float a = u2f((uint32_t)u);
        if (a != a || isinf(a)) continue;
        const float x = (float)((double)a * (1.0 / 127.0));
        const float y = a / 127.0f;
        bad += f2u(x) != f2u(y);
    }
    return bad;
}

uint64_t dqo_check_rint_byte(uint32_t lo, uint32_t hi) {
    uint64_t bad = 0;
    for (uint64_t u = lo; u < hi; ++u) {
        const float p = u2f((uint32_t)u);
        if (p != p || !(fabsf(p) <= 128.0f)) continue;
        const uint8_t got = (uint8_t)(f2u(p + 12582912.0f) & 0xFF);
        const uint8_t want = (uint8_t)(int8_t)(int)rintf(p);
        bad += got != want;
    }
    return bad;
}

uint64_t dqo_check_id_bound(uint32_t lo, uint32_t hi) {
    uint64_t bad = 0;
    for (uint64_t u = lo; u < hi; ++u) {
        const float a = u2f((uint32_t)u);
        if (a != a || isinf(a) || !(a > 0.0f)) continue;
        const float d = a / 127.0f;
        if (d > 0.0f) {
            const float id32 = 1.0f / d;
            if (!isinf(id32)) bad += rintf(a * id32) > 127.0f;
        }
        const float id256 = 127.0f / a;
        if (!isinf(id256)) bad += rintf(a * id256) > 127.0f;
    }
    return bad;
}
