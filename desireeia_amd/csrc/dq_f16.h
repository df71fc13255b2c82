// dq_f16.h - fp16 operand helpers shared by the MFMA kernels (prefill GEMM,
// MoE expert GEMM): magic-number conversion of packed 4/6-bit weights to
// scaled fp16 pairs, and the Q4_K 6-bit scale/min decode.
#pragma once

#include "dq_common.h"

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f16v __attribute__((ext_vector_type(16)));

// Bytes 0/1 (sel 0x04010400) or 2/3 (sel 0x04030402) of v, each below 1024,
// as the fp16 pair (1024 + v_lo, 1024 + v_hi): v_perm_b32 slots the byte under
// the 0x64 exponent byte.
__device__ __forceinline__ h2 magic_pair(uint32_t v, uint32_t sel) {
    return __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, v, sel));
}

// 4 byte values (each < 1024 - bias) of word v -> 2 fp16 pairs (v - bias) * a.
// The subtraction is exact; the product rounds once.
__device__ __forceinline__ void bytes_to_h2(uint32_t v, h2 bias, h2 a, uint32_t* out) {
    const h2 p0 = (magic_pair(v, 0x04010400u) - bias) * a;
    const h2 p1 = (magic_pair(v, 0x04030402u) - bias) * a;
    out[0] = __builtin_bit_cast(uint32_t, p0);
    out[1] = __builtin_bit_cast(uint32_t, p1);
}

// Q4_K 6-bit scale of sub-block j from header words w0 (scale bytes 0-3),
// w1 (4-7), w2 (8-11) (quant/quant.cpp:22-29).
// Branch-free (j may be a run-time value): both forms are computed from the
// byte at position j & 3 and one is kept by a bit mask (a ?: on a uniform j
// is compiled into branches).
__device__ __forceinline__ int q4k_scale(int j, uint32_t w0, uint32_t w1, uint32_t w2) {
    const int sh = 8 * (j & 3);
    const uint32_t b0 = (w0 >> sh) & 0xFF, b2 = (w2 >> sh) & 0xFF;
    const uint32_t hi = 0u - (uint32_t)(j >> 2);  // all ones for j >= 4
    return (int)(((b0 & 63) & ~hi) | (((b2 & 0xF) | ((b0 >> 6) << 4)) & hi));
}
__device__ __forceinline__ int q4k_min(int j, uint32_t w0, uint32_t w1, uint32_t w2) {
    const int sh = 8 * (j & 3);
    const uint32_t b1 = (w1 >> sh) & 0xFF, b2 = (w2 >> sh) & 0xFF;
    const uint32_t hi = 0u - (uint32_t)(j >> 2);
    return (int)(((b1 & 63) & ~hi) | (((b2 >> 4) | ((b1 >> 6) << 4)) & hi));
}

// The 8 6-bit scales (sc_bytes) or mins (m_bytes) of a Q4_K super-block
// header hd (d and dmin in hd.x, the 12 scale bytes in hd.y..hd.w) as bytes:
// j = 0..3 in lo, 4..7 in hi (the packing of quant/quant.cpp:22-29, four at
// a time: sc_j = b0_j & 63, sc_{j+4} = (b2_j & 15) | (b0_j >> 6) << 4, and
// the mins alike from b1 and the high nibbles of b2).
__device__ __forceinline__ void q4k_sc_bytes(const dq_u32x4& hd, uint32_t& lo, uint32_t& hi) {
    lo = hd.y & 0x3F3F3F3Fu;
    hi = (hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u);
}
__device__ __forceinline__ void q4k_m_bytes(const dq_u32x4& hd, uint32_t& lo, uint32_t& hi) {
    lo = hd.z & 0x3F3F3F3Fu;
    hi = ((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u);
}

// Pairs p[i] = (b_2i * f, b_2i+1 * f) in fp16 of the 8 bytes of lo, hi (each
// below 1024): the byte is exact in fp16 and the product rounds once, as the
// float product fp16((float)f * b) does.
__device__ __forceinline__ void bytes8_times(uint32_t lo, uint32_t hi, _Float16 f, h2 (&p)[4]) {
    const h2 bias = {(_Float16)1024.0f, (_Float16)1024.0f}, ff = {f, f};
    p[0] = (magic_pair(lo, 0x04010400u) - bias) * ff;
    p[1] = (magic_pair(lo, 0x04030402u) - bias) * ff;
    p[2] = (magic_pair(hi, 0x04010400u) - bias) * ff;
    p[3] = (magic_pair(hi, 0x04030402u) - bias) * ff;
}

// The 8 values fp16(-dmin * m_j) of a Q4_K super-block header hd: the weight
// side of the super-block's min term as one 8-wide MFMA K slice. Zeros when
// !ok.
__device__ __forceinline__ h8 q4k_neg_mins(const dq_u32x4& hd, bool ok) {
    uint32_t lo, hi;
    q4k_m_bytes(hd, lo, hi);
    const _Float16 f = ok ? __builtin_bit_cast(_Float16, (uint16_t)((hd.x >> 16) ^ 0x8000u)) : (_Float16)0.0f;
    h2 p[4];
    bytes8_times(lo, hi, f, p);
    return __builtin_bit_cast(h8, dq_u32x4{__builtin_bit_cast(uint32_t, p[0]), __builtin_bit_cast(uint32_t, p[1]),
                                           __builtin_bit_cast(uint32_t, p[2]), __builtin_bit_cast(uint32_t, p[3])});
}

// Nibble pairs to scaled fp16 pairs with one v_and_or and one fma: two 4-bit
// values q_a, q_b at bits 6-9 and 22-25 of v (the caller shifts them there)
// are slotted under the exponent of 16.0 (0x4C00, mantissa step 2^-6), so
// each half is 16 + q exactly, and fma(16 + q, s, c) with c = -16 s is
// q * s exactly before its single rounding: the same fp16 as (q) * s.
// Needs 16 |s| finite in fp16: |s| <= 4094. The mask and the exponent word
// come in registers (NibConst): gfx9 VOP3 instructions take no literal.
struct NibConst {
    uint32_t mask;  // 0x03C003C0, in an SGPR
    uint32_t expo;  // 0x4C004C00, in a VGPR
};
__device__ __forceinline__ NibConst nib_const() {
    NibConst k{0x03C003C0u, 0x4C004C00u};
    asm volatile("" : "+s"(k.mask));
    asm volatile("" : "+v"(k.expo));
    return k;
}
__device__ __forceinline__ uint32_t nib_pair_fma(uint32_t v, NibConst k, h2 s, h2 c) {
    const h2 m = __builtin_bit_cast(h2, (v & k.mask) | k.expo);
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(m, s, c));
}


namespace {

// fp16 operands have a range of 65504, and a min column (a sum over a
// 32-block) reaches 32 * max|v| of its activation row. Each activation row is
// therefore multiplied by a power of two s that puts 32 * max|v| at or below
// 2^15 (exact: only the exponent moves; small rows are scaled up, away from
// the fp16 subnormals), and the GEMM multiplies its output row by 1/s.
// row_scale_kernel: one 256-thread workgroup per row of `cols` floats
// (cols % 4 == 0), s = 2^(15 - E) with 32 * max|v| = m * 2^E, m in [0.5, 1).
__device__ __forceinline__ float row_scale_of(float r) {
    int E = 0;
    if (r > 0.0f && r <= 3.0e38f) frexpf(32.0f * r, &E);
    E = E < -100 ? -100 : (E > 115 ? 115 : E);
    return ldexpf(1.0f, 15 - E);
}

__global__ __launch_bounds__(256) void row_scale_kernel(const float* __restrict__ src, int cols,
                                                        float* __restrict__ scale) {
    __shared__ float wmax[4];
    const float* row = src + (size_t)blockIdx.x * cols;
    float m = 0.0f;
    for (int c = threadIdx.x * 4; c < cols; c += 1024) {
        const float4 f = *reinterpret_cast<const float4*>(row + c);
        m = fmaxf(m, fmaxf(fmaxf(fabsf(f.x), fabsf(f.y)), fmaxf(fabsf(f.z), fabsf(f.w))));
    }
    m = dq_wave_max(m);
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) scale[blockIdx.x] = row_scale_of(fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3])));
}

}  // namespace
