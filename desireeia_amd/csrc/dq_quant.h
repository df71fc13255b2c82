// dq_quant.h - the activation quantizers as device functions, shared by the
// quantize kernels and the GEMVs that quantize their activation in-kernel.
//
// One lane per 32-value block. Bit-exactness with the reference: amax is
// exact; d = amax/127 and the reciprocal use IEEE division; q = rint(x*id) is
// v_rndne_f32 (round to nearest even, the lrintf / cvtps2dq rounding of the
// reference); the float block sum is sequential. Files including this are
// built with -ffp-contract=off so no multiply-add is fused.
#pragma once

#include "dq_common.h"

// Quantizes the 32 values v of this lane's block. KIND DQ_ACT_Q8_0: per 32,
// d = amax/127, id = 1/d (core/quant.cpp:15-50). KIND DQ_ACT_Q8K_REP: per 256
// = 8 consecutive lanes (every lane of such a group must take part),
// d = amax/127, id = 127/amax (core/matmul.cpp:1681-1700). Outputs the packed
// int8 words, d, the int32 sum of the q and the float sum of v.
template <int KIND>
__device__ __forceinline__ void dq_quant_block(const float (&v)[32], uint32_t (&packed)[8], float& d_out, int& isum,
                                               float& fsum) {
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        const float a = fabsf(v[i]);
        amax = (amax < a) ? a : amax;
    }
    float d, id;
    if (KIND == DQ_ACT_Q8_0) {
        d = amax > 0.0f ? amax / 127.0f : 0.0f;
        id = d > 0.0f ? 1.0f / d : 0.0f;
    } else {
#pragma unroll
        for (int off = 1; off < 8; off <<= 1) {
            const float o = __shfl_xor(amax, off, DQ_WAVE);
            amax = (amax < o) ? o : amax;
        }
        d = amax > 0.0f ? amax / 127.0f : 0.0f;
        id = d > 0.0f ? 127.0f / amax : 0.0f;
    }
    int s = 0;
#pragma unroll
    for (int w = 0; w < 8; ++w) {
        uint32_t word = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            int iv = (int)rintf(v[4 * w + k] * id);
            iv = iv > 127 ? 127 : (iv < -127 ? -127 : iv);
            s += iv;
            word |= (uint32_t)(iv & 0xFF) << (8 * k);
        }
        packed[w] = word;
    }
    float fs = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) fs += v[i];
    d_out = d;
    isum = s;
    fsum = fs;
}

__device__ __forceinline__ void dq_load32(const float* p, float (&v)[32]) {
    const float4* q = reinterpret_cast<const float4*>(p);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 f = q[i];
        v[4 * i + 0] = f.x;
        v[4 * i + 1] = f.y;
        v[4 * i + 2] = f.z;
        v[4 * i + 3] = f.w;
    }
}
