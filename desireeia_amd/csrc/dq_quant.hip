// dq_quant.hip - activation quantizers (per-32 and per-256-replicated, the
// arithmetic in dq_quant.h) and the GGUF block_q8_1 wire form. One lane per
// 32-value block: the lane loads its 128 bytes as 8 dwordx4, so a wave covers
// 8 KB of contiguous input.
#include "dq_common.h"
#include "dq_quant.h"

namespace {

template <int KIND>
__global__ __launch_bounds__(256) void quantize_act_kernel(const float* __restrict__ x, size_t n_blocks,
                                                           int8_t* __restrict__ q, float* __restrict__ scale,
                                                           int32_t* __restrict__ isum,
                                                           float* __restrict__ fsum) {
    const size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    // KIND 1 reduces over groups of 8 lanes: keep every lane of a group alive.
    const bool valid = b < n_blocks;
    const size_t bb = valid ? b : n_blocks - 1;
    float v[32];
    dq_load32(x + bb * 32, v);
    uint32_t packed[8];
    float d, fs;
    int s;
    dq_quant_block<KIND>(v, packed, d, s, fs);
    if (!valid) return;
    dq_u32x4* qo = reinterpret_cast<dq_u32x4*>(q + b * 32);
    qo[0] = dq_u32x4{packed[0], packed[1], packed[2], packed[3]};
    qo[1] = dq_u32x4{packed[4], packed[5], packed[6], packed[7]};
    scale[b] = d;
    if (isum) isum[b] = s;
    if (fsum) fsum[b] = fs;
}

// block_q8_1: fp16 d, fp16 s (= d * sum q, the GGUF convention), int8 qs[32].
__global__ __launch_bounds__(256) void quantize_q8_1_blocks_kernel(const float* __restrict__ x, size_t n_blocks,
                                                                   uint8_t* __restrict__ out) {
    const size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= n_blocks) return;
    float v[32];
    const float4* p = reinterpret_cast<const float4*>(x + b * 32);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 f = p[i];
        v[4 * i + 0] = f.x;
        v[4 * i + 1] = f.y;
        v[4 * i + 2] = f.z;
        v[4 * i + 3] = f.w;
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        const float a = fabsf(v[i]);
        amax = (amax < a) ? a : amax;
    }
    const float d = amax > 0.0f ? amax / 127.0f : 0.0f;
    const float id = d > 0.0f ? 1.0f / d : 0.0f;
    uint8_t* blk = out + b * DQ_SZ_Q8_1;
    int s = 0;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        int iv = (int)rintf(v[i] * id);
        iv = iv > 127 ? 127 : (iv < -127 ? -127 : iv);
        s += iv;
        blk[4 + i] = (uint8_t)(int8_t)iv;
    }
    const uint16_t hd = dq_f2h(d);
    const uint16_t hs = dq_f2h(d * (float)s);
    blk[0] = (uint8_t)(hd & 0xFF);
    blk[1] = (uint8_t)(hd >> 8);
    blk[2] = (uint8_t)(hs & 0xFF);
    blk[3] = (uint8_t)(hs >> 8);
}

}  // namespace

extern "C" int dq_quantize_act(int kind, const float* d_x, size_t cols, size_t n_tok, int8_t* d_q,
                               float* d_scale, int32_t* d_isum, float* d_fsum, void* stream) {
    if (!d_x || !d_q || !d_scale) return DQ_ERR_INVALID_ARG;
    if (cols == 0 || n_tok == 0) return DQ_OK;
    if (kind == DQ_ACT_Q8_0) {
        if (cols % 32) return DQ_ERR_NOT_SUPPORTED;
    } else if (kind == DQ_ACT_Q8K_REP) {
        if (cols % 256) return DQ_ERR_NOT_SUPPORTED;
    } else {
        return DQ_ERR_INVALID_ARG;
    }
    const size_t nb = cols / 32 * n_tok;
    const unsigned grid = (unsigned)((nb + 255) / 256);
    hipStream_t s = (hipStream_t)stream;
    if (kind == DQ_ACT_Q8_0)
        quantize_act_kernel<DQ_ACT_Q8_0><<<grid, 256, 0, s>>>(d_x, nb, d_q, d_scale, d_isum, d_fsum);
    else
        quantize_act_kernel<DQ_ACT_Q8K_REP><<<grid, 256, 0, s>>>(d_x, nb, d_q, d_scale, d_isum, d_fsum);
    return dq_launch_status();
}

extern "C" int dq_quantize_q8_1_blocks(const float* d_x, size_t n, void* d_blocks, void* stream) {
    if (!d_x || !d_blocks) return DQ_ERR_INVALID_ARG;
    if (n % 32) return DQ_ERR_NOT_SUPPORTED;
    if (n == 0) return DQ_OK;
    const size_t nb = n / 32;
    quantize_q8_1_blocks_kernel<<<(unsigned)((nb + 255) / 256), 256, 0, (hipStream_t)stream>>>(
        d_x, nb, (uint8_t*)d_blocks);
    return dq_launch_status();
}
