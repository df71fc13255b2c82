// dq_common.h - shared device helpers and device-side weight layouts for the
// gfx950 quantized compute path. Wave64 throughout.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/desireeia_hip.h"

#define DQ_WAVE 64

// GGUF block sizes (reference quant/quant.h:41-187).
#define DQ_QK 32
#define DQ_QKK 256
#define DQ_SZ_Q4_0 18
#define DQ_SZ_Q8_0 34
#define DQ_SZ_Q8_1 36
#define DQ_SZ_Q4_K 144
#define DQ_SZ_Q6_K 210

// Every on-device weight layout is split into 256-byte-aligned planes inside
// one allocation. A row is cut into items of 64 weights (cols/64 per row);
// the quant bytes of an item are split over NP "sub-planes" of 16 bytes per
// item, each sub-plane item-major ([rows][items][16 B], rows q_row bytes
// apart). A wave whose lane l reads item 64j+l of a sub-plane thus issues one
// contiguous kilobyte per global_load_dwordx4. Byte counts per row equal the
// GGUF row size, so the HBM traffic of a kernel is the GGUF size of the
// matrix.
//
//   Q8_0 (NP 4): sub-plane k of item i = int8 weights 64i+16k..+16
//         D = fp16 [rows][cols/32] (item i: the scales of blocks 2i, 2i+1)
//   Q4_0 (NP 2): sub-plane k of item i = the 16 nibble bytes of block 2i+k
//         D = fp16 [rows][cols/32]
//   Q4_K (NP 2): item i = (block s = i/4, group g = i%4); sub-plane k = qs bytes
//         32g+16k..+16 of block s (positions 16k..16k+15 of sub-block 2g in the
//         low nibbles and of sub-block 2g+1 in the high nibbles)
//         H = [rows][cols/256][16 B]: bytes 0..15 of each block (d, dmin, scales)
//   Q6_K (NP 3): item i = (block s = i/4, it = i%4 = 2n+k), n = 128-half,
//         k = 16-position half; sub-plane 0 = ql bytes 64n+16k..+16, 1 = ql bytes
//         64n+32+16k..+16, 2 = qh bytes 32n+16k..+16
//         S = [rows][cols/256][4 items][4 int8]: scales 8n+k, 8n+2+k, 8n+4+k, 8n+6+k
//         D = fp16 [rows][cols/256]
struct DqLayout {
    int np;                // number of quant sub-planes
    size_t q_off, q_row;   // sub-plane 0 offset, row stride of a sub-plane (items*16)
    size_t p_stride;       // distance between sub-planes
    size_t s_off, s_row;   // Q4_K header plane H, or Q6_K scale plane S
    size_t d_off, d_row;   // fp16 scale plane D
    size_t total;
};

static inline size_t dq_align256(size_t v) { return (v + 255) & ~(size_t)255; }

static inline bool dq_layout(int fmt, size_t rows, size_t cols, DqLayout* L) {
    *L = DqLayout{};
    switch (fmt) {
    case DQ_FMT_Q8_0:
        if (cols % 64) return false;
        L->np = 4;
        L->d_row = cols / 32 * 2;
        break;
    case DQ_FMT_Q4_0:
        if (cols % 64) return false;
        L->np = 2;
        L->d_row = cols / 32 * 2;
        break;
    case DQ_FMT_Q4_K:
        if (cols % 256) return false;
        L->np = 2;
        L->s_row = cols / 256 * 16;
        break;
    case DQ_FMT_Q6_K:
        if (cols % 256) return false;
        L->np = 3;
        L->s_row = cols / 256 * 16;
        L->d_row = cols / 256 * 2;
        break;
    default:
        return false;
    }
    L->q_row = cols / 64 * 16;
    L->q_off = 0;
    L->p_stride = dq_align256(rows * L->q_row);
    L->s_off = L->p_stride * (size_t)L->np;
    L->d_off = dq_align256(L->s_off + rows * L->s_row);
    L->total = dq_align256(L->d_off + rows * L->d_row);
    return true;
}

static inline size_t dq_gguf_row_bytes(int fmt, size_t cols) {
    switch (fmt) {
    case DQ_FMT_Q8_0: return cols / 32 * DQ_SZ_Q8_0;
    case DQ_FMT_Q4_0: return cols / 32 * DQ_SZ_Q4_0;
    case DQ_FMT_Q4_K: return cols / 256 * DQ_SZ_Q4_K;
    case DQ_FMT_Q6_K: return cols / 256 * DQ_SZ_Q6_K;
    default: return 0;
    }
}

// ---------------------------------------------------------------- device --

__device__ __forceinline__ float dq_h2f(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

// fp32 -> fp16 bits, round to nearest even (v_cvt_f16_f32).
__device__ __forceinline__ uint16_t dq_f2h(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

__device__ __forceinline__ int dq_sdot4(int a, int b, int c) {
    return __builtin_amdgcn_sdot4(a, b, c, false);
}

// Bytes v in [0,63] -> v - 32 as signed bytes, without borrows between bytes.
__device__ __forceinline__ int dq_sub32_bytes(uint32_t v) {
    return (int)(((v | 0x80808080u) - 0x20202020u) ^ 0x80808080u);
}

typedef uint32_t dq_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t dq_u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ dq_u32x4 dq_ld16(const void* p) {
    return *reinterpret_cast<const dq_u32x4*>(p);
}

// Non-temporal 16-byte load for data streamed exactly once (weights).
__device__ __forceinline__ dq_u32x4 dq_ld16_stream(const void* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const dq_u32x4*>(p));
}

// The LDS address of a pointer into a __shared__ array, as the LDS operand of
// __builtin_amdgcn_global_load_lds (direct global -> LDS DMA).
#define DQ_LDS_PTR(p) reinterpret_cast<__attribute__((address_space(3))) void*>(reinterpret_cast<uintptr_t>(p))

// DPP move of a float (gfx9 dpp_ctrl encodings; all rows and banks enabled).
// Workgroup barrier for LDS rings filled by global_load_lds: waits for this
// wave's LDS reads (lgkmcnt 0; gfx9 s_waitcnt encoding, vmcnt and expcnt at
// their maximum) and leaves the vector memory counter alone. __syncthreads
// adds a fence that waits for every outstanding global load, which would
// also wait for the DMAs of the ring stages still in flight; callers wait for
// the DMAs they need with an explicit vmcnt before this barrier.
__device__ __forceinline__ void dq_lds_barrier() {
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

template <int CTRL>
__device__ __forceinline__ float dq_dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum of v over each 16-lane row, in every lane of the row: quad_perm
// [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror (VALU data
// movement, no LDS round trip). Fixed order: deterministic.
__device__ __forceinline__ float dq_row16_sum(float v) {
    v += dq_dpp<0xB1>(v);
    v += dq_dpp<0x4E>(v);
    v += dq_dpp<0x141>(v);
    v += dq_dpp<0x140>(v);
    return v;
}

// Maximum of v over each 16-lane row, in every lane of the row (the same
// DPP steps as dq_row16_sum).
__device__ __forceinline__ float dq_row16_max(float v) {
    v = fmaxf(v, dq_dpp<0xB1>(v));
    v = fmaxf(v, dq_dpp<0x4E>(v));
    v = fmaxf(v, dq_dpp<0x141>(v));
    v = fmaxf(v, dq_dpp<0x140>(v));
    return v;
}

// Full-wave float sum as a wave-uniform value: the four row sums combined as
// (row0 + row1) + (row2 + row3).
__device__ __forceinline__ float dq_wave_sum_uniform(float v) {
    v = dq_row16_sum(v);
    const int b = __builtin_bit_cast(int, v);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
    return (r0 + r1) + (r2 + r3);
}

// Full-wave float maximum as a wave-uniform value (DPP row maxima, then the
// four rows' by readlane: no LDS round trips).
__device__ __forceinline__ float dq_wave_max_uniform(float v) {
    v = dq_row16_max(v);
    const int b = __builtin_bit_cast(int, v);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// Full-wave float sum; every lane receives the total.
__device__ __forceinline__ float dq_wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, DQ_WAVE);
    return v;
}

__device__ __forceinline__ double dq_wave_sum_f64(double v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, DQ_WAVE);
    return v;
}

// A head of HD values (HD = 64, 128 or 256) held by the 64 lanes of a wave:
// x[i] = value lane + 64 i, HD / 64 values per lane.
template <int HD>
constexpr bool dq_head_dim_ok() {
    return HD == 64 || HD == 128 || HD == 256;
}
inline bool dq_head_dim_supported(uint32_t hd) { return hd == 64 || hd == 128 || hd == 256; }

// rms_norm_vec (models/dense_forward.cpp:129-165) of one head held by a wave:
// squares in float summed in double, scale = 1/sqrtf((float)(sum/HD) + eps),
// y = x * scale * w. The per-head QK-norm of :3915-3931. w[i] = weight of
// value lane + 64 i, already in registers.
template <int HD>
__device__ __forceinline__ void dq_head_rms_norm_w(float (&x)[HD / 64], const float (&w)[HD / 64], float eps) {
    double s = 0.0;
#pragma unroll
    for (int i = 0; i < HD / 64; ++i) s += (double)(x[i] * x[i]);
    s = dq_wave_sum_f64(s);
    const float scale = 1.0f / sqrtf((float)(s / (double)HD) + eps);
#pragma unroll
    for (int i = 0; i < HD / 64; ++i) x[i] = x[i] * scale * w[i];
}
template <int HD>
__device__ __forceinline__ void dq_head_rms_norm(float (&x)[HD / 64], const float* __restrict__ w, int lane,
                                                 float eps) {
    float wr[HD / 64];
#pragma unroll
    for (int i = 0; i < HD / 64; ++i) wr[i] = w[lane + 64 * i];
    dq_head_rms_norm_w<HD>(x, wr, eps);
}

// The gated FFN activations of the reference (act(gate) * up):
//  * silu(x) = x / (1 + expf(-x)) (models/dense_forward.cpp:53-55);
//  * the decode branch's GELU, geglu_inplace (:107-126, its 8-wide path):
//    g / (1 + exp(-2u)), u = (0.7978845608 g)(1 + 0.044715 g^2), with exp by
//    exp_ps_avx2 (:69-94): clamp to [-87, 87], t = x log2(e), k = nearest
//    integer (ties to even), r = t - k, 2^r by the degree-5 Horner
//    polynomial (separate multiplies and adds), times 2^k from the exponent
//    bits;
//  * the batch branch's GELU, gelu_tanh (:49-51, :3608-3609).
__device__ __forceinline__ float dq_exp_avx2(float x) {
    x = x > -87.0f ? x : -87.0f;  // _mm256_max_ps(x, -87): NaN -> -87
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
    return p * __builtin_bit_cast(float, ((int)k + 127) << 23);
}
enum DqFfnAct { DQ_ACT_SILU = 0, DQ_ACT_GEGLU = 1, DQ_ACT_GELU_TANH = 2 };
template <int ACT>
__device__ __forceinline__ float dq_ffn_act(float g) {
    if constexpr (ACT == DQ_ACT_SILU) {
        return g / (1.0f + expf(-g));
    } else if constexpr (ACT == DQ_ACT_GEGLU) {
        const float xx = g * g;
        const float u = (0.7978845608028654f * g) * (1.0f + 0.044715f * xx);
        return g / (1.0f + dq_exp_avx2(-2.0f * u));
    } else {
        return 0.5f * g * (1.0f + tanhf(0.7978845608028654f * g * (1.0f + 0.044715f * g * g)));
    }
}

// Q/K/V post-processing of one head held by a wave (x[i] = value lane +
// 64 i), between the projections and RoPE: the bias (add_bias, y += b;
// :3904-3908) and the per-head RMSNorm (:3915-3931). All optional.
struct DqQkvPost {
    const float *bq, *bk, *bv, *q_norm, *k_norm;
    float eps;
    // optional per-head output gate values g_h (device, one per query head):
    // the attention output of head h is scaled by 1 / (1 + exp(-g_h))
    // (dense_forward.cpp:4102-4114)
    const float* gate;
};
// kind 0: query head, 1: key head, 2: value head
template <int HD>
__device__ __forceinline__ void dq_qkv_post(float (&x)[HD / 64], int kind, int head, int lane, const DqQkvPost& P) {
    const float* b = kind == 0 ? P.bq : (kind == 1 ? P.bk : P.bv);
    if (b) {
#pragma unroll
        for (int i = 0; i < HD / 64; ++i) x[i] += b[(size_t)head * HD + lane + 64 * i];
    }
    const float* nw = kind == 0 ? P.q_norm : (kind == 1 ? P.k_norm : nullptr);
    if (nw) dq_head_rms_norm<HD>(x, nw, lane, P.eps);
}

__device__ __forceinline__ float dq_wave_max(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, DQ_WAVE));
    return v;
}

// NeoX RoPE of the pair (x0, x1) = (dim j, dim j + n_rot/2) with (cos, sin) =
// (rope[2j], rope[2j+1]) (models/dense_forward.cpp:668-680), unfused.
__device__ __forceinline__ void dq_rope_pair(float& x0, float& x1, const float* rope, int j) {
    const float c = rope[2 * j], s = rope[2 * j + 1];
    const float a = x0, b = x1;
    x0 = a * c - b * s;
    x1 = a * s + b * c;
}

// NeoX RoPE of a whole head held by a wave (n_rot = HD): pairs (j, j + HD/2)
// with (cos, sin) = (rope[2j], rope[2j+1]) (models/dense_forward.cpp:668-680).
// HD >= 128: both values of a pair sit in one lane (x[i], x[i + HD/128]);
// HD = 64: in lanes j and j + 32.
template <int HD>
__device__ __forceinline__ void dq_rope_head(float (&x)[HD / 64], const float* __restrict__ rope, int lane) {
    if constexpr (HD == 64) {
        const float y = __shfl_xor(x[0], 32, DQ_WAVE);  // the pair's other value
        const int j = lane & 31;
        const float c = rope[2 * j], s = rope[2 * j + 1];
        x[0] = lane < 32 ? x[0] * c - y * s : y * s + x[0] * c;
    } else {
#pragma unroll
        for (int i = 0; i < HD / 128; ++i) dq_rope_pair(x[i], x[i + HD / 128], rope, lane + 64 * i);
    }
}

// kv_quantize_row (kv/kv_quant.cpp:31-56) of one HD-value row held by a wave
// (x[i] = value lane + 64 i): value lane + 64 i is element lane % 32 of block
// 2 i + lane / 32; a block's maximum is a reduction over its 32 lanes. Each
// block is fp16 d followed by 32 int8. dst: HD / 32 * 34 bytes, 2-byte aligned
// (global or LDS).
template <int HD>
__device__ __forceinline__ void dq_q8_0_row(const float (&x)[HD / 64], int lane, uint8_t* dst) {
    float am[HD / 64];
#pragma unroll
    for (int i = 0; i < HD / 64; ++i) am[i] = fabsf(x[i]);
#pragma unroll
    for (int off = 1; off < 32; off <<= 1) {
#pragma unroll
        for (int i = 0; i < HD / 64; ++i) am[i] = fmaxf(am[i], __shfl_xor(am[i], off, DQ_WAVE));
    }
    const int hb = lane >> 5, e = lane & 31;
#pragma unroll
    for (int i = 0; i < HD / 64; ++i) {
        const float amax = am[i];
        const float d = amax > 0.0f ? amax / 127.0f : 0.0f;
        const float id = d > 0.0f ? 1.0f / d : 0.0f;
        int iv = (int)rintf(x[i] * id);
        iv = iv > 127 ? 127 : (iv < -127 ? -127 : iv);
        uint8_t* bp = dst + (2 * i + hb) * DQ_SZ_Q8_0;
        bp[2 + e] = (uint8_t)(iv & 0xFF);
        if (e == 0) *reinterpret_cast<uint16_t*>(bp) = dq_f2h(d);
    }
}

// Host-side status from a HIP error.
static inline int dq_status(hipError_t e) { return e == hipSuccess ? DQ_OK : DQ_ERR_IO; }
static inline int dq_launch_status() { return dq_status(hipGetLastError()); }

// Float ranges an activation quantizer launch clears on the side (the
// outputs of the K-split GEMMs that read its result next); counts are
// multiples of 4, pointers 16-byte aligned, unused slots null.
struct DqZeroSpans {
    static constexpr int N = 4;
    float* p[N] = {nullptr, nullptr, nullptr, nullptr};
    size_t n[N] = {0, 0, 0, 0};
};
// Library-internal parts of the prefill GEMM (dq_gemm.hip): the quantizer
// with spans to clear (with d_gate, of the gated FFN product act(gate) * x,
// act a DqFfnAct: SiLU or gelu_tanh), whether a product's plan adds K-split partials into y
// (so y must start at zero), the plan's workgroup count, and the GEMM on a y
// already cleared. cu_budget > 0 plans the product for that many CUs (a
// product that runs beside others); 0 plans it for the whole GPU.
int dq_quantize_act_f16_zero(int fmt, const float* d_x, size_t cols, size_t n_tok, void* d_out,
                             const DqZeroSpans& z, void* stream, const float* d_gate = nullptr, int act = 0);
bool dq_gemm_adds_into_y(int fmt, size_t rows, size_t cols, size_t n_tok, int cu_budget = 0);
size_t dq_gemm_workgroups(int fmt, size_t rows, size_t cols, size_t n_tok, int cu_budget = 0);
int dq_gemm_f16act_zeroed(int fmt, const void* d_w, size_t rows, size_t cols, const void* d_work, size_t n_tok,
                          float* d_y, bool y_zeroed, void* stream, int cu_budget = 0);
int dq_gemm_cus();
// The RMSNorm of rows of a (+ b, the residual, kept in h when given) with
// weight w (to y when given; rms_norm_rows_kernel's arithmetic) fused with
// the activation quantization of the normalised rows for n_fmt (1 or 2)
// formats of different classes into their workspaces outs[k]; spans z are
// cleared on the side.
int dq_norm_quant_f16(const float* d_a, const float* d_b, float* d_h, const float* d_w, size_t cols, size_t n_tok,
                      float eps, float* d_y, int n_fmt, const int* fmts, void* const* outs, const DqZeroSpans& z,
                      void* stream);
static inline bool dq_zero_span_ok(const float* p, size_t n) {
    return p && n % 4 == 0 && reinterpret_cast<uintptr_t>(p) % 16 == 0;
}
// Library-internal forms of the fused decode attention, the RoPE + K/V-row
// write of one token and of a prompt chunk, with the optional Q/K/V biases
// and per-head QK-norm applied first and the optional per-head output gate
// applied to the attention output (the public entry points pass none); and
// of the plain decode attention with the output gate.
int dq_attn_rope_kv_decode_post(const float* d_q, const float* d_k, const float* d_v, const float* d_rope,
                                uint32_t n_rot, void* d_kc, void* d_vc, uint32_t n_head, uint32_t n_head_kv,
                                uint32_t hd, uint32_t cc_start, uint32_t pos, const int32_t* d_pos, uint32_t n_ctx,
                                float* d_out, int8_t* d_oq, float* d_oscale, int32_t* d_oisum, void* d_work,
                                size_t work_bytes, const DqQkvPost& post, void* stream);
int dq_attn_decode_q8_post(const float* d_q, const void* d_kc, const void* d_vc, uint32_t n_head,
                           uint32_t n_head_kv, uint32_t hd, uint32_t cc_start, uint32_t pos, const int32_t* d_pos,
                           uint32_t n_ctx, float* d_out, int8_t* d_oq, float* d_oscale, int32_t* d_oisum,
                           void* d_work, size_t work_bytes, const DqQkvPost& post, void* stream);
int dq_rope_kv_write_post(float* d_q, const float* d_k, const float* d_v, const float* d_rope, uint32_t n_head,
                          uint32_t n_head_kv, uint32_t hd, uint32_t n_rot, void* d_kc, void* d_vc, uint32_t pos,
                          const int32_t* d_pos, uint32_t n_ctx, const DqQkvPost& post, void* stream);
int dq_rope_kv_write_batch_post(float* d_q, const float* d_k, const float* d_v, size_t q_ld, size_t kv_ld,
                                const float* d_rope, uint32_t n_rot, uint32_t n_tok, uint32_t n_head,
                                uint32_t n_head_kv, uint32_t hd, void* d_kc, void* d_vc, uint32_t pos0,
                                uint32_t n_ctx, const DqQkvPost& post, void* stream);
// The layer's post-processing from its descriptor.
static inline DqQkvPost dq_layer_post(const dq_layer_t* L) {
    return DqQkvPost{L->bq, L->bk, L->bv, L->q_norm, L->k_norm, L->rms_eps, nullptr};
}
// act(gate) * up of the decode layer (gelu 1: geglu_inplace, else silu), then
// the per-256 quantizer (dq_act_quant) or in float (dq_act_mul).
int dq_act_quant(const float* d_gate, const float* d_up, size_t n, int gelu, int8_t* d_q, float* d_scale,
                 int32_t* d_isum, void* stream);
int dq_act_mul(const float* d_gate, const float* d_up, size_t n, int gelu, float* d_h, void* stream);
// out = rms_norm_vec(a, w) + b for each of `rows` rows of n floats (the
// sandwich norm before a residual); out may alias b.
int dq_post_norm_add(const float* d_a, const float* d_w, const float* d_b, float* d_out, size_t n, uint32_t rows,
                     float eps, void* stream);
