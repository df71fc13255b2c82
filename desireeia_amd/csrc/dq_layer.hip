// dq_layer.hip - one Llama-style decoder layer at batch 1 on the device
// (the plain dense branch of models/dense_forward.cpp:3897-4257: RMSNorm,
// Q/K/V, NeoX RoPE, Q8_0 KV write, GQA attention, output projection and
// residual, RMSNorm, gated SiLU FFN and residual), plus the small fused
// kernels it needs between the GEMVs:
//
//   norm_quant   (residual add +) RMSNorm + the per-256 activation quantizer
//                of the K-quant GEMVs (core/matmul.cpp:1660-1778)
//   rope_kv      NeoX RoPE of q and k from the caller's cos/sin table, and the
//                Q8_0 rows of k and v written into the cache
//   silu_quant   silu(gate) * up + the per-256 quantizer (input of ffn_down)
//
// Every float operation follows the reference's order and rounding, without
// contraction (the file is built with -ffp-contract=off): the normalised
// activations, rotated q/k and the cache bytes are those of the reference
// given the same GEMV outputs.
#include <math.h>

#include "dq_common.h"


namespace {

// ------------------------------------------------------------ norm_quant --
// h = a (+ b); y = h * (1/sqrtf(mean(h^2) + eps)) * w (models/dense_forward.cpp
// :129-165: squares in float, summed in double); then per 256 values
// amax, d = amax/127, id = 127/amax, q = rint(y*id) (core/matmul.cpp:1681-1700),
// d replicated into the 8 per-32 slots, int32 sum of q per 32.
// One workgroup of 256 threads; thread t owns chunks of 16 values.
constexpr int NQ_T = 256;

// x = a (+ b) of chunk c: every load issued before the adds (a load whose
// use sits in the same branch would be waited for on its own).
__device__ __forceinline__ void nq_chunk(const float* __restrict__ a, const float* __restrict__ b, int c,
                                         float4 (&x)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = reinterpret_cast<const float4*>(a + c * 16)[i];
    if (b) {
        float4 y[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) y[i] = reinterpret_cast<const float4*>(b + c * 16)[i];
#pragma unroll
        for (int i = 0; i < 4; ++i) x[i].x = x[i].x + y[i].x, x[i].y = x[i].y + y[i].y, x[i].z = x[i].z + y[i].z,
                                    x[i].w = x[i].w + y[i].w;
    }
}

__global__ __launch_bounds__(NQ_T) void norm_quant_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                                          float* __restrict__ h_out, const float* __restrict__ w,
                                                          int n, float eps, int8_t* __restrict__ q,
                                                          float* __restrict__ scale, int32_t* __restrict__ isum,
                                                          float* __restrict__ y_out) {
    __shared__ double wsum[NQ_T / 64];
    __shared__ float s_scale;
    const int t = threadIdx.x;
    const int n_chunks = n / 16;
    double acc = 0.0;
    float4 x0[4];  // the first pass's chunk, kept for the quantization
    for (int c0 = 0; c0 < n_chunks; c0 += NQ_T) {
        const bool live = c0 + t < n_chunks;
        const int c = min(c0 + t, n_chunks - 1);
        float4 x[4];
        nq_chunk(a, b, c, x);
        if (c0 == 0) {
#pragma unroll
            for (int i = 0; i < 4; ++i) x0[i] = x[i];
        }
        if (live) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (b && h_out) reinterpret_cast<float4*>(h_out + c * 16)[i] = x[i];
                const float s0 = x[i].x * x[i].x, s1 = x[i].y * x[i].y, s2 = x[i].z * x[i].z, s3 = x[i].w * x[i].w;
                acc += (double)s0;
                acc += (double)s1;
                acc += (double)s2;
                acc += (double)s3;
            }
        }
    }
    // the weights of the first chunk, in flight during the reduction
    float4 w0[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) w0[i] = reinterpret_cast<const float4*>(w + min(t, n_chunks - 1) * 16)[i];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, DQ_WAVE);
    if ((t & 63) == 0) wsum[t >> 6] = acc;
    __syncthreads();
    if (t == 0) {
        double s = 0.0;
        for (int i = 0; i < NQ_T / 64; ++i) s += wsum[i];
        s_scale = 1.0f / sqrtf((float)(s / (double)n) + eps);
    }
    __syncthreads();
    const float sc = s_scale;
    // 16 threads per 256-value block: chunks c = 16k .. 16k+15 belong to block k
    for (int c0 = 0; c0 < n_chunks; c0 += NQ_T) {
        const bool live = c0 + t < n_chunks;
        const int c = min(c0 + t, n_chunks - 1);
        float4 x[4], ww[4];
        if (c0 == 0) {
#pragma unroll
            for (int i = 0; i < 4; ++i) x[i] = x0[i], ww[i] = w0[i];
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) ww[i] = reinterpret_cast<const float4*>(w + c * 16)[i];
            nq_chunk(a, b, c, x);
        }
        float y[16];
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            y[4 * i + 0] = x[i].x * sc * ww[i].x;
            y[4 * i + 1] = x[i].y * sc * ww[i].y;
            y[4 * i + 2] = x[i].z * sc * ww[i].z;
            y[4 * i + 3] = x[i].w * sc * ww[i].w;
        }
        if (y_out && live) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                reinterpret_cast<float4*>(y_out + c * 16)[i] =
                    make_float4(y[4 * i], y[4 * i + 1], y[4 * i + 2], y[4 * i + 3]);
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(y[i]));
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off, DQ_WAVE));
        const float d = amax > 0.0f ? amax / 127.0f : 0.0f;
        const float id = d > 0.0f ? 127.0f / amax : 0.0f;
        int s = 0;
        uint32_t pk[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t word = 0;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                int iv = (int)rintf(y[4 * i + k] * id);
                iv = iv > 127 ? 127 : (iv < -127 ? -127 : iv);
                s += iv;
                word |= (uint32_t)(iv & 0xFF) << (8 * k);
            }
            pk[i] = word;
        }
        s += __shfl_xor(s, 1, DQ_WAVE);  // two chunks per 32-value block
        if (live) {
            *reinterpret_cast<dq_u32x4*>(q + c * 16) = dq_u32x4{pk[0], pk[1], pk[2], pk[3]};
            if ((c & 1) == 0) {
                scale[c / 2] = d;
                isum[c / 2] = s;
            }
        }
    }
}

// --------------------------------------------------------------- rope_kv --
// Workgroup r < n_head: query head r; n_head <= r < n_head + n_kv: key head;
// then value heads. 64 threads; thread j holds dims j + 64 i of the HD-dim
// head. RoPE (models/dense_forward.cpp:668-680) on the first n_rot dims: pairs
// (j, j + n_rot/2), x0*c - x1*s and x0*s + x1*c with (c, s) = table[2j],
// table[2j+1]. Keys and values are then quantized (kv_quantize_row).
template <int HD>
__global__ __launch_bounds__(64) void rope_kv_kernel(float* __restrict__ q, const float* __restrict__ k,
                                                     const float* __restrict__ v, const float* __restrict__ rope,
                                                     int n_head, int n_kv, int n_rot, uint8_t* __restrict__ kc,
                                                     uint8_t* __restrict__ vc, size_t pos_bytes, int pos_host,
                                                     const int* __restrict__ pos_dev, int n_ctx, DqQkvPost post) {
    constexpr int QV = HD / 64;
    const int r = blockIdx.x, j = threadIdx.x;
    const int kind = r < n_head ? 0 : (r < n_head + n_kv ? 1 : 2);
    const int head = kind == 0 ? r : (kind == 1 ? r - n_head : r - n_head - n_kv);
    const float* src = kind == 0 ? q + (size_t)head * HD : (kind == 1 ? k : v) + (size_t)head * HD;
    float x[QV];
#pragma unroll
    for (int i = 0; i < QV; ++i) x[i] = src[j + 64 * i];
    dq_qkv_post<HD>(x, kind, head, j, post);
    if (kind < 2 && rope) {
        if (n_rot == HD) {
            dq_rope_head<HD>(x, rope, j);
        } else {  // pairs inside [0, n_rot)
            __shared__ float row[HD];
#pragma unroll
            for (int i = 0; i < QV; ++i) row[j + 64 * i] = x[i];
            __syncthreads();
            const int half = n_rot / 2;
            for (int jj = j; jj < half; jj += 64) {
                const float c = rope[2 * jj], s = rope[2 * jj + 1];
                const float x0 = row[jj], x1 = row[jj + half];
                row[jj] = x0 * c - x1 * s;
                row[jj + half] = x0 * s + x1 * c;
            }
            __syncthreads();
#pragma unroll
            for (int i = 0; i < QV; ++i) x[i] = row[j + 64 * i];
        }
    }
    if (kind == 0) {
#pragma unroll
        for (int i = 0; i < QV; ++i) q[(size_t)head * HD + j + 64 * i] = x[i];
        return;
    }
    int p = pos_dev ? *pos_dev : pos_host;
    p = p < 0 ? 0 : (p >= n_ctx ? n_ctx - 1 : p);
    dq_q8_0_row<HD>(x, j, (kind == 1 ? kc : vc) + (size_t)p * pos_bytes + (size_t)head * (HD / 32) * DQ_SZ_Q8_0);
}

// ------------------------------------------------------------ silu_quant --
// h = silu(gate) * up, silu(x) = x / (1 + expf(-x)) (models/dense_forward.cpp
// :53-55, :4230-4235); then the per-256 quantizer. One wave per 256 values,
// 4 per lane.
template <int ACT>
__global__ __launch_bounds__(256) void silu_quant_kernel(const float* __restrict__ gate, const float* __restrict__ up,
                                                         int n, int8_t* __restrict__ q, float* __restrict__ scale,
                                                         int32_t* __restrict__ isum) {
    const int lane = threadIdx.x & 63;
    const int blk = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (blk * 256 >= n) return;  // uniform per wave
    const int e0 = blk * 256 + lane * 4;
    const float4 g = *reinterpret_cast<const float4*>(gate + e0);
    const float4 u = *reinterpret_cast<const float4*>(up + e0);
    float hv[4] = {g.x, g.y, g.z, g.w};
    const float uv[4] = {u.x, u.y, u.z, u.w};
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        hv[i] = dq_ffn_act<ACT>(hv[i]) * uv[i];
        amax = fmaxf(amax, fabsf(hv[i]));
    }
    amax = dq_wave_max(amax);
    const float d = amax > 0.0f ? amax / 127.0f : 0.0f;
    const float id = d > 0.0f ? 127.0f / amax : 0.0f;
    int s = 0;
    uint32_t word = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        int iv = (int)rintf(hv[i] * id);
        iv = iv > 127 ? 127 : (iv < -127 ? -127 : iv);
        s += iv;
        word |= (uint32_t)(iv & 0xFF) << (8 * i);
    }
#pragma unroll
    for (int off = 1; off < 8; off <<= 1) s += __shfl_xor(s, off, DQ_WAVE);  // 8 lanes = 32 values
    *reinterpret_cast<uint32_t*>(q + e0) = word;
    if ((lane & 7) == 0) {
        scale[e0 / 32] = d;
        isum[e0 / 32] = s;
    }
}

// h = silu(gate) * up in float (the input of a Q8_0 / Q4_0 down projection,
// which quantizes per 32 itself). One lane per value.
template <int ACT>
__global__ __launch_bounds__(256) void silu_mul_kernel(const float* __restrict__ gate, const float* __restrict__ up,
                                                       int n, float* __restrict__ h) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    h[i] = dq_ffn_act<ACT>(gate[i]) * up[i];
}

// ------------------------------------------------------------- workspace --
struct LayerWs {
    int8_t* aq;    // per-256 activation (K-quant matrices)
    float* as;
    int32_t* ai;
    int8_t* bq;    // per-32 activation (Q8_0 / Q4_0 matrices)
    float* bs;
    int32_t* bi;
    float* yn;     // float input of the per-32 quantizer
    float *q, *k, *v, *ao, *x2, *up, *gate;
    float* tmp;  // sandwich norms: a projection before its norm
    float* ag;   // attention gate: the per-head gate values
    void* attn;
    size_t attn_bytes, total;
};

bool kquant(int fmt) { return fmt == DQ_FMT_Q4_K || fmt == DQ_FMT_Q6_K; }
bool per32(int fmt) { return fmt == DQ_FMT_Q8_0 || fmt == DQ_FMT_Q4_0; }
bool layer_fmt(int fmt) { return kquant(fmt) || per32(fmt); }

bool layer_ok(const dq_layer_t* L) {
    if (!L || !dq_head_dim_supported(L->head_dim) || L->n_head_kv == 0 || L->n_head % L->n_head_kv) return false;
    if (L->n_embd == 0 || L->n_embd % 256 || L->n_ff == 0 || L->n_ff % 256 || (L->n_head * L->head_dim) % 256)
        return false;
    if (L->n_rot == 0 || L->n_rot > L->head_dim || L->n_rot % 2) return false;
    const int f[7] = {L->fmt_q, L->fmt_k, L->fmt_v, L->fmt_o, L->fmt_gate, L->fmt_up, L->fmt_down};
    for (int i = 0; i < 7; ++i)
        if (!layer_fmt(f[i])) return false;
    return !L->wag || layer_fmt(L->fmt_ag);
}

LayerWs carve(const dq_layer_t* L, uint32_t n_ctx, uint8_t* base) {
    const size_t E = L->n_embd, QD = (size_t)L->n_head * L->head_dim, KVD = (size_t)L->n_head_kv * L->head_dim;
    const size_t F = L->n_ff;
    const size_t AN = E > QD ? (E > F ? E : F) : (QD > F ? QD : F);
    LayerWs w{};
    size_t off = 0;
    auto take = [&](size_t bytes) {
        uint8_t* p = base ? base + off : nullptr;
        off += dq_align256(bytes);
        return p;
    };
    w.aq = (int8_t*)take(AN);
    w.as = (float*)take(AN / 32 * 4);
    w.ai = (int32_t*)take(AN / 32 * 4);
    w.bq = (int8_t*)take(AN);
    w.bs = (float*)take(AN / 32 * 4);
    w.bi = (int32_t*)take(AN / 32 * 4);
    w.yn = (float*)take(AN * 4);
    w.q = (float*)take(QD * 4);
    w.k = (float*)take(KVD * 4);
    w.v = (float*)take(KVD * 4);
    w.ao = (float*)take(QD * 4);
    w.x2 = (float*)take(E * 4);
    w.up = (float*)take(F * 4);
    w.gate = (float*)take(F * 4);
    w.tmp = (float*)take(L->post_attn_norm || L->post_ffn_norm ? E * 4 : 0);
    w.ag = (float*)take(L->wag ? (size_t)L->n_head * 4 : 0);
    size_t ab = 0;
    dq_attn_workspace_bytes(L->n_head, L->n_head_kv, L->head_dim, n_ctx, &ab);
    w.attn = take(ab);
    w.attn_bytes = ab;
    w.total = off;
    return w;
}

#define DQ_TRY(x)                      \
    do {                               \
        const int rc_ = (x);           \
        if (rc_ != DQ_OK) return rc_;  \
    } while (0)

}  // namespace

extern "C" {

int dq_rope_cache(float* cache, uint32_t n_rot, uint32_t pos, float theta_base) {
    // models/dense_forward.cpp:631-657 (rope_cache_init) without YaRN: theta_j =
    // pos * theta_scale^j by repeated float products, theta_scale =
    // powf(base, -2/n_rot). Host code: the same libm as the engine's.
    if (!cache || n_rot == 0 || n_rot % 2) return DQ_ERR_INVALID_ARG;
    const float theta_scale = powf(theta_base, -2.0f / (float)n_rot);
    float theta = (float)pos;
    for (uint32_t j = 0; j < n_rot / 2; ++j) {
        cache[2 * j] = cosf(theta) * 1.0f;
        cache[2 * j + 1] = sinf(theta) * 1.0f;
        theta *= theta_scale;
    }
    return DQ_OK;
}

int dq_norm_quant(const float* d_a, const float* d_b, float* d_h, const float* d_w, size_t n, float eps,
                  int8_t* d_q, float* d_scale, int32_t* d_isum, void* stream) {
    if (!d_a || !d_w || !d_q || !d_scale || !d_isum || n == 0 || n % 256) return DQ_ERR_INVALID_ARG;
    if (n > (1u << 26)) return DQ_ERR_NOT_SUPPORTED;
    norm_quant_kernel<<<1, NQ_T, 0, (hipStream_t)stream>>>(d_a, d_b, d_h, d_w, (int)n, eps, d_q, d_scale, d_isum,
                                                          nullptr);
    return dq_launch_status();
}

int dq_silu_quant(const float* d_gate, const float* d_up, size_t n, int8_t* d_q, float* d_scale, int32_t* d_isum,
                  void* stream) {
    return dq_act_quant(d_gate, d_up, n, 0, d_q, d_scale, d_isum, stream);
}

int dq_silu_mul(const float* d_gate, const float* d_up, size_t n, float* d_h, void* stream) {
    return dq_act_mul(d_gate, d_up, n, 0, d_h, stream);
}

}  // extern "C"

// act(gate) * up with the decode branch's activation (gelu: geglu_inplace),
// then the per-256 quantizer / in float.
int dq_act_quant(const float* d_gate, const float* d_up, size_t n, int gelu, int8_t* d_q, float* d_scale,
                 int32_t* d_isum, void* stream) {
    if (!d_gate || !d_up || !d_q || !d_scale || !d_isum || n == 0 || n % 256) return DQ_ERR_INVALID_ARG;
    const unsigned grid = (unsigned)((n / 256 + 3) / 4);
    if (gelu)
        silu_quant_kernel<DQ_ACT_GEGLU><<<grid, 256, 0, (hipStream_t)stream>>>(d_gate, d_up, (int)n, d_q, d_scale, d_isum);
    else
        silu_quant_kernel<DQ_ACT_SILU><<<grid, 256, 0, (hipStream_t)stream>>>(d_gate, d_up, (int)n, d_q, d_scale, d_isum);
    return dq_launch_status();
}

int dq_act_mul(const float* d_gate, const float* d_up, size_t n, int gelu, float* d_h, void* stream) {
    if (!d_gate || !d_up || !d_h) return DQ_ERR_INVALID_ARG;
    if (n == 0) return DQ_OK;
    if (n > (1u << 30)) return DQ_ERR_NOT_SUPPORTED;
    const unsigned grid = (unsigned)((n + 255) / 256);
    if (gelu)
        silu_mul_kernel<DQ_ACT_GEGLU><<<grid, 256, 0, (hipStream_t)stream>>>(d_gate, d_up, (int)n, d_h);
    else
        silu_mul_kernel<DQ_ACT_SILU><<<grid, 256, 0, (hipStream_t)stream>>>(d_gate, d_up, (int)n, d_h);
    return dq_launch_status();
}

extern "C" {

int dq_rope_kv_write(float* d_q, const float* d_k, const float* d_v, const float* d_rope, uint32_t n_head,
                     uint32_t n_head_kv, uint32_t hd, uint32_t n_rot, void* d_kc, void* d_vc, uint32_t pos,
                     const int32_t* d_pos, uint32_t n_ctx, void* stream) {
    return dq_rope_kv_write_post(d_q, d_k, d_v, d_rope, n_head, n_head_kv, hd, n_rot, d_kc, d_vc, pos, d_pos, n_ctx,
                                 DqQkvPost{}, stream);
}

}  // extern "C"

int dq_rope_kv_write_post(float* d_q, const float* d_k, const float* d_v, const float* d_rope, uint32_t n_head,
                          uint32_t n_head_kv, uint32_t hd, uint32_t n_rot, void* d_kc, void* d_vc, uint32_t pos,
                          const int32_t* d_pos, uint32_t n_ctx, const DqQkvPost& post, void* stream) {
    if (!d_q || !d_k || !d_v || !d_kc || !d_vc || n_ctx == 0) return DQ_ERR_INVALID_ARG;
    if (!dq_head_dim_supported(hd)) return DQ_ERR_NOT_SUPPORTED;
    if (d_rope && (n_rot == 0 || n_rot > hd || n_rot % 2)) return DQ_ERR_INVALID_ARG;
    if (!d_pos && pos >= n_ctx) return DQ_ERR_INVALID_ARG;
    const size_t pos_bytes = (size_t)n_head_kv * (hd / 32) * DQ_SZ_Q8_0;
    auto go = [&](auto kern) {
        kern<<<n_head + 2 * n_head_kv, 64, 0, (hipStream_t)stream>>>(d_q, d_k, d_v, d_rope, (int)n_head,
                                                                      (int)n_head_kv, (int)n_rot, (uint8_t*)d_kc,
                                                                      (uint8_t*)d_vc, pos_bytes, (int)pos, d_pos,
                                                                      (int)n_ctx, post);
    };
    if (hd == 64)
        go(rope_kv_kernel<64>);
    else if (hd == 128)
        go(rope_kv_kernel<128>);
    else
        go(rope_kv_kernel<256>);
    return dq_launch_status();
}

extern "C" {

int dq_layer_workspace_bytes(const dq_layer_t* L, uint32_t n_ctx, size_t* bytes) {
    if (!L || !bytes || n_ctx == 0) return DQ_ERR_INVALID_ARG;
    if (!layer_ok(L)) return DQ_ERR_NOT_SUPPORTED;
    *bytes = carve(L, n_ctx, nullptr).total;
    return DQ_OK;
}

int dq_layer_decode(const dq_layer_t* L, const float* d_x, float* d_x_out, const float* d_rope, uint32_t pos,
                    const int32_t* d_pos, uint32_t cc_start, void* d_kc, void* d_vc, uint32_t n_ctx, void* d_work,
                    size_t work_bytes, void* stream) {
    if (!L || !d_x || !d_x_out || !d_kc || !d_vc || !d_work || n_ctx == 0) return DQ_ERR_INVALID_ARG;
    if (!layer_ok(L)) return DQ_ERR_NOT_SUPPORTED;
    if (!d_pos && (pos >= n_ctx || cc_start > pos)) return DQ_ERR_INVALID_ARG;
    const LayerWs w = carve(L, n_ctx, (uint8_t*)d_work);
    if (work_bytes < w.total) return DQ_ERR_INVALID_ARG;
    const hipStream_t st = (hipStream_t)stream;
    const size_t E = L->n_embd, QD = (size_t)L->n_head * L->head_dim, KVD = (size_t)L->n_head_kv * L->head_dim;
    const size_t F = L->n_ff;
    // The matrices of a group read the normalised input quantized the way
    // their format's reference GEMV does: per 256 for Q4_K / Q6_K
    // (matmul_q4_k_pq / matmul_q6_k_pq on quantize_shared_q8k), per 32 for
    // Q8_0 / Q4_0 (matmul_q8_0 / matmul_q4_0). The per-256 activation comes
    // fused with the norm; the per-32 one, when some matrix needs it, from the
    // normalised float vector.
    auto norm_acts = [&](const float* x, const float* nw, bool need32) -> int {
        norm_quant_kernel<<<1, NQ_T, 0, st>>>(x, nullptr, nullptr, nw, (int)E, L->rms_eps, w.aq, w.as, w.ai,
                                               need32 ? w.yn : nullptr);
        DQ_TRY(dq_launch_status());
        if (need32) DQ_TRY(dq_quantize_act(DQ_ACT_Q8_0, w.yn, E, 1, w.bq, w.bs, w.bi, nullptr, stream));
        return DQ_OK;
    };
    // Jobs of one group split by activation kind: one grouped launch each.
    auto run_group = [&](const dq_gemv_job_t* jobs, int n, size_t cols) -> int {
        dq_gemv_job_t k4[4], k32[4];
        int nk = 0, n32 = 0;
        for (int j = 0; j < n; ++j) {
            if (per32(jobs[j].fmt)) k32[n32++] = jobs[j];
            else k4[nk++] = jobs[j];
        }
        if (nk) DQ_TRY(dq_gemv_group(k4, nk, cols, w.aq, w.as, w.ai, stream));
        if (n32) DQ_TRY(dq_gemv_group(k32, n32, cols, w.bq, w.bs, w.bi, stream));
        return DQ_OK;
    };
    // The RMSNorm and its per-256 quantization inside the group's GEMV kernel
    // when every matrix of the group is a K-quant (no launch before the
    // GEMV); else norm_quant, then the grouped launches.
    auto norm_group = [&](const float* x, const float* nw, const dq_gemv_job_t* jobs, int n) -> int {
        bool need32 = false;
        for (int j = 0; j < n; ++j) need32 = need32 || per32(jobs[j].fmt);
        if (!need32) {
            const int rc = dq_gemv_group_fused(jobs, n, E, DQ_FUSE_NORM, x, nw, L->rms_eps, stream);
            if (rc != DQ_ERR_NOT_SUPPORTED) return rc;
        }
        DQ_TRY(norm_acts(x, nw, need32));
        return run_group(jobs, n, E);
    };
    // ---- attention block
    {
        // the attention gate's matrix reads the same normalised input (:4108)
        const dq_gemv_job_t jobs[4] = {{L->fmt_q, L->wq, QD, w.q, nullptr},
                                       {L->fmt_k, L->wk, KVD, w.k, nullptr},
                                       {L->fmt_v, L->wv, KVD, w.v, nullptr},
                                       {L->fmt_ag, L->wag, L->n_head, w.ag, nullptr}};
        DQ_TRY(norm_group(d_x, L->attn_norm, jobs, L->wag ? 4 : 3));
    }
    // the optional biases and QK-norm, RoPE, the new K/V rows and attention in
    // one launch when the rotation covers the whole head (else the separate
    // post + RoPE + KV-write kernel first)
    DqQkvPost post = dq_layer_post(L);
    post.gate = L->wag ? w.ag : nullptr;
    const bool fused = !d_rope || L->n_rot == L->head_dim;
    if (!fused)
        DQ_TRY(dq_rope_kv_write_post(w.q, w.k, w.v, d_rope, L->n_head, L->n_head_kv, L->head_dim, L->n_rot, d_kc,
                                     d_vc, pos, d_pos, n_ctx, post, stream));
    // the attention also quantizes its output per 256 for a K-quant Wo
    const bool q256 = kquant(L->fmt_o);
    int8_t* oq = q256 ? w.aq : nullptr;
    if (fused)
        DQ_TRY(dq_attn_rope_kv_decode_post(w.q, w.k, w.v, d_rope, L->n_rot, d_kc, d_vc, L->n_head, L->n_head_kv,
                                           L->head_dim, cc_start, pos, d_pos, n_ctx, w.ao, oq, w.as, w.ai, w.attn,
                                           w.attn_bytes, post, stream));
    else
        DQ_TRY(dq_attn_decode_q8_post(w.q, d_kc, d_vc, L->n_head, L->n_head_kv, L->head_dim, cc_start, pos, d_pos,
                                      n_ctx, w.ao, oq, w.as, w.ai, w.attn, w.attn_bytes, post, stream));
    // the output projection plus the residual (x2 = x + Wo a), or with a
    // sandwich norm x2 = x + rms_norm(Wo a, post_attn_norm) (:4140-4147)
    auto residual = [&](int fmt, const void* wm, size_t rows, size_t cols, const int8_t* xq, const float* xs,
                        const int32_t* xi, const float* res, const float* post, float* out) -> int {
        if (!post) return dq_gemv_add(fmt, wm, rows, cols, xq, xs, xi, res, out, stream);
        DQ_TRY(dq_gemv(fmt, wm, rows, cols, xq, xs, xi, w.tmp, stream));
        return dq_post_norm_add(w.tmp, post, res, out, rows, 1, L->rms_eps, stream);
    };
    if (q256) {
        DQ_TRY(residual(L->fmt_o, L->wo, E, QD, w.aq, w.as, w.ai, d_x, L->post_attn_norm, w.x2));
    } else {
        DQ_TRY(dq_quantize_act(DQ_ACT_Q8_0, w.ao, QD, 1, w.bq, w.bs, w.bi, nullptr, stream));
        DQ_TRY(residual(L->fmt_o, L->wo, E, QD, w.bq, w.bs, w.bi, d_x, L->post_attn_norm, w.x2));
    }
    // ---- feed-forward block
    {
        const dq_gemv_job_t jobs[2] = {{L->fmt_gate, L->wgate, F, w.gate, nullptr},
                                       {L->fmt_up, L->wup, F, w.up, nullptr}};
        // gate and up paired in one kernel that also applies the norm before
        // and act(gate) * up after them: h (in w.gate) leaves as one fp32
        // vector, which the down GEMV quantizes in its own kernel (with the
        // residual in its epilogue, or before the sandwich norm)
        const int rc = dq_gemv_group_fused(jobs, 2, E, L->act_gelu ? DQ_FUSE_NORM_GEGLU : DQ_FUSE_NORM_SILU, w.x2,
                                           L->ffn_norm, L->rms_eps, stream);
        if (rc != DQ_ERR_NOT_SUPPORTED) {
            DQ_TRY(rc);
            const float* post = L->post_ffn_norm;
            const dq_gemv_job_t dj = {L->fmt_down, L->wdown, E, post ? w.tmp : d_x_out, post ? nullptr : w.x2};
            DQ_TRY(dq_gemv_group_f32(&dj, 1, F, w.gate, stream));
            return post ? dq_post_norm_add(w.tmp, post, w.x2, d_x_out, E, 1, L->rms_eps, stream) : DQ_OK;
        }
        DQ_TRY(norm_group(w.x2, L->ffn_norm, jobs, 2));
    }
    if (kquant(L->fmt_down)) {
        // act(gate) * up and its per-256 quantization inside the down GEMV's
        // kernel where it applies (with the residual in its epilogue, or
        // before the sandwich norm)
        const float* post = L->post_ffn_norm;
        const dq_gemv_job_t job = {L->fmt_down, L->wdown, E, post ? w.tmp : d_x_out, post ? nullptr : w.x2};
        const int rc = dq_gemv_group_fused(&job, 1, F, L->act_gelu ? DQ_FUSE_GEGLU : DQ_FUSE_SILU, w.gate, w.up, 0.0f,
                                         stream);
        if (rc != DQ_ERR_NOT_SUPPORTED) {
            DQ_TRY(rc);
            return post ? dq_post_norm_add(w.tmp, post, w.x2, d_x_out, E, 1, L->rms_eps, stream) : DQ_OK;
        }
        DQ_TRY(dq_act_quant(w.gate, w.up, F, L->act_gelu, w.aq, w.as, w.ai, stream));
        DQ_TRY(residual(L->fmt_down, L->wdown, E, F, w.aq, w.as, w.ai, w.x2, L->post_ffn_norm, d_x_out));
    } else {
        DQ_TRY(dq_act_mul(w.gate, w.up, F, L->act_gelu, w.yn, stream));
        DQ_TRY(dq_quantize_act(DQ_ACT_Q8_0, w.yn, F, 1, w.bq, w.bs, w.bi, nullptr, stream));
        DQ_TRY(residual(L->fmt_down, L->wdown, E, F, w.bq, w.bs, w.bi, w.x2, L->post_ffn_norm, d_x_out));
    }
    return DQ_OK;
}

}  // extern "C"
