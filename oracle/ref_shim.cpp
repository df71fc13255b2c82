// ref_shim.cpp - C entry points into the reference engine's own CPU code,
// compiled from the reference sources where they lie (see Makefile, target
// `ref`). TEST INFRASTRUCTURE: the resulting oracle/_ref library is used only
// to validate the restatement in dq_oracle.c and as the "reference" CPU
// baseline timed by bench.py. It is never linked into the HIP library.
//
// Each wrapper forwards to one reference function (paths relative to
// src/DesireeIA.LocaleEngine/):
//   desireeia_dequantize_row ...... quant/quant.cpp:912
//   desireeia_fp16<->fp32 ......... quant/quant.h:285-323
//   quantize_q8_0 ................. core/quant.cpp:15
//   quantize_act_q8k_rep .......... core/matmul.cpp:1660
//   matmul_q8_0/q4_0/q4_k/q6_k .... core/matmul.cpp:294,343,2008,2569
//   matmul_*_batch ................ core/matmul.cpp:2090-2125, :848-860
//   kv_quantize_row/dot/axpy ...... kv/kv_quant.cpp:31,58,102
//   moe_route ..................... models/moe_route.cpp:77
//   attention_prefill_cpu_q8 ...... core/attn_cpu.cpp:128
//   decode attention .............. models/dense_forward.cpp:4014-4066: per
//                                   query head (parallel_units over heads)
//                                   kv_dot_q8_0 scores, softmax_inplace
//                                   (:805-821, restated: float max, double
//                                   sum), kv_axpy_q8_0 accumulation
//   Sampler::sample_candidates .... core/sampler.cpp:298 (draw_uniform :131)
//   ThreadPool::set_thread_override core/thread_pool.cpp:36
#include "core/engine.h"
#include "core/i8gemm.h"
#include "core/thread_pool.h"
#include "kv/kv_quant.h"
#include "models/moe_route.h"
#include "core/sampler.h"
#include "quant/quant.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

using namespace desireeia;

extern "C" {

void dqr_set_threads(int n) { ThreadPool::set_thread_override(n); }
int dqr_threads() { return (int)ThreadPool::global().worker_count(); }
const char* dqr_i8_isa() { return i8_gemm_isa(); }

float dqr_fp16_to_fp32(uint16_t h) { return desireeia_fp16_to_fp32(h); }
uint16_t dqr_fp32_to_fp16(float f) { return desireeia_fp32_to_fp16(f); }

int dqr_dequantize_row(int type, const void* src, float* dst, int64_t n) {
    return desireeia_dequantize_row(type, src, dst, n);
}

void dqr_quantize_q8_0(const float* x, size_t n, int8_t* q, float* d) {
    std::vector<int8_t> vq;
    std::vector<float> vd;
    std::vector<uint8_t> signs;
    quantize_q8_0(x, n, vq, vd, signs);
    std::memcpy(q, vq.data(), n);
    std::memcpy(d, vd.data(), vd.size() * sizeof(float));
}

void dqr_quantize_q8k_rep(const float* x, size_t n, int8_t* q, float* d32, int32_t* isum32) {
    std::vector<int8_t> vq;
    std::vector<float> vd;
    std::vector<int32_t> vs;
    quantize_act_q8k_rep(x, n, vq, vd, vs);
    std::memcpy(q, vq.data(), n);
    std::memcpy(d32, vd.data(), vd.size() * sizeof(float));
    std::memcpy(isum32, vs.data(), vs.size() * sizeof(int32_t));
}

int dqr_matmul(int type, const uint8_t* w, size_t rows, size_t cols, const float* x, float* y) {
    switch (type) {
    case 2: return matmul_q4_0(w, rows, cols, x, y);
    case 8: return matmul_q8_0(w, rows, cols, x, y);
    case 12: return matmul_q4_k(w, rows, cols, x, y);
    case 14: return matmul_q6_k(w, rows, cols, x, y);
    default: return DESIREEIA_ERR_NOT_SUPPORTED;
    }
}

int dqr_matmul_batch(int type, const uint8_t* w, size_t rows, size_t cols, const float* x,
                     size_t n_tok, float* y) {
    switch (type) {
    case 2: return matmul_q4_0_batch(w, rows, cols, x, n_tok, y);
    case 8: return matmul_q8_0_batch(w, rows, cols, x, n_tok, y);
    case 12: return matmul_q4_k_batch(w, rows, cols, x, n_tok, y);
    case 14: return matmul_q6_k_batch(w, rows, cols, x, n_tok, y);
    default: return DESIREEIA_ERR_NOT_SUPPORTED;
    }
}

void dqr_kv_quantize_row(const float* x, size_t dim, uint8_t* out) { kv_quantize_row(x, dim, out); }
float dqr_kv_dot_q8_0(const float* q, const uint8_t* row, size_t dim) { return kv_dot_q8_0(q, row, dim); }
void dqr_kv_axpy_q8_0(float* y, const uint8_t* row, size_t dim, float w) { kv_axpy_q8_0(y, row, dim, w); }

uint32_t dqr_moe_route(const float* logits, uint32_t n, uint32_t k, int norm_w, float w_scale,
                       uint32_t* ids, float* wts) {
    std::vector<float> l(logits, logits + n);
    auto sel = moe_route(l, k, norm_w != 0, w_scale);
    for (size_t i = 0; i < sel.size(); ++i) {
        ids[i] = sel[i].first;
        wts[i] = sel[i].second;
    }
    return (uint32_t)sel.size();
}

int dqr_attention_prefill_q8(const float* q_all, float* out, uint32_t n_tok, uint32_t n_head, uint32_t hpk,
                             uint32_t hd, uint32_t q_dim, const uint8_t* kbase, const uint8_t* vbase,
                             size_t row_bytes, size_t pos_bytes, uint32_t pos0, uint32_t n_swa, float inv_d) {
    return attention_prefill_cpu_q8(q_all, out, n_tok, n_head, hpk, hd, q_dim, kbase, vbase, row_bytes, pos_bytes,
                                    pos0, n_swa, inv_d);
}

// Decode attention of one token over positions [cc_start, pos] of a Q8_0
// cache laid out [pos][kv head][hd/32 blocks], as the engine's CPU decode
// step runs it (quantized-KV branch, no ALiBi, no window).
void dqr_attn_decode_q8(const float* q, const uint8_t* kc, const uint8_t* vc, uint32_t n_head, uint32_t n_head_kv,
                        uint32_t hd, uint32_t cc_start, uint32_t pos, float* out) {
    const size_t row_bytes = (size_t)hd / 32 * sizeof(block_q8_0);
    const size_t pos_bytes = (size_t)n_head_kv * row_bytes;
    const uint32_t hpk = n_head / n_head_kv;
    const float inv_d = 1.0f / std::sqrt((float)hd);
    std::vector<float> scores((size_t)n_head * (pos + 1));
    parallel_units(n_head, [&](size_t h0, size_t h1) {
        for (uint32_t h = (uint32_t)h0; h < (uint32_t)h1; ++h) {
            float* s = scores.data() + (size_t)h * (pos + 1);
            const float* qh = q + (size_t)h * hd;
            const uint8_t* kb = kc + (size_t)(h / hpk) * row_bytes;
            const uint8_t* vb = vc + (size_t)(h / hpk) * row_bytes;
            for (uint32_t cc = cc_start; cc <= pos; ++cc) s[cc] = kv_dot_q8_0(qh, kb + cc * pos_bytes, hd) * inv_d;
            float m = -INFINITY;
            for (uint32_t cc = cc_start; cc <= pos; ++cc) m = std::max(m, s[cc]);
            double sum = 0.0;
            for (uint32_t cc = cc_start; cc <= pos; ++cc) {
                s[cc] = expf(s[cc] - m);
                sum += s[cc];
            }
            for (uint32_t cc = cc_start; cc <= pos; ++cc) s[cc] /= (float)sum;
            float* oh = out + (size_t)h * hd;
            for (uint32_t d = 0; d < hd; ++d) oh[d] = 0.0f;
            for (uint32_t cc = cc_start; cc <= pos; ++cc) kv_axpy_q8_0(oh, vb + cc * pos_bytes, hd, s[cc]);
        }
    });
}

// The host draw over candidates, and the uniform number the device path is
// given for the same generator state (draw_uniform on a saved state, which is
// then restored): the device pick for that u must be this pick. `skip` draws
// advance the generator first.
int32_t dqr_sample_candidates(float temperature, int32_t top_k, float top_p, float pen_repeat, float pen_freq,
                              float pen_present, int32_t pen_last_n, uint32_t seed, uint32_t skip,
                              const int32_t* ids, const float* vals, size_t n, const int32_t* hist, size_t nh,
                              float* u_out) {
    SamplerParams p;
    p.temperature = temperature;
    p.top_k = top_k;
    p.top_p = top_p;
    p.penalty_repeat = pen_repeat;
    p.penalty_freq = pen_freq;
    p.penalty_present = pen_present;
    p.penalty_last_n = pen_last_n;
    p.seed = seed;
    Sampler s;
    s.configure(p);
    for (uint32_t i = 0; i < skip; ++i) (void)s.draw_uniform();
    const std::mt19937 st = s.rng_state();
    *u_out = s.draw_uniform();
    s.set_rng_state(st);
    std::vector<int32_t> vi(ids, ids + n);
    std::vector<float> vv(vals, vals + n);
    std::vector<int32_t> h(hist, hist + nh);
    return s.sample_candidates(vi, vv, h);
}

}  // extern "C"
