/*
 * dq_oracle.h - CPU restatement of DesireeIA's quantized-weight compute path.
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT CODE. Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load this library, and only as the
 * checker / the timed CPU baseline. The HIP library never links or calls it.
 *
 * Every function restates one function of the reference engine (paths are
 * relative to src/DesireeIA.LocaleEngine/ in the reference tree); the
 * citation sits next to each definition in dq_oracle.c.
 *
 * Parity pins (what checks each part; see tests/test_oracle_*.py):
 *   fp16<->fp32 ........ exhaustive over all 65536 halves vs numpy and the
 *                        compiled reference; RNE ties + random floats vs numpy
 *   dequant ............ reference KAT (Q4_0 j-8), brute-force round trip of
 *                        the 6-bit scale packing, bit-exact vs compiled ref
 *   quantizers ......... closed-form KATs (zero block, .5 ties, amax->127),
 *                        bit-exact vs compiled ref
 *   GEMV/GEMM .......... fp64 evaluation on the same integers, dequant+fp64
 *                        (the reference selftest's 5% bound), compiled ref
 *   attention/route .... fp64 softmax attention, reference router KATs,
 *                        brute-force top-k, compiled ref
 *   layer/MoE .......... composition of the pinned pieces vs an fp64 twin
 */
#ifndef DQ_ORACLE_H
#define DQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Error codes of the reference ABI (include/desireeia/abi.h:113-122). */
#define DQO_OK 0
#define DQO_ERR_INVALID_ARG (-1)
#define DQO_ERR_NOT_SUPPORTED (-2)

/* GGUF type ids (quant/quant.h:439-476). */
#define DQO_Q4_0 2
#define DQO_Q8_0 8
#define DQO_Q8_1 9
#define DQO_Q4_K 12
#define DQO_Q6_K 14

float dqo_fp16_to_fp32(uint16_t h);
uint16_t dqo_fp32_to_fp16(float f);

size_t dqo_type_size(int type);
int dqo_blck_size(int type);
size_t dqo_row_size(int type, int64_t n);
int dqo_dequantize_row(int type, const void* src, float* dst, int64_t n);

void dqo_get_scale_min_k4(int j, const uint8_t* q, uint8_t* sc, uint8_t* mn);
void dqo_pack_scales_min_k4(const uint8_t* sc, const uint8_t* mn, uint8_t* out);

/* Activation quantizers. n is a multiple of 32 (256 for q8k_rep). */
void dqo_quantize_q8_0(const float* x, size_t n, int8_t* q, float* d);
void dqo_quantize_q8_1(const float* x, size_t n, int8_t* q, float* d,
                       int32_t* isum, float* fsum);
void dqo_quantize_q8k_rep(const float* x, size_t n, int8_t* q, float* d32,
                          int32_t* isum32);
void dqo_kv_quantize_row(const float* x, size_t dim, uint8_t* out);

/* Batch-1 GEMV with the reference CPU semantics (quantizes x itself).
 * Rows [row0, row1) are computed; row1 == 0 means all rows. */
int dqo_matmul(int type, const uint8_t* w, size_t rows, size_t cols,
               const float* x, float* y, size_t row0, size_t row1);
/* Same integers, fp64 accumulation of the exact same formula. */
int dqo_matmul_f64(int type, const uint8_t* w, size_t rows, size_t cols,
                   const float* x, double* y, size_t row0, size_t row1);
/* GEMV on pre-quantized activations (matmul_q4_k_pq / matmul_q6_k_pq). */
int dqo_matmul_pq(int type, const uint8_t* w, size_t rows, size_t cols,
                  const int8_t* xq, const float* d32, const int32_t* isum32,
                  float* y, size_t row0, size_t row1);

/* Prefill GEMM, i8_gemm semantics. y is [n_tok][rows]; rows [row0,row1)
 * and tokens [t0,t1) are computed (0,0 = all). */
int dqo_gemm(int type, const uint8_t* w, size_t rows, size_t cols,
             const float* x, size_t n_tok, float* y,
             size_t row0, size_t row1, size_t t0, size_t t1);
int dqo_gemm_f64(int type, const uint8_t* w, size_t rows, size_t cols,
                 const float* x, size_t n_tok, double* y,
                 size_t row0, size_t row1, size_t t0, size_t t1);
/* unpack_row's integer weights, per-16 scales and per-16 Q4_K offsets of every
 * row (the weight operands of the prefill GEMM semantics). */
int dqo_gemm_operands(int type, const uint8_t* w, size_t rows, size_t cols, int8_t* q, float* a, float* m);

/* Q8_0 KV rows (kv/kv_quant.cpp). */
float dqo_kv_dot_q8_0(const float* q, const uint8_t* row, size_t dim);
void dqo_kv_axpy_q8_0(float* y, const uint8_t* row, size_t dim, float w);

/* Decode attention over a Q8_0 cache laid out [pos][kv_head][row_bytes]
 * (one layer). q/out are [n_head][hd]. Positions [cc_start, pos]. */
void dqo_attn_decode_q8(const float* q, const uint8_t* kc, const uint8_t* vc,
                        uint32_t n_head, uint32_t n_head_kv, uint32_t hd,
                        uint32_t cc_start, uint32_t pos, float* out);
void dqo_attn_decode_q8_f64(const float* q, const uint8_t* kc, const uint8_t* vc,
                            uint32_t n_head, uint32_t n_head_kv, uint32_t hd,
                            uint32_t cc_start, uint32_t pos, double* out);

/* Router: softmax top-k. Writes k ids and weights; returns k. */
uint32_t dqo_moe_route(const float* logits, uint32_t n, uint32_t k, int norm_w,
                       float w_scale, uint32_t* ids, float* wts);

void dqo_rms_norm(const float* x, const float* w, float* y, size_t n, float eps);
void dqo_rope_cache(float* cache, size_t n_rot, uint32_t pos, float theta_base);
void dqo_rope_neox(float* v, size_t n_rot, const float* cache);
float dqo_silu(float v);
float dqo_gelu_tanh(float v);
float dqo_exp_avx2(float x);
float dqo_geglu(float g);
void dqo_softmax(float* s, size_t n);
/* Prefill attention over a Q8_0 KV cache (core/attn_cpu.cpp:128-390):
 * q_all/out [n_tok][q_dim]; K/V row of (pos, kv head) at base + pos*pos_bytes
 * + kv_head*row_bytes; token t at position pos0 + t; n_swa 0 = causal. */
int dqo_attn_prefill_q8(const float* q_all, float* out, uint32_t n_tok, uint32_t n_head, uint32_t hpk,
                        uint32_t hd, uint32_t q_dim, const uint8_t* kbase, const uint8_t* vbase,
                        size_t row_bytes, size_t pos_bytes, uint32_t pos0, uint32_t n_swa, float inv_d);


/* One Llama-style decode layer (models/dense_forward.cpp:3897-4257) with
 * Q4_K/Q6_K weights and a Q8_0 KV cache of one layer. The new K/V rows are
 * written into kc/vc at `pos`. Intermediates are optional (may be NULL). */
typedef struct {
    uint32_t n_embd, n_head, n_head_kv, head_dim, n_ff;
    float rms_eps, rope_theta;
    int fmt_q, fmt_k, fmt_v, fmt_o, fmt_gate, fmt_up, fmt_down; /* GGUF ids */
    const uint8_t *wq, *wk, *wv, *wo, *wgate, *wup, *wdown;
    const float *attn_norm, *ffn_norm;
    /* optional (NULL = absent): Q/K/V biases added to the projections
     * (add_bias, :3904-3908), then the per-head QK-norm (rms_norm_vec over
     * each head with a head_dim weight, :3915-3931), both before RoPE */
    const float *bq, *bk, *bv, *q_norm, *k_norm;
    /* 1: gated GELU instead of SiLU (decode: geglu_inplace, :4212-4213;
     * batch: gelu_tanh per element, :3608-3609) */
    int act_gelu;
    /* optional sandwich norms (NULL = absent): rms_norm_vec of the output
     * projection and of the FFN output, each before its residual
     * (:4140-4142, :4245-4247; batch :3546-3548, :3618-3620) */
    const float *post_attn_norm, *post_ffn_norm;
    /* optional per-head output gate (NULL = absent; DenseQuirks::attn_gate):
     * [n_head][n_embd] of format fmt_ag, multiplied with the same normalized
     * input as Q/K/V; head h of the attention output is scaled by
     * 1 / (1 + exp(-gate_h)) before the output projection (decode :4102-4114,
     * batch :3522-3537) */
    const uint8_t* wag;
    int fmt_ag;
} dqo_layer_t;

/* The per-head output gate of one token: head h of ao ([n_head][hd]) times
 * 1 / (1 + exp(-gate[h])) (dense_forward.cpp:4102-4114). */
void dqo_attn_gate_apply(float* ao, const float* gate, uint32_t n_head, size_t hd);

int dqo_layer_decode(const dqo_layer_t* L, uint8_t* kc, uint8_t* vc, uint32_t pos,
                     const float* x, float* x_out, float* q_out, float* k_out,
                     float* v_out, float* attn_out);

/* The same layer for a prompt chunk of n_tok tokens at positions pos0..
 * (the batch branch of models/dense_forward.cpp:3260-3624): x/x_out
 * [n_tok][n_embd]; the chunk's K/V rows are written into kc/vc. */
int dqo_layer_prefill(const dqo_layer_t* L, uint8_t* kc, uint8_t* vc, uint32_t pos0, uint32_t n_tok,
                      uint32_t n_swa, const float* x, float* x_out);

/* MoE expert FFN for n_tok tokens (dense_forward.cpp:1524-1560, combine at
 * :4160-4181). Experts stacked: gate/up [n_expert*n_ff][n_embd] rows,
 * down [n_expert*n_embd][n_ff] rows, all of format fmt. */
int dqo_moe_ffn(int fmt, const uint8_t* wgate, const uint8_t* wup, const uint8_t* wdown,
                uint32_t n_expert, uint32_t n_embd, uint32_t n_ff,
                const float* x, const float* logits, uint32_t n_tok, uint32_t k_used,
                int norm_w, float* out, uint32_t t0, uint32_t t1);

/* Exhaustive checks, over a range [lo, hi) of float bit patterns, of the
 * float identities the GPU quantizers rely on instead of a division and a
 * clamped conversion. Each returns the number of inputs where the identity
 * fails (NaN and inf inputs are skipped).
 *   div127:    (float)((double)a * (1.0 / 127.0)) == a / 127.0f
 *   rint_byte: low byte of bits(p + 1.5 * 2^23) == (int8_t)rintf(p), |p| <= 128
 *   id_bound:  for a > 0 with finite id, rint(a * id) <= 127 for both
 *              id = 1 / (a / 127) (per-32) and id = 127 / a (per-256), so
 *              |x * id| never needs the clamp when |x| <= a. */
uint64_t dqo_check_div127(uint32_t lo, uint32_t hi);
uint64_t dqo_check_rint_byte(uint32_t lo, uint32_t hi);
uint64_t dqo_check_id_bound(uint32_t lo, uint32_t hi);

#ifdef __cplusplus
}
#endif
#endif
