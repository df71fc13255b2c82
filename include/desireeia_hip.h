/*
 * desireeia_hip.h - C ABI of the MI355X (gfx950) quantized compute path.
 *
 * Two layers, both plain C (extern "C", pointers and sizes, no torch or C++
 * types), all returning a desireeia_error code (0 = OK, -1 invalid argument,
 * -2 not supported: shape/format not covered, nothing was done, -3 device
 * failure). Reference paths are relative to src/DesireeIA.LocaleEngine/.
 *
 * 1. Kernel layer (dq_*): device pointers, stream-ordered, asynchronous, no
 *    allocation. `stream` is a hipStream_t (NULL = the default stream).
 *
 * 2. Engine layer: the GPU operator entry points the reference engine's model
 *    code calls (core/engine.h:502-811, compiled there under
 *    DESIREEIA_CUDA_ENABLED), same names, argument meaning and error
 *    behaviour, with host pointers for x/y and one synchronisation per call;
 *    a thin C++ shim maps the engine's calls (references, std types) onto them.
 */
#ifndef DESIREEIA_HIP_H
#define DESIREEIA_HIP_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes: the values of desireeia_error (include/desireeia/abi.h:113-122). */
#define DQ_OK 0
#define DQ_ERR_INVALID_ARG (-1)
#define DQ_ERR_NOT_SUPPORTED (-2)
#define DQ_ERR_IO (-3)

/* Device weight formats: the values of DESIREEIA_CUDA_FMT_* (core/engine.h:521-527),
 * with 0 = Q8_0 as the reference backend uses it (core/engine.h:726). */
#define DQ_FMT_Q8_0 0
#define DQ_FMT_Q4_0 1
#define DQ_FMT_Q4_K 5
#define DQ_FMT_Q6_K 7
/* Flag on a prefill-GEMM format (dq_gemm, dq_gemm_f16act, dq_gemm_workspace_bytes): the weights are the
 * tile copy of dq_gemm_tiles_pack, not the packed rows. */
#define DQ_FMT_GEMM_TILES 0x200
/* Q4_K experts in the expert-tile layout of dq_moe_tiles_pack (dq_moe_t only). */
#define DQ_FMT_Q4_K_TILES 0x105

/* GGUF type ids for dq_dequantize_row (quant/quant.h:439-476). */
#define DQ_TYPE_Q4_0 2
#define DQ_TYPE_Q8_0 8
#define DQ_TYPE_Q8_1 9
#define DQ_TYPE_Q4_K 12
#define DQ_TYPE_Q6_K 14

/* Activation quantizers for dq_quantize_act. */
#define DQ_ACT_Q8_0 0   /* one scale per 32: core/quant.cpp:15-50 (quantize_q8_0) */
#define DQ_ACT_Q8K_REP 1 /* one scale per 256, replicated per 32: core/matmul.cpp:1660-1778 */

/* ------------------------------------------------------------ kernel layer */

/* Library version / device query. */
int dq_version(void);
int dq_device_count(void);

/* Streaming-read probe (no counterpart in the reference: it measures this
 * device's read ceiling for the benchmark). Reads `bytes` (a multiple of
 * depth_kb KiB, 16-byte aligned) once with waves_per_cu waves per compute
 * unit (1..4, or a multiple of 4 up to 32; others -2); each wave reads depth_kb (4, 8 or 16) KiB per step, all loads
 * of a step in flight together, 64 lanes x 16 contiguous bytes per load
 * instruction. Writes d_sink[0] only if the XOR of the words equals `never`. */
int dq_stream_read(const void* d_src, size_t bytes, uint32_t waves_per_cu, uint32_t depth_kb, uint32_t* d_sink,
                   uint32_t never, void* stream);

/* LDS read probe (no counterpart in the reference: it shows which lanes this
 * device's LDS serves together for a 16-byte read). n_wg one-wave workgroups;
 * lane l of each reads 16 bytes at LDS byte offset d_offsets[l] + it * stride
 * (64 device int32; wrapped into a 64 KiB buffer, 16-byte aligned) for iters
 * iterations (at most 2^20), one ds_read_b128 each; run it under a
 * SQ_LDS_BANK_CONFLICT counter pass. Writes d_sink[0] only if the folded
 * words equal `never`. */
int dq_lds_read_probe(const int32_t* d_offsets, uint32_t iters, uint32_t n_wg, int32_t stride, uint32_t* d_sink,
                      uint32_t never, void* stream);

/* Replaces desireeia_dequantize_row (quant/quant.cpp:912-984) for the on-path
 * types Q4_0, Q8_0, Q8_1, Q4_K, Q6_K: GGUF blocks in, n fp32 values out,
 * bit-exact. n must be a multiple of the block size. Other types: -2. */
int dq_dequantize_row(int type, const void* d_src, float* d_dst, int64_t n, void* stream);

/* Size of the on-device layout of a rows x cols matrix of format fmt, and the
 * on-device conversion from GGUF rows (the layout cuda_upload_weights owns,
 * backend_cuda.cu:2910-2923, 3024-3107). d_gguf and d_dev must not overlap. */
int dq_weights_bytes(int fmt, size_t rows, size_t cols, size_t* bytes);
int dq_weights_pack(int fmt, const void* d_gguf, size_t rows, size_t cols, void* d_dev,
                    void* stream);
/* Dequantizes a packed device matrix to fp32 [rows][cols]; the values are
 * bit-identical to desireeia_dequantize_row on the GGUF rows. */
int dq_weights_dequantize(int fmt, const void* d_dev, size_t rows, size_t cols, float* d_out,
                          void* stream);

/* Activation quantization of n_tok rows of cols floats (cols % 32 == 0; %256
 * for DQ_ACT_Q8K_REP). Outputs: q int8 [n_tok][cols], scale float
 * [n_tok][cols/32], isum int32 [n_tok][cols/32] (sum of the 32 q), fsum float
 * [n_tok][cols/32] (sequential float sum of the 32 inputs, the min-term input
 * of the prefill GEMM, core/i8gemm_impl.h:50-82). isum/fsum may be NULL.
 * The integers and scales are bit-identical to the reference quantizer. */
int dq_quantize_act(int kind, const float* d_x, size_t cols, size_t n_tok, int8_t* d_q,
                    float* d_scale, int32_t* d_isum, float* d_fsum, void* stream);

/* GGUF block_q8_1 form (quant/quant.h:105-116): fp16 d, fp16 s = d * sum(q),
 * 32 int8, for n floats (n % 32 == 0), per-32 quantize_q8_0 integers. */
int dq_quantize_q8_1_blocks(const float* d_x, size_t n, void* d_blocks, void* stream);

/* Batch-1 GEMV y[rows] = W x on a packed device matrix, x given as the
 * activation triple of dq_quantize_act (DQ_ACT_Q8_0 for Q8_0/Q4_0 - the
 * semantics of matmul_q8_0/matmul_q4_0, core/matmul.cpp:294-417; DQ_ACT_Q8K_REP
 * for Q4_K/Q6_K - matmul_q4_k_pq/matmul_q6_k_pq, :2023-2027, :2580-2584).
 * d_xsum is required for Q4_0 and Q4_K. */
int dq_gemv(int fmt, const void* d_w, size_t rows, size_t cols, const int8_t* d_xq,
            const float* d_xscale, const int32_t* d_xsum, float* d_y, void* stream);
/* The same GEMV with a residual: y = W x + res (res may alias y). The
 * residual adds of the decoder layer (models/dense_forward.cpp, proj += x
 * after the output projection, x_out = ffn_out + proj after ffn_down). */
int dq_gemv_add(int fmt, const void* d_w, size_t rows, size_t cols, const int8_t* d_xq,
                const float* d_xscale, const int32_t* d_xsum, const float* d_res, float* d_y, void* stream);

/* Grouped GEMV: up to 4 matrices with the same cols reading the same
 * activation, one launch per distinct format, except that Q4_K and Q6_K
 * matrices share one launch where cols <= 4096 (matmul_fused_pq,
 * core/matmul.cpp:2586-2639, reached through matvec_shared_group,
 * models/dense_forward.cpp:554-601; the device counterpart of
 * matmul_kquant_cuda_resident_same_x, core/engine.h:537-538). Each job's
 * d_res may be NULL (no residual). Every job must use the activation kind of
 * the first (Q8_0/Q4_0: DQ_ACT_Q8_0; Q4_K/Q6_K: DQ_ACT_Q8K_REP); mixing the
 * two kinds or more than 4 jobs: -2, nothing launched. */
typedef struct {
    int fmt;
    const void* d_w;
    size_t rows;
    float* d_y;
    const float* d_res;
} dq_gemv_job_t;
int dq_gemv_group(const dq_gemv_job_t* jobs, size_t n, size_t cols, const int8_t* d_xq, const float* d_xscale,
                  const int32_t* d_xsum, void* stream);

/* The same GEMVs on the fp32 activation d_x [cols]: every workgroup quantizes
 * x in-kernel with the format's reference quantizer (the integers, scales and
 * sums of dq_quantize_act, so the results are bit-identical to dq_quantize_act
 * followed by dq_gemv / dq_gemv_group), saving the separate quantize launch.
 * In the group form every format may be mixed. cols <= 49152; larger: -2. */
int dq_gemv_f32(int fmt, const void* d_w, size_t rows, size_t cols, const float* d_x, float* d_y, void* stream);
int dq_gemv_group_f32(const dq_gemv_job_t* jobs, size_t n, size_t cols, const float* d_x, void* stream);

/* Prefill GEMM y[n_tok][rows] = x[n_tok][cols] W^T for Q4_K, Q6_K, Q8_0 and
 * Q4_0 (cols % 256 == 0), with the semantics of matmul_<fmt>_batch on the
 * i8_gemm path (Q4_K/Q6_K/Q4_0 from 4 tokens, Q8_0 from 2; core/matmul.cpp
 * :848-860, 2090-2125 -> :806-845): per-32 activation quantization, exact
 * float block sums for the Q4_K min term. Runs on fp16
 * MFMA over pre-scaled operands (result within ~3e-4 relative of the
 * reference); each token's operand row carries a power-of-two range scale
 * (undone exactly on the output), so any finite activation magnitude stays
 * inside fp16. `d_work` (dq_gemm_workspace_bytes() bytes) holds the quantized
 * activations, for Q4_K their per-32 block sums (the min-term input, tokens
 * contiguous per super-block), and their row scales. d_y may overlap d_x
 * (the K-split plans then clear y after the quantizer, in a launch of their
 * own, instead of inside it). Other formats and cols % 256 != 0: -2. */
int dq_gemm_workspace_bytes(int fmt, size_t rows, size_t cols, size_t n_tok, size_t* bytes);
int dq_gemm(int fmt, const void* d_w, size_t rows, size_t cols, const float* d_x, size_t n_tok,
            float* d_y, void* d_work, size_t work_bytes, void* stream);
/* The two halves of dq_gemm: the activation quantizer into the workspace
 * layout, and the GEMM on an already quantized activation (several weight
 * matrices reading the same x share one quantization). */
int dq_quantize_act_f16(int fmt, const float* d_x, size_t cols, size_t n_tok, void* d_work, void* stream);
int dq_gemm_f16act(int fmt, const void* d_w, size_t rows, size_t cols, const void* d_work, size_t n_tok,
                   float* d_y, void* stream);
/* An opt-in second copy of a matrix for prefill-heavy use: the tile layout
 * in which every 64-row slice's bytes of one GEMM stage (the quant
 * sub-planes in the kernel's LDS order, then the stage's scales) are one
 * contiguous run, so each weight DMA of the GEMM reads 64 lanes x 16
 * consecutive bytes instead of 4 lanes per 64-byte row piece. d_packed is
 * the packed form of cuda_upload_weights / dq_weights_pack; d_tiles receives
 * dq_gemm_tiles_bytes() bytes (rows rounded up to 256). Pass
 * fmt | DQ_FMT_GEMM_TILES and the tile copy to dq_gemm / dq_gemm_f16act:
 * the results are bit-identical to the packed rows'. The packed rows stay
 * what the decode GEMV reads, so a matrix with both forms holds its weights
 * twice. No counterpart in the reference (its prefill reads the GGUF
 * blocks). */
int dq_gemm_tiles_bytes(int fmt, size_t rows, size_t cols, size_t* bytes);
int dq_gemm_tiles_pack(int fmt, const void* d_packed, size_t rows, size_t cols, void* d_tiles, void* stream);

/* Q8_0 KV cache of one layer, laid out [pos][kv_head][hd/32 blocks of 34 B]
 * (models/dense_forward.cpp:2425, :4038-4043). dq_kv_write replaces
 * write_kv_cache (:2552-2605): it quantizes the new K and V rows
 * (n_head_kv * hd floats each, kv_quantize_row, kv/kv_quant.cpp:31-56,
 * bit-exact) into position `pos`. With d_pos != NULL the position is read
 * from device memory when the kernel runs (graph replay; clamped to
 * [0, n_ctx)) and `pos` is ignored. */
int dq_kv_write(const float* d_k, const float* d_v, uint32_t n_head_kv, uint32_t hd, void* d_kc, void* d_vc,
                uint32_t pos, const int32_t* d_pos, uint32_t n_ctx, void* stream);

/* Batch-1 decode attention over the Q8_0 cache (the quantized-KV branch of
 * models/dense_forward.cpp:3956-4065; the GPU counterpart of cuda_attention_out,
 * core/engine.h:806-811): q [n_head][hd] fp32 (after RoPE), keys/values at
 * positions [cc_start, pos], query head h reads KV head h / (n_head /
 * n_head_kv), scores scaled by 1/sqrt(hd), softmax, out [n_head][hd] fp32.
 * hd in {64, 128, 256}, n_head / n_head_kv in {1, 2, 4, 8} and n_head * hd a
 * multiple of 256; other shapes: -2.
 * d_work holds dq_attn_workspace_bytes(n_ctx) bytes of per-tile partials
 * (calls sharing a workspace must not overlap). d_pos as for dq_kv_write. */
int dq_attn_workspace_bytes(uint32_t n_head, uint32_t n_head_kv, uint32_t hd, uint32_t n_ctx, size_t* bytes);
int dq_attn_decode_q8(const float* d_q, const void* d_kc, const void* d_vc, uint32_t n_head, uint32_t n_head_kv,
                      uint32_t hd, uint32_t cc_start, uint32_t pos, const int32_t* d_pos, uint32_t n_ctx,
                      float* d_out, void* d_work, size_t work_bytes, void* stream);

/* Allocation-free form of dq_attn_decode_q8 (no counterpart in the reference:
 * for callers that cannot allocate device memory, e.g. code under HIP graph
 * capture or a serving loop that forbids hipMalloc). Same arguments and
 * results without d_work: the tile records live in a static 16 MiB device
 * array of the library, one per GPU, held until the process ends. Shapes whose
 * dq_attn_workspace_bytes exceeds 16 MiB (n_head * ceil(n_ctx / 64) * 528
 * bytes at hd = 128: 32 heads up to n_ctx = 63488) return
 * DQ_ERR_NOT_SUPPORTED and do nothing. Every call on a GPU shares that GPU's
 * array: calls that overlap on one GPU (other streams, other threads) race. It
 * calls no hipMalloc/hipFree; its first call on a device looks the array's
 * address up (hipGetSymbolAddress) and must not itself be under capture. */
int dq_attn_decode_q8_noalloc(const float* d_q, const void* d_kc, const void* d_vc, uint32_t n_head,
                              uint32_t n_head_kv, uint32_t hd, uint32_t cc_start, uint32_t pos, const int32_t* d_pos,
                              uint32_t n_ctx, float* d_out, void* stream);
/* The same, also writing the output quantized per 256 values (DQ_ACT_Q8K_REP
 * layout: int8 [n_head*hd], scale and int32 sum per 32), the activation of
 * the output projection's GEMV. */
int dq_attn_decode_q8_act(const float* d_q, const void* d_kc, const void* d_vc, uint32_t n_head,
                          uint32_t n_head_kv, uint32_t hd, uint32_t cc_start, uint32_t pos, const int32_t* d_pos,
                          uint32_t n_ctx, float* d_out, int8_t* d_oq, float* d_oscale, int32_t* d_oisum,
                          void* d_work, size_t work_bytes, void* stream);
/* The decode step of the layer in two launches (tiles, merge): NeoX
 * RoPE (table d_rope, NULL = none; n_rot must equal hd, else -2) of the raw
 * query q and key k, the Q8_0 rows of k and v written at `pos` (bit-exact
 * kv_quantize_row of the rotated k and of v, as dq_rope_kv_write), then the
 * attention as dq_attn_decode_q8; the output also quantized per 256 when
 * d_oq != NULL. q, k, v: the Q/K/V projections of the new token. */
int dq_attn_rope_kv_decode(const float* d_q, const float* d_k, const float* d_v, const float* d_rope,
                           uint32_t n_rot, void* d_kc, void* d_vc, uint32_t n_head, uint32_t n_head_kv, uint32_t hd,
                           uint32_t cc_start, uint32_t pos, const int32_t* d_pos, uint32_t n_ctx, float* d_out,
                           int8_t* d_oq, float* d_oscale, int32_t* d_oisum, void* d_work, size_t work_bytes,
                           void* stream);

/* ------------------------------------------------------------- prefill */

/* K/V rows of n_tok consecutive tokens into positions [pos0, pos0 + n_tok)
 * (kv_quantize_batch_kernel, cuda/backend_cuda.cu:7028-7058; per position
 * write_kv_cache, models/dense_forward.cpp:2552-2605, with kv_quantize_row,
 * kv/kv_quant.cpp:31-56, bit-exact). d_k, d_v: [n_tok][ld] floats, the first
 * n_head_kv * hd of a row are stored. hd % 32 == 0. */
int dq_kv_write_batch(const float* d_k, const float* d_v, size_t ld, uint32_t n_tok, uint32_t n_head_kv, uint32_t hd,
                      void* d_kc, void* d_vc, uint32_t pos0, uint32_t n_ctx, void* stream);
/* The RoPE step of the prefill for n_tok tokens (models/dense_forward.cpp
 * :3347-3362 per token): NeoX RoPE of every query head in place and of every
 * key head with the table row d_rope + t * n_rot (dq_rope_cache(pos0 + t);
 * NULL = no RoPE), then the Q8_0 rows of the rotated k and of v at pos0 + t
 * (as dq_kv_write_batch). q: [n_tok][q_ld], k, v: [n_tok][kv_ld]. hd in {64,
 * 128, 256}. */
int dq_rope_kv_write_batch(float* d_q, const float* d_k, const float* d_v, size_t q_ld, size_t kv_ld,
                           const float* d_rope, uint32_t n_rot, uint32_t n_tok, uint32_t n_head, uint32_t n_head_kv,
                           uint32_t hd, void* d_kc, void* d_vc, uint32_t pos0, uint32_t n_ctx, void* stream);
/* Prefill attention over the Q8_0 cache: the device counterpart of
 * attention_prefill_cpu_q8 (core/attn_cpu.cpp:128-390, core/engine.h:470-477)
 * and of cuda_attention_batch's kernels (cuda/backend_cuda.cu:3799-3870,
 * 7080-8290). q, out: [n_tok][q_dim] fp32; token t at position pos0 + t
 * attends to keys [lo, pos0 + t] of KV head h / (n_head / n_head_kv), lo = 0
 * or pos0 + t + 1 - n_swa (n_swa > 0: sliding window); scores scaled by
 * 1/sqrt(hd). Columns of q_dim past n_head * hd are left untouched. The K/V
 * rows of every position read must already be in the cache. hd in {64, 128,
 * 256}; other hd: -2. Operands run on fp16 MFMA split into hi + lo parts
 * (~2^-22 relative); cached values and queries must lie inside fp16. When the
 * (row block x KV head) grid is too small for the GPU, each block's keys are
 * split over several workgroups whose partial softmax records a second kernel
 * merges; that needs d_work of dq_attn_prefill_workspace_bytes() bytes (NULL
 * or smaller: fewer or no splits, same result to float rounding). Calls
 * sharing a workspace must not overlap. */
int dq_attn_prefill_workspace_bytes(uint32_t n_tok, uint32_t n_head, uint32_t n_head_kv, uint32_t hd,
                                    size_t* bytes);
int dq_attn_prefill_q8(const float* d_q, const void* d_kc, const void* d_vc, uint32_t n_tok, uint32_t n_head,
                       uint32_t n_head_kv, uint32_t hd, uint32_t q_dim, uint32_t pos0, uint32_t n_swa,
                       uint32_t n_ctx, float* d_out, void* d_work, size_t work_bytes, void* stream);

/* ------------------------------------------------------- decoder layer */

/* rope_cache_init (models/dense_forward.cpp:631-657, no YaRN): host code,
 * cache[2j] = cos(theta_j), cache[2j+1] = sin(theta_j), theta_j = pos *
 * powf(base, -2/n_rot)^j by repeated float products. n_rot floats. */
int dq_rope_cache(float* cache, uint32_t n_rot, uint32_t pos, float theta_base);

/* Fused pieces of the layer (device pointers, stream-ordered):
 * dq_norm_quant: h = a (+ b, written to d_h when both are given); rms_norm_vec
 *   (models/dense_forward.cpp:129-165) with weight w, then the per-256
 *   quantizer of the K-quant GEMVs (DQ_ACT_Q8K_REP). n % 256 == 0.
 * dq_silu_quant: silu(gate) * up (:53-55), then the same quantizer.
 * dq_rope_kv_write: NeoX RoPE (:668-680) of q (in place) and k with the
 *   cos/sin table d_rope (dq_rope_cache; NULL = no RoPE), then the Q8_0 rows
 *   of k and v into the caches at pos (as dq_kv_write). hd in {64, 128, 256}. */
int dq_norm_quant(const float* d_a, const float* d_b, float* d_h, const float* d_w, size_t n, float eps,
                  int8_t* d_q, float* d_scale, int32_t* d_isum, void* stream);
int dq_silu_quant(const float* d_gate, const float* d_up, size_t n, int8_t* d_q, float* d_scale, int32_t* d_isum,
                  void* stream);
/* A grouped per-256 GEMV (as dq_gemv_group, jobs of Q4_K and Q6_K; the
 * norm form may mix the two) whose kernel forms the activation from fp32
 * inputs and quantizes it per 256 itself, so no launch sits between it and
 * the kernel that wrote them: the layer's norm_quant + Q/K/V or gate/up, and
 * silu_quant + down, as one launch each. kind DQ_FUSE_NORM: y = rms_norm_vec
 * (d_a) * d_b (d_b the norm weights, eps); DQ_FUSE_SILU / DQ_FUSE_GEGLU:
 * y = act(d_a) * d_b (gate, up; eps unused). The GEMV outputs equal those of
 * dq_norm_quant / dq_silu_quant followed by dq_gemv_group: bit-identical for
 * the activation forms; the norm's double sum of squares runs in another
 * order (the same float scale except within ~1e-13 relative of a float
 * rounding boundary). cols % 256 == 0 and cols <= 16384; -2
 * (DQ_ERR_NOT_SUPPORTED), with nothing launched, for other shapes and
 * formats and where the kernel's grid does not hold the group (more rows
 * than its workgroups can keep in flight at once; at cols <= 4096 a group of
 * one format has a persistent form without that limit). No counterpart in
 * the reference (its CUDA layer runs these as separate kernels).
 * DQ_FUSE_NORM_SILU / DQ_FUSE_NORM_GEGLU: the norm form for the gated FFN's
 * gate (jobs[0]) and up (jobs[1]) matrices, of one format and the same
 * rows, no residuals, cols <= 4096: row r of both is computed by one wave
 * and jobs[0].d_y[r] = act(gate_r) * up_r is the only output (jobs[1].d_y is
 * not written), the fp32 input of the down projection (dq_gemv_f32 then
 * quantizes it in its own kernel). gate_r and up_r are the unpaired form's
 * values, and act the reference's (models/dense_forward.cpp:53-55, :107-126). */
#define DQ_FUSE_NORM 1
#define DQ_FUSE_SILU 2
#define DQ_FUSE_GEGLU 3
#define DQ_FUSE_NORM_SILU 4
#define DQ_FUSE_NORM_GEGLU 5
int dq_gemv_group_fused(const dq_gemv_job_t* jobs, size_t n, size_t cols, int kind, const float* d_a,
                        const float* d_b, float eps, void* stream);
/* h = silu(gate) * up in fp32 (models/dense_forward.cpp:53-55), the input of a
 * Q8_0 / Q4_0 down projection (which quantizes per 32 itself). */
int dq_silu_mul(const float* d_gate, const float* d_up, size_t n, float* d_h, void* stream);
int dq_rope_kv_write(float* d_q, const float* d_k, const float* d_v, const float* d_rope, uint32_t n_head,
                     uint32_t n_head_kv, uint32_t hd, uint32_t n_rot, void* d_kc, void* d_vc, uint32_t pos,
                     const int32_t* d_pos, uint32_t n_ctx, void* stream);

/* One Llama-style decoder layer at batch 1 on the device: the dense branch
 * of models/dense_forward.cpp:3897-4257 with optional Q/K/V biases and
 * per-head QK-norm (Qwen-style layers), a gated SiLU or GELU FFN, optional
 * sandwich norms and attention gate, and a Q8_0 KV cache, that
 * cuda_layer_forward (core/engine.h:698-752) runs as one
 * captured episode. The biases (bq [n_head*head_dim], bk, bv
 * [n_head_kv*head_dim]) are added to the projections (add_bias,
 * :3904-3908); q_norm / k_norm [head_dim] then normalise every q and k head
 * (rms_norm_vec per head, :3915-3931), before RoPE. Each may be NULL.
 * act_gelu selects the gated GELU FFN of GELU architectures: the decode
 * layer uses geglu_inplace (:107-126, :4212-4213), the prefill layer the
 * per-element gelu_tanh of the batch branch (:49-51, :3608-3609).
 * post_attn_norm / post_ffn_norm (Gemma-style sandwich norms) normalise the
 * output projection and the FFN output before their residuals (rms_norm_vec,
 * :4140-4142, :4245-4247). wag (DenseQuirks::attn_gate) is a per-head output
 * gate: its n_head rows times the same normalised input as Q/K/V give g_h,
 * and head h of the attention output is scaled by 1 / (1 + exp(-g_h)) before
 * the output projection (:4102-4114; batch :3522-3537). Weights are packed
 * device matrices (dq_weights_pack), each of any of the four formats (Q4_K /
 * Q6_K read the per-256 activation, Q8_0 / Q4_0 the per-32 one, as the
 * reference CPU GEMVs of those formats do); n_embd, n_ff and n_head*head_dim
 * multiples of 256, head_dim 64, 128 or 256; other shapes: -2. Q/K/V and gate/up each
 * run as one grouped GEMV. x and x_out are device vectors of n_embd floats (they
 * may not alias); d_rope is the device copy of dq_rope_cache(pos); the KV
 * caches are those of dq_kv_write for this layer. d_pos as for dq_kv_write
 * (graph replay). d_work: dq_layer_workspace_bytes(n_ctx) bytes. */
typedef struct {
    uint32_t n_embd, n_head, n_head_kv, head_dim, n_rot, n_ff;
    float rms_eps;
    int fmt_q, fmt_k, fmt_v, fmt_o, fmt_gate, fmt_up, fmt_down; /* DQ_FMT_* */
    const void *wq, *wk, *wv, *wo, *wgate, *wup, *wdown;      /* packed device matrices */
    const float *attn_norm, *ffn_norm;                        /* device, n_embd floats */
    const float *bq, *bk, *bv, *q_norm, *k_norm;              /* device, optional (NULL) */
    int act_gelu; /* 1: gated GELU FFN (decode: geglu_inplace; prefill: gelu_tanh) */
    const float *post_attn_norm, *post_ffn_norm; /* device [n_embd], optional (NULL): sandwich norms */
    const void* wag; /* optional (NULL) per-head attention output gate [n_head][n_embd], packed, format fmt_ag */
    int fmt_ag;
    /* optional (NULL) tile copies (dq_gemm_tiles_pack) of wq .. wdown and wag: the prefill layer's GEMMs read
     * them instead of the packed rows, with the same results; the decode layer ignores them */
    const void *tq, *tk, *tv, *to, *tgate, *tup, *tdown, *tag;
} dq_layer_t;

int dq_layer_workspace_bytes(const dq_layer_t* layer, uint32_t n_ctx, size_t* bytes);
int dq_layer_decode(const dq_layer_t* layer, const float* d_x, float* d_x_out, const float* d_rope, uint32_t pos,
                    const int32_t* d_pos, uint32_t cc_start, void* d_kc, void* d_vc, uint32_t n_ctx, void* d_work,
                    size_t work_bytes, void* stream);

/* The same layer for a prompt chunk of n_tok consecutive tokens at positions
 * [pos0, pos0 + n_tok): the CPU batch branch of models/dense_forward.cpp
 * (:3260-3290 norm and Q/K/V through matvec_batch, :3300-3362 RoPE and KV
 * rows per token, :3430-3460 attention_prefill_cpu_q8, :3539-3560 output
 * projection, residual and FFN norm, :3600-3624 gated SiLU FFN and residual)
 * that cuda_layer_forward_batch (core/engine.h:754-797, backend_cuda.cu:8466)
 * runs on the GPU. Every product is the prefill GEMM (dq_gemm: the i8 GEMM
 * semantics of matmul_<fmt>_batch), each matrix any of Q4_K, Q6_K, Q8_0 and
 * Q4_0; attention is dq_attn_prefill_q8 (n_swa > 0: sliding
 * window). d_x, d_x_out: [n_tok][n_embd] device rows (may alias); d_rope:
 * [n_tok][n_rot] cos/sin tables (dq_rope_cache(pos0 + t)) or NULL. The K/V
 * rows of the chunk are written into the caches. Shapes as dq_layer_decode
 * plus: n_rot even and <= head_dim; n_tok <= 65535. d_work:
 * dq_layer_prefill_workspace_bytes(n_tok) bytes. */
int dq_layer_prefill_workspace_bytes(const dq_layer_t* layer, uint32_t n_tok, size_t* bytes);
int dq_layer_prefill(const dq_layer_t* layer, const float* d_x, float* d_x_out, const float* d_rope, uint32_t pos0,
                     uint32_t n_tok, uint32_t n_swa, void* d_kc, void* d_vc, uint32_t n_ctx, void* d_work,
                     size_t work_bytes, void* stream);


/* rms_norm_vec (models/dense_forward.cpp:129-165) of each of `rows` rows of
 * n floats: x = a (+ b, stored to d_h when given), y = x / sqrt(mean(x^2) +
 * eps) * w, the squares summed in double. n % 4 == 0. */
int dq_rms_norm_rows(const float* d_a, const float* d_b, float* d_h, const float* d_w, size_t n, size_t rows,
                     float eps, float* d_y, void* stream);

/* ------------------------------------------------------------ output head */

/* Logits of the output head for one token: the final RMSNorm (weight d_norm)
 * of x [cols], then the head product [rows] with the activation quantized
 * per the matrix format as the engine's CPU head does (models/dense_forward.cpp
 * final norm + matvec; backend_cuda.cu:3383-3436 head_forward_launch).
 * d_work: dq_head_workspace_bytes() bytes. */
int dq_head_workspace_bytes(int fmt, size_t rows, size_t cols, size_t* bytes);
int dq_head_logits(int fmt, const void* d_w, size_t rows, size_t cols, const float* d_x, const float* d_norm,
                   float eps, float* d_logits, void* d_work, size_t work_bytes, void* stream);
/* The kk (1..256, <= n) largest of n values, largest first, lower index first
 * on equal values (+0 and -0 equal): ids and/or values (device arrays of kk).
 * cuda_head_forward_topk's selection (backend_cuda.cu:3438-3497, 3642-3689).
 * d_work: dq_topk_workspace_bytes() bytes. */
int dq_topk_workspace_bytes(uint32_t n, uint32_t kk, size_t* bytes);
int dq_topk(const float* d_v, uint32_t n, uint32_t kk, int32_t* d_ids, float* d_vals, void* d_work,
            size_t work_bytes, void* stream);

/* Sampling arguments of the pipelined decode, core/engine.h:570-579. */
typedef struct CudaSampleArgs {
    float temperature; int32_t top_k; float top_p;
    float penalty_repeat; float penalty_freq; float penalty_present; int32_t penalty_last_n;
    uint32_t kk;
    float logit_scale;
    float u;
    int append_input;
    uint32_t slot;
} CudaSampleArgs;

/* Device state of the draw: the last drawn token, the recent history the
 * penalties read (a ring of DQ_SAMPLE_HIST tokens, `len` tokens seen, next
 * write at `wpos`), and the token of each readback slot. */
#define DQ_SAMPLE_HIST 256
typedef struct {
    int32_t tok;
    uint32_t len, wpos;
    int32_t ring[4];
    int32_t hist[DQ_SAMPLE_HIST];
} dq_sample_state_t;
/* Resets the state to the last min(n, 256) tokens of hist (host), the last
 * of them as the current token (cuda_sample_history, backend_cuda.cu:3745-3752).
 * Synchronises. */
int dq_sample_reset(void* d_state, const int32_t* hist, size_t n, void* stream);
/* Sampler::sample_candidates (core/sampler.cpp:298-322, finish_ :202-253) on
 * n <= 256 candidates (values, ids): append the current token to the history
 * if args->append_input, penalties over the last penalty_last_n (<= 256)
 * tokens, order by (value desc, id asc), greedy when temperature <= 0, else
 * top-k (> 0), temperature softmax, top-p, and the draw r = u * cum. The
 * token goes to state->tok and state->ring[slot]. */
int dq_sample_candidates(const float* d_vals, const int32_t* d_ids, uint32_t n, const CudaSampleArgs* args,
                         void* d_state, void* stream);
/* x [cols] = the row *d_tok of a packed Q8_0 matrix (d * q, times mul when
 * mul != 0): the embedding of the pipelined decode's next token
 * (backend_cuda.cu:3555-3566). A token outside [0, rows) reads the nearest
 * row. */
int dq_embed_q8_0(const void* d_w, size_t rows, size_t cols, const int32_t* d_tok, float mul, float* d_x,
                  void* stream);

/* ------------------------------------------------------------------ MoE */

/* Router of one MoE layer for n_tok tokens (moe_route_ex with softmax gating,
 * models/moe_route.cpp:10-81): probabilities by softmax (float max, double
 * sum), the k largest in descending order (ties: lower expert index),
 * renormalised by their float sum when norm_w, then times w_scale (0 and 1
 * mean no scaling). logits [n_tok][n_expert] -> ids, wts [n_tok][k].
 * n_expert <= 64, k <= 8: otherwise -2. */
int dq_moe_route(const float* d_logits, uint32_t n_tok, uint32_t n_expert, uint32_t k, int norm_w, float w_scale,
                 int32_t* d_ids, float* d_wts, void* stream);

/* Expert FFN of one MoE layer (models/dense_forward.cpp:1524-1560 expert_ffn,
 * stacked experts, combined as at :4160-4181): for every token, its k routed
 * experts' SwiGLU FFNs (matmul_q4_k semantics: activations quantized per
 * 256) weighted and summed in slot order. Experts are stacked packed
 * matrices (dq_weights_pack): gate and up [n_expert * n_ff][n_embd], down
 * [n_expert * n_embd][n_ff], all Q4_K (other formats: -2); n_embd and n_ff
 * multiples of 256; n_tok <= 65536. x [n_tok][n_embd], logits
 * [n_tok][n_expert], out [n_tok][n_embd] (device). Each expert's weights are
 * read once per call for all its tokens. Results within 4e-3 of the
 * reference composition (fp16 MFMA operands). d_work:
 * dq_moe_workspace_bytes(n_tok) bytes. */
typedef struct {
    uint32_t n_expert, n_expert_used, n_embd, n_ff;
    int norm_w;
    float w_scale;
    int fmt; /* DQ_FMT_Q4_K (packed rows) or DQ_FMT_Q4_K_TILES (expert tiles) */
    const void *wgate, *wup, *wdown;
} dq_moe_t;
int dq_moe_workspace_bytes(const dq_moe_t* m, uint32_t n_tok, size_t* bytes);
/* The expert-tile layout of a stacked Q4_K expert matrix (n_expert experts
 * of rows x cols, cols % 256 == 0), for dq_moe_t with fmt DQ_FMT_Q4_K_TILES:
 * per expert, tile of 128 rows and super-block, the tile's packed bytes as
 * one contiguous run in the order the expert GEMM stages them, so its weight
 * DMA reads contiguous kilobytes. It is the device layout of the expert
 * tensors (the reference keeps them as stacked GGUF rows, loaded by
 * models/dense_forward.cpp:1628-1720 load_matrix; cuda_upload_weights owns the
 * device form, backend_cuda.cu:2910-2923): d_packed is the dq_weights_pack
 * form of the stacked matrix, d_tiles receives dq_moe_tiles_bytes() bytes
 * (the same bytes when rows % 128 == 0). Results of dq_moe_ffn are
 * bit-identical with either layout. */
int dq_moe_tiles_bytes(uint32_t n_expert, size_t rows, size_t cols, size_t* bytes);
int dq_moe_tiles_pack(const void* d_packed, uint32_t n_expert, size_t rows, size_t cols, void* d_tiles, void* stream);
int dq_moe_ffn(const dq_moe_t* m, const float* d_x, const float* d_logits, uint32_t n_tok, float* d_out, void* d_work,
               size_t work_bytes, void* stream);

/* ================================================================ engine layer
 *
 * The GPU operator entry points of the reference engine (core/engine.h
 * :502-811, implemented there by cuda/backend_cuda.cu), with the same names,
 * argument meaning and return conventions, so models/dense_forward.cpp can
 * call them unchanged:
 *   - int results are desireeia_error codes: DQ_OK; DQ_ERR_NOT_SUPPORTED
 *     (shape, format or feature not covered: nothing was done, y untouched,
 *     the caller recomputes on the CPU); DQ_ERR_IO (device failure);
 *   - bool results: false = not done (upload: the matrix stays host-only);
 *   - x / y / proj / x_out are HOST pointers; each call that returns host
 *     data synchronises its stream once;
 *   - one process-global stream, scratch that grows on demand and one device
 *     KV cache; not thread-safe (as the reference backend).
 * Where the reference passes a C++ reference (a struct or an out-parameter),
 * the C ABI takes a pointer (a one-line C++ overload restores the reference form).
 * Arithmetic follows the reference CPU functions the engine would otherwise
 * run (matmul_q8_0 / q4_0 / q4_k / q6_k, their _batch forms, the dense
 * layer); the format ids are those of the reference (0 = Q8_0, 1 = Q4_0,
 * 5 = Q4_K, 7 = Q6_K). */

/* core/engine.h:536 */
typedef struct CudaKQuantJob {
    int format;
    const void* d_w;
    size_t rows;
    float* y; /* host */
} CudaKQuantJob;

/* core/engine.h:598-603 */
typedef struct CudaQ80Job {
    const void* d_qs;
    const void* d_scale;
    size_t rows;
    float* y; /* host */
} CudaQ80Job;

/* core/engine.h:675-691 (field order kept) */
typedef struct CudaQkvAttnArgs {
    const void* wq_qs; const void* wq_scale;
    const void* wk_qs; const void* wk_scale;
    const void* wv_qs; const void* wv_scale;
    const void* wo_qs; const void* wo_scale;
    const float* bq; const float* bk; const float* bv;
    const float* attn_in;
    const float* rope_cache;
    float* proj;
    uint8_t* host_k_row;
    uint8_t* host_v_row;
    size_t n_embd; size_t q_dim; size_t kv_dim;
    uint32_t n_head; uint32_t n_head_kv; uint32_t heads_per_kv;
    uint32_t head_dim; uint32_t n_rot;
    size_t kv_layer_off;
    uint32_t cc_start; uint32_t pos;
} CudaQkvAttnArgs;

/* core/engine.h:698-751 (field order kept) */
typedef struct CudaLayerArgs {
    const void* wq_qs; const void* wq_scale;
    const void* wk_qs; const void* wk_scale;
    const void* wv_qs; const void* wv_scale;
    const void* wo_qs; const void* wo_scale;
    const void* wgate_qs; const void* wgate_scale;
    const void* wup_qs; const void* wup_scale;
    const void* wdown_qs; const void* wdown_scale;
    const void* wag_qs; const void* wag_scale;
    const float* bq; const float* bk; const float* bv;
    const float* attn_norm_w; const float* ffn_norm_w;
    const float* q_norm_w; const float* k_norm_w;
    const float* post_attn_norm_w; const float* post_ffn_norm_w;
    const float* x;
    const float* rope_cache;
    float* x_out;
    size_t n_embd; size_t q_dim; size_t kv_dim; size_t n_ff;
    uint32_t n_head; uint32_t n_head_kv; uint32_t heads_per_kv;
    uint32_t head_dim; uint32_t n_rot;
    size_t kv_layer_off;
    uint32_t cc_start; uint32_t pos;
    float rms_eps; int act_gelu;
    int fmt_q; int fmt_k; int fmt_v; int fmt_o;
    int fmt_gate; int fmt_up; int fmt_down; int fmt_ag;
    int upload_x; int download_x;
    int upload_dyn;
    const uint32_t* dyn_all; const float* rope_all;
    uint32_t n_slots; uint32_t rope_stride; uint32_t layer_slot;
    int x_from_token;
    const void* embd_qs; const void* embd_scale; float embd_mul;
} CudaLayerArgs;

/* The prefill-layer argument block, core/engine.h:764-796 (same fields,
 * same order). x / x_out / rope_caches are host arrays of the whole prompt
 * ([n_total][n_embd], [n_total][n_rot]); the call covers rows
 * [x_row0, x_row0 + n_tok) at positions [pos0, pos0 + n_tok). */
typedef struct CudaLayerBatchArgs {
    const void* wq_qs; const void* wq_scale;
    const void* wk_qs; const void* wk_scale;
    const void* wv_qs; const void* wv_scale;
    const void* wo_qs; const void* wo_scale;
    const void* wgate_qs; const void* wgate_scale;
    const void* wup_qs; const void* wup_scale;
    const void* wdown_qs; const void* wdown_scale;
    const void* wag_qs; const void* wag_scale;
    const float* bq; const float* bk; const float* bv;
    const float* attn_norm_w; const float* ffn_norm_w;
    const float* q_norm_w; const float* k_norm_w;
    const float* post_attn_norm_w; const float* post_ffn_norm_w;
    const float* x;
    float* x_out;
    uint32_t x_out_row0;
    const float* rope_caches;
    void* host_kcache; void* host_vcache;
    size_t n_embd; size_t q_dim; size_t kv_dim; size_t n_ff;
    uint32_t n_head; uint32_t n_head_kv; uint32_t heads_per_kv;
    uint32_t head_dim; uint32_t n_rot;
    size_t kv_layer_off;
    uint32_t pos0; uint32_t n_tok; uint32_t n_swa;
    uint32_t x_row0; uint32_t n_total;
    float rms_eps; int act_gelu;
    int fmt_q; int fmt_k; int fmt_v; int fmt_o;
    int fmt_gate; int fmt_up; int fmt_down; int fmt_ag;
    int upload_x; int download_x; int upload_rope; int prepare_weights;
    int rope_slot;
} CudaLayerBatchArgs;

/* Devices: core/engine.h:627-629. */
int32_t cuda_gpu_count(void);
bool cuda_probe_gpu(int32_t index, char* name, size_t name_len, uint64_t* total, uint64_t* free_bytes,
                    int32_t* cc_major, int32_t* cc_minor, int32_t* sms);

/* Weight upload and lifetime: core/engine.h:516, :532, :556, :557. Q8_0
 * returns the packed matrix in *out_d_qs and a pointer inside it in
 * *out_d_scale (both may be passed to cuda_free_device; only the first frees);
 * K-quants and Q4_0 leave *out_d_scale NULL. Other formats: false. */
bool matmul_q8_0_cuda_upload_weights(const uint8_t* q8_data, size_t rows, size_t cols, void** out_d_qs,
                                     void** out_d_scale);
bool cuda_upload_weights(int format, const uint8_t* data, size_t rows, size_t cols, void** out_d_qs,
                         void** out_d_scale);
void cuda_free_device(void* p);
void cuda_backend_shutdown(void);

/* Decode GEMVs on resident weights: core/engine.h:534, :537-538, :587,
 * :598-605, and the per-call-upload fallback :507. */
int matmul_kquant_cuda_resident(int format, const void* d_w, size_t rows, size_t cols, const float* x, float* y);
int matmul_kquant_cuda_resident_same_x(const CudaKQuantJob* jobs, size_t n, size_t cols, const float* x);
int matmul_q8_0_cuda_resident(const void* d_qs, const void* d_scale, size_t rows, size_t cols, const float* x,
                              float* y);
int matmul_q8_0_cuda_resident_group(const CudaQ80Job* jobs, size_t n, size_t cols, const float* x);
int matmul_q8_0_cuda(const uint8_t* q8_data, size_t rows, size_t cols, const float* x, float* y);

/* Batched (prefill) product y[n_tok][rows] = x[n_tok][cols] W^T, core/engine.h
 * :543: Q4_K / Q6_K / Q8_0 / Q4_0 with the semantics of matmul_<fmt>_batch
 * (i8_gemm from 4 tokens, Q8_0 from 2; per-token GEMVs below). cols % 256 != 0
 * or other formats: NOT_SUPPORTED. */
int matmul_kquant_cuda_batch(int format, const void* d_w, size_t rows, size_t cols, const float* x, size_t n_tok,
                             float* y);

/* Gated FFN on Q8_0 weights (core/engine.h:612-617): up, gate, silu(gate)*up,
 * down, one sync. act_gelu = 1 (GELU): NOT_SUPPORTED. */
int matmul_q8_0_cuda_ffn_gated(const void* d_up_qs, const void* d_up_scale, const void* d_gate_qs,
                               const void* d_gate_scale, const void* d_down_qs, const void* d_down_scale, size_t n_ff,
                               size_t n_embd, const float* x, float* out, int act_gelu);

/* Device KV cache, [layer][pos][kv_head][row] bytes as the host cache
 * (core/engine.h:619-666). */
bool cuda_kv_cache_reserve(size_t total_bytes);
void cuda_kv_cache_release(void);
bool cuda_kv_cache_upload(const void* k_host, const void* v_host, size_t total_bytes);
bool cuda_kv_cache_download(void* k_host, void* v_host, size_t total_bytes);
bool cuda_kv_cache_write(size_t byte_off, const void* k, const void* v, size_t bytes);
bool cuda_kv_cache_read(size_t byte_off, void* k, void* v, size_t bytes);
bool cuda_kv_cache_move(size_t dst_off, size_t src_off, size_t bytes);
void cuda_set_attention_long(bool long_context);
void cuda_drop_graphs(void);

/* Attention episodes over the device Q8_0 KV cache (core/engine.h:806-811,
 * :692, :752). cuda_attention_out: attention of q (host, q_dim floats) at
 * [cc_start, pos] of the layer at layer_off, then proj = Wo * out (host).
 * cuda_qkv_attention_out: Q/K/V (+ optional biases), RoPE, the new KV rows
 * (device cache and host_k_row / host_v_row), attention and Wo.
 * cuda_layer_forward: the whole dense layer; x stays on the device between
 * layers (upload_x on the first, download_x on the last). Q/K/V biases,
 * per-head QK-norm, sandwich norms, gated GELU, the attention output gate,
 * per-layer slots (dyn_all / rope_all) and the embedding from the drawn token
 * are taken; head_dim other than 64, 128 or 256: NOT_SUPPORTED. */
int cuda_attention_out(const void* d_wo_qs, const void* d_wo_scale, const float* q, uint32_t n_head,
                       uint32_t heads_per_kv, uint32_t head_dim, uint32_t kv_dim, size_t layer_off, uint32_t cc_start,
                       uint32_t pos, size_t n_embd, size_t q_dim, float* proj, int kv_quantized, size_t row_bytes);
int cuda_qkv_attention_out(const CudaQkvAttnArgs* args);
int cuda_layer_forward(const CudaLayerArgs* args);

/* Prefill (core/engine.h:550-555, :797-798; backend_cuda.cu:3799-3870,
 * :8457-8860).
 * cuda_attention_batch: attention of n_tokens queries (host q_all, [n][q_dim])
 *   at positions col0.. over the device KV cache of the layer at layer_off
 *   (dq_attn_prefill_q8); out_all (host) receives [n][q_dim] (columns past
 *   n_head * head_dim keep their values). head_dim 64/128/256 with the
 *   cache's row_bytes / pos_bytes; otherwise NOT_SUPPORTED.
 * cuda_layer_forward_batch: the dense layer over a prompt chunk
 *   (dq_layer_prefill). The prompt's activations stay on the device
 *   between layers and chunks: upload_x on the first call, download_x on the
 *   last (rows from x_out_row0 on), which also copies every K/V row the
 *   prompt wrote into host_kcache / host_vcache and synchronises once. RoPE
 *   tables: rope_caches uploaded when upload_rope into slot rope_slot (0-3);
 *   NULL = no RoPE. Matrices: uploads of this library; biases, per-head
 *   QK-norm, sandwich norms, the attention gate and gated GELU are taken;
 *   head_dim other than 64, 128 or 256: NOT_SUPPORTED, before any device
 *   work.
 * cuda_prefill_chunk_tokens: tokens per chunk, 8 per CU within [1024, 4096]. */
int cuda_attention_batch(const float* q_all, float* out_all, uint32_t n_tokens, uint32_t n_head,
                         uint32_t heads_per_kv, uint32_t head_dim, uint32_t q_dim, size_t row_bytes, size_t pos_bytes,
                         size_t layer_off, uint32_t col0, uint32_t n_swa);
int cuda_layer_forward_batch(const struct CudaLayerBatchArgs* args);
int cuda_prefill_chunk_tokens(void);

/* Output head and the pipelined draw (core/engine.h:558-591,
 * backend_cuda.cu:3383-3780): on the x the last cuda_layer_forward left on
 * the device. cuda_head_forward: logits to host y [rows]. cuda_head_forward_topk:
 * the kk (<= 256) largest, largest first, lower id on ties. cuda_head_forward_sample:
 * head + top-kk + the draw (dq_sample_candidates), queued without a
 * synchronisation; cuda_sample_wait returns the token of a slot.
 * cuda_sample_history replaces the device history with the last tokens of
 * hist. cuda_fetch_x copies the device x to the host. The head matrix must be
 * an upload of this library with format / rows / n_embd as given: otherwise
 * NOT_SUPPORTED. With x_from_token (CudaLayerArgs), cuda_layer_forward builds
 * x from the drawn token and a Q8_0 embedding upload (embd_qs, embd_mul). */
int cuda_head_forward(int format, const void* d_qs, const void* d_scale, const float* norm_w, size_t n_embd,
                      float eps, size_t rows, float* y);
int cuda_head_forward_topk(int format, const void* d_qs, const void* d_scale, const float* norm_w, size_t n_embd,
                           float eps, size_t rows, uint32_t kk, int32_t* ids, float* vals);
int cuda_head_forward_sample(int format, const void* d_qs, const void* d_scale, const float* norm_w, size_t n_embd,
                             float eps, size_t rows, const CudaSampleArgs* args);
int cuda_sample_wait(uint32_t slot, int32_t* token);
int cuda_sample_history(const int32_t* hist, size_t n);
int cuda_fetch_x(float* dst, size_t n);

/* ------------------------------------------------------------------------
 * GGUF model files (host): the engine's GgufReader (src/gguf/gguf_reader.cpp
 * :100-305, ModelReader::open / read_tensor_raw) over a read-only memory map,
 * and the upload its caller load_matrix (models/dense_forward.cpp:1628-1720)
 * does through cuda_upload_weights. Header, metadata and tensor directory are
 * parsed and bounds-checked at open; for version >= 2 tensor offsets are
 * relative to the data section (end of the tensor infos rounded up to
 * general.alignment, default 32), for version < 2 they are absolute, as the
 * engine reads them. Errors: DQ_ERR_IO (cannot open or map the file),
 * DQ_ERR_INVALID_ARG (not GGUF, truncated or malformed; a null argument),
 * DQ_ERR_NOT_SUPPORTED (no such key / tensor, or a type without a known row
 * size). Pointers returned (names, strings, array and tensor data) point into
 * the map and stay valid until dq_gguf_close. Not thread-safe per handle.
 * ---------------------------------------------------------------------- */
typedef struct dq_gguf dq_gguf;

typedef struct {
    const char* name;
    int type;           /* GGUF tensor type id (quant/quant.h:439-476) */
    int n_dims;
    uint64_t dims[4];   /* ne0 (columns) first; unused dims are 1 */
    uint64_t offset;    /* absolute file offset of the tensor's bytes */
    uint64_t nbytes;    /* row_size(type, ne0) * rows; 0 for an unknown type */
    const void* data;   /* the bytes in the map (NULL when nbytes is 0) */
} dq_gguf_tensor_t;

/* desireeia_row_size (quant/quant.cpp:905-910): bytes of ne0 values of a
 * tensor type; 0 for an unknown type. */
size_t dq_row_size(int type, int64_t ne0);
/* GGUF type -> backend format id (DQ_FMT_*), -1 where the device path has no kernels. */
int dq_fmt_of_gguf_type(int type);

int dq_gguf_open(const char* path, dq_gguf** out);
void dq_gguf_close(dq_gguf* g);
int dq_gguf_version(const dq_gguf* g);
uint64_t dq_gguf_data_offset(const dq_gguf* g);
int64_t dq_gguf_kv_count(const dq_gguf* g);
const char* dq_gguf_kv_key(const dq_gguf* g, int64_t i);
/* value type of a key (0-12 as in the file), -1 if absent */
int dq_gguf_kv_type(const dq_gguf* g, const char* key);
/* integer kinds (U8..I32, BOOL, U64, I64) */
int dq_gguf_get_int(const dq_gguf* g, const char* key, int64_t* v);
/* any numeric kind */
int dq_gguf_get_float(const dq_gguf* g, const char* key, double* v);
int dq_gguf_get_str(const dq_gguf* g, const char* key, const char** s, uint64_t* len);
/* arrays: element type, count and the raw elements (scalar elements packed;
 * string elements as u64 length + bytes each) */
int dq_gguf_get_array(const dq_gguf* g, const char* key, int* elem_type, uint64_t* n, const void** data);
int64_t dq_gguf_n_tensors(const dq_gguf* g);
/* index of a tensor by name, -1 if absent */
int64_t dq_gguf_find_tensor(const dq_gguf* g, const char* name);
int dq_gguf_tensor_info(const dq_gguf* g, int64_t i, dq_gguf_tensor_t* out);
/* ModelReader::read_tensor_raw (gguf_reader.cpp:288-305): copies the tensor's
 * bytes to dst (cap bytes available; dst NULL: sizes only) and reports its
 * type, ne0 and rows = prod(dims[1..]). */
int dq_gguf_read_tensor_raw(const dq_gguf* g, const char* name, void* dst, size_t cap, int* type, uint64_t* ne0,
                            uint64_t* rows);
/* Uploads a Q8_0 / Q4_0 / Q4_K / Q6_K matrix into the device layout with
 * cuda_upload_weights (release with cuda_free_device), straight from the map:
 * fmt, rows, cols and the engine's (d_qs, d_scale) pair. */
int dq_gguf_upload(const dq_gguf* g, const char* name, int* fmt, uint64_t* rows, uint64_t* cols, void** d_qs,
                   void** d_scale);

#ifdef __cplusplus
}
#endif
#endif
