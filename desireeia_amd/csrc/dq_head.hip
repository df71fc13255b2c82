// dq_head.hip - the step after the last layer: the output head's logits, the
// largest of them on the device, and the sampling draw, so that a decoded
// token can be chosen without the logits leaving the GPU (reference
// cuda/backend_cuda.cu:3383-3780, cuda_head_forward*, and the host sampler
// core/sampler.cpp:202-322 whose draw the device replicates).
//
// Logits: the final RMSNorm (dq_rms_norm_rows) then the head GEMV with the
// fp32 activation quantized in-kernel per the matrix format, as the engine's
// CPU head (matvec -> matmul_<fmt>) quantizes it. HBM-bound: a 128k x 4096
// Q6_K head is 431 MB per token.
//
// Top-k: every (value, id) pair becomes one 64-bit key that sorts ascending
// in the sampler's order - larger value first, lower id on ties - so the
// selection is a plain sort of integers: the high word is the float's bits
// made order-preserving and inverted (+0 and -0 made equal), the low word the
// id. Each pass selects the kk smallest keys of every chunk of 4096 by a
// radix select over LDS histograms; passes repeat on the survivors until one
// chunk remains, whose kk keys are sorted. kk = 1 is a min-reduction instead.
//
// Sampling (sample_kernel): penalties on the candidates that carry them
// (counts over the last penalty_last_n tokens of a 256-token device ring),
// the same order, then temperature, top-k, top-p and the draw on one lane in
// the host's order of operations, with the uniform number u drawn by the
// host sampler's generator: r = u * cum.
#include <cstdlib>
#include <cstring>
#include <vector>

#include "dq_common.h"

namespace {

constexpr int TK_CHUNK = 4096;  // keys per workgroup and pass
constexpr int TK_T = 256;       // threads per workgroup

__device__ __forceinline__ uint64_t order_key(float v, uint32_t id) {
    uint32_t u = __builtin_bit_cast(uint32_t, v == 0.0f ? 0.0f : v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);  // ascending with v
    return ((uint64_t)(~u) << 32) | id;              // descending value, ascending id
}

__device__ __forceinline__ float key_value(uint64_t k) {
    uint32_t u = ~(uint32_t)(k >> 32);
    u = (u & 0x80000000u) ? (u & 0x7FFFFFFFu) : ~u;
    return __builtin_bit_cast(float, u);
}

constexpr int TK_PER = TK_CHUNK / TK_T;  // keys per thread

// Sorts the first P (a power of two <= TK_CHUNK) keys of LDS ascending.
__device__ void bitonic_sort(uint64_t* s, int P) {
    for (int size = 2; size <= P; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int t = threadIdx.x; t < P / 2; t += TK_T) {
                const int i = 2 * t - (t & (stride - 1)), j = i + stride;
                const bool asc = (i & size) == 0;
                const uint64_t a = s[i], b = s[j];
                if ((a > b) == asc) {
                    s[i] = b;
                    s[j] = a;
                }
            }
            __syncthreads();
        }
    }
}

// One selection pass over chunk blockIdx.x (float logits with their index as
// id on the first pass, keys afterwards): the kk smallest keys of the chunk.
// Radix select: eight rounds of an 8-bit LDS histogram over the keys that
// share the prefix fixed so far find the kk-th smallest key K exactly (keys
// are distinct: the id is in them); the keys <= K are then gathered, and on
// the final pass (one chunk) sorted.
__global__ __launch_bounds__(TK_T) void topk_pass_kernel(const float* __restrict__ v, const uint64_t* __restrict__ kin,
                                                         uint32_t n, uint32_t kk, int sorted,
                                                         uint64_t* __restrict__ kout, int32_t* __restrict__ ids,
                                                         float* __restrict__ vals) {
    __shared__ uint32_t hist[256];
    __shared__ uint64_t list[256];
    __shared__ uint64_t s_prefix, s_key;
    __shared__ uint32_t s_rank, s_cnt, s_bin;
    const int t = threadIdx.x;
    const size_t base = (size_t)blockIdx.x * TK_CHUNK;
    uint64_t key[TK_PER];
#pragma unroll
    for (int j = 0; j < TK_PER; ++j) {
        const size_t g = base + (size_t)j * TK_T + t;  // coalesced
        uint64_t k = ~0ull;
        if (g < n) k = kin ? kin[g] : order_key(v[g], (uint32_t)g);
        key[j] = k;
    }
    const size_t m = n - base < (size_t)TK_CHUNK ? n - base : (size_t)TK_CHUNK;  // keys in this chunk
    const uint32_t want = (uint32_t)(kk < m ? kk : m);
    uint64_t prefix = 0;
    uint32_t rank = want;  // 1-based rank of K among the keys with this prefix
    for (int r = 0; r < 8; ++r) {
        const int shift = 56 - 8 * r;
        hist[t] = 0;
        __syncthreads();
#pragma unroll
        for (int j = 0; j < TK_PER; ++j) {
            const bool match = r == 0 || (key[j] >> (shift + 8)) == prefix;
            if (match) atomicAdd(&hist[(key[j] >> shift) & 255], 1u);
        }
        __syncthreads();
        if (t < 64) {  // one wave scans the 256 bins, 4 per lane
            const uint32_t h0 = hist[4 * t], h1 = hist[4 * t + 1], h2 = hist[4 * t + 2], h3 = hist[4 * t + 3];
            const uint32_t tot = h0 + h1 + h2 + h3;
            uint32_t incl = tot;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const uint32_t o = __shfl_up(incl, off, DQ_WAVE);
                if (t >= off) incl += o;
            }
            const uint32_t excl = incl - tot;
            if (excl < rank && rank <= incl) {  // exactly one lane
                uint32_t c = excl, d = 4 * t;
                const uint32_t hv[4] = {h0, h1, h2, h3};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    if (c + hv[q] >= rank) {
                        d = 4 * t + q;
                        break;
                    }
                    c += hv[q];
                }
                s_prefix = (prefix << 8) | d;
                s_rank = rank - c;
                s_bin = hist[d];
            }
        }
        __syncthreads();
        prefix = s_prefix;
        rank = s_rank;
        if (s_bin == 1) {  // one key has this prefix: it is K (uniform branch)
#pragma unroll
            for (int j = 0; j < TK_PER; ++j)
                if ((key[j] >> shift) == prefix) s_key = key[j];
            __syncthreads();
            prefix = s_key;
            break;
        }
    }
    // prefix is now K, the want-th smallest key. Real keys are distinct, so
    // exactly `want` keys are <= K - unless K is the padding key ~0 (a later
    // pass over a chunk holding fewer than kk real keys): then only the keys
    // below it are taken and the rest of the output is padding again.
    if (t == 0) s_cnt = 0;
    __syncthreads();
    const bool real = prefix != ~0ull;
#pragma unroll
    for (int j = 0; j < TK_PER; ++j) {
        if (key[j] < prefix || (real && key[j] == prefix)) {
            const uint32_t pos = atomicAdd(&s_cnt, 1u);
            if (pos < 256) list[pos] = key[j];
        }
    }
    __syncthreads();
    const uint32_t got = s_cnt < want ? s_cnt : want;
    int P = 1;
    while (P < (int)kk) P <<= 1;
    for (int j = got + t; j < P; j += TK_T) list[j] = ~0ull;
    __syncthreads();
    if (sorted) {  // the final pass: ids and values, best first
        bitonic_sort(list, P);
        for (uint32_t j = t; j < kk; j += TK_T) {
            if (ids) ids[j] = (int32_t)(uint32_t)list[j];
            if (vals) vals[j] = key_value(list[j]);
        }
        return;
    }
    for (uint32_t j = t; j < kk; j += TK_T) kout[(size_t)blockIdx.x * kk + j] = list[j];
}

// kk = 1: the smallest key of each chunk.
__global__ __launch_bounds__(TK_T) void argmin_pass_kernel(const float* __restrict__ v, const uint64_t* __restrict__ kin,
                                                           uint32_t n, int final, uint64_t* __restrict__ kout,
                                                           int32_t* __restrict__ ids, float* __restrict__ vals) {
    __shared__ uint64_t part[TK_T / 64];
    const size_t base = (size_t)blockIdx.x * TK_CHUNK;
    uint64_t best = ~0ull;
    for (int j = threadIdx.x; j < TK_CHUNK; j += TK_T) {
        const size_t g = base + j;
        if (g < n) {
            const uint64_t k = kin ? kin[g] : order_key(v[g], (uint32_t)g);
            best = k < best ? k : best;
        }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const uint64_t o = __shfl_xor(best, off, DQ_WAVE);
        best = o < best ? o : best;
    }
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < TK_T / 64; ++w) best = part[w] < best ? part[w] : best;
        if (final) {
            if (ids) ids[0] = (int32_t)(uint32_t)best;
            if (vals) vals[0] = key_value(best);
        } else {
            kout[blockIdx.x] = best;
        }
    }
}

// Sampler::sample_candidates (core/sampler.cpp:298-322) with finish_
// (:202-253) and the history ring of the pipelined decode.
__global__ __launch_bounds__(256) void sample_kernel(const float* __restrict__ vin, const int32_t* __restrict__ iin,
                                                     uint32_t n, CudaSampleArgs a, dq_sample_state_t* st) {
    __shared__ uint64_t s[256];
    __shared__ float probs[256];
    __shared__ int32_t hist[DQ_SAMPLE_HIST];
    const int t = threadIdx.x;
    // the history ring into LDS (one entry per thread), then the step's input
    // token appended to both copies
    const uint32_t len0 = st->len, wpos0 = st->wpos;
    hist[t] = st->hist[t];
    __syncthreads();
    uint32_t len = len0, wpos = wpos0;
    if (a.append_input) {
        if (t == 0) {
            const int32_t tok = st->tok;
            hist[wpos0] = tok;
            st->hist[wpos0] = tok;
            st->wpos = (wpos0 + 1) % DQ_SAMPLE_HIST;
            st->len = len0 + 1;
        }
        wpos = (wpos0 + 1) % DQ_SAMPLE_HIST;
        len = len0 + 1;
        __syncthreads();
    }
    const bool pen = a.penalty_last_n > 0 &&
                     (a.penalty_repeat != 1.0f || a.penalty_freq != 0.0f || a.penalty_present != 0.0f);
    const uint32_t look = min((uint32_t)a.penalty_last_n, min(len, (uint32_t)DQ_SAMPLE_HIST));
    uint64_t key = ~0ull;
    if (t < (int)n) {
        float lg = vin[t];
        const int32_t id = iin[t];
        if (a.logit_scale != 0.0f) lg *= a.logit_scale;
        if (pen) {
            int32_t cnt = 0;
            for (uint32_t j = 0; j < look; ++j)
                cnt += hist[(wpos + DQ_SAMPLE_HIST - 1 - j) % DQ_SAMPLE_HIST] == id;
            if (cnt > 0) {
                if (lg <= 0.0f) lg *= a.penalty_repeat;
                else lg /= a.penalty_repeat;
                lg -= (float)cnt * a.penalty_freq + a.penalty_present;
            }
        }
        key = order_key(lg, (uint32_t)id);
    }
    s[t] = key;
    __syncthreads();
    // sort the 256 keys: each holds its candidate's id and exact penalised value
    for (int size = 2; size <= 256; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            if (t < 128) {
                const int i = 2 * t - (t & (stride - 1)), j = i + stride;
                const bool asc = (i & size) == 0;
                const uint64_t x = s[i], y = s[j];
                if ((x > y) == asc) {
                    s[i] = y;
                    s[j] = x;
                }
            }
            __syncthreads();
        }
    }
    if (t != 0) return;
    // values in sorted order (keys decode to the exact float, -0 read as +0)
    int32_t pick = (int32_t)(uint32_t)s[0];
    if (a.temperature > 0.0f) {
        const uint32_t k = min((uint32_t)a.top_k, n);
        const float inv_t = 1.0f / a.temperature;
        const float max_l = key_value(s[0]) * inv_t;
        float sum = 0.0f;
        for (uint32_t i = 0; i < k; ++i) {
            const float p = expf(key_value(s[i]) * inv_t - max_l);
            probs[i] = p;
            sum += p;
        }
        if (sum > 0.0f) {
            for (uint32_t i = 0; i < k; ++i) probs[i] /= sum;
            uint32_t keep = k;
            if (a.top_p < 1.0f) {
                float cum = 0.0f;
                for (uint32_t i = 0; i < k; ++i) {
                    cum += probs[i];
                    if (cum >= a.top_p) {
                        keep = i + 1;
                        break;
                    }
                }
                if (keep < 1) keep = 1;
            }
            float cum = 0.0f;
            for (uint32_t i = 0; i < keep; ++i) cum += probs[i];
            if (cum > 0.0f) {
                const float r = a.u * cum + 0.0f;
                float acc = 0.0f;
                pick = (int32_t)(uint32_t)s[keep - 1];
                for (uint32_t i = 0; i < keep; ++i) {
                    acc += probs[i];
                    if (r <= acc) {
                        pick = (int32_t)(uint32_t)s[i];
                        break;
                    }
                }
            }
        }
    }
    st->tok = pick;
    st->ring[a.slot & 3] = pick;  // the readback slot of this draw
}

// x = row *tok of a packed Q8_0 matrix, d * q in float, times mul when
// non-zero (the embedding of the pipelined decode's next token,
// backend_cuda.cu:3555-3566). Packed layout: block b of row t holds its 32
// values in bytes [t q_row + 16 (b/2), +16) of sub-planes 2 (b%2) and
// 2 (b%2) + 1.
__global__ __launch_bounds__(256) void embed_q8_0_kernel(const uint8_t* __restrict__ qp, size_t ps, size_t q_row,
                                                         const uint16_t* __restrict__ dp, const int32_t* __restrict__ tok,
                                                         uint32_t rows, uint32_t cols, float mul, float* __restrict__ x) {
    int32_t t = *tok;
    t = t < 0 ? 0 : (t >= (int32_t)rows ? (int32_t)rows - 1 : t);  // a token outside the vocabulary reads row 0/last
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < cols; i += blockDim.x * gridDim.x) {
        const size_t B = (size_t)t * (cols / 32) + i / 32;
        const uint32_t w = i % 32;
        const size_t plane = 2 * (B % 2) + (w >= 16 ? 1 : 0);
        const int8_t q = (int8_t)qp[plane * ps + (size_t)t * q_row + 16 * (i / 64) + (w & 15)];
        float val = dq_h2f(dp[B]) * (float)q;
        if (mul != 0.0f) val *= mul;
        x[i] = val;
    }
}

size_t tk_pass_count(uint32_t n, uint32_t kk, size_t* cap) {
    size_t passes = 0, m = n, big = 0;
    for (;;) {
        const size_t blocks = (m + TK_CHUNK - 1) / TK_CHUNK;
        const size_t out = blocks * kk;
        big = out > big ? out : big;
        ++passes;
        if (blocks == 1) break;
        m = out;
    }
    *cap = big;
    return passes;
}

}  // namespace

extern "C" {

int dq_head_workspace_bytes(int fmt, size_t rows, size_t cols, size_t* bytes) {
    if (!bytes) return DQ_ERR_INVALID_ARG;
    DqLayout L;
    if (!dq_layout(fmt, rows, cols, &L)) return DQ_ERR_NOT_SUPPORTED;
    *bytes = dq_align256(cols * 4);
    return DQ_OK;
}

int dq_head_logits(int fmt, const void* d_w, size_t rows, size_t cols, const float* d_x, const float* d_norm,
                   float eps, float* d_logits, void* d_work, size_t work_bytes, void* stream) {
    size_t need = 0;
    const int rc = dq_head_workspace_bytes(fmt, rows, cols, &need);
    if (rc != DQ_OK) return rc;
    if (!d_w || !d_x || !d_norm || !d_logits || !d_work || work_bytes < need) return DQ_ERR_INVALID_ARG;
    float* xn = (float*)d_work;
    const int r1 = dq_rms_norm_rows(d_x, nullptr, nullptr, d_norm, cols, 1, eps, xn, stream);
    if (r1 != DQ_OK) return r1;
    return dq_gemv_f32(fmt, d_w, rows, cols, xn, d_logits, stream);
}

int dq_topk_workspace_bytes(uint32_t n, uint32_t kk, size_t* bytes) {
    if (!bytes) return DQ_ERR_INVALID_ARG;
    if (kk == 0 || kk > 256 || n < kk) return DQ_ERR_NOT_SUPPORTED;
    size_t cap = 0;
    tk_pass_count(n, kk, &cap);
    *bytes = 2 * dq_align256(cap * 8);
    return DQ_OK;
}

int dq_topk(const float* d_v, uint32_t n, uint32_t kk, int32_t* d_ids, float* d_vals, void* d_work,
            size_t work_bytes, void* stream) {
    size_t need = 0;
    const int rc = dq_topk_workspace_bytes(n, kk, &need);
    if (rc != DQ_OK) return rc;
    if (!d_v || !d_work || work_bytes < need || (!d_ids && !d_vals)) return DQ_ERR_INVALID_ARG;
    size_t cap = 0;
    tk_pass_count(n, kk, &cap);
    uint64_t* buf[2] = {(uint64_t*)d_work, (uint64_t*)((uint8_t*)d_work + dq_align256(cap * 8))};
    const hipStream_t s = (hipStream_t)stream;
    const uint64_t* kin = nullptr;
    size_t m = n;
    int cur = 0;
    for (;;) {
        const unsigned blocks = (unsigned)((m + TK_CHUNK - 1) / TK_CHUNK);
        const int final = blocks == 1;
        if (kk == 1) argmin_pass_kernel<<<blocks, TK_T, 0, s>>>(d_v, kin, (uint32_t)m, final, buf[cur], d_ids, d_vals);
        else topk_pass_kernel<<<blocks, TK_T, 0, s>>>(d_v, kin, (uint32_t)m, kk, final, buf[cur], d_ids, d_vals);
        kin = buf[cur];
        m = (size_t)blocks * kk;
        cur ^= 1;
        if (blocks == 1) break;
    }
    return dq_launch_status();
}

int dq_sample_reset(void* d_state, const int32_t* hist, size_t n, void* stream) {
    if (!d_state || (n && !hist)) return DQ_ERR_INVALID_ARG;
    dq_sample_state_t h;
    memset(&h, 0, sizeof(h));
    const size_t m = n < (size_t)DQ_SAMPLE_HIST ? n : (size_t)DQ_SAMPLE_HIST;
    for (int i = 0; i < DQ_SAMPLE_HIST; ++i) h.hist[i] = -1;
    for (size_t i = 0; i < m; ++i) h.hist[i] = hist[n - m + i];
    h.len = (uint32_t)m;
    h.wpos = (uint32_t)(m % DQ_SAMPLE_HIST);
    h.tok = n ? hist[n - 1] : 0;
    const hipStream_t s = (hipStream_t)stream;
    if (hipMemcpyAsync(d_state, &h, sizeof(h), hipMemcpyHostToDevice, s) != hipSuccess) return dq_launch_status();
    return hipStreamSynchronize(s) == hipSuccess ? DQ_OK : DQ_ERR_IO;
}

int dq_sample_candidates(const float* d_vals, const int32_t* d_ids, uint32_t n, const CudaSampleArgs* args,
                         void* d_state, void* stream) {
    if (!d_vals || !d_ids || !args || !d_state) return DQ_ERR_INVALID_ARG;
    if (n == 0 || n > 256 || args->slot > 3) return DQ_ERR_NOT_SUPPORTED;
    if (args->temperature > 0.0f && args->top_k <= 0) return DQ_ERR_NOT_SUPPORTED;
    if (args->penalty_last_n > DQ_SAMPLE_HIST) return DQ_ERR_NOT_SUPPORTED;
    sample_kernel<<<1, 256, 0, (hipStream_t)stream>>>(d_vals, d_ids, n, *args, (dq_sample_state_t*)d_state);
    return dq_launch_status();
}

int dq_embed_q8_0(const void* d_w, size_t rows, size_t cols, const int32_t* d_tok, float mul, float* d_x,
                  void* stream) {
    DqLayout L;
    if (!dq_layout(DQ_FMT_Q8_0, rows, cols, &L)) return DQ_ERR_NOT_SUPPORTED;
    if (!d_w || !d_tok || !d_x) return DQ_ERR_INVALID_ARG;
    if (rows > 0x7FFFFFFF || cols > 0xFFFFFFFFu) return DQ_ERR_NOT_SUPPORTED;
    const uint8_t* base = (const uint8_t*)d_w;
    const unsigned grid = (unsigned)((cols + 255) / 256 < 64 ? (cols + 255) / 256 : 64);
    embed_q8_0_kernel<<<grid, 256, 0, (hipStream_t)stream>>>(base + L.q_off, L.p_stride, L.q_row,
                                                             (const uint16_t*)(base + L.d_off), d_tok, (uint32_t)rows,
                                                             (uint32_t)cols, mul, d_x);
    return dq_launch_status();
}

}  // extern "C"
