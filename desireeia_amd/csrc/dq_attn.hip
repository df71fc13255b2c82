// dq_attn.hip - the Q8_0 KV cache on the device: row writes (quantize the new
// K/V rows into the cache) and batch-1 decode attention over it.
//
// Cache layout (one layer), as the reference keeps it (models/dense_forward.cpp
// :2425, :4038-4043): [pos][kv_head][hd/32 Q8_0 blocks of 34 bytes], i.e. a
// row of 136 bytes per (pos, kv head) at hd = 128 and 8 * 136 = 1088 bytes per
// position at 8 KV heads.
//
// Attention is split over positions (flash-decoding): workgroup (kv head,
// split) walks tiles of 64 positions, tile j of a split s being s, s+S, ...,
// and keeps a running max / sum / weighted V sum for the HPK query heads that
// share the KV head (GQA), so each K/V byte is read once for all of them. A
// second kernel merges the S partials of each head, and can also quantize the
// merged output for the output projection. The position may be read
// from device memory at run time, so the same launch can be replayed in a
// graph for successive tokens.
//
// Arithmetic (reference models/dense_forward.cpp:3956-4065, kv/kv_quant.cpp):
// score = (sum over blocks of d * sum(q_k * q)) / sqrt(hd) with the query in
// fp32; softmax; out = sum_p w_p * d_p * q_v. The sums run in fp32 in another
// order than the reference's (the reference sums the softmax denominator in
// double); results agree to ~1e-6 relative.
#include <cstdlib>

#include "dq_common.h"

namespace {

constexpr int TP = 64;         // positions per tile
constexpr int NT = 256;        // threads per workgroup
constexpr int MAX_SPLIT = 256;

int g_cus = 0;
int num_cus() {
    if (g_cus == 0) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
            g_cus = n;
        else
            g_cus = 256;
    }
    return g_cus;
}

__device__ __forceinline__ int read_pos(int pos_host, const int* pos_dev, int n_ctx) {
    int p = pos_dev ? *pos_dev : pos_host;
    // a device position outside the cache is clamped: never read or write
    // outside [0, n_ctx)
    return p < 0 ? 0 : (p >= n_ctx ? n_ctx - 1 : p);
}

// ------------------------------------------------------------ row writes --
// kv/kv_quant.cpp:31-56 (kv_quantize_row): per 32 values amax, d = amax/127,
// id = 1/d, q = clamp(lrintf(x*id), -127, 127), fp16 d stored before the 32
// int8. One lane per 32-value block; K blocks first, then V blocks.
__global__ __launch_bounds__(256) void kv_write_kernel(const float* __restrict__ k, const float* __restrict__ v,
                                                      int n_blocks, uint8_t* __restrict__ kc,
                                                      uint8_t* __restrict__ vc, size_t pos_bytes, int pos_host,
                                                      const int* __restrict__ pos_dev, int n_ctx) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= 2 * n_blocks) return;
    const bool is_v = b >= n_blocks;
    const int bb = is_v ? b - n_blocks : b;
    const float* x = (is_v ? v : k) + (size_t)bb * 32;
    const int pos = read_pos(pos_host, pos_dev, n_ctx);
    // the blocks of all heads of one position are contiguous: head h block j
    // is block h*hd/32 + j
    uint8_t* dst = (is_v ? vc : kc) + (size_t)pos * pos_bytes + (size_t)bb * DQ_SZ_Q8_0;
    float xv[32];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 f = reinterpret_cast<const float4*>(x)[i];
        xv[4 * i] = f.x, xv[4 * i + 1] = f.y, xv[4 * i + 2] = f.z, xv[4 * i + 3] = f.w;
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(xv[i]));
    const float d = amax > 0.0f ? amax / 127.0f : 0.0f;
    const float id = d > 0.0f ? 1.0f / d : 0.0f;
    // 34-byte blocks are 2-byte aligned: 17 halfword stores
    uint16_t* o = reinterpret_cast<uint16_t*>(dst);
    o[0] = dq_f2h(d);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        int a = (int)rintf(xv[2 * i] * id), c = (int)rintf(xv[2 * i + 1] * id);
        a = a > 127 ? 127 : (a < -127 ? -127 : a);
        c = c > 127 ? 127 : (c < -127 ? -127 : c);
        o[1 + i] = (uint16_t)((a & 0xFF) | ((c & 0xFF) << 8));
    }
}

// ------------------------------------------------------- split attention --
// Partial record of one (query head, split): HD floats of unnormalised
// weighted V sum, then the running max and the running sum of weights.
template <int HD>
struct Part {
    static constexpr int FLOATS = HD + 2;
};

template <int HD, int HPK>
__global__ __launch_bounds__(NT) void attn_part_kernel(const float* __restrict__ q, const uint8_t* __restrict__ kc,
                                                       const uint8_t* __restrict__ vc, int n_kv, size_t pos_bytes,
                                                       int cc_start, int pos_host, const int* __restrict__ pos_dev,
                                                       int n_ctx, int n_split, float scale, float* __restrict__ part) {
    constexpr int NB = HD / 32;       // Q8_0 blocks per row
    constexpr int RB = NB * DQ_SZ_Q8_0;  // row bytes
    constexpr int RBW = RB / 4;       // row dwords
    constexpr int NW = NT / 64;
    constexpr int DP = HD / 2;        // dim pairs (V phase)
    constexpr int PG = NT / DP;       // position groups (V phase)
    constexpr int PPG = TP / PG;      // positions per group
    constexpr int STAGE_IT = (TP * RBW + NT - 1) / NT;
    static_assert(RB % 4 == 0 && NT % DP == 0 && TP % PG == 0, "shape");

    __shared__ uint32_t ks[TP * RBW];
    __shared__ uint32_t vs[TP * RBW];
    __shared__ float qt[HD][HPK];           // query, transposed
    __shared__ float qsum[NB][HPK];         // per-block sums of the query
    __shared__ float sp[NB][HPK][TP];       // per-block partial scores
    __shared__ float pw[TP][HPK];           // tile weights exp(s - m)
    __shared__ float alpha[HPK];
    __shared__ float red[PG][HPK][HD];      // V-phase cross-group reduction

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // XCD-aware placement: consecutive workgroups go to different XCDs; the
    // heads of one split share an XCD (their rows share cache lines).
    const int n_xcd = 8;
    const int xcd = blockIdx.x % n_xcd, slot = blockIdx.x / n_xcd;
    const int kvh = slot % n_kv;
    const int s = xcd + n_xcd * (slot / n_kv);
    if (s >= n_split) return;
    const int pos = read_pos(pos_host, pos_dev, n_ctx);
    const int c0 = cc_start < pos ? cc_start : pos;
    const int npos = pos + 1 - c0;
    const int n_tiles = (npos + TP - 1) / TP;
    if (s >= n_tiles) return;

    // K/V rows of the first tile: issued before the query is staged
    uint32_t kr[STAGE_IT], vr[STAGE_IT];
    auto load_tile = [&](int t) {
        const int p0 = c0 + t * TP;
        const int nv = min(TP, pos + 1 - p0);
        const uint8_t* kb = kc + (size_t)p0 * pos_bytes + (size_t)kvh * RB;
        const uint8_t* vb = vc + (size_t)p0 * pos_bytes + (size_t)kvh * RB;
#pragma unroll
        for (int it = 0; it < STAGE_IT; ++it) {
            const int i = tid + it * NT;
            const int r = i / RBW, c = i % RBW;
            if (r < nv) {
                kr[it] = *reinterpret_cast<const uint32_t*>(kb + (size_t)r * pos_bytes + 4 * c);
                vr[it] = *reinterpret_cast<const uint32_t*>(vb + (size_t)r * pos_bytes + 4 * c);
            } else {
                kr[it] = 0;
                vr[it] = 0;
            }
        }
    };
    load_tile(s);

    // query of the HPK heads of this KV head
    for (int i = tid; i < HPK * HD; i += NT) qt[i % HD][i / HD] = q[(size_t)(kvh * HPK + i / HD) * HD + i % HD];
    __syncthreads();
    if (tid < NB * HPK) {
        const int b = tid / HPK, h = tid % HPK;
        float a = 0.0f;
        for (int i = 0; i < 32; ++i) a += qt[32 * b + i][h];
        qsum[b][h] = a;
    }

    float m_run = -INFINITY, l_run = 0.0f;  // of head `wave` (waves < HPK)
    float m_run2 = -INFINITY, l_run2 = 0.0f;  // of head wave + NW (HPK == 8)
    float acc[HPK][2];
#pragma unroll
    for (int h = 0; h < HPK; ++h) acc[h][0] = acc[h][1] = 0.0f;
    const int dp = tid % DP, pg = tid / DP;
    const int vblk = (2 * dp) / 32;
    const int voff = vblk * DQ_SZ_Q8_0 + 2 + 2 * (dp % 16);

    for (int t = s; t < n_tiles; t += n_split) {
        const int p0 = c0 + t * TP;
        const int nv = min(TP, pos + 1 - p0);
        __syncthreads();  // previous tile's LDS reads are done
#pragma unroll
        for (int it = 0; it < STAGE_IT; ++it) {
            const int i = tid + it * NT;
            if (i < TP * RBW) {
                ks[i] = kr[it];
                vs[i] = vr[it];
            }
        }
        __syncthreads();
        if (t + n_split < n_tiles) load_tile(t + n_split);  // prefetch the next tile
        // ---- partial scores: wave w takes blocks w, w+NW, ...; lane = position
        for (int b = wave; b < NB; b += NW) {
            const int p = lane;
            const uint32_t* row = ks + p * RBW;
            const int o = b * DQ_SZ_Q8_0;  // byte offset of the block in the row
            const int w0 = o >> 2;
            uint32_t dw[9];
#pragma unroll
            for (int i = 0; i < 9; ++i) dw[i] = row[w0 + i];
            float dk;
            uint32_t qw[8];
            if ((o & 3) == 0) {
                dk = dq_h2f((uint16_t)(dw[0] & 0xFFFF));
#pragma unroll
                for (int i = 0; i < 8; ++i) qw[i] = __builtin_amdgcn_alignbyte(dw[i + 1], dw[i], 2);
            } else {
                dk = dq_h2f((uint16_t)(dw[0] >> 16));
#pragma unroll
                for (int i = 0; i < 8; ++i) qw[i] = dw[i + 1];
            }
            // bytes biased to unsigned (q + 128): one conversion per value,
            // the bias removed with the query's block sum
            float a[HPK];
#pragma unroll
            for (int h = 0; h < HPK; ++h) a[h] = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t u = qw[i] ^ 0x80808080u;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float fv = (float)((u >> (8 * k)) & 0xFF);
                    const int dim = 32 * b + 4 * i + k;
#pragma unroll
                    for (int h = 0; h < HPK; ++h) a[h] = fmaf(fv, qt[dim][h], a[h]);
                }
            }
#pragma unroll
            for (int h = 0; h < HPK; ++h) sp[b][h][p] = dk * fmaf(-128.0f, qsum[b][h], a[h]);
        }
        __syncthreads();
        // ---- tile softmax: wave w takes heads w, w+NW
#pragma unroll
        for (int hh = 0; hh < (HPK + NW - 1) / NW; ++hh) {
            const int h = wave + hh * NW;
            if (h < HPK) {
                const int p = lane;
                float sc = -INFINITY;
                if (p < nv) {
                    float a = 0.0f;
#pragma unroll
                    for (int b = 0; b < NB; ++b) a += sp[b][h][p];
                    sc = a * scale;
                }
                const float tmax = dq_wave_max(sc);
                float& mr = hh == 0 ? m_run : m_run2;
                float& lr = hh == 0 ? l_run : l_run2;
                const float m_new = fmaxf(mr, tmax);
                const float al = __expf(mr - m_new);  // 0 on the first tile
                const float e = p < nv ? __expf(sc - m_new) : 0.0f;
                lr = al * lr + dq_wave_sum(e);
                mr = m_new;
                pw[p][h] = e;
                if (lane == 0) alpha[h] = al;
            }
        }
        __syncthreads();
        // ---- weighted V sum: thread = (dim pair, position group)
        {
#pragma unroll
            for (int h = 0; h < HPK; ++h) {
                const float al = alpha[h];
                acc[h][0] *= al;
                acc[h][1] *= al;
            }
            const uint8_t* vbytes = reinterpret_cast<const uint8_t*>(vs);
            const int pend = min(nv, (pg + 1) * PPG);
            for (int p = pg * PPG; p < pend; ++p) {
                const uint8_t* row = vbytes + p * RB;
                const uint16_t vv = *reinterpret_cast<const uint16_t*>(row + voff);
                const float dv = dq_h2f(*reinterpret_cast<const uint16_t*>(row + vblk * DQ_SZ_Q8_0));
                const float f0 = (float)(int8_t)(vv & 0xFF), f1 = (float)(int8_t)(vv >> 8);
#pragma unroll
                for (int h = 0; h < HPK; ++h) {
                    const float wd = pw[p][h] * dv;
                    acc[h][0] = fmaf(wd, f0, acc[h][0]);
                    acc[h][1] = fmaf(wd, f1, acc[h][1]);
                }
            }
        }
    }
    // ---- reduce the position groups and write the partial record
#pragma unroll
    for (int h = 0; h < HPK; ++h) {
        red[pg][h][2 * dp] = acc[h][0];
        red[pg][h][2 * dp + 1] = acc[h][1];
    }
    __syncthreads();
    float* rec = part + ((size_t)kvh * n_split + s) * HPK * Part<HD>::FLOATS;
    for (int i = tid; i < HPK * HD; i += NT) {
        const int h = i / HD, dd = i % HD;
        float a = 0.0f;
#pragma unroll
        for (int g = 0; g < PG; ++g) a += red[g][h][dd];
        rec[h * Part<HD>::FLOATS + dd] = a;
    }
#pragma unroll
    for (int hh = 0; hh < (HPK + NW - 1) / NW; ++hh) {
        const int h = wave + hh * NW;
        if (h < HPK && lane == 0) {
            rec[h * Part<HD>::FLOATS + HD] = hh == 0 ? m_run : m_run2;
            rec[h * Part<HD>::FLOATS + HD + 1] = hh == 0 ? l_run : l_run2;
        }
    }

}

// Merge of the split partials: workgroup b owns outputs [256b, 256b + 256) of
// the flattened [n_head][HD] output (two heads at HD = 128). out = sum_s
// e^(m_s-M) acc_s / sum_s e^(m_s-M) l_s per head. 1024 threads: thread t sums
// output t % 256 over the splits s = t / 256 (mod 4); up to 32 of its loads
// are issued together with the (m, l) loads, so the merge costs about one
// memory round trip. Optionally quantizes the 256 outputs (the per-256
// activation of the output projection).
constexpr int MT = 1024;
constexpr int MG = MT / 256;  // split groups
constexpr int MPRE = 32;      // acc loads per thread issued up front

template <int HD, int HPK>
__global__ __launch_bounds__(MT) void attn_merge_kernel(const float* __restrict__ part, int n_split, int cc_start,
                                                        int pos_host, const int* __restrict__ pos_dev, int n_ctx,
                                                        float* __restrict__ out, int8_t* __restrict__ oq,
                                                        float* __restrict__ oscale, int32_t* __restrict__ oisum) {
    constexpr int HPB = 256 / HD;  // heads per block
    static_assert(256 % HD == 0, "whole heads per block");
    __shared__ float ml[HPB][2][MAX_SPLIT];
    __shared__ float hsum[HPB];
    __shared__ float red[MG][256];
    __shared__ float wmax[MT / 64];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int pos = read_pos(pos_host, pos_dev, n_ctx);
    const int c0 = cc_start < pos ? cc_start : pos;
    const int n_tiles = (pos + 1 - c0 + TP - 1) / TP;
    const int n_used = min(n_split, n_tiles);
    const int o0 = blockIdx.x * 256;          // first output of the block
    const int d = t & 255, sg = t >> 8;
    const int hq = (o0 + d) / HD, dd = (o0 + d) % HD;
    const int kvh = hq / HPK, h = hq % HPK;
    const size_t stride = (size_t)HPK * Part<HD>::FLOATS;
    const float* base = part + (size_t)kvh * n_split * stride + (size_t)h * Part<HD>::FLOATS;
    float pre[MPRE];
#pragma unroll
    for (int i = 0; i < MPRE; ++i) {
        const int sidx = sg + MG * i;
        pre[i] = sidx < n_used ? base[sidx * stride + dd] : 0.0f;
    }
    // (m, l) of the block's heads: thread t < n_used loads split t
    if (t < HPB * MAX_SPLIT) {
        const int j = t / MAX_SPLIT, sidx = t % MAX_SPLIT;
        const int hqj = o0 / HD + j;
        const float* bj = part + (size_t)(hqj / HPK) * n_split * stride + (size_t)(hqj % HPK) * Part<HD>::FLOATS;
        ml[j][0][sidx] = sidx < n_used ? bj[sidx * stride + HD] : -INFINITY;
        ml[j][1][sidx] = sidx < n_used ? bj[sidx * stride + HD + 1] : 0.0f;
    }
    __syncthreads();
    // per head: M = max m_s, weights f_s = e^(m_s - M), L = sum f_s l_s
    // (waves 0..3 handle head 0, waves 4..7 head 1: MAX_SPLIT = 256 splits)
    if (wave < 4 * HPB) {
        const int j = wave / 4, sidx = (wave % 4) * 64 + lane;
        const float m = ml[j][0][sidx];
        const float M0 = dq_wave_max(m);
        if (lane == 0) wmax[wave] = M0;
    }
    __syncthreads();
    if (wave < 4 * HPB) {
        const int j = wave / 4, sidx = (wave % 4) * 64 + lane;
        const float M = fmaxf(fmaxf(wmax[4 * j], wmax[4 * j + 1]), fmaxf(wmax[4 * j + 2], wmax[4 * j + 3]));
        const float f = sidx < n_used ? __expf(ml[j][0][sidx] - M) : 0.0f;
        const float lw = dq_wave_sum(f * ml[j][1][sidx]);
        ml[j][0][sidx] = f;  // weights replace the maxima
        if (lane == 0) red[0][wave] = lw;
    }
    __syncthreads();
    if (t < HPB) hsum[t] = (red[0][4 * t] + red[0][4 * t + 1]) + (red[0][4 * t + 2] + red[0][4 * t + 3]);
    __syncthreads();
    const int j = d / HD;
    float o = 0.0f;
#pragma unroll
    for (int i = 0; i < MPRE; ++i) {
        const int sidx = sg + MG * i;
        if (sidx < n_used) o = fmaf(ml[j][0][sidx], pre[i], o);
    }
    for (int sidx = sg + MG * MPRE; sidx < n_used; sidx += MG) o = fmaf(ml[j][0][sidx], base[sidx * stride + dd], o);
    red[sg][d] = o;
    __syncthreads();
    float v = 0.0f;
    if (sg == 0) {
        v = ((red[0][d] + red[1][d]) + (red[2][d] + red[3][d])) / hsum[j];
        out[o0 + d] = v;
    }
    if (!oq) return;  // uniform
    // per-256 quantization (core/matmul.cpp:1660-1778) by waves 0..3
    if (sg == 0) {
        const float am = dq_wave_max(fabsf(v));
        if (lane == 0) wmax[wave] = am;
    }
    __syncthreads();
    if (sg != 0) return;
    const float amax = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    const float dsc = amax > 0.0f ? amax / 127.0f : 0.0f;
    const float id = dsc > 0.0f ? 127.0f / amax : 0.0f;
    int iv = (int)rintf(v * id);
    iv = iv > 127 ? 127 : (iv < -127 ? -127 : iv);
    oq[o0 + d] = (int8_t)iv;
    int sum = iv;
#pragma unroll
    for (int off = 1; off < 32; off <<= 1) sum += __shfl_xor(sum, off, DQ_WAVE);
    if ((d & 31) == 0) {
        oscale[(o0 + d) / 32] = dsc;
        oisum[(o0 + d) / 32] = sum;
    }
}

int env_int(const char* name, int dflt) {
    const char* e = getenv(name);
    return e ? atoi(e) : dflt;
}

int split_count(int n_kv, int n_tiles_max) {
    // about `tpw` tiles per workgroup (the next tile's loads overlap the
    // current tile's arithmetic), at most four workgroups per CU, a multiple
    // of the 8 XCDs
    static const int tpw = env_int("DQ_ATTN_TPW", 2) < 1 ? 1 : env_int("DQ_ATTN_TPW", 2);
    int s = (4 * num_cus() + n_kv - 1) / n_kv;
    const int want = (n_tiles_max + tpw - 1) / tpw;
    s = s < want ? s : want;
    s = (s + 7) & ~7;
    return s < MAX_SPLIT ? s : MAX_SPLIT;
}

// Workspace: the split partial records.
size_t work_bytes_for(int n_head, int hd, int n_split) {
    return dq_align256((size_t)n_head * n_split * (hd + 2) * sizeof(float));
}

template <int HD, int HPK>
int launch_attn(const float* q, const uint8_t* kc, const uint8_t* vc, int n_kv, int cc_start, int pos,
                const int* pos_dev, int n_ctx, float* out, uint8_t* work, int n_split, int8_t* oq, float* os,
                int32_t* oi, hipStream_t st) {
    const size_t pos_bytes = (size_t)n_kv * (HD / 32) * DQ_SZ_Q8_0;
    const float scale = 1.0f / sqrtf((float)HD);
    float* part = reinterpret_cast<float*>(work);
    attn_part_kernel<HD, HPK><<<n_kv * n_split, NT, 0, st>>>(q, kc, vc, n_kv, pos_bytes, cc_start, pos, pos_dev,
                                                              n_ctx, n_split, scale, part);
    attn_merge_kernel<HD, HPK><<<n_kv * HPK * HD / 256, MT, 0, st>>>(part, n_split, cc_start, pos, pos_dev, n_ctx,
                                                                       out, oq, os, oi);
    return dq_launch_status();
}

bool attn_shape_ok(uint32_t n_head, uint32_t n_head_kv, uint32_t hd) {
    if (n_head_kv == 0 || n_head % n_head_kv) return false;
    const uint32_t hpk = n_head / n_head_kv;
    // the merge takes whole 256-output blocks
    return hd == 128 && (hpk == 1 || hpk == 2 || hpk == 4 || hpk == 8) && (n_head * hd) % 256 == 0;
}

int attn_run(const float* d_q, const void* d_kc, const void* d_vc, uint32_t n_head, uint32_t n_head_kv, uint32_t hd,
             uint32_t cc_start, uint32_t pos, const int32_t* d_pos, uint32_t n_ctx, float* d_out, void* d_work,
             size_t work_bytes, int8_t* oq, float* os, int32_t* oi, void* stream) {
    if (!d_q || !d_kc || !d_vc || !d_out || !d_work || n_ctx == 0) return DQ_ERR_INVALID_ARG;
    if (!attn_shape_ok(n_head, n_head_kv, hd)) return DQ_ERR_NOT_SUPPORTED;
    if (!d_pos && (pos >= n_ctx || cc_start > pos)) return DQ_ERR_INVALID_ARG;
    const uint32_t hpk = n_head / n_head_kv;
    if (oq && (!os || !oi)) return DQ_ERR_INVALID_ARG;
    // with a host position the split count follows the live context; with a
    // device position it is sized for the whole cache
    const uint32_t span = d_pos ? n_ctx : pos + 1 - cc_start;
    const int n_split = split_count((int)n_head_kv, (int)((span + TP - 1) / TP));
    if (work_bytes < work_bytes_for((int)n_head, (int)hd, n_split)) return DQ_ERR_INVALID_ARG;
    const hipStream_t st = (hipStream_t)stream;
    const uint8_t* kc = (const uint8_t*)d_kc;
    const uint8_t* vc = (const uint8_t*)d_vc;
    uint8_t* w = (uint8_t*)d_work;
    const int a = (int)cc_start, p = (int)pos, nk = (int)n_head_kv, nc = (int)n_ctx;
    switch (hpk) {
    case 1: return launch_attn<128, 1>(d_q, kc, vc, nk, a, p, d_pos, nc, d_out, w, n_split, oq, os, oi, st);
    case 2: return launch_attn<128, 2>(d_q, kc, vc, nk, a, p, d_pos, nc, d_out, w, n_split, oq, os, oi, st);
    case 4: return launch_attn<128, 4>(d_q, kc, vc, nk, a, p, d_pos, nc, d_out, w, n_split, oq, os, oi, st);
    case 8: return launch_attn<128, 8>(d_q, kc, vc, nk, a, p, d_pos, nc, d_out, w, n_split, oq, os, oi, st);
    }
    return DQ_ERR_NOT_SUPPORTED;
}

}  // namespace

extern "C" {

int dq_kv_write(const float* d_k, const float* d_v, uint32_t n_head_kv, uint32_t hd, void* d_kc, void* d_vc,
                uint32_t pos, const int32_t* d_pos, uint32_t n_ctx, void* stream) {
    if (!d_k || !d_v || !d_kc || !d_vc || n_head_kv == 0 || hd == 0 || hd % 32 || n_ctx == 0) return DQ_ERR_INVALID_ARG;
    if (!d_pos && pos >= n_ctx) return DQ_ERR_INVALID_ARG;
    const int n_blocks = (int)(n_head_kv * hd / 32);
    const size_t pos_bytes = (size_t)n_blocks * DQ_SZ_Q8_0;
    kv_write_kernel<<<(2 * n_blocks + 255) / 256, 256, 0, (hipStream_t)stream>>>(
        d_k, d_v, n_blocks, (uint8_t*)d_kc, (uint8_t*)d_vc, pos_bytes, (int)pos, d_pos, (int)n_ctx);
    return dq_launch_status();
}

int dq_attn_workspace_bytes(uint32_t n_head, uint32_t n_head_kv, uint32_t hd, uint32_t n_ctx, size_t* bytes) {
    if (!bytes || n_ctx == 0) return DQ_ERR_INVALID_ARG;
    if (!attn_shape_ok(n_head, n_head_kv, hd)) return DQ_ERR_NOT_SUPPORTED;
    const int n_split = split_count((int)n_head_kv, (int)((n_ctx + TP - 1) / TP));
    *bytes = work_bytes_for((int)n_head, (int)hd, n_split);
    return DQ_OK;
}

int dq_attn_decode_q8(const float* d_q, const void* d_kc, const void* d_vc, uint32_t n_head, uint32_t n_head_kv,
                      uint32_t hd, uint32_t cc_start, uint32_t pos, const int32_t* d_pos, uint32_t n_ctx,
                      float* d_out, void* d_work, size_t work_bytes, void* stream) {
    return attn_run(d_q, d_kc, d_vc, n_head, n_head_kv, hd, cc_start, pos, d_pos, n_ctx, d_out, d_work, work_bytes,
                    nullptr, nullptr, nullptr, stream);
}

int dq_attn_decode_q8_act(const float* d_q, const void* d_kc, const void* d_vc, uint32_t n_head,
                          uint32_t n_head_kv, uint32_t hd, uint32_t cc_start, uint32_t pos, const int32_t* d_pos,
                          uint32_t n_ctx, float* d_out, int8_t* d_oq, float* d_oscale, int32_t* d_oisum,
                          void* d_work, size_t work_bytes, void* stream) {
    if (!d_oq) return DQ_ERR_INVALID_ARG;
    return attn_run(d_q, d_kc, d_vc, n_head, n_head_kv, hd, cc_start, pos, d_pos, n_ctx, d_out, d_work, work_bytes,
                    d_oq, d_oscale, d_oisum, stream);
}

}  // extern "C"
