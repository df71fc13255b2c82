// dq_attn.hip - the Q8_0 KV cache on the device: row writes (quantize the new
// K/V rows into the cache) and batch-1 decode attention over it.
//
// Cache layout (one layer), as the reference keeps it (models/dense_forward.cpp
// :2425, :4038-4043): [pos][kv_head][hd/32 Q8_0 blocks of 34 bytes], i.e. a
// row of 136 bytes per (pos, kv head) at hd = 128 and 8 * 136 = 1088 bytes per
// position at 8 KV heads.
//
// Attention is split over positions (flash-decoding): a workgroup per (KV
// head, tile of 64 positions) keeps the tile's max / sum / weighted V sum for
// the query heads that share the KV head (GQA), and a merge kernel combines
// the tiles and can quantize the output for the output projection (the kernel
// boundary makes the records of every XCD visible without a device-wide cache
// writeback per workgroup). The position may be read from device
// memory at run time, so the same launch can be replayed in a graph for
// successive tokens. A fused form also applies RoPE and writes the new K/V
// rows (the decoder layer's step before attention).
//
// Arithmetic (reference models/dense_forward.cpp:3956-4065, kv/kv_quant.cpp):
// score = (sum over blocks of d * sum(q_k * q)) / sqrt(hd) with the query in
// fp32; softmax; out = sum_p w_p * d_p * q_v. The sums run in fp32 in another
// order than the reference's (the reference sums the softmax denominator in
// double); results agree to ~1e-6 relative.
#include <cstdlib>
#include <mutex>

#include "dq_common.h"

namespace {

constexpr int TP = 64;         // positions per tile
constexpr int NT = 256;        // threads per workgroup

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

// ------------------------------------------------------------ attention --
// One workgroup per (KV head, tile of TP positions): it stages the tile's K
// and V rows through LDS, computes the scores of the HPK query heads that
// share the KV head (GQA: each KV byte is read once for all of them), the
// tile softmax and weighted V sum, and writes a partial record (acc[HD],
// tile max, tile sum) for attn_merge_kernel.
//
// FUSE: q, k, v are the raw projections of the new token: every workgroup
// applies RoPE to its query heads, and the workgroup of the last tile (the
// one holding `pos`) also rotates k, quantizes the new K and V rows of its KV
// head (kv_quantize_row), writes them into the cache and uses them directly.
// This replaces the separate RoPE + KV-write kernel of the decoder layer.
//
// XCD-aware placement: consecutive workgroups go to different XCDs; the KV
// heads of one tile share an XCD, so the 1088-byte position rows they split
// between them are fetched into one L2.
struct AttnArgs {
    const float* q;     // [n_head][HD]: rotated (plain) or raw (FUSE)
    const float* k;     // FUSE: raw new k and v rows [n_kv][HD]
    const float* v;
    const float* rope;  // FUSE: cos/sin table (NULL: no RoPE)
    uint8_t* kc;
    uint8_t* vc;
    size_t pos_bytes;
    int n_kv, cc_start, pos_host, n_ctx, max_tiles;
    const int* pos_dev;
    float scale;
    float* part;          // [n_kv][max_tiles][HPK][HD + 4]
    float* out;           // [n_head][HD]
    int8_t* oq;           // fused per-256 quantization (or NULL)
    float* oscale;
    int32_t* oisum;
    DqQkvPost post;       // FUSE: optional biases and QK-norm before RoPE
};

template <int HD, int HPK, bool FUSE>
__global__ __launch_bounds__(NT) void attn_tile_kernel(AttnArgs A) {
    constexpr int NB = HD / 32;          // Q8_0 blocks per row
    constexpr int RB = NB * DQ_SZ_Q8_0;  // row bytes
    constexpr int RBW = RB / 4;          // row dwords
    constexpr int NW = NT / 64;
    constexpr int DP = HD / 2;           // dim pairs (V phase)
    constexpr int PG = NT / DP;          // position groups (V phase)
    constexpr int PPG = TP / PG;         // positions per group
    constexpr int RBQ = RB / 8;          // row 8-byte words (rows are 8-byte aligned)
    constexpr int STAGE_IT = (TP * RBQ + NT - 1) / NT;
    constexpr int REC = HD + 4;     // acc[HD], max, sum, 2 pad (16-byte records)
    static_assert(HD == 128 && RB % 8 == 0 && NT % DP == 0 && TP % PG == 0, "shape");

    __shared__ uint64_t ks8[TP * RBQ];
    __shared__ uint64_t vs8[TP * RBQ];
    uint32_t* ks = reinterpret_cast<uint32_t*>(ks8);
    uint32_t* vs = reinterpret_cast<uint32_t*>(vs8);
    __shared__ float qt[HD][HPK];        // query, transposed
    __shared__ float qsum[NB][HPK];      // per-block sums of the query
    __shared__ float sp[NB][HPK][TP];    // per-block partial scores
    __shared__ float pw[TP][HPK];        // tile weights exp(s - m)
    __shared__ float red[PG][HPK][HD];   // V-phase cross-group reduction

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n_xcd = 8;
    const int xcd = blockIdx.x % n_xcd, slot = blockIdx.x / n_xcd;
    const int kvh = slot % A.n_kv;
    const int tile = xcd + n_xcd * (slot / A.n_kv);
    const int pos = read_pos(A.pos_host, A.pos_dev, A.n_ctx);
    const int c0 = A.cc_start < pos ? A.cc_start : pos;
    const int n_tiles = (pos + 1 - c0 + TP - 1) / TP;
    if (tile >= n_tiles || tile >= A.max_tiles) return;
    const int p0 = c0 + tile * TP;
    const int nv = min(TP, pos + 1 - p0);
    // the new row (position pos, the last row of the last tile) comes from
    // registers under FUSE
    const int n_load = (FUSE && tile == n_tiles - 1) ? nv - 1 : nv;

    // ---- query values of this wave's heads (FUSE: wave w takes heads w,
    // w+NW) and the new row's RoPE pair, loaded before the tile so that
    // waiting for them leaves the tile's loads in flight
    constexpr int HPW = (HPK + NW - 1) / NW;
    float ql[HPW], qhv[HPW], rc = 1.0f, rs = 0.0f;
    if constexpr (FUSE) {
#pragma unroll
        for (int t = 0; t < HPW; ++t) {
            const int h = min(wave + NW * t, HPK - 1);
            const float* qh = A.q + (size_t)(kvh * HPK + h) * HD;
            ql[t] = qh[lane];
            qhv[t] = qh[lane + 64];
        }
        if (A.rope) {
            rc = A.rope[2 * lane];
            rs = A.rope[2 * lane + 1];
        }
    }
    // ---- K / V rows of the tile (8 bytes per load): issued next, staged after the query
    uint64_t kr[STAGE_IT], vr[STAGE_IT];
    {
        const uint8_t* kb = A.kc + (size_t)p0 * A.pos_bytes + (size_t)kvh * RB;
        const uint8_t* vb = A.vc + (size_t)p0 * A.pos_bytes + (size_t)kvh * RB;
        // unconditional loads (addresses clamped into the tile's first rows,
        // which exist: p0 <= pos < n_ctx) so that all of them are in flight
        // together; the values of slots past the tile are never staged
        const int rmax = n_load > 0 ? n_load - 1 : 0;
#pragma unroll
        for (int it = 0; it < STAGE_IT; ++it) {
            const int i = min(tid + it * NT, TP * RBQ - 1);
            const int r = min(i / RBQ, rmax), c = i % RBQ;
            kr[it] = *reinterpret_cast<const uint64_t*>(kb + (size_t)r * A.pos_bytes + 8 * c);
            vr[it] = *reinterpret_cast<const uint64_t*>(vb + (size_t)r * A.pos_bytes + 8 * c);
        }
    }
    // ---- query of the HPK heads (rotated under FUSE: wave w takes heads w, w+NW)
    if constexpr (FUSE) {
#pragma unroll
        for (int t = 0; t < HPW; ++t) {
            const int h = wave + NW * t;
            if (h < HPK) {  // wave-uniform
                float a = ql[t], b = qhv[t];
                dq_qkv_post(a, b, 0, kvh * HPK + h, lane, A.post);
                // NeoX rotation of the pair (j, j + 64) (dq_rope_pair)
                qt[lane][h] = A.rope ? a * rc - b * rs : a;
                qt[lane + 64][h] = A.rope ? a * rs + b * rc : b;
            }
        }
    } else {
        for (int i = tid; i < HPK * HD; i += NT) qt[i % HD][i / HD] = A.q[(size_t)(kvh * HPK + i / HD) * HD + i % HD];
    }
    // rows >= n_load are not staged: the new row (FUSE) is written there by
    // waves 0 and 1 below, and rows >= nv are never read (their scores are
    // masked, the V sum stops at nv)
#pragma unroll
    for (int it = 0; it < STAGE_IT; ++it) {
        const int i = tid + it * NT;
        if (i < TP * RBQ && i / RBQ < n_load) {
            ks8[i] = kr[it];
            vs8[i] = vr[it];
        }
    }
    if constexpr (FUSE) {
        if (tile == n_tiles - 1 && wave < 2) {
            // the new row of this KV head: wave 0 = K (rotated), wave 1 = V
            const float* src = (wave == 0 ? A.k : A.v) + (size_t)kvh * HD;
            float lo = src[lane], hi = src[lane + 64];
            dq_qkv_post(lo, hi, wave == 0 ? 1 : 2, kvh, lane, A.post);
            if (wave == 0 && A.rope) dq_rope_pair(lo, hi, A.rope, lane);
            uint8_t* lrow = reinterpret_cast<uint8_t*>(wave == 0 ? ks : vs) + (nv - 1) * RB;
            dq_q8_0_row128(lo, hi, lane, lrow);
            uint8_t* grow = (wave == 0 ? A.kc : A.vc) + (size_t)pos * A.pos_bytes + (size_t)kvh * RB;
            dq_q8_0_row128(lo, hi, lane, grow);
        }
    }
    __syncthreads();
    if (tid < NB * HPK) {
        const int b = tid / HPK, h = tid % HPK;
        float a = 0.0f;
        for (int i = 0; i < 32; ++i) a += qt[32 * b + i][h];
        qsum[b][h] = a;
    }
    __syncthreads();
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
        // bytes biased to unsigned (q + 128): one conversion per value, the
        // bias removed with the query's block sum
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
    // ---- tile softmax: wave w takes heads w, w+NW; lane = position
    float* rec = A.part + ((size_t)kvh * A.max_tiles + tile) * HPK * REC;
    for (int h = wave; h < HPK; h += NW) {
        const int p = lane;
        float sc = -INFINITY;
        if (p < nv) {
            float a = 0.0f;
#pragma unroll
            for (int b = 0; b < NB; ++b) a += sp[b][h][p];
            sc = a * A.scale;
        }
        const float m = dq_wave_max(sc);
        const float e = p < nv ? __expf(sc - m) : 0.0f;
        const float l = dq_wave_sum(e);
        pw[p][h] = e;
        if (lane == 0) {
            rec[h * REC + HD] = m;
            rec[h * REC + HD + 1] = l;
        }
    }
    __syncthreads();
    // ---- weighted V sum: thread = (dim pair, position group)
    {
        const int dp = tid % DP, pg = tid / DP;
        const int vblk = (2 * dp) / 32;
        const int voff = vblk * DQ_SZ_Q8_0 + 2 + 2 * (dp % 16);
        float acc[HPK][2];
#pragma unroll
        for (int h = 0; h < HPK; ++h) acc[h][0] = acc[h][1] = 0.0f;
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
#pragma unroll
        for (int h = 0; h < HPK; ++h) {
            red[pg][h][2 * dp] = acc[h][0];
            red[pg][h][2 * dp + 1] = acc[h][1];
        }
    }
    __syncthreads();
    for (int i = tid; i < HPK * HD; i += NT) {
        const int h = i / HD, dd = i % HD;
        float a = 0.0f;
#pragma unroll
        for (int g = 0; g < PG; ++g) a += red[g][h][dd];
        rec[h * REC + dd] = a;
    }
}

// Merge of the tile records: workgroup b owns outputs [256b, 256b + 256) of
// the flattened [n_head][HD] output (HD = 128: two heads). Thread (g, q)
// takes output quad q (4 consecutive outputs, one 16-byte record load per
// tile) and tiles g, g+MG, ... in batches of MB (all of a batch's record
// loads in flight at once: one memory round trip for up to MG*MB tiles),
// keeping an online softmax state (running max M, sum L of e^(m_t - M) l_t,
// and acc of e^(m_t - M) acc_t); the MG group states are then combined in
// group order, each rescaled to the common max. Optionally quantizes the 256
// outputs per 256 (core/matmul.cpp:1660-1778).
constexpr int MNO = 256;              // outputs per merge workgroup
constexpr int MQ = MNO / 4;           // output quads
constexpr int MG = 16;                // tile groups of the merge
constexpr int MNT = MG * MQ;          // its threads
constexpr int MB = 6;                 // tiles per batch and thread
template <int HD, int HPK>
__global__ __launch_bounds__(MNT) void attn_merge_kernel(AttnArgs A) {
    constexpr int REC = HD + 4;
    constexpr int HPB = MNO / HD;        // heads per block
    constexpr int NWO = MNO / 64;        // waves holding the final outputs
    static_assert(MNO % HD == 0 && MNO == NT && HD % 4 == 0, "whole heads per block");
    __shared__ float wred[NWO];
    __shared__ float gm[MG][HPB], gl[MG][HPB];
    __shared__ float4 pacc[MG][MQ];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = tid / MQ, qd = tid % MQ;        // tile group, output quad
    const int pos = read_pos(A.pos_host, A.pos_dev, A.n_ctx);
    const int c0 = A.cc_start < pos ? A.cc_start : pos;
    const int n_tiles = min((pos + 1 - c0 + TP - 1) / TP, A.max_tiles);
    {
        const int ol = 4 * qd;                    // first output of the quad in the block
        const int hb = ol / HD;                   // head within the block
        const int hq = blockIdx.x * HPB + hb;     // query head
        const int kvh = hq / HPK, h = hq % HPK, dd = ol % HD;
        const float* recs = A.part + ((size_t)kvh * A.max_tiles * HPK + h) * REC;  // tile t at + t*HPK*REC
        float M = -INFINITY, L = 0.0f;
        float4 a = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int tb = g; tb < n_tiles; tb += MG * MB) {
            float4 v[MB];
            float2 ml[MB];
#pragma unroll
            for (int k = 0; k < MB; ++k) {
                const float* r = recs + (size_t)min(tb + MG * k, n_tiles - 1) * HPK * REC;
                v[k] = *reinterpret_cast<const float4*>(r + dd);
                ml[k] = *reinterpret_cast<const float2*>(r + HD);
            }
            float bm = M;
#pragma unroll
            for (int k = 0; k < MB; ++k)
                if (tb + MG * k < n_tiles) bm = fmaxf(bm, ml[k].x);
            const float sc = __expf(M - bm);  // M = -inf on the first batch: 0
            a.x *= sc, a.y *= sc, a.z *= sc, a.w *= sc;
            L *= sc;
#pragma unroll
            for (int k = 0; k < MB; ++k)
                if (tb + MG * k < n_tiles) {
                    const float w = __expf(ml[k].x - bm);
                    a.x = fmaf(w, v[k].x, a.x);
                    a.y = fmaf(w, v[k].y, a.y);
                    a.z = fmaf(w, v[k].z, a.z);
                    a.w = fmaf(w, v[k].w, a.w);
                    L = fmaf(w, ml[k].y, L);
                }
            M = bm;
        }
        pacc[g][qd] = a;
        if (dd == 0) {
            gm[g][hb] = M;
            gl[g][hb] = L;
        }
    }
    __syncthreads();
    // the first MNO threads finish output o = tid; the others stay for the barriers
    float v = 0.0f;
    if (tid < MNO) {
        const int hb = tid / HD;
        float Mt = gm[0][hb];
#pragma unroll
        for (int q = 1; q < MG; ++q) Mt = fmaxf(Mt, gm[q][hb]);
        float acc = 0.0f, Lt = 0.0f;
#pragma unroll
        for (int q = 0; q < MG; ++q) {
            const float w = __expf(gm[q][hb] - Mt);  // a group with no tile: e^-inf = 0
            acc = fmaf(w, pacc[q][tid / 4][tid % 4], acc);
            Lt = fmaf(w, gl[q][hb], Lt);
        }
        v = acc / Lt;
        A.out[(size_t)blockIdx.x * MNO + tid] = v;
    }
    if (!A.oq) return;  // uniform
    // per-256 quantization of the block's 256 outputs
    const float am = dq_wave_max(fabsf(v));
    if (lane == 0 && wave < NWO) wred[wave] = am;
    __syncthreads();
    if (tid >= MNO) return;
    float amax = wred[0];
#pragma unroll
    for (int w = 1; w < NWO; ++w) amax = fmaxf(amax, wred[w]);
    const float d = amax > 0.0f ? amax / 127.0f : 0.0f;
    const float id = d > 0.0f ? 127.0f / amax : 0.0f;
    int iv = (int)rintf(v * id);
    iv = iv > 127 ? 127 : (iv < -127 ? -127 : iv);
    const int o = blockIdx.x * MNO + tid;
    A.oq[o] = (int8_t)iv;
    int sum = iv;
#pragma unroll
    for (int off = 1; off < 32; off <<= 1) sum += __shfl_xor(sum, off, DQ_WAVE);
    if ((tid & 31) == 0) {
        A.oscale[o / 32] = d;
        A.oisum[o / 32] = sum;
    }
}

// Workspace: the tile records.
int max_tiles_for(uint32_t n_ctx) { return (int)((n_ctx + TP - 1) / TP); }
size_t work_bytes_for(int n_head, int hd, int max_tiles) {
    return dq_align256((size_t)n_head * max_tiles * (hd + 4) * sizeof(float));
}

template <int HD, int HPK, bool FUSE>
int launch_attn(const AttnArgs& a, int n_head, hipStream_t st) {
    const int slots = a.n_kv * ((a.max_tiles + 7) / 8);  // per XCD
    attn_tile_kernel<HD, HPK, FUSE><<<8 * slots, NT, 0, st>>>(a);
    attn_merge_kernel<HD, HPK><<<n_head * HD / MNO, MNT, 0, st>>>(a);
    return dq_launch_status();
}

bool attn_shape_ok(uint32_t n_head, uint32_t n_head_kv, uint32_t hd) {
    if (n_head_kv == 0 || n_head % n_head_kv || n_head_kv > 4096) return false;
    const uint32_t hpk = n_head / n_head_kv;
    // the merge takes whole 256-output blocks
    return hd == 128 && (hpk == 1 || hpk == 2 || hpk == 4 || hpk == 8) && (n_head * hd) % 256 == 0;
}

int attn_run(const float* d_q, const float* d_k, const float* d_v, const float* d_rope, const void* d_kc,
             const void* d_vc, uint32_t n_head, uint32_t n_head_kv, uint32_t hd, uint32_t cc_start, uint32_t pos,
             const int32_t* d_pos, uint32_t n_ctx, float* d_out, void* d_work, size_t work_bytes, int8_t* oq,
             float* os, int32_t* oi, void* stream, const DqQkvPost& post = DqQkvPost{}) {
    if (!d_q || !d_kc || !d_vc || !d_out || !d_work || n_ctx == 0) return DQ_ERR_INVALID_ARG;
    if (!attn_shape_ok(n_head, n_head_kv, hd)) return DQ_ERR_NOT_SUPPORTED;
    if (!d_pos && (pos >= n_ctx || cc_start > pos)) return DQ_ERR_INVALID_ARG;
    if (oq && (!os || !oi)) return DQ_ERR_INVALID_ARG;
    const bool fuse = d_k != nullptr;
    if (fuse && !d_v) return DQ_ERR_INVALID_ARG;
    const uint32_t hpk = n_head / n_head_kv;
    const int mt = max_tiles_for(n_ctx);
    if (work_bytes < work_bytes_for((int)n_head, (int)hd, mt)) return DQ_ERR_INVALID_ARG;
    const hipStream_t st = (hipStream_t)stream;
    AttnArgs a{};
    a.q = d_q;
    a.k = d_k;
    a.v = d_v;
    a.rope = d_rope;
    a.kc = (uint8_t*)d_kc;
    a.vc = (uint8_t*)d_vc;
    a.pos_bytes = (size_t)n_head_kv * (hd / 32) * DQ_SZ_Q8_0;
    a.n_kv = (int)n_head_kv;
    a.cc_start = (int)cc_start;
    a.pos_host = (int)pos;
    a.pos_dev = d_pos;
    a.n_ctx = (int)n_ctx;
    a.max_tiles = mt;
    a.scale = 1.0f / sqrtf((float)hd);
    a.part = (float*)d_work;
    a.out = d_out;
    a.oq = oq;
    a.oscale = os;
    a.oisum = oi;
    a.post = post;
    const int nh = (int)n_head;
    int rc = DQ_ERR_NOT_SUPPORTED;
#define DQ_ATTN_CASE(H)                                                                              \
    case H:                                                                                          \
        rc = fuse ? launch_attn<128, H, true>(a, nh, st) : launch_attn<128, H, false>(a, nh, st);    \
        break;
    switch (hpk) {
        DQ_ATTN_CASE(1)
        DQ_ATTN_CASE(2)
        DQ_ATTN_CASE(4)
        DQ_ATTN_CASE(8)
    }
#undef DQ_ATTN_CASE
    return rc;
}

// Scratch of the allocation-free entry point: the tile records in a
// file-scope device array, one per device the library runs on, held until the
// process ends. Host code never names the array in a kernel argument or a
// copy: its host-side name is not a device address. The device address comes
// from hipGetSymbolAddress, looked up once per device with that device
// current, and is what the kernels are given.
constexpr size_t NOALLOC_SCRATCH_BYTES = 16u << 20;
__device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[MAX_DEVICES];

// The device address of this device's scratch array (NULL on failure).
void* scratch_ptr() {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return nullptr;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return nullptr;
        g_scratch_ptr[dev] = p;
    }
    return g_scratch_ptr[dev];
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
    *bytes = work_bytes_for((int)n_head, (int)hd, max_tiles_for(n_ctx));
    return DQ_OK;
}

int dq_attn_decode_q8(const float* d_q, const void* d_kc, const void* d_vc, uint32_t n_head, uint32_t n_head_kv,
                      uint32_t hd, uint32_t cc_start, uint32_t pos, const int32_t* d_pos, uint32_t n_ctx,
                      float* d_out, void* d_work, size_t work_bytes, void* stream) {
    return attn_run(d_q, nullptr, nullptr, nullptr, d_kc, d_vc, n_head, n_head_kv, hd, cc_start, pos, d_pos, n_ctx,
                    d_out, d_work, work_bytes, nullptr, nullptr, nullptr, stream);
}

int dq_attn_decode_q8_noalloc(const float* d_q, const void* d_kc, const void* d_vc, uint32_t n_head,
                              uint32_t n_head_kv, uint32_t hd, uint32_t cc_start, uint32_t pos, const int32_t* d_pos,
                              uint32_t n_ctx, float* d_out, void* stream) {
    if (!d_q || !d_kc || !d_vc || !d_out || n_ctx == 0) return DQ_ERR_INVALID_ARG;
    if (!attn_shape_ok(n_head, n_head_kv, hd)) return DQ_ERR_NOT_SUPPORTED;
    const size_t need = work_bytes_for((int)n_head, (int)hd, max_tiles_for(n_ctx));
    if (need > NOALLOC_SCRATCH_BYTES) return DQ_ERR_NOT_SUPPORTED;  // beyond the static scratch
    void* work = scratch_ptr();
    if (!work) return DQ_ERR_IO;
    return attn_run(d_q, nullptr, nullptr, nullptr, d_kc, d_vc, n_head, n_head_kv, hd, cc_start, pos, d_pos, n_ctx,
                    d_out, work, NOALLOC_SCRATCH_BYTES, nullptr, nullptr, nullptr, stream);
}

int dq_attn_decode_q8_act(const float* d_q, const void* d_kc, const void* d_vc, uint32_t n_head,
                          uint32_t n_head_kv, uint32_t hd, uint32_t cc_start, uint32_t pos, const int32_t* d_pos,
                          uint32_t n_ctx, float* d_out, int8_t* d_oq, float* d_oscale, int32_t* d_oisum,
                          void* d_work, size_t work_bytes, void* stream) {
    if (!d_oq) return DQ_ERR_INVALID_ARG;
    return attn_run(d_q, nullptr, nullptr, nullptr, d_kc, d_vc, n_head, n_head_kv, hd, cc_start, pos, d_pos, n_ctx,
                    d_out, d_work, work_bytes, d_oq, d_oscale, d_oisum, stream);
}

int dq_attn_rope_kv_decode(const float* d_q, const float* d_k, const float* d_v, const float* d_rope,
                           uint32_t n_rot, void* d_kc, void* d_vc, uint32_t n_head, uint32_t n_head_kv, uint32_t hd,
                           uint32_t cc_start, uint32_t pos, const int32_t* d_pos, uint32_t n_ctx, float* d_out,
                           int8_t* d_oq, float* d_oscale, int32_t* d_oisum, void* d_work, size_t work_bytes,
                           void* stream) {
    return dq_attn_rope_kv_decode_post(d_q, d_k, d_v, d_rope, n_rot, d_kc, d_vc, n_head, n_head_kv, hd, cc_start, pos,
                                       d_pos, n_ctx, d_out, d_oq, d_oscale, d_oisum, d_work, work_bytes, DqQkvPost{},
                                       stream);
}

}  // extern "C"

int dq_attn_rope_kv_decode_post(const float* d_q, const float* d_k, const float* d_v, const float* d_rope,
                                uint32_t n_rot, void* d_kc, void* d_vc, uint32_t n_head, uint32_t n_head_kv,
                                uint32_t hd, uint32_t cc_start, uint32_t pos, const int32_t* d_pos, uint32_t n_ctx,
                                float* d_out, int8_t* d_oq, float* d_oscale, int32_t* d_oisum, void* d_work,
                                size_t work_bytes, const DqQkvPost& post, void* stream) {
    if (!d_k || !d_v) return DQ_ERR_INVALID_ARG;
    if (d_rope && n_rot != hd) return DQ_ERR_NOT_SUPPORTED;  // partial rotation: dq_rope_kv_write
    return attn_run(d_q, d_k, d_v, d_rope, d_kc, d_vc, n_head, n_head_kv, hd, cc_start, pos, d_pos, n_ctx, d_out,
                    d_work, work_bytes, d_oq, d_oscale, d_oisum, stream, post);
}
