// dq_attn.hip - the Q8_0 KV cache on the device: row writes (quantize the new
// K/V rows into the cache) and batch-1 decode attention over it.
//
// Cache layout (one layer), as the reference keeps it (models/dense_forward.cpp
// :2425, :4038-4043): [pos][kv_head][hd/32 Q8_0 blocks of 34 bytes], i.e. a
// row of 136 bytes per (pos, kv head) at hd = 128 and 8 * 136 = 1088 bytes per
// position at 8 KV heads. Head dims 64, 128 and 256 are supported.
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
// fp32; softmax; out = sum_p w_p * d_p * q_v. Both products run on the matrix
// cores with the fp32 factors split into fp16 hi + lo parts (~22 significant
// bits; the int8 factors are exact) and fp32 sums in another order than the
// reference's (which sums the softmax denominator in double); results agree
// to ~1e-6 relative over any range of K / V scales.
#include <cstdlib>
#include <mutex>
#include <type_traits>

#include "dq_common.h"
#include "dq_f16.h"

namespace {

constexpr int TP = 64;         // positions per tile
constexpr int NT = 256;        // threads per workgroup

typedef float f4v __attribute__((ext_vector_type(4)));

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
// One workgroup per (KV head, tile of TP positions): the tile's K and V rows
// go straight into LDS (dword DMA), and the HPK query heads that share the KV
// head (GQA: each KV byte is read once for all of them) are scored, the tile
// softmax taken and the weighted V sum formed on the matrix cores; the
// workgroup writes a partial record (acc[HD], tile max, tile sum) per head
// for attn_merge_kernel.
//
// Both products run as v_mfma_f32_16x16x32_f16 with exact operands:
//  * scores, per (16 positions, Q8_0 block b): A = the query's 32 values of
//    block b (rows = heads), B = the 32 K bytes of each position (int8 values
//    are exact in fp16); the fp32 result is scaled by the position's block
//    scale dk and summed over the blocks, as the reference's
//    sum_b dk * sum(q * k8);
//  * weighted sum, per (32 positions, 16 dims of block b): A = the weight
//    w[h][p] * dv[p][b] (rows = heads), B = the V bytes, read position-major.
// The fp32 A operands are split into fp16 hi + lo parts (hi*B + lo*B: ~22
// significant bits), after scaling by a power of two that puts the largest
// value of the head (query) or block (weights) in [2^13, 2^14): no fp16
// overflow, full precision for the values that matter, and the scaling is
// undone exactly afterwards.
//
// FUSE: q, k, v are the raw projections of the new token: every workgroup
// applies the optional bias / QK-norm and RoPE to its query heads, and the
// workgroup of the last tile (the one holding `pos`) also processes k and v,
// quantizes the new K and V rows of its KV head (kv_quantize_row), writes
// them into the cache and uses them directly. This replaces the separate
// RoPE + KV-write kernel of the decoder layer.
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

// 8 int8 values (two dwords) -> 8 fp16, exactly: the fp16 of bits
// 0x64 | (b ^ 0x80) is 1024 + b + 128.
__device__ __forceinline__ h8 i8x8_to_h8(uint32_t w0, uint32_t w1) {
    const h2 c = {(_Float16)1152.0f, (_Float16)1152.0f};
    const uint32_t t0 = w0 ^ 0x80808080u, t1 = w1 ^ 0x80808080u;
    const h2 r0 = magic_pair(t0, 0x04010400u) - c, r1 = magic_pair(t0, 0x04030402u) - c;
    const h2 r2 = magic_pair(t1, 0x04010400u) - c, r3 = magic_pair(t1, 0x04030402u) - c;
    const dq_u32x4 w = {__builtin_bit_cast(uint32_t, r0), __builtin_bit_cast(uint32_t, r1),
                        __builtin_bit_cast(uint32_t, r2), __builtin_bit_cast(uint32_t, r3)};
    return __builtin_bit_cast(h8, w);
}

// 8 int8 values held as bytes (zero-extended, one per word) -> 8 fp16.
__device__ __forceinline__ h8 i8_bytes_to_h8(const uint32_t (&u)[8]) {
    const h2 c = {(_Float16)1152.0f, (_Float16)1152.0f};
    dq_u32x4 w;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        w[i] = __builtin_bit_cast(uint32_t,
                                  __builtin_bit_cast(h2, (u[2 * i] | (u[2 * i + 1] << 16)) ^ 0x64806480u) - c);
    return __builtin_bit_cast(h8, w);
}

__device__ __forceinline__ void split_hl(float x, _Float16& hi, _Float16& lo) {
    hi = (_Float16)x;
    lo = (_Float16)(x - (float)hi);
}

// Exponent shift that brings a largest magnitude m into [2^13, 2^14) (0 for
// m == 0 or not finite).
__device__ __forceinline__ int pow2_shift(float m, int cap) {
    if (!(m > 0.0f) || !(m <= 3.0e38f)) return 0;
    int e = 0;
    (void)frexpf(m, &e);
    return min(14 - e, cap);
}

template <int HD, int HPK, bool FUSE>
__global__ __launch_bounds__(NT) void attn_tile_kernel(AttnArgs A) {
    constexpr int NB = HD / 32;            // Q8_0 blocks per row
    constexpr int RB = NB * DQ_SZ_Q8_0;    // row bytes
    constexpr int NW = NT / 64;
    constexpr int GPW = TP / 16 / NW;      // 16-position groups per wave
    constexpr int KS = TP / 32;            // 32-position steps of the V product
    constexpr int RBW = RB / 4;            // row dwords
    constexpr int NDMA = TP * RBW / 64;    // dword-DMA instructions per tensor
    constexpr int DPW = (NDMA + NW - 1) / NW;
    constexpr int QROW = HD + 8;           // fp16 row of the query operands (padded)
    constexpr int REC = HD + 4;            // acc[HD], max, sum, 2 pad (16-byte records)
    constexpr int HPW = (HPK + NW - 1) / NW;
    constexpr int QV = HD / 64;            // values of a head per lane (value lane + 64 i)
    constexpr int CTW = HD / 16 / NW;      // 16-dim output column tiles per wave
    constexpr int RP = HD == 64 ? 1 : QV / 2;  // RoPE pairs per lane
    static_assert(dq_head_dim_ok<HD>() && HPK <= 8 && TP % 64 == 0 && RB % 4 == 0 && CTW >= 1, "shape");

    __shared__ __align__(16) uint32_t kt[TP * RBW];     // K rows of the tile (RB bytes each)
    __shared__ __align__(16) uint32_t vt[TP * RBW];     // V rows
    __shared__ __align__(16) _Float16 qhs[16 * QROW];   // scaled query, fp16 hi (rows >= HPK zero)
    __shared__ __align__(16) _Float16 qls[16 * QROW];   // and lo
    __shared__ __align__(16) float dvf[NB][TP];         // V block scales times dvs (0 past the tile)
    // tile weights exp(s - m) (rows >= HPK zero), rows padded by 4 floats: the
    // weighted V sum reads one column of 16 rows per instruction, which at a
    // 256-byte row stride would fall in one bank
    constexpr int EWS = TP + 4;
    __shared__ __align__(16) float ew[16][EWS];
    __shared__ uint32_t nrow[2][RBW];                   // FUSE: the new K and V rows
    __shared__ float qsc[HPK];                          // per head: 1/sqrt(hd) / query scale
    __shared__ float dvs[NB];                           // per block: weight operand scale
    __shared__ float wmx[NW][HPK], wsm[NW][HPK];        // per-wave maxima and sums
    constexpr int NSTG = FUSE ? (2 * HPW + 5) * HD : HPW * HD;
    __shared__ __align__(16) float stg[NW][NSTG];       // per wave: raw inputs staged by DMA

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n16 = lane & 15, g4 = lane >> 4;
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
    const bool new_row = FUSE && tile == n_tiles - 1;
    const int n_load = new_row ? nv - 1 : nv;

    // ---- raw inputs of this wave's query heads (wave w takes heads w, w+NW)
    // and, under FUSE, their biases, the RoPE table, the QK-norm weights and
    // the new K (wave 0) / V (wave 1) row with its bias: staged into the
    // wave's LDS area by DMA ahead of the tile's K and V rows, and read after
    // a wait counted to cover exactly these (absent inputs stage q and are
    // ignored). The compiler waits for every outstanding load at the first
    // use of a plain load issued next to LDS DMAs, which held the query work
    // behind the whole tile transfer (and, under FUSE, the tile's DMAs behind
    // the query loads).
    const float* const dmy = A.q;
    auto stage = [&](const float* src, int off) {
#pragma unroll
        for (int i = 0; i < HD / 64; ++i)
            __builtin_amdgcn_global_load_lds(src + 64 * i + lane, DQ_LDS_PTR(&stg[wave][off + 64 * i]), 4, 0, 0);
    };
#pragma unroll
    for (int t = 0; t < HPW; ++t) {
        const size_t hq = (size_t)kvh * HPK + min(wave + NW * t, HPK - 1);
        stage(A.q + hq * HD, t * HD);
        if constexpr (FUSE) stage(A.post.bq ? A.post.bq + hq * HD : dmy, (HPW + t) * HD);
    }
    if constexpr (FUSE) {
        stage(A.rope ? A.rope : dmy, (2 * HPW) * HD);
        stage(A.post.q_norm ? A.post.q_norm : dmy, (2 * HPW + 1) * HD);
        const size_t o = (size_t)kvh * HD;
        const float* src = wave == 0 ? A.k : A.v;
        const float* bias = wave == 0 ? A.post.bk : A.post.bv;
        stage(src + o, (2 * HPW + 2) * HD);
        stage(bias ? bias + o : dmy, (2 * HPW + 3) * HD);
        stage(A.post.k_norm ? A.post.k_norm : dmy, (2 * HPW + 4) * HD);
    }
    // ---- the tile's K and V rows, straight into LDS (lane i of a dword DMA
    // writes dword i of the instruction's 64-dword span, row r of the tile at
    // byte RB r: each instruction reads 256 consecutive bytes of rows). Every
    // wave issues the same count (spare slots repeat the last span), and rows
    // at or past n_load read a row of the tile instead: rows >= nv are never
    // used, and the new row is written over afterwards.
    {
        const uint8_t* kb = A.kc + (size_t)p0 * A.pos_bytes + (size_t)kvh * RB;
        const uint8_t* vb = A.vc + (size_t)p0 * A.pos_bytes + (size_t)kvh * RB;
        const int rmax = n_load > 0 ? n_load - 1 : 0;
#pragma unroll
        for (int i = 0; i < DPW; ++i) {
            const int j = min(wave + NW * i, NDMA - 1);
            const int d = 64 * j + lane;
            const int r = d / RBW, c = d - r * RBW;
            const uint32_t go = (uint32_t)min(r, rmax) * (uint32_t)A.pos_bytes + 4u * (uint32_t)c;
            __builtin_amdgcn_global_load_lds(kb + go, DQ_LDS_PTR(kt + 64 * j), 4, 0, 0);
            __builtin_amdgcn_global_load_lds(vb + go, DQ_LDS_PTR(vt + 64 * j), 4, 0, 0);
        }
    }
    // the staged inputs have landed (the tile's DMAs, issued after them, may
    // not); a wave's LDS operations run in issue order, so only the compiler
    // is kept from moving the reads above the wait
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * DPW < 63 ? 2 * DPW : 63) : "memory");
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float qx[HPW][QV], qb[HPW][QV];
    float rc[RP], rs[RP], nq[QV], xr[QV], xbias[QV], xn[QV];
    {
        const float* sg = stg[wave];
#pragma unroll
        for (int t = 0; t < HPW; ++t)
#pragma unroll
            for (int i = 0; i < QV; ++i) {
                qx[t][i] = sg[t * HD + lane + 64 * i];
                qb[t][i] = FUSE ? sg[(HPW + t) * HD + lane + 64 * i] : 0.0f;
            }
#pragma unroll
        for (int i = 0; i < RP; ++i) {
            const int j = HD == 64 ? (lane & 31) : lane + 64 * i;
            rc[i] = FUSE ? sg[2 * HPW * HD + 2 * j] : 1.0f;
            rs[i] = FUSE ? sg[2 * HPW * HD + 2 * j + 1] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < QV; ++i) {
            const int c = lane + 64 * i;
            nq[i] = FUSE ? sg[(2 * HPW + 1) * HD + c] : 0.0f;
            xr[i] = FUSE ? sg[(2 * HPW + 2) * HD + c] : 0.0f;
            xbias[i] = FUSE ? sg[(2 * HPW + 3) * HD + c] : 0.0f;
            xn[i] = FUSE ? sg[(2 * HPW + 4) * HD + c] : 0.0f;
        }
    }
    // ---- zero rows HPK..15 of the query and weight operands (the MFMA rows
    // that no head fills)
    {
        constexpr int QZ = (16 - HPK) * QROW * 2 / 16, EZ = (16 - HPK) * EWS * 4 / 16;
        const uint4 z = {0u, 0u, 0u, 0u};
        for (int i = tid; i < QZ; i += NT) {
            reinterpret_cast<uint4*>(qhs + HPK * QROW)[i] = z;
            reinterpret_cast<uint4*>(qls + HPK * QROW)[i] = z;
        }
        for (int i = tid; i < EZ; i += NT) reinterpret_cast<uint4*>(&ew[HPK][0])[i] = z;
    }
    // NeoX RoPE of a head held as x[i] = value lane + 64 i with the lane's
    // pairs' (cos, sin) in registers (dq_rope_head with the table preloaded)
    auto rope = [&](float(&x)[QV]) {
        if constexpr (HD == 64) {
            const float y = __shfl_xor(x[0], 32, DQ_WAVE);
            x[0] = lane < 32 ? x[0] * rc[0] - y * rs[0] : y * rs[0] + x[0] * rc[0];
        } else {
#pragma unroll
            for (int i = 0; i < RP; ++i) {
                const float a = x[i], b = x[i + RP];
                x[i] = a * rc[i] - b * rs[i];
                x[i + RP] = a * rs[i] + b * rc[i];
            }
        }
    };
    // ---- query operands: bias, QK-norm, RoPE (FUSE), then the head's
    // power-of-two scale and the fp16 hi / lo split
#pragma unroll
    for (int t = 0; t < HPW; ++t) {
        const int h = wave + NW * t;
        if (h < HPK) {  // wave-uniform
            float x[QV];
#pragma unroll
            for (int i = 0; i < QV; ++i) x[i] = qx[t][i];
            if constexpr (FUSE) {
                if (A.post.bq) {
#pragma unroll
                    for (int i = 0; i < QV; ++i) x[i] += qb[t][i];
                }
                if (A.post.q_norm) dq_head_rms_norm_w<HD>(x, nq, A.post.eps);
                if (A.rope) rope(x);
            }
            float m = 0.0f;
#pragma unroll
            for (int i = 0; i < QV; ++i) m = fmaxf(m, fabsf(x[i]));
            const int sh = pow2_shift(dq_wave_max_uniform(m), 100);
            const float sc = ldexpf(1.0f, sh);
#pragma unroll
            for (int i = 0; i < QV; ++i) split_hl(x[i] * sc, qhs[h * QROW + lane + 64 * i], qls[h * QROW + lane + 64 * i]);
            if (lane == 0) qsc[h] = A.scale * ldexpf(1.0f, -sh);
        }
    }
    // ---- new K / V row (FUSE, last tile): bias, K-norm and RoPE of k,
    // kv_quantize_row into the cache and into nrow (copied into the tile once
    // the DMAs have landed)
    if constexpr (FUSE) {
        if (new_row && wave < 2) {
            const float* bias = wave == 0 ? A.post.bk : A.post.bv;
            if (bias) {
#pragma unroll
                for (int i = 0; i < QV; ++i) xr[i] += xbias[i];
            }
            if (wave == 0 && A.post.k_norm) dq_head_rms_norm_w<HD>(xr, xn, A.post.eps);
            if (wave == 0 && A.rope) rope(xr);
            uint8_t* grow = (wave == 0 ? A.kc : A.vc) + (size_t)pos * A.pos_bytes + (size_t)kvh * RB;
            dq_q8_0_row<HD>(xr, lane, grow);
            dq_q8_0_row<HD>(xr, lane, reinterpret_cast<uint8_t*>(nrow[wave]));
        }
    }
    __syncthreads();  // every wave's DMAs have landed; query operands in LDS
    if constexpr (FUSE) {
        if (new_row) {  // workgroup-uniform
            if (wave < 2) {
                for (int l = lane; l < RBW; l += 64) (wave == 0 ? kt : vt)[(nv - 1) * RBW + l] = nrow[wave][l];
            }
            __syncthreads();
        }
    }
    const uint8_t* kb8 = reinterpret_cast<const uint8_t*>(kt);
    const uint8_t* vb8 = reinterpret_cast<const uint8_t*>(vt);

    // ---- scores: lane (n16, g4) of group gi holds rows 4*g4 + r (heads) of
    // column n16 (position 16*(wave + NW*gi) + n16)
    float sc[GPW][4];
    {
        h8 qah[NB], qal[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            qah[b] = *reinterpret_cast<const h8*>(qhs + n16 * QROW + 32 * b + 8 * g4);
            qal[b] = *reinterpret_cast<const h8*>(qls + n16 * QROW + 32 * b + 8 * g4);
        }
        float hs[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) hs[r] = 4 * g4 + r < HPK ? qsc[4 * g4 + r] : 0.0f;
#pragma unroll
        for (int gi = 0; gi < GPW; ++gi) {
            const int p = 16 * (wave + NW * gi) + n16;
            // the row's dwords from 2*g4 on (+ the block's first dword)
            const uint32_t* kl = kt + p * RBW + 2 * g4;
            const uint8_t* kr = kb8 + p * RB;
            float s4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                // quants of block b at row bytes 34b + 2 + 8 g4 ...: dword
                // aligned for odd b, two bytes in for even b (RB is a
                // multiple of 4)
                const int cb = (DQ_SZ_Q8_0 * b + 2) >> 2;
                uint32_t w0, w1;
                if (b & 1) {
                    w0 = kl[cb];
                    w1 = kl[cb + 1];
                } else {
                    const uint32_t d0 = kl[cb], d1 = kl[cb + 1], d2 = kl[cb + 2];
                    w0 = __builtin_amdgcn_alignbyte(d1, d0, 2);
                    w1 = __builtin_amdgcn_alignbyte(d2, d1, 2);
                }
                const h8 kv = i8x8_to_h8(w0, w1);
                f4v c = {0.0f, 0.0f, 0.0f, 0.0f};
                c = __builtin_amdgcn_mfma_f32_16x16x32_f16(qah[b], kv, c, 0, 0, 0);
                c = __builtin_amdgcn_mfma_f32_16x16x32_f16(qal[b], kv, c, 0, 0, 0);
                // the block scale: row bytes 34b, 34b + 1
                const float dk = dq_h2f(*reinterpret_cast<const uint16_t*>(kr + DQ_SZ_Q8_0 * b));
#pragma unroll
                for (int r = 0; r < 4; ++r) s4[r] = fmaf(dk, c[r], s4[r]);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) sc[gi][r] = (4 * g4 + r < HPK && p < nv) ? s4[r] * hs[r] : -INFINITY;
        }
    }
    // V block scales (wave w: blocks w, w + NW, ...) and their power-of-two
    // operand scale
    for (int b = wave; b < NB; b += NW) {  // wave-uniform
        float dv[TP / 64];
        float m = 0.0f;
#pragma unroll
        for (int i = 0; i < TP / 64; ++i) {
            const int p = lane + 64 * i;
            dv[i] = p < nv ? dq_h2f(*reinterpret_cast<const uint16_t*>(vb8 + p * RB + DQ_SZ_Q8_0 * b)) : 0.0f;
            m = fmaxf(m, fabsf(dv[i]));
        }
        // dvf holds dv * s (a power of two: exact); the records divide by s
        const float s = ldexpf(1.0f, pow2_shift(dq_wave_max_uniform(m), 100));
#pragma unroll
        for (int i = 0; i < TP / 64; ++i) dvf[b][lane + 64 * i] = dv[i] * s;
        if (lane == 0) dvs[b] = s;
    }
    // ---- tile softmax: per-wave maxima, then the tile's
    {
        float mx[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            mx[r] = sc[0][r];
#pragma unroll
            for (int gi = 1; gi < GPW; ++gi) mx[r] = fmaxf(mx[r], sc[gi][r]);
            mx[r] = dq_row16_max(mx[r]);
            if (n16 == 0 && 4 * g4 + r < HPK) wmx[wave][4 * g4 + r] = mx[r];
        }
    }
    __syncthreads();
    float ls[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int h = 4 * g4 + r;
        float m = -INFINITY;
        if (h < HPK) {
#pragma unroll
            for (int w = 0; w < NW; ++w) m = fmaxf(m, wmx[w][h]);
        }
        ls[r] = 0.0f;
#pragma unroll
        for (int gi = 0; gi < GPW; ++gi) {
            const int p = 16 * (wave + NW * gi) + n16;
            const float e = (h < HPK && p < nv) ? __expf(sc[gi][r] - m) : 0.0f;
            ls[r] += e;
            if (h < HPK) ew[h][p] = e;
        }
        ls[r] = dq_row16_sum(ls[r]);
        if (n16 == 0 && h < HPK) wsm[wave][h] = ls[r];
    }
    __syncthreads();
    // ---- weighted V sum: wave w takes the output column tiles ct = CTW w +
    // c (dims 16 ct + n16 of block ct / 2); lane (n16, g4) of a step takes
    // positions 32 ks + 8 g4 + j
    float* rec = A.part + ((size_t)kvh * A.max_tiles + tile) * HPK * REC;
    {
        f4v o[CTW];
#pragma unroll
        for (int c = 0; c < CTW; ++c) o[c] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            h8 ah, al;
#pragma unroll
            for (int c = 0; c < CTW; ++c) {
                const int ct = CTW * wave + c, b = ct >> 1, t = ct & 1;
                if (c == 0 || t == 0) {
                    // A: the weights W[h][p] = ew[h][p] * dv[p][b] (times the
                    // block's power of two, in dvf) split into fp16 hi / lo
                    // (rows >= HPK: zero)
                    const int p = 32 * ks + 8 * g4;
                    const float4 e0 = *reinterpret_cast<const float4*>(&ew[n16][p]);
                    const float4 e1 = *reinterpret_cast<const float4*>(&ew[n16][p + 4]);
                    const float4 d0 = *reinterpret_cast<const float4*>(&dvf[b][p]);
                    const float4 d1 = *reinterpret_cast<const float4*>(&dvf[b][p + 4]);
                    const float e[8] = {e0.x, e0.y, e0.z, e0.w, e1.x, e1.y, e1.z, e1.w};
                    const float d[8] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        _Float16 x, y;
                        split_hl(e[j] * d[j], x, y);
                        ah[j] = x;
                        al[j] = y;
                    }
                }
                // the lane's V byte (dim 16 ct + n16) of positions 32 ks + 8 g4 + j
                const uint8_t* col = vb8 + (32 * ks + 8 * g4) * RB + DQ_SZ_Q8_0 * b + 2 + 16 * t + n16;
                uint32_t u[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) u[j] = col[j * RB];
                const h8 bv = i8_bytes_to_h8(u);
                o[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bv, o[c], 0, 0, 0);
                o[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bv, o[c], 0, 0, 0);
            }
        }
#pragma unroll
        for (int c = 0; c < CTW; ++c) {
            const int ct = CTW * wave + c;
            const float inv = 1.0f / dvs[ct >> 1];  // a power of two: exact
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int h = 4 * g4 + r;
                if (h < HPK) rec[h * REC + 16 * ct + n16] = o[c][r] * inv;
            }
        }
    }
    if (tid < HPK) {
        float m = wmx[0][tid], l = wsm[0][tid];
#pragma unroll
        for (int w = 1; w < NW; ++w) m = fmaxf(m, wmx[w][tid]);
#pragma unroll
        for (int w = 1; w < NW; ++w) l += wsm[w][tid];
        rec[tid * REC + HD] = m;
        rec[tid * REC + HD + 1] = l;
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
        if (A.post.gate) {  // per-head output gate (dense_forward.cpp:4102-4114)
            const float g = 1.0f / (1.0f + expf(-A.post.gate[blockIdx.x * HPB + hb]));
            v *= g;
        }
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
    return dq_head_dim_supported(hd) && (hpk == 1 || hpk == 2 || hpk == 4 || hpk == 8) && (n_head * hd) % 256 == 0;
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
    auto by_hpk = [&](auto hdc) {
        constexpr int HD = decltype(hdc)::value;
#define DQ_ATTN_CASE(H)                                                                          \
    case H:                                                                                      \
        rc = fuse ? launch_attn<HD, H, true>(a, nh, st) : launch_attn<HD, H, false>(a, nh, st);  \
        break;
        switch (hpk) {
            DQ_ATTN_CASE(1)
            DQ_ATTN_CASE(2)
            DQ_ATTN_CASE(4)
            DQ_ATTN_CASE(8)
        }
#undef DQ_ATTN_CASE
    };
    if (hd == 64)
        by_hpk(std::integral_constant<int, 64>{});
    else if (hd == 128)
        by_hpk(std::integral_constant<int, 128>{});
    else
        by_hpk(std::integral_constant<int, 256>{});
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

int dq_attn_decode_q8_post(const float* d_q, const void* d_kc, const void* d_vc, uint32_t n_head,
                           uint32_t n_head_kv, uint32_t hd, uint32_t cc_start, uint32_t pos, const int32_t* d_pos,
                           uint32_t n_ctx, float* d_out, int8_t* d_oq, float* d_oscale, int32_t* d_oisum,
                           void* d_work, size_t work_bytes, const DqQkvPost& post, void* stream) {
    if (d_oq && (!d_oscale || !d_oisum)) return DQ_ERR_INVALID_ARG;
    return attn_run(d_q, nullptr, nullptr, nullptr, d_kc, d_vc, n_head, n_head_kv, hd, cc_start, pos, d_pos, n_ctx,
                    d_out, d_work, work_bytes, d_oq, d_oscale, d_oisum, stream, post);
}

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
