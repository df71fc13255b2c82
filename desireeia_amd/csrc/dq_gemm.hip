// dq_gemm.hip - prefill GEMM Y[t][r] = sum_k W[r][k] X[t][k] on fp16 MFMA.
//
// Semantics: the reference prefill (i8_gemm, core/matmul.cpp:806 and
// core/i8gemm_impl.h:326-419) quantizes X per 32 (integers q, scale dx) and
// computes, per weight row r and 32-block b,
//     y += float(sum q_w*q_x) * (a_rb*dx_tb) - m_rb * sx_tb
// with sx the exact float sum of the 32 inputs (Q4_K min term). Here both
// operands enter CDNA4's fp16 MFMA pre-scaled:
//     A[t][k] = fp16(q_x * dx)            (the same integers and scale)
//     B[k][r] = fp16(a_rb * q_w)          (a = d*sc; Q6_K: d*sc16, q-32)
// and the Q4_K min term is K/32 extra columns A = fp16(sx), B = fp16(-m).
// Accumulation is fp32. The only difference from the reference is the fp16
// rounding of the two operands (2^-11 relative), which moves the result by
// ~3e-4 relative - inside the 4e-3 tolerance.
//
// Why fp16 and not int8 MFMA: the per-32 float rescale of every int32 block
// partial costs at least one non-packed fp32 VALU op per output per 32 K,
// which on CDNA4 (16 fp32 lanes/clk/SIMD vs ~1024 int8 MAC/clk/SIMD) caps the
// int8 path below half its peak; pre-scaled fp16 operands need no epilogue.
//
// Tiling: 128 (tokens) x 128 (weight rows) x 64 (K) per 256-thread workgroup,
// 4 waves of 64x64 (2x2 v_mfma_f32_32x32x16_f16 tiles), LDS double-buffered
// with XOR-swizzled 16-byte chunks (no bank conflicts on fragment reads); the
// weight tile is dequantized from the packed layout by the loader threads
// while the MFMAs of the previous step run. Q6_K: K is permuted to the packed
// item order (both operands, see dq_quantize_act_f16), so a 64-column K step
// is exactly one 64-weight item.
#include "dq_common.h"
#include "dq_f16.h"

namespace {


constexpr int BM = 128, BK = 64, NS = 3;  // tile rows (tokens), K per step, ring stages

// ------------------------------------------------------------ LDS layout --
// Ring of NS stages, each holding one K step of both operands:
//   A: BM rows x 8 chunks of 16 bytes (fp16), chunk c of row r at slot
//      r*8 + (c ^ (r & 7)) - XOR swizzle: a wave's 16-byte fragment reads (32
//      rows, one logical chunk) hit all banks.
//   B: the raw bytes of the weight tile, format specific:
//      Q4_K: P0[BN][16] P1[BN][16] H[BN][16]    (qs sub-planes, block header)
//      Q6_K: QA[BN][16] QB[BN][16] QH[BN][16] S[BN][4] D[BN][4] (fp16 in the low half)
// Every stage is filled by global_load_lds (direct global -> LDS DMA, 16, 4 or
// 2 bytes per lane; lane i of a wave writes at base + i*16 for 16-byte loads and
// at base + i*4 for the dword and sub-dword forms).
template <int BN>
struct Ring {
    static constexpr int A_BYTES = BM * BK * 2;
    static constexpr int B_BYTES = BN * 64;
    static constexpr int STAGE = A_BYTES + B_BYTES;
    static constexpr int BYTES = NS * STAGE;
};

enum BKind { B_Q4K = 0, B_Q6K = 1 };

#define DQ_LDS_PTR(p) reinterpret_cast<__attribute__((address_space(3))) void*>(reinterpret_cast<uintptr_t>(p))
template <int SIZE>
__device__ __forceinline__ void lds_dma(const void* g, uint8_t* lds_wave_base);
template <>
__device__ __forceinline__ void lds_dma<16>(const void* g, uint8_t* b) {
    __builtin_amdgcn_global_load_lds(g, DQ_LDS_PTR(b), 16, 0, 0);
}
template <>
__device__ __forceinline__ void lds_dma<4>(const void* g, uint8_t* b) {
    __builtin_amdgcn_global_load_lds(g, DQ_LDS_PTR(b), 4, 0, 0);
}
template <>
__device__ __forceinline__ void lds_dma<2>(const void* g, uint8_t* b) {
    __builtin_amdgcn_global_load_lds(g, DQ_LDS_PTR(b), 2, 0, 0);
}

// s_waitcnt vmcnt(n), other counters untouched (gfx9 encoding: vmcnt in
// bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
__device__ __forceinline__ void wait_vm(int n) {
#define DQ_WAIT_CASE(k) \
    case k: __builtin_amdgcn_s_waitcnt(((k) & 15) | (((k) >> 4) << 14) | (7 << 4) | (15 << 8)); break;
    switch (n) {
        DQ_WAIT_CASE(0) DQ_WAIT_CASE(1) DQ_WAIT_CASE(2) DQ_WAIT_CASE(3) DQ_WAIT_CASE(4) DQ_WAIT_CASE(5)
        DQ_WAIT_CASE(6) DQ_WAIT_CASE(7) DQ_WAIT_CASE(8) DQ_WAIT_CASE(9) DQ_WAIT_CASE(10) DQ_WAIT_CASE(11)
        DQ_WAIT_CASE(12) DQ_WAIT_CASE(13) DQ_WAIT_CASE(14) DQ_WAIT_CASE(15)
        default: __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8)); break;
    }
#undef DQ_WAIT_CASE
}

struct GemmArgs {
    const uint8_t* w;       // packed weights
    DqLayout L;
    const _Float16* A;      // activations [M][lda]
    const _Float16* mins;   // Q4_K min plane [N][ld_min] (fp16 -dmin*m), or null
    const float* inv;       // per token: 1/s of its activation row
    int lda, ld_min, M, N, K;
    int m0, n0;
};

// Issues the DMA of K step `st` (weights and activations) into ring stage
// `stage`. Every wave issues the same, compile-time number of load
// instructions (stage_loads()), so one s_waitcnt vmcnt covers a stage: blocks
// of 64 slots are dealt to the NW waves, and where a region has fewer blocks
// than waves two waves load the same block (identical bytes to the same LDS
// address).
template <int BN, int KIND>
constexpr int stage_loads() {
    constexpr int NW = BN / 32;
    return BM * 8 / 64 / NW + (KIND == B_Q4K ? 2 : 3);
}

template <int BN, int KIND>
__device__ __forceinline__ void issue_stage(const GemmArgs& g, uint8_t* ring, int stage, int st, int main_steps,
                                            int wave, int lane) {
    constexpr int NW = BN / 32;      // waves per workgroup
    constexpr int HB = BN / 64;      // 64-slot blocks per [BN] region (= NW/2)
    uint8_t* base = ring + stage * Ring<BN>::STAGE;
    // A: BM*8 slots of 16 bytes
    {
        const int kcol = st * BK;
#pragma unroll
        for (int j = 0; j < BM * 8 / 64 / NW; ++j) {
            const int jj = j * NW + wave;
            const int slot = jj * 64 + lane;
            const int r = slot >> 3, c = (slot & 7) ^ (r & 7);
            const int m = min(g.m0 + r, g.M - 1);
            lds_dma<16>(g.A + (size_t)m * g.lda + kcol + 8 * c, base + jj * 64 * 16);
        }
    }
    uint8_t* bb = base + Ring<BN>::A_BYTES;
    if constexpr (KIND == B_Q4K) {
        {   // P0/P1: 2*HB = NW blocks, one per wave
            const int region = wave / HB, n = (wave % HB) * 64 + lane;
            const size_t r = (size_t)min(g.n0 + n, g.N - 1);
            lds_dma<16>(g.w + g.L.q_off + (size_t)region * g.L.p_stride + r * g.L.q_row + 16 * (size_t)st,
                        bb + wave * 64 * 16);
        }
        {   // H: HB blocks, waves w and w + HB load block w % HB
            const int blk = wave % HB, n = blk * 64 + lane;
            const size_t r = (size_t)min(g.n0 + n, g.N - 1);
            lds_dma<16>(g.w + g.L.s_off + r * g.L.s_row + 16 * (size_t)(st >> 2), bb + 2 * BN * 16 + blk * 64 * 16);
        }
    } else if constexpr (KIND == B_Q6K) {
        {   // QA/QB/QH blocks 0..NW-1: one per wave
            const int region = wave / HB, n = (wave % HB) * 64 + lane;
            const size_t r = (size_t)min(g.n0 + n, g.N - 1);
            lds_dma<16>(g.w + g.L.q_off + (size_t)region * g.L.p_stride + r * g.L.q_row + 16 * (size_t)st,
                        bb + wave * 64 * 16);
        }
        if (wave < HB) {  // QH blocks (the last HB plane blocks)
            const int n = wave * 64 + lane;
            const size_t r = (size_t)min(g.n0 + n, g.N - 1);
            lds_dma<16>(g.w + g.L.q_off + 2 * g.L.p_stride + r * g.L.q_row + 16 * (size_t)st,
                        bb + (NW + wave) * 64 * 16);
        } else {          // S: HB blocks of dwords
            const int n = (wave - HB) * 64 + lane;
            const size_t r = (size_t)min(g.n0 + n, g.N - 1);
            lds_dma<4>(g.w + g.L.s_off + r * g.L.s_row + 4 * (size_t)st, bb + 3 * BN * 16 + (wave - HB) * 64 * 4);
        }
        {   // D: HB blocks of ushorts, waves w and w + HB load block w % HB. A
            // sub-dword LDS DMA still advances 4 bytes per lane: d sits in the
            // low half of a dword slot.
            const int blk = wave % HB, n = blk * 64 + lane;
            const size_t r = (size_t)min(g.n0 + n, g.N - 1);
            lds_dma<2>(g.w + g.L.d_off + r * g.L.d_row + 2 * (size_t)(st >> 2),
                       bb + 3 * BN * 16 + BN * 4 + blk * 64 * 4);
        }
    }
}

__device__ __forceinline__ const h8& lds_h8(const uint8_t* p) { return *reinterpret_cast<const h8*>(p); }

// B fragments of one ring stage for this lane: bf[kk][j], kk = 16-wide K
// slice, j = 32-row n block. Lane l feeds row n = wn*64 + j*32 + l%32 with the
// 8 K values kk*16 + 8*(l/32) .. +7.
template <int BN, int KIND>
__device__ __forceinline__ void b_fragments(const uint8_t* bb, int st, int wn, int lane, int n_valid, h8 (&bf)[4][2]) {
    const int h = lane >> 5;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int n = wn * 64 + j * 32 + (lane & 31);
        const bool ok = n < n_valid;
        if constexpr (KIND == B_Q4K) {
            const dq_u32x2 p0 = *reinterpret_cast<const dq_u32x2*>(bb + n * 16 + 8 * h);
            const dq_u32x2 p1 = *reinterpret_cast<const dq_u32x2*>(bb + BN * 16 + n * 16 + 8 * h);
            const dq_u32x4 hd = *reinterpret_cast<const dq_u32x4*>(bb + 2 * BN * 16 + n * 16);
            const int g = st & 3;
            const float d = dq_h2f((uint16_t)(hd.x & 0xFFFF));
            const _Float16 a0 = (_Float16)(ok ? d * (float)q4k_scale(2 * g, hd.y, hd.z, hd.w) : 0.0f);
            const _Float16 a1 = (_Float16)(ok ? d * (float)q4k_scale(2 * g + 1, hd.y, hd.z, hd.w) : 0.0f);
            const h2 bias = {(_Float16)1024.0f, (_Float16)1024.0f};
            const h2 v0 = {a0, a0}, v1 = {a1, a1};
            uint32_t t[4];
            // kk 0: P0 low nibbles, 1: P1 low, 2: P0 high, 3: P1 high
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                const dq_u32x2 src = (kk & 1) ? p1 : p0;
                const uint32_t m0 = kk < 2 ? (src.x & 0x0F0F0F0Fu) : ((src.x >> 4) & 0x0F0F0F0Fu);
                const uint32_t m1 = kk < 2 ? (src.y & 0x0F0F0F0Fu) : ((src.y >> 4) & 0x0F0F0F0Fu);
                bytes_to_h2(m0, bias, kk < 2 ? v0 : v1, &t[0]);
                bytes_to_h2(m1, bias, kk < 2 ? v0 : v1, &t[2]);
                bf[kk][j] = __builtin_bit_cast(h8, dq_u32x4{t[0], t[1], t[2], t[3]});
            }
        } else {
            const dq_u32x2 qa = *reinterpret_cast<const dq_u32x2*>(bb + n * 16 + 8 * h);
            const dq_u32x2 qb = *reinterpret_cast<const dq_u32x2*>(bb + BN * 16 + n * 16 + 8 * h);
            const dq_u32x2 qh = *reinterpret_cast<const dq_u32x2*>(bb + 2 * BN * 16 + n * 16 + 8 * h);
            const uint32_t sc = *reinterpret_cast<const uint32_t*>(bb + 3 * BN * 16 + n * 4);
            const float d = dq_h2f(*reinterpret_cast<const uint16_t*>(bb + 3 * BN * 16 + BN * 4 + n * 4));
            const h2 bias = {(_Float16)1056.0f, (_Float16)1056.0f};  // 1024 + 32
            uint32_t t[4];
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                const _Float16 a = (_Float16)(ok ? d * (float)(int8_t)((sc >> (8 * kk)) & 0xFF) : 0.0f);
                const h2 va = {a, a};
                const dq_u32x2 lo = (kk & 1) ? qb : qa;
#pragma unroll
                for (int wd = 0; wd < 2; ++wd) {
                    const uint32_t l4 = kk < 2 ? (lo[wd] & 0x0F0F0F0Fu) : ((lo[wd] >> 4) & 0x0F0F0F0Fu);
                    const uint32_t v6 = l4 | (((qh[wd] >> (2 * kk)) & 0x03030303u) << 4);
                    bytes_to_h2(v6, bias, va, &t[2 * wd]);
                }
                bf[kk][j] = __builtin_bit_cast(h8, dq_u32x4{t[0], t[1], t[2], t[3]});
            }
        }
    }
}

// K steps [s0, s1): fill NS-1 stages, then per step: wait for the oldest
// stage, barrier, issue the DMA NS-1 steps ahead (steps past the end re-issue
// the last one, so every wave issues the same count per stage), run the MFMAs
// of the current stage.
template <int BN, int KIND>
__device__ __forceinline__ void run_steps(const GemmArgs& g, uint8_t* ring, int s0, int s1, int main_steps,
                                          f16v (&acc)[2][2], int wave, int lane) {
    if (s0 >= s1) return;
    constexpr int PER = stage_loads<BN, KIND>();
    const int wm = wave & 1, wn = wave >> 1;
    const int n_valid = g.N - g.n0;
#pragma unroll
    for (int p = 0; p < NS - 1; ++p) issue_stage<BN, KIND>(g, ring, p, min(s0 + p, s1 - 1), main_steps, wave, lane);
    for (int st = s0; st < s1; ++st) {
        const int stage = (st - s0) % NS;
        // this wave's DMAs of `stage` are done (NS-2 stages still in flight);
        // the barrier makes every wave's DMAs visible and retires step st-1
        wait_vm((NS - 2) * PER);
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        issue_stage<BN, KIND>(g, ring, (st - s0 + NS - 1) % NS, min(st + NS - 1, s1 - 1), main_steps, wave, lane);
        const uint8_t* base = ring + stage * Ring<BN>::STAGE;
        h8 bf[4][2];
        b_fragments<BN, KIND>(base + Ring<BN>::A_BYTES, st, wn, lane, n_valid, bf);
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            h8 af[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int r = wm * 64 + i * 32 + (lane & 31);
                af[i] = lds_h8(base + (r * 8 + ((2 * kk + (lane >> 5)) ^ (r & 7))) * 16);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[kk][j], acc[i][j], 0, 0, 0);
        }
    }
    wait_vm(0);  // drain the DMAs issued past the end
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Q4_K min term, steps [s0, s1) of the min columns: A = fp16 block sums
// (activation columns K + ...), B = fp16(-dmin*m) from the min plane. Small
// (K/32 columns), so fragments come straight from global memory.
__device__ __forceinline__ void min_steps(const GemmArgs& g, int s0, int s1, f16v (&acc)[2][2], int wave, int lane) {
    const int wm = wave & 1, wn = wave >> 1, h = lane >> 5;
    for (int e = s0; e < s1; ++e) {
        const int col = e * BK;
        h8 af[4][2], bf[4][2];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int m = min(g.m0 + wm * 64 + i * 32 + (lane & 31), g.M - 1);
                af[kk][i] = *reinterpret_cast<const h8*>(g.A + (size_t)m * g.lda + g.K + col + kk * 16 + 8 * h);
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int n = min(g.n0 + wn * 64 + j * 32 + (lane & 31), g.N - 1);
                bf[kk][j] = *reinterpret_cast<const h8*>(g.mins + (size_t)n * g.ld_min + col + kk * 16 + 8 * h);
            }
        }
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[kk][i], bf[kk][j], acc[i][j], 0, 0, 0);
    }
}

// Tile index -> (m block, n block): tiles are ordered m-major and handed to
// the 8 XCDs in contiguous ranges (workgroup id % 8 is its XCD), so the
// workgroups of one XCD share their activation rows in that XCD's L2.
__device__ __forceinline__ void tile_of(int id, int mb, int nb, int* m_blk, int* n_blk) {
    const int total = mb * nb;
    int t = id;
    if (total % 8 == 0) t = (id % 8) * (total / 8) + id / 8;
    *m_blk = t / nb;
    *n_blk = t % nb;
}

template <int FMT, int BN>
__global__ __launch_bounds__(2 * BN) void gemm_kernel(GemmArgs g, float* __restrict__ y, int main_steps,
                                                      int total_steps, int steps_per_split, int atomic_out) {
    __shared__ __align__(16) uint8_t ring[Ring<BN>::BYTES];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave & 1, wn = wave >> 1;  // 2 x (BN/64) waves of 64x64
    int m_blk, n_blk;
    tile_of(blockIdx.x, (g.M + BM - 1) / BM, (g.N + BN - 1) / BN, &m_blk, &n_blk);
    g.n0 = n_blk * BN;
    g.m0 = m_blk * BM;
    const int s0 = blockIdx.z * steps_per_split;
    const int s1 = min(total_steps, s0 + steps_per_split);

    f16v acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    if constexpr (FMT == DQ_FMT_Q4_K) {
        run_steps<BN, B_Q4K>(g, ring, s0, min(s1, main_steps), main_steps, acc, wave, lane);
        min_steps(g, max(s0, main_steps) - main_steps, s1 - main_steps, acc, wave, lane);
    } else {
        run_steps<BN, B_Q6K>(g, ring, s0, s1, main_steps, acc, wave, lane);
    }

    // D layout of 32x32x16: lane l, register r -> n = l%32, m = (r/4)*8 + (l/32)*4 + r%4
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int n = g.n0 + wn * 64 + j * 32 + (lane & 31);
            if (n >= g.N) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = g.m0 + wm * 64 + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
                if (m < g.M) {
                    float* dst = y + (size_t)m * g.N + n;
                    const float v = acc[i][j][r] * g.inv[m];  // a power of two: exact
                    if (atomic_out) atomicAdd(dst, v);
                    else *dst = v;
                }
            }
        }
}

// Q4_K min plane for the min columns: mins[n][b] = fp16(-dmin*m_b) of row n,
// zero for b >= cols/32 (rows padded to ld_min columns).
__global__ __launch_bounds__(256) void min_plane_kernel(const uint8_t* __restrict__ w, DqLayout L, int N, int nblk,
                                                        int ld_min, _Float16* __restrict__ out) {
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;  // one lane per (row, super-block slot)
    const int per_row = ld_min / 8;
    if (t >= (size_t)N * per_row) return;
    const int n = (int)(t / per_row), s = (int)(t % per_row);
    _Float16 v[8];
    if (s * 8 < nblk) {
        const dq_u32x4 hd = dq_ld16(w + L.s_off + (size_t)n * L.s_row + 16 * (size_t)s);
        const float dmin = dq_h2f((uint16_t)(hd.x >> 16));
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = (_Float16)(-(dmin * (float)q4k_min(j, hd.y, hd.z, hd.w)));
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = (_Float16)0.0f;
    }
    *reinterpret_cast<h8*>(out + (size_t)n * ld_min + 8 * s) = *reinterpret_cast<const h8*>(v);
}

// Activation quantizer for the GEMM: per 32-block the reference integers and
// scale (core/i8gemm_impl.h:50-82), written as fp16(q*d*s) in K order `perm`
// (0 natural, 1 Q6_K item order), plus fp16(exact float block sum * s) in the
// min columns [cols, cols + n_min) (zero past cols/32), s the row's power-of-two
// range scale (row_scale_kernel) and inv[t] = 1/s. One lane per block.
__global__ __launch_bounds__(256) void quantize_f16_kernel(const float* __restrict__ x, int cols, int n_tok,
                                                           _Float16* __restrict__ out, int lda, int with_min,
                                                           int n_min, int perm, const float* __restrict__ rscale,
                                                           float* __restrict__ inv) {
    const int nb = cols / 32;
    const int gb = blockIdx.x * blockDim.x + threadIdx.x;
    const int stride = nb + (with_min ? n_min : 0);
    if (gb >= n_tok * stride) return;
    const int t = gb / stride, b = gb % stride;
    _Float16* o = out + (size_t)t * lda;
    const float sc = rscale[t];
    if (b == 0) inv[t] = 1.0f / sc;
    if (b >= nb) {  // min column b - nb
        const int mb = b - nb;
        if (mb >= nb) {
            o[cols + mb] = (_Float16)0.0f;
            return;
        }
        const float* p = x + (size_t)t * cols + 32 * mb;
        float fs = 0.0f;
        for (int i = 0; i < 32; ++i) fs += p[i];
        o[cols + mb] = (_Float16)(fs * sc);
        return;
    }
    const float* p = x + (size_t)t * cols + 32 * b;
    float v[32];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 f = reinterpret_cast<const float4*>(p)[i];
        v[4 * i] = f.x; v[4 * i + 1] = f.y; v[4 * i + 2] = f.z; v[4 * i + 3] = f.w;
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        const float a = fabsf(v[i]);
        amax = (amax < a) ? a : amax;
    }
    const float d = amax > 0.0f ? amax / 127.0f : 0.0f;
    const float id = d > 0.0f ? 1.0f / d : 0.0f;
    _Float16 h[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        int q = (int)rintf(v[i] * id);
        q = q > 127 ? 127 : (q < -127 ? -127 : q);
        h[i] = (_Float16)(((float)q * d) * sc);
    }
    if (perm == 0) {
        dq_u32x4* dst = reinterpret_cast<dq_u32x4*>(o + 32 * b);
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[i] = __builtin_bit_cast(dq_u32x4, *reinterpret_cast<const h8*>(&h[8 * i]));
    } else {
        // Q6_K item order: position pos in the 256-block -> column
        // s*256 + (2n+k)*64 + qq*16 + e, with pos = 128n + 32qq + 16k + e.
        const int s = b / 8, pos0 = 32 * (b % 8);
        const int n = pos0 / 128, qq = (pos0 % 128) / 32;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int col = s * 256 + (2 * n + k) * 64 + qq * 16;
            dq_u32x4* dst = reinterpret_cast<dq_u32x4*>(o + col);
            dst[0] = __builtin_bit_cast(dq_u32x4, *reinterpret_cast<const h8*>(&h[16 * k]));
            dst[1] = __builtin_bit_cast(dq_u32x4, *reinterpret_cast<const h8*>(&h[16 * k + 8]));
        }
    }
}

__global__ void zero_kernel(float* __restrict__ y, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = 0.0f;
}

int g_cus = 0;
int cus() {
    if (!g_cus) {
        int dev = 0, n = 0;
        g_cus = (hipGetDevice(&dev) == hipSuccess &&
                 hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
                    ? n
                    : 256;
    }
    return g_cus;
}

}  // namespace

// Workspace of the GEMM: the activation [n_tok][lda] fp16 (lda = cols + the
// min columns for Q4_K), the row scales s and 1/s [n_tok], then for Q4_K the
// min plane [rows][n_min] fp16.
static void gemm_act_shape(int fmt, size_t cols, int* lda, int* n_min) {
    *n_min = fmt == DQ_FMT_Q4_K ? (int)((cols / 32 + BK - 1) / BK * BK) : 0;
    *lda = (int)cols + *n_min;
}

static size_t act_bytes(int fmt, size_t cols, size_t n_tok) {
    int lda, n_min;
    gemm_act_shape(fmt, cols, &lda, &n_min);
    return dq_align256(n_tok * (size_t)lda * 2);
}

static size_t scale_off(int fmt, size_t cols, size_t n_tok) { return act_bytes(fmt, cols, n_tok); }
static size_t inv_off(int fmt, size_t cols, size_t n_tok) {
    return scale_off(fmt, cols, n_tok) + dq_align256(n_tok * 4);
}
static size_t min_off(int fmt, size_t cols, size_t n_tok) { return inv_off(fmt, cols, n_tok) + dq_align256(n_tok * 4); }

extern "C" int dq_gemm_workspace_bytes(int fmt, size_t rows, size_t cols, size_t n_tok, size_t* bytes) {
    if (!bytes) return DQ_ERR_INVALID_ARG;
    if (fmt != DQ_FMT_Q4_K && fmt != DQ_FMT_Q6_K) return DQ_ERR_NOT_SUPPORTED;
    if (cols % 256) return DQ_ERR_NOT_SUPPORTED;
    int lda, n_min;
    gemm_act_shape(fmt, cols, &lda, &n_min);
    *bytes = min_off(fmt, cols, n_tok) + dq_align256(rows * (size_t)n_min * 2);
    return DQ_OK;
}

extern "C" int dq_quantize_act_f16(int fmt, const float* d_x, size_t cols, size_t n_tok, void* d_out,
                                   void* stream) {
    if (fmt != DQ_FMT_Q4_K && fmt != DQ_FMT_Q6_K) return DQ_ERR_NOT_SUPPORTED;
    if (cols % 256 || cols > (1u << 24) || n_tok > (1u << 20)) return DQ_ERR_NOT_SUPPORTED;
    if (!d_x || !d_out) return DQ_ERR_INVALID_ARG;
    if (n_tok == 0) return DQ_OK;
    int lda, n_min;
    gemm_act_shape(fmt, cols, &lda, &n_min);
    const int nb = (int)cols / 32;
    const size_t lanes = n_tok * (size_t)(nb + n_min);
    uint8_t* base = (uint8_t*)d_out;
    float* sc = (float*)(base + scale_off(fmt, cols, n_tok));
    float* inv = (float*)(base + inv_off(fmt, cols, n_tok));
    row_scale_kernel<<<(unsigned)n_tok, 256, 0, (hipStream_t)stream>>>(d_x, (int)cols, sc);
    quantize_f16_kernel<<<(unsigned)((lanes + 255) / 256), 256, 0, (hipStream_t)stream>>>(
        d_x, (int)cols, (int)n_tok, (_Float16*)d_out, lda, fmt == DQ_FMT_Q4_K, n_min, fmt == DQ_FMT_Q6_K, sc, inv);
    return dq_launch_status();
}

template <int FMT, int BN>
static int launch_gemm(const GemmArgs& g, size_t rows, size_t n_tok, int main_steps, int total, float* d_y,
                       hipStream_t s) {
    const int mb = (int)((n_tok + BM - 1) / BM), nb = (int)((rows + BN - 1) / BN);
    // split K in two when the tile grid leaves CUs idle (two partials added
    // atomically into zeroed y: a+b == b+a, so the result is deterministic)
    const int split = ((size_t)mb * nb * 2 <= (size_t)cus() && total >= 8) ? 2 : 1;
    const int per = (total + split - 1) / split;
    if (split > 1) {
        const size_t n = rows * n_tok;
        zero_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(d_y, n);
    }
    const dim3 grid((unsigned)(mb * nb), 1, split);
    gemm_kernel<FMT, BN><<<grid, 2 * BN, 0, s>>>(g, d_y, main_steps, total, per, split > 1);
    return dq_launch_status();
}

// GEMM on the workspace written by dq_quantize_act_f16 (its first part); for
// Q4_K the min plane (second part of the workspace) is rebuilt from the
// weights on every call.
extern "C" int dq_gemm_f16act(int fmt, const void* d_w, size_t rows, size_t cols, const void* d_work,
                              size_t n_tok, float* d_y, void* stream) {
    DqLayout L;
    if (fmt != DQ_FMT_Q4_K && fmt != DQ_FMT_Q6_K) return DQ_ERR_NOT_SUPPORTED;
    if (!dq_layout(fmt, rows, cols, &L)) return DQ_ERR_NOT_SUPPORTED;
    if (rows > (1u << 30) || n_tok > (1u << 20)) return DQ_ERR_NOT_SUPPORTED;
    if (rows == 0 || n_tok == 0) return DQ_OK;
    if (!d_w || !d_work || !d_y) return DQ_ERR_INVALID_ARG;
    int lda, n_min;
    gemm_act_shape(fmt, cols, &lda, &n_min);
    hipStream_t s = (hipStream_t)stream;
    GemmArgs g{};
    g.w = (const uint8_t*)d_w;
    g.L = L;
    g.A = (const _Float16*)d_work;
    g.inv = (const float*)((const uint8_t*)d_work + inv_off(fmt, cols, n_tok));
    g.lda = lda;
    g.M = (int)n_tok;
    g.N = (int)rows;
    g.K = (int)cols;
    g.ld_min = n_min;
    if (fmt == DQ_FMT_Q4_K) {
        _Float16* mins = (_Float16*)((uint8_t*)d_work + min_off(fmt, cols, n_tok));
        const size_t lanes = rows * (size_t)(n_min / 8);
        min_plane_kernel<<<(unsigned)((lanes + 255) / 256), 256, 0, s>>>(g.w, L, (int)rows, (int)cols / 32, n_min,
                                                                         mins);
        g.mins = mins;
    }
    const int main_steps = (int)cols / BK;
    const int total = main_steps + n_min / BK;
    // wide tiles (less activation re-reading) when they still fill the CUs
    const size_t mb = (n_tok + BM - 1) / BM;
    const bool wide = mb * ((rows + 255) / 256) * 8 >= (size_t)cus() * 7;
    if (fmt == DQ_FMT_Q4_K)
        return wide ? launch_gemm<DQ_FMT_Q4_K, 256>(g, rows, n_tok, main_steps, total, d_y, s)
                    : launch_gemm<DQ_FMT_Q4_K, 128>(g, rows, n_tok, main_steps, total, d_y, s);
    return wide ? launch_gemm<DQ_FMT_Q6_K, 256>(g, rows, n_tok, main_steps, total, d_y, s)
                : launch_gemm<DQ_FMT_Q6_K, 128>(g, rows, n_tok, main_steps, total, d_y, s);
}

extern "C" int dq_gemm(int fmt, const void* d_w, size_t rows, size_t cols, const float* d_x, size_t n_tok,
                       float* d_y, void* d_work, size_t work_bytes, void* stream) {
    size_t need = 0;
    const int rc = dq_gemm_workspace_bytes(fmt, rows, cols, n_tok, &need);
    if (rc != DQ_OK) return rc;
    if (work_bytes < need || (need && !d_work)) return DQ_ERR_INVALID_ARG;
    const int r1 = dq_quantize_act_f16(fmt, d_x, cols, n_tok, d_work, stream);
    if (r1 != DQ_OK) return r1;
    return dq_gemm_f16act(fmt, d_w, rows, cols, d_work, n_tok, d_y, stream);
}
