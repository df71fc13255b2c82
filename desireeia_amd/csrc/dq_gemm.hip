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
// and the Q4_K min term is one extra 16-wide MFMA slice per super-block: the
// 8 block sums A = fp16(sx) (a token-contiguous plane) against B =
// fp16(-dmin*m_j) from the super-block header.
// Accumulation is fp32. The only difference from the reference is the fp16
// rounding of the two operands (2^-11 relative), which moves the result by
// ~3e-4 relative - inside the 4e-3 tolerance.
//
// Why fp16 and not int8 MFMA: the per-32 float rescale of every int32 block
// partial costs at least one non-packed fp32 VALU op per output per 32 K,
// which on CDNA4 (16 fp32 lanes/clk/SIMD vs ~1024 int8 MAC/clk/SIMD) caps the
// int8 path below half its peak; pre-scaled fp16 operands need no epilogue.
//
// Tiling: 128 (tokens) x BN (weight rows, 256 or 128) x 64 (K) per workgroup
// of BN/32 waves, each 64x64 (2x2 v_mfma_f32_32x32x16_f16 tiles). A 3-stage
// LDS ring filled by global_load_lds DMA holds per step the activation tile
// (XOR-swizzled 16-byte chunks: no bank conflicts on fragment reads), the
// super-block's block sums and the raw packed weight bytes; each wave turns
// its rows' bytes into fp16 fragments in registers. Q6_K: K is permuted to the
// packed item order (both operands, see dq_quantize_act_f16), so a 64-column
// K step is exactly one 64-weight item.
#include <cstdlib>
#include <utility>

#include "dq_common.h"
#include "dq_f16.h"

namespace {


constexpr int BK = 64;  // K per step

// Tile rows (tokens) of a workgroup: 2 waves along M, each WM 32-token blocks.
template <int WM>
constexpr int bm_of() { return 64 * WM; }

enum BKind { B_Q4K = 0, B_Q6K = 1, B_Q80 = 2, B_Q40 = 3 };

template <int FMT>
constexpr int kind_of() {
    return FMT == DQ_FMT_Q4_K ? B_Q4K : FMT == DQ_FMT_Q6_K ? B_Q6K : FMT == DQ_FMT_Q8_0 ? B_Q80 : B_Q40;
}

// ------------------------------------------------------------ LDS layout --
// Ring of NS stages, each holding one K step of both operands:
//   A: BM rows x 8 chunks of 16 bytes (fp16), chunk c of row r at slot
//      r*8 + (c ^ (r & 7)) - XOR swizzle: a wave's 16-byte fragment reads (32
//      rows, one logical chunk) hit all banks.
//   Q4_K only: the 8 min columns of the step's super-block (16 bytes per row).
//   B: the raw bytes of the weight tile, format specific:
//      Q4_K: P0[BN][16] P1[BN][16] H[BN][16]    (qs sub-planes, block header)
//      Q6_K: QA[BN][16] QB[BN][16] QH[BN][16] S[BN][4] D[BN][4] (fp16 in the low half)
//      Q8_0: P0..P3[BN][16] D[BN][4] (the item's two fp16 block scales)
//      Q4_0: P0 P1[BN][16] D[BN][4]
// Every stage is filled by global_load_lds (direct global -> LDS DMA, 16, 4 or
// 2 bytes per lane; lane i of a wave writes at base + i*16 for 16-byte loads and
// at base + i*4 for the dword and sub-dword forms). Three stages: two steps'
// DMAs in flight while one is computed.
template <int BN, int KIND, int WM>
struct Ring {
    static constexpr int BM = bm_of<WM>();
    static constexpr int NS = 3;
    static constexpr int A_BYTES = BM * BK * 2;
    static constexpr int MIN_BYTES = KIND == B_Q4K ? BM * 16 : 0;
    static constexpr int B_OFF = A_BYTES + MIN_BYTES;
    static constexpr int B_BYTES = BN * (KIND == B_Q80 ? 68 : 56);  // Q4_K 48, Q6_K 56, Q8_0 68, Q4_0 36 per row
    static constexpr int STAGE = B_OFF + B_BYTES;
    static constexpr int BYTES = NS * STAGE;
};

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
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

struct GemmArgs {
    const uint8_t* w;       // packed weights
    DqLayout L;
    const _Float16* A;      // activations [M][lda]
    const _Float16* minp;   // Q4_K: activation block sums, [K/256][M][8] (token-contiguous per super-block)
    const float* inv;       // per token: 1/s of its activation row
    int lda, M, N, K;
    int m0, n0;
    uint32_t magic;         // 0x54005400 (kept in a register: see run_steps)
};

// Issues the DMA of K step `st` (weights and activations) into ring stage
// `stage`. Every wave issues the same, compile-time number of load
// instructions (stage_loads()), so one s_waitcnt vmcnt covers a stage: blocks
// of 64 slots are dealt to the NW waves, and where a region has fewer blocks
// than waves several waves load the same block (identical bytes to the same
// LDS address).
template <int BN, int KIND, int WM>
constexpr int stage_loads() {
    constexpr int NW = BN / 32;
    // A, then Q4_K: sums, P0/P1, H; Q6_K: QA/QB, QH or S, D; Q8_0: two plane blocks, D; Q4_0: P0/P1, D
    return bm_of<WM>() * 8 / 64 / NW + (KIND == B_Q40 ? 2 : 3);
}

template <int BN, int KIND, int WM>
__device__ __forceinline__ void issue_stage(const GemmArgs& g, uint8_t* ring, int stage, int st, int wave,
                                            int lane) {
    constexpr int NW = BN / 32;      // waves per workgroup
    constexpr int HB = BN / 64;      // 64-slot blocks per [BN] region (= NW/2)
    using R = Ring<BN, KIND, WM>;
    constexpr int BM = R::BM;
    static_assert(BM / 64 <= NW, "one block-sum block per wave at most");
    uint8_t* base = ring + stage * R::STAGE;
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
    uint8_t* bb = base + R::B_OFF;
    if constexpr (KIND == B_Q4K) {
        {   // block sums of super-block st/4 (16 contiguous bytes per token):
            // BM/64 blocks of 64 rows, block wave % (BM/64)
            const int blk = wave % (BM / 64), m = min(g.m0 + blk * 64 + lane, g.M - 1);
            lds_dma<16>(g.minp + ((size_t)(st >> 2) * g.M + m) * 8, base + R::A_BYTES + blk * 64 * 16);
        }
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
    } else {  // Q8_0 (4 sub-planes) and Q4_0 (2): one item per row and step
        constexpr int NP = KIND == B_Q80 ? 4 : 2;
#pragma unroll
        for (int q = 0; q < NP / 2; ++q) {  // NP * HB plane blocks = NP/2 per wave
            const int blk = wave + q * NW;
            const int region = blk / HB, n = (blk % HB) * 64 + lane;
            const size_t r = (size_t)min(g.n0 + n, g.N - 1);
            lds_dma<16>(g.w + g.L.q_off + (size_t)region * g.L.p_stride + r * g.L.q_row + 16 * (size_t)st,
                        bb + blk * 64 * 16);
        }
        {   // D: the item's two fp16 scales, HB blocks of dwords (waves w and w + HB: block w % HB)
            const int blk = wave % HB, n = blk * 64 + lane;
            const size_t r = (size_t)min(g.n0 + n, g.N - 1);
            lds_dma<4>(g.w + g.L.d_off + r * g.L.d_row + 4 * (size_t)st, bb + NP * BN * 16 + blk * 64 * 4);
        }
    }
}

__device__ __forceinline__ const h8& lds_h8(const uint8_t* p) { return *reinterpret_cast<const h8*>(p); }

// Raw weight bytes of one ring stage that this lane's B fragments need: for
// each of its two 32-row blocks j, lane half h's 8 bytes of the two quant
// sub-planes (Q4_K: P0/P1; Q6_K: QA/QB plus QH) and the row's scales.
struct BRaw {
    dq_u32x2 q0[2], q1[2], q2[2], q3[2];  // Q4_K: P0, P1; Q6_K: QA, QB, QH; Q8_0: P0..P3; Q4_0: P0, P1
    dq_u32x4 hd[2];  // Q4_K: super-block header; Q6_K: .x = 4 int8 scales, .y = d (low half); Q8_0/Q4_0: .x = 2 d
};

template <int BN, int KIND>
__device__ __forceinline__ void b_raw(const uint8_t* bb, int wn, int lane, BRaw& r) {
    const int h = lane >> 5;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int n = wn * 64 + j * 32 + (lane & 31);
        r.q0[j] = *reinterpret_cast<const dq_u32x2*>(bb + n * 16 + 8 * h);
        r.q1[j] = *reinterpret_cast<const dq_u32x2*>(bb + BN * 16 + n * 16 + 8 * h);
        if constexpr (KIND == B_Q4K) {
            r.hd[j] = *reinterpret_cast<const dq_u32x4*>(bb + 2 * BN * 16 + n * 16);
        } else if constexpr (KIND == B_Q80) {
            r.q2[j] = *reinterpret_cast<const dq_u32x2*>(bb + 2 * BN * 16 + n * 16 + 8 * h);
            r.q3[j] = *reinterpret_cast<const dq_u32x2*>(bb + 3 * BN * 16 + n * 16 + 8 * h);
            r.hd[j].x = *reinterpret_cast<const uint32_t*>(bb + 4 * BN * 16 + n * 4);
        } else if constexpr (KIND == B_Q40) {
            r.hd[j].x = *reinterpret_cast<const uint32_t*>(bb + 2 * BN * 16 + n * 4);
        } else {
            r.q2[j] = *reinterpret_cast<const dq_u32x2*>(bb + 2 * BN * 16 + n * 16 + 8 * h);
            r.hd[j].x = *reinterpret_cast<const uint32_t*>(bb + 3 * BN * 16 + n * 4);
            r.hd[j].y = *reinterpret_cast<const uint32_t*>(bb + 3 * BN * 16 + BN * 4 + n * 4);
        }
    }
}

// B fragments of a step of phase G (= st % 4, the item of the super-block)
// from the raw bytes, one 16-wide K slice KK at a time (so a slice can be
// built while the previous slice's MFMAs run): bf[j], j = 32-row n block.
// Lane l feeds row n = wn*64 + j*32 + l%32 with the 8 K values KK*16 +
// 8*(l/32) .. +7. Rows past N hold the clamped last row's bytes (finite
// values whose outputs are never stored). b_scales holds the fp16 scale pair
// of every (j, KK): Q4_K a = d*sc of sub-block 2G (KK 0, 1: low nibbles) or
// 2G+1 (KK 2, 3: high nibbles); Q6_K a = d*sc of the KK-th 16-block.
struct BScale {
    h2 s[2][4];  // Q6_K: scale pair per (j, KK); Q4_K: low-nibble a, high-nibble a, -64a of each
    uint32_t magic;
};

template <int KIND>
__device__ __forceinline__ void b_scales(const BRaw& r, int G, BScale& S) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        if constexpr (KIND == B_Q4K) {
            const dq_u32x4 hd = r.hd[j];
            const float d = dq_h2f((uint16_t)(hd.x & 0xFFFF));
            const _Float16 a0 = (_Float16)(d * (float)q4k_scale(2 * G, hd.y, hd.z, hd.w));
            const _Float16 a1 = (_Float16)(d * (float)q4k_scale(2 * G + 1, hd.y, hd.z, hd.w));
            S.s[j][0] = h2{a0, a0};
            S.s[j][1] = h2{a1, a1};
            // -64a is exact while |a| < 1024 (64*a stays below the fp16 maximum)
            S.s[j][2] = h2{(_Float16)(-64.0f) * a0, (_Float16)(-64.0f) * a0};
            S.s[j][3] = h2{(_Float16)(-64.0f) * a1, (_Float16)(-64.0f) * a1};
        } else if constexpr (KIND == B_Q80 || KIND == B_Q40) {
            // K slices 0, 1: the item's first block (scale d0), 2, 3: the second
            const uint32_t dd = r.hd[j].x;
            const _Float16 d0 = __builtin_bit_cast(_Float16, (uint16_t)(dd & 0xFFFF));
            const _Float16 d1 = __builtin_bit_cast(_Float16, (uint16_t)(dd >> 16));
            S.s[j][0] = S.s[j][1] = h2{d0, d0};
            S.s[j][2] = S.s[j][3] = h2{d1, d1};
        } else {
            const uint32_t sc = r.hd[j].x;
            const float d = dq_h2f((uint16_t)(r.hd[j].y & 0xFFFF));
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                const _Float16 a = (_Float16)(d * (float)(int8_t)((sc >> (8 * kk)) & 0xFF));
                S.s[j][kk] = h2{a, a};
            }
        }
    }
}

template <int KIND, int KK>
__device__ __forceinline__ void b_frag(const BRaw& r, const BScale& S, h8 (&bf)[2]) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        uint32_t t[4];
        if constexpr (KIND == B_Q4K) {
            // KK 0, 1: P0 bytes 8h..8h+3, 8h+4..8h+7; KK 2, 3: the same of P1.
            // From the dword's bytes B0..B3, a nibble ORed into mantissa bits
            // 7:4 under the exponent of 64 (0x5400) is the fp16 64 + q exactly,
            // two per v_and_or; fma(64 + q, a, -64a) = q*a rounded once (as
            // (q)*a would be). Fragment order (the activation tile is permuted
            // to match, dq_quantize_act_f16): lo B0, lo B2, hi B0, hi B2, lo B1,
            // lo B3, hi B1, hi B3; lo = sub-block 2G (scale a0), hi = 2G+1 (a1).
            const dq_u32x2 src = KK < 2 ? r.q0[j] : r.q1[j];
            const uint32_t w = (KK & 1) ? src.y : src.x;
            // the exponent pattern comes from a register (S.magic): with both
            // operands literal the compiler splits each v_and_or into two
            const uint32_t e0 = ((w << 4) & 0x00F000F0u) | S.magic;
            const uint32_t e1 = (w & 0x00F000F0u) | S.magic;
            const uint32_t e2 = ((w >> 4) & 0x00F000F0u) | S.magic;
            const uint32_t e3 = ((w >> 8) & 0x00F000F0u) | S.magic;
            t[0] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(h2, e0), S.s[j][0], S.s[j][2]));
            t[1] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(h2, e1), S.s[j][1], S.s[j][3]));
            t[2] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(h2, e2), S.s[j][0], S.s[j][2]));
            t[3] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(h2, e3), S.s[j][1], S.s[j][3]));
        } else if constexpr (KIND == B_Q80) {
            // slice KK = sub-plane KK, bytes 8h..8h+7: q ^ 0x80 = q + 128 under
            // the exponent of 1024, minus 1152 = q exactly, times d (one rounding)
            const h2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
            const dq_u32x2 src = KK == 0 ? r.q0[j] : KK == 1 ? r.q1[j] : KK == 2 ? r.q2[j] : r.q3[j];
            bytes_to_h2(src.x ^ 0x80808080u, bias, S.s[j][KK], &t[0]);
            bytes_to_h2(src.y ^ 0x80808080u, bias, S.s[j][KK], &t[2]);
        } else if constexpr (KIND == B_Q40) {
            // slices 0, 1: sub-plane 0 (block 2i) low, high nibbles; 2, 3: sub-plane 1;
            // the nibble q under the exponent of 1024, minus 1032 = q - 8, times d
            const h2 bias = {(_Float16)1032.0f, (_Float16)1032.0f};
            const dq_u32x2 src = KK < 2 ? r.q0[j] : r.q1[j];
            const int sh = (KK & 1) ? 4 : 0;
            bytes_to_h2((src.x >> sh) & 0x0F0F0F0Fu, bias, S.s[j][KK], &t[0]);
            bytes_to_h2((src.y >> sh) & 0x0F0F0F0Fu, bias, S.s[j][KK], &t[2]);
        } else {
            const h2 bias = {(_Float16)1056.0f, (_Float16)1056.0f};  // 1024 + 32
            const dq_u32x2 lo = (KK & 1) ? r.q1[j] : r.q0[j];
#pragma unroll
            for (int wd = 0; wd < 2; ++wd) {
                const uint32_t l4 = KK < 2 ? (lo[wd] & 0x0F0F0F0Fu) : ((lo[wd] >> 4) & 0x0F0F0F0Fu);
                const uint32_t v6 = l4 | (((r.q2[j][wd] >> (2 * KK)) & 0x03030303u) << 4);
                bytes_to_h2(v6, bias, S.s[j][KK], &t[2 * wd]);
            }
        }
        bf[j] = __builtin_bit_cast(h8, dq_u32x4{t[0], t[1], t[2], t[3]});
    }
}

// A fragments of K slice kk for the wave's WM 32-token blocks (XOR-swizzled
// 16-byte chunks of the stage's activation tile).
template <int WM>
__device__ __forceinline__ void a_frags(const uint8_t* base, int wm, int kk, int lane, h8 (&af)[WM]) {
#pragma unroll
    for (int i = 0; i < WM; ++i) {
        const int r = wm * 32 * WM + i * 32 + (lane & 31);
        af[i] = lds_h8(base + (r * 8 + ((2 * kk + (lane >> 5)) ^ (r & 7))) * 16);
    }
}

// One K step st (phase G = st % 4, the item of the super-block) in ring
// stage `stage`: wait until the stage has landed (NS-2 later stages may
// still be in flight), barrier (every wave's DMAs visible, step st-1
// retired), DMA of step st+NS-1 into the stage of st-1 (past the end: the
// last step again, so every wave issues the same count per stage), then the
// weight fragments (LDS bytes -> fp16 in registers) and the MFMAs; at the
// last item of a super-block (Q4_K) also its min term.
template <int BN, int KIND, int WM>
__device__ __forceinline__ void gemm_step(const GemmArgs& g, uint8_t* ring, int st, int stage, int s1,
                                          f16v (&acc)[WM][2], int wave, int lane, uint32_t magic) {
    const int G = st & 3;
    using R = Ring<BN, KIND, WM>;
    constexpr int NS = R::NS;
    constexpr int PER = stage_loads<BN, KIND, WM>();
    const int wm = wave & 1, wn = wave >> 1;
    wait_vm<(NS - 2) * PER>();
    dq_lds_barrier();
    issue_stage<BN, KIND, WM>(g, ring, stage == 0 ? NS - 1 : stage - 1, min(st + NS - 1, s1 - 1), wave, lane);
    const uint8_t* base = ring + stage * R::STAGE;
    BRaw raw;
    b_raw<BN, KIND>(base + R::B_OFF, wn, lane, raw);
    BScale S;
    S.magic = magic;
    b_scales<KIND>(raw, G, S);
    // The four K slices in order, slice kk+1's activation fragments (LDS)
    // and weight fragments (VALU) written after slice kk's MFMAs so the
    // scheduler can overlap them.
    h8 af[4][WM], bf[4][2];
    a_frags<WM>(base, wm, 0, lane, af[0]);
    b_frag<KIND, 0>(raw, S, bf[0]);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
        if (kk == 0) { a_frags<WM>(base, wm, 1, lane, af[1]); b_frag<KIND, 1>(raw, S, bf[1]); }
        if (kk == 1) { a_frags<WM>(base, wm, 2, lane, af[2]); b_frag<KIND, 2>(raw, S, bf[2]); }
        if (kk == 2) { a_frags<WM>(base, wm, 3, lane, af[3]); b_frag<KIND, 3>(raw, S, bf[3]); }
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[kk][i], bf[kk][j], acc[i][j], 0, 0, 0);
    }
    h8 bm[2];
    if (KIND == B_Q4K && G == 3) bm[0] = q4k_neg_mins(raw.hd[0], true), bm[1] = q4k_neg_mins(raw.hd[1], true);
    if (KIND == B_Q4K && G == 3) {  // the super-block's min term
        const h8 zero = {};
        h8 am[WM];
#pragma unroll
        for (int i = 0; i < WM; ++i) {
            const h8 v = lds_h8(base + R::A_BYTES + (wm * 32 * WM + i * 32 + (lane & 31)) * 16);
            am[i] = (lane >> 5) == 0 ? v : zero;
        }
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(am[i], bm[j], acc[i][j], 0, 0, 0);
    }
}

// K steps [s0, s1), s0 and s1 multiples of 4 (whole super-blocks, so every
// super-block's min term falls in one split): NS-1 stages in flight before
// the first step, then one step at a time.
template <int BN, int KIND, int WM>
__device__ __forceinline__ void run_steps(const GemmArgs& g, uint8_t* ring, int s0, int s1, f16v (&acc)[WM][2],
                                          int wave, int lane) {
    using R = Ring<BN, KIND, WM>;
    constexpr int NS = R::NS;
    if (s0 >= s1) return;
#pragma unroll
    for (int p = 0; p < NS - 1; ++p) issue_stage<BN, KIND, WM>(g, ring, p, min(s0 + p, s1 - 1), wave, lane);
    // the fp16 exponent pattern of the Q4_K nibble conversion in a VGPR (an
    // identity DPP move the compiler cannot fold), so each nibble pair is one
    // v_and_or_b32 (literal mask, register pattern) instead of an and + or
    const uint32_t magic =
        (uint32_t)__builtin_amdgcn_update_dpp((int)g.magic, (int)g.magic, 0xE4, 0xF, 0xF, false);
    int stage = 0;
    for (int st = s0; st < s1; ++st) {
        gemm_step<BN, KIND, WM>(g, ring, st, stage, s1, acc, wave, lane, magic);
        stage = stage + 1 == NS ? 0 : stage + 1;
    }
    wait_vm<0>();  // drain the DMAs issued past the end
    dq_lds_barrier();
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

// Register budget of two waves per SIMD (256 per lane): an 8-wave (BN 256)
// workgroup per CU, or one or two 4-wave (BN 128) ones. Wave (wm, wn) owns
// tokens wm*32*WM .. +32*WM and rows wn*64 .. +64 of the tile: WM 32x32
// blocks by 2, so each dequantized weight fragment feeds WM MFMAs.
template <int FMT, int BN, int WM>
__global__ __launch_bounds__(2 * BN) __attribute__((amdgpu_waves_per_eu(2, 2))) void gemm_kernel(
    GemmArgs g, float* __restrict__ y, int steps, int steps_per_split, int atomic_out) {
    constexpr int KIND = kind_of<FMT>();
    constexpr int BM = bm_of<WM>();
    __shared__ __align__(16) uint8_t ring[Ring<BN, KIND, WM>::BYTES];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave & 1, wn = wave >> 1;  // 2 x (BN/64) waves of (32*WM) x 64
    int m_blk, n_blk;
    tile_of(blockIdx.x, (g.M + BM - 1) / BM, (g.N + BN - 1) / BN, &m_blk, &n_blk);
    g.n0 = n_blk * BN;
    g.m0 = m_blk * BM;
    const int s0 = blockIdx.z * steps_per_split;
    const int s1 = min(steps, s0 + steps_per_split);

    f16v acc[WM][2];
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    run_steps<BN, KIND, WM>(g, ring, s0, s1, acc, wave, lane);

    // D layout of 32x32x16: lane l, register r -> n = l%32, m = (r/4)*8 + (l/32)*4 + r%4.
    // The row factors 1/s of a 32-token block are loaded together before its
    // stores (unconditional loads of clamped rows; a load inside the store's
    // branch would be waited for one at a time).
#pragma unroll
    for (int i = 0; i < WM; ++i) {
        const int mb0 = g.m0 + wm * 32 * WM + i * 32 + (lane >> 5) * 4;
        float inv[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) inv[r] = g.inv[min(mb0 + (r >> 2) * 8 + (r & 3), g.M - 1)];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int n = g.n0 + wn * 64 + j * 32 + (lane & 31);
            if (n >= g.N) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = mb0 + (r >> 2) * 8 + (r & 3);
                if (m < g.M) {
                    float* dst = y + (size_t)m * g.N + n;
                    const float v = acc[i][j][r] * inv[r];  // a power of two: exact
                    if (atomic_out) atomicAdd(dst, v);
                    else *dst = v;
                }
            }
        }
    }
}

// Activation quantizer for the GEMM: per 32-block the reference integers and
// scale (core/i8gemm_impl.h:50-82), written as fp16(q*d*s) in K order `perm`
// (0 natural, 1 Q6_K item order); with a min plane (Q4_K), fp16(exact float
// block sum * s) of block b at minp[b/8][t][b%8]; s the row's power-of-two
// range scale. One block (or one block sum) per call; the row kernel below
// runs them for its token.
__device__ __forceinline__ void quantize_f16_block(const float* __restrict__ x, int cols, int n_tok,
                                                   _Float16* __restrict__ out, int lda, _Float16* __restrict__ minp,
                                                   int perm, int t, int b, float sc) {
    const int nb = cols / 32;
    _Float16* o = out + (size_t)t * lda;
    if (b >= nb) {  // block sum of block b - nb
        const int mb = b - nb;
        const float* p = x + (size_t)t * cols + 32 * mb;
        float fs = 0.0f;
        for (int i = 0; i < 32; ++i) fs += p[i];
        minp[((size_t)(mb / 8) * n_tok + t) * 8 + (mb % 8)] = (_Float16)(fs * sc);
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
    } else if (perm == 2) {
        // Q4_K fragment order (gemm b_frag): block b is half hi = b % 2 (the
        // high nibbles) of item g = (b % 8) / 2; its element e is byte j = e of
        // the item's 32 qs bytes, in sub-plane j / 16, lane half (j % 16) / 8,
        // slice KK = 2 * plane + (j % 8) / 4, fragment slot f = 4 * (bo & 1) +
        // (bo >> 1) + 2 * hi with bo = j % 4; column 16 KK + 8 half + f.
        const int hi = b & 1;
        _Float16* item = o + 64 * (size_t)(b / 2);
#pragma unroll
        for (int e = 0; e < 32; ++e) {
            const int pl = e / 16, hf = (e % 16) / 8, kk = 2 * pl + (e % 8) / 4, bo = e % 4;
            item[16 * kk + 8 * hf + 4 * (bo & 1) + (bo >> 1) + 2 * hi] = h[e];
        }
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

// One workgroup per token row: the row's power-of-two range scale (as
// row_scale_kernel) and then every block of the row (quantize_f16_block);
// inv[t] = 1/s.
__global__ __launch_bounds__(256) void quantize_f16_rows_kernel(const float* __restrict__ x, int cols, int n_tok,
                                                                _Float16* __restrict__ out, int lda,
                                                                _Float16* __restrict__ minp, int perm,
                                                                float* __restrict__ rscale, float* __restrict__ inv) {
    __shared__ float wmax[4];
    const int t = blockIdx.x;
    const float* row = x + (size_t)t * cols;
    float m = 0.0f;
    for (int c = threadIdx.x * 4; c < cols; c += 1024) {
        const float4 f = *reinterpret_cast<const float4*>(row + c);
        m = fmaxf(m, fmaxf(fmaxf(fabsf(f.x), fabsf(f.y)), fmaxf(fabsf(f.z), fabsf(f.w))));
    }
    m = dq_wave_max(m);
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = m;
    __syncthreads();
    const float sc = row_scale_of(fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3])));
    if (threadIdx.x == 0) {
        rscale[t] = sc;
        inv[t] = 1.0f / sc;
    }
    const int nb = cols / 32;
    const int stride = minp ? 2 * nb : nb;
    for (int b = threadIdx.x; b < stride; b += 256) quantize_f16_block(x, cols, n_tok, out, lda, minp, perm, t, b, sc);
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

// Workspace of the GEMM: the activation [n_tok][cols] fp16, for Q4_K the
// block sums [cols/256][n_tok][8] fp16, then the row scales s and 1/s [n_tok].
// Row stride of the fp16 activation: cols plus 64 halves (128 bytes), so the
// rows a K step reads (same column, consecutive tokens) fall on different L2
// channels; at a power-of-two stride they would all queue on one channel.
static size_t act_lda(size_t cols) { return cols + 64; }
static size_t act_bytes(size_t cols, size_t n_tok) { return dq_align256(n_tok * act_lda(cols) * 2); }
static size_t min_bytes(int fmt, size_t cols, size_t n_tok) {
    return fmt == DQ_FMT_Q4_K ? dq_align256(n_tok * (cols / 32) * 2) : 0;
}
static size_t min_off(size_t cols, size_t n_tok) { return act_bytes(cols, n_tok); }
static size_t scale_off(int fmt, size_t cols, size_t n_tok) {
    return min_off(cols, n_tok) + min_bytes(fmt, cols, n_tok);
}
static size_t inv_off(int fmt, size_t cols, size_t n_tok) {
    return scale_off(fmt, cols, n_tok) + dq_align256(n_tok * 4);
}

extern "C" int dq_gemm_workspace_bytes(int fmt, size_t rows, size_t cols, size_t n_tok, size_t* bytes) {
    (void)rows;
    if (!bytes) return DQ_ERR_INVALID_ARG;
    if (fmt != DQ_FMT_Q4_K && fmt != DQ_FMT_Q6_K && fmt != DQ_FMT_Q8_0 && fmt != DQ_FMT_Q4_0)
        return DQ_ERR_NOT_SUPPORTED;
    if (cols % 256) return DQ_ERR_NOT_SUPPORTED;
    *bytes = inv_off(fmt, cols, n_tok) + dq_align256(n_tok * 4);
    return DQ_OK;
}

extern "C" int dq_quantize_act_f16(int fmt, const float* d_x, size_t cols, size_t n_tok, void* d_out,
                                   void* stream) {
    if (fmt != DQ_FMT_Q4_K && fmt != DQ_FMT_Q6_K && fmt != DQ_FMT_Q8_0 && fmt != DQ_FMT_Q4_0)
        return DQ_ERR_NOT_SUPPORTED;
    if (cols % 256 || cols > (1u << 24) || n_tok > (1u << 20)) return DQ_ERR_NOT_SUPPORTED;
    if (!d_x || !d_out) return DQ_ERR_INVALID_ARG;
    if (n_tok == 0) return DQ_OK;
    const int nb = (int)cols / 32;
    const bool with_min = fmt == DQ_FMT_Q4_K;
    const size_t lanes = n_tok * (size_t)(with_min ? 2 * nb : nb);
    uint8_t* base = (uint8_t*)d_out;
    _Float16* minp = with_min ? (_Float16*)(base + min_off(cols, n_tok)) : nullptr;
    float* sc = (float*)(base + scale_off(fmt, cols, n_tok));
    float* inv = (float*)(base + inv_off(fmt, cols, n_tok));
    (void)lanes;
    quantize_f16_rows_kernel<<<(unsigned)n_tok, 256, 0, (hipStream_t)stream>>>(
        d_x, (int)cols, (int)n_tok, (_Float16*)d_out, (int)act_lda(cols), minp,
        fmt == DQ_FMT_Q6_K ? 1 : (fmt == DQ_FMT_Q4_K ? 2 : 0), sc, inv);
    return dq_launch_status();
}

template <int FMT, int BN, int WM>
static int launch_gemm(const GemmArgs& g, size_t rows, size_t n_tok, int steps, int split, float* d_y, hipStream_t s) {
    constexpr int BM = bm_of<WM>();
    const int mb = (int)((n_tok + BM - 1) / BM), nb = (int)((rows + BN - 1) / BN);
    const int per = (steps / 4 + split - 1) / split * 4;  // whole super-blocks per split
    if (split > 1) {
        const size_t n = rows * n_tok;
        zero_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(d_y, n);
    }
    const dim3 grid((unsigned)(mb * nb), 1, split);
    gemm_kernel<FMT, BN, WM><<<grid, 2 * BN, 0, s>>>(g, d_y, steps, per, split > 1);
    return dq_launch_status();
}

// Tile shape and K split. The K split is 2 when the tile grid leaves at
// least half the CUs idle (two partials added atomically into zeroed y:
// a+b == b+a, so the result is deterministic). Default: 128x256 tiles (8
// waves of 64x64) when their grid, split included, covers 7/8 of the CUs,
// else 128x128. The 256x256 tile (waves of 128x64, each weight fragment
// feeding 4 MFMAs) is selectable with DQ_GEMM_WM=4 for tuning; it measured
// slower at M = 512 (fewer, longer steps; the step is bound by its VALU and
// LDS issue, not by the MFMA count).
struct GemmPlan {
    int bn, wm, split;
};
static size_t bm_of_rt(int wm) { return (size_t)64 * wm; }
static GemmPlan plan_gemm(size_t rows, size_t n_tok, int steps) {
    const size_t c = (size_t)cus();
    auto make = [&](int bn, int wm) {
        const size_t tiles = ((n_tok + bm_of_rt(wm) - 1) / bm_of_rt(wm)) * ((rows + bn - 1) / bn);
        const int split = (tiles * 2 <= c && steps >= 8) ? 2 : 1;
        return std::pair<GemmPlan, size_t>{GemmPlan{bn, wm, split}, tiles * split};
    };
    const char* fw = getenv("DQ_GEMM_WM");  // tuning overrides: tile shape and K split
    const char* fs = getenv("DQ_GEMM_SPLIT");
    GemmPlan pl;
    const auto wide = make(256, 2);
    if (fw) pl = atoi(fw) == 4 ? make(256, 4).first : atoi(fw) == 2 ? wide.first : make(128, 2).first;
    else if (wide.second * 8 >= c * 7) pl = wide.first;
    else pl = make(128, 2).first;
    if (fs && (atoi(fs) == 1 || atoi(fs) == 2)) pl.split = atoi(fs);
    return pl;
}

// GEMM on the workspace written by dq_quantize_act_f16.
extern "C" int dq_gemm_f16act(int fmt, const void* d_w, size_t rows, size_t cols, const void* d_work,
                              size_t n_tok, float* d_y, void* stream) {
    DqLayout L;
    if (fmt != DQ_FMT_Q4_K && fmt != DQ_FMT_Q6_K && fmt != DQ_FMT_Q8_0 && fmt != DQ_FMT_Q4_0)
        return DQ_ERR_NOT_SUPPORTED;
    if (!dq_layout(fmt, rows, cols, &L) || cols % 256) return DQ_ERR_NOT_SUPPORTED;
    if (rows > (1u << 30) || n_tok > (1u << 20)) return DQ_ERR_NOT_SUPPORTED;
    if (rows == 0 || n_tok == 0) return DQ_OK;
    if (!d_w || !d_work || !d_y) return DQ_ERR_INVALID_ARG;
    hipStream_t s = (hipStream_t)stream;
    GemmArgs g{};
    g.w = (const uint8_t*)d_w;
    g.L = L;
    g.A = (const _Float16*)d_work;
    g.minp = (const _Float16*)((const uint8_t*)d_work + min_off(cols, n_tok));
    g.inv = (const float*)((const uint8_t*)d_work + inv_off(fmt, cols, n_tok));
    g.lda = (int)act_lda(cols);
    g.magic = 0x54005400u;
    g.M = (int)n_tok;
    g.N = (int)rows;
    g.K = (int)cols;
    const int steps = (int)cols / BK;
    const GemmPlan pl = plan_gemm(rows, n_tok, steps);
    if (fmt == DQ_FMT_Q4_K) {
        if (pl.wm == 4) return launch_gemm<DQ_FMT_Q4_K, 256, 4>(g, rows, n_tok, steps, pl.split, d_y, s);
        if (pl.bn == 256) return launch_gemm<DQ_FMT_Q4_K, 256, 2>(g, rows, n_tok, steps, pl.split, d_y, s);
        return launch_gemm<DQ_FMT_Q4_K, 128, 2>(g, rows, n_tok, steps, pl.split, d_y, s);
    }
    if (fmt == DQ_FMT_Q8_0) {
        if (pl.bn == 256) return launch_gemm<DQ_FMT_Q8_0, 256, 2>(g, rows, n_tok, steps, pl.split, d_y, s);
        return launch_gemm<DQ_FMT_Q8_0, 128, 2>(g, rows, n_tok, steps, pl.split, d_y, s);
    }
    if (fmt == DQ_FMT_Q4_0) {
        if (pl.bn == 256) return launch_gemm<DQ_FMT_Q4_0, 256, 2>(g, rows, n_tok, steps, pl.split, d_y, s);
        return launch_gemm<DQ_FMT_Q4_0, 128, 2>(g, rows, n_tok, steps, pl.split, d_y, s);
    }
    if (pl.wm == 4) return launch_gemm<DQ_FMT_Q6_K, 256, 4>(g, rows, n_tok, steps, pl.split, d_y, s);
    if (pl.bn == 256) return launch_gemm<DQ_FMT_Q6_K, 256, 2>(g, rows, n_tok, steps, pl.split, d_y, s);
    return launch_gemm<DQ_FMT_Q6_K, 128, 2>(g, rows, n_tok, steps, pl.split, d_y, s);
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
