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
// Tiling: a workgroup of 4 waves computes 128 tokens x 64*NWN weight rows;
// the waves are NWN (64-row blocks) x KSW (K groups). Wave (wn, kg) owns all
// 128 tokens of its 64 rows over the kg-th share of the workgroup's K steps:
// 4 x 2 v_mfma_f32_32x32x16_f16 tiles, so each weight fragment it turns into
// fp16 feeds 4 MFMAs, and no other wave converts the same bytes. Each K group
// has LDS rings filled by global_load_lds DMA: NS (2 or 3) activation stages
// of one K step (64 columns; XOR-swizzled 16-byte chunks, no bank conflicts
// on fragment reads) and NB super-stages of SB packed weight items of the
// group's rows (with the super-block header and, for Q4_K, the block sums
// of the min term; see Ring). KSW = 2 partials are
// added through LDS at the end in a fixed order. Q6_K: K is permuted to the
// packed item order (both operands, see dq_quantize_act_f16), so a 64-column
// K step is exactly one 64-weight item.
#include <cstdlib>
#include <utility>

#include "dq_common.h"
#include "dq_f16.h"

namespace {


constexpr int BK = 64;  // K per step

constexpr int BM = 128;  // tokens per workgroup (and per wave)

enum BKind { B_Q4K = 0, B_Q6K = 1, B_Q80 = 2, B_Q40 = 3 };

template <int FMT>
constexpr int kind_of() {
    return FMT == DQ_FMT_Q4_K ? B_Q4K : FMT == DQ_FMT_Q6_K ? B_Q6K : FMT == DQ_FMT_Q8_0 ? B_Q80 : B_Q40;
}

// ------------------------------------------------------------ LDS layout --
// Per K group: an A ring of NS stages, one K step each - the activation tile
// as fp16, BM rows x 8 chunks of 16 bytes, chunk c of row r at slot
// r*8 + (c ^ aswz(r)) - and a B ring of NB super-stages, each
// holding SB consecutive weight items (K steps) of the group's BN rows:
//   Q4_K (SB 4): P0[BN][4][16] P1[BN][4][16] H[BN][16] MIN[BM][16]
//   Q4_0 (SB 4): P0[BN][4][16] P1[BN][4][16] D[4][BN][4]
//   Q6_K (SB 2): QA[BN][2][16] QB[BN][2][16] QH[BN][2][16] S[2][BN][4] D[BN][4]
//   Q8_0 (SB 2): P0..P3[BN][2][16] D[2][BN][4]
// (H: the super-block header; MIN: the super-block's 8 activation block sums
// per token; S: an item's four int8 scales; D: fp16 scales, Q6_K's in the low
// half of a dword slot.) Item t of row n of a [BN][SB][16] plane sits in
// chunk slot t ^ swz(n). The swizzles make the 16-byte fragment reads
// conflict-free: gfx950's LDS serves a 16-byte read for 16 lanes per cycle
// over 64 banks (a 256-byte window), and the 16 lanes of a cycle are four
// lane quads q = lane / 4 of one half-wave with the same parity of q % 8's
// three bits: lanes 0-3, 12-15, 20-23, 24-27 together, then 4-7, 8-11,
// 16-19, 28-31, and the same for lanes 32-63 (dq_lds_read_probe's quad-pair
// patterns under SQ_LDS_BANK_CONFLICT). A fragment read's lane l takes row
// l % 32, so the rows of a cycle must fall on distinct 16-byte slots of the
// window: A (128-byte rows) the pairs (row parity, slot), SB 4 (64-byte rows)
// the pairs (row % 4, slot) - swz = (row / 4) % 4 is distinct over the four
// quads of either parity class - and SB 2 (32-byte rows) the pairs
// (row % 8, slot). Every region is filled by global_load_lds (direct global -> LDS DMA: lane i of a
// wave writes base + 16i, or base + 4i for the dword and sub-dword forms);
// the plane DMA reads a row's SB*16 contiguous bytes with SB consecutive
// lanes (whole cache-line pieces, not one 16-byte item of a different row
// per lane).
template <int KIND>
constexpr int sb_of() { return (KIND == B_Q6K || KIND == B_Q80) ? 2 : 4; }
template <int KIND>
constexpr int planes_of() { return KIND == B_Q80 ? 4 : KIND == B_Q6K ? 3 : 2; }
template <int KIND>
constexpr int aux_row_of() { return KIND == B_Q6K ? 12 : KIND == B_Q80 ? 8 : 16; }

template <int NWN, int KIND>
struct Ring {
    static constexpr int BN = 64 * NWN;
    static constexpr int SB = sb_of<KIND>();
    static constexpr int NB = SB == 4 ? 2 : 3;       // B super-stages in the ring
    static constexpr int A_STAGE = BM * BK * 2;
    static constexpr int PLANE = BN * SB * 16;
    static constexpr int AUX = planes_of<KIND>() * PLANE;
    static constexpr int MIN = AUX + BN * aux_row_of<KIND>();
    static constexpr int B_STAGE = MIN + (KIND == B_Q4K ? BM * 16 : 0);
    template <int NS>
    static constexpr int group_bytes() { return NS * A_STAGE + NB * B_STAGE; }
};

template <int SB>
__device__ __forceinline__ int swz(int n) { return SB == 4 ? (n >> 2) & 3 : ((n >> 2) ^ (n >> 3)) & 1; }
__device__ __forceinline__ int aswz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

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
    int n_stages;           // tiled weights: super-stages per row
};

// DMA issue. Every wave issues the same, compile-time number of load
// instructions per call (a_loads(), b_loads()), so s_waitcnt vmcnt counts
// cover whole stages. A: the NWN waves of a K group deal the activation
// tile's 64-slot blocks among them. B: wave wn loads its own 64 weight rows
// only (so the B side of a step needs no barrier, only the wave's own vmcnt),
// plus one of the two 64-token blocks of Q4_K block sums (waves wn % 2;
// identical bytes to the same LDS address where NWN > 2).
template <int NWN>
constexpr int a_loads() { return BM * 8 / 64 / NWN; }
template <int KIND>
constexpr int b_loads() {
    constexpr int SB = sb_of<KIND>();
    // planes: 64 rows x SB x 16 bytes = SB kilobytes each; then the aux region
    return planes_of<KIND>() * SB + (KIND == B_Q4K ? 2 : KIND == B_Q40 ? 4 : KIND == B_Q6K ? 3 : 2);
}

template <int NWN, int KIND>
__device__ __forceinline__ void issue_a(const GemmArgs& g, uint8_t* stage_base, int st, int wn, int lane) {
    const int kcol = st * BK;
#pragma unroll
    for (int j = 0; j < a_loads<NWN>(); ++j) {
        const int jj = j * NWN + wn;
        const int slot = jj * 64 + lane;
        const int r = slot >> 3, c = (slot & 7) ^ aswz(r);
        const int m = min(g.m0 + r, g.M - 1);
        lds_dma<16>(g.A + (size_t)m * g.lda + kcol + 8 * c, stage_base + jj * 64 * 16);
    }
}

// Weight tiles (dq_gemm_tiles_pack, opt-in): for every 64-row slice of the
// matrix and super-stage, the bytes one wave stages into its ring slot, in
// the ring's own order (items already at their swizzled slots, the scales as
// the ring's 4-byte slots), one contiguous run: per quant sub-plane
// [64 rows][SB slots][16 B], then the aux region (Q4_K: 64 super-block
// headers of 16 B; Q6_K: the 64 rows' 4 int8 scales of each of the 2 items,
// then d in the low half of a 4-byte slot; Q8_0 / Q4_0: the two fp16 block
// scales of each of the SB items). Slices run over whole 256-row tiles (rows
// past the matrix are zero), super-stages fastest, so a wave's K steps read
// one contiguous stream and every DMA instruction 64 lanes x 16 (or 4)
// consecutive bytes.
template <int KIND>
constexpr int tile_plane_bytes() { return 64 * sb_of<KIND>() * 16; }
template <int KIND>
constexpr int tile_aux_bytes() { return KIND == B_Q4K ? 64 * 16 : KIND == B_Q6K ? 3 * 256 : sb_of<KIND>() * 256; }
template <int KIND>
constexpr int tile_slice_bytes() { return planes_of<KIND>() * tile_plane_bytes<KIND>() + tile_aux_bytes<KIND>(); }

template <int NWN, int KIND, bool TL = false>
__device__ __forceinline__ void issue_b(const GemmArgs& g, uint8_t* bb, int sb, int wn, int lane) {
    using R = Ring<NWN, KIND>;
    constexpr int SB = R::SB, BN = R::BN;
    if constexpr (TL) {
        constexpr int PL = tile_plane_bytes<KIND>();
        const uint8_t* src = g.w + ((size_t)(g.n0 / 64 + wn) * g.n_stages + sb) * tile_slice_bytes<KIND>();
#pragma unroll
        for (int p = 0; p < planes_of<KIND>(); ++p)
#pragma unroll
            for (int k = 0; k < SB; ++k)
                lds_dma<16>(src + p * PL + (64 * k + lane) * 16, bb + p * R::PLANE + (64 * wn * SB + 64 * k) * 16);
        const uint8_t* aux = src + planes_of<KIND>() * PL;
        if constexpr (KIND == B_Q4K) {
            lds_dma<16>(aux + lane * 16, bb + R::AUX + 64 * wn * 16);
            const int blk = wn & 1, m = min(g.m0 + blk * 64 + lane, g.M - 1);
            lds_dma<16>(g.minp + ((size_t)sb * g.M + m) * 8, bb + R::MIN + blk * 64 * 16);
        } else {
            constexpr int NA = KIND == B_Q6K ? 3 : SB;  // 4-byte aux slots per row
#pragma unroll
            for (int c = 0; c < NA; ++c) lds_dma<4>(aux + c * 256 + lane * 4, bb + R::AUX + c * BN * 4 + 64 * wn * 4);
        }
        return;
    }
    const int item0 = SB * sb;
    // planes: instruction k covers own rows 64 SB^-1 ... : slot s = 64k + lane
#pragma unroll
    for (int p = 0; p < planes_of<KIND>(); ++p) {
#pragma unroll
        for (int k = 0; k < SB; ++k) {
            const int s = 64 * k + lane;
            const int n = 64 * wn + s / SB;                 // row in the tile
            const int t = (s % SB) ^ swz<SB>(n);            // the item this LDS slot holds
            const size_t r = (size_t)min(g.n0 + n, g.N - 1);
            const uint8_t* src = g.w + g.L.q_off + p * g.L.p_stride + r * g.L.q_row + 16 * (size_t)(item0 + t);
            lds_dma<16>(src, bb + p * R::PLANE + (64 * wn * SB + 64 * k) * 16);
        }
    }
    const int n = 64 * wn + lane;
    const size_t r = (size_t)min(g.n0 + n, g.N - 1);
    uint8_t* aux = bb + R::AUX;
    if constexpr (KIND == B_Q4K) {
        lds_dma<16>(g.w + g.L.s_off + r * g.L.s_row + 16 * (size_t)sb, aux + 64 * wn * 16);
        const int blk = wn & 1, m = min(g.m0 + blk * 64 + lane, g.M - 1);
        lds_dma<16>(g.minp + ((size_t)sb * g.M + m) * 8, bb + R::MIN + blk * 64 * 16);
    } else if constexpr (KIND == B_Q6K) {
#pragma unroll
        for (int c = 0; c < 2; ++c)
            lds_dma<4>(g.w + g.L.s_off + r * g.L.s_row + 4 * (size_t)(item0 + c), aux + c * BN * 4 + 64 * wn * 4);
        // a sub-dword LDS DMA still advances 4 bytes per lane: d sits in the
        // low half of a dword slot
        lds_dma<2>(g.w + g.L.d_off + r * g.L.d_row + 2 * (size_t)(item0 >> 2), aux + 2 * BN * 4 + 64 * wn * 4);
    } else {
        constexpr int ND = KIND == B_Q80 ? 2 : 4;  // one dword (two fp16 block scales) per item
#pragma unroll
        for (int c = 0; c < ND; ++c)
            lds_dma<4>(g.w + g.L.d_off + r * g.L.d_row + 4 * (size_t)(item0 + c), aux + c * BN * 4 + 64 * wn * 4);
    }
}

__device__ __forceinline__ const h8& lds_h8(const uint8_t* p) { return *reinterpret_cast<const h8*>(p); }
__device__ __forceinline__ dq_u32x4 lds_u4(const uint8_t* p) { return *reinterpret_cast<const dq_u32x4*>(p); }
__device__ __forceinline__ uint32_t lds_u1(const uint8_t* p) { return *reinterpret_cast<const uint32_t*>(p); }

// Raw weight bytes of item t of a B super-stage that this lane's B fragments
// need: for each of its two 32-row blocks j, 8 bytes of each quant sub-plane
// (Q4_K: all 16 bytes of sub-plane h = lane/32, see b_frag; the other
// formats: bytes 8h..8h+7 of each sub-plane, a 16-byte read and a select, so
// the reads stay conflict-free) and the row's scales.
struct BRaw {
    dq_u32x2 q0[2], q1[2], q2[2], q3[2];  // Q4_K: words 0-1 / 2-3 of sub-plane h; Q6_K: QA, QB, QH; Q8_0: P0..P3; Q4_0: P0, P1
    dq_u32x4 hd[2];  // Q4_K: super-block header; Q6_K: .x = 4 int8 scales, .y = d (low half); Q8_0/Q4_0: .x = 2 d
};

__device__ __forceinline__ dq_u32x2 half_of(const dq_u32x4& v, bool h) {
    return dq_u32x2{h ? v.z : v.x, h ? v.w : v.y};
}

template <int NWN, int KIND>
__device__ __forceinline__ void b_raw_j(const uint8_t* bb, int t, int wn, int lane, BRaw& r, int j) {
    using R = Ring<NWN, KIND>;
    constexpr int SB = R::SB, BN = R::BN;
    const int h = lane >> 5;
    {
        const int n = wn * 64 + j * 32 + (lane & 31);
        const int off = n * SB * 16 + 16 * (t ^ swz<SB>(n));
        if constexpr (KIND == B_Q4K) {
            const dq_u32x4 v = lds_u4(bb + h * R::PLANE + off);
            r.q0[j] = dq_u32x2{v.x, v.y};
            r.q1[j] = dq_u32x2{v.z, v.w};
            r.hd[j] = lds_u4(bb + R::AUX + n * 16);
        } else {
            r.q0[j] = half_of(lds_u4(bb + off), h);
            r.q1[j] = half_of(lds_u4(bb + R::PLANE + off), h);
            if constexpr (KIND == B_Q6K || KIND == B_Q80) r.q2[j] = half_of(lds_u4(bb + 2 * R::PLANE + off), h);
            if constexpr (KIND == B_Q80) r.q3[j] = half_of(lds_u4(bb + 3 * R::PLANE + off), h);
            r.hd[j].x = lds_u1(bb + R::AUX + t * BN * 4 + n * 4);
            if constexpr (KIND == B_Q6K) r.hd[j].y = lds_u1(bb + R::AUX + 2 * BN * 4 + n * 4);
        }
    }
}

template <int NWN, int KIND>
__device__ __forceinline__ void b_raw(const uint8_t* bb, int t, int wn, int lane, BRaw& r) {
    b_raw_j<NWN, KIND>(bb, t, wn, lane, r, 0);
    b_raw_j<NWN, KIND>(bb, t, wn, lane, r, 1);
}

// B fragments of a step of phase G (= st % 4, the item of the super-block)
// from the raw bytes, one 16-wide K slice KK at a time (so a slice can be
// built while the previous slice's MFMAs run): bf[j], j = 32-row n block.
// Lane l feeds row n = wn*64 + j*32 + l%32 with the 8 K values KK*16 +
// 8*(l/32) .. +7. Rows past N hold the clamped last row's bytes (finite
// values whose outputs are never stored). b_scales holds the fp16 scale pair
// of every (j, KK): Q4_K (the same for every slice) a0 = d*sc of sub-block 2G
// (the low nibbles), a1 = d*sc of 2G+1 (the high nibbles), -64 a0, -64 a1;
// Q6_K a = d*sc of the KK-th 16-block.
struct BScale {
    h2 s[2][4];  // Q6_K: scale pair per (j, KK); Q4_K: low-nibble a, high-nibble a, -64a of each
    uint32_t magic;
};

template <int KIND>
__device__ __forceinline__ void b_scales_j(const BRaw& r, int G, BScale& S, int j) {
    {
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

template <int KIND>
__device__ __forceinline__ void b_scales(const BRaw& r, int G, BScale& S) {
    b_scales_j<KIND>(r, G, S, 0);
    b_scales_j<KIND>(r, G, S, 1);
}

template <int KIND, int KK>
__device__ __forceinline__ h8 b_frag_j(const BRaw& r, const BScale& S, int j) {
    {
        uint32_t t[4];
        if constexpr (KIND == B_Q4K) {
            // Slice KK: word KK of sub-plane h (lane half h holds all 16 bytes
            // of sub-plane h). From the dword's bytes B0..B3, a nibble ORed into mantissa bits
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
        return __builtin_bit_cast(h8, dq_u32x4{t[0], t[1], t[2], t[3]});
    }
}

template <int KIND, int KK>
__device__ __forceinline__ void b_frag(const BRaw& r, const BScale& S, h8 (&bf)[2]) {
    bf[0] = b_frag_j<KIND, KK>(r, S, 0);
    bf[1] = b_frag_j<KIND, KK>(r, S, 1);
}

// A fragments of K slice kk for the wave's 4 32-token blocks (XOR-swizzled
// 16-byte chunks of a stage's activation tile).
__device__ __forceinline__ void a_frags(const uint8_t* base, int kk, int lane, h8 (&af)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = i * 32 + (lane & 31);
        af[i] = lds_h8(base + (r * 8 + ((2 * kk + (lane >> 5)) ^ aswz(r))) * 16);
    }
}

// What a wave holds for its next step before that step starts: the slice-0
// activation fragments and the B side (raw bytes, scales, slice-0 weight
// fragments); Q4_K: the super-block's min-term weight fragments, built during
// the super-block's second step.
struct Pre {
    h8 af[4];
    BRaw raw;
    BScale S;
    h8 bf[2];
    h8 bm[2];
};

// s_waitcnt vmcnt at the middle of a step of phase T: the A stage of the next
// step must have landed (and, at the last phase, this wave's part of the next
// B super-stage). DMAs are issued in the middle of each step - A(st + NS),
// then at phase 0 the B super-stage NB-1 ahead - so the count of DMA
// instructions issued after the needed one depends only on the phase.
template <int NWN, int KIND, int NS, int T>
constexpr int mid_wait() {
    constexpr int SB = sb_of<KIND>(), PA = a_loads<NWN>(), PB = b_loads<KIND>();
    // A(st+1) was issued NS-1 steps back; B issues in between at phase 0
    int w = 0;
    for (int back = NS - 1; back >= 1; --back) {
        // issues of step st - back, after A(st+1) itself (which is issued by step st+1-NS)
        const int ph = ((T - back) % SB + SB) % SB;
        if (back < NS - 1) w += PA;          // A issued by a later step
        if (ph == 0) w += PB;                 // that step's B issue (after its A)
    }
    return w;
}

__device__ __forceinline__ h8 a_frag(const uint8_t* base, int kk, int i, int lane) {
    const int r = i * 32 + (lane & 31);
    return lds_h8(base + (r * 8 + ((2 * kk + (lane >> 5)) ^ aswz(r))) * 16);
}

// MFMA q of a slice (32x32 block i = q/2 of the tokens, j = q%2 of the rows),
// and the pin that keeps the companion work written after it in place: a
// wave issues in order and an MFMA waits for the matrix pipe, so the LDS
// reads and conversions of the next slice are placed one or two per MFMA
// rather than in runs the scheduler would build (a run of MFMAs holds back
// every instruction behind it).
#define DQ_MF(AF, BF, Q) \
    acc[(Q) >> 1][(Q)&1] = __builtin_amdgcn_mfma_f32_32x32x16_f16((AF)[(Q) >> 1], (BF)[(Q)&1], acc[(Q) >> 1][(Q)&1], 0, 0, 0)
#define DQ_PIN() __builtin_amdgcn_sched_barrier(0)

// One K step st (phase T of super-stage sb) of a wave whose registers P hold
// the step's slice-0 fragments. Slices 0-2: each MFMA is followed by a piece
// of the next slice's work (its four activation fragments, LDS; its weight
// fragments, VALU) and, within a super-stage, of the next step's B side (this
// wave's own rows: raw bytes, scales, slice-0 fragments). Then, once every A
// read of the step is issued: the wait for the next step's stage, the
// workgroup barrier (this stage free, the next one visible), the DMAs into
// the freed stage (and at phase 0 the B super-stage NB-1 ahead), and slice
// 3 with the next step's slice-0 activation fragments; at the last phase the
// next super-stage's B side (landed by the wait), overlapped with the Q4_K
// min-term slice. Q4_K builds the min-term weight fragments in phase 1.
template <int NWN, int KIND, int NS, int T, bool TL>
__device__ __forceinline__ void gemm_step(const GemmArgs& g, uint8_t* aring, uint8_t* bring, int& astage, int sb,
                                          int a_next, int b_next, Pre& P, f16v (&acc)[4][2], int wn, int lane) {
    using R = Ring<NWN, KIND>;
    constexpr int SB = R::SB, NB = R::NB;
    constexpr bool LAST = T + 1 == SB;
    constexpr int T1 = LAST ? 0 : T + 1;
    constexpr bool MINT = KIND == B_Q4K && T == 3;  // min-term slice
    const uint8_t* abase = aring + astage * R::A_STAGE;
    const uint8_t* bbase = bring + (sb % NB) * R::B_STAGE;
    const int next_stage = astage + 1 == NS ? 0 : astage + 1;
    const uint8_t* anext = aring + next_stage * R::A_STAGE;
    const uint8_t* bnext = bring + ((sb + 1) % NB) * R::B_STAGE;
    h8 af1[4], af2[4], af3[4], bf1[2], bf2[2], bf3[2], bn[2], am[4];
    BRaw rn;
    BScale sn;
    sn.magic = P.S.magic;
    // slice 0
    DQ_MF(P.af, P.bf, 0); af1[0] = a_frag(abase, 1, 0, lane); DQ_PIN();
    DQ_MF(P.af, P.bf, 1); af1[1] = a_frag(abase, 1, 1, lane); DQ_PIN();
    DQ_MF(P.af, P.bf, 2); af1[2] = a_frag(abase, 1, 2, lane); DQ_PIN();
    DQ_MF(P.af, P.bf, 3); af1[3] = a_frag(abase, 1, 3, lane); DQ_PIN();
    DQ_MF(P.af, P.bf, 4); bf1[0] = b_frag_j<KIND, 1>(P.raw, P.S, 0); DQ_PIN();
    DQ_MF(P.af, P.bf, 5); if constexpr (!LAST) b_raw_j<NWN, KIND>(bbase, T1, wn, lane, rn, 0); DQ_PIN();
    DQ_MF(P.af, P.bf, 6); bf1[1] = b_frag_j<KIND, 1>(P.raw, P.S, 1); DQ_PIN();
    DQ_MF(P.af, P.bf, 7); if constexpr (!LAST) b_raw_j<NWN, KIND>(bbase, T1, wn, lane, rn, 1); DQ_PIN();
    // slice 1
    DQ_MF(af1, bf1, 0); af2[0] = a_frag(abase, 2, 0, lane); DQ_PIN();
    DQ_MF(af1, bf1, 1); if constexpr (KIND == B_Q4K && T == 1) P.bm[0] = q4k_neg_mins(P.raw.hd[0], true); DQ_PIN();
    DQ_MF(af1, bf1, 2); af2[1] = a_frag(abase, 2, 1, lane); af2[2] = a_frag(abase, 2, 2, lane); DQ_PIN();
    DQ_MF(af1, bf1, 3); if constexpr (KIND == B_Q4K && T == 1) P.bm[1] = q4k_neg_mins(P.raw.hd[1], true); DQ_PIN();
    DQ_MF(af1, bf1, 4); af2[3] = a_frag(abase, 2, 3, lane); bf2[0] = b_frag_j<KIND, 2>(P.raw, P.S, 0); DQ_PIN();
    DQ_MF(af1, bf1, 5); if constexpr (!LAST) b_scales_j<KIND>(rn, T1, sn, 0); DQ_PIN();
    DQ_MF(af1, bf1, 6); bf2[1] = b_frag_j<KIND, 2>(P.raw, P.S, 1); DQ_PIN();
    DQ_MF(af1, bf1, 7); if constexpr (!LAST) b_scales_j<KIND>(rn, T1, sn, 1); DQ_PIN();
    // slice 2
    DQ_MF(af2, bf2, 0); af3[0] = a_frag(abase, 3, 0, lane); DQ_PIN();
    DQ_MF(af2, bf2, 1); af3[1] = a_frag(abase, 3, 1, lane); DQ_PIN();
    DQ_MF(af2, bf2, 2); af3[2] = a_frag(abase, 3, 2, lane); DQ_PIN();
    DQ_MF(af2, bf2, 3); af3[3] = a_frag(abase, 3, 3, lane); DQ_PIN();
    DQ_MF(af2, bf2, 4); bf3[0] = b_frag_j<KIND, 3>(P.raw, P.S, 0); DQ_PIN();
    DQ_MF(af2, bf2, 5); if constexpr (!LAST) bn[0] = b_frag_j<KIND, 0>(rn, sn, 0); DQ_PIN();
    DQ_MF(af2, bf2, 6); bf3[1] = b_frag_j<KIND, 3>(P.raw, P.S, 1); DQ_PIN();
    DQ_MF(af2, bf2, 7); if constexpr (!LAST) bn[1] = b_frag_j<KIND, 0>(rn, sn, 1); DQ_PIN();
    // the next step's stage, the barrier, the DMAs into this step's stage
    wait_vm<mid_wait<NWN, KIND, NS, T>()>();
    dq_lds_barrier();
    issue_a<NWN, KIND>(g, aring + astage * R::A_STAGE, a_next, wn, lane);
    if constexpr (T == 0) issue_b<NWN, KIND, TL>(g, bring + (b_next % NB) * R::B_STAGE, b_next, wn, lane);
    DQ_PIN();
    // slice 3
    DQ_MF(af3, bf3, 0); P.af[0] = a_frag(anext, 0, 0, lane); DQ_PIN();
    DQ_MF(af3, bf3, 1); P.af[1] = a_frag(anext, 0, 1, lane); DQ_PIN();
    DQ_MF(af3, bf3, 2); P.af[2] = a_frag(anext, 0, 2, lane); DQ_PIN();
    DQ_MF(af3, bf3, 3); P.af[3] = a_frag(anext, 0, 3, lane); DQ_PIN();
    DQ_MF(af3, bf3, 4); if constexpr (LAST) b_raw_j<NWN, KIND>(bnext, 0, wn, lane, P.raw, 0); DQ_PIN();
    DQ_MF(af3, bf3, 5); if constexpr (LAST) b_raw_j<NWN, KIND>(bnext, 0, wn, lane, P.raw, 1); DQ_PIN();
    DQ_MF(af3, bf3, 6);
    if constexpr (MINT) {
        am[0] = lds_h8(bbase + R::MIN + (0 * 32 + (lane & 31)) * 16);
        am[1] = lds_h8(bbase + R::MIN + (1 * 32 + (lane & 31)) * 16);
    }
    DQ_PIN();
    DQ_MF(af3, bf3, 7);
    if constexpr (MINT) {
        am[2] = lds_h8(bbase + R::MIN + (2 * 32 + (lane & 31)) * 16);
        am[3] = lds_h8(bbase + R::MIN + (3 * 32 + (lane & 31)) * 16);
    }
    DQ_PIN();
    if constexpr (MINT) {
        // the super-block's min term: the block sums (lanes 0-31: the 8 K
        // values; lanes 32-63 zero) against -dmin*m; the next super-stage's
        // B side is converted behind it
        const h8 zero = {};
#pragma unroll
        for (int i = 0; i < 4; ++i) am[i] = (lane >> 5) == 0 ? am[i] : zero;
        DQ_MF(am, P.bm, 0); b_scales_j<KIND>(P.raw, 0, P.S, 0); DQ_PIN();
        DQ_MF(am, P.bm, 1); DQ_PIN();
        DQ_MF(am, P.bm, 2); b_scales_j<KIND>(P.raw, 0, P.S, 1); DQ_PIN();
        DQ_MF(am, P.bm, 3); DQ_PIN();
        DQ_MF(am, P.bm, 4); P.bf[0] = b_frag_j<KIND, 0>(P.raw, P.S, 0); DQ_PIN();
        DQ_MF(am, P.bm, 5); DQ_PIN();
        DQ_MF(am, P.bm, 6); P.bf[1] = b_frag_j<KIND, 0>(P.raw, P.S, 1); DQ_PIN();
        DQ_MF(am, P.bm, 7); DQ_PIN();
    } else if constexpr (LAST) {
        b_scales<KIND>(P.raw, 0, P.S);
        b_frag<KIND, 0>(P.raw, P.S, P.bf);
    } else {
        P.raw = rn;
        P.S = sn;
        P.bf[0] = bn[0];
        P.bf[1] = bn[1];
    }
    astage = next_stage;
}
#undef DQ_MF
#undef DQ_PIN

// The K group's super-stages [sb0, sb1) (whole super-blocks): the prologue
// puts the first B super-stage(s) and NS A stages in flight in the order the
// steady state would have issued them, waits for the first step's, and
// prefetches it; then SB steps per iteration. DMAs past the range re-read the
// group's last step / super-stage (valid addresses, never consumed).
template <int NWN, int KIND, int NS, bool TL>
__device__ __forceinline__ void run_steps(const GemmArgs& g, uint8_t* aring, uint8_t* bring, int sb0, int sb1,
                                          f16v (&acc)[4][2], int wn, int lane) {
    using R = Ring<NWN, KIND>;
    constexpr int SB = R::SB, NB = R::NB, PA = a_loads<NWN>(), PB = b_loads<KIND>();
    if (sb0 >= sb1) return;  // uniform over the workgroup (the planner gives every K group the same count)
    const int s0 = SB * sb0, s_last = SB * sb1 - 1, sb_last = sb1 - 1;
    issue_b<NWN, KIND, TL>(g, bring + (sb0 % NB) * R::B_STAGE, sb0, wn, lane);
    issue_a<NWN, KIND>(g, aring, s0, wn, lane);
    issue_a<NWN, KIND>(g, aring + R::A_STAGE, min(s0 + 1, s_last), wn, lane);
    if constexpr (NB == 3)
        issue_b<NWN, KIND, TL>(g, bring + ((sb0 + 1) % NB) * R::B_STAGE, min(sb0 + 1, sb_last), wn, lane);
    if constexpr (NS == 3) issue_a<NWN, KIND>(g, aring + 2 * R::A_STAGE, min(s0 + 2, s_last), wn, lane);
    // wait for B(sb0) and A(s0): the loads issued after A(s0) may stay in flight
    wait_vm<(NS - 1) * PA + (NB == 3 ? PB : 0)>();
    dq_lds_barrier();
    Pre P;
    P.S.magic = (uint32_t)__builtin_amdgcn_update_dpp((int)g.magic, (int)g.magic, 0xE4, 0xF, 0xF, false);
    a_frags(aring, 0, lane, P.af);
    b_raw<NWN, KIND>(bring + (sb0 % NB) * R::B_STAGE, 0, wn, lane, P.raw);
    b_scales<KIND>(P.raw, 0, P.S);
    b_frag<KIND, 0>(P.raw, P.S, P.bf);
    int astage = 0;
    for (int sb = sb0; sb < sb1; ++sb) {
        const int st = SB * sb;
        const int bn = min(sb + NB - 1, sb_last);
        gemm_step<NWN, KIND, NS, 0, TL>(g, aring, bring, astage, sb, min(st + NS, s_last), bn, P, acc, wn, lane);
        gemm_step<NWN, KIND, NS, 1, TL>(g, aring, bring, astage, sb, min(st + 1 + NS, s_last), bn, P, acc, wn, lane);
        if constexpr (SB == 4) {
            gemm_step<NWN, KIND, NS, 2, TL>(g, aring, bring, astage, sb, min(st + 2 + NS, s_last), bn, P, acc, wn, lane);
            gemm_step<NWN, KIND, NS, 3, TL>(g, aring, bring, astage, sb, min(st + 3 + NS, s_last), bn, P, acc, wn, lane);
        }
    }
    wait_vm<0>();  // drain the DMAs issued past the end
    dq_lds_barrier();
}

// Tile index -> (m block, n block): tiles are ordered m-major and handed to
// the 8 XCDs in contiguous ranges (workgroup id % 8 is its XCD), so the
// workgroups of one XCD share their activation rows in that XCD's L2.
// Tile of workgroup `id`. Workgroups are dealt to the 8 XCDs round-robin (id
// % 8), each XCD with its own L2: XCD x takes the x-th eighth of the tiles,
// ordered M-block fastest, so the M blocks sharing a weight tile run at the
// same time on one XCD and the weight bytes come from HBM once per XCD
// instead of once per M block (Q8_0 142 -> 113 us, Q6_K 142 -> 122 us at
// M = 512).
__device__ __forceinline__ void tile_of(int id, int mb, int nb, int* m_blk, int* n_blk) {
    const int total = mb * nb;
    int t = id;
    if (total % 8 == 0) t = (id % 8) * (total / 8) + id / 8;
    *m_blk = t % mb;
    *n_blk = t / mb;
}

// Workgroup of NWN x KSW = 4 waves, one per SIMD, one workgroup per CU (its
// LDS rings). The accumulators (128 per lane) live in AGPRs. blockIdx.z
// selects a K split (atomic_out: partials added into zeroed y, at most 2 so
// the sum is order-independent). KSW = 2: the K groups' partials are added
// through LDS in group order.
template <int FMT, int NWN, int KSW, int NS, bool TL>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void gemm_kernel(GemmArgs g, float* __restrict__ y, int nsb, int sb_per_split, int atomic_out) {
    static_assert(NWN * KSW == 4, "4 waves per workgroup");
    constexpr int KIND = kind_of<FMT>();
    using R = Ring<NWN, KIND>;
    constexpr int SB = R::SB, GROUP = R::template group_bytes<NS>();
    static_assert(KSW * GROUP <= 160 * 1024, "LDS");
    __shared__ __align__(16) uint8_t ring[KSW * GROUP];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = wave % NWN, kg = wave / NWN;
    int m_blk, n_blk;
    tile_of(blockIdx.x, (g.M + BM - 1) / BM, (g.N + R::BN - 1) / R::BN, &m_blk, &n_blk);
    g.n0 = n_blk * R::BN;
    g.m0 = m_blk * BM;
    // this split's super-blocks, then this K group's half (equal counts: the
    // planner only splits even ranges), in super-stages of SB items
    const int b0 = min(nsb, (int)blockIdx.z * sb_per_split);
    const int b1 = min(nsb, b0 + sb_per_split);
    const int half = (b1 - b0) / KSW;
    const int per = 4 / SB;  // super-stages per super-block
    const int sb0 = per * (b0 + kg * half), sb1 = per * (KSW == 1 ? b1 : b0 + (kg + 1) * half);

    f16v acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    uint8_t* gr = ring + kg * GROUP;
    run_steps<NWN, KIND, NS, TL>(g, gr, gr + NS * R::A_STAGE, sb0, sb1, acc, wn, lane);

    // K group 1 hands its partial to group 0 through the (drained) ring, one
    // half of the tile (j) at a time: acc0 + acc1 in that order
    if constexpr (KSW > 1) {
        float* red = reinterpret_cast<float*>(ring) + (size_t)wn * 4 * 16 * 64;
        static_assert(NWN * 4 * 16 * 64 * 4 <= KSW * GROUP, "reduction fits the ring");
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            if (kg == 1) {
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int r = 0; r < 16; ++r) red[(i * 16 + r) * 64 + lane] = acc[i][j][r];
            }
            __syncthreads();
            if (kg == 0) {
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[i][j][r] += red[(i * 16 + r) * 64 + lane];
            }
            __syncthreads();
        }
        if (kg != 0) return;
    }

    // D layout of 32x32x16: lane l, register r -> n = l%32, m = (r/4)*8 + (l/32)*4 + r%4.
    // The row factors 1/s of a 32-token block are loaded together before its
    // stores (unconditional loads of clamped rows; a load inside the store's
    // branch would be waited for one at a time).
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int mb0 = g.m0 + i * 32 + (lane >> 5) * 4;
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
// (0 natural, 1 Q6_K item order, 2 Q4_K fragment order with a min plane:
// fp16(exact float block sum * s) of block b at minp[b/8][t][b%8]); s the
// row's power-of-two range scale.

// The quantizer's row kernel: one workgroup per token row, thread j taking
// the 8-value groups j, j + TPR, ... of the row (up to G of them, kept in
// registers between the passes); a 32-block is 4 consecutive lanes, a Q4_K
// item (blocks 2i and 2i+1) 8. Per row: the power-of-two range scale s from
// the maximum over the row, then per block the reference integers and scale
// (amax over the 4 lanes) and, for the Q4_K min plane, the exact float sum
// of the block in element order (a running sum handed lane to lane), stored
// for up to two format classes (the block arithmetic does not depend on the
// layout). The input per SRC: the row x itself, the gated FFN product
// act(g) * x (the expression of the FFN's activation pass, so the same
// bits), or the RMSNorm of a (+ b, the residual, kept in h) with weight w,
// written to y when given (float squares summed in double, then
// (x * (1 / sqrt(mean + eps))) * w, rms_norm_rows_kernel's arithmetic). The
// workgroups also clear the outputs of the K-split GEMMs that read this
// activation next (z: float counts, multiples of 4, split evenly over the
// workgroups), which saves those GEMMs a fill launch.
struct QuantDst {
    _Float16* out;
    _Float16* minp;  // Q4_K block sums (perm 2), else unused
    float* rscale;
    float* inv;
    int perm;        // 2 Q4_K fragment order, 1 Q6_K item order, 0 natural
};
enum QuantSrcKind { Q_PLAIN = 0, Q_SILU = 1, Q_GELU = 2, Q_NORM = 3 };
struct QuantSrc {
    const float* x;  // the row input (Q_NORM: a)
    const float* g;  // gated: the gate; Q_NORM: the residual b (or null)
    const float* w;  // Q_NORM: the norm weight
    float* h;        // Q_NORM: a + b (when b and h are given)
    float* y;        // Q_NORM: the normalised row (when given)
    float eps;
};

// Group c (columns 8c .. 8c+7) of row `row`: the raw input (Q_NORM: a + b),
// or for the other kinds the quantizer's input itself.
template <int SRC>
__device__ __forceinline__ void group_in(const QuantSrc& S, size_t row, int c, float (&v)[8]) {
    const size_t o = row + 8 * (size_t)c;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        float4 f = *reinterpret_cast<const float4*>(S.x + o + 4 * k);
        if constexpr (SRC == Q_SILU || SRC == Q_GELU) {
            constexpr int A = SRC == Q_SILU ? DQ_ACT_SILU : DQ_ACT_GELU_TANH;
            const float4 gg = *reinterpret_cast<const float4*>(S.g + o + 4 * k);
            f = make_float4(dq_ffn_act<A>(gg.x) * f.x, dq_ffn_act<A>(gg.y) * f.y, dq_ffn_act<A>(gg.z) * f.z,
                            dq_ffn_act<A>(gg.w) * f.w);
        } else if constexpr (SRC == Q_NORM) {
            if (S.g) {
                const float4 c4 = *reinterpret_cast<const float4*>(S.g + o + 4 * k);
                f = make_float4(f.x + c4.x, f.y + c4.y, f.z + c4.z, f.w + c4.w);
            }
        }
        v[4 * k] = f.x; v[4 * k + 1] = f.y; v[4 * k + 2] = f.z; v[4 * k + 3] = f.w;
    }
}

// The 8 fp16 values h of group c (lane c % 4 of its block, c % 8 of its
// Q4_K item) into layout d of row t; for Q4_K the lane also receives its
// item partner's values (lanes 4 apart) and the last lane of a block writes
// the block sum fs.
__device__ __forceinline__ void store_group(const QuantDst& d, int lda, int n_tok, int t, int c, const h8& hv,
                                            float fs_scaled, bool sum_lane, bool ok) {
    _Float16* o = d.out + (size_t)t * lda;
    const int b = c / 4, q = c % 4;  // block, group in the block
    if (d.perm == 0) {
        if (ok) *reinterpret_cast<h8*>(o + 8 * (size_t)c) = hv;
    } else if (d.perm == 1) {
        // Q6_K item order: position pos of the 256-block -> column s*256 +
        // (2n+k)*64 + qq*16 + e, pos = 128n + 32qq + 16k + e
        const int sb = b / 8, pos0 = 32 * (b % 8);
        const int n = pos0 / 128, qq = (pos0 % 128) / 32, k = q / 2;
        if (ok) *reinterpret_cast<h8*>(o + sb * 256 + (2 * n + k) * 64 + qq * 16 + 8 * (q % 2)) = hv;
    } else {
        // Q4_K fragment order: chunk (kk, hf) at column 16 kk + 8 hf of item i
        // holds elements e0..e0+3 (e0 = 16 hf + 4 kk) of the low block and of
        // the high block as {lo e0, lo e0+2, hi e0, hi e0+2, lo e0+1, lo e0+3,
        // hi e0+1, hi e0+3}. Group q of the low block (elements 8q..8q+7)
        // writes chunk kk = 2 (q % 2), hf = q / 2 with the partner's first
        // four; the high block's group q the chunk kk + 1 with the low
        // group's last four.
        const bool hi = (c / 4) & 1;
        const dq_u32x4 mine = __builtin_bit_cast(dq_u32x4, hv);
        // low lanes send their last four values, high lanes their first four
        const uint32_t s0 = hi ? mine.x : mine.z, s1 = hi ? mine.y : mine.w;
        const uint32_t r0 = __shfl_xor(s0, 4, DQ_WAVE), r1 = __shfl_xor(s1, 4, DQ_WAVE);
        h8 lo4, hi4;  // elements e0..e0+3 of the two blocks (in their first four slots)
        if (!hi) {
            lo4 = hv;
            hi4 = __builtin_bit_cast(h8, dq_u32x4{r0, r1, 0u, 0u});
        } else {
            lo4 = __builtin_bit_cast(h8, dq_u32x4{r0, r1, 0u, 0u});
            hi4 = __builtin_bit_cast(h8, dq_u32x4{mine.z, mine.w, 0u, 0u});
        }
        const int kk = 2 * (q % 2) + (hi ? 1 : 0), hf = q / 2;
        const h8 ch = {lo4[0], lo4[2], hi4[0], hi4[2], lo4[1], lo4[3], hi4[1], hi4[3]};
        if (!ok) return;
        *reinterpret_cast<h8*>(o + 64 * (size_t)(b / 2) + 16 * kk + 8 * hf) = ch;
        if (sum_lane) d.minp[((size_t)(b / 8) * n_tok + t) * 8 + (b % 8)] = (_Float16)fs_scaled;
    }
}

template <int SRC, int G>
__global__ __launch_bounds__(1024) void quant_rows_kernel(QuantSrc S, int cols, int n_tok, int lda, QuantDst d0,
                                                          QuantDst d1, int n_dst, DqZeroSpans z) {
    __shared__ double dpart[16];
    __shared__ float fpart[16];
    const int tid = threadIdx.x, lane = tid & 63, TPR = blockDim.x, nw = TPR / 64;
    const int t = blockIdx.x;
#pragma unroll
    for (int k = 0; k < DqZeroSpans::N; ++k) {
        if (!z.p[k]) continue;
        const size_t n4 = z.n[k] / 4, per = (n4 + gridDim.x - 1) / gridDim.x;
        const size_t e = min(n4, per * (t + 1));
        for (size_t i = per * t + tid; i < e; i += TPR)
            reinterpret_cast<float4*>(z.p[k])[i] = float4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    const size_t row = (size_t)t * cols;
    const int ng = cols / 8;  // groups of the row (a multiple of 32)
    float v[G][8];
    // ng is a multiple of 32 and TPR of 64: a wave's groups are all
    // present, all absent, or present in its first half (whole blocks and
    // items either way)
#pragma unroll
    for (int it = 0; it < G; ++it) {
        const int c = tid + it * TPR;
        if (c < ng) group_in<SRC>(S, row, c, v[it]);
    }
    float nsc = 1.0f;
    if constexpr (SRC == Q_NORM) {
        double acc = 0.0;
#pragma unroll
        for (int it = 0; it < G; ++it) {
            const int c = tid + it * TPR;
            if (c >= ng) continue;
            if (S.g && S.h) {
                float* hp = S.h + row + 8 * (size_t)c;
                *reinterpret_cast<float4*>(hp) = make_float4(v[it][0], v[it][1], v[it][2], v[it][3]);
                *reinterpret_cast<float4*>(hp + 4) = make_float4(v[it][4], v[it][5], v[it][6], v[it][7]);
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float sq = v[it][e] * v[it][e];
                acc += (double)sq;
            }
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, DQ_WAVE);
        if (lane == 0) dpart[tid >> 6] = acc;
        __syncthreads();
        acc = 0.0;
        for (int w = 0; w < nw; ++w) acc += dpart[w];
        nsc = 1.0f / sqrtf((float)(acc / (double)cols) + S.eps);
#pragma unroll
        for (int it = 0; it < G; ++it) {
            const int c = tid + it * TPR;
            if (c >= ng) continue;
            const float4 w0 = *reinterpret_cast<const float4*>(S.w + 8 * (size_t)c);
            const float4 w1 = *reinterpret_cast<const float4*>(S.w + 8 * (size_t)c + 4);
            const float ww[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) v[it][e] = v[it][e] * nsc * ww[e];
            if (S.y) {
                float* yp = S.y + row + 8 * (size_t)c;
                *reinterpret_cast<float4*>(yp) = make_float4(v[it][0], v[it][1], v[it][2], v[it][3]);
                *reinterpret_cast<float4*>(yp + 4) = make_float4(v[it][4], v[it][5], v[it][6], v[it][7]);
            }
        }
    }
    float m = 0.0f;
#pragma unroll
    for (int it = 0; it < G; ++it)
        if (tid + it * TPR < ng)
#pragma unroll
            for (int e = 0; e < 8; ++e) m = fmaxf(m, fabsf(v[it][e]));
    m = dq_wave_max(m);
    if (lane == 0) fpart[tid >> 6] = m;
    __syncthreads();
    m = fpart[0];
    for (int w = 1; w < nw; ++w) m = fmaxf(m, fpart[w]);
    const float sc = row_scale_of(m);
    if (tid == 0) {
        d0.rscale[t] = sc;
        d0.inv[t] = 1.0f / sc;
        if (n_dst > 1) {
            d1.rscale[t] = sc;
            d1.inv[t] = 1.0f / sc;
        }
    }
    const bool sums = d0.perm == 2 || (n_dst > 1 && d1.perm == 2);
#pragma unroll
    for (int it = 0; it < G; ++it) {
        const int c = tid + it * TPR;
        if (it * TPR + (tid & ~63) >= ng) break;  // wave-uniform: the wave's groups are absent
        // the block's maximum over its 4 lanes
        float amax = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float a = fabsf(v[it][e]);
            amax = (amax < a) ? a : amax;
        }
        amax = fmaxf(amax, __shfl_xor(amax, 1, DQ_WAVE));
        amax = fmaxf(amax, __shfl_xor(amax, 2, DQ_WAVE));
        const float d = amax > 0.0f ? amax / 127.0f : 0.0f;
        const float id = d > 0.0f ? 1.0f / d : 0.0f;
        h8 hv;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            int q = (int)rintf(v[it][e] * id);
            q = q > 127 ? 127 : (q < -127 ? -127 : q);
            hv[e] = (_Float16)(((float)q * d) * sc);
        }
        // the block's exact float sum in element order: lane q of the block
        // continues the running sum of lane q - 1
        float fs = 0.0f;
        if (sums) {
            const int q = lane & 3;
            if (q == 0)
#pragma unroll
                for (int e = 0; e < 8; ++e) fs += v[it][e];
#pragma unroll
            for (int k = 1; k < 4; ++k) {
                const float p = __shfl_up(fs, 1, DQ_WAVE);
                if (q == k) {
                    fs = p;
#pragma unroll
                    for (int e = 0; e < 8; ++e) fs += v[it][e];
                }
            }
        }
        // lanes past the row (in a wave the row half covers) compute on
        // unset values but take part in the shuffles, which stay within
        // blocks and items, all present or all absent; they store nothing
        const bool sum_lane = (lane & 3) == 3, ok = c < ng;
        store_group(d0, lda, n_tok, t, c, hv, fs * sc, sum_lane, ok);
        if (n_dst > 1) store_group(d1, lda, n_tok, t, c, hv, fs * sc, sum_lane, ok);
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

int dq_gemm_cus() { return cus(); }

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
    fmt &= ~DQ_FMT_GEMM_TILES;
    if (!bytes) return DQ_ERR_INVALID_ARG;
    if (fmt != DQ_FMT_Q4_K && fmt != DQ_FMT_Q6_K && fmt != DQ_FMT_Q8_0 && fmt != DQ_FMT_Q4_0)
        return DQ_ERR_NOT_SUPPORTED;
    if (cols % 256) return DQ_ERR_NOT_SUPPORTED;
    *bytes = inv_off(fmt, cols, n_tok) + dq_align256(n_tok * 4);
    return DQ_OK;
}

static bool quant_fmt_ok(int fmt) {
    return fmt == DQ_FMT_Q4_K || fmt == DQ_FMT_Q6_K || fmt == DQ_FMT_Q8_0 || fmt == DQ_FMT_Q4_0;
}
static QuantDst quant_dst(int fmt, size_t cols, size_t n_tok, void* out) {
    uint8_t* base = (uint8_t*)out;
    QuantDst d{};
    d.out = (_Float16*)base;
    d.minp = fmt == DQ_FMT_Q4_K ? (_Float16*)(base + min_off(cols, n_tok)) : nullptr;
    d.rscale = (float*)(base + scale_off(fmt, cols, n_tok));
    d.inv = (float*)(base + inv_off(fmt, cols, n_tok));
    d.perm = fmt == DQ_FMT_Q6_K ? 1 : (fmt == DQ_FMT_Q4_K ? 2 : 0);
    return d;
}
// One workgroup per row of 64 (threads per row, up to 1024) times up to 8
// groups of 8 columns per thread: rows of up to 65536 columns.
constexpr size_t QUANT_MAX_COLS = 65536;
template <int SRC>
static int launch_quant_rows(const QuantSrc& S, size_t cols, size_t n_tok, const QuantDst (&d)[2], int n_dst,
                             const DqZeroSpans& z, hipStream_t s) {
    const int lda = (int)act_lda(cols);
    const size_t ng = cols / 8;
    int G = 1;
    while ((ng + G - 1) / G > 1024) G *= 2;
    const unsigned tpr = (unsigned)(((ng + G - 1) / G + 63) / 64 * 64);
    const unsigned grid = (unsigned)n_tok;
    switch (G) {
    case 1: quant_rows_kernel<SRC, 1><<<grid, tpr, 0, s>>>(S, (int)cols, (int)n_tok, lda, d[0], d[1], n_dst, z); break;
    case 2: quant_rows_kernel<SRC, 2><<<grid, tpr, 0, s>>>(S, (int)cols, (int)n_tok, lda, d[0], d[1], n_dst, z); break;
    case 4: quant_rows_kernel<SRC, 4><<<grid, tpr, 0, s>>>(S, (int)cols, (int)n_tok, lda, d[0], d[1], n_dst, z); break;
    default: quant_rows_kernel<SRC, 8><<<grid, tpr, 0, s>>>(S, (int)cols, (int)n_tok, lda, d[0], d[1], n_dst, z);
    }
    return dq_launch_status();
}

int dq_quantize_act_f16_zero(int fmt, const float* d_x, size_t cols, size_t n_tok, void* d_out,
                             const DqZeroSpans& z, void* stream, const float* d_gate, int act) {
    if (!quant_fmt_ok(fmt)) return DQ_ERR_NOT_SUPPORTED;
    if (cols % 256 || cols > QUANT_MAX_COLS || n_tok > (1u << 20)) return DQ_ERR_NOT_SUPPORTED;
    if (!d_x || !d_out) return DQ_ERR_INVALID_ARG;
    if (n_tok == 0) return DQ_OK;
    const QuantDst d[2] = {quant_dst(fmt, cols, n_tok, d_out), QuantDst{}};
    QuantSrc S{};
    S.x = d_x;
    S.g = d_gate;
    const hipStream_t s = (hipStream_t)stream;
    if (!d_gate) return launch_quant_rows<Q_PLAIN>(S, cols, n_tok, d, 1, z, s);
    if (act == DQ_ACT_SILU) return launch_quant_rows<Q_SILU>(S, cols, n_tok, d, 1, z, s);
    if (act == DQ_ACT_GELU_TANH) return launch_quant_rows<Q_GELU>(S, cols, n_tok, d, 1, z, s);
    return DQ_ERR_NOT_SUPPORTED;
}

int dq_norm_quant_f16(const float* d_a, const float* d_b, float* d_h, const float* d_w, size_t cols, size_t n_tok,
                      float eps, float* d_y, int n_fmt, const int* fmts, void* const* outs, const DqZeroSpans& z,
                      void* stream) {
    if (n_fmt < 1 || n_fmt > 2 || !fmts || !outs || !d_a || !d_w) return DQ_ERR_INVALID_ARG;
    if (cols % 256 || cols > QUANT_MAX_COLS || n_tok > (1u << 20)) return DQ_ERR_NOT_SUPPORTED;
    if (n_tok == 0) return DQ_OK;
    QuantDst d[2] = {};
    for (int k = 0; k < n_fmt; ++k) {
        if (!quant_fmt_ok(fmts[k])) return DQ_ERR_NOT_SUPPORTED;
        if (!outs[k]) return DQ_ERR_INVALID_ARG;
        d[k] = quant_dst(fmts[k], cols, n_tok, outs[k]);
    }
    QuantSrc S{};
    S.x = d_a;
    S.g = d_b;
    S.w = d_w;
    S.h = d_h;
    S.y = d_y;
    S.eps = eps;
    return launch_quant_rows<Q_NORM>(S, cols, n_tok, d, n_fmt, z, (hipStream_t)stream);
}

extern "C" int dq_quantize_act_f16(int fmt, const float* d_x, size_t cols, size_t n_tok, void* d_out,
                                   void* stream) {
    return dq_quantize_act_f16_zero(fmt, d_x, cols, n_tok, d_out, DqZeroSpans{}, stream);
}

template <int FMT, int NWN, int KSW, int NS, bool TL>
static int launch_gemm(const GemmArgs& g, size_t rows, size_t n_tok, int nsb, int split, float* d_y, bool y_zeroed,
                       hipStream_t s) {
    const int mb = (int)((n_tok + BM - 1) / BM), nb = (int)((rows + 64 * NWN - 1) / (64 * NWN));
    const int per = (nsb + split - 1) / split;  // super-blocks per split
    // both K groups of a workgroup must run the same number of steps (they
    // meet at every barrier): every split's range divides evenly
    if (KSW > 1 && (nsb % (split * KSW) != 0)) return DQ_ERR_NOT_SUPPORTED;
    if (split > 1 && !y_zeroed) {
        const size_t n = rows * n_tok;
        zero_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(d_y, n);
    }
    const dim3 grid((unsigned)(mb * nb), 1, split);
    gemm_kernel<FMT, NWN, KSW, NS, TL><<<grid, 256, 0, s>>>(g, d_y, nsb, per, split > 1);
    return dq_launch_status();
}

// Workgroup shapes: 4x1 (128 tokens x 256 rows, one K group, 3 A stages) or
// 2x2 (128 x 128, the K steps split between two wave pairs, 2 A stages; not
// for Q8_0, whose B super-stages leave no room for a second ring), optionally
// with a 2-way K split over workgroups (two partials added atomically into
// zeroed y: a+b == b+a, so the result is deterministic). One workgroup per
// CU; the plan with the fewest super-blocks on the busiest CU wins (rounds of
// the grid times super-blocks per K group), ties going to no split and then
// to 4x1. DQ_GEMM_SHAPE (41 or 22) and DQ_GEMM_SPLIT (1 or 2) override it for
// tuning where the override is valid.
struct GemmPlan {
    int nwn, split;
};
static bool plan_ok(int fmt, int nwn, int split, int nsb) {
    if (split == 2 && nsb < 2) return false;
    if (nwn == 2) return fmt != DQ_FMT_Q8_0 && nsb % (2 * split) == 0;
    return true;
}
static GemmPlan plan_gemm(int fmt, size_t rows, size_t n_tok, int nsb, int cu_budget = 0) {
    const size_t c = cu_budget > 0 ? (size_t)cu_budget : (size_t)cus();
    const size_t mb = (n_tok + BM - 1) / BM;
    GemmPlan best{4, 1};
    size_t best_cost = ~(size_t)0;
    for (int split = 1; split <= 2; ++split) {
        for (int nwn = 4; nwn >= 2; nwn -= 2) {
            if (!plan_ok(fmt, nwn, split, nsb)) continue;
            const int ksw = 4 / nwn;
            const size_t wgs = mb * ((rows + 64 * nwn - 1) / (64 * nwn)) * split;
            const int per_split = (nsb + split - 1) / split;
            const size_t cost = ((wgs + c - 1) / c) * (size_t)((per_split + ksw - 1) / ksw);
            if (cost < best_cost) {
                best_cost = cost;
                best = GemmPlan{nwn, split};
            }
        }
    }
    // tuning overrides, read once per process
    static const int force_shape = [] { const char* e = getenv("DQ_GEMM_SHAPE"); return e ? atoi(e) : 0; }();
    static const int force_split = [] { const char* e = getenv("DQ_GEMM_SPLIT"); return e ? atoi(e) : 0; }();
    GemmPlan o = best;
    if (force_shape == 41 || force_shape == 22) o.nwn = force_shape / 10;
    if (force_split == 1 || force_split == 2) o.split = force_split;
    return plan_ok(fmt, o.nwn, o.split, nsb) ? o : best;
}

template <int FMT, bool TL>
static int launch_plan(const GemmArgs& g, size_t rows, size_t n_tok, int nsb, float* d_y, bool y_zeroed,
                       hipStream_t s, int cu_budget) {
    const GemmPlan p = plan_gemm(FMT, rows, n_tok, nsb, cu_budget);
    if constexpr (FMT != DQ_FMT_Q8_0) {
        if (p.nwn == 2) return launch_gemm<FMT, 2, 2, 2, TL>(g, rows, n_tok, nsb, p.split, d_y, y_zeroed, s);
    }
    return launch_gemm<FMT, 4, 1, 3, TL>(g, rows, n_tok, nsb, p.split, d_y, y_zeroed, s);
}

bool dq_gemm_adds_into_y(int fmt, size_t rows, size_t cols, size_t n_tok, int cu_budget) {
    if (cols % 256 || rows == 0 || n_tok == 0) return false;
    return plan_gemm(fmt, rows, n_tok, (int)(cols / 256), cu_budget).split > 1;
}

size_t dq_gemm_workgroups(int fmt, size_t rows, size_t cols, size_t n_tok, int cu_budget) {
    if (cols % 256 || rows == 0 || n_tok == 0) return 0;
    const GemmPlan p = plan_gemm(fmt, rows, n_tok, (int)(cols / 256), cu_budget);
    return ((n_tok + BM - 1) / BM) * ((rows + 64 * p.nwn - 1) / (64 * p.nwn)) * p.split;
}

// ------------------------------------------------------------ weight tiles --
namespace {
template <int KIND>
__global__ __launch_bounds__(256) void gemm_tiles_pack_kernel(const uint8_t* __restrict__ w, DqLayout L, int rows,
                                                              int n_stages, long n_units, uint8_t* __restrict__ out) {
    constexpr int SB = sb_of<KIND>(), PL = tile_plane_bytes<KIND>();
    const long u = (long)blockIdx.x * 256 + threadIdx.x;  // (slice, super-stage, row of the slice)
    if (u >= n_units) return;
    const int nl = (int)(u % 64);
    const long ss = u / 64;
    const int st = (int)(ss % n_stages), slice = (int)(ss / n_stages);
    const int row = slice * 64 + nl;
    const bool live = row < rows;
    uint8_t* dst = out + (size_t)ss * tile_slice_bytes<KIND>();
    const dq_u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int p = 0; p < planes_of<KIND>(); ++p)
#pragma unroll
        for (int slot = 0; slot < SB; ++slot) {
            const int item = SB * st + (slot ^ swz<SB>(nl));
            const dq_u32x4 v = live ? *reinterpret_cast<const dq_u32x4*>(w + L.q_off + p * L.p_stride +
                                                                        (size_t)row * L.q_row + 16 * (size_t)item)
                                    : z;
            *reinterpret_cast<dq_u32x4*>(dst + p * PL + (nl * SB + slot) * 16) = v;
        }
    uint8_t* aux = dst + planes_of<KIND>() * PL;
    if constexpr (KIND == B_Q4K) {
        const dq_u32x4 v = live ? *reinterpret_cast<const dq_u32x4*>(w + L.s_off + (size_t)row * L.s_row + 16 * (size_t)st)
                                : z;
        *reinterpret_cast<dq_u32x4*>(aux + nl * 16) = v;
    } else if constexpr (KIND == B_Q6K) {
#pragma unroll
        for (int c = 0; c < 2; ++c)
            *reinterpret_cast<uint32_t*>(aux + c * 256 + nl * 4) =
                live ? *reinterpret_cast<const uint32_t*>(w + L.s_off + (size_t)row * L.s_row + 4 * (size_t)(SB * st + c))
                     : 0u;
        *reinterpret_cast<uint32_t*>(aux + 512 + nl * 4) =
            live ? (uint32_t)*reinterpret_cast<const uint16_t*>(w + L.d_off + (size_t)row * L.d_row +
                                                                2 * (size_t)((SB * st) >> 2))
                 : 0u;
    } else {
#pragma unroll
        for (int c = 0; c < SB; ++c)
            *reinterpret_cast<uint32_t*>(aux + c * 256 + nl * 4) =
                live ? *reinterpret_cast<const uint32_t*>(w + L.d_off + (size_t)row * L.d_row + 4 * (size_t)(SB * st + c))
                     : 0u;
    }
}

int tiles_geometry(int fmt, size_t rows, size_t cols, int* n_stages, long* n_slices, size_t* bytes) {
    int kind, sb;
    size_t slice;
    switch (fmt) {
    case DQ_FMT_Q4_K: kind = B_Q4K; slice = tile_slice_bytes<B_Q4K>(); break;
    case DQ_FMT_Q6_K: kind = B_Q6K; slice = tile_slice_bytes<B_Q6K>(); break;
    case DQ_FMT_Q8_0: kind = B_Q80; slice = tile_slice_bytes<B_Q80>(); break;
    case DQ_FMT_Q4_0: kind = B_Q40; slice = tile_slice_bytes<B_Q40>(); break;
    default: return DQ_ERR_NOT_SUPPORTED;
    }
    if (cols % 256 || cols == 0 || rows == 0 || rows > (1u << 30)) return DQ_ERR_NOT_SUPPORTED;
    sb = (kind == B_Q6K || kind == B_Q80) ? 2 : 4;
    *n_stages = (int)(cols / 64) / sb;
    *n_slices = (long)((rows + 255) / 256) * 4;  // whole 256-row tiles
    *bytes = (size_t)*n_slices * *n_stages * slice;
    return DQ_OK;
}
}  // namespace

extern "C" int dq_gemm_tiles_bytes(int fmt, size_t rows, size_t cols, size_t* bytes) {
    if (!bytes) return DQ_ERR_INVALID_ARG;
    int ns;
    long nsl;
    return tiles_geometry(fmt, rows, cols, &ns, &nsl, bytes);
}

extern "C" int dq_gemm_tiles_pack(int fmt, const void* d_packed, size_t rows, size_t cols, void* d_tiles,
                                  void* stream) {
    int ns;
    long nsl;
    size_t bytes;
    const int rc = tiles_geometry(fmt, rows, cols, &ns, &nsl, &bytes);
    if (rc != DQ_OK) return rc;
    if (!d_packed || !d_tiles) return DQ_ERR_INVALID_ARG;
    DqLayout L;
    if (!dq_layout(fmt, rows, cols, &L)) return DQ_ERR_NOT_SUPPORTED;
    const long units = nsl * ns * 64;
    const unsigned grid = (unsigned)((units + 255) / 256);
    const hipStream_t s = (hipStream_t)stream;
    const uint8_t* w = (const uint8_t*)d_packed;
    uint8_t* o = (uint8_t*)d_tiles;
    switch (fmt) {
    case DQ_FMT_Q4_K: gemm_tiles_pack_kernel<B_Q4K><<<grid, 256, 0, s>>>(w, L, (int)rows, ns, units, o); break;
    case DQ_FMT_Q6_K: gemm_tiles_pack_kernel<B_Q6K><<<grid, 256, 0, s>>>(w, L, (int)rows, ns, units, o); break;
    case DQ_FMT_Q8_0: gemm_tiles_pack_kernel<B_Q80><<<grid, 256, 0, s>>>(w, L, (int)rows, ns, units, o); break;
    default: gemm_tiles_pack_kernel<B_Q40><<<grid, 256, 0, s>>>(w, L, (int)rows, ns, units, o); break;
    }
    return dq_launch_status();
}

// GEMM on the workspace written by dq_quantize_act_f16.
extern "C" int dq_gemm_f16act(int fmt, const void* d_w, size_t rows, size_t cols, const void* d_work,
                              size_t n_tok, float* d_y, void* stream) {
    return dq_gemm_f16act_zeroed(fmt, d_w, rows, cols, d_work, n_tok, d_y, false, stream);
}

int dq_gemm_f16act_zeroed(int fmt_in, const void* d_w, size_t rows, size_t cols, const void* d_work, size_t n_tok,
                          float* d_y, bool y_zeroed, void* stream, int cu_budget) {
    DqLayout L;
    const bool tiled = (fmt_in & DQ_FMT_GEMM_TILES) != 0;
    const int fmt = fmt_in & ~DQ_FMT_GEMM_TILES;
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
    const int nsb = (int)cols / 256;  // super-blocks (cols % 256 == 0)
    g.n_stages = (int)(cols / 64) / (fmt == DQ_FMT_Q6_K || fmt == DQ_FMT_Q8_0 ? 2 : 4);
    if (tiled) {
        switch (fmt) {
        case DQ_FMT_Q4_K: return launch_plan<DQ_FMT_Q4_K, true>(g, rows, n_tok, nsb, d_y, y_zeroed, s, cu_budget);
        case DQ_FMT_Q8_0: return launch_plan<DQ_FMT_Q8_0, true>(g, rows, n_tok, nsb, d_y, y_zeroed, s, cu_budget);
        case DQ_FMT_Q4_0: return launch_plan<DQ_FMT_Q4_0, true>(g, rows, n_tok, nsb, d_y, y_zeroed, s, cu_budget);
        default: return launch_plan<DQ_FMT_Q6_K, true>(g, rows, n_tok, nsb, d_y, y_zeroed, s, cu_budget);
        }
    }
    switch (fmt) {
    case DQ_FMT_Q4_K: return launch_plan<DQ_FMT_Q4_K, false>(g, rows, n_tok, nsb, d_y, y_zeroed, s, cu_budget);
    case DQ_FMT_Q8_0: return launch_plan<DQ_FMT_Q8_0, false>(g, rows, n_tok, nsb, d_y, y_zeroed, s, cu_budget);
    case DQ_FMT_Q4_0: return launch_plan<DQ_FMT_Q4_0, false>(g, rows, n_tok, nsb, d_y, y_zeroed, s, cu_budget);
    default: return launch_plan<DQ_FMT_Q6_K, false>(g, rows, n_tok, nsb, d_y, y_zeroed, s, cu_budget);
    }
}


extern "C" int dq_gemm(int fmt_in, const void* d_w, size_t rows, size_t cols, const float* d_x, size_t n_tok,
                       float* d_y, void* d_work, size_t work_bytes, void* stream) {
    const int fmt = fmt_in & ~DQ_FMT_GEMM_TILES;  // the activation side is the format's
    size_t need = 0;
    const int rc = dq_gemm_workspace_bytes(fmt, rows, cols, n_tok, &need);
    if (rc != DQ_OK) return rc;
    if (work_bytes < need || (need && !d_work)) return DQ_ERR_INVALID_ARG;
    // the K-split plans add their partials into y: the quantizer clears it,
    // unless y overlaps x (the quantizer is still reading x), in which case
    // the GEMM launch clears y itself after the quantizer has finished
    const uintptr_t xb = reinterpret_cast<uintptr_t>(d_x), yb = reinterpret_cast<uintptr_t>(d_y);
    const bool overlap = xb < yb + rows * n_tok * sizeof(float) && yb < xb + n_tok * cols * sizeof(float);
    DqZeroSpans z{};
    const bool zero = !overlap && dq_zero_span_ok(d_y, rows * n_tok) && rows <= (1u << 30) &&
                      dq_gemm_adds_into_y(fmt, rows, cols, n_tok);
    if (zero) {
        z.p[0] = d_y;
        z.n[0] = rows * n_tok;
    }
    const int r1 = dq_quantize_act_f16_zero(fmt, d_x, cols, n_tok, d_work, z, stream);
    if (r1 != DQ_OK) return r1;
    return dq_gemm_f16act_zeroed(fmt_in, d_w, rows, cols, d_work, n_tok, d_y, zero, stream);
}
