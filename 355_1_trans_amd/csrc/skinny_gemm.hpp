// Skinny-M / split-K GEMM for gfx950 (decode shapes and the LDS-bypass path).
//
// Decode GEMMs stream B once and are HBM-bound.  Two MI355X facts shape the
// kernel (measured with streaming-read microbenchmarks):
//  * one CU sustains only ~50 GB/s of streaming reads (8 waves, >= 64 KB in
//    flight), so HBM bandwidth needs ~150-200 CUs streaming at once;
//  * that per-CU rate is a rate of cache-line requests: a wave load that
//    touches 16 half lines (the scaled-MFMA fragment order, lane 16q+r =
//    row r) moves half the bytes of one that touches 8 whole lines.
// So the host picks the N-tile width (16, 32 or 64 columns: NB blocks of 16)
// to put work on as many CUs as possible in one round, splitting K across
// workgroups only when 16-column tiles leave too many CUs idle, and B is
// read in whole 128-byte lines:
//  * row-major / K-panel B: buffer -> LDS DMA in whole-line order (8 rows x
//    128 B per instruction), into a per-wave LDS ring, then ds_read_b128
//    into MFMA fragments.  The 16-byte chunks of a row are XOR-swizzled on
//    the way in (the DMA lane picks which chunk it fetches), which makes the
//    fragment reads bank-conflict free;
//  * B'' (LDS-bypass entry): already in fragment order and 1 KB contiguous
//    per wave load, so it goes straight into registers.
// A fragments (small, L2-resident) and scales are loaded into registers.
//
// A workgroup (8 wave64) owns NB*16 output columns, MB*16 rows and a slice
// of the K-tiles (128 bytes of K each).  Wave w takes K-tiles w, w+8, ... of
// the slice; its loads run D K-tiles ahead of the MFMAs.  All loads are raw
// buffer loads with a loop-invariant per-lane offset and a wave-uniform
// K-tile offset; a ring slot past the wave's last K-tile loads through a
// zero-range descriptor (zeros, no memory traffic), so the loads stay
// unconditional and the compiler's wait counts stay exact.  The eight
// waves' partial sums meet in LDS and are added in a fixed order (the result
// does not depend on timing).  With split-K > 1 each workgroup stores its
// fp32 partial tile into the caller's workspace and the last workgroup of a
// tile (atomic counter) sums the partials in slice order, rounds and re-arms
// the counter, all in the same launch.
//
// Register layout of the scaled MFMA 16x16x128 (pinned by the layout probes,
// probe.hip): operand lane L = 16q + r holds row r; fp8 dwords 0-3 carry K
// [16q, 16q+16) and dwords 4-7 K [64+16q, 64+16q+16) (16-byte chunks q and
// q+4 of a 128-byte row), fp4 dwords 0-3 carry K [32q, 32q+32) (chunk 2q, then
// 2q+1 in the second instruction); lane group q's scale byte covers K [32q,
// 32q+32).  srcA = B fragment, srcB = A fragment; the accumulator of lane
// L = 16q + r holds C[m = r][n = 4q .. 4q+3] of a 16 x 16 block.
//
// B layouts: RAW [N][Kbytes]; KPANEL [K/128][N][128]; FRAG (this library's
// B'' for the LDS-bypass entry): for every 16-row block nb and K-tile kt,
// 2048 contiguous bytes [nb][kt][h][lane][16] where lane L = 16q + r holds
// row 16nb + r and h selects the lane's first or second 16-byte operand
// chunk.
#pragma once
#include <utility>

#include "launch.hpp"
#include "tile_args.hpp"

namespace qg {

constexpr BLay kBFrag = BLay::FRAG;
constexpr int kSkinnyWaves = 8;

struct SkinnyArgs {
    TileArgs t;              // operands, shapes, strides (tiles_* / group_m unused)
    float* ws;               // fp32 partials [splitk][batch][M][N] (splitk > 1)
    unsigned* counters;      // [batch][m_tiles][n_tiles]: epoch-tagged arrival counters
    unsigned epoch;          // this launch's counter epoch (split_arrive)
    int splitk, kt_per_split, n_tiles, m_tiles;
    int scale_panel;         // MX: per-wave scale panels (skinny_scale_panel_ok)
};

// MX scale panels: a wave takes a contiguous run of at most 64 / kt_bytes
// K-tiles (kt_bytes = scale bytes per row and K-tile; runs start on a
// 16-byte boundary of the scale row) and DMAs its rows' scale bytes for the
// whole run once, 64 bytes per row, into its own LDS panel; needs 16-byte
// aligned scale rows and K slices starting on a 16-byte boundary.
__host__ __device__ constexpr int skinny_panel_run(int slice_kt, int waves, int kt_bytes) {
    const int g = 16 / kt_bytes;
    return ((slice_kt + waves - 1) / waves + g - 1) / g * g;
}
// the panels fit next to at least two LDS ring stages of B (mx: B rows
// have panel blocks too)
__host__ __device__ constexpr bool skinny_scp_fits(int mb, int nb, bool mx = true) {
    return 2 * 8 * nb * 2048 + 8 * (mb + (mx ? nb : 1)) * 1024 <= 152 * 1024;
}

// blockIdx.x -> (n-tile, m-tile): the m-tiles that share one B slice get
// workgroup ids 8 apart, i.e. the same XCD (ids are dealt round-robin over
// the 8 XCDs), so the second read of the slice hits that XCD's L2.
// Grid x = ceil(n_tiles / 8) * 8 * m_tiles; ids past n_tiles exit at once.
__host__ __device__ inline int skinny_grid_x(int n_tiles, int m_tiles) { return (n_tiles + 7) / 8 * 8 * m_tiles; }

// K-tiles in flight per wave.  Register budget: D stages of A fragments
// (8*MB dwords + scales) next to 4*MB*NB accumulators (and, without the LDS
// ring, 8*NB dwords of B per stage).  LDS budget (LDS ring): 8 waves x D
// stages x NB*2 KB <= 152 KB, less the scale panels ((MB + NB) KB per wave).
__host__ __device__ constexpr int skinny_depth(int mb, int nb, bool lds_b, bool scp = false, bool mx = true) {
    const int lds = 152 * 1024 - (scp ? kSkinnyWaves * (mb + (mx ? nb : 1)) * 1024 : 0);
    int d = lds_b ? (150 - 8 * mb * nb) / (8 * mb + 6) : (150 - 4 * mb * nb) / (8 * (mb + nb) + 6);
    if (lds_b && d > lds / (kSkinnyWaves * nb * 2048)) d = lds / (kSkinnyWaves * nb * 2048);
    return d > 8 ? 8 : (d < 2 ? 2 : d);
}

template <int N, class F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
// f(std::integral_constant<int, i>) for i = 0 .. N-1, unrolled at compile time.
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl<N>(f, std::make_integer_sequence<int, N>{});
}

// NTB: B moves with the nontemporal cache policy (one M tile: each B byte
// is read once; with several M tiles the other tiles re-read it from cache)
template <int FMT, ScaleKind SK, BLay BL, int MB, int NB, bool BF16, bool SCP, bool NTB>
__global__ __launch_bounds__(kSkinnyWaves * 64) void skinny_gemm_kernel(const SkinnyArgs sp) {
    constexpr int BKB = 128, W = kSkinnyWaves;
    static_assert(MB == 1 || MB == 2 || MB == 4, "16, 32 or 64 rows per M-tile");
    static_assert(NB == 1 || NB == 2 || NB == 4, "16, 32 or 64 columns per N-tile");
    static_assert(SK == ScaleKind::MX || SK == ScaleKind::BSF32, "E8M0 or fp32 block scales");
    static_assert(BL == BLay::RAW || BL == BLay::KPANEL || BL == kBFrag, "row-major, K-panel or B''");
    constexpr bool FP4 = (FMT == kFmtFp4);
    constexpr bool MX = (SK == ScaleKind::MX);
    constexpr bool VALU_SCALE = (SK == ScaleKind::BSF32);
    constexpr bool LDS_B = (BL != kBFrag);
    constexpr int D = skinny_depth(MB, NB, LDS_B, SCP, SK == ScaleKind::MX);
    // scale bytes per row and K-tile: E8M0 bytes (MX) or one fp32 word
    constexpr int KT_BYTES = FP4 ? 8 : 4;
    // a wave's panel: 16-row blocks x 64-byte rows -- MX: A and B rows;
    // fp32 scales: A rows and one block whose rows all hold the tile's
    // 128-column weight-scale row (row-major row scales only)
    constexpr int PB_BLOCKS = MB + (MX ? NB : 1);
    constexpr int PANEL_W = PB_BLOCKS * 1024;
    constexpr int ROWS = MB * 16, COLS = NB * 16;
    constexpr int RP = COLS + 4;           // reduction row pitch in floats (breaks the bank period)
    constexpr int REGION = ROWS * RP;
    constexpr int NT = W * 64;
    constexpr int SLOT = NB * 2048;        // one wave's B bytes per K-tile
    constexpr int RING = LDS_B ? W * SLOT : 16;
    // one LDS object per ring stage: the compiler tracks DMA completion per
    // object, so reading stage d waits only for stage d's DMAs
    __shared__ __attribute__((aligned(16))) uint8_t ring0[RING];
    __shared__ __attribute__((aligned(16))) uint8_t ring1[D > 1 ? RING : 16];
    __shared__ __attribute__((aligned(16))) uint8_t ring2[D > 2 ? RING : 16];
    __shared__ __attribute__((aligned(16))) uint8_t ring3[D > 3 ? RING : 16];
    __shared__ __attribute__((aligned(16))) uint8_t ring4[D > 4 ? RING : 16];
    __shared__ __attribute__((aligned(16))) uint8_t ring5[D > 5 ? RING : 16];
    __shared__ __attribute__((aligned(16))) uint8_t ring6[D > 6 ? RING : 16];
    __shared__ __attribute__((aligned(16))) uint8_t ring7[D > 7 ? RING : 16];
    __shared__ __attribute__((aligned(16))) uint8_t spanel[SCP ? W * PANEL_W : 16];
    // two reduction regions; with the LDS ring they reuse ring0 once every
    // wave has left the K loop
    constexpr int RED_BYTES = 2 * REGION * 4;
    static_assert(!LDS_B || RED_BYTES <= RING, "reduction regions fit in ring0");
    __shared__ __attribute__((aligned(16))) float red_own[LDS_B ? 4 : 2 * REGION];
    __shared__ int last_flag;
    float* const red = LDS_B ? reinterpret_cast<float*>(ring0) : red_own;
    // LDS-typed views, formed here in the kernel body (not inside lambdas)
    QG_LDS uint8_t* const lr0 = (QG_LDS uint8_t*)ring0;
    QG_LDS uint8_t* const lr1 = (QG_LDS uint8_t*)ring1;
    QG_LDS uint8_t* const lr2 = (QG_LDS uint8_t*)ring2;
    QG_LDS uint8_t* const lr3 = (QG_LDS uint8_t*)ring3;
    QG_LDS uint8_t* const lr4 = (QG_LDS uint8_t*)ring4;
    QG_LDS uint8_t* const lr5 = (QG_LDS uint8_t*)ring5;
    QG_LDS uint8_t* const lr6 = (QG_LDS uint8_t*)ring6;
    QG_LDS uint8_t* const lr7 = (QG_LDS uint8_t*)ring7;
    auto ring = [&](auto dc) -> QG_LDS uint8_t* {
        constexpr int d = decltype(dc)::value;
        if constexpr (d == 0) return lr0;
        else if constexpr (d == 1) return lr1;
        else if constexpr (d == 2) return lr2;
        else if constexpr (d == 3) return lr3;
        else if constexpr (d == 4) return lr4;
        else if constexpr (d == 5) return lr5;
        else if constexpr (d == 6) return lr6;
        else return lr7;
    };

    const TileArgs& p = sp.t;
    const int M = p.m, N = p.n, KB = p.kbytes, LDA = p.lda, LDB = p.ldb, LDC = p.ldc;
    const int SFA_SM = p.sfa_sm, SFA_SK = p.sfa_sk, SFB_SN = p.sfb_sn;
    const int nk = KB / BKB;
    const int slot = blockIdx.x >> 3;
    const int mt = slot % sp.m_tiles;
    const int nt = (slot / sp.m_tiles) * 8 + (blockIdx.x & 7);
    if (nt >= sp.n_tiles) return;
    const int sk = blockIdx.y, bz = blockIdx.z;
    const int n0 = nt * COLS, m0 = mt * ROWS;
    const int kt_begin = sk * sp.kt_per_split;
    const int kt_end = min(nk, kt_begin + sp.kt_per_split);

    // the wave index is uniform: keep it (and every K-tile index) in SGPRs
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), L = tid & 63;
    const int q = L >> 4, l16 = L & 15;
    if (sp.splitk > 1 && tid == 0)
        split_claim(sp.counters + ((long long)bz * sp.m_tiles + mt) * sp.n_tiles + nt, sp.epoch);

    const uint8_t* A = p.a + bz * p.a_batch;
    const uint8_t* B = p.b + bz * p.b_batch;
    const uint8_t* SFA = p.sfa + bz * p.sfa_batch * (VALU_SCALE ? 4 : 1);
    const uint8_t* SFB = p.sfb + bz * p.sfb_batch * (VALU_SCALE ? 4 : 1);

    // ---- loop-invariant per-lane byte offsets (the host bounds every operand below 2^31 bytes) ----
    const int c0 = FP4 ? 2 * q : q;            // first 16-byte chunk of the lane's fragment
    const int c1 = FP4 ? 2 * q + 1 : q + 4;    // second chunk
    int aoff[MB][2], sa_voff[MB];
#pragma unroll
    for (int i = 0; i < MB; ++i) {
        const int m = min(m0 + i * 16 + l16, M - 1);
        aoff[i][0] = m * LDA + c0 * 16;
        aoff[i][1] = m * LDA + c1 * 16;
        sa_voff[i] = MX ? m * SFA_SM + (FP4 ? 2 * q : q) : m * SFA_SM * 4;
    }
    int boff[NB][2], sb_voff[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
        const int n = min(n0 + j * 16 + l16, N - 1);
        sb_voff[j] = MX ? n * SFB_SN + (FP4 ? 2 * q : q) : ((n0 >> 7) * SFB_SN) * 4;   // a tile never crosses a 128-column scale block
        if constexpr (LDS_B) {
            // DMA instruction h of block j moves rows 8h .. 8h+7 in whole
            // lines: lane L fetches row R = 8h + L/8, logical chunk
            // (L % 8) ^ swz(R), landing at physical chunk L % 8 of row R
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int R = 8 * h + (L >> 3);
                const int row = min(n0 + j * 16 + R, N - 1);
                const int c = (L & 7) ^ swz<FP4>(R);
                boff[j][h] = (BL == BLay::RAW ? row * LDB : row * BKB) + c * 16;
            }
        } else {
            const int base = (n >> 4) * nk * 2048 + L * 16;
            boff[j][0] = base;
            boff[j][1] = base + 1024;
        }
    }
    // bytes between consecutive K-tiles of B, A, and the scale arrays
    const int b_kstep = (BL == BLay::KPANEL) ? N * BKB : ((BL == BLay::RAW) ? BKB : 2048);
    const int s_kstep = MX ? (FP4 ? 8 : 4) : 4;
    const int sa_kstep = MX ? s_kstep : SFA_SK * 4;
    // fragment-read offsets inside a wave's ring slot: row l16, chunks c0 / c1
    const int frag0 = l16 * BKB + ((c0 ^ swz<FP4>(l16)) * 16);
    const int frag1 = l16 * BKB + ((c1 ^ swz<FP4>(l16)) * 16);

    auto rsrc = [](const void* base, bool valid) {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, valid ? 0x7FFFFFFF : 0, 0x00020000);
    };
    auto ld16 = [](__amdgpu_buffer_rsrc_t r, int voff, int soff) -> i32x4 {
        return __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
    };
    auto ld16b = [](__amdgpu_buffer_rsrc_t r, int voff, int soff) -> i32x4 {
        return __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, NTB ? 2 : 0));
    };
    auto cat8 = [](i32x4 lo, i32x4 hi) { return i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]}; };

    struct Stage {
        i32x8 a[MB];
        i32x8 b[LDS_B ? 1 : NB];
        int sa[MB];
        int sb[NB];
        float fa[MB];
        float fb;
    };
    auto load = [&](auto dc, Stage& s, int kt, bool valid) {
        const __amdgpu_buffer_rsrc_t rB = rsrc(B, valid), rA = rsrc(A, valid);
        const __amdgpu_buffer_rsrc_t rSA = rsrc(SFA, valid), rSB = rsrc(SFB, valid);
        if constexpr (LDS_B) {
            QG_LDS uint8_t* dst = ring(dc) + w * SLOT;
#pragma unroll
            for (int j = 0; j < NB; ++j)
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    if constexpr (NTB) dma16_buf_nt(rB, dst + j * 2048 + h * 1024, boff[j][h], kt * b_kstep);
                    else dma16_buf(rB, dst + j * 2048 + h * 1024, boff[j][h], kt * b_kstep);
        } else {
#pragma unroll
            for (int j = 0; j < NB; ++j)
                s.b[j] = cat8(ld16b(rB, boff[j][0], kt * b_kstep), ld16b(rB, boff[j][1], kt * b_kstep));
        }
#pragma unroll
        for (int i = 0; i < MB; ++i) s.a[i] = cat8(ld16(rA, aoff[i][0], kt * BKB), ld16(rA, aoff[i][1], kt * BKB));
        if constexpr (SCP) {
            // scales come from the wave's panel (compute)
        } else if constexpr (MX) {
#pragma unroll
            for (int i = 0; i < MB; ++i) {
                if constexpr (FP4) s.sa[i] = __builtin_amdgcn_raw_buffer_load_b16(rSA, sa_voff[i], kt * sa_kstep, 0);
                else s.sa[i] = __builtin_amdgcn_raw_buffer_load_b8(rSA, sa_voff[i], kt * sa_kstep, 0);
            }
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                if constexpr (FP4) s.sb[j] = __builtin_amdgcn_raw_buffer_load_b16(rSB, sb_voff[j], kt * s_kstep, 0);
                else s.sb[j] = __builtin_amdgcn_raw_buffer_load_b8(rSB, sb_voff[j], kt * s_kstep, 0);
            }
        } else {
#pragma unroll
            for (int i = 0; i < MB; ++i)
                s.fa[i] = __builtin_bit_cast(float,
                                             __builtin_amdgcn_raw_buffer_load_b32(rSA, sa_voff[i], kt * sa_kstep, 0));
            s.fb = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rSB, sb_voff[0], kt * 4, 0));
        }
    };

    f32x4 acc[MB][NB];
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int unit = p.unit_scale;

    auto mma = [&](int i, int j, const Stage& s, const i32x8& bf) {
        if constexpr (FP4) {
            const i32x8 b0 = i32x8{bf[0], bf[1], bf[2], bf[3], 0, 0, 0, 0};
            const i32x8 b1 = i32x8{bf[4], bf[5], bf[6], bf[7], 0, 0, 0, 0};
            const i32x8 a0 = i32x8{s.a[i][0], s.a[i][1], s.a[i][2], s.a[i][3], 0, 0, 0, 0};
            const i32x8 a1 = i32x8{s.a[i][4], s.a[i][5], s.a[i][6], s.a[i][7], 0, 0, 0, 0};
            acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(b0, a0, acc[i][j], kFmtFp4, kFmtFp4, 0,
                                                                         s.sb[j], 0, s.sa[i]);
            acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(b1, a1, acc[i][j], kFmtFp4, kFmtFp4, 1,
                                                                         s.sb[j], 1, s.sa[i]);
        } else if constexpr (VALU_SCALE) {
            const f32x4 part = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                bf, s.a[i], f32x4{0.f, 0.f, 0.f, 0.f}, kFmtFp8, kFmtFp8, 0, unit, 0, unit);
            const float sc = s.fa[i] * s.fb;
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[i][j][r] = __builtin_fmaf(part[r], sc, acc[i][j][r]);
        } else {
            acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bf, s.a[i], acc[i][j], kFmtFp8, kFmtFp8, 0,
                                                                         s.sb[j], 0, s.sa[i]);
        }
    };
    auto compute = [&](auto dc, const Stage& s0, int kl) {
        // kl: the K-tile's index in the wave's run (scale panel column)
        Stage s = s0;
        if constexpr (SCP && MX) {
            const QG_LDS uint8_t* pw = (const QG_LDS uint8_t*)spanel + w * PANEL_W + l16 * 64 + kl * KT_BYTES;
#pragma unroll
            for (int i = 0; i < MB; ++i)
                s.sa[i] = FP4 ? *(const QG_LDS uint16_t*)(pw + i * 1024 + 2 * q) : pw[i * 1024 + q];
#pragma unroll
            for (int j = 0; j < NB; ++j)
                s.sb[j] = FP4 ? *(const QG_LDS uint16_t*)(pw + (MB + j) * 1024 + 2 * q) : pw[(MB + j) * 1024 + q];
        } else if constexpr (SCP) {
            const QG_LDS uint8_t* pw = (const QG_LDS uint8_t*)spanel + w * PANEL_W + kl * 4;
#pragma unroll
            for (int i = 0; i < MB; ++i) s.fa[i] = *(const QG_LDS float*)(pw + i * 1024 + l16 * 64);
            s.fb = *(const QG_LDS float*)(pw + MB * 1024);
        }
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            i32x8 bf;
            if constexpr (LDS_B) {
                const QG_LDS uint8_t* src = ring(dc) + w * SLOT + j * 2048;
                bf = cat8(*(const QG_LDS i32x4*)(src + frag0), *(const QG_LDS i32x4*)(src + frag1));
            } else {
                bf = s.b[j];
            }
#pragma unroll
            for (int i = 0; i < MB; ++i) mma(i, j, s, bf);
        }
    };

    // ---- K loop: wave w takes K-tiles kt_begin + w, + W, ...; D in flight ----
    // interleaved K-tiles (wave w: kt_begin + w, + W, ...) or, with scale
    // panels, a contiguous run per wave
    const int run = SCP ? skinny_panel_run(kt_end - kt_begin, W, KT_BYTES) : 1;
    const int kfirst = kt_begin + (SCP ? w * run : w);
    const int kstep = SCP ? 1 : W;
    const int ntw = SCP ? max(0, min(kt_end, kfirst + run) - kfirst)
                        : (kt_end - kfirst + W - 1) / W;     // K-tiles of this wave
    if (ntw > 0) {
        if constexpr (SCP) {
            // the run's scale bytes, 64 per row: 4 lanes per row, 16 rows per
            // DMA (one cache line per row for the whole run); the byte range
            // of the scale array bounds the buffer (the run's end may pass K)
            QG_LDS uint8_t* pw = (QG_LDS uint8_t*)spanel + w * PANEL_W;
            const int kb = kfirst * KT_BYTES + (L & 3) * 16;
            // row strides in bytes (the fp32 strides count words)
            const int a_rs = MX ? SFA_SM : 4 * SFA_SM, b_rs = MX ? SFB_SN : 4 * SFB_SN;
            const auto rSAp = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(SFA), 0,
                                                                (unsigned)((M - 1) * a_rs + nk * KT_BYTES), 0x00020000);
#pragma unroll
            for (int i = 0; i < MB; ++i)
                dma16_buf(rSAp, pw + i * 1024, min(m0 + i * 16 + (L >> 2), M - 1) * a_rs + kb, 0);
            if constexpr (MX) {
                const auto rSBp = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(SFB), 0,
                                                                    (unsigned)((N - 1) * b_rs + nk * KT_BYTES), 0x00020000);
#pragma unroll
                for (int j = 0; j < NB; ++j)
                    dma16_buf(rSBp, pw + (MB + j) * 1024, min(n0 + j * 16 + (L >> 2), N - 1) * b_rs + kb, 0);
            } else {
                const int nbr = (N - 1) >> 7;    // last 128-column scale row
                const auto rSBp = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(SFB), 0,
                                                                    (unsigned)(nbr * b_rs + nk * KT_BYTES), 0x00020000);
                dma16_buf(rSBp, pw + MB * 1024, min(n0 >> 7, nbr) * b_rs + kb, 0);
            }
        }
        Stage st[D];
        static_for<D>([&](auto dc) {
            constexpr int d = decltype(dc)::value;
            load(dc, st[d], kfirst + kstep * d, d < ntw);
        });
        int i = 0;
        for (; i + D <= ntw; i += D) {
            static_for<D>([&](auto dc) {
                constexpr int d = decltype(dc)::value;
                compute(dc, st[d], i + d);
                load(dc, st[d], kfirst + kstep * (i + d + D), i + d + D < ntw);
                __builtin_amdgcn_sched_barrier(0);   // keep the ring order
            });
        }
        static_for<D - 1>([&](auto dc) {
            constexpr int d = decltype(dc)::value;
            if (d < ntw - i) compute(dc, st[d], i + d);
        });
    }

    // ---- reduce the eight waves in LDS, in a fixed order:
    // region r (r < 2) = acc(6+r) + acc(4+r) + acc(2+r) + acc(r); tile = region 0 + region 1
    auto put = [&](int region, bool add) {
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                f32x4* dst = (f32x4*)&red[region * REGION + (i * 16 + l16) * RP + j * 16 + 4 * q];
                if (add) {
                    const f32x4 u = *dst;
                    f32x4 v = acc[i][j];
                    for (int r = 0; r < 4; ++r) v[r] += u[r];
                    *dst = v;
                } else {
                    *dst = acc[i][j];
                }
            }
    };
    wait_vmcnt<0>();                          // ring slots past the last K-tile still receive zeros
    __syncthreads();                          // every wave has left the K loop (ring0 becomes red)
    if (w >= 6) put(w - 6, false);
    __syncthreads();
    if (w >= 4 && w < 6) put(w - 4, true);
    __syncthreads();
    if (w >= 2 && w < 4) put(w - 2, true);
    __syncthreads();
    if (w < 2) put(w, true);
    __syncthreads();
    auto tile_sum = [&](int e) -> f32x4 {    // e = row * COLS + col, col % 4 == 0
        const int o = (e / COLS) * RP + e % COLS;
        f32x4 v = *(const f32x4*)&red[o];
        const f32x4 u = *(const f32x4*)&red[REGION + o];
        for (int r = 0; r < 4; ++r) v[r] += u[r];
        return v;
    };

    // ---- output: 4 adjacent columns per thread and pass ----
    auto store4 = [&](int row, int col, f32x4 v) {
        const int m = m0 + row, n = n0 + col;
        if (m >= M) return;
        if constexpr (BF16) {
            uint16_t* c = (uint16_t*)p.c + bz * p.c_batch + (long long)m * LDC + n;
            if (n + 3 < N && p.c_vec >= 4) {
                *(u32x2*)c = u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
            } else {
                for (int r = 0; r < 4; ++r)
                    if (n + r < N) c[r] = bf16_bits(v[r]);
            }
        } else {
            float* c = (float*)p.c + bz * p.c_batch + (long long)m * LDC + n;
            if (n + 3 < N && p.c_vec >= 4) {
                *(f32x4*)c = v;
            } else {
                for (int r = 0; r < 4; ++r)
                    if (n + r < N) c[r] = v[r];
            }
        }
    };
    if (sp.splitk == 1) {
        for (int e = tid * 4; e < ROWS * COLS; e += NT * 4) store4(e / COLS, e % COLS, tile_sum(e));
        return;
    }

    // split-K: store this slice's partial tile, then the last workgroup of
    // the tile reduces all slices in order 0..splitk-1.  Publication:
    // device-coherent partial stores, completed before a barrier, then one
    // relaxed counter atomic per workgroup (see store_partial4, common.hpp).
    const long long plane = (long long)M * N;
    const int batch = gridDim.z;
    const long long split_stride = (long long)batch * plane;
    const auto part = partial_rsrc(sp.ws + ((long long)sk * batch + bz) * plane);
    const bool vec_ok = (N & 3) == 0;
    for (int e = tid * 4; e < ROWS * COLS; e += NT * 4) {
        const int m = m0 + e / COLS, n = n0 + e % COLS;
        if (m >= M) continue;
        const f32x4 v = tile_sum(e);
        const int x = m * N + n;
        if (n + 3 < N && vec_ok) {
            store_partial4(part, x, v);
        } else {
            for (int r = 0; r < 4; ++r)
                if (n + r < N) store_partial1(part, x + r, v[r]);
        }
    }
    wait_vmcnt<0>();
    __syncthreads();
    unsigned* ctr = sp.counters + ((long long)bz * sp.m_tiles + mt) * sp.n_tiles + nt;
    if (tid == 0)
        last_flag = split_arrive(ctr, sp.epoch, sp.splitk);
    __syncthreads();
    if (!last_flag) return;
    const float* ws0 = sp.ws + (long long)bz * plane;
    // PASSES groups of 4 columns per thread; with whole-vector rows every
    // pass's loads of a group of SG slices are in flight together, the
    // slices summed in order 0 .. splitk - 1
    constexpr int PASSES = (ROWS * COLS + NT * 4 - 1) / (NT * 4);
    constexpr int SG = 16 / PASSES < 8 ? 16 / PASSES : 8;
    int rr[PASSES], cc[PASSES];
    bool live[PASSES];
    f32x4 v[PASSES];
#pragma unroll
    for (int q = 0; q < PASSES; ++q) {
        const int e = tid * 4 + q * NT * 4;
        rr[q] = e / COLS;
        cc[q] = e % COLS;
        live[q] = e < ROWS * COLS && m0 + rr[q] < M;
        v[q] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    if (vec_ok) {
        // N % 4 == 0: a thread's 4 columns are all in or all out
        for (int s0 = 0; s0 < sp.splitk; s0 += SG) {
            f32x4 u[SG][PASSES];
#pragma unroll
            for (int t = 0; t < SG; ++t)
#pragma unroll
                for (int q = 0; q < PASSES; ++q)
                    if (s0 + t < sp.splitk && live[q] && n0 + cc[q] < N)
                        u[t][q] = load_partial4(partial_rsrc(ws0 + (s0 + t) * split_stride),
                                                (m0 + rr[q]) * N + n0 + cc[q]);
#pragma unroll
            for (int t = 0; t < SG; ++t)
#pragma unroll
                for (int q = 0; q < PASSES; ++q)
                    if (s0 + t < sp.splitk && live[q] && n0 + cc[q] < N) v[q] += u[t][q];
        }
    } else {
#pragma unroll
        for (int q = 0; q < PASSES; ++q) {
            if (!live[q]) continue;
            const int x = (m0 + rr[q]) * N + n0 + cc[q];
            for (int s0 = 0; s0 < sp.splitk; ++s0) {
                const auto src = partial_rsrc(ws0 + s0 * split_stride);
                for (int r = 0; r < 4; ++r)
                    if (n0 + cc[q] + r < N) v[q][r] += load_partial1(src, x + r);
            }
        }
    }
#pragma unroll
    for (int q = 0; q < PASSES; ++q)
        if (live[q]) store4(rr[q], cc[q], v[q]);
    if (tid == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Launches one instantiation of a format / scale / B-layout family.
template <int FMT, ScaleKind SK, BLay BL>
hipError_t launch_skinny_family(const SkinnyArgs& a, int mb, int nb, int batch, bool bf16, hipStream_t s) {
    const dim3 grid(skinny_grid_x(a.n_tiles, a.m_tiles), a.splitk, batch);
    const dim3 block(kSkinnyWaves * 64);
#define QG_SKINNY_LAUNCH(MBV, NBV, SCPV, NTV)                                                        \
    if (bf16) skinny_gemm_kernel<FMT, SK, BL, MBV, NBV, true, SCPV, NTV><<<grid, block, 0, s>>>(a);  \
    else skinny_gemm_kernel<FMT, SK, BL, MBV, NBV, false, SCPV, NTV><<<grid, block, 0, s>>>(a);      \
    trace_launch("skinny_gemm<%s,%s,%s,mb%d,nb%d,%s%s%s,splitk%d>", FMT == kFmtFp4 ? "fp4" : "fp8",    \
                 scale_name(SK), layout_name(BL), MBV, NBV, bf16 ? "bf16" : "fp32", SCPV ? ",scp" : "",  \
                 NTV ? ",ntb" : "", a.splitk);                                                       \
    return hipGetLastError();
// mb < 4 always means one M tile (the plan takes mb = 4 beyond 32 rows)
#define QG_SKINNY_NT(MBV, NBV, SCPV)                                                                 \
    if (MBV < 4 || a.m_tiles == 1) { QG_SKINNY_LAUNCH(MBV, NBV, SCPV, true) }                        \
    else { QG_SKINNY_LAUNCH(MBV, NBV, SCPV, (MBV < 4)) }
#define QG_SKINNY_CASE(MBV, NBV)                                                                     \
    if (mb == MBV && nb == NBV) {                                                                    \
        if constexpr (skinny_scp_fits(MBV, NBV, SK == ScaleKind::MX)) {                              \
            if (a.scale_panel) { QG_SKINNY_NT(MBV, NBV, true) }                                      \
        }                                                                                            \
        QG_SKINNY_NT(MBV, NBV, false)                                                                \
    }
    QG_SKINNY_CASE(1, 1) QG_SKINNY_CASE(1, 2) QG_SKINNY_CASE(1, 4)
    QG_SKINNY_CASE(2, 1) QG_SKINNY_CASE(2, 2) QG_SKINNY_CASE(2, 4)
    QG_SKINNY_CASE(4, 1) QG_SKINNY_CASE(4, 2) QG_SKINNY_CASE(4, 4)
#undef QG_SKINNY_CASE
#undef QG_SKINNY_NT
#undef QG_SKINNY_LAUNCH
    return hipErrorInvalidValue;
}

}  // namespace qg
