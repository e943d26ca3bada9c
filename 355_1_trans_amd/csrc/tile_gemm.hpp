// LDS-staged tile GEMM for gfx950 on the scaled MFMA 16x16x128.
//
// One workgroup of 8 wave64 (2 per SIMD) computes a 256 x 256 tile of C.
// The K loop walks 128-byte K-tiles (128 e4m3 or 256 e2m1 values per row):
//   * global -> LDS by DMA (global_load_lds_dwordx4), two LDS stages; the
//     copy of K-tile t+1 is in flight while K-tile t is multiplied;
//   * each 128-byte LDS row is XOR-swizzled per 16-byte chunk (common.hpp:
//     swz) so that the per-lane 16-byte operand reads are conflict free;
//   * v_mfma_scale_f32_16x16x128_f8f6f4, lane L = 16q + r of an operand
//     holds row r.  Its E8M0 scale byte covers K elements [32q, 32q+32) of
//     the instruction.  Register layout (pinned by the layout probes and the
//     per-K-group scale tests): fp8 -- dwords 0-3 hold K [16q, 16q+16) and
//     dwords 4-7 hold K [64+16q, 64+16q+16), so the lane fetches 16-byte
//     chunks q and q+4 of the row; fp4 -- dwords 0-3 hold K [32q, 32q+32),
//     i.e. 16-byte chunk 2q for the first and 2q+1 for the second MFMA of a
//     256-element K-tile;
//   * srcA is the B fragment and srcB the A fragment, so the accumulator of
//     lane L holds C[m = L%16][n = 4*(L/16) + r], r = 0..3 (four adjacent
//     columns of one row: one 8- or 16-byte store per block in the epilogue,
//     and one fp32 block scale per lane in the BSF32 policy).
//
// Scale policies (one K-tile = 128 bytes of K):
//   MX    one E8M0 per 32 K elements, row-major [rows][K/32] (MX8 host.cc:282-285,
//         MX4 host.cc:207-208).  A row's scales of one K-tile are 4 (fp8) or
//         8 (fp4) bytes of a different cache line per row, so they are moved
//         as 16-byte panels covering 4 (fp8) or 2 (fp4) K-tiles, double
//         buffered: one L1 request per row per panel instead of per K-tile.
//   BS8   one E8M0 per 128 K elements: SFA column-major [K/128][M], SFB
//         [N/128][K/128] (SNAP gemm_a8w8_mxfp8_scale_common.h:28-35), broadcast
//         to the four 32-element lane groups in the matrix core.
//   BSF32 fp32 scales per 1x128 (A) and 128x128 (B) block (BPS host.cc:66-90):
//         the MFMA runs unscaled (E8M0 127 = 1.0) into a fresh fp32 partial
//         and the VALU adds partial * (sfa*sfb) into the accumulator, the
//         reference's order of operations (scale each K-group, then sum).
// B layouts: RAW [N][Kbytes]; KPANEL [Kbytes/128][N][128] (BPS host.cc:92-111);
//            W16 shuffle_weight(16,16) [N/16][Kbytes/16][16][16] (SNAP host.cc:161-179).
#pragma once
#include "common.hpp"

namespace qg {

enum class ScaleKind : int { MX = 0, BS8 = 1, BSF32 = 2 };
enum class BLay : int { RAW = 0, KPANEL = 1, W16 = 2 };

struct TileArgs {
    const uint8_t* a;
    const uint8_t* b;
    void* c;
    const uint8_t* sfa;
    const uint8_t* sfb;
    int m, n;
    int kbytes;          // bytes of K per row: K (fp8) or K/2 (fp4); multiple of 128
    int lda, ldb;        // row pitch in bytes (ldb: RAW only)
    int ldc;             // row pitch of C in elements
    long long a_batch, b_batch, c_batch, sfa_batch, sfb_batch;  // batch strides (bytes / elements)
    // scale addressing (in scale elements):
    //   MX    : sfa(m, g) = sfa[m*sfa_sm + g], sfb(n, g) = sfb[n*sfb_sn + g]
    //   BS8   : sfa(m, kt) = sfa[kt*sfa_sk + m], sfb(nb, kt) = sfb[nb*sfb_sn + kt]
    //   BSF32 : sfa(m, kt) = sfa[kt*sfa_sk + m*sfa_sm], sfb(nb, kt) = sfb[nb*sfb_sn + kt]
    int sfa_sm, sfa_sk, sfb_sn;
    int tiles_m, tiles_n;
    int group_m;         // tile-rows per raster group
    int unit_scale;      // E8M0 127, passed at run time
};

// 8 waves: 2 x 4 waves of 128 x 64 (hardware-scaled policies) or 4 x 2 waves
// of 64 x 128 (BSF32, whose VALU-updated accumulators live in VGPRs).
template <ScaleKind SK>
struct TileShape {
    static constexpr int WAVES_M = 2, WAVES_N = 4, BLK_M = 8, BLK_N = 4;
};
template <>
struct TileShape<ScaleKind::BSF32> {
    static constexpr int WAVES_M = 4, WAVES_N = 2, BLK_M = 4, BLK_N = 8;
};

template <ScaleKind SK>
constexpr int tile_threads() {
    return 64 * TileShape<SK>::WAVES_M * TileShape<SK>::WAVES_N;
}

// PB (MX only): bytes of one row's scale panel moved per DMA lane: 16
// (needs 16-byte aligned scale rows whose length K/32 is a multiple of 16)
// or the K-tile's own 4 (fp8) / 8 (fp4) bytes.
template <int FMT, ScaleKind SK, BLay BL, bool BF16, int PB = 16>
__global__ __launch_bounds__(tile_threads<SK>(), 1) void tile_gemm_kernel(const TileArgs p) {
    using Shape = TileShape<SK>;
    constexpr int WAVES_N = Shape::WAVES_N, WAVES_M = Shape::WAVES_M;
    constexpr int BLK_M = Shape::BLK_M, BLK_N = Shape::BLK_N;
    constexpr int NW = WAVES_M * WAVES_N;
    constexpr int BM = WAVES_M * BLK_M * 16, BN = WAVES_N * BLK_N * 16, BKB = 128;
    static_assert(BM == 256 && BN == 256, "tile is 256 x 256");
    constexpr int DMA_PER_WAVE = BM / 8 / NW;  // 16-byte-per-lane DMAs per operand
    constexpr bool FP4 = (FMT == kFmtFp4);
    constexpr bool MX = (SK == ScaleKind::MX);
    constexpr bool VALU_SCALE = (SK == ScaleKind::BSF32);
    // MX scale panels: PB bytes per row = SPAN K-tiles, double buffered.
    // LDS image of one panel (256 rows):
    //   PB = 16       : [row][16 B]          (one dwordx4 DMA lane per row)
    //   PB = 4  (fp8) : [row][4 B]           (one dword DMA lane per row)
    //   PB = 8  (fp4) : [2 halves][row][4 B] (two dword DMAs per row)
    constexpr int KT_BYTES = FP4 ? 8 : 4;   // scale bytes per row per K-tile
    static_assert(PB == 16 || PB == KT_BYTES, "panel width");
    constexpr int SPAN = PB / KT_BYTES;
    constexpr int PANEL = 256 * 16;
    // per-stage scale slots of the block-scale policies
    constexpr int SA_BYTES = MX ? 2 * PANEL : (SK == ScaleKind::BS8 ? 256 : 1024);
    constexpr int SB_BYTES = MX ? 2 * PANEL : 256 * NW;

    __shared__ __attribute__((aligned(1024))) uint8_t lA0[BM * BKB];
    __shared__ __attribute__((aligned(1024))) uint8_t lA1[BM * BKB];
    __shared__ __attribute__((aligned(1024))) uint8_t lB0[BN * BKB];
    __shared__ __attribute__((aligned(1024))) uint8_t lB1[BN * BKB];
    // MX: lSA0/lSB0 hold both panel buffers; block-scale: per-stage slots
    __shared__ __attribute__((aligned(256))) uint8_t lSA0[SA_BYTES];
    __shared__ __attribute__((aligned(256))) uint8_t lSA1[MX ? 16 : SA_BYTES];
    __shared__ __attribute__((aligned(256))) uint8_t lSB0[SB_BYTES];
    __shared__ __attribute__((aligned(256))) uint8_t lSB1[MX ? 16 : SB_BYTES];

    // ---- tile coordinates: XCD-contiguous remap, then grouped raster ----
    const int T = p.tiles_m * p.tiles_n;
    int bid = blockIdx.x;
    if ((T & 7) == 0) bid = (bid & 7) * (T >> 3) + (bid >> 3);
    const int gfull = p.group_m * p.tiles_n;
    const int g = bid / gfull;
    const int first_m = g * p.group_m;
    const int gm = min(p.tiles_m - first_m, p.group_m);
    const int within = bid - g * gfull;
    const int tm = first_m + within % gm;
    const int tn = within / gm;
    const int bz = blockIdx.z;
    const int m0 = tm * BM, n0 = tn * BN;

    // Kernel arguments are copied into locals once: lambdas below must not
    // read the argument block through a reference inside the K loop (that
    // becomes vector loads whose vmcnt wait also drains the DMA queue).
    const int M = p.m, N = p.n, KB = p.kbytes, LDA = p.lda, LDB = p.ldb, LDC = p.ldc;
    const int SFA_SM = p.sfa_sm, SFA_SK = p.sfa_sk, SFB_SN = p.sfb_sn;

    const int tid = threadIdx.x;
    const int w = tid >> 6, L = tid & 63;
    const int wm = w / WAVES_N, wn = w % WAVES_N;
    const int q = L >> 4, l16 = L & 15;

    const uint8_t* A = p.a + bz * p.a_batch + (long long)m0 * LDA;
    // B rebased to the tile's first column, so per-lane DMA offsets stay
    // within 32 bits (256 rows of one K-tile, or one K-panel)
    const uint8_t* B = p.b + bz * p.b_batch +
                       (BL == BLay::RAW ? (long long)n0 * LDB
                                        : BL == BLay::KPANEL ? (long long)n0 * BKB : (long long)(n0 >> 4) * 16 * KB);
    const uint8_t* SFA = p.sfa + bz * p.sfa_batch * (VALU_SCALE ? 4 : 1);
    const uint8_t* SFB = p.sfb + bz * p.sfb_batch * (VALU_SCALE ? 4 : 1);

    // ---- per-lane DMA source offsets ----
    // DMA t of wave w fills LDS rows (w*DMA_PER_WAVE + t)*8 .. +8; lane L
    // writes row +L/8, physical chunk L%8 = logical chunk (L%8) ^ swz(row).
    int aoff[DMA_PER_WAVE], boff[DMA_PER_WAVE];
#pragma unroll
    for (int t = 0; t < DMA_PER_WAVE; ++t) {
        const int r = (w * DMA_PER_WAVE + t) * 8 + (L >> 3);
        const int c = (L & 7) ^ swz<FP4>(r);
        aoff[t] = (min(m0 + r, M - 1) - m0) * LDA + c * 16;
        const int gn = min(n0 + r, N - 1) - n0;
        if constexpr (BL == BLay::RAW) boff[t] = gn * LDB + c * 16;
        else if constexpr (BL == BLay::KPANEL) boff[t] = gn * BKB + c * 16;
        else boff[t] = (gn >> 4) * 16 * KB + (gn & 15) * 16 + c * 256;
    }

    // ---- scale sources ----
    const int nblk_last = (N - 1) >> 7;
    const int wave_nblk = min((n0 >> 7) + ((wn * BLK_N * 16) >> 7), nblk_last);
    // MX panels: 8 DMA tasks (A/B x 4 quarters of 64 rows, lane L = row
    // quarter*64 + L); wave w runs tasks w, w+NW, ...
    constexpr int MX_TASKS = 8;
    constexpr int MX_PER_WAVE = (MX_TASKS + NW - 1) / NW;
    const uint8_t* mx_src[MX_PER_WAVE];
    int mx_qq[MX_PER_WAVE];
    bool mx_isb[MX_PER_WAVE], mx_on[MX_PER_WAVE];
#pragma unroll
    for (int u = 0; u < MX_PER_WAVE; ++u) {
        const int task = u * NW + w;
        mx_on[u] = task < MX_TASKS;
        mx_isb[u] = task >= 4;
        mx_qq[u] = task & 3;
        const int row = mx_qq[u] * 64 + L;
        mx_src[u] = (task >= 4) ? SFB + (long long)min(n0 + row, N - 1) * SFB_SN
                                : SFA + (long long)min(m0 + row, M - 1) * SFA_SM;
    }
    auto panel_dma = [&](const uint8_t* src, QG_LDS uint8_t* panel, int qq) {
        if constexpr (PB == 16) {
            dma16(src, panel + qq * 1024);
        } else if constexpr (PB == 4) {
            dma4(src, panel + qq * 256);
        } else {
            dma4(src, panel + qq * 256);
            dma4(src + 4, panel + 1024 + qq * 256);
        }
    };
    // scale byte(s) of (row, lane group q) for K-tile kt: fp8 one byte, fp4
    // the two bytes of groups 2q (byte 0) and 2q+1 (byte 1)
    auto panel_read = [&](const QG_LDS uint8_t* panel, int row, int kt) -> int {
        if constexpr (PB == 16) {
            const QG_LDS uint8_t* p0 = panel + row * 16 + (kt % SPAN) * KT_BYTES;
            if constexpr (FP4) return *(const QG_LDS uint16_t*)(p0 + 2 * q);
            else return p0[q];
        } else if constexpr (PB == 4) {
            return panel[row * 4 + q];
        } else {
            return *(const QG_LDS uint16_t*)(panel + (q >> 1) * 1024 + row * 4 + (q & 1) * 2);
        }
    };
    const uint8_t* bs_src_a = SFA + (SK == ScaleKind::BS8 ? (long long)m0 + 4 * L
                                                          : 4ll * min(m0 + (w & 3) * 64 + L, M - 1) * SFA_SM);
    const long long bs_b_idx = (long long)wave_nblk * SFB_SN;

    // Scale DMAs that go with K-tile kt.  MX: the panel of K-tiles
    // [kt, kt+SPAN) when kt starts a panel (the host picks PB = 16 only when
    // every 16-byte panel lies inside its row and is 16-byte aligned).
    auto issue_scales = [&](int kt, QG_LDS uint8_t* sSA, QG_LDS uint8_t* sSB) {
        if constexpr (MX) {
            if (kt % SPAN == 0) {
                const int buf = (kt / SPAN) & 1;
#pragma unroll
                for (int u = 0; u < MX_PER_WAVE; ++u) {
                    if (!mx_on[u]) continue;
                    QG_LDS uint8_t* panel =
                        (mx_isb[u] ? (QG_LDS uint8_t*)lSB0 : (QG_LDS uint8_t*)lSA0) + buf * PANEL;
                    panel_dma(mx_src[u] + kt * KT_BYTES, panel, mx_qq[u]);
                }
            }
        } else if constexpr (SK == ScaleKind::BS8) {
            // LDS DMA gives every lane a dword slot (lane L -> base + 4L), so
            // bytes move as dwords: SFA's 256 contiguous row bytes of this
            // K-tile in one wave; SFB as the aligned dword holding the byte
            // (an aligned dword never crosses a page, so it stays mapped).
            if (w == 0) dma4(bs_src_a + (long long)kt * SFA_SK, sSA);
            dma4(SFB + ((bs_b_idx + kt) & ~3ll), sSB + w * 256);
        } else {
            if (w < 4) dma4(bs_src_a + 4ll * kt * SFA_SK, sSA + w * 256);
            dma4(SFB + 4 * (bs_b_idx + kt), sSB + w * 256);
        }
    };

    // DMA of K-tile kt into one stage, in BLK_M parts: part j moves the
    // operand rows of this wave's DMAs t with t*BLK_M/DMA_PER_WAVE == j, of
    // A and B (part 0 also the scales).  The parts are issued between the
    // MFMA groups of the previous K-tile, so no wave stalls on a long run
    // of DMA issues while its SIMD's matrix core idles.
    // Operand DMAs go through buffer descriptors whose range is empty when
    // `valid` is false: the DMA then reads nothing and writes zeros into a
    // stage no wave reads again, so the issue needs no branch (a branch would
    // split the schedule the MFMAs are interleaved into).
    auto issue_part = [&](int kt, int j, bool valid, QG_LDS uint8_t* sA, QG_LDS uint8_t* sB,
                          QG_LDS uint8_t* sSA, QG_LDS uint8_t* sSB) {
        const uint8_t* Ak = A + kt * BKB;
        const uint8_t* Bk;
        if constexpr (BL == BLay::RAW) Bk = B + kt * BKB;
        else if constexpr (BL == BLay::KPANEL) Bk = B + (long long)kt * N * BKB;
        else Bk = B + kt * 2048;
        const unsigned nrec = valid ? 0x7FFFFFFFu : 0u;
        const __amdgpu_buffer_rsrc_t rA = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(Ak), 0, nrec, 0x00020000);
        const __amdgpu_buffer_rsrc_t rB = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(Bk), 0, nrec, 0x00020000);
        if (j == 0 && valid) issue_scales(kt, sSA, sSB);
#pragma unroll
        for (int t = 0; t < DMA_PER_WAVE; ++t) {
            if (t * BLK_M / DMA_PER_WAVE != j) continue;
            dma16_buf(rA, sA + (w * DMA_PER_WAVE + t) * 8 * BKB, aoff[t], 0);
            dma16_buf(rB, sB + (w * DMA_PER_WAVE + t) * 8 * BKB, boff[t], 0);
        }
    };
    auto issue = [&](int kt, QG_LDS uint8_t* sA, QG_LDS uint8_t* sB, QG_LDS uint8_t* sSA,
                     QG_LDS uint8_t* sSB) {
#pragma unroll
        for (int j = 0; j < BLK_M; ++j) issue_part(kt, j, true, sA, sB, sSA, sSB);
    };

    f32x4 acc[BLK_M][BLK_N];
#pragma unroll
    for (int i = 0; i < BLK_M; ++i)
#pragma unroll
        for (int j = 0; j < BLK_N; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // per-lane operand read offsets inside a 16-row block:
    // fp8 chunks q and q+4, fp4 chunks 2q and 2q+1 (see the layout note above)
    const int rd0 = l16 * BKB + (((FP4 ? 2 * q : q) ^ swz<FP4>(l16)) << 4);
    const int rd1 = rd0 ^ (FP4 ? 16 : 64);
    const int unit = p.unit_scale;

    auto compute = [&](int kt, const QG_LDS uint8_t* sA, const QG_LDS uint8_t* sB,
                       const QG_LDS uint8_t* sSA, const QG_LDS uint8_t* sSB, auto&& hook) {
        int sa[BLK_M], sb[BLK_N];
        float fs[BLK_M];
        if constexpr (MX) {
            const int buf = ((kt / SPAN) & 1) * PANEL;
            const QG_LDS uint8_t* pa = (const QG_LDS uint8_t*)lSA0 + buf;
            const QG_LDS uint8_t* pb = (const QG_LDS uint8_t*)lSB0 + buf;
#pragma unroll
            for (int i = 0; i < BLK_M; ++i) sa[i] = panel_read(pa, wm * BLK_M * 16 + i * 16 + l16, kt);
#pragma unroll
            for (int j = 0; j < BLK_N; ++j) sb[j] = panel_read(pb, wn * BLK_N * 16 + j * 16 + l16, kt);
        } else if constexpr (SK == ScaleKind::BS8) {
#pragma unroll
            for (int i = 0; i < BLK_M; ++i) sa[i] = sSA[wm * BLK_M * 16 + i * 16 + l16];
            const int s = sSB[w * 256 + (int)((bs_b_idx + kt) & 3)];
#pragma unroll
            for (int j = 0; j < BLK_N; ++j) sb[j] = s;
        } else {
            const float sbv = *(const QG_LDS float*)(sSB + w * 256);
#pragma unroll
            for (int i = 0; i < BLK_M; ++i)
                fs[i] = *(const QG_LDS float*)(sSA + 4 * (wm * BLK_M * 16 + i * 16 + l16)) * sbv;
#pragma unroll
            for (int i = 0; i < BLK_M; ++i) sa[i] = unit;
#pragma unroll
            for (int j = 0; j < BLK_N; ++j) sb[j] = unit;
        }
        // The wave's BLK_N B fragments stay in registers for the K-tile and
        // the A fragments stream through one block at a time (fewer live
        // registers than the other way round, BLK_M >= BLK_N); hook(i) runs
        // before A block i's MFMAs.
        auto read_frag = [&](const QG_LDS uint8_t* blk) -> i32x8 {
            const i32x4 lo = *(const QG_LDS i32x4*)(blk + rd0);
            const i32x4 hi = *(const QG_LDS i32x4*)(blk + rd1);
            return i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        };
        i32x8 bfr[BLK_N];
#pragma unroll
        for (int j = 0; j < BLK_N; ++j) bfr[j] = read_frag(sB + (wn * BLK_N * 16 + j * 16) * BKB);
#pragma unroll
        for (int i = 0; i < BLK_M; ++i) {
            hook(i);
            const i32x8 af = read_frag(sA + (wm * BLK_M * 16 + i * 16) * BKB);
#pragma unroll
            for (int j = 0; j < BLK_N; ++j) {
                const i32x8& bf = bfr[j];
                if constexpr (FP4) {
                    const i32x8 b0 = i32x8{bf[0], bf[1], bf[2], bf[3], 0, 0, 0, 0};
                    const i32x8 b1 = i32x8{bf[4], bf[5], bf[6], bf[7], 0, 0, 0, 0};
                    const i32x8 a0 = i32x8{af[0], af[1], af[2], af[3], 0, 0, 0, 0};
                    const i32x8 a1 = i32x8{af[4], af[5], af[6], af[7], 0, 0, 0, 0};
                    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                        b0, a0, acc[i][j], kFmtFp4, kFmtFp4, 0, sb[j], 0, sa[i]);
                    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                        b1, a1, acc[i][j], kFmtFp4, kFmtFp4, 1, sb[j], 1, sa[i]);
                } else if constexpr (VALU_SCALE) {
                    const f32x4 part = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                        bf, af, f32x4{0.f, 0.f, 0.f, 0.f}, kFmtFp8, kFmtFp8, 0, sb[j], 0, sa[i]);
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[i][j][r] = __builtin_fmaf(part[r], fs[i], acc[i][j][r]);
                } else {
                    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                        bf, af, acc[i][j], kFmtFp8, kFmtFp8, 0, sb[j], 0, sa[i]);
                }
            }
        }
    };

    QG_LDS uint8_t* pA0 = (QG_LDS uint8_t*)lA0;
    QG_LDS uint8_t* pA1 = (QG_LDS uint8_t*)lA1;
    QG_LDS uint8_t* pB0 = (QG_LDS uint8_t*)lB0;
    QG_LDS uint8_t* pB1 = (QG_LDS uint8_t*)lB1;
    QG_LDS uint8_t* pSA0 = (QG_LDS uint8_t*)lSA0;
    QG_LDS uint8_t* pSA1 = (QG_LDS uint8_t*)lSA1;
    QG_LDS uint8_t* pSB0 = (QG_LDS uint8_t*)lSB0;
    QG_LDS uint8_t* pSB1 = (QG_LDS uint8_t*)lSB1;

    // One loop body with a runtime stage select keeps the accumulators
    // resident (two copies of the body make the register allocator shuffle
    // them).  DMA(kt+1) is issued in parts during compute(kt), after the
    // barrier that retires every read of K-tile kt-1 from the same stage.
    // The barrier is s_barrier
    // behind an explicit lgkmcnt(0): __syncthreads() would also wait for the
    // LDS DMA issued just before (vmcnt(0)) on the next iteration's path.
    const int nk = KB / BKB;
    issue(0, pA0, pB0, pSA0, pSB0);
    for (int kt = 0; kt < nk; ++kt) {
        wait_vmcnt<0>();
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        const int s = kt & 1;
        const bool more = kt + 1 < nk;
        QG_LDS uint8_t* nA = s ? pA0 : pA1;
        QG_LDS uint8_t* nB = s ? pB0 : pB1;
        QG_LDS uint8_t* nSA = s ? pSA0 : pSA1;
        QG_LDS uint8_t* nSB = s ? pSB0 : pSB1;
        compute(kt, s ? pA1 : pA0, s ? pB1 : pB0, s ? pSA1 : pSA0, s ? pSB1 : pSB0, [&](int j) {
            issue_part(kt + 1, j, more, nA, nB, nSA, nSB);
        });
    }

    // ---- epilogue: lane holds C[m][n..n+3] for each (i, j) block ----
    const int mrow0 = m0 + wm * BLK_M * 16 + l16;
    const int ncol0 = n0 + wn * BLK_N * 16 + 4 * q;
    const bool vec_ok = (LDC & 3) == 0;
#pragma unroll
    for (int i = 0; i < BLK_M; ++i) {
        const int mm = mrow0 + i * 16;
        if (mm < M) {
#pragma unroll
            for (int j = 0; j < BLK_N; ++j) {
                const int nn = ncol0 + j * 16;
                const f32x4 v = acc[i][j];
                if constexpr (BF16) {
                    uint16_t* crow = (uint16_t*)p.c + bz * p.c_batch + (long long)mm * LDC;
                    if (vec_ok && nn + 3 < N) {
                        *(u32x2*)(crow + nn) = u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
                    } else {
                        for (int r = 0; r < 4; ++r)
                            if (nn + r < N) crow[nn + r] = bf16_bits(v[r]);
                    }
                } else {
                    float* crow = (float*)p.c + bz * p.c_batch + (long long)mm * LDC;
                    if (vec_ok && nn + 3 < N) {
                        *(f32x4*)(crow + nn) = v;
                    } else {
                        for (int r = 0; r < 4; ++r)
                            if (nn + r < N) crow[nn + r] = v[r];
                    }
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

}  // namespace qg
