// LDS-staged tile GEMM for gfx950 on the scaled MFMA 16x16x128.
//
// One workgroup computes a 256 x 256 tile of C.  The K loop walks 128-byte
// K-tiles (128 e4m3 or 256 e2m1 values per row):
//   * global -> LDS by DMA (global_load_lds_dwordx4), two LDS stages; the
//     copy of K-tile t+1 is in flight while K-tile t is multiplied;
//   * each 128-byte LDS row is XOR-swizzled per 16-byte chunk (common.hpp:
//     swz) so that the per-lane 32-byte operand reads are conflict free;
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
//         MX4 host.cc:207-208): fp8 uses byte q of the K-tile's 4 groups; fp4
//         uses groups 2q and 2q+1 of its 8 (first and second MFMA).
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

template <ScaleKind SK>
struct TileShape {
    static constexpr int WAVES_M = 2, WAVES_N = 2, BLK_M = 8, BLK_N = 8;
};
template <>
struct TileShape<ScaleKind::BSF32> {
    static constexpr int WAVES_M = 4, WAVES_N = 2, BLK_M = 4, BLK_N = 8;
};

template <ScaleKind SK>
constexpr int tile_threads() {
    return 64 * TileShape<SK>::WAVES_M * TileShape<SK>::WAVES_N;
}

template <int FMT, ScaleKind SK, BLay BL, bool BF16>
__global__ __launch_bounds__(tile_threads<SK>(), 1) void tile_gemm_kernel(const TileArgs p) {
    using Shape = TileShape<SK>;
    constexpr int WAVES_N = Shape::WAVES_N, WAVES_M = Shape::WAVES_M;
    constexpr int BLK_M = Shape::BLK_M, BLK_N = Shape::BLK_N;
    constexpr int NW = WAVES_M * WAVES_N;
    constexpr int BM = WAVES_M * BLK_M * 16, BN = WAVES_N * BLK_N * 16, BKB = 128;
    static_assert(BM == 256 && BN == 256, "tile is 256 x 256");
    constexpr int DMA_PER_WAVE = BM / 8 / NW;  // 16-byte-per-lane DMAs per operand
    constexpr bool FP4 = (FMT == kFmtFp4);
    constexpr bool VALU_SCALE = (SK == ScaleKind::BSF32);
    // LDS scale panels per stage
    constexpr int SA_BYTES = (SK == ScaleKind::MX) ? (FP4 ? 2048 : 1024) : (SK == ScaleKind::BS8 ? 256 : 1024);
    constexpr int SB_BYTES = (SK == ScaleKind::MX) ? SA_BYTES : 256 * NW;

    __shared__ __attribute__((aligned(1024))) uint8_t lA0[BM * BKB];
    __shared__ __attribute__((aligned(1024))) uint8_t lA1[BM * BKB];
    __shared__ __attribute__((aligned(1024))) uint8_t lB0[BN * BKB];
    __shared__ __attribute__((aligned(1024))) uint8_t lB1[BN * BKB];
    __shared__ __attribute__((aligned(256))) uint8_t lSA0[SA_BYTES];
    __shared__ __attribute__((aligned(256))) uint8_t lSA1[SA_BYTES];
    __shared__ __attribute__((aligned(256))) uint8_t lSB0[SB_BYTES];
    __shared__ __attribute__((aligned(256))) uint8_t lSB1[SB_BYTES];

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

    const int tid = threadIdx.x;
    const int w = tid >> 6, L = tid & 63;
    const int wm = w / WAVES_N, wn = w % WAVES_N;
    const int q = L >> 4, l16 = L & 15;

    const uint8_t* A = p.a + bz * p.a_batch + (long long)m0 * p.lda;
    const uint8_t* B = p.b + bz * p.b_batch;
    const uint8_t* SFA = p.sfa + bz * p.sfa_batch * (VALU_SCALE ? 4 : 1);
    const uint8_t* SFB = p.sfb + bz * p.sfb_batch * (VALU_SCALE ? 4 : 1);

    // ---- per-lane DMA source offsets ----
    // DMA t of wave w fills LDS rows (w*DMA_PER_WAVE + t)*8 .. +8; lane L
    // writes row +L/8, physical chunk L%8 = logical chunk (L%8) ^ swz(row).
    int aoff[DMA_PER_WAVE], boff[DMA_PER_WAVE];
#pragma unroll
    for (int t = 0; t < DMA_PER_WAVE; ++t) {
        const int r = (w * DMA_PER_WAVE + t) * 8 + (L >> 3);
        const int c = (L & 7) ^ swz(r);
        aoff[t] = (min(m0 + r, p.m - 1) - m0) * p.lda + c * 16;
        const int gn = min(n0 + r, p.n - 1);
        if constexpr (BL == BLay::RAW) boff[t] = gn * p.ldb + c * 16;
        else if constexpr (BL == BLay::KPANEL) boff[t] = gn * BKB + c * 16;
        else boff[t] = (gn >> 4) * 16 * p.kbytes + (gn & 15) * 16 + c * 256;
    }

    // ---- scale DMA tasks (wave-uniform branches) ----
    // quarter = 64 consecutive tile rows, one DMA lane per row.
    const int nblk_last = (p.n - 1) >> 7;
    const int wave_nblk = min((n0 >> 7) + ((wn * BLK_N * 16) >> 7), nblk_last);
    auto issue_scales = [&](int kt, QG_LDS uint8_t* sSA, QG_LDS uint8_t* sSB) {
        if constexpr (SK == ScaleKind::MX) {
            constexpr int HALVES = FP4 ? 2 : 1;            // dwords per row per K-tile
            constexpr int TASKS = 2 * 4 * HALVES;         // {A,B} x quarter x half
#pragma unroll
            for (int task0 = 0; task0 < TASKS; task0 += NW) {
                const int task = task0 + w;
                if (task < TASKS) {
                    const int isb = task / (4 * HALVES);
                    const int qq = (task / HALVES) % 4;
                    const int h = task % HALVES;
                    const int row = qq * 64 + L;
                    if (isb == 0) {
                        const int gr = min(m0 + row, p.m - 1);
                        dma4(SFA + (long long)gr * p.sfa_sm + kt * 4 * HALVES + 4 * h, sSA + h * 1024 + qq * 256);
                    } else {
                        const int gr = min(n0 + row, p.n - 1);
                        dma4(SFB + (long long)gr * p.sfb_sn + kt * 4 * HALVES + 4 * h, sSB + h * 1024 + qq * 256);
                    }
                }
            }
        } else if constexpr (SK == ScaleKind::BS8) {
            // LDS DMA gives every lane a dword slot (lane L -> base + 4L), so
            // bytes move as dwords: SFA's 256 contiguous row bytes of this
            // K-tile in one wave; SFB as the aligned dword holding the byte
            // (an aligned dword never crosses a page, so it stays mapped).
            if (w == 0) dma4(SFA + (long long)kt * p.sfa_sk + m0 + 4 * L, sSA);
            const long long bidx = (long long)wave_nblk * p.sfb_sn + kt;
            dma4(SFB + (bidx & ~3ll), sSB + w * 256);
        } else {
            if (w < 4) {
                const int gr = min(m0 + w * 64 + L, p.m - 1);
                dma4(SFA + 4 * ((long long)kt * p.sfa_sk + (long long)gr * p.sfa_sm), sSA + w * 256);
            }
            dma4(SFB + 4 * ((long long)wave_nblk * p.sfb_sn + kt), sSB + w * 256);
        }
    };

    auto issue = [&](int kt, QG_LDS uint8_t* sA, QG_LDS uint8_t* sB, QG_LDS uint8_t* sSA,
                     QG_LDS uint8_t* sSB) {
        const uint8_t* Ak = A + kt * BKB;
        const uint8_t* Bk;
        if constexpr (BL == BLay::RAW) Bk = B + kt * BKB;
        else if constexpr (BL == BLay::KPANEL) Bk = B + (long long)kt * p.n * BKB;
        else Bk = B + kt * 2048;
#pragma unroll
        for (int t = 0; t < DMA_PER_WAVE; ++t) dma16(Ak + aoff[t], sA + (w * DMA_PER_WAVE + t) * 8 * BKB);
#pragma unroll
        for (int t = 0; t < DMA_PER_WAVE; ++t) dma16(Bk + boff[t], sB + (w * DMA_PER_WAVE + t) * 8 * BKB);
        issue_scales(kt, sSA, sSB);
    };

    f32x4 acc[BLK_M][BLK_N];
#pragma unroll
    for (int i = 0; i < BLK_M; ++i)
#pragma unroll
        for (int j = 0; j < BLK_N; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // per-lane operand read offsets inside a 16-row block:
    // fp8 chunks q and q+4, fp4 chunks 2q and 2q+1 (see the layout note above)
    const int rd0 = l16 * BKB + (((FP4 ? 2 * q : q) ^ swz(l16)) << 4);
    const int rd1 = rd0 ^ (FP4 ? 16 : 64);
    const int unit = p.unit_scale;

    auto compute = [&](int kt_cur, const QG_LDS uint8_t* sA, const QG_LDS uint8_t* sB,
                       const QG_LDS uint8_t* sSA, const QG_LDS uint8_t* sSB) {
        int sa[BLK_M], sb[BLK_N];
        float fs[BLK_M];
        if constexpr (SK == ScaleKind::MX) {
#pragma unroll
            for (int i = 0; i < BLK_M; ++i) {
                const int ra = wm * BLK_M * 16 + i * 16 + l16;
                if constexpr (FP4) sa[i] = *(const QG_LDS uint16_t*)(sSA + (q >> 1) * 1024 + ra * 4 + (q & 1) * 2);
                else sa[i] = sSA[ra * 4 + q];
            }
#pragma unroll
            for (int j = 0; j < BLK_N; ++j) {
                const int rb = wn * BLK_N * 16 + j * 16 + l16;
                if constexpr (FP4) sb[j] = *(const QG_LDS uint16_t*)(sSB + (q >> 1) * 1024 + rb * 4 + (q & 1) * 2);
                else sb[j] = sSB[rb * 4 + q];
            }
        } else if constexpr (SK == ScaleKind::BS8) {
#pragma unroll
            for (int i = 0; i < BLK_M; ++i) sa[i] = sSA[wm * BLK_M * 16 + i * 16 + l16];
            const int s = sSB[w * 256 + (int)(((long long)wave_nblk * p.sfb_sn + kt_cur) & 3)];
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
        i32x8 af[BLK_M];
#pragma unroll
        for (int i = 0; i < BLK_M; ++i) {
            const QG_LDS uint8_t* blk = sA + (wm * BLK_M * 16 + i * 16) * BKB;
            const i32x4 lo = *(const QG_LDS i32x4*)(blk + rd0);
            const i32x4 hi = *(const QG_LDS i32x4*)(blk + rd1);
            af[i] = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
#pragma unroll
        for (int j = 0; j < BLK_N; ++j) {
            const QG_LDS uint8_t* blk = sB + (wn * BLK_N * 16 + j * 16) * BKB;
            const i32x4 lo = *(const QG_LDS i32x4*)(blk + rd0);
            const i32x4 hi = *(const QG_LDS i32x4*)(blk + rd1);
#pragma unroll
            for (int i = 0; i < BLK_M; ++i) {
                if constexpr (FP4) {
                    const i32x8 b0 = i32x8{lo[0], lo[1], lo[2], lo[3], 0, 0, 0, 0};
                    const i32x8 b1 = i32x8{hi[0], hi[1], hi[2], hi[3], 0, 0, 0, 0};
                    const i32x8 a0 = i32x8{af[i][0], af[i][1], af[i][2], af[i][3], 0, 0, 0, 0};
                    const i32x8 a1 = i32x8{af[i][4], af[i][5], af[i][6], af[i][7], 0, 0, 0, 0};
                    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                        b0, a0, acc[i][j], kFmtFp4, kFmtFp4, 0, sb[j], 0, sa[i]);
                    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                        b1, a1, acc[i][j], kFmtFp4, kFmtFp4, 1, sb[j], 1, sa[i]);
                } else {
                    const i32x8 bf = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                    if constexpr (VALU_SCALE) {
                        const f32x4 part = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                            bf, af[i], f32x4{0.f, 0.f, 0.f, 0.f}, kFmtFp8, kFmtFp8, 0, sb[j], 0, sa[i]);
#pragma unroll
                        for (int r = 0; r < 4; ++r) acc[i][j][r] = __builtin_fmaf(part[r], fs[i], acc[i][j][r]);
                    } else {
                        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                            bf, af[i], acc[i][j], kFmtFp8, kFmtFp8, 0, sb[j], 0, sa[i]);
                    }
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
    // them).  DMA(kt+1) is issued right after the barrier that retires every
    // read of K-tile kt-1 from the same stage.
    const int nk = p.kbytes / BKB;
    issue(0, pA0, pB0, pSA0, pSB0);
    for (int kt = 0; kt < nk; ++kt) {
        wait_vmcnt<0>();
        __syncthreads();
        const int s = kt & 1;
        if (kt + 1 < nk) issue(kt + 1, s ? pA0 : pA1, s ? pB0 : pB1, s ? pSA0 : pSA1, s ? pSB0 : pSB1);
        compute(kt, s ? pA1 : pA0, s ? pB1 : pB0, s ? pSA1 : pSA0, s ? pSB1 : pSB0);
    }

    // ---- epilogue: lane holds C[m][n..n+3] for each (i, j) block ----
    const int mrow0 = m0 + wm * BLK_M * 16 + l16;
    const int ncol0 = n0 + wn * BLK_N * 16 + 4 * q;
    const bool vec_ok = (p.ldc & 3) == 0;
#pragma unroll
    for (int i = 0; i < BLK_M; ++i) {
        const int mm = mrow0 + i * 16;
        if (mm >= p.m) continue;
#pragma unroll
        for (int j = 0; j < BLK_N; ++j) {
            const int nn = ncol0 + j * 16;
            const f32x4 v = acc[i][j];
            if constexpr (BF16) {
                uint16_t* crow = (uint16_t*)p.c + bz * p.c_batch + (long long)mm * p.ldc;
                if (vec_ok && nn + 3 < p.n) {
                    *(u32x2*)(crow + nn) = u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
                } else {
                    for (int r = 0; r < 4; ++r)
                        if (nn + r < p.n) crow[nn + r] = (uint16_t)bf16_rne_bits(v[r]);
                }
            } else {
                float* crow = (float*)p.c + bz * p.c_batch + (long long)mm * p.ldc;
                if (vec_ok && nn + 3 < p.n) {
                    *(f32x4*)(crow + nn) = v;
                } else {
                    for (int r = 0; r < 4; ++r)
                        if (nn + r < p.n) crow[nn + r] = v[r];
                }
            }
        }
    }
}

}  // namespace qg
