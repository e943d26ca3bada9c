// LDS-staged tile GEMM for gfx950 on the scaled MFMA 32x32x64.
//
// One workgroup of 8 wave64 (2 per SIMD) computes a 256 x 256 tile of C on
// v_mfma_scale_f32_32x32x64_f8f6f4.  The K loop walks 128-byte K-tiles,
// moved global -> LDS by DMA (global_load_lds_dwordx4) into two LDS stages:
// the copy of K-tile t+1 is in flight while K-tile t is multiplied, and one
// barrier per K-tile retires a stage.  The library runs the fp32 block-scale
// policy (BSF32) here: its VALU rescale of every partial product keeps the
// accumulators in VGPRs, which the 8-wave layout (128 accumulators per
// wave) leaves room for; the MFMA-scaled policies run on the four-wave
// kernel (wide_gemm.hpp).  Scale policies and B layouts: tile_args.hpp.
//
// Register layout (pinned by the layout probes, csrc/probe.hip):
//   * operand lane L = 32g + r holds row r; lanes r and 32 + r split K;
//   * fp8 (K = 64 per instruction, two E8M0 blocks of 32): dwords 0-3 of lane
//     group g hold K [16g, 16g+16) and dwords 4-7 hold K [32+16g, 32+16g+16);
//     block b's scale comes from lane group b.  A lane therefore fetches
//     16-byte chunks g and 2+g of each 64-byte sub-tile;
//   * fp4 (K = 64 per instruction = 32 bytes): dwords 0-3 of lane group g hold
//     K [32g, 32g+32), i.e. 16-byte chunk g of the sub-tile, scaled by its
//     own lane group's byte;
//   * accumulator register v of lane L holds D[i][j] with srcA row
//     i = 8(v/4) + 4(L/32) + v%4 and srcB row j = L%32.  With srcA = B and
//     srcB = A the lane holds C[m = L%32][n = 8c + 4g + 0..3], c = 0..3.
// A 128-byte K-tile is 2 (fp8) or 4 (fp4) instructions per 32 x 32 block.
// The E8M0 byte of each instruction comes from a per-lane register whose
// bytes 0 and 2 hold the lane group's blocks of two consecutive sub-tiles
// (one shift per K-tile and operand block), selected with op_sel.
//
// LDS rows are 128 bytes with 16-byte chunks XOR-swizzled by (row >> 1) & 7:
// a 16-lane read phase covers rows r..r+15 of one chunk and hits 16 distinct
// bank groups.
#pragma once
#include <utility>

#include "tile_args.hpp"

namespace qg {

typedef float f32x16 __attribute__((ext_vector_type(16)));

// 8 waves: 2 x 4 waves of 128 x 64 (hardware-scaled policies) or 4 x 2 waves
// of 64 x 128 (BSF32); blocks of 32 x 32.
template <ScaleKind SK>
struct Tile32Shape {
    static constexpr int WAVES_M = 2, WAVES_N = 4, BLK_M = 4, BLK_N = 2;
};
template <>
struct Tile32Shape<ScaleKind::BSF32> {
    static constexpr int WAVES_M = 4, WAVES_N = 2, BLK_M = 2, BLK_N = 4;
};

__device__ __forceinline__ int swz32(int r) { return (r >> 1) & 7; }

template <int N, class F, int... I>
__device__ __forceinline__ void unroll_impl(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
// f(std::integral_constant<int, i>) for i = 0 .. N-1, unrolled at compile time.
template <int N, class F>
__device__ __forceinline__ void unroll(F&& f) {
    unroll_impl<N>(f, std::make_integer_sequence<int, N>{});
}

template <int FMT, ScaleKind SK, BLay BL, bool BF16, int PB = 16>
__global__ __launch_bounds__(512, 1) void tile32_gemm_kernel(const TileArgs p) {
    using Shape = Tile32Shape<SK>;
    constexpr int WAVES_N = Shape::WAVES_N, WAVES_M = Shape::WAVES_M;
    constexpr int BLK_M = Shape::BLK_M, BLK_N = Shape::BLK_N;
    constexpr int NW = WAVES_M * WAVES_N;
    constexpr int BM = WAVES_M * BLK_M * 32, BN = WAVES_N * BLK_N * 32, BKB = 128;
    static_assert(BM == 256 && BN == 256 && NW == 8, "tile is 256 x 256, 8 waves");
    constexpr int DMA_PER_WAVE = BM / 8 / NW;
    constexpr bool FP4 = (FMT == kFmtFp4);
    constexpr bool MX = (SK == ScaleKind::MX);
    constexpr bool VALU_SCALE = (SK == ScaleKind::BSF32);
    constexpr int NS = FP4 ? 4 : 2;          // instructions (K sub-tiles) per 128-byte K-tile
    constexpr int KT_BYTES = FP4 ? 8 : 4;    // MX scale bytes per row per K-tile
    static_assert(PB == 16 || PB == KT_BYTES, "panel width");
    constexpr int SPAN = PB / KT_BYTES;
    constexpr int PANEL = 256 * 16;
    constexpr int SA_BYTES = MX ? 2 * PANEL : (SK == ScaleKind::BS8 ? 256 : 1024);
    constexpr int SB_BYTES = MX ? 2 * PANEL : 256 * NW;

    __shared__ __attribute__((aligned(1024))) uint8_t lA0[BM * BKB];
    __shared__ __attribute__((aligned(1024))) uint8_t lA1[BM * BKB];
    __shared__ __attribute__((aligned(1024))) uint8_t lB0[BN * BKB];
    __shared__ __attribute__((aligned(1024))) uint8_t lB1[BN * BKB];
    __shared__ __attribute__((aligned(256))) uint8_t lSA0[SA_BYTES];
    __shared__ __attribute__((aligned(256))) uint8_t lSA1[MX ? 16 : SA_BYTES];
    __shared__ __attribute__((aligned(256))) uint8_t lSB0[SB_BYTES];
    __shared__ __attribute__((aligned(256))) uint8_t lSB1[MX ? 16 : SB_BYTES];

    // ---- tile coordinates: XCD-contiguous remap, then grouped raster ----
    const int T = p.tiles_m * p.tiles_n;
    int bid = blockIdx.x;
    if ((T & 7) == 0) bid = (bid & 7) * (T >> 3) + (bid >> 3);
    const int gfull = p.group_m * p.tiles_n;
    const int gidx = bid / gfull;
    const int first_m = gidx * p.group_m;
    const int gm = min(p.tiles_m - first_m, p.group_m);
    const int within = bid - gidx * gfull;
    const int tm = first_m + within % gm;
    const int tn = within / gm;
    const int bz = blockIdx.z;
    const int m0 = tm * BM, n0 = tn * BN;

    // kernel arguments copied into locals once: lambdas must not read the
    // argument block inside the K loop (vector loads whose vmcnt wait would
    // also drain the DMA queue)
    const int M = p.m, N = p.n, KB = p.kbytes, LDA = p.lda, LDB = p.ldb, LDC = p.ldc;
    const int SFA_SM = p.sfa_sm, SFA_SK = p.sfa_sk, SFB_SN = p.sfb_sn;

    const int tid = threadIdx.x;
    const int w = tid >> 6, L = tid & 63;
    const int wm = w / WAVES_N, wn = w % WAVES_N;
    const int g = L >> 5, l32 = L & 31;

    const uint8_t* A = p.a + bz * p.a_batch + (long long)m0 * LDA;
    const uint8_t* B = p.b + bz * p.b_batch;
    const uint8_t* SFA = p.sfa + bz * p.sfa_batch * (VALU_SCALE ? 4 : 1);
    const uint8_t* SFB = p.sfb + bz * p.sfb_batch * (VALU_SCALE ? 4 : 1);

    // ---- per-lane DMA source offsets: lane L writes row +L/8, physical
    // chunk L%8 = logical chunk (L%8) ^ swz32(row)
    int aoff[DMA_PER_WAVE], boff[DMA_PER_WAVE];
#pragma unroll
    for (int t = 0; t < DMA_PER_WAVE; ++t) {
        const int r = (w * DMA_PER_WAVE + t) * 8 + (L >> 3);
        const int c = (L & 7) ^ swz32(r);
        aoff[t] = (min(m0 + r, M - 1) - m0) * LDA + c * 16;
        const int gn = min(n0 + r, N - 1);
        if constexpr (BL == BLay::RAW) boff[t] = gn * LDB + c * 16;
        else if constexpr (BL == BLay::KPANEL) boff[t] = gn * BKB + c * 16;
        else boff[t] = (gn >> 4) * 16 * KB + (gn & 15) * 16 + c * 256;
    }

    // ---- scale sources ----
    const int nblk_last = (N - 1) >> 7;
    const int wave_nblk = min((n0 >> 7) + ((wn * BLK_N * 32) >> 7), nblk_last);
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
    // the lane group's scale bytes of K-tile kt for one row, arranged for
    // op_sel: word h (fp4: h = 0, 1) holds blocks (4h + g) in byte 0 and
    // (4h + 2 + g) in byte 2 -> instruction s uses word s/2, byte 2*(s%2)
    auto panel_read = [&](const QG_LDS uint8_t* panel, int row, int kt, int* out) {
        if constexpr (PB == 16) {
            const QG_LDS uint8_t* p0 = panel + row * 16 + (kt % SPAN) * KT_BYTES;
            out[0] = (int)(*(const QG_LDS uint32_t*)p0 >> (8 * g));
            if constexpr (FP4) out[1] = (int)(*(const QG_LDS uint32_t*)(p0 + 4) >> (8 * g));
        } else if constexpr (PB == 4) {
            out[0] = (int)(*(const QG_LDS uint32_t*)(panel + row * 4) >> (8 * g));
        } else {
            out[0] = (int)(*(const QG_LDS uint32_t*)(panel + row * 4) >> (8 * g));
            out[1] = (int)(*(const QG_LDS uint32_t*)(panel + 1024 + row * 4) >> (8 * g));
        }
    };
    const uint8_t* bs_src_a = SFA + (SK == ScaleKind::BS8 ? (long long)m0 + 4 * L
                                                          : 4ll * min(m0 + (w & 3) * 64 + L, M - 1) * SFA_SM);
    const long long bs_b_idx = (long long)wave_nblk * SFB_SN;

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
            if (w == 0) dma4(bs_src_a + (long long)kt * SFA_SK, sSA);
            dma4(SFB + ((bs_b_idx + kt) & ~3ll), sSB + w * 256);
        } else {
            if (w < 4) dma4(bs_src_a + 4ll * kt * SFA_SK, sSA + w * 256);
            dma4(SFB + 4 * (bs_b_idx + kt), sSB + w * 256);
        }
    };

    auto issue = [&](int kt, QG_LDS uint8_t* sA, QG_LDS uint8_t* sB, QG_LDS uint8_t* sSA,
                     QG_LDS uint8_t* sSB) {
        const uint8_t* Ak = A + kt * BKB;
        const uint8_t* Bk;
        if constexpr (BL == BLay::RAW) Bk = B + kt * BKB;
        else if constexpr (BL == BLay::KPANEL) Bk = B + (long long)kt * N * BKB;
        else Bk = B + kt * 2048;
#pragma unroll
        for (int t = 0; t < DMA_PER_WAVE; ++t) dma16(Ak + aoff[t], sA + (w * DMA_PER_WAVE + t) * 8 * BKB);
#pragma unroll
        for (int t = 0; t < DMA_PER_WAVE; ++t) dma16(Bk + boff[t], sB + (w * DMA_PER_WAVE + t) * 8 * BKB);
        issue_scales(kt, sSA, sSB);
    };

    f32x16 acc[BLK_M][BLK_N];
#pragma unroll
    for (int i = 0; i < BLK_M; ++i)
#pragma unroll
        for (int j = 0; j < BLK_N; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

    // per-lane operand read offsets inside a 32-row block (row l32): chunk
    // of instruction s and dword half h
    auto chunk_of = [&](int s, int h) { return FP4 ? 2 * s + g : 4 * s + 2 * h + g; };
    auto rd_off = [&](int s, int h) { return l32 * BKB + ((chunk_of(s, h) ^ swz32(l32)) << 4); };
    const int unit = p.unit_scale;

    auto load_frag = [&](const QG_LDS uint8_t* blk, int s) -> i32x8 {
        const i32x4 lo = *(const QG_LDS i32x4*)(blk + rd_off(s, 0));
        if constexpr (FP4) {
            return i32x8{lo[0], lo[1], lo[2], lo[3], 0, 0, 0, 0};
        } else {
            const i32x4 hi = *(const QG_LDS i32x4*)(blk + rd_off(s, 1));
            return i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
    };

    auto compute = [&](int kt, const QG_LDS uint8_t* sA, const QG_LDS uint8_t* sB,
                       const QG_LDS uint8_t* sSA, const QG_LDS uint8_t* sSB) {
        int sa[BLK_M][2], sb[BLK_N][2];
        float fs[BLK_M];
        if constexpr (MX) {
            const int buf = ((kt / SPAN) & 1) * PANEL;
            const QG_LDS uint8_t* pa = (const QG_LDS uint8_t*)lSA0 + buf;
            const QG_LDS uint8_t* pb = (const QG_LDS uint8_t*)lSB0 + buf;
#pragma unroll
            for (int i = 0; i < BLK_M; ++i) panel_read(pa, wm * BLK_M * 32 + i * 32 + l32, kt, sa[i]);
#pragma unroll
            for (int j = 0; j < BLK_N; ++j) panel_read(pb, wn * BLK_N * 32 + j * 32 + l32, kt, sb[j]);
        } else if constexpr (SK == ScaleKind::BS8) {
            // one scale per 128-element K-tile: the byte in every op_sel position
#pragma unroll
            for (int i = 0; i < BLK_M; ++i) sa[i][0] = sa[i][1] = sSA[wm * BLK_M * 32 + i * 32 + l32] * 0x01010101;
            const int s = sSB[w * 256 + (int)((bs_b_idx + kt) & 3)] * 0x01010101;
#pragma unroll
            for (int j = 0; j < BLK_N; ++j) sb[j][0] = sb[j][1] = s;
        } else {
            const float sbv = *(const QG_LDS float*)(sSB + w * 256);
#pragma unroll
            for (int i = 0; i < BLK_M; ++i)
                fs[i] = *(const QG_LDS float*)(sSA + 4 * (wm * BLK_M * 32 + i * 32 + l32)) * sbv;
#pragma unroll
            for (int i = 0; i < BLK_M; ++i) sa[i][0] = sa[i][1] = unit;
#pragma unroll
            for (int j = 0; j < BLK_N; ++j) sb[j][0] = sb[j][1] = unit;
        }
        i32x8 af[BLK_M][NS];
#pragma unroll
        for (int i = 0; i < BLK_M; ++i) {
            const QG_LDS uint8_t* blk = sA + (wm * BLK_M * 32 + i * 32) * BKB;
#pragma unroll
            for (int s = 0; s < NS; ++s) af[i][s] = load_frag(blk, s);
        }
#pragma unroll
        for (int j = 0; j < BLK_N; ++j) {
            const QG_LDS uint8_t* blk = sB + (wn * BLK_N * 32 + j * 32) * BKB;
            i32x8 bf[NS];
#pragma unroll
            for (int s = 0; s < NS; ++s) bf[s] = load_frag(blk, s);
#pragma unroll
            for (int i = 0; i < BLK_M; ++i) {
                if constexpr (VALU_SCALE) {
                    f32x16 part;
#pragma unroll
                    for (int v = 0; v < 16; ++v) part[v] = 0.f;
                    unroll<NS>([&](auto sc) {
                        constexpr int s = decltype(sc)::value;
                        part = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(bf[s], af[i][s], part, FMT, FMT, 0,
                                                                                unit, 0, unit);
                    });
#pragma unroll
                    for (int v = 0; v < 16; ++v) acc[i][j][v] = __builtin_fmaf(part[v], fs[i], acc[i][j][v]);
                } else {
                    unroll<NS>([&](auto sc) {
                        constexpr int s = decltype(sc)::value;
                        constexpr int OPS = 2 * (s & 1);    // byte 0 or 2 of word s/2
                        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                            bf[s], af[i][s], acc[i][j], FMT, FMT, OPS, sb[j][s >> 1], OPS, sa[i][s >> 1]);
                    });
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
    // them).  DMA(kt+1) goes right after the barrier that retires the reads
    // of kt-1; the barrier is s_barrier behind explicit waits, because
    // __syncthreads() would also drain the DMA just issued.
    const int nk = KB / BKB;
    issue(0, pA0, pB0, pSA0, pSB0);
    for (int kt = 0; kt < nk; ++kt) {
        wait_vmcnt<0>();
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        const int s = kt & 1;
        if (kt + 1 < nk) issue(kt + 1, s ? pA0 : pA1, s ? pB0 : pB1, s ? pSA0 : pSA1, s ? pSB0 : pSB1);
        compute(kt, s ? pA1 : pA0, s ? pB1 : pB0, s ? pSA1 : pSA0, s ? pSB1 : pSB0);
    }

    // ---- epilogue: lane holds C[m][n .. n+3] for n = 8c + 4g, c = 0..3, per block ----
    const int mrow0 = m0 + wm * BLK_M * 32 + l32;
    const int ncol0 = n0 + wn * BLK_N * 32 + 4 * g;
    const bool vec_ok = (LDC & 3) == 0;
#pragma unroll
    for (int i = 0; i < BLK_M; ++i) {
        const int mm = mrow0 + i * 32;
        if (mm < M) {
#pragma unroll
            for (int j = 0; j < BLK_N; ++j) {
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int nn = ncol0 + j * 32 + 8 * c;
                    const f32x4 v = {acc[i][j][4 * c], acc[i][j][4 * c + 1], acc[i][j][4 * c + 2],
                                     acc[i][j][4 * c + 3]};
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
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

}  // namespace qg
