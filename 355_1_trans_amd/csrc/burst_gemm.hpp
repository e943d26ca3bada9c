// Burst GEMM for decode shapes (M <= 64) on gfx950: every global load of a
// workgroup's K slice is issued in one burst.  fp8 with fp32 block scales
// (K-panel B' or fragment-order B''), MXFP8 / MXFP4 with row-major B and
// row-major E8M0 scales, or MXFP4 in aiter's bpreshuffle formats: B in
// shuffle_weight(16,16) order (for fp4 the same bytes as B'': a 16-row
// block's K-tile is the two 1 KB operands of the 16x16x128 MFMA) and both
// scale tensors in e8m0_shuffle order.
//
// A decode GEMM streams B once; at configs[0] size (11 MB) the whole launch
// lasts a few microseconds, so what bounds it is how many bytes are in flight
// at once, not a steady-state rate.  Measured on MI355X (graph-replayed
// launches over rotating copies of an 11 MB operand): a launch that issues
// all of its 16-byte whole-line loads up front streams in 3.1 us; loading in
// the scaled MFMA's fragment order (16 rows x 64 B per instruction, every
// 128-byte line requested twice) takes 3.6 us; LDS DMAs issued by few
// workgroups 4.5-6 us; an empty kernel 1.8 us.  Hence:
//
//  * a workgroup (4, 8 or 16 waves) owns NB*16 columns and all ROWS = MB*16
//    rows of one K slice; wave w takes a contiguous run of the slice's
//    K-tiles.  Splitting K over the waves of one workgroup costs an LDS
//    reduction; splitting it over workgroups costs ~2.5 us more per launch
//    (the partial stores, the counter and the last workgroup's loads are
//    device-coherent round trips, one after the other), so the host
//    splits over workgroups only when 16 waves cannot cover K;
//  * each wave issues all its loads before any compute: per 128-byte K-tile,
//    B's 16-row blocks (two whole-line 1 KB loads each, or, for the
//    fragment-order B'', the two 1 KB halves that already are the MFMA
//    operands), A's rows (whole lines, from L2: every N tile re-reads A) and
//    the fp32 block scales -- into registers;
//  * per K-tile the wave writes its A (and B' or row-major B) lines into its
//    own LDS slot, XOR-swizzled, and reads them back as 16x16x128 fragments
//    (the LDS unit executes one wave's accesses in order, so one slot serves
//    every K-tile with no barrier); fp32 block scales: unscaled MFMA partials
//    rescaled in VALU, acc += part * (sa * sb), the reference's
//    scale-then-sum order; MX: the E8M0 bytes ride on the scaled MFMA (fp8:
//    one instruction per K-tile, the lane group's byte of the row's 4; fp4:
//    two, chunks q and q + 4, bytes q and q + 4 of the row's 8);
//  * the waves' partial tiles meet in LDS and are summed in wave order;
//  * K is split over workgroups (grid.x = n_tiles * splitk): fp32 partial
//    tiles with device-coherent stores, one relaxed counter atomic per
//    workgroup, and the last workgroup sums the slices in slice order with
//    all of its waves (deterministic, one launch; see common.hpp).
//
// Register layout of the scaled MFMA 16x16x128 (probe.hip): operand lane
// L = 16q + r holds row r, fp8 16-byte chunks q and q+4; srcA = B,
// srcB = A; accumulator of lane L holds C[m = r][n = 4q .. 4q+3].
#pragma once
#include <type_traits>

#include "skinny_gemm.hpp"

namespace qg {

struct BurstArgs {
    TileArgs t;           // operands, shapes, strides (tiles_* / group_m unused)
    float* ws;            // fp32 partials [splitk][batch][M][N] (splitk > 1)
    unsigned* counters;   // [batch][n_tiles]: epoch-tagged arrival counters
    unsigned epoch;       // this launch's counter epoch (split_arrive)
    int splitk, kt_per_split, n_tiles;
    long long b_bytes;    // bytes of B per batch (loads past it read zeros)
};

// Most K-tiles per wave the registers hold, by tile shape and waves per
// workgroup (16 waves leave 128 VGPRs per wave); the kernel is instantiated
// for 1, 2, 4 and 8 (up to this) K-tiles per wave and launched with the
// smallest that covers the slice.
// MX keeps the rows' E8M0 bytes of every K-tile in registers as well (fp4:
// 8 bytes per row), which leaves 16-wave 32 x 32 tiles room for 2.
__host__ __device__ constexpr int burst_max_kpw(int mb, int nb, int waves, bool mx = false) {
    return waves == 16 ? (mb <= 2 ? (mx && mb * nb > 2 ? 2 : 4) : 0) : (mb * nb <= 2 ? 8 : 4);
}
constexpr int kBurstLdsMax = 159 * 1024;    // 160 KB per CU, less the kernel's few scalar LDS words
// LDS of one workgroup: a slot of (MB + NB) 2 KB blocks per wave (B'' needs
// none for B), and the waves' partial tiles
__host__ __device__ constexpr int burst_lds_bytes(int mb, int nb, int waves, bool stage_b) {
    const int slots = waves * (mb + (stage_b ? nb : 0)) * 2048, red = waves * mb * nb * 1024;
    return slots > red ? slots : red;
}

// Plan of a burst launch: NB, waves per workgroup and the K split, chosen by
// a cost model fitted to MI355X measurements (graph-replayed launches,
// M <= 64, K <= 8192, B' and B''): a launch costs ~2.5 us, plus ~25 ns per
// KB that one CU streams (B and A bytes of a workgroup times the workgroups
// per CU), plus ~3.4 us when K is split over workgroups (and, for MX, 0.6
// us per slice past 4; device-coherent
// partial stores, counter and loads, one after the other).  ok == false:
// no burst plan (M > 64, or K too long for 16 waves without a split).
struct BurstPlan {
    bool ok = false;
    int mb = 1, nb = 1, waves = 8, splitk = 1, kt_per_split = 1, n_tiles = 1;
    double cost_us = 1e30;
};

// gate: apply the measured acceptance rule below (off when a caller forces
// the burst kernel); max_split: largest K split considered
inline BurstPlan burst_plan(int m, int n, int k_tiles, int batch, int cus, long long max_counters, bool gate = true,
                            int max_split = 16, bool mx = false) {
    BurstPlan best;
    if (m < 1 || m > 64 || k_tiles < 1 || k_tiles > 64 || n < 1 || batch < 1 || cus < 1) return best;
    const int mb = m <= 16 ? 1 : (m <= 32 ? 2 : 4);
    for (int nb : {2, 1}) {
        const long long tiles = (((long long)n + 16 * nb - 1) / (16 * nb)) * batch;
        for (int s = 1; s <= max_split; ++s) {
            const int kt_per = (k_tiles + s - 1) / s;
            const int split = (k_tiles + kt_per - 1) / kt_per;
            if (split != s) continue;
            int waves = 0;
            for (int w : {8, 16})
                if (!waves && (kt_per + w - 1) / w <= burst_max_kpw(mb, nb, w, mx) &&
                    burst_lds_bytes(mb, nb, w, true) <= kBurstLdsMax)
                    waves = w;
            if (!waves) continue;
            if (split > 1 && (tiles > max_counters || (long long)m * n >= (1LL << 29))) continue;
            const long long wgs = tiles * split;
            // past one round of workgroups (N > 8192): 16-wave plans lose
            // 2.2-2.4x (fp32 scales, M = 17-32, K = 7168, N = 16384 - 129280:
            // N = 32768, M = 32 100.4 us vs 41.2 on the decode kernel), and
            // with fp32 scales so does K past 16 K-tiles (M <= 16, K = 7168:
            // 1.1-1.25x slower than skinny / decode); 8-wave plans over short
            // K keep it (K = 1536, N = 12288 - 129280: best or within 8%)
            if (gate && wgs > cus && (waves == 16 || (!mx && k_tiles > 16))) continue;
            // fp32 scales, M = 17-32: a 16-wave plan over more than half a
            // round re-reads A's rows per 32-column tile as often as B's
            // (N = 8192, K = 7168: 26.4 us vs 15.8 on the skinny / decode
            // kernels)
            if (gate && !mx && waves == 16 && m > 16 && 2 * wgs > cus) continue;
            const double kb = (16.0 * nb + m) * kt_per * 128 / 1024.0;
            // MX plans: + 0.6 us per slice past 4.  Without it the model took
            // 8-16 slices of 1-2 K-tiles per wave for MX decode shapes whose
            // few slices ran 1.2-2.5x faster (graph-replayed, 29 shapes M =
            // 16-64, N = 512-7168, K = 4096-16384, aiter and row-major: MXFP4
            // aiter M = 48, N = 1536, K = 8192 18.5 -> 9.1 us, M = 64, N =
            // 512, K = 4096 13.8 -> 5.6; geometric mean 1.39x, two shapes
            // 1-5% slower); the fp32 block-scale plans keep the fitted model
            const double cost = 2.5 + 0.025 * kb * (double)((wgs + cus - 1) / cus) + (split > 1 ? 3.4 : 0.0) +
                                (mx && split > 4 ? 0.6 * (split - 4) : 0.0);
            if (cost < best.cost_us) {
                best.ok = true;
                best.mb = mb;
                best.nb = nb;
                best.waves = waves;
                best.splitk = split;
                best.kt_per_split = kt_per;
                best.n_tiles = (int)(tiles / batch);
                best.cost_us = cost;
            }
        }
    }
    // measured against the skinny / decode kernels (M <= 64, K <= 8192): the
    // burst kernel wins or ties for M <= 32 (M = 1-16: 1.05-1.35x); for
    // M = 33-64 only when one round of workgroups covers the plan and K is
    // split at most 5 ways (more rounds re-read the 64 rows of A per tile)
    if (gate && best.ok && best.mb == 4 &&
        ((long long)best.n_tiles * batch * best.splitk > cus || best.splitk > 5))
        best.ok = false;
    return best;
}

// One work item of the burst kernel: output tile nt (NB * 16 columns, all
// rows) of batch entry bz over K slice sk, with its split-K reduce.  Called
// once per workgroup by burst_gemm_kernel and once per item by the grouped
// kernel's persistent loop; every thread of the workgroup returns together.
template <int FMT, BLay BL, int MB, int NB, int WAVES, int KPW, bool BF16>
__device__ __forceinline__ void burst_tile(const BurstArgs& bp, const int nt, const int sk, const int bz,
                                           const int batch) {
    constexpr int kBurstWaves = WAVES;
    // RAW: MXFP8 / MXFP4 with row-major B and E8M0 scales; fp4 FRAG: MXFP4
    // with W16 B and e8m0_shuffle scales (MXS); else fp8 with fp32 block
    // scales on B' (K-panel) or B'' (fragment order)
    constexpr bool FP4 = FMT == kFmtFp4;
    constexpr bool MXS = FP4 && BL == BLay::FRAG;
    constexpr bool MX = BL == BLay::RAW || MXS;
    static_assert(BL == BLay::KPANEL || BL == BLay::FRAG || BL == BLay::RAW, "B layout");
    static_assert(MX || !FP4, "fp4 comes with E8M0 scales");
    static_assert((MB == 1 || MB == 2 || MB == 4) && (NB == 1 || NB == 2), "tile shape");
    constexpr int BKB = 128;
    constexpr int KT_SC = FP4 ? 8 : 4;                    // MX: scale bytes per row and K-tile
    constexpr bool STAGE_B = BL != BLay::FRAG;            // B' / row-major B go through LDS; B'' already is fragment order
    constexpr int SLOT = (MB + (STAGE_B ? NB : 0)) * 2048; // one K-tile of the wave's A (and B') lines
    constexpr int LDS_BYTES = burst_lds_bytes(MB, NB, WAVES, STAGE_B);
    static_assert(LDS_BYTES <= kBurstLdsMax, "LDS");
    constexpr int ROWS = MB * 16, COLS = NB * 16;
    static_assert(128 % COLS == 0, "a tile's columns share one 128-row weight-scale block");
    __shared__ __attribute__((aligned(16))) uint8_t lds_mem[LDS_BYTES];
    __shared__ int last_flag;
    QG_LDS uint8_t* const lds = (QG_LDS uint8_t*)lds_mem;

    const TileArgs& p = bp.t;
    const int M = p.m, N = p.n, KB = p.kbytes, LDA = p.lda, LDB = p.ldb, LDC = p.ldc;
    const int SFA_SM = p.sfa_sm, SFA_SK = p.sfa_sk, SFB_SN = p.sfb_sn;
    const int nk = KB / BKB;
    const int n0 = nt * COLS;
    const int kt_begin = sk * bp.kt_per_split;
    const int kt_end = min(nk, kt_begin + bp.kt_per_split);
    const int per_wave = (bp.kt_per_split + kBurstWaves - 1) / kBurstWaves;    // <= KPW (host plan)
    static_assert(KPW <= burst_max_kpw(MB, NB, WAVES, MX), "registers");
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), L = tid & 63;
    if (bp.splitk > 1 && tid == 0) split_claim(bp.counters + (long long)bz * bp.n_tiles + nt, bp.epoch);
    const int q = L >> 4, l16 = L & 15;
    const int kw0 = kt_begin + w * per_wave;
    const int nkw = max(0, min(kt_end, kw0 + per_wave) - kw0);     // this wave's K-tiles

    const uint8_t* A = p.a + bz * p.a_batch;
    const uint8_t* B = p.b + bz * p.b_batch;
    // scale bases: fp32 elements (block scales) or E8M0 bytes (MX)
    const void* SFA = MX ? (const void*)(p.sfa + bz * p.sfa_batch) : (const void*)((const float*)p.sfa + bz * p.sfa_batch);
    const void* SFB = MX ? (const void*)(p.sfb + bz * p.sfb_batch) : (const void*)((const float*)p.sfb + bz * p.sfb_batch);
    auto rsrc = [](const void* base, int bytes) __attribute__((always_inline)) {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
    };
    const int b_range = (int)min(bp.b_bytes, 0x7fffffffLL);

    // ---- the burst: every load of the wave's K-tiles ----
    // whole-line loads: instruction h of a 16-row block covers rows 8h .. 8h+7,
    // lane L taking row 8h + L/8, 16-byte chunk L%8
    i32x4 av[KPW][MB][2], bv[KPW][NB][2];
    float sa[KPW][MB], sb[KPW];
    // MX: the row's scale bytes of the K-tile (fp8 one dword, fp4 two); MXS:
    // the e8m0_shuffle dword holding the lane's two groups (q and q + 4) for
    // both 16-row halves of its 32-row block
    using SX = std::conditional_t<FP4 && !MXS, u32x2, uint32_t>;
    SX xa[KPW][MB], xb[KPW][NB];
    int a_off[MB][2], b_off[NB][2];
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int h = 0; h < 2; ++h) a_off[i][h] = min(16 * i + 8 * h + (L >> 3), M - 1) * LDA + (L & 7) * 16;
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int h = 0; h < 2; ++h) b_off[b][h] = min(n0 + 16 * b + 8 * h + (L >> 3), N - 1) * LDB + (L & 7) * 16;
    int sa_off[MB], xb_off[NB];
    // MXS dword of row r, lane group q: 32-row block r / 32 (SFA_SM / SFB_SN
    // bytes each), q * 64 + (r % 16) * 4 within its 256-byte K-tile
    auto mxs_off = [&](int r, int sm) __attribute__((always_inline)) { return (r >> 5) * sm + q * 64 + (r & 15) * 4; };
#pragma unroll
    for (int i = 0; i < MB; ++i)
        sa_off[i] = MXS ? mxs_off(min(16 * i + l16, M - 1), SFA_SM) : min(16 * i + l16, M - 1) * SFA_SM * (MX ? 1 : 4);
#pragma unroll
    for (int b = 0; b < NB; ++b)
        xb_off[b] = MXS ? mxs_off(min(n0 + 16 * b + l16, N - 1), SFB_SN) : min(n0 + 16 * b + l16, N - 1) * SFB_SN;
    const int sb_off = ((min(n0, N - 1) >> 7) * SFB_SN) * 4;
#pragma unroll
    for (int j = 0; j < KPW; ++j) {
        const bool valid = j < nkw;
        const int kt = kw0 + j;
        const auto rA = rsrc(A, valid ? 0x7fffffff : 0), rB = rsrc(B, valid ? b_range : 0);
        const auto rSA = rsrc(SFA, valid ? 0x7fffffff : 0), rSB = rsrc(SFB, valid ? 0x7fffffff : 0);
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                // each B byte is read once: nontemporal
                if constexpr (BL == BLay::RAW) {                                            // [N][K] rows
                    bv[j][b][h] = __builtin_bit_cast(
                        i32x4, __builtin_amdgcn_raw_buffer_load_b128(rB, b_off[b][h], kt * BKB, 2));
                } else {
                    int soff;
                    if constexpr (BL == BLay::KPANEL) soff = (kt * N + n0 + 16 * b) * BKB;    // [K/128][N][128]
                    else soff = (((n0 / 16 + b) * nk + kt) * 2) * 1024;                      // [N/16][K/128][2][1 KB]
                    bv[j][b][h] = __builtin_bit_cast(
                        i32x4, __builtin_amdgcn_raw_buffer_load_b128(rB, h * 1024 + L * 16, soff, 2));
                }
            }
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
            for (int h = 0; h < 2; ++h)
                av[j][i][h] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(rA, a_off[i][h],
                                                                                              kt * BKB, 0));
        if constexpr (MXS) {
            // lane (q, r): the dword of its row's block for this K-tile
#pragma unroll
            for (int i = 0; i < MB; ++i) xa[j][i] = __builtin_amdgcn_raw_buffer_load_b32(rSA, sa_off[i], kt * 256, 0);
#pragma unroll
            for (int b = 0; b < NB; ++b) xb[j][b] = __builtin_amdgcn_raw_buffer_load_b32(rSB, xb_off[b], kt * 256, 0);
        } else if constexpr (MX) {
            // lane (q, r): the KT_SC scale bytes of its row for this K-tile
#pragma unroll
            for (int i = 0; i < MB; ++i) {
                if constexpr (FP4) xa[j][i] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rSA, sa_off[i], kt * KT_SC, 0));
                else xa[j][i] = __builtin_amdgcn_raw_buffer_load_b32(rSA, sa_off[i], kt * KT_SC, 0);
            }
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                if constexpr (FP4) xb[j][b] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rSB, xb_off[b], kt * KT_SC, 0));
                else xb[j][b] = __builtin_amdgcn_raw_buffer_load_b32(rSB, xb_off[b], kt * KT_SC, 0);
            }
        } else {
#pragma unroll
            for (int i = 0; i < MB; ++i)
                sa[j][i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rSA, sa_off[i],
                                                                                          kt * SFA_SK * 4, 0));
            sb[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rSB, sb_off, kt * 4, 0));
        }
    }

    // keep the whole burst ahead of the first use (the scheduler otherwise
    // sinks some loads next to their consumers)
    __builtin_amdgcn_sched_barrier(0);

    // ---- per K-tile: lines -> LDS slot -> fragments -> MFMA ----
    QG_LDS uint8_t* slot = lds + w * SLOT;
    const int wr = (L >> 3), wc = L & 7;                    // row within 8 / chunk of a whole-line lane
    const int frag0 = l16 * BKB + ((q ^ swz<false>(l16)) * 16);
    const int frag1 = l16 * BKB + (((q + 4) ^ swz<false>(l16)) * 16);
    const int unit = p.unit_scale;
    f32x4 acc[MB][NB];
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[i][b] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto cat8 = [](i32x4 lo, i32x4 hi) __attribute__((always_inline)) {
        return i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    };
    // no branch on nkw here: K-tiles past the wave's run loaded zeros (empty
    // descriptors, no traffic) and add 0, and straight-line code keeps the
    // compiler from sinking the burst's loads next to their uses
#pragma unroll
    for (int j = 0; j < KPW; ++j) {
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int r = 8 * h + wr;
                *(QG_LDS i32x4*)(slot + (16 * i + r) * BKB + ((wc ^ swz<false>(r)) * 16)) = av[j][i][h];
            }
        if constexpr (STAGE_B) {
#pragma unroll
            for (int b = 0; b < NB; ++b)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int r = 8 * h + wr;
                    *(QG_LDS i32x4*)(slot + MB * 2048 + (16 * b + r) * BKB + ((wc ^ swz<false>(r)) * 16)) =
                        bv[j][b][h];
                }
        }
        i32x8 bf[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            if constexpr (STAGE_B) {
                const QG_LDS uint8_t* bs = slot + MB * 2048 + b * 2048;
                bf[b] = cat8(*(const QG_LDS i32x4*)(bs + frag0), *(const QG_LDS i32x4*)(bs + frag1));
            } else {
                bf[b] = cat8(bv[j][b][0], bv[j][b][1]);
            }
        }
        if constexpr (MX) {
            // the lane group's scale byte in byte 0: fp8 byte q of the
            // row's 4; fp4 bytes q (chunk q) and q + 4 (chunk q + 4)
            // MXS: byte (r % 32) / 16 of the dword for group q, 2 + that
            // for group q + 4 (rows of B block b: (n0 / 16 + b) % 2)
            int sxb[NB][2];
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                if constexpr (MXS) {
                    const int hb = 8 * (((n0 >> 4) + b) & 1);
                    sxb[b][0] = (int)(xb[j][b] >> hb);
                    sxb[b][1] = (int)(xb[j][b] >> (hb + 16));
                } else if constexpr (FP4) {
                    sxb[b][0] = (int)(xb[j][b][0] >> (8 * q));
                    sxb[b][1] = (int)(xb[j][b][1] >> (8 * q));
                } else {
                    sxb[b][0] = (int)(xb[j][b] >> (8 * q));
                }
            }
#pragma unroll
            for (int i = 0; i < MB; ++i) {
                const QG_LDS uint8_t* as = slot + i * 2048;
                const i32x4 a0 = *(const QG_LDS i32x4*)(as + frag0), a1 = *(const QG_LDS i32x4*)(as + frag1);
                if constexpr (FP4) {
                    int s0, s1;
                    if constexpr (MXS) {
                        s0 = (int)(xa[j][i] >> (8 * (i & 1)));
                        s1 = (int)(xa[j][i] >> (8 * (i & 1) + 16));
                    } else {
                        s0 = (int)(xa[j][i][0] >> (8 * q));
                        s1 = (int)(xa[j][i][1] >> (8 * q));
                    }
                    const i32x8 a0w = i32x8{a0[0], a0[1], a0[2], a0[3], 0, 0, 0, 0};
                    const i32x8 a1w = i32x8{a1[0], a1[1], a1[2], a1[3], 0, 0, 0, 0};
#pragma unroll
                    for (int b = 0; b < NB; ++b) {
                        const i32x8 b0w = i32x8{bf[b][0], bf[b][1], bf[b][2], bf[b][3], 0, 0, 0, 0};
                        const i32x8 b1w = i32x8{bf[b][4], bf[b][5], bf[b][6], bf[b][7], 0, 0, 0, 0};
                        acc[i][b] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(b0w, a0w, acc[i][b], kFmtFp4,
                                                                                     kFmtFp4, 0, sxb[b][0], 0, s0);
                        acc[i][b] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(b1w, a1w, acc[i][b], kFmtFp4,
                                                                                     kFmtFp4, 0, sxb[b][1], 0, s1);
                    }
                } else {
                    const int s0 = (int)(xa[j][i] >> (8 * q));
                    const i32x8 af = cat8(a0, a1);
#pragma unroll
                    for (int b = 0; b < NB; ++b)
                        acc[i][b] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bf[b], af, acc[i][b], kFmtFp8,
                                                                                     kFmtFp8, 0, sxb[b][0], 0, s0);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < MB; ++i) {
                const QG_LDS uint8_t* as = slot + i * 2048;
                const i32x8 af = cat8(*(const QG_LDS i32x4*)(as + frag0), *(const QG_LDS i32x4*)(as + frag1));
                const float s = sa[j][i] * sb[j];
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    const f32x4 part = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                        bf[b], af, f32x4{0.f, 0.f, 0.f, 0.f}, kFmtFp8, kFmtFp8, 0, unit, 0, unit);
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[i][b][r] = __builtin_fmaf(part[r], s, acc[i][b][r]);
                }
            }
        }
    }

    // ---- the four waves' partial tiles, summed in wave order ----
    __syncthreads();    // every wave is done with its slot
    f32x4* red = (f32x4*)lds_mem;
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int b = 0; b < NB; ++b) red[((w * MB + i) * NB + b) * 64 + L] = acc[i][b];
    __syncthreads();
    // unit u = (i, b) of the tile, lane layout; wave w takes units u = w, w + 4, ...
    constexpr int UNITS = MB * NB;
    f32x4 tile[(UNITS + kBurstWaves - 1) / kBurstWaves];
#pragma unroll
    for (int t = 0; t < (UNITS + kBurstWaves - 1) / kBurstWaves; ++t) {
        const int u = w + t * kBurstWaves;
        f32x4 v = {0.f, 0.f, 0.f, 0.f};
        if (u < UNITS) {
#pragma unroll
            for (int ww = 0; ww < kBurstWaves; ++ww) {
                const f32x4 x = red[(ww * UNITS + u) * 64 + L];
#pragma unroll
                for (int r = 0; r < 4; ++r) v[r] += x[r];
            }
        }
        tile[t] = v;
    }

    auto store_c = [&](int m, int n, f32x4 v) __attribute__((always_inline)) {
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
    // unit u -> output rows 16i + l16, columns n0 + 16b + 4q
    auto unit_m = [&](int u) __attribute__((always_inline)) { return 16 * (u / NB) + l16; };
    auto unit_n = [&](int u) __attribute__((always_inline)) { return n0 + 16 * (u % NB) + 4 * q; };

    if (bp.splitk == 1) {
#pragma unroll
        for (int t = 0; t < (UNITS + kBurstWaves - 1) / kBurstWaves; ++t) {
            const int u = w + t * kBurstWaves;
            if (u < UNITS) store_c(unit_m(u), unit_n(u), tile[t]);
        }
        return;
    }

    // ---- split-K: partial tile out, the last workgroup of the tile sums ----
    const long long plane = (long long)M * N;
    const long long split_stride = (long long)batch * plane;
    const bool vec_ok = (N & 3) == 0;
    {
        const auto part = partial_rsrc(bp.ws + ((long long)sk * batch + bz) * plane);
#pragma unroll
        for (int t = 0; t < (UNITS + kBurstWaves - 1) / kBurstWaves; ++t) {
            const int u = w + t * kBurstWaves;
            const int m = unit_m(u), n = unit_n(u);
            if (u >= UNITS || m >= M) continue;
            const int e = m * N + n;
            if (n + 3 < N && vec_ok) {
                store_partial4(part, e, tile[t]);
            } else {
                for (int r = 0; r < 4; ++r)
                    if (n + r < N) store_partial1(part, e + r, tile[t][r]);
            }
        }
    }
    wait_vmcnt<0>();
    __syncthreads();
    unsigned* ctr = bp.counters + (long long)bz * bp.n_tiles + nt;
    if (tid == 0)
        last_flag = split_arrive(ctr, bp.epoch, bp.splitk);
    __syncthreads();
    if (!last_flag) return;
    const float* ws0 = bp.ws + (long long)bz * plane;
#pragma unroll
    for (int t = 0; t < (UNITS + kBurstWaves - 1) / kBurstWaves; ++t) {
        const int u = w + t * kBurstWaves;
        const int m = unit_m(u), n = unit_n(u);
        if (u >= UNITS || m >= M) continue;
        const int e = m * N + n;
        f32x4 v = {0.f, 0.f, 0.f, 0.f};
        if (n + 3 < N && vec_ok) {
            // every slice's load in flight together (up to 16 at a time), summed in slice order
            for (int s0 = 0; s0 < bp.splitk; s0 += 16) {
                f32x4 x[16];
#pragma unroll
                for (int s = 0; s < 16; ++s)
                    if (s0 + s < bp.splitk) x[s] = load_partial4(partial_rsrc(ws0 + (s0 + s) * split_stride), e);
#pragma unroll
                for (int s = 0; s < 16; ++s)
                    if (s0 + s < bp.splitk)
#pragma unroll
                        for (int r = 0; r < 4; ++r) v[r] += x[s][r];
            }
        } else {
            for (int s = 0; s < bp.splitk; ++s) {
                const auto src = partial_rsrc(ws0 + s * split_stride);
                for (int r = 0; r < 4; ++r)
                    if (n + r < N) v[r] += load_partial1(src, e + r);
            }
        }
        store_c(m, n, v);
    }
    __syncthreads();
    if (tid == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int FMT, BLay BL, int MB, int NB, int WAVES, int KPW, bool BF16>
__global__ __launch_bounds__(WAVES * 64) void burst_gemm_kernel(const BurstArgs bp) {
    burst_tile<FMT, BL, MB, NB, WAVES, KPW, BF16>(bp, blockIdx.x % bp.n_tiles, blockIdx.x / bp.n_tiles, blockIdx.y,
                                                  gridDim.y);
}

// ---- grouped launch: several decode GEMMs (own N, K, operands, scales and
// output; M <= 64 each) in one grid over one list of work items ----
// Problem j owns items [item_begin[j], item_begin[j + 1]): its n_tiles *
// splitk (tile, K slice) pairs, tile-major within a slice, as one problem's
// own launch would number its workgroups.  Workgroup b takes items b,
// b + gridDim.x, ... (gridDim.x = the item count for one workgroup per item,
// or fewer for a persistent grid).  Every problem carries its own counter
// block and partial planes (batch 1), all under the launch's one epoch.
constexpr int kGroupMax = 16;
struct BurstGroup {
    BurstArgs p[kGroupMax];
    int item_begin[kGroupMax + 1];    // item_begin[count] = items in total
    int count;
};
static_assert(sizeof(BurstGroup) <= 4096, "a grouped launch passes its problems as kernel arguments");

template <int FMT, BLay BL, int MB, int NB, int WAVES, int KPW, bool BF16>
__global__ __launch_bounds__(WAVES * 64) void burst_grouped_kernel(const BurstGroup g) {
    const int items = g.item_begin[g.count];
    for (int item = blockIdx.x; item < items; item += gridDim.x) {
        int j = 0;    // the problem of the item (uniform: a scalar scan of at most 16 bounds)
        while (j + 1 < g.count && item >= g.item_begin[j + 1]) ++j;
        const int local = item - g.item_begin[j];
        burst_tile<FMT, BL, MB, NB, WAVES, KPW, BF16>(g.p[j], local % g.p[j].n_tiles, local / g.p[j].n_tiles, 0, 1);
        __syncthreads();    // the next item's slot writes reuse the LDS the reduction just read
    }
}

}  // namespace qg
