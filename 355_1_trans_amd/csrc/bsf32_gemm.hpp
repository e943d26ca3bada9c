// Eight-wave 256 x 256 tile GEMM for fp8 with fp32 block scales (BSF32:
// 1 x 128 activation scales, 128 x 128 weight scales) on gfx950.
//
// Why eight waves: fp32 scales cannot ride on the MFMA (its block scales are
// powers of two), so every 128-deep K-tile's partial product is rescaled in
// VALU, acc += part * (sa * sb), and the accumulators must be VGPRs.  Two
// waves per SIMD give each wave 128 accumulators (a 64 x 128 sub-tile; wave
// w = (wm, wn) = (w / 2, w % 2)), and while one wave rescales the other one
// keeps the matrix core busy.
//
// MFMA: v_mfma_f32_16x16x128_f8f6f4 (fp8, unscaled).  One instruction per
// 16 x 16 block covers a whole K-tile (= one scale block), so its result is
// the partial.  srcA = B rows, srcB = A rows: lane L = 16q + r holds row r,
// 16-byte chunks q and q+4 of the 128-byte K-tile, and receives
// C[m = L%16][n = 4(L/16) + 0..3].  The partial of block k is rescaled after
// block k+1's MFMA has issued (two partial registers), so the VALU work runs
// under the matrix core.
//
// Pipeline.  The K loop runs in half-steps: half-step h = 2t + jh multiplies
// K-tile t's A rows (64 per wave, 4 blocks, read into registers at jh = 0)
// by the B rows [wn*128 + jh*64, +64) (4 blocks, read one block ahead).  LDS
// holds two A stages (256 rows x 128 B + the K-tile's scales) and a ring of
// four B half-slots (128 rows x 128 B: 64 rows for each wn), and there is
// one barrier per half-step.  It comes as soon as the previous half-step has
// read its last B block into registers: that block's 4 MFMAs run after the
// barrier, while the new half-step's first fragments are read, so the
// matrix core does not idle through the barrier and the LDS latency.  The
// DMAs (buffer_load_dwordx4 ... lds) issued in half-step h refill what its
// barrier freed, spread over its MFMAs:
//   * B half h+3 (2 DMAs per wave) into the slot of half h-1;
//   * odd h = 2t+1: K-tile t+2's scales (1 DMA per wave) and rows 0-31 of
//     each 64-row group of its A tile (2 DMAs) into K-tile t's A stage,
//     whose rows have been in registers since half-step 2t;
//   * even h = 2t: rows 32-63 of each group of K-tile t+1's A (2 DMAs).
// That is 5 DMAs per wave at odd and 4 at even half-steps, so the barrier of
// an even half-step waits vmcnt(7) (its K-tile's A and scales landed) and
// that of an odd one vmcnt(9) (its B half landed): the DMA queue never
// drains, and B is prefetched 1.5 K-tiles ahead.  DMAs past the last K-tile
// go through an empty-range buffer descriptor (they write zeros into the
// freed region and read nothing), so there are no branches around DMAs, and
// every LDS region is its own object with a compile-time index (the loop is
// unrolled by four half-steps), so the compiler's own DMA waits stay exact.
//
// LDS rows are 128 bytes with 16-byte chunks XOR-swizzled by row & 7 (DMA
// writes and fragment reads are conflict free).
//
// Tail split (the data-parallel + split-K form of stream-K).  One workgroup
// fills a CU, so batch x tiles = R rounds of `cus` tiles plus a tail of
// fewer; unsplit, the last round leaves CUs idle (M = 3072, N = 7168: 336
// tiles = one round and 80 tiles).  The host may run the first dp_tiles
// (whole rounds) as they are and cut each tail tile's K into tail_split
// slices of kt_per_split K-tiles, one workgroup each, so the last round is
// full.  A slice stores its fp32 partial tile (a flat 256 x 256 image,
// device-coherent) into the workspace, then one relaxed counter atomic per
// workgroup; the last slice of a tile to arrive sums the slices' images in
// slice order (deterministic whichever arrives last) with all 512 threads
// reading whole lines, rounds and stores C, and re-arms the counter.
#pragma once
#include "tile_args.hpp"

namespace qg {

struct Bsf32Args {
    TileArgs t;
    float* ws;            // tail_split > 1: fp32 partial images [tail][tail_split][256 * 256]
    unsigned* counters;   // tail_split > 1: one per tail tile, epoch-tagged arrival counters
    unsigned epoch;       // this launch's counter epoch (split_arrive)
    int dp_tiles;         // batch x tiles run whole (the rest is the tail)
    int tail_split;       // K slices per tail tile (1: no tail split)
    int kt_per_split;     // K-tiles per slice
};

namespace bsf {
template <int V>
struct I {
    static constexpr int value = V;
};
// Partial product of one 16 x 16 block over one 128-deep K-tile, fp8 x fp8.
// Zero scale operands make the compiler select the unscaled instruction
// v_mfma_f32_16x16x128_f8f6f4 (a plain product, which the parity tests pin),
// which issues faster than the scaled form with unit scales; the builtin
// keeps the compiler's hazard tracking for the VALU reads of the result.
__device__ __forceinline__ f32x4 mfma_part(const i32x8& b, const i32x8& a) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(b, a, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0, 0, 0, 0);
}
}  // namespace bsf

template <bool BF16, BLay BL>
__global__ __launch_bounds__(512, 1) void bsf32_gemm_kernel(const Bsf32Args ba) {
    const TileArgs& p = ba.t;
    static_assert(BL == BLay::KPANEL || BL == BLay::FRAG, "K-panel B' or fragment-order B''");
    constexpr bool FRAG = (BL == BLay::FRAG);
    constexpr int BKB = 128, BM = 256;
    constexpr int A_BYTES = BM * BKB;       // 32 KB
    constexpr int SA_OFF = A_BYTES;         // 256 fp32 row scales
    constexpr int SB_OFF = A_BYTES + 1024;  // 4 slots of 256 B, one per wave 4-7
    constexpr int ASTAGE = A_BYTES + 2048;
    constexpr int BHALF = 128 * BKB;        // 16 KB

    __shared__ __attribute__((aligned(1024))) uint8_t lA0[ASTAGE];
    __shared__ __attribute__((aligned(1024))) uint8_t lA1[ASTAGE];
    __shared__ __attribute__((aligned(1024))) uint8_t lB0[BHALF];
    __shared__ __attribute__((aligned(1024))) uint8_t lB1[BHALF];
    __shared__ __attribute__((aligned(1024))) uint8_t lB2[BHALF];
    __shared__ __attribute__((aligned(1024))) uint8_t lB3[BHALF];

    __shared__ int last_flag;

    // ---- work item: tile v of the batch x tiles list (workgroups past
    // dp_tiles: slice sk of tail tile dp_tiles + (b - dp_tiles) / S) ----
    const int T = p.tiles_m * p.tiles_n;
    const int S = ba.tail_split;
    const int b = blockIdx.x;
    const bool slice = b >= ba.dp_tiles && S > 1;
    const int v = slice ? ba.dp_tiles + (b - ba.dp_tiles) / S : b;
    const int sk = slice ? (b - ba.dp_tiles) % S : 0;
    const int bz = v / T;
    // ---- tile coordinates: XCD-contiguous remap, then grouped raster ----
    int bid = v - bz * T;
    if ((T & 7) == 0) bid = (bid & 7) * (T >> 3) + (bid >> 3);
    const int gfull = p.group_m * p.tiles_n;
    const int gi = bid / gfull;
    const int first_m = gi * p.group_m;
    const int gm = min(p.tiles_m - first_m, p.group_m);
    const int within = bid - gi * gfull;
    const int tm = first_m + within % gm;
    const int tn = within / gm;
    const int m0 = tm * BM, n0 = tn * BM;

    // kernel arguments copied into locals once (the loop must not reload the
    // argument block: a vector-memory wait for it would drain the DMAs)
    const int M = p.m, N = p.n, KB = p.kbytes, LDA = p.lda, LDC = p.ldc;
    const int SFA_SM = p.sfa_sm, SFA_SK = p.sfa_sk, SFB_SN = p.sfb_sn;

    const int tid = threadIdx.x;
    if (slice && tid == 0) split_claim(ba.counters + (v - ba.dp_tiles), ba.epoch);
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6), L = tid & 63;
    const int wm = w >> 1, wn = w & 1;
    const int q = L >> 4, l16 = L & 15;

    // NKT K-tiles per row; this work item runs K-tiles [kt0, kt0 + nk)
    const int NKT = KB / BKB;
    const int kt0 = sk * ba.kt_per_split;
    const int nk = slice ? min(NKT, kt0 + ba.kt_per_split) - kt0 : NKT;
    const uint8_t* A = p.a + bz * p.a_batch + (long long)m0 * LDA + (long long)kt0 * BKB;
    // B' (K-panel): K-tile kt is [N][128 B] at kt * N * 128.  B'' (FRAG):
    // block nb of 16 rows, K-tile kt at (nb * NKT + kt) * 2048
    const uint8_t* B = p.b + bz * p.b_batch +
                       (FRAG ? (long long)(n0 >> 4) * NKT * 2048 + (long long)kt0 * 2048
                             : (long long)n0 * BKB + (long long)kt0 * N * BKB);
    const uint8_t* SFA = p.sfa + 4ll * bz * p.sfa_batch;
    const uint8_t* SFB = p.sfb + 4ll * bz * p.sfb_batch;

    // ---- per-lane DMA offsets: lane L writes row +L/8 of an 8-row group,
    // physical chunk L%8 = logical chunk (L%8) ^ (row & 7) ----
    // A part pt, DMA u of wave w: 8-row group g = 2w + u of the 128 rows
    // {64 gg + 32 pt + 0..31 : gg = 0..3}
    int aoff[2][2], adst[2][2];
#pragma unroll
    for (int pt = 0; pt < 2; ++pt)
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int g = 2 * w + u;
            const int r0 = (g >> 2) * 64 + pt * 32 + (g & 3) * 8;
            const int r = r0 + (L >> 3);
            const int c = (L & 7) ^ (r & 7);
            aoff[pt][u] = (min(m0 + r, M - 1) - m0) * LDA + c * 16;
            adst[pt][u] = r0 * BKB;
        }
    // B half jh, DMA u of wave w fills slot bytes [1024 (2w + u), +1024):
    //  B': slot rows 8(2w + u) + L/8; slot row s holds tile column
    //      (s / 64) * 128 + jh * 64 + s % 64;
    //  B'': half u of the 2 KB operand block of slot block w (16 slot rows,
    //      the same columns), copied as is
    int boff[2][2];
#pragma unroll
    for (int jh = 0; jh < 2; ++jh)
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            if constexpr (FRAG) {
                const int tb = (w >> 2) * 8 + jh * 4 + (w & 3);    // 16-column block of the tile
                const int nb = min((n0 >> 4) + tb, ((N + 15) >> 4) - 1) - (n0 >> 4);
                boff[jh][u] = nb * NKT * 2048 + u * 1024 + L * 16;
            } else {
                const int s = (2 * w + u) * 8 + (L >> 3);
                const int n = (s >> 6) * 128 + jh * 64 + (s & 63);
                const int c = (L & 7) ^ (s & 7);
                boff[jh][u] = (min(n0 + n, N - 1) - n0) * BKB + c * 16;
            }
        }
    // scales: waves 0-3 move the fp32 row scales of A rows [64w, 64w + 64)
    // (lane L: row 64w + L); wave 4 + j the weight scale of the tile's
    // 128-column block j & 1 (every lane the same dword)
    const bool sc_is_a = w < 4;
    const uint8_t* sc_base = sc_is_a ? SFA + 4ll * m0 * SFA_SM + 4ll * kt0 * SFA_SK
                                     : SFB + 4ll * min((n0 >> 7) + (w & 1), (N - 1) >> 7) * SFB_SN + 4ll * kt0;
    const int sc_voff = sc_is_a ? 4 * (min(m0 + 64 * w + L, M - 1) - m0) * SFA_SM : 0;
    const long long sc_kstride = sc_is_a ? 4ll * SFA_SK : 4ll;
    const int sc_dst = sc_is_a ? SA_OFF + 256 * w : SB_OFF + 256 * (w - 4);

    QG_LDS uint8_t* const pA0 = (QG_LDS uint8_t*)lA0;
    QG_LDS uint8_t* const pA1 = (QG_LDS uint8_t*)lA1;
    QG_LDS uint8_t* const pB0 = (QG_LDS uint8_t*)lB0;
    QG_LDS uint8_t* const pB1 = (QG_LDS uint8_t*)lB1;
    QG_LDS uint8_t* const pB2 = (QG_LDS uint8_t*)lB2;
    QG_LDS uint8_t* const pB3 = (QG_LDS uint8_t*)lB3;
    auto stageA = [&](int s) __attribute__((always_inline)) { return s ? pA1 : pA0; };
    auto slotB = [&](int s) __attribute__((always_inline)) {
        return s == 0 ? pB0 : s == 1 ? pB1 : s == 2 ? pB2 : pB3;
    };

    auto rsrc = [&](const uint8_t* base, bool valid) __attribute__((always_inline)) {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base), 0, valid ? 0x7FFFFFFFu : 0u,
                                                 0x00020000);
    };
    // DMA d of half-step h, HP = h & 3 (h < 0 in the prologue).
    //   odd HP:  d = 0 scales(t+2), 1-2 A(t+2) rows 0-31, 3-4 B half h+3
    //   even HP: d = 0-1 A(t+1) rows 32-63,              2-3 B half h+3
    struct Src {
        __amdgpu_buffer_rsrc_t sc, a, b;
    };
    auto sources = [&](auto HPC, int h) __attribute__((always_inline)) {
        constexpr int HP = decltype(HPC)::value;
        const int t = h >> 1;  // floor(h / 2)
        const int ka = (HP & 1) ? t + 2 : t + 1;
        const int kb = (h + 3) >> 1;
        Src s;
        s.sc = rsrc(sc_base + ka * sc_kstride, ka < nk);
        s.a = rsrc(A + (long long)ka * BKB, ka < nk);
        s.b = rsrc(B + (FRAG ? (long long)kb * 2048 : (long long)kb * N * BKB), kb < nk);
        return s;
    };
    auto dma = [&](auto HPC, const Src& s, int d) __attribute__((always_inline)) {
        constexpr int HP = decltype(HPC)::value;
        constexpr int JB = (HP + 3) & 1;  // B half index of half-step h + 3
        QG_LDS uint8_t* sl = slotB((HP + 3) & 3);
        if constexpr (HP & 1) {
            QG_LDS uint8_t* st = stageA(HP >> 1);
            if (d == 0) dma4_buf(s.sc, st + sc_dst, sc_voff, 0);
            else if (d < 3) dma16_buf(s.a, st + adst[0][d - 1], aoff[0][d - 1], 0);
            else dma16_buf(s.b, sl + (2 * w + d - 3) * 8 * BKB, boff[JB][d - 3], 0);
        } else {
            QG_LDS uint8_t* st = stageA(((HP >> 1) + 1) & 1);
            if (d < 2) dma16_buf(s.a, st + adst[1][d], aoff[1][d], 0);
            else dma16_buf(s.b, sl + (2 * w + d - 2) * 8 * BKB, boff[JB][d - 2], 0);
        }
    };
    auto issue_all = [&](auto HPC, int h) __attribute__((always_inline)) {
        constexpr int HP = decltype(HPC)::value;
        const Src s = sources(HPC, h);
#pragma unroll
        for (int d = 0; d < ((HP & 1) ? 5 : 4); ++d) dma(HPC, s, d);
    };

    // ---- registers ----
    f32x4 acc[4][8];  // [A block i][B block jj of the wave's 128 columns]
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    i32x8 af[4], bf[2];
    f32x4 part[2];
    float fs[4] = {0.f, 0.f, 0.f, 0.f};
    // fragment of a 16-row block: chunks q and q+4 of row l16, swizzled rows
    // (A, B'); B'' blocks hold the operand order itself (lane L at 16 L)
    const int rd8 = l16 * BKB + ((q ^ (l16 & 7)) << 4);
    const int rdb0 = FRAG ? L * 16 : rd8, rdb1 = FRAG ? 1024 + L * 16 : rd8 ^ 64;
    auto ld_frag = [&](const QG_LDS uint8_t* blk) __attribute__((always_inline)) -> i32x8 {
        const i32x4 lo = *(const QG_LDS i32x4*)(blk + rd8);
        const i32x4 hi = *(const QG_LDS i32x4*)(blk + (rd8 ^ 64));
        return i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    };
    auto ld_bfrag = [&](const QG_LDS uint8_t* blk) __attribute__((always_inline)) -> i32x8 {
        const i32x4 lo = *(const QG_LDS i32x4*)(blk + rdb0);
        const i32x4 hi = *(const QG_LDS i32x4*)(blk + rdb1);
        return i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    };
    // acc[i][jj] += part[x] * fs[i]
    auto rescale = [&](int i, int jj, int x) __attribute__((always_inline)) {
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[i][jj][e] = __builtin_fmaf(part[x][e], fs[i], acc[i][jj][e]);
    };

    // One half-step.  Its barrier comes as soon as the previous half-step has
    // read its last B block into registers, so that block's 4 MFMAs (slots
    // 12-15 of the previous half-step, `deferred`) run after the barrier,
    // while this half-step's first fragments are read: the matrix core does
    // not idle through barrier and LDS latency.  Partial k is rescaled after
    // MFMA k+1 has issued; the previous half-step's last partials use its
    // scales, which this half-step replaces (at jh = 0) only afterwards.
    auto half = [&](auto HPC, int h, bool deferred) __attribute__((always_inline)) {
        constexpr int HP = decltype(HPC)::value;
        constexpr int JH = HP & 1;
        constexpr int JP = (JH ^ 1) * 4;  // first accumulator column block of the previous half-step
        if constexpr (JH == 0) asm volatile("s_waitcnt vmcnt(7) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(9) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        const QG_LDS uint8_t* sB = slotB(HP) + wn * 64 * BKB;
        const QG_LDS uint8_t* sA = stageA(HP >> 1) + wm * 64 * BKB;
        const Src src = sources(HPC, h);
        float fsn[4];
        // deferred slots 12-15 of the previous half-step (B block 3 in bf[1]);
        // this half-step's block 0 goes to bf[0], its A blocks replace af[d]
        // once MFMA d has read the old ones
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            if (deferred) {
                part[d & 1] = bsf::mfma_part(bf[1], af[d]);
                __builtin_amdgcn_sched_barrier(0);
                rescale((d + 3) & 3, JP + (d == 0 ? 2 : 3), (d + 1) & 1);
            }
            if (d == 0) bf[0] = ld_bfrag(sB);
            if constexpr (JH == 0) {
                af[d] = ld_frag(sA + 16 * d * BKB);
                if (d == 3) {
                    const QG_LDS uint8_t* st = stageA(HP >> 1);
                    const float sb = *(const QG_LDS float*)(st + SB_OFF + 256 * wn);
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        fsn[i] = *(const QG_LDS float*)(st + SA_OFF + 4 * (wm * 64 + 16 * i + l16)) * sb;
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        // slots 0-11: B blocks 0-2, block j+1 read while block j multiplies
#pragma unroll
        for (int k = 0; k < 12; ++k) {
            const int j = k >> 2, i = k & 3;
            if (i == 0) bf[(j + 1) & 1] = ld_bfrag(sB + (j + 1) * 16 * BKB);
            part[k & 1] = bsf::mfma_part(bf[j & 1], af[i]);
            __builtin_amdgcn_sched_barrier(0);
            if (k == 0) {
                if (deferred) rescale(3, JP + 3, 1);
                if constexpr (JH == 0) {
#pragma unroll
                    for (int x = 0; x < 4; ++x) fs[x] = fsn[x];
                }
            } else {
                rescale((k - 1) & 3, JH * 4 + ((k - 1) >> 2), (k - 1) & 1);
            }
            if constexpr (HP & 1) {
                if (k % 2 == 1 && k < 10) dma(HPC, src, k / 2);
            } else {
                if (k % 3 == 1) dma(HPC, src, k / 3);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // slots 12-15 of the last half-step (odd) and the last rescales
    auto drain = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            part[d & 1] = bsf::mfma_part(bf[1], af[d]);
            __builtin_amdgcn_sched_barrier(0);
            rescale((d + 3) & 3, 4 + (d == 0 ? 2 : 3), (d + 1) & 1);
            __builtin_amdgcn_sched_barrier(0);
        }
        rescale(3, 7, 1);
    };

    // ---- prologue: the DMAs of half-steps -3, -2, -1 ----
    issue_all(bsf::I<1>{}, -3);
    issue_all(bsf::I<2>{}, -2);
    issue_all(bsf::I<3>{}, -1);

    const int nh = 2 * nk;
    int h = 0;
    if (h + 4 <= nh) {
        half(bsf::I<0>{}, 0, false);
        half(bsf::I<1>{}, 1, true);
        half(bsf::I<2>{}, 2, true);
        half(bsf::I<3>{}, 3, true);
        for (h = 4; h + 4 <= nh; h += 4) {
            half(bsf::I<0>{}, h, true);
            half(bsf::I<1>{}, h + 1, true);
            half(bsf::I<2>{}, h + 2, true);
            half(bsf::I<3>{}, h + 3, true);
        }
    }
    if (h < nh) {  // nk odd: one K-tile left
        half(bsf::I<0>{}, h, h > 0);
        half(bsf::I<1>{}, h + 1, true);
    }
    drain();
    wait_vmcnt<0>();
    (void)SFB_SN;

    if (slice) {
        // ---- tail slice: the partial image, the counter, and for the last
        // slice to arrive the sum of the slices in slice order ----
        const int r = v - ba.dp_tiles;
        float* const img0 = ba.ws + (long long)r * S * (BM * BM);
        {
            const auto out = partial_rsrc(img0 + (long long)sk * (BM * BM));
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int jj = 0; jj < 8; ++jj)
                    store_partial4(out, (wm * 64 + 16 * i + l16) * BM + wn * 128 + 16 * jj + 4 * q, acc[i][jj]);
        }
        wait_vmcnt<0>();
        __syncthreads();
        if (tid == 0)
            last_flag = split_arrive(ba.counters + r, ba.epoch, S);
        __syncthreads();
        if (!last_flag) return;
        // thread tid sums 4 consecutive columns of rows tid / 64 + 8u
        // (u = 0..31): 8 rows per group of loads, every slice's loads of a
        // group issued before the first add
        const auto src = partial_rsrc(img0);
        const int col = 4 * (tid & 63), row0 = tid >> 6;
        const bool vec_ok = p.c_vec >= 4;
        for (int ug = 0; ug < 32; ug += 8) {
            f32x4 sum[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) sum[u] = load_partial4(src, (row0 + 8 * (ug + u)) * BM + col);
            for (int s2 = 1; s2 < S; s2 += 2) {
                f32x4 x0[8], x1[8];
                const bool two = s2 + 1 < S;
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const int e = (row0 + 8 * (ug + u)) * BM + col;
                    x0[u] = load_partial4(src, s2 * (BM * BM) + e);
                    if (two) x1[u] = load_partial4(src, (s2 + 1) * (BM * BM) + e);
                }
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    sum[u] += x0[u];
                    if (two) sum[u] += x1[u];
                }
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int mm = m0 + row0 + 8 * (ug + u), nn = n0 + col;
                if (mm >= M) continue;
                const f32x4 sv = sum[u];
                if constexpr (BF16) {
                    uint16_t* crow = (uint16_t*)p.c + bz * p.c_batch + (long long)mm * LDC;
                    if (vec_ok && nn + 3 < N) {
                        *(u32x2*)(crow + nn) = u32x2{pack_bf16x2(sv[0], sv[1]), pack_bf16x2(sv[2], sv[3])};
                    } else {
                        for (int e = 0; e < 4; ++e)
                            if (nn + e < N) crow[nn + e] = bf16_bits(sv[e]);
                    }
                } else {
                    float* crow = (float*)p.c + bz * p.c_batch + (long long)mm * LDC;
                    if (vec_ok && nn + 3 < N) {
                        *(f32x4*)(crow + nn) = sv;
                    } else {
                        for (int e = 0; e < 4; ++e)
                            if (nn + e < N) crow[nn + e] = sv[e];
                    }
                }
            }
        }
        if (tid == 0) __hip_atomic_store(ba.counters + r, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }

    // ---- epilogue: lane holds C[16i + l16][16jj + 4q + 0..3] of the wave's
    // 64 x 128 block ----
    // 4-element stores need 8- (bf16) or 16-byte (fp32) aligned row starts;
    // the bf16 whole-tile path stores 16 bytes (8 elements) per lane
    const bool vec_ok = p.c_vec >= 4;
    if (p.c_vec >= (BF16 ? 8 : 4) && m0 + BM <= M && n0 + BM <= N) {
        if constexpr (BF16) {
            // bf16 through the wave's own 16 KB of LDS (rows of 256 B, 16-byte
            // chunks XOR-swizzled by row) so that every global store writes
            // whole 128-byte lines
            asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
            QG_LDS uint8_t* img = w < 4 ? stageA(w >> 1) + (w & 1) * 16384 : slotB(w - 4);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int jj = 0; jj < 8; ++jj) {
                    const int r = 16 * i + l16, cbyte = 32 * jj + 8 * q;
                    const int c = (cbyte >> 4) ^ (r & 15);
                    const f32x4 a = acc[i][jj];
                    *(QG_LDS u32x2*)(img + r * 256 + c * 16 + (cbyte & 15)) =
                        u32x2{pack_bf16x2(a[0], a[1]), pack_bf16x2(a[2], a[3])};
                }
            const int rr = L >> 4, cc = L & 15;
            uint16_t* cbase = (uint16_t*)p.c + (long long)bz * p.c_batch + (long long)(m0 + wm * 64 + rr) * LDC +
                              n0 + wn * 128 + cc * 8;
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const int r = u * 4 + rr;
                const i32x4 v = *(const QG_LDS i32x4*)(img + r * 256 + ((cc ^ (r & 15)) << 4));
                // non-temporal: the output is not re-read, keep L2 and MALL for A and B
                __builtin_nontemporal_store(v, (i32x4*)(cbase + (long long)u * 4 * LDC));
            }
        } else {
            float* cw = (float*)p.c + (long long)bz * p.c_batch + (long long)(m0 + wm * 64 + l16) * LDC + n0 +
                        wn * 128 + 4 * q;
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int jj = 0; jj < 8; ++jj) *(f32x4*)(cw + (long long)16 * i * LDC + 16 * jj) = acc[i][jj];
        }
        return;
    }
    // edge tiles: masked element stores
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int mm = m0 + wm * 64 + 16 * i + l16;
        if (mm < M) {
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) {
                const int nn = n0 + wn * 128 + 16 * jj + 4 * q;
                const f32x4 v = acc[i][jj];
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
