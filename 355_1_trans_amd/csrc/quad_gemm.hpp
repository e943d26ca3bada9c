// One-by-four wave MXFP4 tile GEMM for gfx950 (256 x 256 tiles, 32x32x64
// scaled MFMA): each wave owns all 256 rows of A and a quarter of B's 256
// rows (64 output columns).
//
// Against the two-by-two layout (wide_gemm.hpp) B never touches LDS:
//  * A goes global -> LDS by DMA (two stages of 256 rows x 128 B, whole-line
//    DMAs, 16-byte chunks XOR-swizzled by row) and every wave reads all of it;
//  * each wave loads its own 64 B rows of a K-tile straight into registers
//    as MFMA operands, double-buffered (K-tile t + 1's loaded over the first
//    three quadrants of K-tile t), so half of the LDS writes of a K-tile
//    disappear and the LDS reads stay what they were (every wave reads 32 KB
//    per K-tile);
//  * one workgroup barrier per K-tile: at the start of quadrant 3 every wave
//    has read its last A operands of K-tile t (freeing t's stage for the DMA
//    of t + 2) and K-tile t + 1's DMAs have landed (vmcnt counts only the
//    8 B loads of t + 1 issued after them);
//  * the bf16 epilogue stages each wave's 256 x 64 block through its own
//    16 KB of LDS in two passes, rows of 128 B = one C line each, so every
//    store instruction writes whole lines; the region is the wave's alone, so
//    the epilogue has no workgroup barrier.
//
// Scales are E8M0 in aiter's e8m0_shuffle order (MXS: per 32-row block and
// K-tile 256 bytes, byte (g%4)*64 + (r%16)*4 + ((g%8)/4)*2 + (r%32)/16; the
// row-major entry shuffles its scales into the workspace first).  A lane of
// the 32x32x64 operand holds row r of the block and 16-byte chunk g of the
// 32-byte sub-tile s, i.e. scale group 2s + g: the dword at g*64 +
// (r%16)*4 + (s%2)*128 holds it in byte 2(s/2) + (r%32)/16.  The MFMA picks
// a scale byte per instruction (op_sel), the same for every lane, so an MFMA
// block is built from rows with the same (r%32)/16: block (P, h) is rows
// 64P + 16h + [0, 16) and 64P + 32 + 16h + [0, 16) -- two halves of
// neighbouring 32-row scale blocks -- and its scale byte is 2(s/2) + h.  The
// B operand's blocks are built the same way from the wave's 64 rows, and the
// epilogue maps the accumulators back to rows and columns.
//
// B layouts: W16 (aiter shuffle_weight(16,16): a 16-row block's K-tile is
// 2 KB, [8 chunks][16 rows][16 B], so an operand load is two 512-byte runs)
// or RAW ([N][K/2] rows: 32 rows x 32 B per operand load, from L2).
//
// Register layout (probe.hip): srcA = B rows, srcB = A rows; accumulator
// register v of lane L = 32g + r holds C[m = r][n = 8(v/4) + 4g + v%4] of the
// 32 x 32 block (m, n in the blocks' row orders above).
#pragma once
#include <utility>

#include "tile_args.hpp"

namespace qg {

typedef float f32x16 __attribute__((ext_vector_type(16)));

namespace quad {

template <int V>
struct I {
    static constexpr int value = V;
};
template <class F, int... Is>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, Is...>) {
    (f(I<Is>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// acc += the fp4 32x32x64 scaled MFMA, accumulator pinned to AGPRs; OA / OB:
// scale byte of srcA (B rows) / srcB (A rows): op_sel bit 0 and op_sel_hi
// bit 1 of each scale operand.  The leading s_nop covers a VALU write of an
// operand register (the compiler's hazard tracking does not see inline asm).
// The accumulator is always an in-out operand: with an output-only form for
// a tile's first K-tile (accumulator input 0) the compiler moved the results
// between AGPRs right after the asm, before the MFMA had written them.
#define QG_QUAD_MFMA(A0, B0, A1, B1)                                                                            \
    asm("s_nop 1\n\tv_mfma_scale_f32_32x32x64_f8f6f4 %0, %1, %2, %0, %3, %4 op_sel:[" #A0 "," #B0 ",0] "         \
        "op_sel_hi:[" #A1 "," #B1 ",0] cbsz:4 blgp:4"                                                            \
        : "+a"(acc)                                                                                             \
        : "v"(b), "v"(a), "v"(sb), "v"(sa))
template <int OA, int OB>
__device__ __forceinline__ void mfma(f32x16& acc, const i32x4& b, const i32x4& a, int sb, int sa) {
    static_assert(OA >= 0 && OA < 4 && OB >= 0 && OB < 4, "scale byte");
    if constexpr (OA == 0 && OB == 0) QG_QUAD_MFMA(0, 0, 0, 0);
    else if constexpr (OA == 1 && OB == 0) QG_QUAD_MFMA(1, 0, 0, 0);
    else if constexpr (OA == 2 && OB == 0) QG_QUAD_MFMA(0, 0, 1, 0);
    else if constexpr (OA == 3 && OB == 0) QG_QUAD_MFMA(1, 0, 1, 0);
    else if constexpr (OA == 0 && OB == 1) QG_QUAD_MFMA(0, 1, 0, 0);
    else if constexpr (OA == 1 && OB == 1) QG_QUAD_MFMA(1, 1, 0, 0);
    else if constexpr (OA == 2 && OB == 1) QG_QUAD_MFMA(0, 1, 1, 0);
    else if constexpr (OA == 3 && OB == 1) QG_QUAD_MFMA(1, 1, 1, 0);
    else if constexpr (OA == 0 && OB == 2) QG_QUAD_MFMA(0, 0, 0, 1);
    else if constexpr (OA == 1 && OB == 2) QG_QUAD_MFMA(1, 0, 0, 1);
    else if constexpr (OA == 2 && OB == 2) QG_QUAD_MFMA(0, 0, 1, 1);
    else if constexpr (OA == 3 && OB == 2) QG_QUAD_MFMA(1, 0, 1, 1);
    else if constexpr (OA == 0 && OB == 3) QG_QUAD_MFMA(0, 1, 0, 1);
    else if constexpr (OA == 1 && OB == 3) QG_QUAD_MFMA(1, 1, 0, 1);
    else if constexpr (OA == 2 && OB == 3) QG_QUAD_MFMA(0, 1, 1, 1);
    else QG_QUAD_MFMA(1, 1, 1, 1);
}
#undef QG_QUAD_MFMA

}  // namespace quad

// p: TileArgs with sfa_sm / sfb_sn = e8m0_shuffle bytes per 32-row block
// (the K-tile step is 256 bytes), tiles_m / tiles_n / group_m set by the host;
// W16 B: ldb = the bytes of K per row (16-row blocks 16 * ldb apart), which
// exceeds kbytes when batch entries are K slices of one GEMM.
// (A persistent form of this kernel -- each workgroup walking the tile list
// and issuing the next tile's first K-tiles during this one's last -- ran
// 1.1-1.4x slower: the C stores of one tile sit in the in-order vmcnt queue
// ahead of the next tile's DMAs, and the tile hand-over spilled registers.)
template <BLay BL, bool BF16>
__global__ __launch_bounds__(256, 1) void quad_gemm_kernel(const TileArgs p) {
    static_assert(BL == BLay::W16 || BL == BLay::RAW, "B layout");
    constexpr int BKB = 128, BM = 256;
    constexpr int SC_A = 0, SC_B = 2048;      // scale stage: A's 8 blocks, then B's, 256 B each
    __shared__ __attribute__((aligned(1024))) uint8_t lA0[BM * BKB];
    __shared__ __attribute__((aligned(1024))) uint8_t lA1[BM * BKB];
    __shared__ __attribute__((aligned(1024))) uint8_t lS0[4096];
    __shared__ __attribute__((aligned(1024))) uint8_t lS1[4096];
    __shared__ __attribute__((aligned(1024))) uint8_t lC[4 * 16384];

    // ---- tile: XCD-contiguous remap (workgroup b runs on XCD b % 8), then a
    // grouped raster of group_m tile rows ----
    const int T = p.tiles_m * p.tiles_n;
    const int bz = blockIdx.z;
    int bid = blockIdx.x;
    if ((T & 7) == 0) bid = (bid & 7) * (T >> 3) + (bid >> 3);
    const int gfull = p.group_m * p.tiles_n;
    const int gi = bid / gfull;
    const int first_m = gi * p.group_m;
    const int gm = min(p.tiles_m - first_m, p.group_m);
    const int within = bid - gi * gfull;
    const int m0 = (first_m + within % gm) * BM, n0 = (within / gm) * BM;

    const int M = p.m, N = p.n, KB = p.kbytes, LDA = p.lda, LDB = p.ldb, LDC = p.ldc;
    const int nk = KB / BKB;
    const int tid = threadIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6), L = tid & 63;
    const int r32 = L & 31, g = L >> 5, rlo = r32 & 15, rhi = r32 >> 4;

    QG_LDS uint8_t* const sA[2] = {(QG_LDS uint8_t*)lA0, (QG_LDS uint8_t*)lA1};
    QG_LDS uint8_t* const sS[2] = {(QG_LDS uint8_t*)lS0, (QG_LDS uint8_t*)lS1};

    // ---- sources; buffer ranges end at the last valid row (rows past M or N
    // read zeros), and past the last K-tile the range is empty (no traffic) ----
    const uint8_t* A = p.a + bz * p.a_batch + (long long)m0 * LDA;
    // (the host bounds every operand's bytes per batch entry below 2^31)
    const int a_bytes = min(M - m0, BM) * LDA;
    const uint8_t* B;
    int b_bytes;
    if constexpr (BL == BLay::W16) {
        // 16-row blocks 16 * LDB bytes apart (LDB = the whole row's K bytes;
        // a K slice of a split launch covers the first KB of each block
        // from its batch offset on); the range ends with the last block's
        // slice
        B = p.b + bz * p.b_batch + (long long)(n0 >> 4) * 16 * LDB;
        b_bytes = (min(((N + 15) >> 4) - (n0 >> 4), BM / 16) - 1) * 16 * LDB + 16 * KB;
    } else {
        B = p.b + bz * p.b_batch + (long long)n0 * LDB;
        b_bytes = min(N - n0, BM) * LDB;
    }
    const int SFA_SM = p.sfa_sm, SFB_SM = p.sfb_sn;
    const uint8_t* SA = p.sfa + bz * p.sfa_batch + (long long)(m0 >> 5) * SFA_SM;
    const uint8_t* SB = p.sfb + bz * p.sfb_batch + (long long)(n0 >> 5) * SFB_SM;
    const int sa_bytes = min(((M + 31) >> 5) - (m0 >> 5), 8) * SFA_SM;
    const int sb_bytes = min(((N + 31) >> 5) - (n0 >> 5), 8) * SFB_SM;
    // range: bytes from `base` on (K-tile kt's base: the tile's bytes less kt
    // steps, positive while kt < nk); past the last K-tile an empty range
    auto rsrc = [](const uint8_t* base, int range) __attribute__((always_inline)) {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base), 0, range, 0x00020000);
    };

    // ---- per-lane offsets ----
    // A DMA t of wave w: rows 8(8w + t) + L/8, physical chunk L%8 holds logical
    // chunk (L%8) ^ ((row >> 1) & 7).  (common.hpp's fp4 swizzle, (row & 7) ^
    // (row >> 3 & 1), measured the same bank-conflict count and a 5-13%
    // slower kernel.)
    int aoff[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        const int r = (w * 8 + t) * 8 + (L >> 3);
        aoff[t] = r * LDA + (((L & 7) ^ ((r >> 1) & 7)) << 4);
    }
    // A operand of MFMA block (P, h), sub-tile s: row 64P + 32 rhi + 16h + rlo,
    // logical chunk 2s + g; (row >> 1) & 7 = rlo >> 1 for these rows
    // (each offset passes through an empty asm: written as a plain lane-id
    // expression, the compiler loses track of which LDS array a read hits and
    // waits for every DMA in flight before it)
    int ard[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        ard[s] = (32 * rhi + rlo) * BKB + (((2 * s + g) ^ (rlo >> 1)) << 4);
        asm("" : "+v"(ard[s]));
    }
    // B operand of the wave's block h (rows 16h + rlo and 32 + 16h + rlo of its
    // 64), sub-tile s: W16 block 4w + 2 rhi + h, chunk 2s + g, row rlo; RAW row
    // 64w + 32 rhi + 16h + rlo, bytes 32s + 16g.  The sub-tile step is an
    // instruction offset (512 or 32 bytes).
    int boff[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        if constexpr (BL == BLay::W16) boff[h] = (4 * w + 2 * rhi + h) * 16 * LDB + g * 256 + rlo * 16;
        else boff[h] = (64 * w + 32 * rhi + 16 * h + rlo) * LDB + g * 16;
    }
    // scale DMA of wave w (one per K-tile): waves 0-1 A's blocks 4(w&1) + L/16,
    // waves 2-3 B's; 16 bytes per lane of the block's 256
    const int soff = (4 * (w & 1) + (L >> 4)) * (w < 2 ? SFA_SM : SFB_SM) + (L & 15) * 16;
    const int sdst = (w < 2 ? SC_A : SC_B) + (w & 1) * 1024;
    // scale reads: lane's dword of block pair P (A) or the wave's pair (B)
    int srd = rhi * 256 + g * 64 + rlo * 4;
    asm("" : "+v"(srd));

    auto dma_tile = [&](int kt, int stage, int d0, int d1) __attribute__((always_inline)) {
        // A DMAs d0 .. d1 - 1 of K-tile kt (d == 8: the scale DMA)
        const bool in = kt < nk;
        const auto ra = rsrc(A + kt * BKB, in ? a_bytes - kt * BKB : 0);
        for (int d = d0; d < d1; ++d) {
            if (d < 8) {
                dma16_buf(ra, sA[stage] + (w * 8 + d) * 8 * BKB, aoff[d], 0);
            } else {
                const auto rs = w < 2 ? rsrc(SA + kt * 256, in ? sa_bytes - kt * 256 : 0)
                                      : rsrc(SB + kt * 256, in ? sb_bytes - kt * 256 : 0);
                dma16_buf(rs, sS[stage] + sdst, soff, 0);
            }
        }
    };

    f32x16 acc[8][2];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;
    i32x4 aq[2][2][4];          // [quadrant parity][h][s]
    i32x4 bq[2][2][4];          // [K-tile parity][h][s]
    int sa[2][4][2], sb[2][2];  // [K-tile parity][pair P][word], [K-tile parity][word]

    auto load_b = [&](int kt, int buf, int h, int s) __attribute__((always_inline)) {
        const bool in = kt < nk;
        if constexpr (BL == BLay::W16) {
            const auto rb = rsrc(B + kt * 2048, in ? b_bytes - kt * 2048 : 0);
            bq[buf][h][s] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(rb, boff[h] + 512 * s, 0, 0));
        } else {
            const auto rb = rsrc(B + kt * BKB, in ? b_bytes - kt * BKB : 0);
            bq[buf][h][s] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(rb, boff[h] + 32 * s, 0, 0));
        }
    };
    auto read_a = [&](int stage, int P, int par) __attribute__((always_inline)) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int s = 0; s < 4; ++s)
                aq[par][h][s] = *(const QG_LDS i32x4*)(sA[stage] + (64 * P + 16 * h) * BKB + ard[s]);
    };
    auto read_scales = [&](int stage, int par) __attribute__((always_inline)) {
#pragma unroll
        for (int P = 0; P < 4; ++P)
#pragma unroll
            for (int wd = 0; wd < 2; ++wd)
                sa[par][P][wd] = *(const QG_LDS int*)(sS[stage] + SC_A + 512 * P + srd + 128 * wd);
#pragma unroll
        for (int wd = 0; wd < 2; ++wd) sb[par][wd] = *(const QG_LDS int*)(sS[stage] + SC_B + 512 * w + srd + 128 * wd);
    };

    // The K loop runs in phases that start right after a barrier: phase t is
    // quadrant 3 of K-tile t - 1 and quadrants 0-2 of K-tile t, ending in the
    // barrier of K-tile t.  At a barrier every DMA of the stage to be read
    // next has landed, and the waits are builtins the compiler sees, so it
    // knows that no DMA is in flight into a stage the next reads touch: with
    // the loop's header anywhere else it merged the DMA tracking of the two
    // incoming paths and made the first LDS reads after the header wait for
    // the DMAs just issued into the other stage.
    // The barrier's wait: K-tile t + 1's DMAs (issued before the 8 B loads of
    // t + 1) landed, and this wave's LDS reads of stage t & 1 completed.
    constexpr unsigned kPhaseWait = 8u | (7u << 4) | (0u << 8) | (0u << 14);    // vmcnt(8) lgkmcnt(0)
    auto barrier = [&]() __attribute__((always_inline)) {
        __builtin_amdgcn_s_waitcnt(kPhaseWait);
        __builtin_amdgcn_s_barrier();
    };

    // quadrants 0-2 of K-tile t (parity S = t & 1: stage and B buffer), then
    // the barrier of quadrant 3
    auto q012 = [&](auto PC, int t) __attribute__((always_inline)) {
        constexpr int S = decltype(PC)::value;
        quad::static_for<3>([&](auto QC) __attribute__((always_inline)) {
            constexpr int Q = decltype(QC)::value;
            quad::static_for<16>([&](auto KC) __attribute__((always_inline)) {
                constexpr int k = decltype(KC)::value;
                constexpr int s = k >> 2, ha = (k >> 1) & 1, hb = k & 1;
                quad::mfma<2 * (s >> 1) + hb, 2 * (s >> 1) + ha>(acc[2 * Q + ha][hb], bq[S][hb][s],
                                                                 aq[Q & 1][ha][s], sb[S][s & 1],
                                                                 sa[S][Q][s & 1]);
                __builtin_amdgcn_sched_barrier(0);
                // fills: the next quadrant's A operands (one read per two
                // MFMAs) and K-tile t + 1's B (one load per six)
                if constexpr (k % 2 == 1) {
                    constexpr int x = k >> 1, h = x >> 2, ss = x & 3;
                    aq[(Q + 1) & 1][h][ss] = *(const QG_LDS i32x4*)(sA[S] + (64 * (Q + 1) + 16 * h) * BKB + ard[ss]);
                }
                if constexpr (k % 6 == 0 && 3 * Q + k / 6 < 8) {
                    constexpr int x = 3 * Q + k / 6, h = x >> 2, ss = x & 3;
                    load_b(t + 1, S ^ 1, h, ss);
                }
                __builtin_amdgcn_sched_barrier(0);
            });
        });
        barrier();
    };
    // quadrant 3 of K-tile t; fills: K-tile t + 1's scales and first A
    // operands (stage S ^ 1) and the DMAs of t + 2 into stage S, whose reads
    // every wave finished before the barrier
    auto q3 = [&](auto PC, int t) __attribute__((always_inline)) {
        constexpr int S = decltype(PC)::value;
        quad::static_for<16>([&](auto KC) __attribute__((always_inline)) {
            constexpr int k = decltype(KC)::value;
            constexpr int s = k >> 2, ha = (k >> 1) & 1, hb = k & 1;
            quad::mfma<2 * (s >> 1) + hb, 2 * (s >> 1) + ha>(acc[6 + ha][hb], bq[S][hb][s], aq[1][ha][s],
                                                             sb[S][s & 1], sa[S][3][s & 1]);
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (k == 0) read_scales(S ^ 1, S ^ 1);
            if constexpr (k % 2 == 1) {
                constexpr int x = k >> 1, h = x >> 2, ss = x & 3;
                aq[0][h][ss] = *(const QG_LDS i32x4*)(sA[S ^ 1] + 16 * h * BKB + ard[ss]);
            }
            // A DMAs 0-7 one per two MFMAs, the scale DMA with the last
            if constexpr (k % 2 == 0) dma_tile(t + 2, S, k / 2, k == 14 ? 9 : k / 2 + 1);
            __builtin_amdgcn_sched_barrier(0);
        });
    };

    // ---- prologue: A, scales and B of K-tile 0; then what quadrant 3 of
    // K-tile -1 would fill: K-tile 1's DMAs, K-tile 0's scales and first A
    // operands ----
    dma_tile(0, 0, 0, 9);
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int s = 0; s < 4; ++s) load_b(0, 0, h, s);
    barrier();
    dma_tile(1, 1, 0, 9);
    read_scales(0, 0);
    read_a(0, 0, 0);
    q012(quad::I<0>{}, 0);
    // phases t, t + 1 per iteration (t odd)
    int t = 1;
    for (; t + 2 <= nk; t += 2) {
        q3(quad::I<0>{}, t - 1);
        q012(quad::I<1>{}, t);
        q3(quad::I<1>{}, t);
        q012(quad::I<0>{}, t + 1);
    }
    if (t < nk) {
        q3(quad::I<0>{}, t - 1);
        q012(quad::I<1>{}, t);
        q3(quad::I<1>{}, t);
    } else {
        q3(quad::I<0>{}, t - 1);
    }
    // the accumulators come from inline-asm MFMAs: cover the result latency
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
    wait_vmcnt<0>();    // no DMA may land in LDS after the workgroup ends

    // ---- epilogue ----
    // accumulator (J = 2P + h, jb), register v = 4 v4 + e of lane (g, r32):
    // row 64P + 32 rhi + 16h + rlo; column (in the wave's 64) c = 8 v4 + 4g + e
    // of B block jb: c < 16 -> 16 jb + c, else 32 + 16 jb + c - 16
    auto out_row = [&](int J) __attribute__((always_inline)) { return 64 * (J >> 1) + 32 * rhi + 16 * (J & 1) + rlo; };
    auto out_col = [&](int jb, int v4) __attribute__((always_inline)) {
        const int c = 8 * v4 + 4 * g;
        return c < 16 ? 16 * jb + c : 32 + 16 * jb + c - 16;
    };
    const int wc0 = n0 + 64 * w;    // the wave's first output column
    if (BF16 && p.c_vec >= 8 && m0 + BM <= M && n0 + BM <= N) {
        // whole tile: two passes of 128 rows through the wave's 16 KB of LDS
        // (rows of 128 B = the wave's 64 columns, 16-byte chunks XOR-swizzled
        // by row), stored as whole 128-byte lines
        QG_LDS uint8_t* img = (QG_LDS uint8_t*)lC + w * 16384;
#pragma unroll
        for (int pass = 0; pass < 2; ++pass) {
#pragma unroll
            for (int J = 4 * pass; J < 4 * pass + 4; ++J)
#pragma unroll
                for (int jb = 0; jb < 2; ++jb)
#pragma unroll
                    for (int v4 = 0; v4 < 4; ++v4) {
                        const int r = out_row(J) - 128 * pass, cb = 2 * out_col(jb, v4);
                        const f32x16& a = acc[J][jb];
                        *(QG_LDS u32x2*)(img + r * 128 + ((((cb >> 4) ^ (r & 7)) << 4) | (cb & 15))) =
                            u32x2{pack_bf16x2(a[4 * v4], a[4 * v4 + 1]), pack_bf16x2(a[4 * v4 + 2], a[4 * v4 + 3])};
                    }
            uint16_t* cbase = (uint16_t*)p.c + (long long)bz * p.c_batch + (long long)(m0 + 128 * pass) * LDC + wc0;
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const int r = 8 * u + (L >> 3), ch = L & 7;
                const i32x4 v = *(const QG_LDS i32x4*)(img + r * 128 + ((ch ^ (r & 7)) << 4));
                __builtin_nontemporal_store(v, (i32x4*)(cbase + (long long)r * LDC + ch * 8));
            }
        }
        return;
    }
    // edge tiles and fp32 output: masked stores from the accumulators
#pragma unroll
    for (int J = 0; J < 8; ++J) {
        const int mm = m0 + out_row(J);
        if (mm < M) {
#pragma unroll
            for (int jb = 0; jb < 2; ++jb)
#pragma unroll
                for (int v4 = 0; v4 < 4; ++v4) {
                    const int nn = wc0 + out_col(jb, v4);
                    const f32x16& a = acc[J][jb];
                    const f32x4 v = f32x4{a[4 * v4], a[4 * v4 + 1], a[4 * v4 + 2], a[4 * v4 + 3]};
                    if constexpr (BF16) {
                        uint16_t* crow = (uint16_t*)p.c + bz * p.c_batch + (long long)mm * LDC;
                        if (p.c_vec >= 4 && nn + 3 < N) {
                            *(u32x2*)(crow + nn) = u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
                        } else {
                            for (int e = 0; e < 4; ++e)
                                if (nn + e < N) crow[nn + e] = bf16_bits(v[e]);
                        }
                    } else {
                        float* crow = (float*)p.c + bz * p.c_batch + (long long)mm * LDC;
                        if (p.c_vec >= 4 && nn + 3 < N) {
                            *(f32x4*)(crow + nn) = v;
                        } else {
                            for (int e = 0; e < 4; ++e)
                                if (nn + e < N) crow[nn + e] = v[e];
                        }
                    }
                }
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

}  // namespace qg
