// Four-wave 256 x 256 tile GEMM for gfx950: fp8 on the scaled MFMA 16x16x128,
// fp4 on the scaled MFMA 32x32x64.
//
// One workgroup of 4 wave64 (one per SIMD) computes a 256 x 256 tile of C;
// wave (wm, wn) owns a 128 x 128 sub-tile, whose 256 fp32 accumulators live in
// AGPRs (fp8: 8 x 8 blocks of 16 x 16; fp4: 4 x 4 blocks of 32 x 32).  Against
// the 8-wave tile kernel this halves the LDS bytes read per MFMA (each wave
// reads 128 + 128 rows per K-tile for 64 MFMA-slots instead of 128 + 64 rows
// for 32), and it keeps the global->LDS DMA stream from draining at every
// K-tile:
//
//  * operands are staged in registers: the wave's A rows and B rows of one
//    128-byte K-tile are four register halves (A rows 0-63 / 64-127, B rows
//    0-63 / 64-127, 32 VGPRs each).  A K-tile runs as four quadrants of
//    64 x 64 outputs (16 MFMAs) in Gray-code order over (A half, B half), so
//    consecutive quadrants share one half; the order rotates by one quadrant
//    per K-tile.  A half is reloaded with the next K-tile's rows as soon as
//    its last quadrant has issued, so the next K-tile's LDS reads run under
//    this K-tile's MFMAs: two halves during quadrants 3-4, two during
//    quadrant 1 of the next K-tile;
//  * two LDS stages hold K-tiles t+1 (being read) and t+2 (being written).
//    Barrier B1 after quadrant 1 (every read of K-tile t done) frees K-tile
//    t's stage for the DMA of t+2, spread over quadrants 2-4; barrier B2
//    after quadrant 2 waits only for K-tile t+1's DMA (vmcnt = the DMAs of
//    t+2 issued in quadrant 2), so the DMA queue never runs empty;
//  * DMAs go through buffer descriptors whose range is empty past the last
//    K-tile, so the steady-state code has no branches around them.
//  * PERSIST: a grid of about one workgroup per CU, each walking the tile
//    list (aiter's persistent grid_blocks mode); otherwise one tile each.
//
// Register layouts of the two MFMAs (pinned by the layout probes,
// csrc/probe.hip; srcA = B rows, srcB = A rows):
//  * 16x16x128 fp8: lane L = 16q + r holds row r, 16-byte chunks q and q+4
//    of the 128-byte row; scale byte of lane group q covers K [32q, 32q+32);
//    accumulator of lane L holds C[m = L%16][n = 4(L/16) + 0..3];
//  * 32x32x64 fp4 (K = 64 = 32 bytes per instruction, 4 per K-tile): lane
//    L = 32g + r holds row r, 16-byte chunk g of the 32-byte sub-tile, scaled
//    by its own lane group's byte; accumulator register v of lane L holds
//    C[m = L%32][n = 8(v/4) + 4(L/32) + v%4].
// Operand LDS rows are 128 bytes with 16-byte chunks XOR-swizzled per row
// (fp8: r & 7; fp4: (r >> 1) & 7) so both the DMA writes and the fragment
// reads are conflict free.  Scale policies (MX panels, BS8) and B layouts:
// tile_args.hpp.
//
// K-major operands (fp8 only): B in [K][N] (BL = KN) and, with AKM, A in
// [K][M] are staged as they lie -- a K-tile is 128 K-rows of the tile's 256
// columns, rows of 256 bytes in LDS, the 16 chunks of 16 columns swizzled by
// chunk ^ kn_swz(k) -- and transposed on the way out of LDS by
// ds_read_b64_tr_b8: within each 16-lane group, output lane i receives byte
// (i % 8) of the 8-byte pieces addressed by lanes 2j + (i / 8), j = 0..7, as
// its bytes j.  Lane 2j + h of group q addresses K-row k0 + j, columns
// 8h..8h+7 of the 16-column block, so lane 16q + r ends up with the eight K
// values k0..k0+7 of column r; four such reads (k0 = 16q, 16q + 8, 64 + 16q,
// 72 + 16q) build the same 16x16x128 operand the row-major path reads with
// two ds_read_b128.  The swizzle puts the 16 rows that half a wave touches
// (k0 + 0..7 of groups q and q + 1) on 16 different chunks: all 64 banks.
#pragma once
#include <type_traits>
#include <utility>

#include "tile_args.hpp"

namespace qg {

typedef float f32x16 __attribute__((ext_vector_type(16)));

namespace wide {
// Gray-code cycle over (A half, B half): (0,0) (0,1) (1,1) (1,0)
constexpr int qa(int g) { return (g & 3) >= 2 ? 1 : 0; }
constexpr int qb(int g) { return ((g & 3) == 1 || (g & 3) == 2) ? 1 : 0; }
// quadrant k of the K-tile in phase P runs cycle entry (k + P) & 3; the half
// shared by quadrants k and k+1: {is_a, half}
constexpr bool shared_is_a(int P, int k) { return qa((k + P) & 3) == qa((k + 1 + P) & 3); }
constexpr int shared_half(int P, int k) {
    return shared_is_a(P, k) ? qa((k + P) & 3) : qb((k + P) & 3);
}
template <int V>
struct I {
    static constexpr int value = V;
};
template <class F, int... Is>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, Is...>) {
    (f(I<Is>{}), ...);
}
// f(I<0>{}), ..., f(I<N-1>{})
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}
// acc += scaled MFMA with the accumulator pinned to AGPRs (the "a"
// constraint): left to the register allocator, 256 accumulators plus 128
// operand registers get shuffled between AGPRs, VGPRs and scratch.  The
// compiler's hazard tracking does not look inside inline asm, so the
// statement opens with the two wait states a VALU write of an operand VGPR
// needs before an MFMA reads it; they issue while the previous MFMA occupies
// the matrix core.
__device__ __forceinline__ void mfma_fp8(f32x4& acc, const i32x8& b, const i32x8& a, int sb, int sa) {
    asm("s_nop 1\n\tv_mfma_scale_f32_16x16x128_f8f6f4 %0, %1, %2, %0, %3, %4 op_sel_hi:[0,0,0]"
        : "+a"(acc)
        : "v"(b), "v"(a), "v"(sb), "v"(sa));
}
// fp4 32x32x64; OPS2 selects byte 2 (else byte 0) of both scale registers
template <bool OPS2>
__device__ __forceinline__ void mfma_fp4(f32x16& acc, const i32x4& b, const i32x4& a, int sb, int sa) {
    if constexpr (OPS2)
        asm("s_nop 1\n\tv_mfma_scale_f32_32x32x64_f8f6f4 %0, %1, %2, %0, %3, %4 op_sel_hi:[1,1,0] cbsz:4 blgp:4"
            : "+a"(acc)
            : "v"(b), "v"(a), "v"(sb), "v"(sa));
    else
        asm("s_nop 1\n\tv_mfma_scale_f32_32x32x64_f8f6f4 %0, %1, %2, %0, %3, %4 op_sel_hi:[0,0,0] cbsz:4 blgp:4"
            : "+a"(acc)
            : "v"(b), "v"(a), "v"(sb), "v"(sa));
}
}  // namespace wide

// physical 16-byte chunk of logical chunk c in K-row k of a K-major stage: c ^ kn_swz(k)
__device__ __forceinline__ int kn_swz(int k) { return (k & 7) | (((k >> 4) & 1) << 3); }

// AKM: A in [K][M] (row pitch lda >= M), for aiter's TT / TN layouts.
// K-major operands cover whole 256-column tiles (M, N multiples of 256).
template <int FMT, ScaleKind SK, BLay BL, bool BF16, int PB = 16, bool PERSIST = false, bool AKM = false>
__global__ __launch_bounds__(256, 1) void wide_gemm_kernel(const TileArgs p) {
    constexpr bool FP4 = (FMT == kFmtFp4);
    constexpr bool BKN = (BL == BLay::KN);
    static_assert(!FP4 || (!BKN && !AKM), "K-major operands: fp8");
    // MXS (e8m0_shuffle scales) goes with fp4 and shuffle_weight(16,16) B:
    // aiter's gemm_a4w4 bpreshuffle operands
    constexpr bool MXS = (SK == ScaleKind::MXS);
    static_assert(SK != ScaleKind::BSF32 && (!FP4 || SK == ScaleKind::MX || MXS), "MFMA-applied scales");
    static_assert(!MXS || (FP4 && BL == BLay::W16 && (PB == 32 || PB == 8)), "shuffled scales: fp4, W16 B");
    constexpr bool MX = (SK == ScaleKind::MX) || MXS;
    constexpr int BKB = 128, BM = 256;
    constexpr int RB = FP4 ? 32 : 16;          // rows per MFMA block
    constexpr int NBLK = 128 / RB;             // blocks per wave and operand
    constexpr int KT_BYTES = FP4 ? 8 : 4;      // MX scale bytes per row per K-tile
    static_assert(PB == 16 || PB == 32 || PB == KT_BYTES, "panel width");
    constexpr bool WIDE = PB >= 16;               // [row][PB] panels of whole 16-byte pieces
    constexpr int SPAN = MX ? PB / KT_BYTES : 1;  // K-tiles per scale DMA (MXS: 4 or 1)
    constexpr int PANEL = 256 * (PB > 16 ? PB : 16);
    // BS8: a 256-byte SFA slot per stage, then the landing slots of the no-op
    // SFA DMAs of waves 1-3 (an empty-range buffer DMA still writes zeros to
    // its LDS destination)
    constexpr int SA_BYTES = MX ? 2 * PANEL : 2 * 256 + 4 * 256;
    constexpr int SB_BYTES = MX ? 2 * PANEL : 2 * 4 * 256;
    // a register half: fp8 4 fragments of 8 VGPRs (one per 16-row block);
    // fp4 8 of 4 VGPRs (2 32-row blocks x 4 sub-tiles)
    using Frag = std::conditional_t<FP4, i32x4, i32x8>;
    constexpr int NF = FP4 ? 8 : 4;
    using Acc = std::conditional_t<FP4, f32x16, f32x4>;

    __shared__ __attribute__((aligned(1024))) uint8_t lA0[BM * BKB];
    __shared__ __attribute__((aligned(1024))) uint8_t lA1[BM * BKB];
    __shared__ __attribute__((aligned(1024))) uint8_t lB0[BM * BKB];
    __shared__ __attribute__((aligned(1024))) uint8_t lB1[BM * BKB];
    __shared__ __attribute__((aligned(256))) uint8_t lSA[SA_BYTES];
    __shared__ __attribute__((aligned(256))) uint8_t lSB[SB_BYTES];

    // ---- tile loop: one tile per workgroup (grid = tiles x batch), or with
    // PERSIST each workgroup walks the batch x tiles list with stride
    // gridDim.x.  Tile ids go through an XCD-contiguous remap (workgroup b
    // runs on XCD b % 8; with a grid that is a multiple of 8 the tiles an XCD
    // holds at one time stay neighbours), then a grouped raster. ----
    const int T = p.tiles_m * p.tiles_n;
    const int total = PERSIST ? T * p.batch : 1;
    for (int it = PERSIST ? (int)blockIdx.x : 0; it < total; it += PERSIST ? (int)gridDim.x : 1) {
        // the previous tile's epilogue read its C image from the operand
        // stages: every wave's LDS reads finish before the DMAs overwrite
        // them.  Its global stores may still be in flight: the prologue's
        // vmcnt wait counts them as well (vector loads complete in issue
        // order, so that wait still means K-tile 0 has landed), and the
        // stores drain under the first DMAs' latency
        if (PERSIST && it != (int)blockIdx.x) asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        const int bz = PERSIST ? it / T : (int)blockIdx.z;
        int bid = PERSIST ? it - bz * T : (int)blockIdx.x;
        if ((T & 7) == 0) bid = (bid & 7) * (T >> 3) + (bid >> 3);
        const int gfull = p.group_m * p.tiles_n;
        const int gi = bid / gfull;
        const int first_m = gi * p.group_m;
        const int gm = min(p.tiles_m - first_m, p.group_m);
        const int within = bid - gi * gfull;
        const int tm = first_m + within % gm;
        const int tn = within / gm;
        const int m0 = tm * BM, n0 = tn * BM;

        const int M = p.m, N = p.n, KB = p.kbytes, LDA = p.lda, LDB = p.ldb, LDC = p.ldc;
        const int SFA_SM = p.sfa_sm, SFA_SK = p.sfa_sk, SFB_SN = p.sfb_sn;
        // MX: bytes from one K-tile's scales to the next along K -- KT_BYTES in
        // the callers' row-major [rows][K/32], rows * KT_BYTES in the panel-major
        // copy [K/32/PB][rows][PB] (row pitch PB), whose panel DMAs read 1 KB
        // contiguously instead of one cache line per row
        const int SFA_KT = MX ? SFA_SK : 0, SFB_KT = MX ? p.sfb_sk : 0;

        int tid = threadIdx.x;
        // persistent loop: an opaque copy per tile keeps the lane offsets
        // derived from tid out of loop-invariant code motion, whose hoisted
        // values would stay live across the whole K loop
        if constexpr (PERSIST) asm volatile("" : "+v"(tid));
        const int w = __builtin_amdgcn_readfirstlane(tid >> 6), L = tid & 63;
        const int wm = w >> 1, wn = w & 1;

        const uint8_t* A = p.a + bz * p.a_batch + (AKM ? (long long)m0 : (long long)m0 * LDA);
        const uint8_t* B = p.b + bz * p.b_batch +
                           (BL == BLay::RAW ? (long long)n0 * LDB
                            : BL == BLay::KPANEL ? (long long)n0 * BKB
                            : BKN                ? (long long)n0
                                                 : (long long)(n0 >> 4) * 16 * KB);
        const uint8_t* SFA = p.sfa + bz * p.sfa_batch;
        const uint8_t* SFB = p.sfb + bz * p.sfb_batch;

        // ---- per-lane DMA offsets: wave w fills rows [64w, 64w + 64) of A and
        // B, eight 8-row DMAs each; lane L writes row +L/8, physical chunk L%8 =
        // logical chunk (L%8) ^ swizzle(row).  B in shuffle_weight(16,16) order
        // (W16) instead moves whole 16-row blocks as is: a block's K-tile is 2 KB
        // contiguous ([8 chunks][16 rows][16 B], already the 16x16x128 operand
        // order), two linear 1 KB DMAs, read back linearly.  (Gathering W16 into
        // 128-byte rows made every lane of a DMA hit a different cache line:
        // 18% more cycles per K-tile.)  A K-major operand's K-tile is 128 K-rows
        // of 256 bytes: wave w's DMA t fills K-rows 32w + 4t .. +3, lane L K-row
        // +L/16, physical chunk L%16. ----
        int aoff[8], boff[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const int r = (w * 8 + t) * 8 + (L >> 3);
            const int c = (L & 7) ^ (FP4 ? ((r >> 1) & 7) : (r & 7));
            const int kr = (w * 8 + t) * 4 + (L >> 4);
            const int kc = ((L & 15) ^ kn_swz(kr)) << 4;
            if constexpr (AKM) aoff[t] = kr * LDA + kc;
            else aoff[t] = (min(m0 + r, M - 1) - m0) * LDA + c * 16;
            const int gn = min(n0 + r, N - 1) - n0;
            if constexpr (BKN) boff[t] = kr * LDB + kc;
            else if constexpr (BL == BLay::RAW) boff[t] = gn * LDB + c * 16;
            else if constexpr (BL == BLay::KPANEL) boff[t] = gn * BKB + c * 16;
            else {
                const int blk = min((n0 >> 4) + w * 4 + (t >> 1), ((N + 15) >> 4) - 1) - (n0 >> 4);
                boff[t] = blk * 16 * KB + (t & 1) * 1024 + L * 16;
            }
        }

        // ---- scale sources (buffer DMAs; empty range = no-op) ----
        // MX panels: wave w moves the panel rows of A quarter w and B quarter w:
        // lane L = row 64w + L (PB <= 16), or with 32-byte panels two lanes per
        // row (row 64w + 32u + L/2, 16-byte half L%2, DMA u = 0, 1), so that a
        // DMA touches 32 cache lines instead of 64
        // MXS: the tile's eight 32-row blocks per operand, each block's K-tile
        // 256 contiguous bytes: with PB = 32 four K-tiles (1 KB) per block and
        // DMA, wave w moving blocks 2w + u; with PB = 8 one K-tile, waves 0-1
        // moving A's blocks 4(w%2) + L/16 and waves 2-3 B's.  Blocks past the
        // last row re-read the last block (the buffer holds ceil(rows/32)).
        const uint8_t* SFA_t = SFA + (MXS ? (long long)(m0 >> 5) * SFA_SM : (long long)m0 * (MX ? SFA_SM : 1));
        const uint8_t* SFB_t = SFB + (MXS ? (long long)(n0 >> 5) * SFB_SN : MX ? (long long)n0 * SFB_SN : 0ll);
        int mx_voff_a[2], mx_voff_b[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            if constexpr (MXS) {
                const int j = PB == 32 ? 2 * w + u : 4 * (w & 1) + (L >> 4);
                const int off = PB == 32 ? L * 16 : (L & 15) * 16;
                mx_voff_a[u] = (min((m0 >> 5) + j, ((M + 31) >> 5) - 1) - (m0 >> 5)) * SFA_SM + off;
                mx_voff_b[u] = (min((n0 >> 5) + j, ((N + 31) >> 5) - 1) - (n0 >> 5)) * SFB_SN + off;
            } else {
                const int r = PB == 32 ? w * 64 + 32 * u + (L >> 1) : w * 64 + L;
                const int h = PB == 32 ? (L & 1) * 16 : 0;
                mx_voff_a[u] = (min(m0 + r, M - 1) - m0) * SFA_SM + h;
                mx_voff_b[u] = (min(n0 + r, N - 1) - n0) * SFB_SN + h;
            }
        }
        // BS8: SFA's 256 row bytes of a K-tile by wave 0; SFB's byte of the
        // wave's 128-column block as the aligned dword holding it
        const long long bs_b_idx = (long long)min((n0 >> 7) + wn, (N - 1) >> 7) * SFB_SN;

        QG_LDS uint8_t* pA0 = (QG_LDS uint8_t*)lA0;
        QG_LDS uint8_t* pA1 = (QG_LDS uint8_t*)lA1;
        QG_LDS uint8_t* pB0 = (QG_LDS uint8_t*)lB0;
        QG_LDS uint8_t* pB1 = (QG_LDS uint8_t*)lB1;
        QG_LDS uint8_t* pSA = (QG_LDS uint8_t*)lSA;
        QG_LDS uint8_t* pSB = (QG_LDS uint8_t*)lSB;

        const int nk = KB / BKB;

        auto rsrc = [&](const uint8_t* base, bool valid) __attribute__((always_inline)) {
            return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base), 0, valid ? 0x7FFFFFFFu : 0u,
                                                     0x00020000);
        };
        auto a_ktile = [&](int kt) __attribute__((always_inline)) -> const uint8_t* {
            if constexpr (AKM) return A + (long long)kt * BKB * LDA;
            else return A + kt * BKB;
        };
        auto b_ktile = [&](int kt) __attribute__((always_inline)) -> const uint8_t* {
            if constexpr (BKN) return B + (long long)kt * BKB * LDB;
            else if constexpr (BL == BLay::RAW) return B + kt * BKB;
            else if constexpr (BL == BLay::KPANEL) return B + (long long)kt * N * BKB;
            else return B + kt * 2048;
        };
        auto dma_a = [&](int kt, bool valid, QG_LDS uint8_t* sA) __attribute__((always_inline)) {
            const auto r = rsrc(a_ktile(kt), valid);
#pragma unroll
            for (int t = 0; t < 8; ++t) dma16_buf(r, sA + (w * 8 + t) * 8 * BKB, aoff[t], 0);
        };
        auto dma_b = [&](int kt, bool valid, QG_LDS uint8_t* sB) __attribute__((always_inline)) {
            const auto r = rsrc(b_ktile(kt), valid);
#pragma unroll
            for (int t = 0; t < 8; ++t) dma16_buf(r, sB + (w * 8 + t) * 8 * BKB, boff[t], 0);
        };
        // scale DMAs that go with K-tile kt (MX: only when kt starts a panel,
        // which the callers know at compile time); `valid` false = no-op DMAs.
        // MX panel images: PB = 16, 32: [row][PB]; PB = 4 (fp8): [row][4 B];
        // PB = 8 (fp4): [2 halves][row][4 B]
        auto dma_scales = [&](int kt, bool valid) __attribute__((always_inline)) {
            if constexpr (MXS) {
                // images [block][SPAN K-tiles][256 B]
                const int buf = ((kt / SPAN) & 1) * PANEL;
                const auto ra = rsrc(SFA_t + (long long)kt * 256, valid);
                const auto rb = rsrc(SFB_t + (long long)kt * 256, valid);
                if constexpr (PB == 32) {
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        dma16_buf(ra, pSA + buf + w * 2048 + u * 1024, mx_voff_a[u], 0);
                        dma16_buf(rb, pSB + buf + w * 2048 + u * 1024, mx_voff_b[u], 0);
                    }
                } else if (w < 2) {
                    dma16_buf(ra, pSA + buf + (w & 1) * 1024, mx_voff_a[0], 0);
                } else {
                    dma16_buf(rb, pSB + buf + (w & 1) * 1024, mx_voff_b[0], 0);
                }
            } else if constexpr (MX) {
                const int buf = ((kt / SPAN) & 1) * PANEL;
                const auto ra = rsrc(SFA_t + (long long)kt * SFA_KT, valid);
                const auto rb = rsrc(SFB_t + (long long)kt * SFB_KT, valid);
                if constexpr (PB == 32) {
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        dma16_buf(ra, pSA + buf + w * 2048 + u * 1024, mx_voff_a[u], 0);
                        dma16_buf(rb, pSB + buf + w * 2048 + u * 1024, mx_voff_b[u], 0);
                    }
                } else if constexpr (PB == 16) {
                    dma16_buf(ra, pSA + buf + w * 1024, mx_voff_a[0], 0);
                    dma16_buf(rb, pSB + buf + w * 1024, mx_voff_b[0], 0);
                } else {
                    dma4_buf(ra, pSA + buf + w * 256, mx_voff_a[0], 0);
                    dma4_buf(rb, pSB + buf + w * 256, mx_voff_b[0], 0);
                    if constexpr (PB == 8) {
                        dma4_buf(ra, pSA + buf + 1024 + w * 256, mx_voff_a[0] + 4, 0);
                        dma4_buf(rb, pSB + buf + 1024 + w * 256, mx_voff_b[0] + 4, 0);
                    }
                }
            } else {
                const int st = kt & 1;
                const auto ra = rsrc(SFA_t + (long long)kt * SFA_SK, valid && w == 0);
                const auto rb = rsrc(SFB + ((bs_b_idx + kt) & ~3ll), valid);
                dma4_buf(ra, w == 0 ? pSA + st * 256 : pSA + 256 + w * 256, 4 * L, 0);
                dma4_buf(rb, pSB + st * 1024 + w * 256, 0, 0);
            }
        };
        // Scale registers of K-tile kt, x = 0..7 (A and B rows of the wave):
        //  fp8: block x's byte for lane group q (sa[x], sb[x]); BS8 has one B
        //       scale per wave, read with x = 0;
        //  fp4: block x/2, word x%2, which holds the lane group's blocks of
        //       instructions 2(x%2) (byte 0) and 2(x%2)+1 (byte 2) once
        //       finish_scale has shifted the lane group's bytes down.  The shift
        //       is a separate step, issued a few MFMAs after the read, so the
        //       wave does not stall on the LDS latency.
        const int q = L >> 4, l16 = L & 15, g = L >> 5, l32 = L & 31;
        //  MXS: block x/2, words x%2 = the dwords at g*64 and g*64 + 128 of
        //       the block's K-tile: after the shift by the lane's row half
        //       (l32/16), sub-tile s reads word s%2, byte 2(s/2).
        auto read_scale = [&](int kt, int x, int (&sa)[8], int (&sb)[8]) __attribute__((always_inline)) {
            if constexpr (MXS) {
                if ((x & 1) == 0) {
                    const int off = ((kt / SPAN) & 1) * PANEL + (kt % SPAN) * 256 + g * 64 + (l32 & 15) * 4;
                    const QG_LDS uint8_t* ba = pSA + off + (wm * 4 + (x >> 1)) * SPAN * 256;
                    const QG_LDS uint8_t* bb = pSB + off + (wn * 4 + (x >> 1)) * SPAN * 256;
                    sa[x] = *(const QG_LDS int*)ba;
                    sa[x + 1] = *(const QG_LDS int*)(ba + 128);
                    sb[x] = *(const QG_LDS int*)bb;
                    sb[x + 1] = *(const QG_LDS int*)(bb + 128);
                }
            } else if constexpr (MX && !FP4) {
                const int buf = ((kt / SPAN) & 1) * PANEL;
                const int col = WIDE ? (kt % SPAN) * KT_BYTES + q : q;
                sa[x] = pSA[buf + (wm * 128 + x * 16 + l16) * PB + col];
                sb[x] = pSB[buf + (wn * 128 + x * 16 + l16) * PB + col];
            } else if constexpr (MX) {
                const int buf = ((kt / SPAN) & 1) * PANEL;
                const int ra = wm * 128 + (x >> 1) * 32 + l32, rb = wn * 128 + (x >> 1) * 32 + l32;
                if constexpr (WIDE) {
                    // both words of the block in one read (x even; x odd is a no-op)
                    if ((x & 1) == 0) {
                        const i32x2 va = *(const QG_LDS i32x2*)(pSA + buf + ra * PB + (kt % SPAN) * KT_BYTES);
                        const i32x2 vb = *(const QG_LDS i32x2*)(pSB + buf + rb * PB + (kt % SPAN) * KT_BYTES);
                        sa[x] = va[0];
                        sa[x + 1] = va[1];
                        sb[x] = vb[0];
                        sb[x + 1] = vb[1];
                    }
                } else {
                    sa[x] = (int)*(const QG_LDS uint32_t*)(pSA + buf + (x & 1) * 1024 + ra * 4);
                    sb[x] = (int)*(const QG_LDS uint32_t*)(pSB + buf + (x & 1) * 1024 + rb * 4);
                }
            } else {
                const int st = kt & 1;
                sa[x] = pSA[st * 256 + wm * 128 + x * 16 + l16];
                if (x == 0) {
                    const int v = pSB[st * 1024 + w * 256 + (int)((bs_b_idx + kt) & 3)];
#pragma unroll
                    for (int j = 0; j < 8; ++j) sb[j] = v;
                }
            }
        };
        auto finish_scale = [&](int x, int (&sa)[8], int (&sb)[8]) __attribute__((always_inline)) {
            if constexpr (FP4) {
                const int sh = MXS ? 8 * (l32 >> 4) : 8 * g;
                sa[x] = (int)((uint32_t)sa[x] >> sh);
                sb[x] = (int)((uint32_t)sb[x] >> sh);
            }
        };

        // per-lane operand read offsets: fp8 chunks q and q+4 of row l16 of a
        // 16-row block; fp4 chunk 2s+g of row l32 of a 32-row block
        const int rd8 = l16 * BKB + ((q ^ (l16 & 7)) << 4);
        auto rd4 = [&](int s) __attribute__((always_inline)) {
            return l32 * BKB + (((2 * s + g) ^ ((l32 >> 1) & 7)) << 4);
        };
        // fp4 B in W16 blocks: row l32 % 16 of block l32 / 16, chunk 2s + g (+ 512 s).
        // The offset passes through an empty asm: written as a plain lane-id
        // expression, the compiler lost track of which LDS array these reads
        // hit and put a vmcnt(0) (wait for every DMA in flight) before them.
        int rdw = (l32 >> 4) * 2048 + g * 256 + (l32 & 15) * 16;
        asm("" : "+v"(rdw));
        // K-major stages: lane 2j + h of group q addresses K-row 16q + j (+8,
        // +64, +72 for the other three reads), bytes 8h..8h+7 of the logical
        // chunk wsel * 8 + (16-column block of the wave): chunk bits XOR in
        // kn_swz(row) = j | (q & 1) << 3 and the wave's column half
        const int kfl = (l16 >> 1) | ((q & 1) << 3);
        const int krow = (16 * q + (l16 >> 1)) * 256 + (l16 & 1) * 8;
        int tra = krow | (((wm * 8) ^ kfl) << 4), trb = krow | (((wn * 8) ^ kfl) << 4);
        asm("" : "+v"(tra));
        asm("" : "+v"(trb));

        Acc acc[NBLK][NBLK];
#pragma unroll
        for (int i = 0; i < NBLK; ++i)
#pragma unroll
            for (int j = 0; j < NBLK; ++j)
#pragma unroll
                for (int v = 0; v < (FP4 ? 16 : 4); ++v) acc[i][j][v] = 0.f;
        Frag ah[2][NF], bh[2][NF];

        // read unit x (0..3) of register half h of A (is_a) or B: two
        // ds_read_b128 -- fp8: the 16-row block x; fp4: sub-tiles 2(x%2) and
        // 2(x%2)+1 of the 32-row block x/2
        auto read_one = [&](bool is_a, int h, int x, const QG_LDS uint8_t* sA,
                            const QG_LDS uint8_t* sB) __attribute__((always_inline)) {
            const QG_LDS uint8_t* base = is_a ? sA + wm * 128 * BKB : sB + wn * 128 * BKB;
            Frag(&dst)[2][NF] = is_a ? ah : bh;
            if constexpr (FP4) {
                const QG_LDS uint8_t* blk = base + (2 * h + (x >> 1)) * 32 * BKB;
                const int s0 = 2 * (x & 1);
                if (BL == BLay::W16 && !is_a) {
                    // the 32-row block is W16 blocks 2b, 2b + 1 ([8 chunks][16 rows][16 B] each)
                    dst[h][4 * (x >> 1) + s0] = *(const QG_LDS i32x4*)(blk + rdw + 2 * s0 * 256);
                    dst[h][4 * (x >> 1) + s0 + 1] = *(const QG_LDS i32x4*)(blk + rdw + 2 * (s0 + 1) * 256);
                } else {
                    dst[h][4 * (x >> 1) + s0] = *(const QG_LDS i32x4*)(blk + rd4(s0));
                    dst[h][4 * (x >> 1) + s0 + 1] = *(const QG_LDS i32x4*)(blk + rd4(s0 + 1));
                }
            } else if ((is_a && AKM) || (!is_a && BKN)) {
                const QG_LDS uint8_t* stg = (is_a ? sA : sB) + ((is_a ? tra : trb) ^ ((4 * h + x) << 4));
                const i32x2 r0 = __builtin_amdgcn_ds_read_tr8_b64_v2i32((QG_LDS i32x2*)stg);
                const i32x2 r1 = __builtin_amdgcn_ds_read_tr8_b64_v2i32((QG_LDS i32x2*)(stg + 8 * 256));
                const i32x2 r2 = __builtin_amdgcn_ds_read_tr8_b64_v2i32((QG_LDS i32x2*)(stg + 64 * 256));
                const i32x2 r3 = __builtin_amdgcn_ds_read_tr8_b64_v2i32((QG_LDS i32x2*)(stg + 72 * 256));
                dst[h][x] = i32x8{r0[0], r0[1], r1[0], r1[1], r2[0], r2[1], r3[0], r3[1]};
            } else {
                const QG_LDS uint8_t* blk = base + (4 * h + x) * 16 * BKB;
                const bool lin = BL == BLay::W16 && !is_a;    // W16 blocks: operand order
                const i32x4 lo = *(const QG_LDS i32x4*)(blk + (lin ? L * 16 : rd8));
                const i32x4 hi = *(const QG_LDS i32x4*)(blk + (lin ? 1024 + L * 16 : rd8 ^ 64));
                dst[h][x] = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            }
        };
        // quadrant (ha, hb): 16 MFMAs; after MFMA k, fill(k) issues this step's
        // share of LDS reads and DMAs.  Each step is fenced so the order stays
        // as written: the LDS reads and DMAs spread between MFMAs, and no read
        // of a register half moves above the last MFMA that uses its old rows.
        // fp4 walks the 4 sub-tiles outermost, so consecutive MFMAs never chain
        // on one accumulator.
        auto quadrant = [&](int ha, int hb, const int (&sa)[8], const int (&sb)[8],
                            auto&& fill) __attribute__((always_inline)) {
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                if constexpr (FP4) {
                    const int s = k >> 2, bi = (k >> 1) & 1, bj = k & 1;
                    const int i = 2 * ha + bi, j = 2 * hb + bj;
                    // scale word and byte of sub-tile s: MX word s/2, byte 2(s%2);
                    // MXS word s%2, byte 2(s/2)
                    const int sw = MXS ? (s & 1) : (s >> 1);
                    if (MXS ? (s >> 1) : (s & 1))
                        wide::mfma_fp4<true>(acc[i][j], bh[hb][4 * bj + s], ah[ha][4 * bi + s], sb[2 * j + sw],
                                             sa[2 * i + sw]);
                    else
                        wide::mfma_fp4<false>(acc[i][j], bh[hb][4 * bj + s], ah[ha][4 * bi + s], sb[2 * j + sw],
                                              sa[2 * i + sw]);
                } else {
                    const int i = k >> 2, j = k & 3;
                    wide::mfma_fp8(acc[4 * ha + i][4 * hb + j], bh[hb][j], ah[ha][i], sb[4 * hb + j], sa[4 * ha + i]);
                }
                __builtin_amdgcn_sched_barrier(0);
                fill(k);
                __builtin_amdgcn_sched_barrier(0);
            }
        };

        // One K-tile t in phase P = t % 4 (LDS stage P & 1 holds t and then
        // t + 2).  sa/sb: this K-tile's scales; san/sbn receive K-tile t + 1's.
        auto ktile = [&](auto PC, int t, const int (&sa)[8], const int (&sb)[8], int (&san)[8],
                         int (&sbn)[8]) __attribute__((always_inline)) {
            constexpr int P = decltype(PC)::value;
            QG_LDS uint8_t* sA = (P & 1) ? pA1 : pA0;
            QG_LDS uint8_t* sB = (P & 1) ? pB1 : pB0;
            QG_LDS uint8_t* nA = (P & 1) ? pA0 : pA1;
            QG_LDS uint8_t* nB = (P & 1) ? pB0 : pB1;
            constexpr bool r1a = wide::shared_is_a(P, 1), r2a = wide::shared_is_a(P, 2), r0a = wide::shared_is_a(P, 0);
            constexpr int r1 = wide::shared_half(P, 1), r2 = wide::shared_half(P, 2), r0 = wide::shared_half(P, 0);
            __builtin_amdgcn_sched_barrier(0);
            // quadrant 1: K-tile t's two halves freed at the end of the previous
            // K-tile, one read unit after each of the first 8 MFMAs
            quadrant(wide::qa(P), wide::qb(P), sa, sb, [&](int k) __attribute__((always_inline)) {
                if (k < 4) read_one(r1a, r1, k, sA, sB);
                else if (k < 8) read_one(r2a, r2, k - 4, sA, sB);
            });
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // B1: stage P&1 is free
            // quadrants 2-4: the 16 operand DMAs of K-tile t + 2 (A rows 0-7,
            // then B rows 0-7, in 8-row groups) into this K-tile's stage, one
            // after every third MFMA, so the CU's texture path is never asked
            // for more than it streams (a wave blocks on a DMA it cannot queue);
            // the scale DMAs go first, so B2's vmcnt covers them
            const bool more = t + 2 < nk;
            if constexpr ((P + 2) % SPAN == 0) dma_scales(t + 2, more);
            const auto rA = rsrc(a_ktile(t + 2), more);
            const auto rB = rsrc(b_ktile(t + 2), more);
            auto dma_op = [&](int d) __attribute__((always_inline)) {
                if (d < 8) dma16_buf(rA, sA + (w * 8 + d) * 8 * BKB, aoff[d], 0);
                else dma16_buf(rB, sB + (w * 8 + d - 8) * 8 * BKB, boff[d - 8], 0);
            };
            // quadrant 2: DMAs 0-5
            quadrant(wide::qa(P + 1), wide::qb(P + 1), sa, sb, [&](int k) __attribute__((always_inline)) {
                if (k % 3 == 0) dma_op(k / 3);
            });
            asm volatile("s_waitcnt vmcnt(6)\n\ts_barrier" ::: "memory");  // B2: K-tile t + 1 landed
            // quadrant 3: DMAs 6-10; first half of t + 1
            quadrant(wide::qa(P + 2), wide::qb(P + 2), sa, sb, [&](int k) __attribute__((always_inline)) {
                if (k % 3 == 2) dma_op(6 + k / 3);
                if (k < 8 && (k & 1) == 0) read_one(r0a, r0, k >> 1, nA, nB);
            });
            // quadrant 4: DMAs 11-15; second half and scales of t + 1
            quadrant(wide::qa(P + 3), wide::qb(P + 3), sa, sb, [&](int k) __attribute__((always_inline)) {
                if (k % 3 == 1) dma_op(11 + k / 3);
                if (k < 4) read_one(r1a, r1, k, nA, nB);
                if (k < 8) read_scale(t + 1, k, san, sbn);
                else finish_scale(k - 8, san, sbn);
            });
        };

        // ---- prologue: DMA K-tiles 0 and 1 (scales of 1 first, so vmcnt(16)
        // leaves only the operand DMAs of K-tile 1 outstanding) ----
        dma_scales(0, true);
        dma_a(0, true, pA0);
        dma_b(0, true, pB0);
        if constexpr (SPAN == 1) dma_scales(1, nk > 1);
        dma_a(1, nk > 1, pA1);
        dma_b(1, nk > 1, pB1);
        asm volatile("s_waitcnt vmcnt(16)\n\ts_barrier" ::: "memory");
        // halves and scales used by quadrant 1 of K-tile 0
        int s0a[8], s0b[8], s1a[8], s1b[8];
#pragma unroll
        for (int x = 0; x < 4; ++x) {
            read_one(wide::shared_is_a(0, 3), wide::shared_half(0, 3), x, pA0, pB0);
            read_one(wide::shared_is_a(0, 0), wide::shared_half(0, 0), x, pA0, pB0);
        }
#pragma unroll
        for (int x = 0; x < 8; ++x) read_scale(0, x, s0a, s0b);
#pragma unroll
        for (int x = 0; x < 8; ++x) finish_scale(x, s0a, s0b);

        // the loop runs U K-tiles per iteration: the quadrant rotation repeats
        // every 4 and the scale-panel DMA every SPAN, both at compile time
        constexpr int U = SPAN > 4 ? SPAN : 4;
        auto step = [&](auto PC, int tt) __attribute__((always_inline)) {
            if constexpr (decltype(PC)::value & 1) ktile(PC, tt, s1a, s1b, s0a, s0b);
            else ktile(PC, tt, s0a, s0b, s1a, s1b);
        };
        int t = 0;
        for (; t + U <= nk; t += U) wide::static_for<U>([&](auto pc) __attribute__((always_inline)) { step(pc, t + pc.value); });
        wide::static_for<U - 1>([&](auto pc) __attribute__((always_inline)) {
            if (t + pc.value < nk) step(pc, t + pc.value);
        });
        wait_vmcnt<0>();
        // the accumulators come from inline-asm MFMAs, which the compiler's hazard
        // tracking does not see: cover the MFMA-result-to-VALU-read latency
        asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");

        // ---- epilogue ----
        // Output element (r, c) of the wave's 128 x 128 block for accumulator
        // element 4*v4 + e of block (i, j):
        //   fp8: r = 16i + l16, c = 16j + 4q + e            (v4 = 0)
        //   fp4: r = 32i + l32, c = 32j + 8*v4 + 4g + e     (v4 = 0..3)
        auto out_row = [&](int i) __attribute__((always_inline)) { return FP4 ? 32 * i + l32 : 16 * i + l16; };
        auto out_col = [&](int j, int v4) __attribute__((always_inline)) {
            return FP4 ? 32 * j + 8 * v4 + 4 * g : 16 * j + 4 * q;
        };
        constexpr int NV4 = FP4 ? 4 : 1;
        // 4-element stores need 8- (bf16) or 16-byte (fp32) aligned row starts;
        // the bf16 whole-tile path stores 16 bytes (8 elements) per lane
        const bool vec_ok = p.c_vec >= 4;
        if (p.c_vec >= (BF16 ? 8 : 4) && m0 + BM <= M && n0 + BM <= N) {
            if constexpr (BF16) {
                // Whole tile inside C, bf16: the wave's 128 x 128 block goes
                // through its own 32 KB of LDS (one operand stage, rows of 256 B,
                // 16-byte chunks XOR-swizzled by row) so that every global store
                // writes whole 128-byte lines: 16 B per lane, 4 rows of 256 B
                // per instruction, instead of 16 rows x 32 B.
                asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
                QG_LDS uint8_t* img = w == 0 ? pA0 : w == 1 ? pA1 : w == 2 ? pB0 : pB1;
#pragma unroll
                for (int i = 0; i < NBLK; ++i)
#pragma unroll
                    for (int j = 0; j < NBLK; ++j)
#pragma unroll
                        for (int v4 = 0; v4 < NV4; ++v4) {
                            const int r = out_row(i), cbyte = 2 * out_col(j, v4);
                            const int c = (cbyte >> 4) ^ (r & 15);
                            const Acc& a = acc[i][j];
                            *(QG_LDS u32x2*)(img + r * 256 + c * 16 + (cbyte & 15)) =
                                u32x2{pack_bf16x2(a[4 * v4], a[4 * v4 + 1]), pack_bf16x2(a[4 * v4 + 2], a[4 * v4 + 3])};
                        }
                const int rr = L >> 4, cc = L & 15;
                uint16_t* cbase = (uint16_t*)p.c + (long long)bz * p.c_batch + (long long)(m0 + wm * 128 + rr) * LDC +
                                  n0 + wn * 128 + cc * 8;
#pragma unroll
                for (int u = 0; u < 32; ++u) {
                    const int r = u * 4 + rr;
                    const i32x4 v = *(const QG_LDS i32x4*)(img + r * 256 + ((cc ^ (r & 15)) << 4));
                    // non-temporal: the output is not re-read, keep L2 and MALL for A and B
                    __builtin_nontemporal_store(v, (i32x4*)(cbase + (long long)u * 4 * LDC));
                }
            } else {
                float* cw = (float*)p.c + (long long)bz * p.c_batch + (long long)(m0 + wm * 128) * LDC + n0 + wn * 128;
#pragma unroll
                for (int i = 0; i < NBLK; ++i)
#pragma unroll
                    for (int j = 0; j < NBLK; ++j)
#pragma unroll
                        for (int v4 = 0; v4 < NV4; ++v4) {
                            const Acc& a = acc[i][j];
                            *(f32x4*)(cw + (long long)out_row(i) * LDC + out_col(j, v4)) =
                                f32x4{a[4 * v4], a[4 * v4 + 1], a[4 * v4 + 2], a[4 * v4 + 3]};
                        }
            }
            continue;
        }
        // edge tiles: masked element stores
#pragma unroll
        for (int i = 0; i < NBLK; ++i) {
            const int mm = m0 + wm * 128 + out_row(i);
            if (mm < M) {
#pragma unroll
                for (int j = 0; j < NBLK; ++j)
#pragma unroll
                    for (int v4 = 0; v4 < NV4; ++v4) {
                        const int nn = n0 + wn * 128 + out_col(j, v4);
                        const Acc& a = acc[i][j];
                        const f32x4 v = f32x4{a[4 * v4], a[4 * v4 + 1], a[4 * v4 + 2], a[4 * v4 + 3]};
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
}

}  // namespace qg
