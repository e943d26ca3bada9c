// Slice decode GEMM for gfx950: MXFP8 / MXFP4 with row-major B, M <= 64.
//
// What bounds a decode GEMM's loads on MI355X (copy-only replays, 224
// workgroups, 16 B per lane, configs[4]'s 7168 x 8 KB B):
//  * B straight from HBM in MFMA-fragment order (16 rows x 64 B per load)
//    streams 5.3 TB/s when each wave walks one 16-row block over a contiguous
//    2 KB of K (whether 8 or 32 loads are in flight), but 3.7 TB/s when each
//    wave walks two blocks over 1 KB;
//  * a CU takes L2-resident data at ~31 GB/s in fragment order but ~75 GB/s
//    in 1 KB runs, and what it loads from L2 delays its B loads: every wave
//    re-reading A's fragments from L2 (as the skinny kernel does) adds ~7 us
//    per 256 KB of A per workgroup, while 128 KB of A in 1 KB runs adds 1.5.
// So here:
//  * a workgroup (8 waves) owns 16 NBW columns of C, all M (<= 64) rows and a
//    K slice of KPS K-tiles, with NBW x KQ = 8 and KPS = 16 KQ chosen so that
//    the slice of A is 128 KB (MB = 1, 2, 4 blocks of 16 A rows: NBW = 2, 4,
//    8; KQ = 4, 2, 1; KPS = 64, 32, 16);
//  * it loads the slice of A (1 KB of one row per instruction) and the
//    slice's E8M0 bytes of A and of its B rows into LDS once, then one
//    barrier;
//  * wave w takes B block w / KQ over the contiguous 16 K-tiles (2 KB)
//    (w % KQ) of the slice: each K-tile's two fragment loads (bytes 0-63 and
//    64-127 of 16 rows) go straight into registers, D K-tiles ahead, and meet
//    A's fragments read from LDS -- B never passes through LDS and no wave
//    waits for another inside the K loop; row-major B loads with the default
//    cache policy (the non-temporal one ran configs[4] M = 1-64 10-15%
//    slower), W16 B non-temporal;
//  * the KQ waves of a block add their tiles in K order through LDS; a K
//    split over workgroups uses the epoch-tagged counters and device-coherent
//    partials of common.hpp, the last workgroup of a tile summing the slices
//    in slice order.
//
// Every load's descriptor starts at its K offset with the operand's range
// shrunk by it (the hardware checks the VGPR offset against the range, not
// the SGPR offset), so no byte past an operand is read; B K-tiles past the
// slice load through an empty descriptor (zeros), and A's and the scales'
// K-tiles past it are written to LDS as zeros, so they add nothing.
//
// Register layout of the scaled MFMA 16x16x128 (probe.hip): operand lane
// L = 16q + r holds row r, 16-byte chunks q and q + 4 of the 128-byte K-tile
// (fp8: one MFMA; fp4: chunk q in the first MFMA, q + 4 in the second); lane
// group q's scale byte covers those 32 elements; srcA = B, srcB = A; the
// accumulator of lane L holds C[m = r][n = 4q .. 4q + 3].
//
// W16 (MXFP4 in aiter's gemm_a4w4 bpreshuffle formats): B in
// shuffle_weight(16,16) order, where a 16-row block's K-tile is 2 KB laid out
// [8 chunks][16 rows][16 B], so the lane order above makes each fragment
// load one contiguous 1 KB run; scales in e8m0_shuffle order (per 32-row
// block and K-tile 256 bytes, the dword at q * 64 + (r % 16) * 4 holding
// groups q and q + 4 of rows r % 16 and 16 + r % 16).  A's slice of those
// bytes comes into LDS as it lies; the wave's B scale dword of each K-tile
// is loaded with its B fragments.
#pragma once
#include <utility>

#include "runs_gemm.hpp"

namespace qg {

constexpr int kSliceWaves = 8;
constexpr int kSliceKtw = 16;      // K-tiles per wave: 2 KB of each of its 16 B rows
constexpr int kSliceDepth = 8;     // K-tiles of B loads in flight per wave
__host__ __device__ constexpr int slice_nbw(int mb) { return mb == 1 ? 2 : (mb == 2 ? 4 : 8); }
__host__ __device__ constexpr int slice_kq(int mb) { return kSliceWaves / slice_nbw(mb); }
__host__ __device__ constexpr int slice_kps(int mb) { return kSliceKtw * slice_kq(mb); }

template <int FMT, int MB, bool BF16, bool W16 = false>
__global__ __launch_bounds__(kSliceWaves * 64, 1) void slice_gemm_kernel(const RunsArgs ra) {
    constexpr bool FP4 = FMT == kFmtFp4;
    static_assert(MB == 1 || MB == 2 || MB == 4, "A rows: 16, 32 or 64");
    static_assert(!W16 || FP4, "W16 / e8m0_shuffle operands: MXFP4");
    constexpr int BKB = 128, KW = kSliceKtw, D = kSliceDepth;
    constexpr int NBW = slice_nbw(MB), KQ = slice_kq(MB), KPS = slice_kps(MB);
    constexpr int RA = 16 * MB, RB = 16 * NBW;
    constexpr int KT_SC = FP4 ? 8 : 4;            // scale bytes per row and K-tile
    constexpr int A_ROW = KPS * BKB;              // A row of the slice in LDS
    static_assert(RA * A_ROW == 128 * 1024, "A slice: 128 KB");
    // scales in LDS as [K-tile][row] entries of KT_SC bytes: a fragment's 16
    // rows read one contiguous 64 / 128 bytes
    constexpr int SA_KT = RA * KT_SC, SB_KT = RB * KT_SC;
    // W16: A's e8m0_shuffle bytes of the slice, [32-row block][K-tile][256]
    constexpr int NBA = (RA + 31) / 32, SA_W = NBA * KPS * 256;
    constexpr int OFF_SA = RA * A_ROW, OFF_SB = OFF_SA + (W16 ? SA_W : KPS * SA_KT);
    constexpr int LDS_BYTES = W16 ? OFF_SB : OFF_SB + KPS * SB_KT;
    static_assert(LDS_BYTES <= 160 * 1024, "LDS");
    static_assert(kSliceWaves * MB * 64 * 16 <= RA * A_ROW, "the waves' partial tiles fit the A image");
    // A loads: 1 KB of one row each, 16 per wave
    constexpr int A_PIECES = A_ROW / 1024, A_PER_WAVE = RA * A_PIECES / kSliceWaves;
    static_assert(A_PER_WAVE == 16, "A loads per wave");
    // scale loads: 16-byte pieces (16 / KT_SC K-tiles of one row), A's rows then B's
    constexpr int SPR = KPS * KT_SC / 16;                 // pieces per row
    constexpr int S_PIECES = (RA + RB) * SPR;
    constexpr int S_PER_WAVE = (S_PIECES / 64 + kSliceWaves - 1) / kSliceWaves;
    constexpr int KT_PER_PIECE = 16 / KT_SC;
    static_assert(RA * SPR % 64 == 0, "A's and B's scale pieces meet at an instruction boundary");
    constexpr int SW_PIECES = SA_W / 16, SW_PER_WAVE = (SW_PIECES / 64 + kSliceWaves - 1) / kSliceWaves;
    static_assert(SW_PIECES % 64 == 0, "W16: A's scale pieces fill whole instructions");
    __shared__ __attribute__((aligned(16))) uint8_t lds_mem[LDS_BYTES];
    __shared__ int last_flag;
    QG_LDS uint8_t* const lds = (QG_LDS uint8_t*)lds_mem;

    const TileArgs& p = ra.t;
    const int M = p.m, N = p.n, LDA = p.lda, LDB = p.ldb, LDC = p.ldc;
    const int SFA_SM = p.sfa_sm, SFB_SN = p.sfb_sn;
    const int nk = p.kbytes / BKB;
    const int nt = blockIdx.x % ra.n_tiles, sk = blockIdx.x / ra.n_tiles, bz = blockIdx.y, batch = gridDim.y;
    const int n0 = nt * RB;
    const int kt_begin = sk * ra.kt_per_split;
    const int kt_end = min(nk, kt_begin + ra.kt_per_split);
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), L = tid & 63;
    const int q = L >> 4, l16 = L & 15;
    const int bw = w / KQ, kq = w % KQ;    // the wave's B block and K part
    if (ra.splitk > 1 && tid == 0) split_claim(ra.counters + (long long)bz * ra.n_tiles + nt, ra.epoch);

    const uint8_t* A = p.a + bz * p.a_batch;
    const uint8_t* B = p.b + bz * p.b_batch;
    const uint8_t* SFA = p.sfa + bz * p.sfa_batch;
    const uint8_t* SFB = p.sfb + bz * p.sfb_batch;
    // loads at K offset koff (bytes, wave-uniform) of an operand of `range`
    // bytes: the base moves by koff and the range shrinks by it
    auto rsrc = [](const uint8_t* base, int range, int koff, bool live) __attribute__((always_inline)) {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base) + koff, 0,
                                                 live && range > koff ? range - koff : 0, 0x00020000);
    };
    const int b_range = (int)min(ra.b_bytes, 0x7fffffffLL);
    const int a_range = (M - 1) * LDA + p.kbytes;
    // W16: SFA_SM / SFB_SN are the bytes of one 32-row block, K-tile step 256
    const int rows32a = (M + 31) / 32, rows32b = (N + 31) / 32;
    const int sa_range = W16 ? (rows32a - 1) * SFA_SM + nk * 256 : (M - 1) * SFA_SM + nk * KT_SC;
    const int sb_range = (N - 1) * SFB_SN + nk * KT_SC;
    const i32x4 z = {0, 0, 0, 0};

    // ---- A's slice and the scale bytes -> registers (issued first) ----
    const auto rA = rsrc(A, a_range, kt_begin * BKB, true);
    i32x4 av[A_PER_WAVE];
#pragma unroll
    for (int j = 0; j < A_PER_WAVE; ++j) {
        const int g = w * A_PER_WAVE + j, row = g / A_PIECES, pc = g % A_PIECES;
        av[j] = __builtin_bit_cast(
            i32x4, __builtin_amdgcn_raw_buffer_load_b128(rA, min(row, M - 1) * LDA + pc * 1024 + L * 16, 0, 0));
    }
    i32x4 sv[W16 ? SW_PER_WAVE : S_PER_WAVE];
    if constexpr (W16) {
        // A's e8m0_shuffle bytes of the slice: KPS * 256 contiguous bytes per
        // 32-row block; blocks past the last read zeros
        const auto rSA = rsrc(SFA, sa_range, kt_begin * 256, true);
#pragma unroll
        for (int j = 0; j < SW_PER_WAVE; ++j) {
            const int pc = (w + j * kSliceWaves) * 64 + L, blk = pc / (KPS * 16), within = pc % (KPS * 16);
            sv[j] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                  rSA, pc < SW_PIECES ? blk * SFA_SM + within * 16 : 0, 0, 0));
        }
    }
    const auto rSA = rsrc(SFA, sa_range, kt_begin * KT_SC, !W16);
    const auto rSB = rsrc(SFB + (long long)n0 * SFB_SN, sb_range - n0 * SFB_SN, kt_begin * KT_SC, !W16);
#pragma unroll
    for (int j = 0; j < (W16 ? 0 : S_PER_WAVE); ++j) {
        const int ins = w + j * kSliceWaves, pc = ins * 64 + L;    // instruction, piece
        const bool is_a = ins * 64 < RA * SPR;                      // wave-uniform
        const int pr = is_a ? pc : pc - RA * SPR, row = pr / SPR, piece = pr % SPR;
        const bool live = pc < S_PIECES;
        const int off = is_a ? min(row, M - 1) * SFA_SM + piece * 16 : min(row, N - 1 - n0) * SFB_SN + piece * 16;
        // lanes past the pieces load piece 0 of row 0 and are not written
        sv[j] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(is_a ? rSA : rSB,
                                                                                 live ? off : 0, 0, 0));
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- the wave's B: 16 rows, K-tiles [kt_w, kt_w + KW) ----
    const int kt_w = kt_begin + kq * KW;
    // W16: the wave's 16-row block blk16 (its K-tile kt at blk16 * 16 * LDB +
    // kt * 2048; a block past N reads zeros) and its scale dwords (32-row
    // block blk16 / 2, half blk16 % 2)
    const int blk16 = n0 / 16 + bw;
    const auto rB = W16 ? rsrc(B, b_range, blk16 * 16 * LDB + kt_w * 2048, true) : rsrc(B, b_range, kt_w * BKB, true);
    const auto rZ = rsrc(B, 0, 0, false);
    const auto rSW = rsrc(SFB + (long long)(blk16 >> 1) * SFB_SN, nk * 256, kt_w * 256, W16 && (blk16 >> 1) < rows32b);
    const int b_off = W16 ? L * 16 : min(n0 + 16 * bw + l16, N - 1) * LDB + q * 16;
    constexpr int B_KT = W16 ? 2048 : BKB, B_HI = W16 ? 1024 : 64;
    // cache policy of the B loads: non-temporal for W16 (aiter configs[4]
    // M = 32 / 64 18.4 / 22.1 -> 16.5 / 20.5 us with the rotated walk), the
    // default for row-major B (non-temporal 5-8% slower there)
    constexpr int B_AUX = W16 ? 2 : 0;
    i32x4 bq[D][2];
    int bsw[D];
    // step j of the wave's walk takes K-tile jr(j) of its part.  Without the
    // rotation every wave of the grid reads the same 2 KB offset of a 32 KB
    // K window at the same step, and with W16's contiguous 2 KB K-tiles those
    // reads crowd into few HBM channels: rotating by wave, K part and tile
    // (weights replayed from HBM, one box: W16 configs[4] M = 16 / 32 / 48 /
    // 64 14.0 / 19.2 / 24.2 / 26.3 -> 13.8 / 18.2 / 20.3 / 22.0 us; row-major
    // 64-row plans 2.8-3.2% faster, its 16-row plans 2% slower, so those keep
    // the plain walk)
    const int rot = W16 || MB == 4 ? (5 * bw + 3 * kq + 7 * nt) & (KW - 1) : 0;
    auto jr = [&](int j) __attribute__((always_inline)) { return (j + rot) & (KW - 1); };
    auto issue = [&](auto dd, int j) __attribute__((always_inline)) {
        constexpr int d = decltype(dd)::value;
        const int jj = jr(j);
        const auto r = kt_w + jj < kt_end ? rB : rZ;
        bq[d][0] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(r, b_off + jj * B_KT, 0, B_AUX));
        bq[d][1] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(r, b_off + jj * B_KT + B_HI, 0, B_AUX));
        if constexpr (W16)
            bsw[d] = (int)__builtin_amdgcn_raw_buffer_load_b32(kt_w + jj < kt_end ? rSW : rZ, jj * 256 + L * 4, 0, 0);
    };
    runs::static_for<D>([&](auto dd) __attribute__((always_inline)) { issue(dd, decltype(dd)::value); });
    __builtin_amdgcn_sched_barrier(0);

    // A into LDS: chunk c of row r at c ^ (r % 16); K-tiles past the slice as zeros
#pragma unroll
    for (int j = 0; j < A_PER_WAVE; ++j) {
        const int g = w * A_PER_WAVE + j, row = g / A_PIECES, pc = g % A_PIECES;
        const int c = pc * 64 + L;
        *(QG_LDS i32x4*)(lds + row * A_ROW + ((c ^ (row & 15)) << 4)) = kt_begin + (c >> 3) < kt_end ? av[j] : z;
    }
    // W16: A's scale bytes as they lie, K-tiles past the slice as zeros
    if constexpr (W16) {
#pragma unroll
        for (int j = 0; j < SW_PER_WAVE; ++j) {
            const int pc = (w + j * kSliceWaves) * 64 + L;
            if (pc < SW_PIECES)
                *(QG_LDS i32x4*)(lds + OFF_SA + pc * 16) = kt_begin + (pc % (KPS * 16)) / 16 < kt_end ? sv[j] : z;
        }
    }
    // scale pieces into [K-tile][row]
#pragma unroll
    for (int j = 0; j < (W16 ? 0 : S_PER_WAVE); ++j) {
        const int ins = w + j * kSliceWaves, pc = ins * 64 + L;
        if (pc < S_PIECES) {
            const bool is_a = ins * 64 < RA * SPR;
            const int pr = is_a ? pc : pc - RA * SPR, row = pr / SPR, piece = pr % SPR;
            QG_LDS uint8_t* dst = lds + (is_a ? OFF_SA + row * KT_SC : OFF_SB + row * KT_SC);
            const int kt0 = piece * KT_PER_PIECE;
#pragma unroll
            for (int e = 0; e < KT_PER_PIECE; ++e) {
                const bool ok = kt_begin + kt0 + e < kt_end;
                if constexpr (FP4) {
                    *(QG_LDS u32x2*)(dst + (kt0 + e) * (is_a ? SA_KT : SB_KT)) =
                        ok ? u32x2{(uint32_t)sv[j][2 * e], (uint32_t)sv[j][2 * e + 1]} : u32x2{0u, 0u};
                } else {
                    *(QG_LDS uint32_t*)(dst + (kt0 + e) * (is_a ? SA_KT : SB_KT)) = ok ? (uint32_t)sv[j][e] : 0u;
                }
            }
        }
    }
    __syncthreads();

    // ---- K loop: K-tile j of the wave's part, slice K-tile kq * KW + j ----
    f32x4 acc[MB];
#pragma unroll
    for (int i = 0; i < MB; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    runs::static_for<KW>([&](auto jj) __attribute__((always_inline)) {
        constexpr int j = decltype(jj)::value;
        const int kt = kq * KW + jr(j);
        const i32x4 b_lo = bq[j % D][0], b_hi = bq[j % D][1];
        const QG_LDS uint8_t* sbp = lds + OFF_SB + kt * SB_KT + (16 * bw + l16) * KT_SC;
        int sb0, sb1 = 0;
        if constexpr (W16) {
            // bytes hB (groups 0-3) and 2 + hB (groups 4-7) of the dword, hB = blk16 % 2
            const int x = bsw[j % D] >> (8 * (blk16 & 1));
            sb0 = x;
            sb1 = x >> 16;
        } else if constexpr (FP4) {
            const u32x2 x = *(const QG_LDS u32x2*)sbp;
            sb0 = (int)(x[0] >> (8 * q));
            sb1 = (int)(x[1] >> (8 * q));
        } else {
            sb0 = (int)(*(const QG_LDS uint32_t*)sbp >> (8 * q));
        }
        const int alo = ((kt * 8 + q) ^ l16) << 4, ahi = ((kt * 8 + 4 + q) ^ l16) << 4;
#pragma unroll
        for (int i = 0; i < MB; ++i) {
            const QG_LDS uint8_t* arow = lds + (16 * i + l16) * A_ROW;
            const i32x4 a_lo = *(const QG_LDS i32x4*)(arow + alo);
            const i32x4 a_hi = *(const QG_LDS i32x4*)(arow + ahi);
            const QG_LDS uint8_t* sap = W16 ? lds + OFF_SA + ((i >> 1) * KPS + kt) * 256 + L * 4
                                            : lds + OFF_SA + kt * SA_KT + (16 * i + l16) * KT_SC;
            if constexpr (FP4) {
                int sa0, sa1;
                if constexpr (W16) {
                    // rows 16 i + r: half i % 2 of 32-row block i / 2
                    const int x = (int)(*(const QG_LDS uint32_t*)sap >> (8 * (i & 1)));
                    sa0 = x;
                    sa1 = x >> 16;
                } else {
                    const u32x2 x = *(const QG_LDS u32x2*)sap;
                    sa0 = (int)(x[0] >> (8 * q));
                    sa1 = (int)(x[1] >> (8 * q));
                }
                const i32x8 b0 = i32x8{b_lo[0], b_lo[1], b_lo[2], b_lo[3], 0, 0, 0, 0};
                const i32x8 b1 = i32x8{b_hi[0], b_hi[1], b_hi[2], b_hi[3], 0, 0, 0, 0};
                const i32x8 a0 = i32x8{a_lo[0], a_lo[1], a_lo[2], a_lo[3], 0, 0, 0, 0};
                const i32x8 a1 = i32x8{a_hi[0], a_hi[1], a_hi[2], a_hi[3], 0, 0, 0, 0};
                acc[i] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(b0, a0, acc[i], kFmtFp4, kFmtFp4, 0, sb0, 0,
                                                                         sa0);
                acc[i] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(b1, a1, acc[i], kFmtFp4, kFmtFp4, 0, sb1, 0,
                                                                         sa1);
            } else {
                const int sa0 = (int)(*(const QG_LDS uint32_t*)sap >> (8 * q));
                const i32x8 bf = i32x8{b_lo[0], b_lo[1], b_lo[2], b_lo[3], b_hi[0], b_hi[1], b_hi[2], b_hi[3]};
                const i32x8 af = i32x8{a_lo[0], a_lo[1], a_lo[2], a_lo[3], a_hi[0], a_hi[1], a_hi[2], a_hi[3]};
                acc[i] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bf, af, acc[i], kFmtFp8, kFmtFp8, 0, sb0, 0,
                                                                         sa0);
            }
        }
        (void)sb1;
        if constexpr (j + D < KW) issue(runs::I<j % D>{}, j + D);
        __builtin_amdgcn_sched_barrier(0);
    });

    // ---- the KQ waves of a block: tiles summed in K order through LDS ----
    if constexpr (KQ > 1) {
        __syncthreads();    // every wave is done with the A image
        f32x4* red = (f32x4*)lds_mem;
#pragma unroll
        for (int i = 0; i < MB; ++i) red[(w * MB + i) * 64 + L] = acc[i];
        __syncthreads();
        if (kq == 0) {
#pragma unroll
            for (int i = 0; i < MB; ++i) {
                f32x4 v = red[((bw * KQ) * MB + i) * 64 + L];
#pragma unroll
                for (int t = 1; t < KQ; ++t) {
                    const f32x4 x = red[((bw * KQ + t) * MB + i) * 64 + L];
#pragma unroll
                    for (int r = 0; r < 4; ++r) v[r] += x[r];
                }
                acc[i] = v;
            }
        }
    }

    // ---- epilogue (the K part 0 wave of each block): lane's outputs
    // C[16 i + l16][n0 + 16 bw + 4 q + 0..3] ----
    const bool owner = kq == 0;
    const int n = n0 + 16 * bw + 4 * q;
    auto store_c = [&](int m, f32x4 x) __attribute__((always_inline)) {
        if (!owner || m >= M || n >= N) return;
        if constexpr (BF16) {
            uint16_t* c = (uint16_t*)p.c + bz * p.c_batch + (long long)m * LDC + n;
            if (n + 3 < N && p.c_vec >= 4) {
                *(u32x2*)c = u32x2{pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3])};
            } else {
                for (int r = 0; r < 4; ++r)
                    if (n + r < N) c[r] = bf16_bits(x[r]);
            }
        } else {
            float* c = (float*)p.c + bz * p.c_batch + (long long)m * LDC + n;
            if (n + 3 < N && p.c_vec >= 4) {
                *(f32x4*)c = x;
            } else {
                for (int r = 0; r < 4; ++r)
                    if (n + r < N) c[r] = x[r];
            }
        }
    };
    if (ra.splitk == 1) {
#pragma unroll
        for (int i = 0; i < MB; ++i) store_c(16 * i + l16, acc[i]);
        return;
    }

    // ---- split-K: partial tile out, the last workgroup of the tile sums ----
    const long long plane = (long long)M * N;
    const long long split_stride = (long long)batch * plane;
    const bool vec_ok = (N & 3) == 0;
    if (owner) {
        const auto part = partial_rsrc(ra.ws + ((long long)sk * batch + bz) * plane);
#pragma unroll
        for (int i = 0; i < MB; ++i) {
            const int m = 16 * i + l16;
            if (m < M && n < N) {
                const int e = m * N + n;
                if (n + 3 < N && vec_ok) {
                    store_partial4(part, e, acc[i]);
                } else {
                    for (int r = 0; r < 4; ++r)
                        if (n + r < N) store_partial1(part, e + r, acc[i][r]);
                }
            }
        }
    }
    wait_vmcnt<0>();
    __syncthreads();
    unsigned* ctr = ra.counters + (long long)bz * ra.n_tiles + nt;
    if (tid == 0) last_flag = split_arrive(ctr, ra.epoch, ra.splitk);
    __syncthreads();
    if (!last_flag) return;
    if (owner && n + 3 < N && vec_ok) {
        // every row block's loads of a group of SG slices in flight before
        // the adds (one round trip per group, not one per row block); the
        // slices summed in order 0 .. splitk - 1, this workgroup's own slice
        // from its registers (the bits it stored)
        constexpr int SG = 16 / MB < 8 ? 16 / MB : 8;
        const float* ws0 = ra.ws + (long long)bz * plane;
        f32x4 sum[MB];
#pragma unroll
        for (int i = 0; i < MB; ++i) sum[i] = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int s0 = 0; s0 < ra.splitk; s0 += SG) {
            f32x4 x[SG][MB];
#pragma unroll
            for (int s = 0; s < SG; ++s)
#pragma unroll
                for (int i = 0; i < MB; ++i)
                    if (s0 + s < ra.splitk && s0 + s != sk && 16 * i + l16 < M)
                        x[s][i] = load_partial4(partial_rsrc(ws0 + (s0 + s) * split_stride), (16 * i + l16) * N + n);
#pragma unroll
            for (int s = 0; s < SG; ++s)
#pragma unroll
                for (int i = 0; i < MB; ++i)
                    if (s0 + s < ra.splitk && 16 * i + l16 < M) sum[i] += s0 + s == sk ? acc[i] : x[s][i];
        }
#pragma unroll
        for (int i = 0; i < MB; ++i) store_c(16 * i + l16, sum[i]);
    } else if (owner) {
        const float* ws0 = ra.ws + (long long)bz * plane;
#pragma unroll
        for (int i = 0; i < MB; ++i) {
            const int m = 16 * i + l16;
            if (m >= M || n >= N) continue;
            const int e = m * N + n;
            f32x4 sum = {0.f, 0.f, 0.f, 0.f};
            for (int s = 0; s < ra.splitk; ++s) {
                const auto src = partial_rsrc(ws0 + s * split_stride);
                for (int r = 0; r < 4; ++r)
                    if (n + r < N) sum[r] += load_partial1(src, e + r);
            }
            store_c(m, sum);
        }
    }
    __syncthreads();
    if (tid == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace qg
