// Row-run decode GEMM for gfx950: MXFP8 / MXFP4 with row-major B, 16 < M <= 64.
//
// A decode GEMM streams B once, so the rate at which a load pattern streams
// row-major B is the ceiling.  Measured on MI355X (copy-only replays, 224
// workgroups, 16 B per lane): loads that take 512 B or 1 KB contiguous of
// one or two rows per instruction stream 5.1-5.3 TB/s; the 16-row MFMA
// fragment order (16 rows x 64 B per instruction) and 8 rows x 128 B whole
// lines stay at 3.7-4.2 TB/s.  The skinny, band and decode kernels read B
// per 128-byte K-tile (an MFMA operand needs 16 rows of one K-tile), which
// caps them there.  This kernel reads B in runs instead:
//
//  * a workgroup (8 waves) owns 32 columns of C (two 16-row blocks of B), all
//    M (<= 64) rows, and a slice of K; the slice runs in stages of 4 K-tiles
//    (512 bytes of every row);
//  * per stage each wave issues 2 B loads (rows 2u, 2u + 1: lanes 0-31 take
//    one row's 512-byte run, lanes 32-63 the next), MB A loads of the same
//    form (A is L2-resident) and one scale load; the loads land in
//    registers D stages ahead of their use (D x ~33 KB in flight per CU);
//  * a stage's registers are written into one of two LDS buffers (rows of
//    512 B, 16-byte chunk c of row r at c ^ (r % 16): the fragment reads
//    below touch 16 rows of one chunk and so hit all 64 banks once), one
//    barrier, then wave w computes K-tile w % 4 of the stage for B block
//    w / 4 and every A block from LDS: scaled 16x16x128 MFMAs (fp4: two per
//    K-tile) with the E8M0 bytes from LDS panels written by the same stage;
//  * the four waves of a B block sum their partial tiles in K-tile order
//    through LDS (deterministic); a K split over workgroups uses the
//    epoch-tagged counters and device-coherent partials of common.hpp, and
//    the last workgroup of a tile sums the slices in slice order.
//
// K-tiles past the slice (a slice length that is not a multiple of 4) are
// loaded as they lie (the buffer range stops at the end of B) and written
// to LDS as zeros, data and scale bytes alike, so they add nothing.
//
// Register layout of the scaled MFMA 16x16x128 (probe.hip): operand lane
// L = 16q + r holds row r, fp8 16-byte chunks q and q + 4 of the 128-byte
// K-tile (fp4: chunk q in the first, q + 4 in the second instruction);
// lane group q's scale byte covers those 32 elements; srcA = B, srcB = A;
// the accumulator of lane L holds C[m = r][n = 4q .. 4q + 3].
#pragma once
#include <utility>

#include "tile_args.hpp"

namespace qg {

struct RunsArgs {
    TileArgs t;           // operands, shapes, strides (tiles_* / group_m unused)
    float* ws;            // fp32 partials [splitk][batch][M][N] (splitk > 1)
    unsigned* counters;   // [batch][n_tiles]: epoch-tagged arrival counters
    unsigned epoch;       // this launch's counter epoch (split_arrive)
    int splitk, kt_per_split, n_tiles;
    long long b_bytes;    // bytes of B per batch entry (the load range)
};

constexpr int kRunsWaves = 8;
constexpr int kRunsStage = 4;     // K-tiles per stage: 512 bytes of each row
constexpr int kRunsDepth = 4;     // stages of loads in flight per wave
constexpr int kRunsCols = 32;     // columns of C per workgroup

namespace runs {
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
// LDS bytes of one stage buffer: B [32][512], A [16 MB][512], then the scale
// panels SB [32][4 KT_SC], SA [16 MB][4 KT_SC]
__host__ __device__ constexpr int buf_bytes(int mb, bool fp4) {
    return (kRunsCols + 16 * mb) * (kRunsStage * 128 + kRunsStage * (fp4 ? 8 : 4));
}
}  // namespace runs

// NST: stages per workgroup (the host's slice is at most 4 NST K-tiles)
template <int FMT, int MB, int NST, bool BF16>
__global__ __launch_bounds__(kRunsWaves * 64, 1) void runs_gemm_kernel(const RunsArgs ra) {
    constexpr bool FP4 = FMT == kFmtFp4;
    static_assert(MB == 1 || MB == 2 || MB == 4, "A rows: 16, 32 or 64");
    constexpr int BKB = 128, ST = kRunsStage, D = kRunsDepth;
    constexpr int RUN = ST * BKB;                 // bytes of a row per stage
    constexpr int RA = 16 * MB, RB = kRunsCols;   // A rows, B rows per workgroup
    constexpr int KT_SC = FP4 ? 8 : 4;            // scale bytes per row and K-tile
    constexpr int SC_RUN = ST * KT_SC;            // scale bytes per row and stage
    constexpr int OFF_A = RB * RUN, OFF_SB = OFF_A + RA * RUN, OFF_SA = OFF_SB + RB * SC_RUN;
    constexpr int BUF = runs::buf_bytes(MB, FP4);
    static_assert(OFF_SA + RA * SC_RUN == BUF, "buffer layout");
    constexpr int RED = kRunsWaves * MB * 1024;   // the waves' partial tiles (f32x4 per lane per block)
    // + 1 KB where the waves without a scale job write their (empty) scale
    // loads: the write stays unconditional, and a conditional one let the
    // compiler sink that load next to it, behind a wait for every load
    constexpr int SINK = 2 * BUF > RED ? 2 * BUF : RED;
    constexpr int LDS_BYTES = SINK + 1024;
    // scale loads: rows per 16-byte-per-lane instruction (fp4 two lanes per
    // row, fp8 one: lanes past the rows repeat the last ones and are not written)
    constexpr int SC_LANES = SC_RUN / 16;         // lanes per row: 2 (fp4) or 1 (fp8)
    constexpr int SC_ROWS = 64 / SC_LANES;        // rows per instruction
    constexpr int SA_INSTR = (RA + SC_ROWS - 1) / SC_ROWS;
    static_assert(1 + SA_INSTR <= kRunsWaves, "one scale load per wave");
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
    const int nst = (kt_end - kt_begin + ST - 1) / ST;    // stages of the slice
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), L = tid & 63;
    const int q = L >> 4, l16 = L & 15;
    if (ra.splitk > 1 && tid == 0) split_claim(ra.counters + (long long)bz * ra.n_tiles + nt, ra.epoch);

    const uint8_t* A = p.a + bz * p.a_batch;
    const uint8_t* B = p.b + bz * p.b_batch;
    const uint8_t* SFA = p.sfa + bz * p.sfa_batch;
    const uint8_t* SFB = p.sfb + bz * p.sfb_batch;
    // loads at K offset koff (bytes, wave-uniform) of an operand of `range`
    // bytes: the base moves by koff and the range shrinks by it, so that the
    // hardware's bounds check (the VGPR offset against the range; the SGPR
    // offset is not checked) returns zeros for every byte past the operand
    auto rsrc = [](const uint8_t* base, int range, int koff) __attribute__((always_inline)) {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base) + koff, 0, range > koff ? range - koff : 0,
                                                 0x00020000);
    };
    // load ranges: each operand's own extent, so the K-tiles past the end of
    // the last row (read and then zeroed) load nothing past the buffer
    const int b_range = (int)min(ra.b_bytes, 0x7fffffffLL);
    const int a_range = (M - 1) * LDA + p.kbytes;
    const int sa_range = (M - 1) * SFA_SM + nk * KT_SC, sb_range = (N - 1) * SFB_SN + nk * KT_SC;

    // ---- per-lane load offsets (the stage's K offset moves the descriptor's base) ----
    // B load j of wave w: rows 2u, 2u + 1 of the tile (u = 2w + j); lane L:
    // row + L / 32, 16-byte chunk L % 32 of the 512-byte run
    const int run_c = L & 31;              // chunk of the run this lane loads
    const int run_kt = run_c >> 3;         // its K-tile within the stage
    int b_off[2], b_row[2], a_off[MB], a_row[MB];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        b_row[j] = 2 * (2 * w + j) + (L >> 5);
        b_off[j] = min(n0 + b_row[j], N - 1) * LDB + run_c * 16;
    }
#pragma unroll
    for (int j = 0; j < MB; ++j) {
        a_row[j] = 2 * (MB * w + j) + (L >> 5);
        a_off[j] = min(a_row[j], M - 1) * LDA + run_c * 16;
    }
    // scale load: wave 0 the B panel, waves 1 .. SA_INSTR the A panel; lane
    // L: row L / SC_LANES (+ SC_ROWS per A instruction), 16-byte piece L % SC_LANES
    const int sc_piece = L % SC_LANES;
    const int sc_row = (w == 0 ? 0 : (w - 1) * SC_ROWS) + L / SC_LANES;
    const bool sc_is_b = w == 0, sc_job = w <= SA_INSTR;
    const bool sc_write = sc_job && sc_row < (sc_is_b ? RB : RA);
    const int sc_off = sc_is_b ? min(n0 + sc_row, N - 1) * SFB_SN + sc_piece * 16
                               : min(sc_row, M - 1) * SFA_SM + sc_piece * 16;

    i32x4 bq[D][2], aq[D][MB], sq[D];
    // loads of stage s into register slot d; stages past the slice load
    // through empty descriptors (no traffic, zeros) so every wave issues the
    // same count per stage and the waits stay exact
    auto issue = [&](auto dd, int s) __attribute__((always_inline)) {
        constexpr int d = decltype(dd)::value;
        const bool live = s < nst;
        const int kt0 = kt_begin + s * ST;
        const auto rB = rsrc(B, live ? b_range : 0, kt0 * BKB), rA = rsrc(A, live ? a_range : 0, kt0 * BKB);
        const auto rS = rsrc(sc_is_b ? SFB : SFA, live && sc_job ? (sc_is_b ? sb_range : sa_range) : 0, kt0 * KT_SC);
#pragma unroll
        for (int j = 0; j < 2; ++j)
            bq[d][j] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(rB, b_off[j], 0, 2));
#pragma unroll
        for (int j = 0; j < MB; ++j)
            aq[d][j] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(rA, a_off[j], 0, 0));
        sq[d] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(rS, sc_off, 0, 0));
    };
    // register slot d -> LDS buffer of stage s, K-tiles past the slice as zeros
    auto write = [&](auto dd, int s) __attribute__((always_inline)) {
        constexpr int d = decltype(dd)::value;
        QG_LDS uint8_t* buf = lds + (s & 1) * BUF;
        const int kt0 = kt_begin + s * ST;
        const bool kt_ok = kt0 + run_kt < kt_end;
        const i32x4 z = {0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < 2; ++j)
            *(QG_LDS i32x4*)(buf + b_row[j] * RUN + ((run_c ^ (b_row[j] & 15)) << 4)) = kt_ok ? bq[d][j] : z;
#pragma unroll
        for (int j = 0; j < MB; ++j)
            *(QG_LDS i32x4*)(buf + OFF_A + a_row[j] * RUN + ((run_c ^ (a_row[j] & 15)) << 4)) = kt_ok ? aq[d][j] : z;
        {
            // the piece's K-tiles: fp4 2 x 8 bytes (K-tiles 2 piece, 2 piece + 1),
            // fp8 4 x 4 bytes
            i32x4 v = sq[d];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int kt = kt0 + (FP4 ? 2 * sc_piece + e / 2 : e);
                if (kt >= kt_end) v[e] = 0;
            }
            *(QG_LDS i32x4*)(sc_write ? buf + (sc_is_b ? OFF_SB : OFF_SA) + sc_row * SC_RUN + sc_piece * 16
                                      : lds + SINK + L * 16) = v;
        }
    };

    // ---- compute: wave w takes K-tile w % 4 of each stage, B block w / 4 ----
    const int ct = w & 3, cb = w >> 2;
    const int frag_b = (16 * cb + l16) * RUN;
    const int frag_lo = ((ct * 8 + q) ^ l16) << 4, frag_hi = ((ct * 8 + 4 + q) ^ l16) << 4;
    f32x4 acc[MB];
#pragma unroll
    for (int i = 0; i < MB; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto compute = [&](int s) __attribute__((always_inline)) {
        const QG_LDS uint8_t* buf = lds + (s & 1) * BUF;
        const i32x4 b_lo = *(const QG_LDS i32x4*)(buf + frag_b + frag_lo);
        const i32x4 b_hi = *(const QG_LDS i32x4*)(buf + frag_b + frag_hi);
        // scale bytes of the K-tile: fp4 8 (lane group q: bytes q and q + 4), fp8 4 (byte q)
        const QG_LDS uint8_t* sbp = buf + OFF_SB + (16 * cb + l16) * SC_RUN + ct * KT_SC;
        int sb0, sb1 = 0;
        if constexpr (FP4) {
            const u32x2 x = *(const QG_LDS u32x2*)sbp;
            sb0 = (int)(x[0] >> (8 * q));
            sb1 = (int)(x[1] >> (8 * q));
        } else {
            sb0 = (int)(*(const QG_LDS uint32_t*)sbp >> (8 * q));
        }
#pragma unroll
        for (int i = 0; i < MB; ++i) {
            const int ar = (16 * i + l16) * RUN;
            const i32x4 a_lo = *(const QG_LDS i32x4*)(buf + OFF_A + ar + frag_lo);
            const i32x4 a_hi = *(const QG_LDS i32x4*)(buf + OFF_A + ar + frag_hi);
            const QG_LDS uint8_t* sap = buf + OFF_SA + (16 * i + l16) * SC_RUN + ct * KT_SC;
            if constexpr (FP4) {
                const u32x2 x = *(const QG_LDS u32x2*)sap;
                const int sa0 = (int)(x[0] >> (8 * q)), sa1 = (int)(x[1] >> (8 * q));
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
    };

    // ---- the stages, straight-line code (NST of them, a compile-time count:
    // with a loop the compiler's wait counts lost track of the register slots
    // at the back edge and drained every load at its top); D stages of loads
    // in flight; stages past the slice (a shorter last slice) load nothing and
    // add zeros ----
    runs::static_for<(D < NST ? D : NST)>([&](auto dd) __attribute__((always_inline)) {
        issue(dd, decltype(dd)::value);
    });
    runs::static_for<NST>([&](auto ss) __attribute__((always_inline)) {
        constexpr int s = decltype(ss)::value;
        write(runs::I<s % D>{}, s);      // waits for slot s % D's loads (the compiler's exact vmcnt)
        if constexpr (s + D < NST) issue(runs::I<s % D>{}, s + D);
        __syncthreads();                 // stage s is in LDS; every wave is done with stage s - 2
        compute(s);
        __builtin_amdgcn_sched_barrier(0);
    });

    // ---- the four waves of each B block: partial tiles summed in K-tile order ----
    __syncthreads();
    f32x4* red = (f32x4*)lds_mem;
#pragma unroll
    for (int i = 0; i < MB; ++i) red[(w * MB + i) * 64 + L] = acc[i];
    __syncthreads();
    // unit u = (b, i) of the tile -> wave u; rows 16 i + l16, columns n0 + 16 b + 4 q
    constexpr int UNITS = 2 * MB;
    const int u = w, ub = u / MB, ui = u % MB;
    const bool has_unit = u < UNITS;
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if (has_unit) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const f32x4 x = red[((4 * ub + t) * MB + ui) * 64 + L];
#pragma unroll
            for (int r = 0; r < 4; ++r) v[r] += x[r];
        }
    }
    const int m = 16 * ui + l16, n = n0 + 16 * ub + 4 * q;

    auto store_c = [&](f32x4 x) __attribute__((always_inline)) {
        if (!has_unit || m >= M) return;
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
        store_c(v);
        return;
    }

    // ---- split-K: partial tile out, the last workgroup of the tile sums ----
    const long long plane = (long long)M * N;
    const long long split_stride = (long long)batch * plane;
    const bool vec_ok = (N & 3) == 0;
    if (has_unit && m < M) {
        const auto part = partial_rsrc(ra.ws + ((long long)sk * batch + bz) * plane);
        const int e = m * N + n;
        if (n + 3 < N && vec_ok) {
            store_partial4(part, e, v);
        } else {
            for (int r = 0; r < 4; ++r)
                if (n + r < N) store_partial1(part, e + r, v[r]);
        }
    }
    wait_vmcnt<0>();
    __syncthreads();
    unsigned* ctr = ra.counters + (long long)bz * ra.n_tiles + nt;
    if (tid == 0) last_flag = split_arrive(ctr, ra.epoch, ra.splitk);
    __syncthreads();
    if (!last_flag) return;
    if (has_unit && m < M) {
        const float* ws0 = ra.ws + (long long)bz * plane;
        const int e = m * N + n;
        f32x4 sum = {0.f, 0.f, 0.f, 0.f};
        if (n + 3 < N && vec_ok) {
            for (int s0 = 0; s0 < ra.splitk; s0 += 16) {
                f32x4 x[16];
#pragma unroll
                for (int s = 0; s < 16; ++s)
                    if (s0 + s < ra.splitk) x[s] = load_partial4(partial_rsrc(ws0 + (s0 + s) * split_stride), e);
#pragma unroll
                for (int s = 0; s < 16; ++s)
                    if (s0 + s < ra.splitk)
#pragma unroll
                        for (int r = 0; r < 4; ++r) sum[r] += x[s][r];
            }
        } else {
            for (int s = 0; s < ra.splitk; ++s) {
                const auto src = partial_rsrc(ws0 + s * split_stride);
                for (int r = 0; r < 4; ++r)
                    if (n + r < N) sum[r] += load_partial1(src, e + r);
            }
        }
        store_c(sum);
    }
    __syncthreads();
    if (tid == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace qg
