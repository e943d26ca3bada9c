// Row-streaming decode kernel for MX operands with row-major B (M <= 4).
//
// Decode GEMMs are bound by how fast B leaves HBM.  A 16x16x128 MFMA
// fragment takes 16 rows x 64 (fp4) or 128 (fp8) bytes, and loads in that
// order stream row-major B at ~3.7 TB/s on MI355X, while loads that each take
// 1 KB of one row stream at ~5.2 TB/s (copy-only replays of a 7168 x 8 KB
// matrix, same launch shape).  This kernel feeds the matrix core from whole
// 1 KB row pieces:
//
//   * one MFMA covers 2048 K elements of ONE row of B (a "piece": 1 KB of
//     fp4, 2 KB of fp8) against the same 2048 K elements of one row of A.
//     Operand row i of the B side holds K-chunk i of the piece, operand row
//     j of the A side holds K-chunk j of A, so D[i][j] = chunk i of B times
//     chunk j of A and the row's dot product is the trace of D.  Only the 16
//     diagonal entries are used: per MFMA the A side is one row of A, so the
//     matrix work is M MFMAs per piece and the kernel is for M <= 4 (MB =
//     1, 2 or 4 rows of A; the code takes MB = 8 too);
//   * the chunk of a lane is chosen so that one load instruction reads the
//     piece's 1 KB contiguously and each lane's 32 elements (fp4) or two
//     16-element halves (fp8) are exactly the E8M0 groups its scale byte
//     covers: fp4 lane (q, i) = 16q + i holds group 4i + q (bytes 64i + 16q);
//     fp8 lane (q, i) holds bytes 64i + 16q of each 1 KB half h (groups
//     32h + 2i + q/2), its scale byte scales logical block q, i.e. group
//     32(q/2) + 2i + q%2;
//   * a workgroup (8 waves) owns R consecutive rows of B (R*np pieces, np =
//     pieces per row); wave w takes pieces [wT, wT + T) of them in row order,
//     so each wave walks its rows front to back and the workgroup's loads
//     cover its rows contiguously; D pieces per wave are in flight in
//     registers (no LDS for B);
//   * A (all M rows, every piece) and its scales are copied into LDS once
//     per workgroup, in lane order, so the MFMA operand of (m, piece) is one
//     conflict-free 16-byte LDS read per lane and half;
//   * a wave chains the MFMAs of one row and one m into one accumulator;
//     when the row (or the wave's range) ends, each lane picks its diagonal
//     entry (lane 20g + r holds D[4g + r][4g + r] in register r), quads sum
//     by DPP and lanes 0, 20, 40, 60 write four partial sums per (row, m) to
//     LDS; the workgroup then adds, for each output, the partials of the
//     (at most two) waves that covered its row in wave order -- a fixed
//     order, so results are deterministic;
//   * tails: lanes past K load through an out-of-range offset (zeros, no
//     traffic), so the last piece may be partial (K a multiple of 128 (fp8)
//     or 256 (fp4), the MX entries' contract); pieces past a wave's range
//     load through an empty buffer descriptor.
//
// Follows the MX GEMM semantics of MX8 host.cc:96-122 / MX4 host.cc:66-115:
// y[m][n] = sum_k a[m][k] * 2^(sfa-127) * b[n][k] * 2^(sfb-127).
#pragma once
#include <utility>
#include "tile_args.hpp"

namespace qg {

struct StreamArgs {
    TileArgs t;
    int rows_per_wg;    // R: rows of B (output columns) per workgroup, 1 .. kStreamMaxRows
};

constexpr int kStreamWaves = 8;
constexpr int kStreamMaxRows = 56;        // keeps a wave within kStreamRowsPerWave rows
constexpr int kStreamRowsPerWave = 8;
constexpr int kStreamMaxK = 16384;        // K held in LDS: A rows (8 or 16 KB) and their scales
constexpr int kStreamXsBytes = 512;       // A scale bytes per row held in LDS (K / 32)
constexpr int kStreamWsBytes = 16384;     // the workgroup's B scales: R rows x 256 * ceil(np / 4) bytes

namespace strm {
template <int N, class F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl<N>(f, std::make_integer_sequence<int, N>{});
}
}  // namespace strm

template <bool FP4, int MB, bool BF16>
__global__ __launch_bounds__(kStreamWaves * 64, 1) void stream_gemm_kernel(const StreamArgs sa) {
    static_assert(MB == 1 || MB == 2 || MB == 4 || MB == 8, "1, 2, 4 or 8 rows of A");
    constexpr int NH = FP4 ? 1 : 2;              // 1 KB halves per piece
    constexpr int PIECE = 1024 * NH;             // bytes of one row per MFMA (2048 K elements)
    constexpr int D = FP4 ? 8 : 4;               // pieces in flight per wave
    constexpr int FMT = FP4 ? kFmtFp4 : kFmtFp8;
    constexpr int OOB = 0x40000000;              // voffset past every descriptor's range
    constexpr int XB = kStreamMaxK / (FP4 ? 2 : 1);                   // A image bytes per row
    constexpr int XS_CH = (MB * kStreamXsBytes / 256) < kStreamWaves ? kStreamWaves : MB * kStreamXsBytes / 256;
    constexpr int RW = kStreamRowsPerWave;

    __shared__ __attribute__((aligned(1024))) uint8_t xi[MB * XB];
    __shared__ __attribute__((aligned(256))) uint8_t xs[XS_CH * 256];
    __shared__ __attribute__((aligned(256))) uint8_t wsi[kStreamWsBytes];
    __shared__ float part[kStreamWaves][RW][MB][4];

    const TileArgs& p = sa.t;
    const int tid = threadIdx.x, L = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int li = L & 15, lq = L >> 4;
    const int bz = blockIdx.y;
    const int r0 = blockIdx.x * sa.rows_per_wg;
    const int R = min(sa.rows_per_wg, p.n - r0);
    const int M = p.m, KB = p.kbytes, ldb = p.ldb, lds = p.sfb_sn;
    const int np = (KB + PIECE - 1) / PIECE;
    const int ngroups = FP4 ? KB / 16 : KB / 32;     // E8M0 groups (32 elements) per row
    const int plast = (ngroups % 64) ? np - 1 : np;   // index of a partial last piece (np: none)

    // per-lane byte offsets inside a piece and the groups they belong to
    int voff[NH], vlast[NH];
#pragma unroll
    for (int h = 0; h < NH; ++h) {
        voff[h] = h * 1024 + 64 * li + 16 * lq;
        const int g = FP4 ? 4 * li + lq : 32 * h + 2 * li + (lq >> 1);
        vlast[h] = 64 * (np - 1) + g < ngroups ? voff[h] : OOB;
    }
    const int gs = FP4 ? 4 * li + lq : 32 * (lq >> 1) + 2 * li + (lq & 1);   // the lane's scale group
    const int wsp = 256 * ((np + 3) / 4);        // B scale image: bytes per row (whole 256-byte DMAs)

    // ---- A and its scales into LDS (lane order), issued first -------------
    {
        const uint8_t* A = p.a + (long long)bz * p.a_batch;
        const auto rA = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(A), 0, M * p.lda, 0x00020000);
        constexpr int XC = MB * (XB / 1024) / kStreamWaves;   // 1 KB chunks per wave
#pragma unroll
        for (int j = 0; j < XC; ++j) {
            const int c = w + kStreamWaves * j;
            const int m = c / (XB / 1024), ph = c % (XB / 1024);
            const int pc = ph / NH, h = ph % NH;
            const int g = FP4 ? 4 * li + lq : 32 * h + 2 * li + (lq >> 1);
            int v = OOB;
            if (m < M && 64 * pc + g < ngroups) v = m * p.lda + pc * PIECE + h * 1024 + 64 * li + 16 * lq;
            dma16_buf(rA, (QG_LDS uint8_t*)xi + c * 1024, v, 0);
        }
        const uint8_t* SA = p.sfa + (long long)bz * p.sfa_batch;
        const auto rS = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(SA), 0, M * p.sfa_sm, 0x00020000);
#pragma unroll
        for (int j = 0; j < XS_CH / kStreamWaves; ++j) {
            const int c = w + kStreamWaves * j;
            const int m = c / (kStreamXsBytes / 256), off = (c % (kStreamXsBytes / 256)) * 256 + 4 * L;
            const int v = (m < M && off < ngroups) ? m * p.sfa_sm + off : OOB;
            dma4_buf(rS, (QG_LDS uint8_t*)xs + c * 256, v, 0);
        }
        // B scales of the workgroup's R rows: one 64-byte run per piece
        // would cost a load instruction per piece, as many as the data
        const uint8_t* SB = p.sfb + (long long)bz * p.sfb_batch + (long long)r0 * lds;
        const auto rW = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(SB), 0, R * lds, 0x00020000);
        const int cpr = wsp / 256;
#pragma unroll
        for (int j = 0; j < kStreamWsBytes / 256 / kStreamWaves; ++j) {
            const int c = w + kStreamWaves * j;
            const int row = c / cpr, off = (c - row * cpr) * 256 + 4 * L;
            const int v = (row < R && off < ngroups) ? row * lds + off : OOB;
            dma4_buf(rW, (QG_LDS uint8_t*)wsi + c * 256, v, 0);
        }
    }

    // ---- this wave's pieces ------------------------------------------------
    const int P = R * np;
    const int T = (P + kStreamWaves - 1) / kStreamWaves;
    const int tb = min(w * T, P), te = min(tb + T, P);
    // (wave-uniform; the division runs in VALU, so say so for the scalar offsets)
    const int fr = __builtin_amdgcn_readfirstlane(tb / np);   // first row this wave touches
    const int fp = __builtin_amdgcn_readfirstlane(tb - fr * np);

    const uint8_t* Bw = p.b + (long long)bz * p.b_batch + (long long)r0 * ldb;

    i32x4 wd[D][NH];
    int lt = tb, lrow = fr, lp = fp;             // next piece to load
    auto issue = [&](auto dI) __attribute__((always_inline)) {
        constexpr int d = decltype(dI)::value;
        const bool ok = lt < te;    // past the range: empty descriptors (zeros, no traffic)
        const auto rd = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(Bw), 0, ok ? R * ldb : 0, 0x00020000);
        const bool last = lp == plast;
        const int soff = lrow * ldb + lp * PIECE;
#pragma unroll
        for (int h = 0; h < NH; ++h)
            wd[d][h] = __builtin_bit_cast(
                i32x4, __builtin_amdgcn_raw_buffer_load_b128(rd, last ? vlast[h] : voff[h], soff, 2 /* nt */));
        ++lt;
        if (++lp == np) { lp = 0; ++lrow; }
    };
    strm::static_for<D>(issue);
    // the LDS images' DMAs were issued before the D * NH loads of the ring
    wait_vmcnt<D * NH>();
    __syncthreads();

    f32x4 acc[MB];
#pragma unroll
    for (int m = 0; m < MB; ++m) acc[m] = f32x4{0.f, 0.f, 0.f, 0.f};
    const bool diag = ((L & 15) >> 2) == (L >> 4);
    const bool writer = diag && (L & 3) == 0;    // lanes 0, 20, 40, 60

    auto flush = [&](int rl) __attribute__((always_inline)) {
#pragma unroll
        for (int m = 0; m < MB; ++m) {
            const f32x4 a = acc[m];
            const float v0 = (L & 1) ? a[1] : a[0];
            const float v1 = (L & 1) ? a[3] : a[2];
            float v = (L & 2) ? v1 : v0;
            v = diag ? v : 0.f;
            v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
            v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
            if (writer) part[w][rl][m][L >> 4] = v;
            acc[m] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    };

    int ct = tb, crow = fr, cp = fp;             // next piece to consume
    // A operands of the next piece: read from LDS one piece ahead, so their
    // latency hides behind the current piece's MFMAs
    i32x4 xq[MB][NH];
    int xsq[MB], wsq;
    auto xload = [&](int row, int pc) __attribute__((always_inline)) {
        wsq = ((const QG_LDS uint8_t*)wsi)[row * wsp + pc * 64 + gs];
#pragma unroll
        for (int m = 0; m < MB; ++m) {
            const QG_LDS uint8_t* x = (const QG_LDS uint8_t*)xi + m * XB + pc * PIECE + 16 * L;
#pragma unroll
            for (int h = 0; h < NH; ++h) xq[m][h] = *(const QG_LDS i32x4*)(x + h * 1024);
            xsq[m] = ((const QG_LDS uint8_t*)xs)[m * kStreamXsBytes + pc * 64 + gs];
        }
    };
    xload(crow, cp);
    auto consume = [&](auto dI) __attribute__((always_inline)) {
        constexpr int d = decltype(dI)::value;
        if (ct < te) {
            i32x8 bf;
            if constexpr (FP4) bf = i32x8{wd[d][0][0], wd[d][0][1], wd[d][0][2], wd[d][0][3], 0, 0, 0, 0};
            else bf = i32x8{wd[d][0][0], wd[d][0][1], wd[d][0][2], wd[d][0][3],
                            wd[d][1][0], wd[d][1][1], wd[d][1][2], wd[d][1][3]};
            i32x8 af[MB];
            int xsc[MB];
            const int wsc = wsq;
#pragma unroll
            for (int m = 0; m < MB; ++m) {
                if constexpr (FP4) af[m] = i32x8{xq[m][0][0], xq[m][0][1], xq[m][0][2], xq[m][0][3], 0, 0, 0, 0};
                else af[m] = i32x8{xq[m][0][0], xq[m][0][1], xq[m][0][2], xq[m][0][3],
                                   xq[m][1][0], xq[m][1][1], xq[m][1][2], xq[m][1][3]};
                xsc[m] = xsq[m];
            }
            const bool row_end = cp == np - 1 || ct == te - 1;
            const int rl = crow - fr;
            ++ct;
            if (++cp == np) { cp = 0; ++crow; }
            xload(min(crow, R - 1), cp);    // (past the wave's range: read, never used)
#pragma unroll
            for (int m = 0; m < MB; ++m)
                acc[m] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bf, af[m], acc[m], FMT, FMT, 0, wsc,
                                                                          0, xsc[m]);
            if (row_end) flush(rl);
        }
    };

    for (int t0 = tb; t0 < te; t0 += D) {
        strm::static_for<D>([&](auto dI) __attribute__((always_inline)) {
            consume(dI);
            issue(dI);
        });
    }
    wait_vmcnt<0>();
    __syncthreads();

    // ---- outputs: the partials of the waves that covered each row ---------
    if (T > 0) {
        for (int idx = tid; idx < MB * R; idx += kStreamWaves * 64) {
            const int m = idx / R, rl = idx - m * R;
            if (m >= M) continue;
            const int wlo = (rl * np) / T, whi = (rl * np + np - 1) / T;
            float s = 0.f;
            for (int ww = wlo; ww <= whi; ++ww) {
                const float* pp = part[ww][rl - (ww * T) / np][m];
                s += pp[0];
                s += pp[1];
                s += pp[2];
                s += pp[3];
            }
            const long long o = (long long)bz * p.c_batch + (long long)m * p.ldc + r0 + rl;
            if constexpr (BF16) ((uint16_t*)p.c)[o] = bf16_bits(s);
            else ((float*)p.c)[o] = s;
        }
    }
}

}  // namespace qg
