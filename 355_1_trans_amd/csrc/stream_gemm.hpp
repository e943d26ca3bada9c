// Row-streaming decode kernel for MX operands with row-major B (small M).
//
// Decode GEMMs are bound by how fast B leaves HBM.  A 16x16x128 MFMA
// fragment takes 16 rows x 64 (fp4) or 128 (fp8) bytes, and loads in that
// order stream row-major B at ~3.8 TB/s on MI355X, while loads that each take
// 1 KB of one row stream at ~5.3 TB/s and 2 rows x 512 B at ~5.1 TB/s
// (copy-only replays of a 7168 x 8 KB matrix, same launch shape).  This
// kernel feeds the matrix core from such long row runs:
//
//   * one MFMA covers WR rows of B (WR = 1, 2 or 4) over a *segment* of
//     2048 / WR K elements each, against WR rows of A over the same K:
//     operand row i of the B side is (B row i / CH, K-chunk i % CH), operand
//     row j of the A side is (A row j / CH, K-chunk j % CH), CH = 16 / WR
//     chunks of 128 K.  D[i][j] multiplies chunk c of a B row by chunk c' of
//     an A row; the entries with c == c' sum, over the CH chunks, to the
//     WR x WR dot products of the segment, the others are discarded.  The
//     matrix work is M / WR MFMAs per WR x segment of B ("piece"), so WR = 1
//     suits M = 1, larger WR larger M; each load instruction still reads
//     1 KB: WR rows x 1024 / WR contiguous bytes;
//   * the chunk of a lane is chosen so that each lane's 32 elements (fp4) or
//     two 16-element halves (fp8) are exactly the E8M0 groups its scale
//     byte covers: lane (q, i) = 16q + i, chunk c = i % CH, holds fp4 bytes
//     64c + 16q of its row's segment (group 4c + q), or fp8 bytes 64c + 16q
//     of each half h of the segment (groups h * H/32 + 2c + q/2, H = 1024/WR
//     bytes per half); its scale byte scales logical block q, i.e. group
//     (q/2) * H/32 + 2c + q%2 -- the 16x16x128 operand and scale layouts
//     pinned by the layout probes;
//   * a workgroup (8 waves) owns R consecutive rows of B, in groups of WR;
//     wave w takes pieces [wT, wT + T) of the (row group, segment) pieces in
//     row order, so each wave walks its rows front to back and the
//     workgroup's loads cover its rows contiguously; D pieces per wave are
//     in flight in registers (no LDS for B);
//   * A (all M rows, every segment, in lane order), A's scales and the
//     workgroup's B scales are DMA'd into LDS once; the A operands and scale
//     bytes of the next piece are read from LDS while the current piece's
//     MFMAs run;
//   * a wave chains one row group's MFMAs per group of WR rows of A; when
//     the row group (or the wave's range) ends, each lane picks its one
//     useful register (lane L: register L % 4, when its two chunks match),
//     quads add by DPP and the quads' first lanes write partial sums to
//     LDS; the workgroup then adds, for each output, the partials of the (at
//     most two) waves that covered its row group in wave order -- a fixed
//     order, so results are deterministic;
//   * tails: lanes past K or past the workgroup's last row load through an
//     out-of-range offset (zeros, no traffic), so K needs no multiple of the
//     segment (K a multiple of 128 (fp8) or 256 (fp4), the MX entries'
//     contract); pieces past a wave's range load through an empty buffer
//     descriptor.
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
constexpr int kStreamMaxRows = 56;        // keeps a wave within kStreamGroupsPerWave row groups
constexpr int kStreamGroupsPerWave = 8;
constexpr int kStreamMaxK = 16384;        // K held in LDS: A rows (8 or 16 KB) and their scales
constexpr int kStreamXsBytes = 512;       // A scale bytes per row held in LDS (K / 32)
constexpr int kStreamWsBytes = 16384;     // the workgroup's B scales: R rows x 256 * ceil(K/8192) bytes

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

template <bool FP4, int WR, int MB, bool BF16>
__global__ __launch_bounds__(kStreamWaves * 64, 1) void stream_gemm_kernel(const StreamArgs sa) {
    static_assert(WR == 1 || WR == 2 || WR == 4, "1, 2 or 4 rows of B per MFMA");
    static_assert(MB % WR == 0 && MB <= 8, "rows of A: a multiple of WR, at most 8");
    constexpr int NH = FP4 ? 1 : 2;              // 1 KB load instructions per piece
    constexpr int CH = 16 / WR;                  // 128-K chunks per row and MFMA
    constexpr int H = 1024 / WR;                 // bytes of one row per load instruction
    constexpr int SEG = H * NH;                  // bytes of one row per MFMA
    constexpr int GPS = 64 / WR;                 // E8M0 groups per row and segment
    constexpr int MG = MB / WR;                  // MFMAs per piece (groups of WR rows of A)
    constexpr int NE = 4 / WR;                   // partial sums per output and wave
    constexpr int D = FP4 ? 8 : 4;               // pieces in flight per wave
    constexpr int FMT = FP4 ? kFmtFp4 : kFmtFp8;
    constexpr int OOB = 0x40000000;              // voffset past every descriptor's range
    constexpr int XB = kStreamMaxK / (FP4 ? 2 : 1);                   // A image bytes per row
    constexpr int XS_CH = (MB * kStreamXsBytes / 256) < kStreamWaves ? kStreamWaves : MB * kStreamXsBytes / 256;
    constexpr int RG = kStreamGroupsPerWave;

    __shared__ __attribute__((aligned(1024))) uint8_t xi[MB * XB];
    __shared__ __attribute__((aligned(256))) uint8_t xs[XS_CH * 256];
    __shared__ __attribute__((aligned(256))) uint8_t wsi[kStreamWsBytes];
    __shared__ float part[kStreamWaves][RG][4 * MB];

    const TileArgs& p = sa.t;
    const int tid = threadIdx.x, L = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int li = L & 15, lq = L >> 4;
    const int lr = li / CH, lc = li % CH;        // the lane's operand row: (row of its group, chunk)
    const int bz = blockIdx.y;
    const int r0 = blockIdx.x * sa.rows_per_wg;
    const int R = min(sa.rows_per_wg, p.n - r0);
    const int M = p.m, KB = p.kbytes, ldb = p.ldb, lds = p.sfb_sn;
    const int nseg = (KB + SEG - 1) / SEG;
    const int nrg = (R + WR - 1) / WR;
    const int ngroups = FP4 ? KB / 16 : KB / 32;     // E8M0 groups (32 elements) per row
    const int slast = (ngroups % GPS) ? nseg - 1 : nseg;   // index of a partial last segment (nseg: none)

    // per-lane byte offsets inside a segment and the groups they belong to
    int voff[NH], vlast[NH];
#pragma unroll
    for (int h = 0; h < NH; ++h) {
        voff[h] = lr * ldb + h * H + 64 * lc + 16 * lq;
        const int g = FP4 ? 4 * lc + lq : h * (H / 32) + 2 * lc + (lq >> 1);
        vlast[h] = GPS * (nseg - 1) + g < ngroups ? voff[h] : OOB;
    }
    const int gs = FP4 ? 4 * lc + lq : (lq >> 1) * (H / 32) + 2 * lc + (lq & 1);   // the lane's scale group
    const int wsp = 256 * ((ngroups + 255) / 256);    // B scale image: bytes per row (whole 256-byte DMAs)

    // ---- A, its scales and the workgroup's B scales into LDS, issued first --
    {
        const uint8_t* A = p.a + (long long)bz * p.a_batch;
        const auto rA = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(A), 0, M * p.lda, 0x00020000);
        constexpr int XPG = WR * XB / 1024;                       // 1 KB chunks per group of A rows
        constexpr int XC = MB * (XB / 1024) / kStreamWaves;       // 1 KB chunks per wave
#pragma unroll
        for (int j = 0; j < XC; ++j) {
            const int c = w + kStreamWaves * j;
            const int mg = c / XPG, rem = c % XPG;
            const int s = rem / NH, h = rem % NH;
            const int m = mg * WR + lr;
            const int g = FP4 ? 4 * lc + lq : h * (H / 32) + 2 * lc + (lq >> 1);
            int v = OOB;
            if (m < M && GPS * s + g < ngroups) v = m * p.lda + s * SEG + h * H + 64 * lc + 16 * lq;
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
        // B scales of the workgroup's R rows (a 64-byte scale load per piece
        // would cost as many load instructions as the data)
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
    const int P = nrg * nseg;
    const int T = (P + kStreamWaves - 1) / kStreamWaves;
    const int tb = min(w * T, P), te = min(tb + T, P);
    // (wave-uniform; the division runs in VALU, so say so for the scalar offsets)
    const int fg = __builtin_amdgcn_readfirstlane(tb / nseg);   // first row group this wave touches
    const int fs = __builtin_amdgcn_readfirstlane(tb - fg * nseg);

    const uint8_t* Bw = p.b + (long long)bz * p.b_batch + (long long)r0 * ldb;

    i32x4 wd[D][NH];
    int lt = tb, lg = fg, ls = fs;               // next piece to load
    auto issue = [&](auto dI) __attribute__((always_inline)) {
        constexpr int d = decltype(dI)::value;
        const bool ok = lt < te;    // past the range: empty descriptors (zeros, no traffic)
        const auto rd = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(Bw), 0, ok ? R * ldb : 0, 0x00020000);
        const bool last = ls == slast;
        const bool rows_cut = WR > 1 && (lg + 1) * WR > R;    // the workgroup's last, partial row group
        const int soff = lg * WR * ldb + ls * SEG;
#pragma unroll
        for (int h = 0; h < NH; ++h) {
            int v = last ? vlast[h] : voff[h];
            if (WR > 1) v = (rows_cut && lg * WR + lr >= R) ? OOB : v;
            wd[d][h] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(rd, v, soff, 2 /* nt */));
        }
        ++lt;
        if (++ls == nseg) { ls = 0; ++lg; }
    };
    strm::static_for<D>(issue);
    // the LDS images' DMAs were issued before the D * NH loads of the ring
    wait_vmcnt<D * NH>();
    __syncthreads();

    f32x4 acc[MG];
#pragma unroll
    for (int g = 0; g < MG; ++g) acc[g] = f32x4{0.f, 0.f, 0.f, 0.f};
    // lane L holds D[4q + r][L % 16] in register r: operand row 4q + r is
    // (B row (4q + r) / CH, chunk (4q + r) % CH), operand column L % 16 is
    // (A row lr, chunk lc); the chunks match in register L % 4 when
    // ((4q) % CH) / 4 == lc / 4 -- whole quads, one chunk per lane
    const bool useful = WR == 4 || ((4 * lq) % CH) / 4 == lc / 4;
    const bool writer = useful && (L & 3) == 0;
    const int e_w = ((lq * WR) / 4) * MB * NE + lr * NE + lq % NE;   // writer's slot: (B row, A row, partial)

    auto flush = [&](int gl) __attribute__((always_inline)) {
#pragma unroll
        for (int g = 0; g < MG; ++g) {
            const f32x4 a = acc[g];
            const float v0 = (L & 1) ? a[1] : a[0];
            const float v1 = (L & 1) ? a[3] : a[2];
            float v = (L & 2) ? v1 : v0;
            v = useful ? v : 0.f;
            v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
            v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
            if (writer) part[w][gl][e_w + g * WR * NE] = v;
            acc[g] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    };

    int ct = tb, cg = fg, cs = fs;               // next piece to consume
    // operands of the next piece, read from LDS one piece ahead so that
    // their latency hides behind the current piece's MFMAs
    i32x4 xq[MG][NH];
    int xsq[MG], wsq;
    auto xload = [&](int grp, int s) __attribute__((always_inline)) {
        wsq = ((const QG_LDS uint8_t*)wsi)[min(grp * WR + lr, R - 1) * wsp + s * GPS + gs];
#pragma unroll
        for (int g = 0; g < MG; ++g) {
            const QG_LDS uint8_t* x = (const QG_LDS uint8_t*)xi + g * WR * XB + s * NH * 1024 + 16 * L;
#pragma unroll
            for (int h = 0; h < NH; ++h) xq[g][h] = *(const QG_LDS i32x4*)(x + h * 1024);
            xsq[g] = ((const QG_LDS uint8_t*)xs)[(g * WR + lr) * kStreamXsBytes + s * GPS + gs];
        }
    };
    xload(cg, cs);
    auto consume = [&](auto dI) __attribute__((always_inline)) {
        constexpr int d = decltype(dI)::value;
        if (ct < te) {
            i32x8 bf;
            if constexpr (FP4) bf = i32x8{wd[d][0][0], wd[d][0][1], wd[d][0][2], wd[d][0][3], 0, 0, 0, 0};
            else bf = i32x8{wd[d][0][0], wd[d][0][1], wd[d][0][2], wd[d][0][3],
                            wd[d][1][0], wd[d][1][1], wd[d][1][2], wd[d][1][3]};
            i32x8 af[MG];
            int xsc[MG];
            const int wsc = wsq;
#pragma unroll
            for (int g = 0; g < MG; ++g) {
                if constexpr (FP4) af[g] = i32x8{xq[g][0][0], xq[g][0][1], xq[g][0][2], xq[g][0][3], 0, 0, 0, 0};
                else af[g] = i32x8{xq[g][0][0], xq[g][0][1], xq[g][0][2], xq[g][0][3],
                                   xq[g][1][0], xq[g][1][1], xq[g][1][2], xq[g][1][3]};
                xsc[g] = xsq[g];
            }
            const bool group_end = cs == nseg - 1 || ct == te - 1;
            const int gl = cg - fg;
            ++ct;
            if (++cs == nseg) { cs = 0; ++cg; }
            xload(min(cg, nrg - 1), cs);    // (past the wave's range: read, never used)
#pragma unroll
            for (int g = 0; g < MG; ++g)
                acc[g] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bf, af[g], acc[g], FMT, FMT, 0, wsc, 0,
                                                                          xsc[g]);
            if (group_end) flush(gl);
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

    // ---- outputs: the partials of the waves that covered each row group ---
    if (T > 0) {
        for (int idx = tid; idx < MB * R; idx += kStreamWaves * 64) {
            const int m = idx / R, rl = idx - m * R;
            if (m >= M) continue;
            const int rg = rl / WR, wr = rl - rg * WR;
            const int wlo = (rg * nseg) / T, whi = (rg * nseg + nseg - 1) / T;
            float s = 0.f;
            for (int ww = wlo; ww <= whi; ++ww) {
                const float* pp = &part[ww][rg - (ww * T) / nseg][(wr * MB + m) * NE];
#pragma unroll
                for (int k = 0; k < NE; ++k) s += pp[k];
            }
            const long long o = (long long)bz * p.c_batch + (long long)m * p.ldc + r0 + rl;
            if constexpr (BF16) ((uint16_t*)p.c)[o] = bf16_bits(s);
            else ((float*)p.c)[o] = s;
        }
    }
}

}  // namespace qg
