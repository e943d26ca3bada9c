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
//     descriptor;
//   * K split: A's LDS image holds 16384 K elements per row, so longer K
//     splits over workgroups (grid.z); each writes fp32 partials
//     device-coherently, and the last workgroup of each row block (relaxed
//     counter, see store_partial4 in common.hpp) adds the slices in slice
//     order and re-arms the counter;
//   * why M <= 8: a 16x16x128 MFMA with fp4 operands runs at the fp8 rate,
//     and only 1 / CH of its products are used, so the matrix work is
//     (16 / WR) x the GEMM's; at WR = 4 and M = 32 (N = 7168, K = 16384,
//     K split 4 ways) the kernel took 33 us against the skinny kernel's
//     19.7 us (full 16-row fragments).
//
// Follows the MX GEMM semantics of MX8 host.cc:96-122 / MX4 host.cc:66-115:
// y[m][n] = sum_k a[m][k] * 2^(sfa-127) * b[n][k] * 2^(sfb-127).
#pragma once
#include <utility>
#include "tile_args.hpp"

namespace qg {

struct StreamArgs {
    TileArgs t;
    int rows_per_wg;      // R: rows of B (output columns) per workgroup, 1 .. stream_max_rows(wr)
    int splitk;           // K slices (grid.z)
    int seg_per_split;    // segments per slice (stream_seg_cap at most)
    float* ws;            // splitk > 1: fp32 partials [splitk][batch][M][N]
    unsigned* counters;   // splitk > 1: one per (batch, row block), epoch-tagged arrival counters
    unsigned epoch;       // this launch's counter epoch (split_arrive)
};

constexpr int kStreamWaves = 8;
constexpr int kStreamGroupsPerWave = 8;   // row groups one wave may touch
constexpr int kStreamWsBytes = 16384;     // the workgroup's B scales: R rows x (slice groups, power of 2)

// A image bytes per row of A held in LDS: 16384 K elements
__host__ __device__ constexpr int stream_xbytes(bool fp4, int mb) {
    return (void)mb, 16384 / (fp4 ? 2 : 1);
}
// segments of one K slice (a segment: 2048 / wr K elements of a row)
__host__ __device__ constexpr int stream_seg_cap(bool fp4, int wr, int mb) {
    return stream_xbytes(fp4, mb) / ((fp4 ? 1024 : 2048) / wr);
}
// log2 of the B scale image's row pitch for a slice of `groups` E8M0 groups
__host__ __device__ constexpr int stream_ws_log2(int groups) {
    int l = 2;
    while ((1 << l) < groups) ++l;
    return l;
}
// rows per workgroup: kStreamGroupsPerWave - 1 row groups per wave at most
__host__ __device__ constexpr int stream_max_rows(int wr) { return wr * kStreamWaves * (kStreamGroupsPerWave - 1); }

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
    // pieces in flight per wave: 4 (1 KB fp4 / 2 KB fp8 each); configs[4]
    // M = 1 / 8 with fp4: D = 4, 5, 6, 8 -> 12.7, 12.8, 12.9, 13.4 us / 13.9,
    // 14.3, 14.3, 15.0 us (fewer requests in flight per wave keep each row's
    // reads closer together); fp8 M = 1: D = 3, 4, 6 -> 21.1, 20.7, 21.1 us
    constexpr int D = 4;
    constexpr int FMT = FP4 ? kFmtFp4 : kFmtFp8;
    constexpr int OOB = 0x40000000;              // voffset past every descriptor's range
    constexpr int XB = stream_xbytes(FP4, MB);   // A image bytes per row
    constexpr int XSB = (XB * (FP4 ? 2 : 1) / 32) < 256 ? 256 : XB * (FP4 ? 2 : 1) / 32;   // A scale bytes per row
    constexpr int XS_CH = (MB * XSB / 256) < kStreamWaves ? kStreamWaves : MB * XSB / 256;
    constexpr int RG = kStreamGroupsPerWave;

    __shared__ __attribute__((aligned(1024))) uint8_t xi[MB * XB];
    __shared__ __attribute__((aligned(256))) uint8_t xs[XS_CH * 256];
    __shared__ __attribute__((aligned(256))) uint8_t wsi[kStreamWsBytes];
    __shared__ float part[kStreamWaves][RG][4 * MB];
    __shared__ int last_flag;

    const TileArgs& p = sa.t;
    const int tid = threadIdx.x, L = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int li = L & 15, lq = L >> 4;
    const int lr = li / CH, lc = li % CH;        // the lane's operand row: (row of its group, chunk)
    const int bz = blockIdx.y, z = blockIdx.z;
    if (sa.splitk > 1 && tid == 0) split_claim(sa.counters + (long long)bz * gridDim.x + blockIdx.x, sa.epoch);
    const int r0 = blockIdx.x * sa.rows_per_wg;
    const int R = min(sa.rows_per_wg, p.n - r0);
    const int M = p.m, KB = p.kbytes, ldb = p.ldb, lds = p.sfb_sn;
    const int nseg_all = (KB + SEG - 1) / SEG;
    const int s0 = z * sa.seg_per_split;                      // this slice's first segment
    const int nseg = min(sa.seg_per_split, nseg_all - s0);    // and its segments
    const int nrg = (R + WR - 1) / WR;
    const int ngroups = FP4 ? KB / 16 : KB / 32;     // E8M0 groups (32 elements) per row
    const int slast = ((ngroups % GPS) ? nseg_all - 1 : nseg_all) - s0;   // local index of a partial last segment

    // per-lane byte offsets inside a segment and the groups they belong to
    int voff[NH], vlast[NH];
#pragma unroll
    for (int h = 0; h < NH; ++h) {
        voff[h] = lr * ldb + h * H + 64 * lc + 16 * lq;
        const int g = FP4 ? 4 * lc + lq : h * (H / 32) + 2 * lc + (lq >> 1);
        vlast[h] = GPS * (nseg_all - 1) + g < ngroups ? voff[h] : OOB;
    }
    const int gs = FP4 ? 4 * lc + lq : (lq >> 1) * (H / 32) + 2 * lc + (lq & 1);   // the lane's scale group
    // B scale image: the slice's groups of each row (zeros past K), row pitch
    // the power of two >= every group a lane of the slice reads
    const int sgroups = min(nseg * GPS, ngroups - s0 * GPS);
    const int wsl = stream_ws_log2(nseg * GPS);
    const int wsp = 1 << wsl;

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
            if (m < M && s < nseg && GPS * (s0 + s) + g < ngroups)
                v = m * p.lda + (s0 + s) * SEG + h * H + 64 * lc + 16 * lq;
            dma16_buf(rA, (QG_LDS uint8_t*)xi + c * 1024, v, 0);
        }
        const uint8_t* SA = p.sfa + (long long)bz * p.sfa_batch;
        const auto rS = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(SA), 0, M * p.sfa_sm, 0x00020000);
#pragma unroll
        for (int j = 0; j < XS_CH / kStreamWaves; ++j) {
            const int c = w + kStreamWaves * j;
            const int m = c / (XSB / 256), off = (c % (XSB / 256)) * 256 + 4 * L;
            const int v = (m < M && off < sgroups) ? m * p.sfa_sm + s0 * GPS + off : OOB;
            dma4_buf(rS, (QG_LDS uint8_t*)xs + c * 256, v, 0);
        }
        // B scales of the workgroup's R rows (a 64-byte scale load per piece
        // would cost as many load instructions as the data)
        const uint8_t* SB = p.sfb + (long long)bz * p.sfb_batch + (long long)r0 * lds;
        const auto rW = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(SB), 0, R * lds, 0x00020000);
#pragma unroll
        for (int j = 0; j < kStreamWsBytes / 256 / kStreamWaves; ++j) {
            const int c = w + kStreamWaves * j;
            const int b = c * 256 + 4 * L, row = b >> wsl, off = b & (wsp - 1);
            const int v = (row < R && off < sgroups) ? row * lds + s0 * GPS + off : OOB;
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
        const int soff = lg * WR * ldb + (s0 + ls) * SEG;
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
            xsq[g] = ((const QG_LDS uint8_t*)xs)[(g * WR + lr) * XSB + s * GPS + gs];
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
    auto row_sum = [&](int m, int rl) __attribute__((always_inline)) {
        const int rg = rl / WR, wr = rl - rg * WR;
        const int wlo = (rg * nseg) / T, whi = (rg * nseg + nseg - 1) / T;
        float s = 0.f;
        for (int ww = wlo; ww <= whi; ++ww) {
            const float* pp = &part[ww][rg - (ww * T) / nseg][(wr * MB + m) * NE];
#pragma unroll
            for (int k = 0; k < NE; ++k) s += pp[k];
        }
        return s;
    };
    auto store_c = [&](int m, int rl, float v) __attribute__((always_inline)) {
        const long long o = (long long)bz * p.c_batch + (long long)m * p.ldc + r0 + rl;
        if constexpr (BF16) ((uint16_t*)p.c)[o] = bf16_bits(v);
        else ((float*)p.c)[o] = v;
    };
    if (sa.splitk == 1) {
        for (int idx = tid; idx < MB * R; idx += kStreamWaves * 64) {
            const int m = idx / R, rl = idx - m * R;
            if (m < M) store_c(m, rl, row_sum(m, rl));
        }
        return;
    }
    const int N = p.n;
    const long long plane = (long long)M * N;
    const int nbatch = gridDim.y;
    const auto mine = partial_rsrc(sa.ws + ((long long)z * nbatch + bz) * plane);
    for (int idx = tid; idx < MB * R; idx += kStreamWaves * 64) {
        const int m = idx / R, rl = idx - m * R;
        if (m < M) store_partial1(mine, m * N + r0 + rl, row_sum(m, rl));
    }
    wait_vmcnt<0>();
    __syncthreads();
    unsigned* ctr = sa.counters + (long long)bz * gridDim.x + blockIdx.x;
    if (tid == 0)
        last_flag = split_arrive(ctr, sa.epoch, sa.splitk);
    __syncthreads();
    if (!last_flag) return;
    for (int idx = tid; idx < MB * R; idx += kStreamWaves * 64) {
        const int m = idx / R, rl = idx - m * R;
        if (m >= M) continue;
        float v = 0.f;
        for (int zz = 0; zz < sa.splitk; ++zz)
            v += load_partial1(partial_rsrc(sa.ws + ((long long)zz * nbatch + bz) * plane), m * N + r0 + rl);
        store_c(m, rl, v);
    }
    if (tid == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace qg
