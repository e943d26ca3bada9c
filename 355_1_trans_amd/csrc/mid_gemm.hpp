// Four-wave 128 x 128 tile GEMM with split-K for the middle of the M range
// on gfx950: fp8 with fp32 block scales (BSF32), and MXFP8 / MXFP4 (MX).
//
// At M ~ 256-4096 with narrow N the 256 x 256 tiles of bsf32_gemm.hpp leave
// most of the 256 CUs idle (M = 1024, N = 2112: 36 tiles).  This kernel cuts
// the tile to 128 x 128 (4 x the tiles) and can split K over workgroups; a
// workgroup is 4 waves (one per SIMD) and two workgroups share a CU (66 KB of
// LDS each), so one workgroup's barrier and DMA waits are covered by the
// other's MFMAs.
//
//  * wave (wm, wn) = (w / 2, w % 2) owns 64 x 64 outputs: 4 x 4 blocks of
//    v_mfma_f32_16x16x128_f8f6f4 (unscaled fp8; one instruction = one
//    128-deep K-tile = one scale block), 64 VGPR accumulators, each
//    partial rescaled acc += part * (sa * sb) after the next MFMA issued;
//  * two LDS stages of one K-tile (A 128 rows, B 128 rows, the K-tile's
//    scales), one barrier per K-tile; the 9 DMAs per wave of K-tile t+1
//    (buffer_load ... lds, 4 A, 4 B, 1 scale) go into the other stage,
//    spread over K-tile t's MFMAs; DMAs past the slice use an empty-range
//    descriptor (no branches, so the compiler's DMA waits stay exact; the
//    loop is unrolled by two so every stage is its own LDS object);
//  * B' (K-panel): the tile's 128 rows of a K-tile are 16 contiguous KB;
//    B'' (the LDS-bypass entry's fragment order): 8 blocks of 2 KB, copied
//    as is and read back linearly (the block is the MFMA operand order);
//  * MX (row-major B, its rows DMA'd like A's): the K-tile's E8M0 bytes of
//    the tile's 128 A and 128 B rows ride in the stage beside the operands
//    (4 bytes per row for fp8, 8 for fp4; one or two dword DMAs per wave)
//    and the scaled MFMA applies them, accumulating in place (no VALU
//    rescale).  fp8: lane (q, r) holds chunks q and q + 4 of row r with
//    scale byte q; fp4: two MFMAs per K-tile, chunks 2q and 2q + 1 with
//    scale bytes 2q and 2q + 1 (op_sel 0 and 1 of one 16-bit read);
//  * split-K: every workgroup stores its fp32 partial tile and returns;
//    splitk_reduce_kernel, launched next on the stream, adds the slices in
//    slice order (deterministic) over the whole chip.  A last-arriving
//    workgroup summing its tile instead streams all slices back through one
//    CU at the end of the launch: 5-10 us of a 20-60 us kernel (M = 256,
//    N = 2112, K = 7168: 26.5 us vs 22.4 us with the separate reduce), and
//    it capped how deep K could split.
//
// LDS rows are 128 bytes, 16-byte chunks XOR-swizzled by row & 7.
#pragma once
#include <utility>
#include "tile_args.hpp"

namespace qg {

struct MidArgs {
    TileArgs t;            // tiles_m / tiles_n count 128 x 128 tiles
    float* ws;             // fp32 partials [splitk][batch][M][N] (splitk > 1)
    int splitk, kt_per_split;
};

// Sums the fp32 partials [splitk][batch][M][N] in slice order into C (row
// pitch ldc elements, batch stride c_batch); c_vec as in TileArgs.
struct SplitReduceArgs {
    const float* ws;
    void* c;
    int m, n, ldc, c_vec, splitk, batch;
    long long c_batch;
};

// One thread per 4 consecutive elements of a row (VEC: N % 4 == 0) or per
// element; v = ((0 + p0) + p1) + ... (slice order: the same bits on every
// run).
template <bool BF16, bool VEC>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const SplitReduceArgs r) {
    constexpr int E = VEC ? 4 : 1;
    const long long plane = (long long)r.m * r.n, total = plane * r.batch;
    const long long e = ((long long)blockIdx.x * 256 + threadIdx.x) * E;
    if (e >= total) return;
    const int bz = (int)(e / plane);
    const long long x = e - bz * plane;
    const int m = (int)(x / r.n), n = (int)(x - (long long)m * r.n);
    float v[E];
#pragma unroll
    for (int i = 0; i < E; ++i) v[i] = 0.f;
    // four slices' loads in flight before their adds (order kept); the
    // partials are read once, so nontemporal (36 split shapes: 1.01x
    // geomean, up to 1.07x)
    for (int s0 = 0; s0 < r.splitk; s0 += 4) {
        float u[4][E];
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            if (s0 + d >= r.splitk) break;
            const float* src = r.ws + (long long)(s0 + d) * total + e;
            if constexpr (VEC) {
                const f32x4 w = __builtin_nontemporal_load((const f32x4*)src);
#pragma unroll
                for (int i = 0; i < 4; ++i) u[d][i] = w[i];
            } else {
                u[d][0] = __builtin_nontemporal_load(src);
            }
        }
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            if (s0 + d >= r.splitk) break;
#pragma unroll
            for (int i = 0; i < E; ++i) v[i] += u[d][i];
        }
    }
    const long long co = (long long)bz * r.c_batch + (long long)m * r.ldc + n;
    if constexpr (BF16) {
        uint16_t* c = (uint16_t*)r.c + co;
        if (VEC && r.c_vec >= 4) {
            *(u32x2*)c = u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
        } else {
#pragma unroll
            for (int i = 0; i < E; ++i) c[i] = bf16_bits(v[i]);
        }
    } else {
        float* c = (float*)r.c + co;
        if (VEC && r.c_vec >= 4) {
            if constexpr (VEC) *(f32x4*)c = f32x4{v[0], v[1], v[2], v[3]};
        } else {
#pragma unroll
            for (int i = 0; i < E; ++i) c[i] = v[i];
        }
    }
}

namespace mid {
template <int V>
struct I {
    static constexpr int value = V;
};
template <int N, class F, int... K>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, K...>) {
    (f(I<K>{}), ...);
}
// f(I<k>) for k = 0 .. N-1, unrolled at compile time
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl<N>(f, std::make_integer_sequence<int, N>{});
}
}  // namespace mid

// SK = BSF32: fp8, fp32 block scales, B' or B''; SK = MX: fp8 or fp4 (FMT),
// E8M0 scales per 32 K, row-major B, the scales applied by the MFMA.
// NTB: B through the nontemporal cache policy (one M tile: B is read once)
template <bool BF16, BLay BL, int STAGES, ScaleKind SK = ScaleKind::BSF32, int FMT = kFmtFp8, bool NTB = false>
__global__ __launch_bounds__(256, STAGES == 2 ? 2 : 1) void mid_gemm_kernel(const MidArgs mp) {
    static_assert(STAGES == 2 || STAGES == 4, "two stages (two workgroups per CU) or four (one)");
    constexpr bool MX = (SK == ScaleKind::MX);
    constexpr bool FP4 = (FMT == kFmtFp4);
    static_assert(MX ? BL == BLay::RAW : (BL == BLay::KPANEL || BL == BLay::FRAG && !FP4),
                  "MX: row-major B; fp32 block scales: fp8 with K-panel B' or fragment-order B''");
    constexpr bool FRAG = (BL == BLay::FRAG);
    constexpr bool RAW = (BL == BLay::RAW);
    constexpr int BKB = 128, BT = 128;
    constexpr int OPB = BT * BKB;              // 16 KB per operand and K-tile
    constexpr int KTB = MX ? (FP4 ? 8 : 4) : 4;   // scale bytes per row and K-tile (MX)
    constexpr int SA_OFF = 2 * OPB;            // BSF32: 128 fp32 row scales; MX: [128][KTB] of A
    constexpr int SB_OFF = SA_OFF + (MX ? 128 * KTB : 512);   // BSF32: 2 slots of 256 B; MX: [128][KTB] of B
    constexpr int STAGE = SB_OFF + (MX ? 128 * KTB : 512);
    constexpr int SCD = MX && FP4 ? 2 : 1;     // scale DMAs per wave and K-tile
    constexpr int NDMA = 8 + SCD;              // DMAs per wave and K-tile

    __shared__ __attribute__((aligned(1024))) uint8_t st0[STAGE];
    __shared__ __attribute__((aligned(1024))) uint8_t st1[STAGE];
    __shared__ __attribute__((aligned(1024))) uint8_t st2[STAGES > 2 ? STAGE : 1];
    __shared__ __attribute__((aligned(1024))) uint8_t st3[STAGES > 2 ? STAGE : 1];

    const TileArgs& p = mp.t;
    // ---- tile coordinates: XCD-contiguous remap, then grouped raster ----
    const int T = p.tiles_m * p.tiles_n;
    int bid = blockIdx.x;
    if ((T & 7) == 0) bid = (bid & 7) * (T >> 3) + (bid >> 3);
    const int gfull = p.group_m * p.tiles_n;
    const int gi = bid / gfull;
    const int first_m = gi * p.group_m;
    const int gm = min(p.tiles_m - first_m, p.group_m);
    const int within = bid - gi * gfull;
    const int tm = first_m + within % gm;
    const int tn = within / gm;
    const int tile = tm * p.tiles_n + tn;
    const int sk = blockIdx.y, bz = blockIdx.z;
    const int m0 = tm * BT, n0 = tn * BT;

    const int M = p.m, N = p.n, KB = p.kbytes, LDA = p.lda, LDC = p.ldc;
    const int SFA_SM = p.sfa_sm, SFA_SK = p.sfa_sk, SFB_SN = p.sfb_sn;
    const int NKT = KB / BKB;
    const int kt0 = sk * mp.kt_per_split;
    const int nk = min(NKT, kt0 + mp.kt_per_split) - kt0;    // K-tiles of this slice

    const int tid = threadIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6), L = tid & 63;
    const int wm = w >> 1, wn = w & 1;
    const int q = L >> 4, l16 = L & 15;

    const uint8_t* A = p.a + bz * p.a_batch + (long long)m0 * LDA + (long long)kt0 * BKB;
    const int LDB = p.ldb;
    const uint8_t* B = p.b + bz * p.b_batch +
                       (RAW ? (long long)n0 * LDB + (long long)kt0 * BKB
                            : FRAG ? (long long)(n0 >> 4) * NKT * 2048 + (long long)kt0 * 2048
                                   : (long long)kt0 * N * BKB + (long long)n0 * BKB);
    const long long b_kstep = RAW ? BKB : FRAG ? 2048 : (long long)N * BKB;
    const uint8_t* SFA = p.sfa + (MX ? 1ll : 4ll) * bz * p.sfa_batch;
    const uint8_t* SFB = p.sfb + (MX ? 1ll : 4ll) * bz * p.sfb_batch;

    // ---- DMA offsets: wave w moves 8-row groups 4w .. 4w+3 of A and of B'
    // (lane L: row +L/8, physical chunk L%8 = logical (L%8) ^ (row & 7)),
    // or blocks 2w, 2w+1 of B'' (two 1 KB halves each) ----
    int aoff[4], boff[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int r = (4 * w + u) * 8 + (L >> 3);
        const int c = (L & 7) ^ (r & 7);
        aoff[u] = (min(m0 + r, M - 1) - m0) * LDA + c * 16;
        if constexpr (RAW) {
            boff[u] = (min(n0 + r, N - 1) - n0) * LDB + c * 16;
        } else if constexpr (FRAG) {
            const int blk = 2 * w + (u >> 1);
            const int nb = min((n0 >> 4) + blk, ((N + 15) >> 4) - 1) - (n0 >> 4);
            boff[u] = nb * NKT * 2048 + (u & 1) * 1024 + L * 16;
        } else {
            boff[u] = (min(n0 + r, N - 1) - n0) * BKB + c * 16;
        }
    }
    // scales: BSF32 -- waves 0, 1 move the fp32 row scales of rows [64w,
    // 64w + 64); waves 2, 3 the tile's weight scale (its 128 columns are one
    // scale block).  MX -- waves 0, 1 the K-tile's E8M0 bytes of A rows
    // [64w, 64w + 64), waves 2, 3 those of B rows [64(w-2), +64): KTB bytes
    // per row, one dword per lane (fp4: two DMAs of 32 rows)
    const bool sc_is_a = w < 2;
    const uint8_t* sc_base;
    int sc_voff[SCD], sc_dst[SCD];
    long long sc_kstep;
    if constexpr (MX) {
        const int r64 = 64 * (w & 1);
        sc_base = sc_is_a ? SFA + (long long)m0 * SFA_SM + (long long)kt0 * SFA_SK
                          : SFB + (long long)n0 * SFB_SN + (long long)kt0 * p.sfb_sk;
        sc_kstep = sc_is_a ? SFA_SK : p.sfb_sk;
#pragma unroll
        for (int s2 = 0; s2 < SCD; ++s2) {
            const int row = FP4 ? r64 + 32 * s2 + (L >> 1) : r64 + L;
            const int sm = sc_is_a ? SFA_SM : SFB_SN;
            const int lim = sc_is_a ? M - 1 - m0 : N - 1 - n0;
            sc_voff[s2] = min(row, lim) * sm + (FP4 ? (L & 1) * 4 : 0);
            sc_dst[s2] = (sc_is_a ? SA_OFF : SB_OFF) + (FP4 ? (r64 + 32 * s2) * 8 : r64 * 4);
        }
    } else {
        sc_base = sc_is_a ? SFA + 4ll * m0 * SFA_SM + 4ll * kt0 * SFA_SK
                          : SFB + 4ll * min(n0 >> 7, (N - 1) >> 7) * SFB_SN + 4ll * kt0;
        sc_voff[0] = sc_is_a ? 4 * (min(m0 + 64 * w + L, M - 1) - m0) * SFA_SM : 0;
        sc_kstep = sc_is_a ? 4ll * SFA_SK : 4ll;
        sc_dst[0] = sc_is_a ? SA_OFF + 256 * w : SB_OFF + 256 * (w - 2);
    }

    QG_LDS uint8_t* const pS0 = (QG_LDS uint8_t*)st0;
    QG_LDS uint8_t* const pS1 = (QG_LDS uint8_t*)st1;
    QG_LDS uint8_t* const pS2 = (QG_LDS uint8_t*)st2;
    QG_LDS uint8_t* const pS3 = (QG_LDS uint8_t*)st3;
    auto stage = [&](auto SC) __attribute__((always_inline)) {
        constexpr int S = decltype(SC)::value % STAGES;
        return S == 0 ? pS0 : (S == 1 ? pS1 : (S == 2 ? pS2 : pS3));
    };

    auto rsrc = [&](const uint8_t* base, bool valid) __attribute__((always_inline)) {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base), 0, valid ? 0x7FFFFFFFu : 0u,
                                                 0x00020000);
    };
    struct Src {
        __amdgpu_buffer_rsrc_t a, b, sc;
    };
    auto sources = [&](int kt) __attribute__((always_inline)) {
        const bool v = kt < nk;
        Src s;
        s.a = rsrc(A + (long long)kt * BKB, v);
        s.b = rsrc(B + (long long)kt * b_kstep, v);
        s.sc = rsrc(sc_base + kt * sc_kstep, v);
        return s;
    };
    // DMA d (0 .. NDMA-1) of a K-tile into stage st: 0-3 A, 4-7 B, then scales
    auto dma = [&](QG_LDS uint8_t* st, const Src& s, int d) __attribute__((always_inline)) {
        if (d < 4) dma16_buf(s.a, st + (4 * w + d) * 1024, aoff[d], 0);
        else if (d < 8) {
            if constexpr (NTB) dma16_buf_nt(s.b, st + OPB + (4 * w + d - 4) * 1024, boff[d - 4], 0);
            else dma16_buf(s.b, st + OPB + (4 * w + d - 4) * 1024, boff[d - 4], 0);
        }
        else if (d == 8) dma4_buf(s.sc, st + sc_dst[0], sc_voff[0], 0);
        else dma4_buf(s.sc, st + sc_dst[SCD - 1], sc_voff[SCD - 1], 0);
    };

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    i32x8 af[4], bf[2];
    f32x4 part[2];
    float fs[4];
    // fragment chunks of row l16: fp8 q and q + 4; fp4 2q and 2q + 1 (the
    // two MFMAs of a 256-element K-tile, scale bytes 2q and 2q + 1)
    const int ca = FP4 ? 2 * q : q, cb = FP4 ? 2 * q + 1 : q + 4;
    const int rd8 = l16 * BKB + ((ca ^ (l16 & 7)) << 4);
    const int rd8b = l16 * BKB + ((cb ^ (l16 & 7)) << 4);
    const int rdb0 = FRAG ? L * 16 : rd8, rdb1 = FRAG ? 1024 + L * 16 : rd8b;
    auto frag = [&](const QG_LDS uint8_t* blk, int o0, int o1) __attribute__((always_inline)) -> i32x8 {
        const i32x4 lo = *(const QG_LDS i32x4*)(blk + o0);
        const i32x4 hi = *(const QG_LDS i32x4*)(blk + o1);
        return i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    };
    auto mfma_part = [&](const i32x8& b, const i32x8& a) __attribute__((always_inline)) {
        // zero scale operands select the unscaled fp8 MFMA (a plain product)
        return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(b, a, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0, 0, 0, 0);
    };
    auto rescale = [&](int i, int j, int x) __attribute__((always_inline)) {
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[i][j][e] = __builtin_fmaf(part[x][e], fs[i], acc[i][j][e]);
    };

    // K-tile t (local index) from stage ST; the 9 DMAs of K-tile
    // t + STAGES - 1 go into the stage K-tile t - 1 read (freed by this
    // barrier), one after each of the first 9 MFMAs; the barrier waits for
    // K-tile t's DMAs only (the later K-tiles' 9 (STAGES - 2) stay in flight)
    auto ktile = [&](auto STC, int t) __attribute__((always_inline)) {
        constexpr int ST = decltype(STC)::value;
        QG_LDS uint8_t* cur = stage(mid::I<ST>{});
        QG_LDS uint8_t* nxt = stage(mid::I<ST + STAGES - 1>{});
        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(NDMA * (STAGES - 2)) : "memory");
        __builtin_amdgcn_sched_barrier(0);
        const QG_LDS uint8_t* sA = cur + wm * 64 * BKB;
        const QG_LDS uint8_t* sB = cur + OPB + wn * 64 * BKB;
        bf[0] = frag(sB, rdb0, rdb1);
#pragma unroll
        for (int i = 0; i < 4; ++i) af[i] = frag(sA + 16 * i * BKB, rd8, rd8b);
        if constexpr (MX) {
            // E8M0 bytes of the lane's rows: fp8 byte q, fp4 bytes 2q, 2q + 1
            int sa[4], sb[4];
#pragma unroll
            for (int x = 0; x < 4; ++x) {
                const QG_LDS uint8_t* pa = cur + SA_OFF + (wm * 64 + 16 * x + l16) * KTB;
                const QG_LDS uint8_t* pb = cur + SB_OFF + (wn * 64 + 16 * x + l16) * KTB;
                sa[x] = FP4 ? *(const QG_LDS uint16_t*)(pa + 2 * q) : pa[q];
                sb[x] = FP4 ? *(const QG_LDS uint16_t*)(pb + 2 * q) : pb[q];
            }
            const Src src = sources(t + STAGES - 1);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                const int j = k >> 2, i = k & 3;
                if (i == 0 && j < 3) bf[(j + 1) & 1] = frag(sB + (j + 1) * 16 * BKB, rdb0, rdb1);
                const i32x8& b = bf[j & 1];
                if constexpr (FP4) {
                    const i32x8 b0 = i32x8{b[0], b[1], b[2], b[3], 0, 0, 0, 0};
                    const i32x8 b1 = i32x8{b[4], b[5], b[6], b[7], 0, 0, 0, 0};
                    const i32x8 a0 = i32x8{af[i][0], af[i][1], af[i][2], af[i][3], 0, 0, 0, 0};
                    const i32x8 a1 = i32x8{af[i][4], af[i][5], af[i][6], af[i][7], 0, 0, 0, 0};
                    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(b0, a0, acc[i][j], kFmtFp4, kFmtFp4,
                                                                                 0, sb[j], 0, sa[i]);
                    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(b1, a1, acc[i][j], kFmtFp4, kFmtFp4,
                                                                                 1, sb[j], 1, sa[i]);
                } else {
                    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(b, af[i], acc[i][j], kFmtFp8,
                                                                                 kFmtFp8, 0, sb[j], 0, sa[i]);
                }
                __builtin_amdgcn_sched_barrier(0);
                if (k < NDMA) dma(nxt, src, k);
                __builtin_amdgcn_sched_barrier(0);
            }
        } else {
            const float sb = *(const QG_LDS float*)(cur + SB_OFF);
#pragma unroll
            for (int i = 0; i < 4; ++i)
                fs[i] = *(const QG_LDS float*)(cur + SA_OFF + 4 * (wm * 64 + 16 * i + l16)) * sb;
            const Src src = sources(t + STAGES - 1);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                const int j = k >> 2, i = k & 3;
                if (i == 0 && j < 3) bf[(j + 1) & 1] = frag(sB + (j + 1) * 16 * BKB, rdb0, rdb1);
                part[k & 1] = mfma_part(bf[j & 1], af[i]);
                __builtin_amdgcn_sched_barrier(0);
                if (k > 0) rescale((k - 1) & 3, (k - 1) >> 2, (k - 1) & 1);
                if (k < NDMA) dma(nxt, src, k);
                __builtin_amdgcn_sched_barrier(0);
            }
            rescale(3, 3, 1);
        }
    };

    // ---- prologue: K-tiles 0 .. STAGES - 2 into their stages ----
    mid::static_for<STAGES - 1>([&](auto SC) __attribute__((always_inline)) {
        const Src s0 = sources(decltype(SC)::value);
#pragma unroll
        for (int d = 0; d < NDMA; ++d) dma(stage(SC), s0, d);
    });
    int t = 0;
    for (; t + STAGES <= nk; t += STAGES)
        mid::static_for<STAGES>([&](auto SC) __attribute__((always_inline)) { ktile(SC, t + decltype(SC)::value); });
    mid::static_for<STAGES - 1>([&](auto SC) __attribute__((always_inline)) {
        if (t + decltype(SC)::value < nk) ktile(SC, t + decltype(SC)::value);
    });
    wait_vmcnt<0>();    // the DMAs past the slice still write zeros

    // ---- output: lane holds C[16i + l16][16j + 4q + 0..3] of the wave's block ----
    const int mw = m0 + wm * 64 + l16, nw0 = n0 + wn * 64 + 4 * q;
    const bool vec_ok = p.c_vec >= 4;    // aligned 4-element C stores
    auto store_c = [&](int m, int n, f32x4 v) __attribute__((always_inline)) {
        if (m >= M) return;
        if constexpr (BF16) {
            uint16_t* c = (uint16_t*)p.c + (long long)bz * p.c_batch + (long long)m * LDC + n;
            if (vec_ok && n + 3 < N) {
                *(u32x2*)c = u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
            } else {
                for (int r = 0; r < 4; ++r)
                    if (n + r < N) c[r] = bf16_bits(v[r]);
            }
        } else {
            float* c = (float*)p.c + (long long)bz * p.c_batch + (long long)m * LDC + n;
            if (vec_ok && n + 3 < N) {
                *(f32x4*)c = v;
            } else {
                for (int r = 0; r < 4; ++r)
                    if (n + r < N) c[r] = v[r];
            }
        }
    };
    if (mp.splitk == 1) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) store_c(mw + 16 * i, nw0 + 16 * j, acc[i][j]);
        return;
    }

    // split-K: this slice's partial tile (the kernel boundary orders these
    // stores before splitk_reduce_kernel's loads)
    const long long plane = (long long)M * N;
    const long long split_stride = (long long)gridDim.z * plane;
    float* const slice = mp.ws + sk * split_stride + (long long)bz * plane;
    const bool nvec = (N & 3) == 0;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int m = mw + 16 * i, n = nw0 + 16 * j;
            if (m >= M) continue;
            float* dst = slice + m * N + n;
            if (nvec && n + 3 < N) {
                *(f32x4*)dst = acc[i][j];
            } else {
                for (int r = 0; r < 4; ++r)
                    if (n + r < N) dst[r] = acc[i][j][r];
            }
        }
}

}  // namespace qg
