// Band GEMM for MX decode shapes (M <= 64, row-major B, E8M0 scales) on
// gfx950: a workgroup owns a band of B rows (output columns) and a K slice,
// with that slice of A held in LDS.
//
// The skinny kernel gives each workgroup 16-64 output columns and all of K,
// so every workgroup re-reads all of A (M = 32, K = 16384 fp4: 256 KB per
// workgroup, as much as its B), and reads it in the scaled MFMA's fragment
// order (a wave load touches 16 half lines), which costs a CU about two B
// bytes' worth of line requests per A byte.  Here a workgroup takes
// 8 x 16 x CB columns and at most KTM K-tiles (<= 64 KB of A):
//
//  * A's slice comes into LDS once, in whole lines (8 rows x 128 B per DMA),
//    as [K-tile][row][128 B] with the 16-byte chunks XOR-swizzled by row,
//    shared by the eight waves (one barrier);
//  * wave w owns B rows [n0 + 16 CB w, +16 CB) and streams them through its
//    own LDS ring of D K-tiles (whole-line DMAs, the same swizzle), waiting
//    only for its own DMAs: no barrier in the K loop;
//  * the E8M0 scales of A's rows and of each wave's B rows for the whole
//    slice come once into LDS panels ([row][KTM x KT_SB bytes], 4-byte DMAs:
//    one cache line per row instead of one request per row and K-tile);
//  * MFMA: v_mfma_scale_f32_16x16x128_f8f6f4, MB x CB blocks per K-tile
//    (fp4: two instructions per block, chunks 2q / 2q + 1 with scale bytes
//    2q / 2q + 1 through op_sel; fp8: chunks q / q + 4, scale byte q);
//  * K slices meet in the split-K workspace ([splitk][batch][M][N] fp32,
//    device-coherent stores, one relaxed counter per band); the last slice
//    to arrive sums the slices in slice order with all 512 threads and
//    re-arms the counter (deterministic whichever slice is last).
//
// Register layout (probe.hip): srcA = B fragment, srcB = A fragment; lane
// L = 16q + r holds row r; the accumulator of lane L holds C[m = r][n = 4q ..
// 4q + 3] of a 16 x 16 block.
#pragma once
#include <utility>

#include "tile_args.hpp"

namespace qg {

struct BandArgs {
    TileArgs t;            // operands, shapes, strides (tiles_* / group_m unused)
    float* ws;             // fp32 partials [splitk][batch][M][N] (splitk > 1)
    unsigned* counters;    // [batch][bands] (splitk > 1): epoch-tagged arrival counters
    unsigned epoch;        // this launch's counter epoch (split_arrive)
    int splitk, kt_per_split, bands;
};

constexpr int kBandWaves = 8;
constexpr int kBandLds = 152 * 1024;
// most K-tiles of one slice: the A image stays within 64 KB (16 at most)
__host__ __device__ constexpr int band_kt_max(int mb) { return mb >= 4 ? 8 : 16; }
// fixed LDS: A image + A scale panel + the waves' B scale panels
__host__ __device__ constexpr int band_fixed_lds(int mb, int cb, bool fp4) {
    const int kt = band_kt_max(mb), sp = kt * (fp4 ? 8 : 4);
    return mb * 16 * kt * 128 + mb * 16 * sp + kBandWaves * cb * 16 * sp;
}
// ring depth: K-tiles of B in flight per wave (at most 4)
__host__ __device__ constexpr int band_depth(int mb, int cb, bool fp4) {
    const int d = (kBandLds - band_fixed_lds(mb, cb, fp4)) / (kBandWaves * cb * 2048);
    return d > 4 ? 4 : d;
}
// columns of one band
__host__ __device__ constexpr int band_cols(int cb) { return kBandWaves * 16 * cb; }

namespace band {
template <int N, class F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl<N>(f, std::make_integer_sequence<int, N>{});
}
}  // namespace band

template <int FMT, int MB, int CB, bool BF16>
__global__ __launch_bounds__(kBandWaves * 64, 1) void band_gemm_kernel(const BandArgs ba) {
    constexpr bool FP4 = (FMT == kFmtFp4);
    constexpr int BKB = 128, W = kBandWaves, NT = W * 64;
    constexpr int ROWS = MB * 16, COLS = band_cols(CB);
    constexpr int KTM = band_kt_max(MB);
    constexpr int KT_SB = FP4 ? 8 : 4;       // E8M0 bytes per row and K-tile
    constexpr int SP = KTM * KT_SB;          // scale panel row pitch
    constexpr int DW_ROW = SP / 4;           // dwords per panel row
    constexpr int D = band_depth(MB, CB, FP4);
    static_assert(D >= 2, "at least two ring stages");
    static_assert((ROWS * SP) % 256 == 0 && (CB * 16 * SP) % 256 == 0, "whole 4-byte DMAs per panel");
    constexpr int SLOT = CB * 2048;          // one wave's B bytes per K-tile
    constexpr int STAGE = W * SLOT;
    constexpr int NDMA = CB * 2;             // B DMAs per wave and K-tile

    __shared__ __attribute__((aligned(1024))) uint8_t img[KTM * ROWS * BKB];
    __shared__ __attribute__((aligned(16))) uint8_t sap[ROWS * SP];
    __shared__ __attribute__((aligned(16))) uint8_t sbp[W * CB * 16 * SP];
    __shared__ __attribute__((aligned(1024))) uint8_t ring0[STAGE];
    __shared__ __attribute__((aligned(1024))) uint8_t ring1[STAGE];
    __shared__ __attribute__((aligned(1024))) uint8_t ring2[D > 2 ? STAGE : 16];
    __shared__ __attribute__((aligned(1024))) uint8_t ring3[D > 3 ? STAGE : 16];
    __shared__ int last_flag;
    QG_LDS uint8_t* const limg = (QG_LDS uint8_t*)img;
    QG_LDS uint8_t* const lsa = (QG_LDS uint8_t*)sap;
    QG_LDS uint8_t* const lsb = (QG_LDS uint8_t*)sbp;
    QG_LDS uint8_t* const lr0 = (QG_LDS uint8_t*)ring0;
    QG_LDS uint8_t* const lr1 = (QG_LDS uint8_t*)ring1;
    QG_LDS uint8_t* const lr2 = (QG_LDS uint8_t*)ring2;
    QG_LDS uint8_t* const lr3 = (QG_LDS uint8_t*)ring3;
    auto ring = [&](auto sc) __attribute__((always_inline)) -> QG_LDS uint8_t* {
        constexpr int s = decltype(sc)::value % D;
        if constexpr (s == 0) return lr0;
        else if constexpr (s == 1) return lr1;
        else if constexpr (s == 2) return lr2;
        else return lr3;
    };

    const TileArgs& p = ba.t;
    const int M = p.m, N = p.n, LDA = p.lda, LDB = p.ldb, LDC = p.ldc;
    const int NKT = p.kbytes / BKB;
    const int bnd = blockIdx.x, sk = blockIdx.y, bz = blockIdx.z;
    const int kt0 = sk * ba.kt_per_split;
    const int nk = min(NKT, kt0 + ba.kt_per_split) - kt0;    // 1 .. KTM (host plan)
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), L = tid & 63;
    const int q = L >> 4, l16 = L & 15;
    if (ba.splitk > 1 && tid == 0) split_claim(ba.counters + (long long)bz * ba.bands + bnd, ba.epoch);
    const int n0 = bnd * COLS;
    const int nw = n0 + w * CB * 16;         // the wave's first B row

    const uint8_t* A = p.a + bz * p.a_batch + (long long)kt0 * BKB;
    const uint8_t* B = p.b + bz * p.b_batch + (long long)kt0 * BKB;
    const uint8_t* SFA = p.sfa + bz * p.sfa_batch + (long long)kt0 * KT_SB;
    const uint8_t* SFB = p.sfb + bz * p.sfb_batch + (long long)kt0 * KT_SB;
    auto rsrc = [](const void* base, bool valid) __attribute__((always_inline)) {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, valid ? 0x7FFFFFFF : 0, 0x00020000);
    };

    // ---- prologue: A image, scale panels, then the first D K-tiles of B ----
    {
        // A: DMA d moves rows 8g .. 8g+7 of K-tile t (d = t * ROWS/8 + g);
        // lane L fetches row 8g + L/8, logical chunk (L%8) ^ swz(row)
        const auto rA = rsrc(A, true);
        constexpr int G = ROWS / 8;
        for (int d = w; d < nk * G; d += W) {
            const int t = d / G, g = d - t * G;
            const int r = g * 8 + (L >> 3);
            const int c = (L & 7) ^ swz<FP4>(r & 15);
            dma16_buf(rA, limg + (t * ROWS + g * 8) * BKB, min(r, M - 1) * LDA + c * 16, t * BKB);
        }
        // scale panels: dword x of a panel is row x / DW_ROW, dword x % DW_ROW
        // of the row's slice (past the slice: its last dword, never read)
        const int dw_last = nk * KT_SB / 4 - 1;
        const auto rSA = rsrc(SFA, true);
        for (int d = w; d < ROWS * DW_ROW / 64; d += W) {
            const int x = d * 64 + L, r = x / DW_ROW, dw = min(x % DW_ROW, dw_last);
            dma4_buf(rSA, lsa + d * 256, min(r, M - 1) * p.sfa_sm + dw * 4, 0);
        }
        const auto rSB = rsrc(SFB, true);
#pragma unroll
        for (int d = 0; d < CB * 16 * DW_ROW / 64; ++d) {
            const int x = d * 64 + L, r = x / DW_ROW, dw = min(x % DW_ROW, dw_last);
            dma4_buf(rSB, lsb + w * CB * 16 * SP + d * 256, min(nw + r, N - 1) * p.sfb_sn + dw * 4, 0);
        }
    }
    // B ring: DMA (j, h) moves rows 8h .. 8h+7 of the wave's 16-row block j
    int boff[CB][2];
#pragma unroll
    for (int j = 0; j < CB; ++j)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int R = 8 * h + (L >> 3);
            const int c = (L & 7) ^ swz<FP4>(R);
            boff[j][h] = min(nw + j * 16 + R, N - 1) * LDB + c * 16;
        }
    // B is read once: non-temporal DMAs (one box, graph-replayed from HBM:
    // configs[4] MXFP4 M = 32 17.8 -> 16.5 us, MXFP8 M = 32, N = 7168,
    // K = 8192 17.1 -> 15.9, every band plan measured 4-8% faster)
    auto load_b = [&](auto sc, int t) __attribute__((always_inline)) {
        const auto rB = rsrc(B, t < nk);    // past the slice: zeros, no memory read
        QG_LDS uint8_t* dst = ring(sc) + w * SLOT;
#pragma unroll
        for (int j = 0; j < CB; ++j)
#pragma unroll
            for (int h = 0; h < 2; ++h) dma16_buf_nt(rB, dst + j * 2048 + h * 1024, boff[j][h], t * BKB);
    };
    band::static_for<D>([&](auto sc) __attribute__((always_inline)) { load_b(sc, decltype(sc)::value); });
    // the image and panels landed (this wave's; the barrier: every wave's)
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(D * NDMA) : "memory");

    // ---- K loop ----
    // lane offsets of the LDS reads pass through an empty asm: written as
    // plain lane-id expressions, some let the compiler lose track of which
    // LDS array a read hits, and it then waits for every DMA in flight
    const int c0 = FP4 ? 2 * q : q, c1 = FP4 ? 2 * q + 1 : q + 4;
    int frag0 = l16 * BKB + ((c0 ^ swz<FP4>(l16)) << 4);
    int frag1 = l16 * BKB + ((c1 ^ swz<FP4>(l16)) << 4);
    int sc_off = l16 * SP + (FP4 ? 2 * q : q);     // + (block * 16) * SP + t * KT_SB
    asm("" : "+v"(frag0), "+v"(frag1), "+v"(sc_off));
    auto rd8 = [&](const QG_LDS uint8_t* blk) __attribute__((always_inline)) -> i32x8 {
        const i32x4 lo = *(const QG_LDS i32x4*)(blk + frag0);
        const i32x4 hi = *(const QG_LDS i32x4*)(blk + frag1);
        return i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    };
    f32x4 acc[MB][CB];
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < CB; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    const QG_LDS uint8_t* const sbw = lsb + w * CB * 16 * SP;

    auto step = [&](auto sc, int t) __attribute__((always_inline)) {
        // K-tile t's B landed: the later D - 1 stages may stay in flight
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"((D - 1) * NDMA) : "memory");
        __builtin_amdgcn_sched_barrier(0);
        const QG_LDS uint8_t* rb = ring(sc) + w * SLOT;
        i32x8 af[MB], bf[CB];
        int sa[MB], sb[CB];
#pragma unroll
        for (int j = 0; j < CB; ++j) {
            bf[j] = rd8(rb + j * 2048);
            const QG_LDS uint8_t* ps = sbw + j * 16 * SP + t * KT_SB + sc_off;
            sb[j] = FP4 ? *(const QG_LDS uint16_t*)ps : *ps;
        }
#pragma unroll
        for (int i = 0; i < MB; ++i) {
            af[i] = rd8(limg + (t * ROWS + i * 16) * BKB);
            const QG_LDS uint8_t* ps = lsa + i * 16 * SP + t * KT_SB + sc_off;
            sa[i] = FP4 ? *(const QG_LDS uint16_t*)ps : *ps;
        }
#pragma unroll
        for (int j = 0; j < CB; ++j)
#pragma unroll
            for (int i = 0; i < MB; ++i) {
                if constexpr (FP4) {
                    const i32x8 b0 = i32x8{bf[j][0], bf[j][1], bf[j][2], bf[j][3], 0, 0, 0, 0};
                    const i32x8 b1 = i32x8{bf[j][4], bf[j][5], bf[j][6], bf[j][7], 0, 0, 0, 0};
                    const i32x8 a0 = i32x8{af[i][0], af[i][1], af[i][2], af[i][3], 0, 0, 0, 0};
                    const i32x8 a1 = i32x8{af[i][4], af[i][5], af[i][6], af[i][7], 0, 0, 0, 0};
                    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(b0, a0, acc[i][j], kFmtFp4,
                                                                                 kFmtFp4, 0, sb[j], 0, sa[i]);
                    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(b1, a1, acc[i][j], kFmtFp4,
                                                                                 kFmtFp4, 1, sb[j], 1, sa[i]);
                } else {
                    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bf[j], af[i], acc[i][j], kFmtFp8,
                                                                                 kFmtFp8, 0, sb[j], 0, sa[i]);
                }
            }
        // the stage's reads are done (the MFMAs consumed them): refill it
        // with K-tile t + D
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        load_b(sc, t + D);
        __builtin_amdgcn_sched_barrier(0);
    };
    int t = 0;
    for (; t + D <= nk; t += D)
        band::static_for<D>([&](auto sc) __attribute__((always_inline)) { step(sc, t + decltype(sc)::value); });
    band::static_for<D - 1>([&](auto sc) __attribute__((always_inline)) {
        if (t + decltype(sc)::value < nk) step(sc, t + decltype(sc)::value);
    });
    wait_vmcnt<0>();    // ring stages past the slice still receive zeros

    // ---- output: lane holds C[16i + l16][nw + 16j + 4q + 0..3] ----
    auto store4 = [&](int m, int n, f32x4 v) __attribute__((always_inline)) {
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
    if (ba.splitk == 1) {
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
            for (int j = 0; j < CB; ++j) store4(16 * i + l16, nw + 16 * j + 4 * q, acc[i][j]);
        return;
    }

    // split-K: this slice's partial, device-coherent; then the band's counter
    const long long plane = (long long)M * N;
    const int batch = gridDim.z;
    const long long split_stride = (long long)batch * plane;
    const bool vec = (N & 3) == 0;
    {
        const auto part = partial_rsrc(ba.ws + ((long long)sk * batch + bz) * plane);
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
            for (int j = 0; j < CB; ++j) {
                const int m = 16 * i + l16, n = nw + 16 * j + 4 * q;
                if (m >= M) continue;
                if (vec && n + 3 < N) {
                    store_partial4(part, m * N + n, acc[i][j]);
                } else {
                    for (int r = 0; r < 4; ++r)
                        if (n + r < N) store_partial1(part, m * N + n + r, acc[i][j][r]);
                }
            }
    }
    wait_vmcnt<0>();
    __syncthreads();
    unsigned* ctr = ba.counters + (long long)bz * ba.bands + bnd;
    if (tid == 0)
        last_flag = split_arrive(ctr, ba.epoch, ba.splitk);
    __syncthreads();
    if (!last_flag) return;
    // the band's ROWS x COLS outputs, 4 per thread and element: E elements
    // per thread, every slice's loads of a group of SG slices in flight
    // before the adds, slices summed in order 0 .. splitk - 1
    constexpr int E = (ROWS * COLS / 4 + NT - 1) / NT;
    constexpr int SG = 32 / E > 8 ? 8 : (32 / E < 1 ? 1 : 32 / E);
    const float* ws0 = ba.ws + (long long)bz * plane;
    f32x4 v[E];
    int mm[E], nn[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const int x = (tid + e * NT) * 4;
        mm[e] = x < ROWS * COLS ? x / COLS : M;      // M: no output
        nn[e] = n0 + x % COLS;
        v[e] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    if (vec) {
        for (int s0 = 0; s0 < ba.splitk; s0 += SG) {
            f32x4 u[SG][E];
#pragma unroll
            for (int s = 0; s < SG; ++s)
#pragma unroll
                for (int e = 0; e < E; ++e)
                    if (s0 + s < ba.splitk && mm[e] < M && nn[e] < N)
                        u[s][e] = load_partial4(partial_rsrc(ws0 + (s0 + s) * split_stride), mm[e] * N + nn[e]);
#pragma unroll
            for (int s = 0; s < SG; ++s)
#pragma unroll
                for (int e = 0; e < E; ++e)
                    if (s0 + s < ba.splitk && mm[e] < M && nn[e] < N) v[e] += u[s][e];
        }
    } else {
#pragma unroll
        for (int e = 0; e < E; ++e) {
            if (mm[e] >= M) continue;
            for (int s = 0; s < ba.splitk; ++s) {
                const auto src = partial_rsrc(ws0 + s * split_stride);
                for (int r = 0; r < 4; ++r)
                    if (nn[e] + r < N) v[e][r] += load_partial1(src, mm[e] * N + nn[e] + r);
            }
        }
    }
#pragma unroll
    for (int e = 0; e < E; ++e)
        if (nn[e] < N) store4(mm[e], nn[e], v[e]);
    if (tid == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace qg
