// Decode GEMM (M <= 64) for gfx950: B streamed once from HBM, A shared.
//
// A decode GEMM is HBM-bound on B; A is M x K, small, and needed by every
// workgroup.  The layout of this kernel follows from two MI355X facts
// (measured with streaming microbenchmarks): one CU streams only ~50 GB/s, and
// that rate is a rate of cache-line requests, so a load in the scaled MFMA's
// fragment order (lane 16q + r = row r, 16 rows x 32 B per instruction)
// moves half the bytes of a whole-line load (8 rows x 128 B).  Loading A in
// fragment order per wave made A cost more line requests than B.  Here:
//
//  * a workgroup of NW waves owns all ROWS = MB*16 rows and NW*16 columns;
//    wave w owns columns [16w, 16w + 16) of the tile and every K-tile of the
//    workgroup's K slice, so no cross-wave reduction is needed;
//  * per 128-byte K-tile, A (ROWS rows) and each wave's 16 B rows move
//    global -> LDS by DMA in whole lines (A is shared by the NW waves: each
//    wave moves an equal share of it), 16-byte chunks XOR-swizzled per row so
//    the fragment reads are conflict free;
//  * a ring of D K-tile stages (one LDS object per stage, so the compiler's
//    wait tracking stays per stage) keeps D-1 K-tiles of DMAs in flight; one
//    barrier per K-tile: every wave waits for its own DMAs of K-tile k, the
//    barrier makes the other waves' rows of A visible and frees the stage of
//    K-tile k-1, into which the DMAs of K-tile k+D-1 go;
//  * MX scale bytes go straight into registers with the same look-ahead;
//    fp32 row scales by one DMA per K-tile into the stage (one cache-line
//    request per row; per-wave register loads made one per row and wave);
//  * K is split over workgroups when the N tiles alone leave CUs idle; the
//    last workgroup of a tile sums the fp32 partial slices in slice order
//    (deterministic), one launch.
//
// Register layout of the scaled MFMA 16x16x128 (probe.hip): operand lane
// L = 16q + r holds row r, fp8 16-byte chunks q and q+4, fp4 chunks 2q and
// 2q+1 (second instruction, op_sel 1); srcA = B, srcB = A; accumulator of
// lane L holds C[m = r][n = 4q .. 4q+3].
#pragma once
#include "skinny_gemm.hpp"

namespace qg {

struct DecodeArgs {
    TileArgs t;           // operands, shapes, strides (tiles_* / group_m unused)
    float* ws;            // fp32 partials [splitk][batch][M][N] (splitk > 1)
    unsigned* counters;   // [batch][n_tiles]: epoch-tagged arrival counters
    unsigned epoch;       // this launch's counter epoch (split_arrive)
    int splitk, kt_per_split, n_tiles;
};

// LDS bytes of one K-tile stage and the ring depth for MB row blocks, NW
// waves; fp32 block scales add a 256-byte row-scale slot per wave
__host__ __device__ constexpr int decode_stage_bytes(int mb, int nw, bool lds_sa) {
    return (mb + nw) * 2048 + (lds_sa ? 256 * nw : 0);
}
__host__ __device__ constexpr int decode_depth(int mb, int nw, bool lds_sa) {
    const int d = 150 * 1024 / decode_stage_bytes(mb, nw, lds_sa);
    return d > 8 ? 8 : d;
}

template <int FMT, ScaleKind SK, BLay BL, int MB, int NW, bool BF16>
__global__ __launch_bounds__(NW * 64) void decode_gemm_kernel(const DecodeArgs dp) {
    constexpr int BKB = 128;
    static_assert(MB == 1 || MB == 2 || MB == 4, "16, 32 or 64 rows");
    static_assert(NW == 4 || NW == 8, "4 or 8 waves");
    static_assert(SK == ScaleKind::MX || SK == ScaleKind::BSF32, "E8M0 or fp32 block scales");
    static_assert(BL == BLay::RAW || BL == BLay::KPANEL, "row-major or K-panel B");
    constexpr bool FP4 = (FMT == kFmtFp4);
    constexpr bool MX = (SK == ScaleKind::MX);
    // fp32 row scales of a K-tile go into the stage by one DMA (wave 0; the
    // other waves' no-op DMAs land in their own slots): one cache-line
    // request per row, instead of one per row and wave from register loads
    constexpr bool LDS_SA = !MX;
    constexpr int D = decode_depth(MB, NW, LDS_SA);
    static_assert(D >= 3, "ring depth");
    constexpr int ROWS = MB * 16, COLS = NW * 16, NT = NW * 64;
    constexpr int STAGE = decode_stage_bytes(MB, NW, LDS_SA);
    constexpr int SA_OFF = (MB + NW) * 2048;
    constexpr int A_BYTES = MB * 2048;               // A rows of one K-tile
    constexpr int A_SHARE = A_BYTES / NW;            // bytes of A each wave moves
    constexpr int A_DMAS = A_SHARE >= 1024 ? A_SHARE / 1024 : A_SHARE / 256;   // x4 or x1 DMAs
    constexpr bool A_X4 = A_SHARE >= 1024;
    constexpr int P = A_DMAS + 2 + (MX ? MB : 1) + 1;   // vector-memory instructions per wave and K-tile

    __shared__ __attribute__((aligned(16))) uint8_t ring0[STAGE];
    __shared__ __attribute__((aligned(16))) uint8_t ring1[STAGE];
    __shared__ __attribute__((aligned(16))) uint8_t ring2[STAGE];
    __shared__ __attribute__((aligned(16))) uint8_t ring3[D > 3 ? STAGE : 16];
    __shared__ __attribute__((aligned(16))) uint8_t ring4[D > 4 ? STAGE : 16];
    __shared__ __attribute__((aligned(16))) uint8_t ring5[D > 5 ? STAGE : 16];
    __shared__ __attribute__((aligned(16))) uint8_t ring6[D > 6 ? STAGE : 16];
    __shared__ __attribute__((aligned(16))) uint8_t ring7[D > 7 ? STAGE : 16];
    __shared__ int last_flag;
    QG_LDS uint8_t* const lr0 = (QG_LDS uint8_t*)ring0;
    QG_LDS uint8_t* const lr1 = (QG_LDS uint8_t*)ring1;
    QG_LDS uint8_t* const lr2 = (QG_LDS uint8_t*)ring2;
    QG_LDS uint8_t* const lr3 = (QG_LDS uint8_t*)ring3;
    QG_LDS uint8_t* const lr4 = (QG_LDS uint8_t*)ring4;
    QG_LDS uint8_t* const lr5 = (QG_LDS uint8_t*)ring5;
    QG_LDS uint8_t* const lr6 = (QG_LDS uint8_t*)ring6;
    QG_LDS uint8_t* const lr7 = (QG_LDS uint8_t*)ring7;
    auto ring = [&](auto dc) __attribute__((always_inline)) -> QG_LDS uint8_t* {
        constexpr int d = decltype(dc)::value % D;
        if constexpr (d == 0) return lr0;
        else if constexpr (d == 1) return lr1;
        else if constexpr (d == 2) return lr2;
        else if constexpr (d == 3) return lr3;
        else if constexpr (d == 4) return lr4;
        else if constexpr (d == 5) return lr5;
        else if constexpr (d == 6) return lr6;
        else return lr7;
    };

    const TileArgs& p = dp.t;
    const int M = p.m, N = p.n, KB = p.kbytes, LDA = p.lda, LDB = p.ldb, LDC = p.ldc;
    const int SFA_SM = p.sfa_sm, SFA_SK = p.sfa_sk, SFB_SN = p.sfb_sn;
    const int nk = KB / BKB;
    const int nt = blockIdx.x, sk = blockIdx.y, bz = blockIdx.z;
    const int n0 = nt * COLS;
    const int kt_begin = sk * dp.kt_per_split;
    const int nkt = min(nk, kt_begin + dp.kt_per_split) - kt_begin;

    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), L = tid & 63;
    const int q = L >> 4, l16 = L & 15;
    if (dp.splitk > 1 && tid == 0) split_claim(dp.counters + (long long)bz * dp.n_tiles + nt, dp.epoch);
    const int nw0 = n0 + 16 * w;                     // the wave's first column

    const uint8_t* A = p.a + bz * p.a_batch;
    const uint8_t* B = p.b + bz * p.b_batch;
    const uint8_t* SFA = p.sfa + bz * p.sfa_batch * (MX ? 1 : 4);
    const uint8_t* SFB = p.sfb + bz * p.sfb_batch * (MX ? 1 : 4);

    // ---- loop-invariant per-lane byte offsets (operands below 2^31 bytes) ----
    // A share of wave w: x4 DMAs cover 8 rows each (lane: row L/8, physical
    // chunk L%8); x1 DMAs cover 2 rows (lane: row L/32, physical chunk
    // (L%32)/4, word L%4).  Physical chunk pc of row R holds logical chunk
    // pc ^ swz(R).
    int a_dma_off[A_DMAS], a_dma_lds[A_DMAS];
#pragma unroll
    for (int u = 0; u < A_DMAS; ++u) {
        const int first = w * A_SHARE + u * (A_X4 ? 1024 : 256);     // LDS byte of the DMA
        const int R = first / BKB + (A_X4 ? (L >> 3) : (L >> 5));
        const int pc = A_X4 ? (L & 7) : ((L & 31) >> 2);
        const int lc = pc ^ swz<FP4>(R);
        const int m = min(R, M - 1);
        a_dma_off[u] = m * LDA + lc * 16 + (A_X4 ? 0 : (L & 3) * 4);
        a_dma_lds[u] = first;
    }
    // B rows of the wave: DMA h moves rows 8h .. 8h+7 of the wave's 16
    int b_off[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int R = 8 * h + (L >> 3);
        const int n = min(nw0 + R, N - 1);
        const int lc = (L & 7) ^ swz<FP4>(R);
        b_off[h] = (BL == BLay::RAW ? n * LDB : n * BKB) + lc * 16;
    }
    const int b_kstep = (BL == BLay::KPANEL) ? N * BKB : BKB;
    // scales: MX bytes of the lane's group(s); BSF32 fp32 words
    int sa_voff[MB];
#pragma unroll
    for (int i = 0; i < MB; ++i) {
        const int m = min(i * 16 + l16, M - 1);
        sa_voff[i] = MX ? m * SFA_SM + (FP4 ? 2 * q : q) : m * SFA_SM * 4;
    }
    const int nb = min(nw0 + l16, N - 1);
    const int sb_voff = MX ? nb * SFB_SN + (FP4 ? 2 * q : q) : ((min(nw0, N - 1) >> 7) * SFB_SN) * 4;
    const int sa_kstep = MX ? (FP4 ? 8 : 4) : SFA_SK * 4;
    const int sa_dma_voff = min(L, M - 1) * SFA_SM * 4;      // fp32: lane L moves row L's scale
    const int sb_kstep = MX ? (FP4 ? 8 : 4) : 4;
    // fragment reads inside a 16-row block: row l16, chunks c0 / c1
    const int c0 = FP4 ? 2 * q : q, c1 = FP4 ? 2 * q + 1 : q + 4;
    const int frag0 = l16 * BKB + ((c0 ^ swz<FP4>(l16)) * 16);
    const int frag1 = l16 * BKB + ((c1 ^ swz<FP4>(l16)) * 16);

    auto rsrc = [](const void* base, bool valid) __attribute__((always_inline)) {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, valid ? 0x7FFFFFFF : 0, 0x00020000);
    };
    struct Scales {
        int sa[MB];
        int sb;
        float fa[MB];
        float fb;
    };
    // all vector-memory instructions of K-tile kt (P per wave), into stage dc
    auto issue = [&](auto dc, Scales& sc, int kt, bool valid) __attribute__((always_inline)) {
        QG_LDS uint8_t* st = ring(dc);
        const auto rA = rsrc(A, valid), rB = rsrc(B, valid);
#pragma unroll
        for (int u = 0; u < A_DMAS; ++u) {
            if constexpr (A_X4) dma16_buf(rA, st + a_dma_lds[u], a_dma_off[u], kt * BKB);
            else dma4_buf(rA, st + a_dma_lds[u], a_dma_off[u], kt * BKB);
        }
#pragma unroll
        // (nontemporal: M <= 64 is one M tile, each B byte is read once)
        for (int h = 0; h < 2; ++h) dma16_buf_nt(rB, st + A_BYTES + w * 2048 + h * 1024, b_off[h], kt * b_kstep);
        const auto rSA = rsrc(SFA, valid), rSB = rsrc(SFB, valid);
        if constexpr (MX) {
#pragma unroll
            for (int i = 0; i < MB; ++i) {
                if constexpr (FP4) sc.sa[i] = __builtin_amdgcn_raw_buffer_load_b16(rSA, sa_voff[i], kt * sa_kstep, 0);
                else sc.sa[i] = __builtin_amdgcn_raw_buffer_load_b8(rSA, sa_voff[i], kt * sa_kstep, 0);
            }
            if constexpr (FP4) sc.sb = __builtin_amdgcn_raw_buffer_load_b16(rSB, sb_voff, kt * sb_kstep, 0);
            else sc.sb = __builtin_amdgcn_raw_buffer_load_b8(rSB, sb_voff, kt * sb_kstep, 0);
        } else {
            dma4_buf(rsrc(SFA, valid && w == 0), st + SA_OFF + w * 256, sa_dma_voff, kt * sa_kstep);
            sc.fb = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rSB, sb_voff, kt * sb_kstep, 0));
        }
    };

    f32x4 acc[MB];
#pragma unroll
    for (int i = 0; i < MB; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int unit = p.unit_scale;
    auto cat8 = [](i32x4 lo, i32x4 hi) __attribute__((always_inline)) {
        return i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    };
    auto compute = [&](auto dc, const Scales& sc) __attribute__((always_inline)) {
        const QG_LDS uint8_t* st = ring(dc);
        const QG_LDS uint8_t* bsrc = st + A_BYTES + w * 2048;
        const i32x8 bf = cat8(*(const QG_LDS i32x4*)(bsrc + frag0), *(const QG_LDS i32x4*)(bsrc + frag1));
#pragma unroll
        for (int i = 0; i < MB; ++i) {
            const QG_LDS uint8_t* asrc = st + i * 2048;
            const i32x8 af = cat8(*(const QG_LDS i32x4*)(asrc + frag0), *(const QG_LDS i32x4*)(asrc + frag1));
            if constexpr (FP4) {
                const i32x8 b0 = i32x8{bf[0], bf[1], bf[2], bf[3], 0, 0, 0, 0};
                const i32x8 b1 = i32x8{bf[4], bf[5], bf[6], bf[7], 0, 0, 0, 0};
                const i32x8 a0 = i32x8{af[0], af[1], af[2], af[3], 0, 0, 0, 0};
                const i32x8 a1 = i32x8{af[4], af[5], af[6], af[7], 0, 0, 0, 0};
                acc[i] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(b0, a0, acc[i], kFmtFp4, kFmtFp4, 0, sc.sb, 0,
                                                                          sc.sa[i]);
                acc[i] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(b1, a1, acc[i], kFmtFp4, kFmtFp4, 1, sc.sb, 1,
                                                                          sc.sa[i]);
            } else if constexpr (MX) {
                acc[i] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bf, af, acc[i], kFmtFp8, kFmtFp8, 0, sc.sb, 0,
                                                                          sc.sa[i]);
            } else {
                const f32x4 part = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                    bf, af, f32x4{0.f, 0.f, 0.f, 0.f}, kFmtFp8, kFmtFp8, 0, unit, 0, unit);
                const float s = *(const QG_LDS float*)(st + SA_OFF + 4 * (i * 16 + l16)) * sc.fb;
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[i][r] = __builtin_fmaf(part[r], s, acc[i][r]);
            }
        }
    };

    // ---- K loop over the slice: stage of local K-tile k is k % D ----
    Scales sc[D];
    static_for<D - 1>([&](auto dc) {
        constexpr int d = decltype(dc)::value;
        issue(dc, sc[d], kt_begin + d, d < nkt);
    });
    // one K-tile: own loads of k landed (the D-2 later K-tiles may still be in
    // flight), LDS reads of k-1 done, barrier; then K-tile k + D - 1 into
    // the stage of k - 1, and the MFMAs of k
    auto step = [&](auto dc, int k) __attribute__((always_inline)) {
        constexpr int d = decltype(dc)::value;
        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(P * (D - 2)) : "memory");
        issue(std::integral_constant<int, (d + D - 1) % D>{}, sc[(d + D - 1) % D], kt_begin + k + D - 1,
              k + D - 1 < nkt);
        compute(dc, sc[d]);
    };
    int k = 0;
    for (; k + D <= nkt; k += D) {
        static_for<D>([&](auto dc) { step(dc, k + decltype(dc)::value); });
    }
    static_for<D>([&](auto dc) {
        if (k + decltype(dc)::value < nkt) step(dc, k + decltype(dc)::value);
    });
    wait_vmcnt<0>();    // stages past the slice still receive zeros

    // ---- output ----
    const int n = nw0 + 4 * q;
    auto store4 = [&](int m, f32x4 v) __attribute__((always_inline)) {
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
    if (dp.splitk == 1) {
#pragma unroll
        for (int i = 0; i < MB; ++i) store4(i * 16 + l16, acc[i]);
        return;
    }

    // split-K: store this slice's partial tile; the last workgroup of the
    // tile sums all slices in slice order.  Publication: device-coherent
    // partial stores, completed before a barrier, then one relaxed counter
    // atomic per workgroup (see store_partial4 in common.hpp).
    const long long plane = (long long)M * N;
    const int batch = gridDim.z;
    const long long split_stride = (long long)batch * plane;
    const auto part = partial_rsrc(dp.ws + ((long long)sk * batch + bz) * plane);
    const bool vec_ok = (N & 3) == 0;
#pragma unroll
    for (int i = 0; i < MB; ++i) {
        const int m = i * 16 + l16;
        if (m >= M) continue;
        const int e = m * N + n;
        if (n + 3 < N && vec_ok) {
            store_partial4(part, e, acc[i]);
        } else {
            for (int r = 0; r < 4; ++r)
                if (n + r < N) store_partial1(part, e + r, acc[i][r]);
        }
    }
    wait_vmcnt<0>();
    __syncthreads();
    unsigned* ctr = dp.counters + (long long)bz * dp.n_tiles + nt;
    if (tid == 0)
        last_flag = split_arrive(ctr, dp.epoch, dp.splitk);
    __syncthreads();
    if (!last_flag) return;
    const float* ws0 = dp.ws + (long long)bz * plane;
    // MB passes of 4 columns per thread; with whole-vector rows every pass's
    // loads of a group of SG slices are in flight together (one round trip
    // per group, not one per pass), the slices summed in order 0 .. splitk - 1
    static_assert(ROWS * COLS == MB * NT * 4, "reduction passes");
    constexpr int SG = 16 / MB < 8 ? 16 / MB : 8;
    int rm[MB], rn[MB];
    f32x4 v[MB];
#pragma unroll
    for (int it = 0; it < MB; ++it) {
        const int x = tid * 4 + it * NT * 4;
        rm[it] = x / COLS;
        rn[it] = n0 + x % COLS;
        v[it] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    if (vec_ok) {
        // N % 4 == 0: a thread's 4 columns are all in or all out
        for (int s0 = 0; s0 < dp.splitk; s0 += SG) {
            f32x4 u[SG][MB];
#pragma unroll
            for (int t = 0; t < SG; ++t)
#pragma unroll
                for (int it = 0; it < MB; ++it)
                    if (s0 + t < dp.splitk && rm[it] < M && rn[it] < N)
                        u[t][it] = load_partial4(partial_rsrc(ws0 + (s0 + t) * split_stride), rm[it] * N + rn[it]);
#pragma unroll
            for (int t = 0; t < SG; ++t)
#pragma unroll
                for (int it = 0; it < MB; ++it)
                    if (s0 + t < dp.splitk && rm[it] < M && rn[it] < N) v[it] += u[t][it];
        }
    } else {
#pragma unroll
        for (int it = 0; it < MB; ++it) {
            if (rm[it] >= M) continue;
            for (int s0 = 0; s0 < dp.splitk; ++s0) {
                const auto src = partial_rsrc(ws0 + s0 * split_stride);
                for (int r = 0; r < 4; ++r)
                    if (rn[it] + r < N) v[it][r] += load_partial1(src, rm[it] * N + rn[it] + r);
            }
        }
    }
#pragma unroll
    for (int it = 0; it < MB; ++it) {
        const int m = rm[it], nn = rn[it];
        if (m >= M) continue;
        // the thread's 4 columns start at nn
        if constexpr (BF16) {
            uint16_t* c = (uint16_t*)p.c + bz * p.c_batch + (long long)m * LDC + nn;
            if (nn + 3 < N && p.c_vec >= 4) {
                *(u32x2*)c = u32x2{pack_bf16x2(v[it][0], v[it][1]), pack_bf16x2(v[it][2], v[it][3])};
            } else {
                for (int r = 0; r < 4; ++r)
                    if (nn + r < N) c[r] = bf16_bits(v[it][r]);
            }
        } else {
            float* c = (float*)p.c + bz * p.c_batch + (long long)m * LDC + nn;
            if (nn + 3 < N && p.c_vec >= 4) {
                *(f32x4*)c = v[it];
            } else {
                for (int r = 0; r < 4; ++r)
                    if (nn + r < N) c[r] = v[it][r];
            }
        }
    }
    if (tid == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace qg
