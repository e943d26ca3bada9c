// Skinny-M / split-K GEMM for gfx950 (decode shapes and the LDS-bypass path).
//
// Decode GEMMs stream B once and are HBM-bound.  On MI355X one CU sustains
// only ~45-55 GB/s of streaming reads (8 waves, >= 64 KB in flight), so
// reaching HBM bandwidth needs work on every one of the 256 CUs: the host
// picks the N-tile width (16, 32 or 64 columns: NB blocks of 16) so that the
// grid has about one workgroup per CU, and splits K across workgroups only
// when even 16-column tiles leave CUs idle.
//
// A workgroup (8 wave64) owns NB*16 output columns, MB*16 rows and a slice
// of the K-tiles (128 bytes of K each).  B is streamed straight from global
// memory into MFMA fragments, and A fragments come from global memory too
// (the small A operand is L2-resident).  Wave w takes K-tiles w, w+8, ... of
// the slice; loads run D K-tiles ahead of the MFMAs in a register ring.
// The eight waves' partial sums meet in LDS and are added in a fixed order
// (the result does not depend on timing).  With split-K > 1 each workgroup
// stores its fp32 partial tile into the caller's workspace and the last
// workgroup of a tile (atomic counter) sums the partials in slice order,
// rounds and re-arms the counter, all in the same launch.
//
// Register layout of the scaled MFMA (pinned by the layout probes): see
// tile_gemm.hpp.  srcA = B fragment, srcB = A fragment; the accumulator of
// lane L = 16q + r holds C[m = r][n = 4q .. 4q+3] of a 16 x 16 block.
//
// B layouts: RAW [N][Kbytes]; KPANEL [K/128][N][128]; W16 shuffle_weight(16,16);
// FRAG (this library's B'' for the LDS-bypass entry): for every 16-row block
// nb and K-tile kt, 2048 contiguous bytes [nb][kt][h][lane][16] where lane L
// = 16q + r holds row 16nb + r and h selects the lane's first or second
// 16-byte operand chunk, so each fragment load is one coalesced 1 KB read.
#pragma once
#include "tile_gemm.hpp"

namespace qg {

constexpr BLay kBFrag = static_cast<BLay>(3);
constexpr int kSkinnyWaves = 8;

struct SkinnyArgs {
    TileArgs t;              // operands, shapes, strides (tiles_* / group_m unused)
    float* ws;               // fp32 partials [splitk][batch][M][N] (splitk > 1)
    unsigned* counters;      // [batch][m_tiles][n_tiles], zero between launches
    int splitk, kt_per_split, n_tiles, m_tiles;
};

// blockIdx.x -> (n-tile, m-tile): the m-tiles that share one B slice get
// workgroup ids 8 apart, i.e. the same XCD (ids are dealt round-robin over
// the 8 XCDs), so the second read of the slice hits that XCD's L2.
// Grid x = ceil(n_tiles / 8) * 8 * m_tiles; ids past n_tiles exit at once.
__host__ __device__ inline int skinny_grid_x(int n_tiles, int m_tiles) { return (n_tiles + 7) / 8 * 8 * m_tiles; }

// K-tiles in flight per wave: the register ring holds D stages of
// 8*(MB+NB) operand dwords (+ scales) next to 4*MB*NB accumulators, within
// the 256 VGPRs a wave gets at two waves per SIMD.
__host__ __device__ constexpr int skinny_depth(int mb, int nb) {
    const int d = (200 - 4 * mb * nb) / (8 * (mb + nb) + 4);
    return d > 8 ? 8 : (d < 2 ? 2 : d);
}

template <int FMT, ScaleKind SK, BLay BL, int MB, int NB, bool BF16>
__global__ __launch_bounds__(kSkinnyWaves * 64) void skinny_gemm_kernel(const SkinnyArgs sp) {
    constexpr int BKB = 128, W = kSkinnyWaves;
    static_assert(MB == 1 || MB == 2 || MB == 4, "16, 32 or 64 rows per M-tile");
    static_assert(NB == 1 || NB == 2 || NB == 4, "16, 32 or 64 columns per N-tile");
    static_assert(SK == ScaleKind::MX || SK == ScaleKind::BSF32, "E8M0 or fp32 block scales");
    constexpr bool FP4 = (FMT == kFmtFp4);
    constexpr bool MX = (SK == ScaleKind::MX);
    constexpr bool VALU_SCALE = (SK == ScaleKind::BSF32);
    constexpr int D = skinny_depth(MB, NB);
    constexpr int ROWS = MB * 16, COLS = NB * 16;
    constexpr int RP = COLS + 4;           // LDS row pitch in floats (breaks the bank period)
    constexpr int REGION = ROWS * RP;
    constexpr int NT = W * 64;
    __shared__ __attribute__((aligned(16))) float red[4 * REGION];
    __shared__ int last_flag;

    const TileArgs& p = sp.t;
    const int M = p.m, N = p.n, KB = p.kbytes, LDA = p.lda, LDB = p.ldb, LDC = p.ldc;
    const int SFA_SM = p.sfa_sm, SFA_SK = p.sfa_sk, SFB_SN = p.sfb_sn;
    const int nk = KB / BKB;
    const int slot = blockIdx.x >> 3;
    const int mt = slot % sp.m_tiles;
    const int nt = (slot / sp.m_tiles) * 8 + (blockIdx.x & 7);
    if (nt >= sp.n_tiles) return;
    const int sk = blockIdx.y, bz = blockIdx.z;
    const int n0 = nt * COLS, m0 = mt * ROWS;
    const int kt_begin = sk * sp.kt_per_split;
    const int kt_end = min(nk, kt_begin + sp.kt_per_split);

    // the wave index is uniform: keep it (and every K-tile index) in SGPRs
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), L = tid & 63;
    const int q = L >> 4, l16 = L & 15;

    const uint8_t* A = p.a + bz * p.a_batch;
    const uint8_t* B = p.b + bz * p.b_batch;
    const uint8_t* SFA = p.sfa + bz * p.sfa_batch * (VALU_SCALE ? 4 : 1);
    const uint8_t* SFB = p.sfb + bz * p.sfb_batch * (VALU_SCALE ? 4 : 1);

    // ---- per-lane sources (32-bit offsets: the host bounds every operand below 2^31 bytes) ----
    const int c0 = FP4 ? 2 * q : q;            // first 16-byte chunk of the lane
    const int c1 = FP4 ? 2 * q + 1 : q + 4;    // second chunk
    int arow[MB], sa_base[MB];
#pragma unroll
    for (int i = 0; i < MB; ++i) {
        const int m = min(m0 + i * 16 + l16, M - 1);
        arow[i] = m * LDA;
        if constexpr (MX) sa_base[i] = m * SFA_SM + (FP4 ? 2 * q : q);
        else sa_base[i] = m * SFA_SM;
    }
    int bsrc[NB], sb_base[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
        const int n = min(n0 + j * 16 + l16, N - 1);
        if constexpr (BL == BLay::RAW) bsrc[j] = n * LDB;
        else if constexpr (BL == BLay::KPANEL) bsrc[j] = n * BKB;
        else if constexpr (BL == BLay::W16) bsrc[j] = (n >> 4) * 16 * KB + (n & 15) * 16;
        else bsrc[j] = (n >> 4) * nk * 2048 + L * 16;
        if constexpr (MX) sb_base[j] = n * SFB_SN + (FP4 ? 2 * q : q);
        else sb_base[j] = (n >> 7) * SFB_SN;   // a tile never crosses a 128-column scale block
    }
    // Operands are read with raw buffer loads: per-lane byte offsets that do
    // not change along K (VGPRs) plus a wave-uniform K-tile offset (SGPR).  A
    // ring slot past the wave's last K-tile loads through a zero-range
    // descriptor, which the hardware answers with zeros and no memory
    // traffic; the loads stay unconditional, so the compiler's wait counts
    // stay exact (a load inside a branch makes it wait for every
    // outstanding load).
    int boff[NB][2];               // B chunk h of block j at K-tile 0
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            if constexpr (BL == kBFrag) boff[j][h] = bsrc[j] + h * 1024;
            else if constexpr (BL == BLay::W16) boff[j][h] = bsrc[j] + (h ? c1 : c0) * 256;
            else boff[j][h] = bsrc[j] + (h ? c1 : c0) * 16;
        }
    // bytes between consecutive K-tiles of B, A, and the scale arrays
    const int b_kstep = (BL == BLay::KPANEL) ? N * BKB : ((BL == BLay::RAW) ? BKB : 2048);
    const int s_kstep = MX ? (FP4 ? 8 : 4) : 4;
    const int sa_kstep = MX ? s_kstep : SFA_SK * 4;
    auto rsrc = [](const void* base, bool valid) {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, valid ? 0x7FFFFFFF : 0, 0x00020000);
    };
    auto ld16 = [](__amdgpu_buffer_rsrc_t r, int voff, int soff) -> i32x4 {
        return __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
    };
    int sa_voff[MB], sb_voff[NB];
#pragma unroll
    for (int i = 0; i < MB; ++i) sa_voff[i] = MX ? sa_base[i] : sa_base[i] * 4;
#pragma unroll
    for (int j = 0; j < NB; ++j) sb_voff[j] = MX ? sb_base[j] : sb_base[j] * 4;

    struct Stage {
        i32x8 a[MB];
        i32x8 b[NB];
        int sa[MB];
        int sb[NB];
        float fa[MB];
        float fb;
    };
    auto load = [&](Stage& s, int kt, bool valid) {
        const __amdgpu_buffer_rsrc_t rB = rsrc(B, valid), rA = rsrc(A, valid);
        const __amdgpu_buffer_rsrc_t rSA = rsrc(SFA, valid), rSB = rsrc(SFB, valid);
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const i32x4 lo = ld16(rB, boff[j][0], kt * b_kstep);
            const i32x4 hi = ld16(rB, boff[j][1], kt * b_kstep);
            s.b[j] = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
#pragma unroll
        for (int i = 0; i < MB; ++i) {
            const i32x4 lo = ld16(rA, arow[i] + c0 * 16, kt * BKB);
            const i32x4 hi = ld16(rA, arow[i] + c1 * 16, kt * BKB);
            s.a[i] = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
        if constexpr (MX) {
#pragma unroll
            for (int i = 0; i < MB; ++i) {
                if constexpr (FP4) s.sa[i] = __builtin_amdgcn_raw_buffer_load_b16(rSA, sa_voff[i], kt * sa_kstep, 0);
                else s.sa[i] = __builtin_amdgcn_raw_buffer_load_b8(rSA, sa_voff[i], kt * sa_kstep, 0);
            }
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                if constexpr (FP4) s.sb[j] = __builtin_amdgcn_raw_buffer_load_b16(rSB, sb_voff[j], kt * s_kstep, 0);
                else s.sb[j] = __builtin_amdgcn_raw_buffer_load_b8(rSB, sb_voff[j], kt * s_kstep, 0);
            }
        } else {
#pragma unroll
            for (int i = 0; i < MB; ++i)
                s.fa[i] = __builtin_bit_cast(float,
                                             __builtin_amdgcn_raw_buffer_load_b32(rSA, sa_voff[i], kt * sa_kstep, 0));
            s.fb = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rSB, sb_voff[0], kt * 4, 0));
        }
    };

    f32x4 acc[MB][NB];
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int unit = p.unit_scale;

    auto compute = [&](const Stage& s) {
#pragma unroll
        for (int j = 0; j < NB; ++j) {
#pragma unroll
            for (int i = 0; i < MB; ++i) {
                if constexpr (FP4) {
                    const i32x8 b0 = i32x8{s.b[j][0], s.b[j][1], s.b[j][2], s.b[j][3], 0, 0, 0, 0};
                    const i32x8 b1 = i32x8{s.b[j][4], s.b[j][5], s.b[j][6], s.b[j][7], 0, 0, 0, 0};
                    const i32x8 a0 = i32x8{s.a[i][0], s.a[i][1], s.a[i][2], s.a[i][3], 0, 0, 0, 0};
                    const i32x8 a1 = i32x8{s.a[i][4], s.a[i][5], s.a[i][6], s.a[i][7], 0, 0, 0, 0};
                    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                        b0, a0, acc[i][j], kFmtFp4, kFmtFp4, 0, s.sb[j], 0, s.sa[i]);
                    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                        b1, a1, acc[i][j], kFmtFp4, kFmtFp4, 1, s.sb[j], 1, s.sa[i]);
                } else if constexpr (VALU_SCALE) {
                    const f32x4 part = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                        s.b[j], s.a[i], f32x4{0.f, 0.f, 0.f, 0.f}, kFmtFp8, kFmtFp8, 0, unit, 0, unit);
                    const float sc = s.fa[i] * s.fb;
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[i][j][r] = __builtin_fmaf(part[r], sc, acc[i][j][r]);
                } else {
                    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                        s.b[j], s.a[i], acc[i][j], kFmtFp8, kFmtFp8, 0, s.sb[j], 0, s.sa[i]);
                }
            }
        }
    };

    // ---- K loop: wave w takes K-tiles kt_begin + w, + W, ...; D in flight ----
    const int kfirst = kt_begin + w;
    const int ntw = (kt_end - kfirst + W - 1) / W;     // K-tiles of this wave
    if (ntw > 0) {
        Stage st[D];
#pragma unroll
        for (int d = 0; d < D; ++d) load(st[d], kfirst + W * d, d < ntw);
        int i = 0;
        for (; i + D <= ntw; i += D) {
#pragma unroll
            for (int d = 0; d < D; ++d) {
                compute(st[d]);
                load(st[d], kfirst + W * (i + d + D), i + d + D < ntw);
                __builtin_amdgcn_sched_barrier(0);   // keep the ring order
            }
        }
#pragma unroll
        for (int d = 0; d < D - 1; ++d)
            if (d < ntw - i) compute(st[d]);
    }

    // ---- reduce the eight waves in LDS, in a fixed order:
    // region r (r < 4) = acc(wave r + 4) + acc(wave r); tile = sum of regions 0..3
    auto put = [&](int region, bool add) {
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                f32x4* dst = (f32x4*)&red[region * REGION + (i * 16 + l16) * RP + j * 16 + 4 * q];
                if (add) {
                    const f32x4 u = *dst;
                    f32x4 v = acc[i][j];
                    for (int r = 0; r < 4; ++r) v[r] += u[r];
                    *dst = v;
                } else {
                    *dst = acc[i][j];
                }
            }
    };
    if (w >= 4) put(w - 4, false);
    __syncthreads();
    if (w < 4) put(w, true);
    __syncthreads();
    auto tile_sum = [&](int e) -> f32x4 {    // e = row * COLS + col, col % 4 == 0
        const int o = (e / COLS) * RP + e % COLS;
        f32x4 v = *(const f32x4*)&red[o];
#pragma unroll
        for (int r2 = 1; r2 < 4; ++r2) {
            const f32x4 u = *(const f32x4*)&red[r2 * REGION + o];
            for (int r = 0; r < 4; ++r) v[r] += u[r];
        }
        return v;
    };

    // ---- output: 4 adjacent columns per thread and pass ----
    auto store4 = [&](int row, int col, f32x4 v) {
        const int m = m0 + row, n = n0 + col;
        if (m >= M) return;
        if constexpr (BF16) {
            uint16_t* c = (uint16_t*)p.c + bz * p.c_batch + (long long)m * LDC + n;
            if (n + 3 < N && (LDC & 3) == 0) {
                *(u32x2*)c = u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
            } else {
                for (int r = 0; r < 4; ++r)
                    if (n + r < N) c[r] = bf16_bits(v[r]);
            }
        } else {
            float* c = (float*)p.c + bz * p.c_batch + (long long)m * LDC + n;
            if (n + 3 < N && (LDC & 3) == 0) {
                *(f32x4*)c = v;
            } else {
                for (int r = 0; r < 4; ++r)
                    if (n + r < N) c[r] = v[r];
            }
        }
    };
    if (sp.splitk == 1) {
        for (int e = tid * 4; e < ROWS * COLS; e += NT * 4) store4(e / COLS, e % COLS, tile_sum(e));
        return;
    }

    // split-K: store this slice's partial tile, then the last workgroup of
    // the tile reduces all slices in order 0..splitk-1.  Publication is one
    // acq_rel counter atomic per workgroup (its L2 write-back / invalidate
    // is what makes the partials visible across XCDs); every wave's stores
    // have completed before the barrier that precedes it.
    const long long plane = (long long)M * N;
    const int batch = gridDim.z;
    const long long split_stride = (long long)batch * plane;
    float* part = sp.ws + ((long long)sk * batch + bz) * plane;
    const bool vec_ok = (N & 3) == 0;
    for (int e = tid * 4; e < ROWS * COLS; e += NT * 4) {
        const int m = m0 + e / COLS, n = n0 + e % COLS;
        if (m >= M) continue;
        const f32x4 v = tile_sum(e);
        float* dst = part + (long long)m * N + n;
        if (n + 3 < N && vec_ok) {
            *(f32x4*)dst = v;
        } else {
            for (int r = 0; r < 4; ++r)
                if (n + r < N) dst[r] = v[r];
        }
    }
    wait_vmcnt<0>();
    __syncthreads();
    unsigned* ctr = sp.counters + ((long long)bz * sp.m_tiles + mt) * sp.n_tiles + nt;
    if (tid == 0)
        last_flag = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) ==
                    (unsigned)(sp.splitk - 1);
    __syncthreads();
    if (!last_flag) return;
    const float* ws0 = sp.ws + (long long)bz * plane;
    for (int e = tid * 4; e < ROWS * COLS; e += NT * 4) {
        const int row = e / COLS, col = e % COLS;
        const int m = m0 + row, n = n0 + col;
        if (m >= M) continue;
        const float* src = ws0 + (long long)m * N + n;
        f32x4 v = {0.f, 0.f, 0.f, 0.f};
        if (n + 3 < N && vec_ok) {
            // eight slices in flight per batch of loads, summed in slice order
            for (int s0 = 0; s0 < sp.splitk; s0 += 8) {
                f32x4 u[8];
#pragma unroll
                for (int t = 0; t < 8; ++t)
                    if (s0 + t < sp.splitk) u[t] = *(const f32x4*)(src + (s0 + t) * split_stride);
#pragma unroll
                for (int t = 0; t < 8; ++t)
                    if (s0 + t < sp.splitk)
                        for (int r = 0; r < 4; ++r) v[r] += u[t][r];
            }
        } else {
            for (int s0 = 0; s0 < sp.splitk; ++s0)
                for (int r = 0; r < 4; ++r)
                    if (n + r < N) v[r] += src[s0 * split_stride + r];
        }
        store4(row, col, v);
    }
    if (tid == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Launches one instantiation of a format / scale / B-layout family.
template <int FMT, ScaleKind SK, BLay BL>
hipError_t launch_skinny_family(const SkinnyArgs& a, int mb, int nb, int batch, bool bf16, hipStream_t s) {
    const dim3 grid(skinny_grid_x(a.n_tiles, a.m_tiles), a.splitk, batch);
    const dim3 block(kSkinnyWaves * 64);
#define QG_SKINNY_CASE(MBV, NBV)                                                                  \
    if (mb == MBV && nb == NBV) {                                                                 \
        if (bf16) skinny_gemm_kernel<FMT, SK, BL, MBV, NBV, true><<<grid, block, 0, s>>>(a);      \
        else skinny_gemm_kernel<FMT, SK, BL, MBV, NBV, false><<<grid, block, 0, s>>>(a);          \
        return hipGetLastError();                                                                 \
    }
    QG_SKINNY_CASE(1, 1) QG_SKINNY_CASE(1, 2) QG_SKINNY_CASE(1, 4)
    QG_SKINNY_CASE(2, 1) QG_SKINNY_CASE(2, 2) QG_SKINNY_CASE(2, 4)
    QG_SKINNY_CASE(4, 1) QG_SKINNY_CASE(4, 2) QG_SKINNY_CASE(4, 4)
#undef QG_SKINNY_CASE
    return hipErrorInvalidValue;
}

}  // namespace qg
