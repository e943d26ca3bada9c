// Launch helpers of the burst kernel, shared by its instantiation units
// (kernels_burst.hip: fp8 with fp32 block scales; kernels_burst_mx.hip:
// MXFP8 / MXFP4 with row-major B): the tile shape, wave count and K-tiles per
// wave picked at run time map onto one compiled instantiation, of the
// single-problem kernel (BurstArgs, grid = tiles x slices x batch) or of the
// grouped kernel (BurstGroup, grid = work items or a persistent grid).
#pragma once
#include "burst_gemm.hpp"
#include "launch.hpp"

namespace qg {
namespace burst {

// K-tiles per wave the launch needs: the largest slice over its problems
inline int per_wave(const BurstArgs& a, int w) { return (a.kt_per_split + w - 1) / w; }
inline int per_wave(const BurstGroup& g, int w) {
    int pw = 0;
    for (int j = 0; j < g.count; ++j) pw = pw > per_wave(g.p[j], w) ? pw : per_wave(g.p[j], w);
    return pw;
}
inline bool valid(const BurstArgs& a) { return a.n_tiles >= 1 && a.splitk >= 1; }
inline bool valid(const BurstGroup& g) {
    if (g.count < 1 || g.count > kGroupMax || g.item_begin[0] != 0) return false;
    for (int j = 0; j < g.count; ++j)
        if (!valid(g.p[j]) || g.item_begin[j + 1] - g.item_begin[j] != g.p[j].n_tiles * g.p[j].splitk) return false;
    return true;
}

// scale policy of an instantiation: row-major E8M0 (RAW B), e8m0_shuffle
// (fp4 with W16 = B'' bytes), or fp32 block scales
template <int FMT, BLay BL>
constexpr const char* scale_tag() {
    return BL == BLay::RAW ? "MX" : (FMT == kFmtFp4 && BL == BLay::FRAG) ? "MXS" : "BSF32";
}
template <int FMT, BLay BL>
constexpr bool is_mx() {
    return BL == BLay::RAW || (FMT == kFmtFp4 && BL == BLay::FRAG);
}

template <int FMT, BLay BL, int MB, int NB, int W, int KPW>
hipError_t launch_kpw(const BurstArgs& a, int batch, bool bf16, hipStream_t s) {
    const dim3 grid(a.n_tiles * a.splitk, batch);
    if (bf16) burst_gemm_kernel<FMT, BL, MB, NB, W, KPW, true><<<grid, W * 64, 0, s>>>(a);
    else burst_gemm_kernel<FMT, BL, MB, NB, W, KPW, false><<<grid, W * 64, 0, s>>>(a);
    trace_launch("burst_gemm<%s,%s,%s,mb%d,nb%d,w%d,kpw%d,%s,splitk%d>", FMT == kFmtFp4 ? "fp4" : "fp8",
                 scale_tag<FMT, BL>(), layout_name(BL), MB, NB, W, KPW, bf16 ? "bf16" : "fp32", a.splitk);
    return hipGetLastError();
}

// grouped: `grid` workgroups (the item count, or fewer for a persistent grid)
template <int FMT, BLay BL, int MB, int NB, int W, int KPW>
hipError_t launch_kpw(const BurstGroup& g, int grid, bool bf16, hipStream_t s) {
    if (bf16) burst_grouped_kernel<FMT, BL, MB, NB, W, KPW, true><<<grid, W * 64, 0, s>>>(g);
    else burst_grouped_kernel<FMT, BL, MB, NB, W, KPW, false><<<grid, W * 64, 0, s>>>(g);
    trace_launch("burst_grouped<%s,%s,%s,mb%d,nb%d,w%d,kpw%d,%s,g%d,items%d,grid%d>", FMT == kFmtFp4 ? "fp4" : "fp8",
                 scale_tag<FMT, BL>(), layout_name(BL), MB, NB, W, KPW, bf16 ? "bf16" : "fp32", g.count,
                 g.item_begin[g.count], grid);
    return hipGetLastError();
}

// `extent`: the batch count (BurstArgs) or the grid (BurstGroup)
template <int FMT, BLay BL, int MB, int NB, int W, class Args>
hipError_t launch_waves(const Args& a, int extent, bool bf16, hipStream_t s) {
    constexpr int KMAX = burst_max_kpw(MB, NB, W, is_mx<FMT, BL>());
    constexpr bool fits = burst_lds_bytes(MB, NB, W, BL != BLay::FRAG) <= kBurstLdsMax && KMAX > 0;
    if constexpr (!fits) {
        return hipErrorInvalidValue;
    } else {
        const int pw = per_wave(a, W);
        if (pw < 1 || pw > KMAX) return hipErrorInvalidValue;
        if (pw == 1) return launch_kpw<FMT, BL, MB, NB, W, 1>(a, extent, bf16, s);
        if (pw == 2) return launch_kpw<FMT, BL, MB, NB, W, 2>(a, extent, bf16, s);
        if constexpr (KMAX >= 4)
            if (pw <= 4) return launch_kpw<FMT, BL, MB, NB, W, 4>(a, extent, bf16, s);
        if constexpr (KMAX >= 8) return launch_kpw<FMT, BL, MB, NB, W, 8>(a, extent, bf16, s);
        return hipErrorInvalidValue;
    }
}

template <int FMT, BLay BL, int MB, int NB, class Args>
hipError_t launch_shape(const Args& a, int waves, int extent, bool bf16, hipStream_t s) {
    if (!valid(a) || extent < 1) return hipErrorInvalidValue;
    if (waves == 8) return launch_waves<FMT, BL, MB, NB, 8>(a, extent, bf16, s);
    if (waves == 16) return launch_waves<FMT, BL, MB, NB, 16>(a, extent, bf16, s);
    return hipErrorInvalidValue;
}

template <int FMT, BLay BL, class Args>
hipError_t launch_layout(const Args& a, int mb, int nb, int waves, int extent, bool bf16, hipStream_t s) {
#define QG_BURST(MBV, NBV) \
    if (mb == MBV && nb == NBV) return launch_shape<FMT, BL, MBV, NBV>(a, waves, extent, bf16, s);
    QG_BURST(1, 1) QG_BURST(1, 2) QG_BURST(2, 1) QG_BURST(2, 2) QG_BURST(4, 1) QG_BURST(4, 2)
#undef QG_BURST
    return hipErrorInvalidValue;
}

}  // namespace burst
}  // namespace qg
