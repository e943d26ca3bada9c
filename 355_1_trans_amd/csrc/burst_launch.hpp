// Launch helpers of the burst kernel, shared by its instantiation units
// (kernels_burst.hip: fp8 with fp32 block scales; kernels_burst_mx.hip:
// MXFP8 / MXFP4 with row-major B): the tile shape, wave count and K-tiles per
// wave picked at run time map onto one compiled instantiation.
#pragma once
#include "burst_gemm.hpp"
#include "launch.hpp"

namespace qg {
namespace burst {

template <int FMT, BLay BL, int MB, int NB, int W, int KPW>
hipError_t launch_kpw(const BurstArgs& a, int batch, bool bf16, hipStream_t s) {
    const dim3 grid(a.n_tiles * a.splitk, batch);
    if (bf16) burst_gemm_kernel<FMT, BL, MB, NB, W, KPW, true><<<grid, W * 64, 0, s>>>(a);
    else burst_gemm_kernel<FMT, BL, MB, NB, W, KPW, false><<<grid, W * 64, 0, s>>>(a);
    trace_launch("burst_gemm<%s,%s,%s,mb%d,nb%d,w%d,kpw%d,%s,splitk%d>", FMT == kFmtFp4 ? "fp4" : "fp8",
                 BL == BLay::RAW ? "MX" : "BSF32", layout_name(BL), MB, NB, W, KPW, bf16 ? "bf16" : "fp32", a.splitk);
    return hipGetLastError();
}

template <int FMT, BLay BL, int MB, int NB, int W>
hipError_t launch_waves(const BurstArgs& a, int batch, bool bf16, hipStream_t s) {
    constexpr bool MX = BL == BLay::RAW;
    constexpr int KMAX = burst_max_kpw(MB, NB, W, MX);
    constexpr bool fits = burst_lds_bytes(MB, NB, W, BL != BLay::FRAG) <= kBurstLdsMax && KMAX > 0;
    if constexpr (!fits) {
        return hipErrorInvalidValue;
    } else {
        const int per_wave = (a.kt_per_split + W - 1) / W;
        if (per_wave < 1 || per_wave > KMAX) return hipErrorInvalidValue;
        if (per_wave == 1) return launch_kpw<FMT, BL, MB, NB, W, 1>(a, batch, bf16, s);
        if (per_wave == 2) return launch_kpw<FMT, BL, MB, NB, W, 2>(a, batch, bf16, s);
        if constexpr (KMAX >= 4)
            if (per_wave <= 4) return launch_kpw<FMT, BL, MB, NB, W, 4>(a, batch, bf16, s);
        if constexpr (KMAX >= 8) return launch_kpw<FMT, BL, MB, NB, W, 8>(a, batch, bf16, s);
        return hipErrorInvalidValue;
    }
}

template <int FMT, BLay BL, int MB, int NB>
hipError_t launch_shape(const BurstArgs& a, int waves, int batch, bool bf16, hipStream_t s) {
    if (a.n_tiles < 1 || a.splitk < 1) return hipErrorInvalidValue;
    if (waves == 8) return launch_waves<FMT, BL, MB, NB, 8>(a, batch, bf16, s);
    if (waves == 16) return launch_waves<FMT, BL, MB, NB, 16>(a, batch, bf16, s);
    return hipErrorInvalidValue;
}

template <int FMT, BLay BL>
hipError_t launch_layout(const BurstArgs& a, int mb, int nb, int waves, int batch, bool bf16, hipStream_t s) {
#define QG_BURST(MBV, NBV) \
    if (mb == MBV && nb == NBV) return launch_shape<FMT, BL, MBV, NBV>(a, waves, batch, bf16, s);
    QG_BURST(1, 1) QG_BURST(1, 2) QG_BURST(2, 1) QG_BURST(2, 2) QG_BURST(4, 1) QG_BURST(4, 2)
#undef QG_BURST
    return hipErrorInvalidValue;
}

}  // namespace burst
}  // namespace qg
