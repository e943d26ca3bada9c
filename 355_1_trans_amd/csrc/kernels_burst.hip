// Instantiations and launcher of the burst kernel (fp8, fp32 block scales,
// M <= 64, K-panel B' or fragment-order B'').
#include "burst_gemm.hpp"
#include "launch.hpp"

namespace qg {

namespace {
template <BLay BL, int MB, int NB, int W, int KPW>
hipError_t launch_burst_kpw(const BurstArgs& a, int batch, bool bf16, hipStream_t s) {
    const dim3 grid(a.n_tiles * a.splitk, batch);
    if (bf16) burst_gemm_kernel<BL, MB, NB, W, KPW, true><<<grid, W * 64, 0, s>>>(a);
    else burst_gemm_kernel<BL, MB, NB, W, KPW, false><<<grid, W * 64, 0, s>>>(a);
    trace_launch("burst_gemm<fp8,BSF32,%s,mb%d,nb%d,w%d,kpw%d,%s,splitk%d>", layout_name(BL), MB, NB, W, KPW,
                 bf16 ? "bf16" : "fp32", a.splitk);
    return hipGetLastError();
}

template <BLay BL, int MB, int NB, int W>
hipError_t launch_burst_waves(const BurstArgs& a, int batch, bool bf16, hipStream_t s) {
    constexpr bool fits = burst_lds_bytes(MB, NB, W, BL == BLay::KPANEL) <= kBurstLdsMax &&
                          burst_max_kpw(MB, NB, W) > 0;
    if constexpr (!fits) {
        return hipErrorInvalidValue;
    } else {
        const int per_wave = (a.kt_per_split + W - 1) / W;
        if (per_wave < 1 || per_wave > burst_max_kpw(MB, NB, W)) return hipErrorInvalidValue;
        if (per_wave == 1) return launch_burst_kpw<BL, MB, NB, W, 1>(a, batch, bf16, s);
        if (per_wave == 2) return launch_burst_kpw<BL, MB, NB, W, 2>(a, batch, bf16, s);
        if (per_wave <= 4) return launch_burst_kpw<BL, MB, NB, W, 4>(a, batch, bf16, s);
        if constexpr (burst_max_kpw(MB, NB, W) >= 8) return launch_burst_kpw<BL, MB, NB, W, 8>(a, batch, bf16, s);
        return hipErrorInvalidValue;
    }
}

template <BLay BL, int MB, int NB>
hipError_t launch_burst_shape(const BurstArgs& a, int waves, int batch, bool bf16, hipStream_t s) {
    if (a.n_tiles < 1 || a.splitk < 1) return hipErrorInvalidValue;
    if (waves == 4) return launch_burst_waves<BL, MB, NB, 4>(a, batch, bf16, s);
    if (waves == 8) return launch_burst_waves<BL, MB, NB, 8>(a, batch, bf16, s);
    if (waves == 16) return launch_burst_waves<BL, MB, NB, 16>(a, batch, bf16, s);
    return hipErrorInvalidValue;
}

template <BLay BL>
hipError_t launch_burst_layout(const BurstArgs& a, int mb, int nb, int waves, int batch, bool bf16, hipStream_t s) {
#define QG_BURST(MBV, NBV) \
    if (mb == MBV && nb == NBV) return launch_burst_shape<BL, MBV, NBV>(a, waves, batch, bf16, s);
    QG_BURST(1, 1) QG_BURST(1, 2) QG_BURST(2, 1) QG_BURST(2, 2) QG_BURST(4, 1) QG_BURST(4, 2)
#undef QG_BURST
    return hipErrorInvalidValue;
}
}  // namespace

hipError_t launch_burst(const BurstArgs& a, bool frag, int mb, int nb, int waves, int batch, bool bf16,
                        hipStream_t s) {
    return frag ? launch_burst_layout<BLay::FRAG>(a, mb, nb, waves, batch, bf16, s)
                : launch_burst_layout<BLay::KPANEL>(a, mb, nb, waves, batch, bf16, s);
}

}  // namespace qg
