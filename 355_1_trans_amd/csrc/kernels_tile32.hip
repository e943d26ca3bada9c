// Instantiations and launchers of the 32x32x64 tile kernel.
#include "launch.hpp"
#include "tile32_gemm.hpp"

namespace qg {

namespace {
template <int FMT, ScaleKind SK, BLay BL, int PB = 16>
hipError_t launch_tile32(const TileArgs& a, int batch, bool bf16, hipStream_t s) {
    const dim3 grid(a.tiles_m * a.tiles_n, 1, batch);
    if (bf16) tile32_gemm_kernel<FMT, SK, BL, true, PB><<<grid, 512, 0, s>>>(a);
    else tile32_gemm_kernel<FMT, SK, BL, false, PB><<<grid, 512, 0, s>>>(a);
    return hipGetLastError();
}
}  // namespace

hipError_t launch_tile32_mx8_raw(const TileArgs& a, int batch, bool bf16, bool wide_panels, hipStream_t s) {
    return wide_panels ? launch_tile32<kFmtFp8, ScaleKind::MX, BLay::RAW, 16>(a, batch, bf16, s)
                       : launch_tile32<kFmtFp8, ScaleKind::MX, BLay::RAW, 4>(a, batch, bf16, s);
}
hipError_t launch_tile32_mx4_raw(const TileArgs& a, int batch, bool bf16, bool wide_panels, hipStream_t s) {
    return wide_panels ? launch_tile32<kFmtFp4, ScaleKind::MX, BLay::RAW, 16>(a, batch, bf16, s)
                       : launch_tile32<kFmtFp4, ScaleKind::MX, BLay::RAW, 8>(a, batch, bf16, s);
}
hipError_t launch_tile32_bs8_w16(const TileArgs& a, int batch, bool bf16, hipStream_t s) {
    return launch_tile32<kFmtFp8, ScaleKind::BS8, BLay::W16>(a, batch, bf16, s);
}
hipError_t launch_tile32_bsf32_kpanel(const TileArgs& a, int batch, bool bf16, hipStream_t s) {
    return launch_tile32<kFmtFp8, ScaleKind::BSF32, BLay::KPANEL>(a, batch, bf16, s);
}

}  // namespace qg
