// Instantiations and launchers of the four-wave tile kernel.
#include "launch.hpp"
#include "wide_gemm.hpp"

namespace qg {

namespace {
template <int FMT, ScaleKind SK, BLay BL, int PB = 16>
hipError_t launch_wide(const TileArgs& a, int batch, bool bf16, hipStream_t s) {
    const dim3 grid(a.tiles_m * a.tiles_n, 1, batch);
    const dim3 block(256);
    if (bf16) wide_gemm_kernel<FMT, SK, BL, true, PB><<<grid, block, 0, s>>>(a);
    else wide_gemm_kernel<FMT, SK, BL, false, PB><<<grid, block, 0, s>>>(a);
    return hipGetLastError();
}
}  // namespace

hipError_t launch_wide_mx8_raw(const TileArgs& a, int batch, bool bf16, int panel_bytes, hipStream_t s) {
    if (panel_bytes == 16) return launch_wide<kFmtFp8, ScaleKind::MX, BLay::RAW, 16>(a, batch, bf16, s);
    return launch_wide<kFmtFp8, ScaleKind::MX, BLay::RAW, 4>(a, batch, bf16, s);
}
hipError_t launch_wide_mx4_raw(const TileArgs& a, int batch, bool bf16, int panel_bytes, hipStream_t s) {
    if (panel_bytes == 32) return launch_wide<kFmtFp4, ScaleKind::MX, BLay::RAW, 32>(a, batch, bf16, s);
    if (panel_bytes == 16) return launch_wide<kFmtFp4, ScaleKind::MX, BLay::RAW, 16>(a, batch, bf16, s);
    return launch_wide<kFmtFp4, ScaleKind::MX, BLay::RAW, 8>(a, batch, bf16, s);
}
hipError_t launch_wide_bs8_w16(const TileArgs& a, int batch, bool bf16, hipStream_t s) {
    return launch_wide<kFmtFp8, ScaleKind::BS8, BLay::W16>(a, batch, bf16, s);
}

}  // namespace qg
