// Instantiation and launcher of the 8-wave 32x32x64 tile kernel (fp32 block scales).
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

hipError_t launch_tile32_bsf32_kpanel(const TileArgs& a, int batch, bool bf16, hipStream_t s) {
    return launch_tile32<kFmtFp8, ScaleKind::BSF32, BLay::KPANEL>(a, batch, bf16, s);
}

}  // namespace qg
