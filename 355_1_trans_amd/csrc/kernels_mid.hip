// Instantiations and launcher of the four-wave 128 x 128 kernel: fp8 with fp32
// block scales (K-panel B' or fragment-order B''), MXFP8 and MXFP4 (row-major B).
#include "launch.hpp"
#include "mid_gemm.hpp"

namespace qg {

template <BLay BL, int ST, ScaleKind SK, int FMT>
static void mid_go(const MidArgs& a, const dim3& grid, bool bf16, hipStream_t s) {
    if (bf16) mid_gemm_kernel<true, BL, ST, SK, FMT><<<grid, 256, 0, s>>>(a);
    else mid_gemm_kernel<false, BL, ST, SK, FMT><<<grid, 256, 0, s>>>(a);
}

template <int ST>
static void mid_kind(const MidArgs& a, const dim3& grid, bool bf16, MidKind kind, hipStream_t s) {
    switch (kind) {
    case MidKind::BS_KPANEL: mid_go<BLay::KPANEL, ST, ScaleKind::BSF32, kFmtFp8>(a, grid, bf16, s); break;
    case MidKind::BS_FRAG: mid_go<BLay::FRAG, ST, ScaleKind::BSF32, kFmtFp8>(a, grid, bf16, s); break;
    case MidKind::MX8: mid_go<BLay::RAW, ST, ScaleKind::MX, kFmtFp8>(a, grid, bf16, s); break;
    case MidKind::MX4: mid_go<BLay::RAW, ST, ScaleKind::MX, kFmtFp4>(a, grid, bf16, s); break;
    }
}

hipError_t launch_mid(const MidArgs& a, int batch, bool bf16, MidKind kind, int stages, hipStream_t s) {
    const dim3 grid(a.t.tiles_m * a.t.tiles_n, a.splitk, batch);
    if (stages == 2) mid_kind<2>(a, grid, bf16, kind, s);
    else if (stages == 4) mid_kind<4>(a, grid, bf16, kind, s);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace qg
