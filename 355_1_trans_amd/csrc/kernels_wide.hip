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

// E8M0 scales [rows][ngroups] (row pitch ld) -> panel-major [ngroups/pb][rows][pb]
// for both operands (grid.z), one 16-byte piece per thread; writes are
// contiguous, reads one piece of a row each.
__global__ __launch_bounds__(256) void mx_scale_panels_kernel(const ScalePanelArgs a) {
    const int op = blockIdx.z, bz = blockIdx.y;
    const int rows = a.rows[op], pieces = a.pb / 16;
    const long long units = (long long)(a.ngroups / a.pb) * rows * pieces;
    const uint8_t* src = a.src[op] + (long long)bz * a.src_batch[op];
    uint8_t* dst = a.dst[op] + (long long)bz * a.dst_batch[op];
    for (long long u = (long long)blockIdx.x * 256 + threadIdx.x; u < units; u += (long long)gridDim.x * 256) {
        const int h = (int)(u % pieces);
        const long long rp = u / pieces;
        const int r = (int)(rp % rows), pnl = (int)(rp / rows);
        const i32x4 v = *(const i32x4*)(src + (long long)r * a.ld[op] + pnl * a.pb + 16 * h);
        *(i32x4*)(dst + u * 16) = v;
    }
}

hipError_t launch_mx_scale_panels(const ScalePanelArgs& a, int batch, hipStream_t s) {
    if ((a.pb != 16 && a.pb != 32) || a.ngroups % a.pb) return hipErrorInvalidValue;
    const long long units = (long long)(a.ngroups / a.pb) * (a.rows[0] > a.rows[1] ? a.rows[0] : a.rows[1]) * (a.pb / 16);
    const long long blocks = (units + 255) / 256;
    const dim3 grid((unsigned)(blocks < 1024 ? blocks : 1024), batch, 2);
    mx_scale_panels_kernel<<<grid, 256, 0, s>>>(a);
    return hipGetLastError();
}

}  // namespace qg
