// Instantiations and launchers of the four-wave tile kernel.
#include "launch.hpp"
#include "wide_gemm.hpp"

namespace qg {

namespace {
template <int FMT, ScaleKind SK, BLay BL, int PB = 16, bool AKM = false>
hipError_t launch_wide(const TileArgs& a, int batch, bool bf16, hipStream_t s) {
    const dim3 grid(a.tiles_m * a.tiles_n, 1, batch);
    const dim3 block(256);
    if (bf16) wide_gemm_kernel<FMT, SK, BL, true, PB, false, AKM><<<grid, block, 0, s>>>(a);
    else wide_gemm_kernel<FMT, SK, BL, false, PB, false, AKM><<<grid, block, 0, s>>>(a);
    trace_launch("wide_gemm<%s,%s,%s,%s,pb%d%s>", FMT == kFmtFp4 ? "fp4" : "fp8", scale_name(SK), layout_name(BL),
                 bf16 ? "bf16" : "fp32", PB, AKM ? ",akm" : "");
    return hipGetLastError();
}
// persistent grid of `blocks` workgroups (a.persist = 1, a.batch set)
template <int FMT, ScaleKind SK, BLay BL, int PB>
hipError_t launch_wide_persist(const TileArgs& a, int blocks, bool bf16, hipStream_t s) {
    const dim3 grid(blocks, 1, 1);
    const dim3 block(256);
    if (bf16) wide_gemm_kernel<FMT, SK, BL, true, PB, true><<<grid, block, 0, s>>>(a);
    else wide_gemm_kernel<FMT, SK, BL, false, PB, true><<<grid, block, 0, s>>>(a);
    trace_launch("wide_gemm<%s,%s,%s,%s,pb%d,persist%d>", FMT == kFmtFp4 ? "fp4" : "fp8", scale_name(SK),
                 layout_name(BL), bf16 ? "bf16" : "fp32", PB, blocks);
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
hipError_t launch_wide_mx4_w16s(const TileArgs& a, int batch, bool bf16, int panel_bytes, int persist_blocks,
                                hipStream_t s) {
    if (persist_blocks > 0) {
        TileArgs t = a;
        t.persist = 1;
        t.batch = batch;
        if (panel_bytes == 32)
            return launch_wide_persist<kFmtFp4, ScaleKind::MXS, BLay::W16, 32>(t, persist_blocks, bf16, s);
        return launch_wide_persist<kFmtFp4, ScaleKind::MXS, BLay::W16, 8>(t, persist_blocks, bf16, s);
    }
    if (panel_bytes == 32) return launch_wide<kFmtFp4, ScaleKind::MXS, BLay::W16, 32>(a, batch, bf16, s);
    return launch_wide<kFmtFp4, ScaleKind::MXS, BLay::W16, 8>(a, batch, bf16, s);
}
hipError_t launch_wide_bs8_w16(const TileArgs& a, int batch, bool bf16, hipStream_t s) {
    return launch_wide<kFmtFp8, ScaleKind::BS8, BLay::W16>(a, batch, bf16, s);
}
hipError_t launch_wide_bs8_kmajor(const TileArgs& a, int batch, bool bf16, bool a_km, bool b_kn, hipStream_t s) {
    if (a_km && b_kn) return launch_wide<kFmtFp8, ScaleKind::BS8, BLay::KN, 16, true>(a, batch, bf16, s);
    if (a_km) return launch_wide<kFmtFp8, ScaleKind::BS8, BLay::RAW, 16, true>(a, batch, bf16, s);
    if (b_kn) return launch_wide<kFmtFp8, ScaleKind::BS8, BLay::KN>(a, batch, bf16, s);
    return hipErrorInvalidValue;
}

// E8M0 scales [rows][ngroups] (row pitch ld) -> panel-major [ngroups/pb][rows][pb]
// for both operands (grid.z), one 16-byte piece per thread: consecutive
// threads take consecutive pieces of a row (a wave reads 1 KB of whole rows
// contiguously) and write them into their panels (runs of 64 bytes).
__global__ __launch_bounds__(256) void mx_scale_panels_kernel(const ScalePanelArgs a) {
    const int op = blockIdx.z, bz = blockIdx.y;
    const int rows = a.rows[op], per_row = a.ngroups / 16, pieces = a.pb / 16;
    const long long units = (long long)rows * per_row;
    const uint8_t* src = a.src[op] + (long long)bz * a.src_batch[op];
    uint8_t* dst = a.dst[op] + (long long)bz * a.dst_batch[op];
    for (long long u = (long long)blockIdx.x * 256 + threadIdx.x; u < units; u += (long long)gridDim.x * 256) {
        const int r = (int)(u / per_row), j = (int)(u - (long long)r * per_row);
        const int pnl = j / pieces, h = j - pnl * pieces;
        const i32x4 v = *(const i32x4*)(src + (long long)r * a.ld[op] + 16 * j);
        *(i32x4*)(dst + ((long long)pnl * rows + r) * a.pb + 16 * h) = v;
    }
}

hipError_t launch_mx_scale_panels(const ScalePanelArgs& a, int batch, hipStream_t s) {
    if ((a.pb != 16 && a.pb != 32) || a.ngroups % a.pb) return hipErrorInvalidValue;
    const long long units = (long long)(a.rows[0] > a.rows[1] ? a.rows[0] : a.rows[1]) * (a.ngroups / 16);
    const long long blocks = (units + 255) / 256;
    const dim3 grid((unsigned)(blocks < 1024 ? blocks : 1024), batch, 2);
    mx_scale_panels_kernel<<<grid, 256, 0, s>>>(a);
    trace_launch("mx_scale_panels<pb%d>", a.pb);
    return hipGetLastError();
}

}  // namespace qg
