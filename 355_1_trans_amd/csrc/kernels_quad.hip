// Instantiations and launcher of the one-by-four wave MXFP4 tile kernel
// (quad_gemm.hpp): B in shuffle_weight(16,16) order (W16) or row-major,
// scales in e8m0_shuffle order, bf16 or fp32 output.
#include "launch.hpp"
#include "quad_gemm.hpp"

namespace qg {

hipError_t launch_quad_mx4(const TileArgs& a, int batch, bool w16, bool bf16, hipStream_t s) {
    const dim3 grid(a.tiles_m * a.tiles_n, 1, batch);
    if (w16) {
        if (bf16) quad_gemm_kernel<BLay::W16, true><<<grid, 256, 0, s>>>(a);
        else quad_gemm_kernel<BLay::W16, false><<<grid, 256, 0, s>>>(a);
    } else {
        if (bf16) quad_gemm_kernel<BLay::RAW, true><<<grid, 256, 0, s>>>(a);
        else quad_gemm_kernel<BLay::RAW, false><<<grid, 256, 0, s>>>(a);
    }
    trace_launch("quad_gemm<fp4,MXS,%s,%s>", w16 ? "W16" : "RAW", bf16 ? "bf16" : "fp32");
    return hipGetLastError();
}

}  // namespace qg
