// Instantiations and launcher of the eight-wave fp32-block-scale kernel.
#include "bsf32_gemm.hpp"
#include "launch.hpp"

namespace qg {

hipError_t launch_bsf32(const TileArgs& a, int batch, bool bf16, bool frag, hipStream_t s) {
    const dim3 grid(a.tiles_m * a.tiles_n, 1, batch);
    if (frag) {
        if (bf16) bsf32_gemm_kernel<true, BLay::FRAG><<<grid, 512, 0, s>>>(a);
        else bsf32_gemm_kernel<false, BLay::FRAG><<<grid, 512, 0, s>>>(a);
    } else {
        if (bf16) bsf32_gemm_kernel<true, BLay::KPANEL><<<grid, 512, 0, s>>>(a);
        else bsf32_gemm_kernel<false, BLay::KPANEL><<<grid, 512, 0, s>>>(a);
    }
    trace_launch("bsf32_gemm<fp8,BSF32,%s,%s>", frag ? "FRAG" : "KPANEL", bf16 ? "bf16" : "fp32");
    return hipGetLastError();
}

}  // namespace qg
