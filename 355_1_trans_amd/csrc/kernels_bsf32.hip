// Instantiations and launcher of the eight-wave fp32-block-scale kernel.
#include "bsf32_gemm.hpp"
#include "launch.hpp"

namespace qg {

hipError_t launch_bsf32(const Bsf32Args& a, int batch, bool bf16, bool frag, hipStream_t s) {
    const long long items = (long long)a.t.tiles_m * a.t.tiles_n * batch;
    const long long tail = items - a.dp_tiles;
    const dim3 grid((unsigned)(a.tail_split > 1 ? a.dp_tiles + tail * a.tail_split : items), 1, 1);
    if (frag) {
        if (bf16) bsf32_gemm_kernel<true, BLay::FRAG><<<grid, 512, 0, s>>>(a);
        else bsf32_gemm_kernel<false, BLay::FRAG><<<grid, 512, 0, s>>>(a);
    } else {
        if (bf16) bsf32_gemm_kernel<true, BLay::KPANEL><<<grid, 512, 0, s>>>(a);
        else bsf32_gemm_kernel<false, BLay::KPANEL><<<grid, 512, 0, s>>>(a);
    }
    if (a.tail_split > 1)
        trace_launch("bsf32_gemm<fp8,BSF32,%s,%s,tail%lldx%d>", frag ? "FRAG" : "KPANEL", bf16 ? "bf16" : "fp32", tail,
                     a.tail_split);
    else
        trace_launch("bsf32_gemm<fp8,BSF32,%s,%s>", frag ? "FRAG" : "KPANEL", bf16 ? "bf16" : "fp32");
    return hipGetLastError();
}

}  // namespace qg
