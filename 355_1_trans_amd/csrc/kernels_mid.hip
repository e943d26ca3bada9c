// Instantiations and launcher of the four-wave 128 x 128 fp32-block-scale kernel.
#include "launch.hpp"
#include "mid_gemm.hpp"

namespace qg {

hipError_t launch_mid(const MidArgs& a, int batch, bool bf16, bool frag, int stages, hipStream_t s) {
    const dim3 grid(a.t.tiles_m * a.t.tiles_n, a.splitk, batch);
#define QG_MID(ST)                                                                    \
    if (frag) {                                                                       \
        if (bf16) mid_gemm_kernel<true, BLay::FRAG, ST><<<grid, 256, 0, s>>>(a);      \
        else mid_gemm_kernel<false, BLay::FRAG, ST><<<grid, 256, 0, s>>>(a);          \
    } else {                                                                          \
        if (bf16) mid_gemm_kernel<true, BLay::KPANEL, ST><<<grid, 256, 0, s>>>(a);    \
        else mid_gemm_kernel<false, BLay::KPANEL, ST><<<grid, 256, 0, s>>>(a);        \
    }
    if (stages == 2) { QG_MID(2) }
    else if (stages == 4) { QG_MID(4) }
    else return hipErrorInvalidValue;
#undef QG_MID
    return hipGetLastError();
}

}  // namespace qg
