// MXFP4 instantiations of the skinny-M / split-K kernel.
#include "launch.hpp"
#include "skinny_gemm.hpp"

namespace qg {

hipError_t launch_skinny_mx4(const SkinnyArgs& a, int mb, int nb, int batch, bool bf16, hipStream_t s) {
    return launch_skinny_family<kFmtFp4, ScaleKind::MX, BLay::RAW>(a, mb, nb, batch, bf16, s);
}

}  // namespace qg
