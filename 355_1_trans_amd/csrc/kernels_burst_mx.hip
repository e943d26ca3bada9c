// Instantiations and launchers of the burst kernel for MXFP8 / MXFP4 with
// row-major B and row-major E8M0 scales (M <= 64); the grouped kernel's are
// in kernels_burst_mx_grouped.hip.
#include "burst_launch.hpp"

namespace qg {

hipError_t launch_burst_mx(const BurstArgs& a, bool fp4, int mb, int nb, int waves, int batch, bool bf16,
                           hipStream_t s) {
    return fp4 ? burst::launch_layout<kFmtFp4, BLay::RAW>(a, mb, nb, waves, batch, bf16, s)
               : burst::launch_layout<kFmtFp8, BLay::RAW>(a, mb, nb, waves, batch, bf16, s);
}

}  // namespace qg
