// Instantiations and launcher of the grouped burst kernel for MXFP8 / MXFP4
// with row-major B and row-major E8M0 scales (several decode GEMMs in one
// launch).
#include "burst_launch.hpp"

namespace qg {

hipError_t launch_burst_mx_grouped(const BurstGroup& g, bool fp4, int mb, int nb, int waves, int grid, bool bf16,
                                   hipStream_t s) {
    return fp4 ? burst::launch_layout<kFmtFp4, BLay::RAW>(g, mb, nb, waves, grid, bf16, s)
               : burst::launch_layout<kFmtFp8, BLay::RAW>(g, mb, nb, waves, grid, bf16, s);
}

}  // namespace qg
