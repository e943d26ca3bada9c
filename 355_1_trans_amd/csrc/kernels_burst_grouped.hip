// Instantiations and launcher of the grouped burst kernel for fp8 with fp32
// block scales (several decode GEMMs in one launch; K-panel B' or
// fragment-order B'').
#include "burst_launch.hpp"

namespace qg {

hipError_t launch_burst_grouped(const BurstGroup& g, bool frag, int mb, int nb, int waves, int grid, bool bf16,
                                hipStream_t s) {
    return frag ? burst::launch_layout<kFmtFp8, BLay::FRAG>(g, mb, nb, waves, grid, bf16, s)
                : burst::launch_layout<kFmtFp8, BLay::KPANEL>(g, mb, nb, waves, grid, bf16, s);
}

}  // namespace qg
