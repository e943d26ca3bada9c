// Instantiations and launcher of the burst kernel for MXFP4 in aiter's
// bpreshuffle formats (M <= 64): B in shuffle_weight(16,16) order, whose
// 16-row blocks are B'' (fragment order), and e8m0_shuffle scales.
#include "burst_launch.hpp"

namespace qg {

hipError_t launch_burst_mx4s(const BurstArgs& a, int mb, int nb, int waves, int batch, bool bf16, hipStream_t s) {
    return burst::launch_layout<kFmtFp4, BLay::FRAG>(a, mb, nb, waves, batch, bf16, s);
}

}  // namespace qg
