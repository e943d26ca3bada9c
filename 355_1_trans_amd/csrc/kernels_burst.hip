// Instantiations and launchers of the burst kernel for fp8 with fp32 block
// scales (M <= 64, K-panel B' or fragment-order B''); the grouped kernel's
// are in kernels_burst_grouped.hip.
#include "burst_launch.hpp"

namespace qg {

hipError_t launch_burst(const BurstArgs& a, bool frag, int mb, int nb, int waves, int batch, bool bf16,
                        hipStream_t s) {
    return frag ? burst::launch_layout<kFmtFp8, BLay::FRAG>(a, mb, nb, waves, batch, bf16, s)
                : burst::launch_layout<kFmtFp8, BLay::KPANEL>(a, mb, nb, waves, batch, bf16, s);
}

}  // namespace qg
