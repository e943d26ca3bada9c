// Host-side launch wrappers shared between the kernel translation units and
// the C ABI layer (abi.cpp).  Each wrapper launches exactly one kernel.
#pragma once
#include <hip/hip_runtime.h>
#include "tile_gemm.hpp"

namespace qg {

// kernels_tile.hip
// wide_panels: MX scale rows are 16-byte aligned and K % 512 == 0, so the
// kernel may move 16-byte scale panels (4 fp8 / 2 fp4 K-tiles per DMA).
hipError_t launch_tile_mx8_raw(const TileArgs& a, int batch, bool bf16, bool wide_panels, hipStream_t s);
hipError_t launch_tile_mx4_raw(const TileArgs& a, int batch, bool bf16, bool wide_panels, hipStream_t s);
hipError_t launch_tile_bs8_w16(const TileArgs& a, int batch, bool bf16, hipStream_t s);
hipError_t launch_tile_bsf32_kpanel(const TileArgs& a, int batch, bool bf16, hipStream_t s);

// probe.hip
hipError_t launch_probe(int32_t* dev_out, hipStream_t s);
constexpr int kProbeWords = 2096;

}  // namespace qg
