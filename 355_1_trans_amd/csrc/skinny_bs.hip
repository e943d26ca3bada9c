// Block-scale (fp32 scales) instantiations of the skinny-M / split-K kernel
// for the K-panel B' and fragment-order B'' layouts, the B' -> B'' repack,
// and the family dispatcher.
#include "launch.hpp"
#include "skinny_gemm.hpp"

#include <algorithm>

namespace qg {

hipError_t launch_skinny(SkinnyKind kind, const SkinnyArgs& a, int mb, int nb, int batch, bool bf16, hipStream_t s) {
    switch (kind) {
        case SkinnyKind::MX8_RAW: return launch_skinny_mx8(a, mb, nb, batch, bf16, s);
        case SkinnyKind::MX4_RAW: return launch_skinny_mx4(a, mb, nb, batch, bf16, s);
        case SkinnyKind::BSF32_KPANEL:
            return launch_skinny_family<kFmtFp8, ScaleKind::BSF32, BLay::KPANEL>(a, mb, nb, batch, bf16, s);
        case SkinnyKind::BSF32_FRAG:
            return launch_skinny_family<kFmtFp8, ScaleKind::BSF32, kBFrag>(a, mb, nb, batch, bf16, s);
    }
    return hipErrorInvalidValue;
}

namespace {
// B' (K-panel [K/128][N][128]) -> B'' (fragment order, see skinny_gemm.hpp):
// one thread per 16-byte unit of B''; rows past N are zero.
__global__ __launch_bounds__(256) void repack_frag_kernel(const uint8_t* __restrict__ bk, uint8_t* __restrict__ bpp,
                                                          int n, int nk, long long bk_batch, long long bpp_batch) {
    const long long units = (long long)((n + 15) / 16) * nk * 128;
    const uint8_t* src_b = bk + blockIdx.y * bk_batch;
    uint8_t* dst_b = bpp + blockIdx.y * bpp_batch;
    for (long long u = blockIdx.x * 256ll + threadIdx.x; u < units; u += (long long)gridDim.x * 256) {
        const int L = (int)(u & 63), h = (int)((u >> 6) & 1);
        const long long blk = u >> 7;                 // nb * nk + kt
        const int kt = (int)(blk % nk), nb = (int)(blk / nk);
        const int row = nb * 16 + (L & 15), q = L >> 4;
        const int c = h ? q + 4 : q;
        i32x4 v = {0, 0, 0, 0};
        if (row < n) v = *(const i32x4*)(src_b + ((long long)kt * n + row) * 128 + c * 16);
        *(i32x4*)(dst_b + u * 16) = v;
    }
}
}  // namespace

hipError_t launch_repack_frag(const uint8_t* bk, uint8_t* bpp, int n, int k, int batch, long long bk_batch,
                              long long bpp_batch, hipStream_t s) {
    const long long units = (long long)((n + 15) / 16) * (k / 128) * 128;
    const int blocks = (int)std::min<long long>((units + 255) / 256, 4096);
    repack_frag_kernel<<<dim3(blocks, batch), 256, 0, s>>>(bk, bpp, n, k / 128, bk_batch, bpp_batch);
    trace_launch("repack_frag");
    return hipGetLastError();
}

}  // namespace qg
