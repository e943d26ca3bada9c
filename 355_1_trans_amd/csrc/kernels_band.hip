// Instantiations and launcher of the band kernel (band_gemm.hpp): MX decode
// shapes with row-major B, A's K slice in LDS.
#include "band_gemm.hpp"
#include "launch.hpp"

namespace qg {

namespace {
template <int FMT>
hipError_t launch_band_fmt(const BandArgs& a, int mb, int cb, int batch, bool bf16, hipStream_t s) {
    const dim3 grid(a.bands, a.splitk, batch);
#define QG_BAND_CASE(MBV, CBV)                                                                           \
    if (mb == MBV && cb == CBV) {                                                                        \
        if (bf16) band_gemm_kernel<FMT, MBV, CBV, true><<<grid, kBandWaves * 64, 0, s>>>(a);             \
        else band_gemm_kernel<FMT, MBV, CBV, false><<<grid, kBandWaves * 64, 0, s>>>(a);                 \
        trace_launch("band_gemm<%s,mb%d,cb%d,d%d,%s,splitk%d>", FMT == kFmtFp4 ? "fp4" : "fp8", MBV, CBV,  \
                     band_depth(MBV, CBV, FMT == kFmtFp4), bf16 ? "bf16" : "fp32", a.splitk);             \
        return hipGetLastError();                                                                        \
    }
    QG_BAND_CASE(1, 1) QG_BAND_CASE(1, 2) QG_BAND_CASE(2, 1) QG_BAND_CASE(4, 1) QG_BAND_CASE(4, 2)
#undef QG_BAND_CASE
    return hipErrorInvalidValue;
}
}  // namespace

hipError_t launch_band(const BandArgs& a, bool fp4, int mb, int cb, int batch, bool bf16, hipStream_t s) {
    return fp4 ? launch_band_fmt<kFmtFp4>(a, mb, cb, batch, bf16, s)
               : launch_band_fmt<kFmtFp8>(a, mb, cb, batch, bf16, s);
}

}  // namespace qg
