// Instantiations and launcher of the slice decode kernel (slice_gemm.hpp).
#include "launch.hpp"
#include "slice_gemm.hpp"

namespace qg {

namespace {
template <int FMT, int MB>
hipError_t launch_mb(const RunsArgs& a, int batch, bool bf16, hipStream_t s) {
    if (a.kt_per_split != slice_kps(MB)) return hipErrorInvalidValue;
    const dim3 grid(a.n_tiles * a.splitk, batch);
    if (bf16) slice_gemm_kernel<FMT, MB, true><<<grid, kSliceWaves * 64, 0, s>>>(a);
    else slice_gemm_kernel<FMT, MB, false><<<grid, kSliceWaves * 64, 0, s>>>(a);
    trace_launch("slice_gemm<%s,MX,RAW,mb%d,nb%d,%s,splitk%d>", FMT == kFmtFp4 ? "fp4" : "fp8", MB, slice_nbw(MB),
                 bf16 ? "bf16" : "fp32", a.splitk);
    return hipGetLastError();
}
template <int FMT>
hipError_t launch_fmt(const RunsArgs& a, int mb, int batch, bool bf16, hipStream_t s) {
    if (mb == 1) return launch_mb<FMT, 1>(a, batch, bf16, s);
    if (mb == 2) return launch_mb<FMT, 2>(a, batch, bf16, s);
    if (mb == 4) return launch_mb<FMT, 4>(a, batch, bf16, s);
    return hipErrorInvalidValue;
}
// W16 B and e8m0_shuffle scales (MXFP4, aiter's formats)
template <int MB>
hipError_t launch_w16(const RunsArgs& a, int batch, bool bf16, hipStream_t s) {
    if (a.kt_per_split != slice_kps(MB)) return hipErrorInvalidValue;
    const dim3 grid(a.n_tiles * a.splitk, batch);
    if (bf16) slice_gemm_kernel<kFmtFp4, MB, true, true><<<grid, kSliceWaves * 64, 0, s>>>(a);
    else slice_gemm_kernel<kFmtFp4, MB, false, true><<<grid, kSliceWaves * 64, 0, s>>>(a);
    trace_launch("slice_gemm<fp4,MXS,W16,mb%d,nb%d,%s,splitk%d>", MB, slice_nbw(MB), bf16 ? "bf16" : "fp32",
                 a.splitk);
    return hipGetLastError();
}
}  // namespace

hipError_t launch_slice_mx4s(const RunsArgs& a, int mb, int batch, bool bf16, hipStream_t s) {
    if (a.n_tiles < 1 || a.splitk < 1 || batch < 1) return hipErrorInvalidValue;
    if (mb == 1) return launch_w16<1>(a, batch, bf16, s);
    if (mb == 2) return launch_w16<2>(a, batch, bf16, s);
    if (mb == 4) return launch_w16<4>(a, batch, bf16, s);
    return hipErrorInvalidValue;
}

hipError_t launch_slice(const RunsArgs& a, bool fp4, int mb, int batch, bool bf16, hipStream_t s) {
    if (a.n_tiles < 1 || a.splitk < 1 || batch < 1) return hipErrorInvalidValue;
    return fp4 ? launch_fmt<kFmtFp4>(a, mb, batch, bf16, s) : launch_fmt<kFmtFp8>(a, mb, batch, bf16, s);
}

}  // namespace qg
