// Instantiations and launcher of the row-run decode kernel (runs_gemm.hpp).
#include "launch.hpp"
#include "runs_gemm.hpp"

namespace qg {

namespace {
template <int FMT, int MB, int NST>
hipError_t launch_nst(const RunsArgs& a, int batch, bool bf16, hipStream_t s) {
    const dim3 grid(a.n_tiles * a.splitk, batch);
    if (bf16) runs_gemm_kernel<FMT, MB, NST, true><<<grid, kRunsWaves * 64, 0, s>>>(a);
    else runs_gemm_kernel<FMT, MB, NST, false><<<grid, kRunsWaves * 64, 0, s>>>(a);
    trace_launch("runs_gemm<%s,MX,RAW,mb%d,st%d,%s,splitk%d>", FMT == kFmtFp4 ? "fp4" : "fp8", MB, NST,
                 bf16 ? "bf16" : "fp32", a.splitk);
    return hipGetLastError();
}
// the fewest stages (4, 8 or 16) that cover the slice
template <int FMT, int MB>
hipError_t launch_mb(const RunsArgs& a, int batch, bool bf16, hipStream_t s) {
    const int st = (a.kt_per_split + kRunsStage - 1) / kRunsStage;
    if (st <= 4) return launch_nst<FMT, MB, 4>(a, batch, bf16, s);
    if (st <= 8) return launch_nst<FMT, MB, 8>(a, batch, bf16, s);
    if (st <= 16) return launch_nst<FMT, MB, 16>(a, batch, bf16, s);
    return hipErrorInvalidValue;
}
template <int FMT>
hipError_t launch_fmt(const RunsArgs& a, int mb, int batch, bool bf16, hipStream_t s) {
    if (mb == 1) return launch_mb<FMT, 1>(a, batch, bf16, s);
    if (mb == 2) return launch_mb<FMT, 2>(a, batch, bf16, s);
    if (mb == 4) return launch_mb<FMT, 4>(a, batch, bf16, s);
    return hipErrorInvalidValue;
}
}  // namespace

hipError_t launch_runs(const RunsArgs& a, bool fp4, int mb, int batch, bool bf16, hipStream_t s) {
    if (a.n_tiles < 1 || a.splitk < 1 || a.kt_per_split < 1 || batch < 1) return hipErrorInvalidValue;
    return fp4 ? launch_fmt<kFmtFp4>(a, mb, batch, bf16, s) : launch_fmt<kFmtFp8>(a, mb, batch, bf16, s);
}

}  // namespace qg
