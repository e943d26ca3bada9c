// Instantiations and launcher of the row-streaming decode kernel (M <= 8,
// row-major MX B; wr rows of B per MFMA, mb rows of A).
#include "stream_gemm.hpp"
#include "launch.hpp"

namespace qg {

hipError_t launch_stream(const StreamArgs& a, bool fp4, int wr, int mb, int batch, bool bf16, hipStream_t s) {
    if (a.rows_per_wg < 1 || a.rows_per_wg > stream_max_rows(wr) || a.splitk < 1 || a.seg_per_split < 1 ||
        a.seg_per_split > stream_seg_cap(fp4, wr, mb))
        return hipErrorInvalidValue;
    const dim3 grid((a.t.n + a.rows_per_wg - 1) / a.rows_per_wg, batch, a.splitk);
#define QG_STREAM_CASE(F, WRV, MBV)                                                                \
    if (fp4 == F && wr == WRV && mb == MBV) {                                                      \
        if (bf16) stream_gemm_kernel<F, WRV, MBV, true><<<grid, kStreamWaves * 64, 0, s>>>(a);     \
        else stream_gemm_kernel<F, WRV, MBV, false><<<grid, kStreamWaves * 64, 0, s>>>(a);         \
        trace_launch("stream_gemm<%s,wr%d,mb%d,%s,splitk%d>", F ? "fp4" : "fp8", WRV, MBV,          \
                     bf16 ? "bf16" : "fp32", a.splitk);                                            \
        return hipGetLastError();                                                                  \
    }
#define QG_STREAM_FMT(F) QG_STREAM_CASE(F, 1, 1) QG_STREAM_CASE(F, 2, 2) QG_STREAM_CASE(F, 4, 4) QG_STREAM_CASE(F, 4, 8)
    QG_STREAM_FMT(true)
    QG_STREAM_FMT(false)
#undef QG_STREAM_FMT
#undef QG_STREAM_CASE
    return hipErrorInvalidValue;
}

}  // namespace qg
