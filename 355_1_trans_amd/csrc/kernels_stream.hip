// Instantiations and launcher of the row-streaming decode kernel (M <= 4,
// row-major MX B).
#include "stream_gemm.hpp"
#include "launch.hpp"

namespace qg {

hipError_t launch_stream(const StreamArgs& a, bool fp4, int mb, int batch, bool bf16, hipStream_t s) {
    if (a.rows_per_wg < 1 || a.rows_per_wg > kStreamMaxRows) return hipErrorInvalidValue;
    const dim3 grid((a.t.n + a.rows_per_wg - 1) / a.rows_per_wg, batch);
#define QG_STREAM_CASE(F, MBV)                                                                     \
    if (fp4 == F && mb == MBV) {                                                                   \
        if (bf16) stream_gemm_kernel<F, MBV, true><<<grid, kStreamWaves * 64, 0, s>>>(a);          \
        else stream_gemm_kernel<F, MBV, false><<<grid, kStreamWaves * 64, 0, s>>>(a);              \
        return hipGetLastError();                                                                  \
    }
    QG_STREAM_CASE(true, 1) QG_STREAM_CASE(true, 2) QG_STREAM_CASE(true, 4)
    QG_STREAM_CASE(false, 1) QG_STREAM_CASE(false, 2) QG_STREAM_CASE(false, 4)
#undef QG_STREAM_CASE
    return hipErrorInvalidValue;
}

}  // namespace qg
