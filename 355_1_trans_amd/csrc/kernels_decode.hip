// Instantiations and launcher of the decode kernel (M <= 64, LDS-staged B).
#include "decode_gemm.hpp"
#include "launch.hpp"

namespace qg {

namespace {
template <int FMT, ScaleKind SK, BLay BL>
hipError_t launch_decode_family(const DecodeArgs& a, int mb, int nw, int batch, bool bf16, hipStream_t s) {
    const dim3 grid(a.n_tiles, a.splitk, batch);
#define QG_DECODE_CASE(MBV, NWV)                                                                  \
    if (mb == MBV && nw == NWV) {                                                                 \
        if (bf16) decode_gemm_kernel<FMT, SK, BL, MBV, NWV, true><<<grid, NWV * 64, 0, s>>>(a);   \
        else decode_gemm_kernel<FMT, SK, BL, MBV, NWV, false><<<grid, NWV * 64, 0, s>>>(a);       \
        trace_launch("decode_gemm<%s,%s,%s,mb%d,nw%d,%s,splitk%d>", FMT == kFmtFp4 ? "fp4" : "fp8",  \
                     scale_name(SK), layout_name(BL), MBV, NWV, bf16 ? "bf16" : "fp32", a.splitk);  \
        return hipGetLastError();                                                                 \
    }
    QG_DECODE_CASE(1, 4) QG_DECODE_CASE(2, 4) QG_DECODE_CASE(4, 4)
    QG_DECODE_CASE(1, 8) QG_DECODE_CASE(2, 8) QG_DECODE_CASE(4, 8)
#undef QG_DECODE_CASE
    return hipErrorInvalidValue;
}
}  // namespace

hipError_t launch_decode(SkinnyKind kind, const DecodeArgs& a, int mb, int nw, int batch, bool bf16, hipStream_t s) {
    switch (kind) {
        case SkinnyKind::MX8_RAW: return launch_decode_family<kFmtFp8, ScaleKind::MX, BLay::RAW>(a, mb, nw, batch, bf16, s);
        case SkinnyKind::MX4_RAW: return launch_decode_family<kFmtFp4, ScaleKind::MX, BLay::RAW>(a, mb, nw, batch, bf16, s);
        case SkinnyKind::BSF32_KPANEL:
            return launch_decode_family<kFmtFp8, ScaleKind::BSF32, BLay::KPANEL>(a, mb, nw, batch, bf16, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace qg
