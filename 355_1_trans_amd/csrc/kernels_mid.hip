// Instantiations and launcher of the four-wave 128 x 128 kernel: fp8 with fp32
// block scales (K-panel B' or fragment-order B''), MXFP8 and MXFP4 (row-major B).
#include <climits>

#include "launch.hpp"
#include "mid_gemm.hpp"

namespace qg {

template <BLay BL, int ST, ScaleKind SK, int FMT, bool NTB = false>
static void mid_go(const MidArgs& a, const dim3& grid, bool bf16, hipStream_t s) {
    if (bf16) mid_gemm_kernel<true, BL, ST, SK, FMT, NTB><<<grid, 256, 0, s>>>(a);
    else mid_gemm_kernel<false, BL, ST, SK, FMT, NTB><<<grid, 256, 0, s>>>(a);
    trace_launch("mid_gemm<%s,%s,%s,%s,st%d%s,splitk%d>", FMT == kFmtFp4 ? "fp4" : "fp8", scale_name(SK),
                 layout_name(BL), bf16 ? "bf16" : "fp32", ST, NTB ? ",ntb" : "", (int)grid.y);
}

// MX with one M tile reads B once: nontemporal B loads (N = 7168,
// K = 16384, MXFP4 M = 128 37.9 -> 37.6 us, MXFP8 61.4 -> 60.9 us, M = 96
// alike); with several M tiles the other tiles re-read B from L2, which
// nontemporal loads evict (up to 50% slower)
template <int ST, int FMT>
static void mid_mx(const MidArgs& a, const dim3& grid, bool bf16, hipStream_t s) {
    if (a.t.tiles_m == 1) mid_go<BLay::RAW, ST, ScaleKind::MX, FMT, true>(a, grid, bf16, s);
    else mid_go<BLay::RAW, ST, ScaleKind::MX, FMT>(a, grid, bf16, s);
}

template <int ST>
static void mid_kind(const MidArgs& a, const dim3& grid, bool bf16, MidKind kind, hipStream_t s) {
    switch (kind) {
    case MidKind::BS_KPANEL: mid_go<BLay::KPANEL, ST, ScaleKind::BSF32, kFmtFp8>(a, grid, bf16, s); break;
    case MidKind::BS_FRAG: mid_go<BLay::FRAG, ST, ScaleKind::BSF32, kFmtFp8>(a, grid, bf16, s); break;
    case MidKind::MX8: mid_mx<ST, kFmtFp8>(a, grid, bf16, s); break;
    case MidKind::MX4: mid_mx<ST, kFmtFp4>(a, grid, bf16, s); break;
    }
}

// The slice sum after a split-K launch: one thread per 4 elements (N % 4
// == 0) or per element, over batch x M x N.
hipError_t launch_splitk_reduce(const SplitReduceArgs& r, bool bf16, hipStream_t s) {
    const bool vec = r.n % 4 == 0;
    const long long total = (long long)r.m * r.n * r.batch;
    const long long blocks = ((vec ? total / 4 : total) + 255) / 256;
    if (blocks <= 0 || blocks > INT_MAX) return hipErrorInvalidValue;
    const dim3 grid((unsigned)blocks);
    if (bf16) {
        if (vec) splitk_reduce_kernel<true, true><<<grid, 256, 0, s>>>(r);
        else splitk_reduce_kernel<true, false><<<grid, 256, 0, s>>>(r);
    } else {
        if (vec) splitk_reduce_kernel<false, true><<<grid, 256, 0, s>>>(r);
        else splitk_reduce_kernel<false, false><<<grid, 256, 0, s>>>(r);
    }
    trace_launch("splitk_reduce<%s,%s,splitk%d>", bf16 ? "bf16" : "fp32", vec ? "x4" : "x1", r.splitk);
    return hipGetLastError();
}

hipError_t launch_mid(const MidArgs& a, int batch, bool bf16, MidKind kind, int stages, hipStream_t s) {
    const dim3 grid(a.t.tiles_m * a.t.tiles_n, a.splitk, batch);
    if (stages == 2) mid_kind<2>(a, grid, bf16, kind, s);
    else if (stages == 4) mid_kind<4>(a, grid, bf16, kind, s);
    else return hipErrorInvalidValue;
    const hipError_t st = hipGetLastError();
    if (st != hipSuccess || a.splitk == 1) return st;
    SplitReduceArgs r{};
    r.ws = a.ws;
    r.c = a.t.c;
    r.m = a.t.m;
    r.n = a.t.n;
    r.ldc = a.t.ldc;
    r.c_vec = a.t.c_vec;
    r.splitk = a.splitk;
    r.batch = batch;
    r.c_batch = a.t.c_batch;
    return launch_splitk_reduce(r, bf16, s);
}

}  // namespace qg
