// Whole-output GPU reference GEMM: every output element of a full-size
// launch checked against an independent computation, the way the reference
// checks its 8192^3 kernels against gemm_ref_gpu (MX4
// gemm_a4w4_mxfp4_4wave_host.cc:66-94, 219-257).  It shares nothing with the
// product kernels: no MFMA, no layouts beyond row-major, no split.
//
// Each operand element is decoded from its code (e4m3: bias 7, subnormals
// m * 2^-9, 0x7F / 0xFF NaN; e2m1: {0, .5, 1, 1.5, 2, 3, 4, 6}, sign in bit
// 3, even k in the low nibble) and multiplied by its block scale in fp64
// (exact: a 4-bit code times a power of two or an fp32 scale fits 53 bits);
// the products are summed in fp64 in K order and rounded once to fp32.
// Scales: MX E8M0 per (row, 32 K); fp32 block scales per (row, 128 K) of A
// and (128 rows, 128 K) of B; E8M0 block scales likewise.
//
// Tiling: a workgroup of 256 threads owns 64 x 64 outputs, each thread
// 4 x 4; K moves in chunks of 32 through LDS as decoded fp64 values.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "launch.hpp"

namespace qg {

namespace {

__device__ __forceinline__ double e4m3_value(uint32_t c) {
    const uint32_t e = (c >> 3) & 15u, m = c & 7u;
    if ((c & 0x7Fu) == 0x7Fu) return __builtin_nan("");
    const double mag = e ? __builtin_ldexp(1.0 + m / 8.0, (int)e - 7) : __builtin_ldexp((double)m, -9);
    return (c & 0x80u) ? -mag : mag;
}

__device__ __forceinline__ double e2m1_value(uint32_t c) {
    const uint32_t e = (c >> 1) & 3u, m = c & 1u;    // exponent bias 1; e = 0: subnormal m * 0.5
    const double mag = e ? __builtin_ldexp(1.0 + 0.5 * m, (int)e - 1) : 0.5 * m;
    return (c & 8u) ? -mag : mag;
}

__device__ __forceinline__ double e8m0_value(uint32_t e) { return __builtin_ldexp(1.0, (int)e - 127); }

constexpr int kRefTile = 64, kRefChunk = 32, kRefThreads = 256;

// Decoded, scaled value of operand X (A: is_b false) at (row, k).
template <RefFam F>
__device__ __forceinline__ double ref_value(const RefArgs& p, bool is_b, int row, int k) {
    const uint8_t* x = is_b ? p.b : p.a;
    const long long ld = is_b ? p.ldb : p.lda;
    double v;
    if constexpr (F == RefFam::MX4) {
        const uint32_t byte = x[(long long)row * ld + k / 2];
        v = e2m1_value((k & 1) ? byte >> 4 : byte & 15u);
    } else {
        v = e4m3_value(x[(long long)row * ld + k]);
    }
    double s;
    if constexpr (F == RefFam::MX8 || F == RefFam::MX4) {
        const uint8_t* sc = is_b ? p.sfb : p.sfa;
        s = e8m0_value(sc[(long long)row * (is_b ? p.sfb_sm : p.sfa_sm) + k / 32]);
    } else {
        const int kg = k / 128;
        const long long ia = (long long)row * p.sfa_sm + (long long)kg * p.sfa_sk;
        const long long ib = (long long)(row / 128) * p.sfb_sm + kg;
        if constexpr (F == RefFam::BSF32)
            s = is_b ? ((const float*)p.sfb)[ib] : ((const float*)p.sfa)[ia];
        else
            s = e8m0_value(is_b ? p.sfb[ib] : p.sfa[ia]);
    }
    return v * s;
}

template <RefFam F>
__global__ __launch_bounds__(kRefThreads) void ref_gemm_kernel(const RefArgs p) {
    __shared__ double as[kRefChunk][kRefTile + 1];
    __shared__ double bs[kRefChunk][kRefTile + 1];
    const int tid = threadIdx.x, tx = tid % 16, ty = tid / 16;
    const int m0 = blockIdx.y * kRefTile, n0 = blockIdx.x * kRefTile;
    double acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = 0.0;
    for (int k0 = 0; k0 < p.k; k0 += kRefChunk) {
        // thread t decodes elements t, t + 256, ...: row e / 32, k e % 32
#pragma unroll
        for (int i = 0; i < kRefTile * kRefChunk / kRefThreads; ++i) {
            const int e = tid + kRefThreads * i, r = e / kRefChunk, kk = e % kRefChunk;
            as[kk][r] = m0 + r < p.m ? ref_value<F>(p, false, m0 + r, k0 + kk) : 0.0;
            bs[kk][r] = n0 + r < p.n ? ref_value<F>(p, true, n0 + r, k0 + kk) : 0.0;
        }
        __syncthreads();
        for (int kk = 0; kk < kRefChunk; ++kk) {
            double a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = as[kk][ty * 4 + i];
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = bs[kk][tx * 4 + j];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fma(a[i], b[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = m0 + ty * 4 + i;
        if (m >= p.m) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int n = n0 + tx * 4 + j;
            if (n < p.n) p.c[(long long)m * p.ldc + n] = (float)acc[i][j];
        }
    }
}

}  // namespace

hipError_t launch_ref_gemm(const RefArgs& a, RefFam fam, hipStream_t s) {
    const dim3 grid((a.n + kRefTile - 1) / kRefTile, (a.m + kRefTile - 1) / kRefTile);
    switch (fam) {
        case RefFam::BSF32: ref_gemm_kernel<RefFam::BSF32><<<grid, kRefThreads, 0, s>>>(a); break;
        case RefFam::BS8: ref_gemm_kernel<RefFam::BS8><<<grid, kRefThreads, 0, s>>>(a); break;
        case RefFam::MX8: ref_gemm_kernel<RefFam::MX8><<<grid, kRefThreads, 0, s>>>(a); break;
        case RefFam::MX4: ref_gemm_kernel<RefFam::MX4><<<grid, kRefThreads, 0, s>>>(a); break;
        default: return hipErrorInvalidValue;
    }
    trace_launch("ref_gemm<%s>", fam == RefFam::BSF32 ? "BSF32" : fam == RefFam::BS8 ? "BS8" : fam == RefFam::MX8 ? "MX8" : "MX4");
    return hipGetLastError();
}

}  // namespace qg
