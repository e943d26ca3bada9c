// Device-side quantizers and weight-layout transforms: the steps before the
// GEMM, on the GPU.
//
//   * fp32 / bf16 -> e4m3 with fp32 block scales amax / 448, per 1x128
//     activation block or 128x128 weight block (the block-scale recipe the
//     reference's fp32-scale kernels consume, BPS host.cc:66-90);
//   * the same with E8M0 block scales 2^ceil(log2(amax / 448)) (the SNAP
//     kernel's input, SNAP blockscale_bpreshuffle.py:3-4);
//   * MXFP8 (e4m3) and MXFP4 (e2m1, two per byte, even k in the low nibble)
//     with one E8M0 scale 2^ceil(log2(amax / qmax)) per 32 K elements, the
//     scales written row-major [rows][K/32] or in aiter's e8m0_shuffle order
//     (quant(..., shuffle=True), MX4 candidate_m9/README.md:6-12);
//   * the weight layouts: K-panel B' (BPS host.cc:92-111),
//     shuffle_weight(16,16) (SNAP host.cc:161-179, MX4 candidate_m10
//     host.cc:215-225), this library's B'' and e8m0_shuffle (MX4
//     candidate_m10 host.cc:194-206).
//
// All of it is HBM-bound byte work: one pass over the input with 16-byte
// loads, coalesced stores, no LDS round trips beyond the 128x128 weight
// block's amax.  The value codecs below are written from the format
// definitions (OCP E4M3 / E2M1, round to nearest even, saturating) so that
// the codes are bit-identical to the host quantizers the tests compare with.
#include <hip/hip_runtime.h>

#include "common.hpp"
#include "launch.hpp"

namespace qg {

namespace {

// ---------------------------------------------------------------- codecs
// OCP E4M3FN, round to nearest even, saturating at 448 (0x7E); NaN -> 0x7F.
__device__ __forceinline__ uint32_t f32_to_e4m3(float x) {
    const uint32_t b = __float_as_uint(x);
    const uint32_t sign = (b >> 24) & 0x80u;
    const uint32_t a = b & 0x7fffffffu;
    if (a > 0x7f800000u) return sign | 0x7fu;             // NaN
    if (a >= 0x43e00000u) return sign | 0x7eu;            // |x| >= 448: saturate
    if (a < 0x3c800000u)                                  // |x| < 2^-6: subnormals, step 2^-9
        return sign | (uint32_t)__builtin_rintf(__uint_as_float(a) * 512.0f);   // 0..8 (8 = 2^-6)
    const uint32_t e = (a >> 23) - 120u;                  // biased e4m3 exponent 1..15
    uint32_t m = (a >> 20) & 7u;
    const uint32_t rem = a & 0xfffffu;
    if (rem > 0x80000u || (rem == 0x80000u && (m & 1u))) ++m;
    const uint32_t code = (e << 3) + m;                   // m == 8 carries into the exponent
    return sign | (code > 0x7eu ? 0x7eu : code);
}

// E2M1 {0, .5, 1, 1.5, 2, 3, 4, 6}, sign in bit 3, round to nearest even,
// saturating at 6; NaN -> 6 with its sign.
__device__ __forceinline__ uint32_t f32_to_e2m1(float x) {
    const uint32_t b = __float_as_uint(x);
    const uint32_t sign = (b >> 28) & 8u;
    const uint32_t a = b & 0x7fffffffu;
    if (a > 0x7f800000u) return sign | 7u;
    if (a < 0x3f800000u)                                  // |x| < 1: step 0.5
        return sign | (uint32_t)__builtin_rintf(__uint_as_float(a) * 2.0f);      // 0, 1, 2 (2 = 1.0)
    const int E = (int)(a >> 23) - 127;
    if (E > 2) return sign | 7u;
    uint32_t m = (a >> 22) & 1u;
    const uint32_t rem = a & 0x3fffffu;
    if (rem > 0x200000u || (rem == 0x200000u && (m & 1u))) ++m;
    const uint32_t code = ((uint32_t)(E + 1) << 1) + m;   // m == 2 carries
    return sign | (code > 7u ? 7u : code);
}

// ceil(log2(v)) of a positive float, subnormals included.
__device__ __forceinline__ int ceil_log2(float v) {
    const uint32_t b = __float_as_uint(v);
    const int e = (int)(b >> 23);
    const uint32_t m = b & 0x7fffffu;
    if (e == 0) return (31 - __clz((int)m)) - 149 + ((m & (m - 1u)) != 0u);
    return e - 127 + (m != 0u);
}

// Power-of-two scale exponent: the smallest E with amax / 2^E <= qmax,
// clamped to the E8M0 range; 0 (code 127) for an all-zero group.
__device__ __forceinline__ int mx_exp(float amax, float qmax) {
    if (!(amax > 0.0f)) return 0;
    const float v = amax / qmax;                          // IEEE division
    if (v == 0.0f) return -127;                           // the quotient underflows: the clamp
    const int e = ceil_log2(v);
    return e < -127 ? -127 : (e > 127 ? 127 : e);
}

// Four consecutive input elements as fp32 (bf16 widens exactly).
template <bool BF16IN>
__device__ __forceinline__ f32x4 load4(const void* base, long long elem) {
    if constexpr (BF16IN) {
        const uint2 v = *(const uint2*)((const uint16_t*)base + elem);
        return f32x4{__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u), __uint_as_float(v.y << 16),
                     __uint_as_float(v.y & 0xffff0000u)};
    } else {
        return *(const f32x4*)((const float*)base + elem);
    }
}

__device__ __forceinline__ float amax4(f32x4 v) {
    return fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
}

// max over `width` consecutive lanes (width a power of two <= 64)
template <int WIDTH>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
    for (int d = 1; d < WIDTH; d <<= 1) v = fmaxf(v, __shfl_xor(v, d, 64));
    return v;
}

// byte offset of (row, group) in aiter's e8m0_shuffle order (rows padded to
// 32, groups to 8; MX4 candidate_m10 host.cc:194-206)
__device__ __forceinline__ long long shuffled_scale_offset(int r, int g, int kg8) {
    return ((long long)(r >> 5) * (kg8 >> 3) + (g >> 3)) * 256 + (g & 3) * 64 + (r & 15) * 4 + ((g & 7) >> 2) * 2 +
           ((r & 31) >> 4);
}

struct QuantArgs {
    const void* x;
    uint8_t* q;
    void* s;                 // scales: fp32 or E8M0 bytes
    long long ldx, ldq;      // elements / bytes
    long long s_sm, s_sk;    // scale element strides along rows and K blocks (row-major / column-major)
    int rows, k;
    int kg8;                 // e8m0_shuffle: K/32 rounded up to 8
};

// Row-wise group quantizer: one thread per 4 consecutive elements, GROUP
// elements per scale (32 for MX, 128 for the 1x128 activation blocks).
//   FMT  0: e4m3 with fp32 scale amax / 448 (x / scale, IEEE division)
//        1: e4m3 with E8M0 scale 2^ceil(log2(amax / 448))
//        2: e2m1 with E8M0 scale 2^ceil(log2(amax / 6))
// SHUF: E8M0 scales in e8m0_shuffle order instead of (s_sm, s_sk) strides.
template <int FMT, int GROUP, bool BF16IN, bool SHUF>
__global__ __launch_bounds__(256) void quant_rows_kernel(const QuantArgs p) {
    constexpr int TPG = GROUP / 4;    // threads per group
    const long long per_row = p.k / 4;
    const long long units = (long long)p.rows * per_row;
    for (long long u = (long long)blockIdx.x * 256 + threadIdx.x; u < units; u += (long long)gridDim.x * 256) {
        const int r = (int)(u / per_row);
        const int c4 = (int)(u - (long long)r * per_row);
        const f32x4 v = load4<BF16IN>(p.x, (long long)r * p.ldx + 4 * c4);
        const float amax = group_max<TPG>(amax4(v));
        const int g = (4 * c4) / GROUP;
        const bool lead = (c4 % TPG) == 0;
        if constexpr (FMT == 0) {
            const float sc = amax > 0.0f ? amax / 448.0f : 1.0f;
            const uint32_t w = f32_to_e4m3(v[0] / sc) | (f32_to_e4m3(v[1] / sc) << 8) |
                               (f32_to_e4m3(v[2] / sc) << 16) | (f32_to_e4m3(v[3] / sc) << 24);
            *(uint32_t*)(p.q + (long long)r * p.ldq + 4 * c4) = w;
            if (lead) ((float*)p.s)[r * p.s_sm + g * p.s_sk] = sc;
        } else {
            const int E = mx_exp(amax, FMT == 2 ? 6.0f : 448.0f);
            if constexpr (FMT == 1) {
                const uint32_t w = f32_to_e4m3(__builtin_ldexpf(v[0], -E)) |
                                   (f32_to_e4m3(__builtin_ldexpf(v[1], -E)) << 8) |
                                   (f32_to_e4m3(__builtin_ldexpf(v[2], -E)) << 16) |
                                   (f32_to_e4m3(__builtin_ldexpf(v[3], -E)) << 24);
                *(uint32_t*)(p.q + (long long)r * p.ldq + 4 * c4) = w;
            } else {
                const uint32_t lo = f32_to_e2m1(__builtin_ldexpf(v[0], -E)) | (f32_to_e2m1(__builtin_ldexpf(v[1], -E)) << 4);
                const uint32_t hi = f32_to_e2m1(__builtin_ldexpf(v[2], -E)) | (f32_to_e2m1(__builtin_ldexpf(v[3], -E)) << 4);
                *(uint16_t*)(p.q + (long long)r * p.ldq + 2 * c4) = (uint16_t)(lo | (hi << 8));
            }
            if (lead) {
                uint8_t* e = (uint8_t*)p.s;
                const long long off = SHUF ? shuffled_scale_offset(r, g, p.kg8) : r * p.s_sm + g * p.s_sk;
                e[off] = (uint8_t)(E + 127);
            }
        }
    }
}

// 128 x 128 weight-block quantizer: one workgroup (4 waves) per block;
// thread t holds columns 4(t % 32) .. +3 of rows t/32 + 8i (i < 16) -- each
// load instruction covers two whole 512-byte rows -- then the block's amax
// meets in LDS.  Rows past N belong to no block element (masked).
//   FMT 0: fp32 scale amax / 448; 1: E8M0 2^ceil(log2(amax / 448)).
template <int FMT, bool BF16IN>
__global__ __launch_bounds__(256) void quant_wgt_block_kernel(const QuantArgs p) {
    __shared__ float wmax[4];
    const int g = blockIdx.x, nb = blockIdx.y, t = threadIdx.x;
    const int c4 = t & 31, r0 = t >> 5;
    const int rows = min(128, p.rows - nb * 128);
    f32x4 v[16];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int r = r0 + 8 * i;
        v[i] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (r < rows) v[i] = load4<BF16IN>(p.x, (long long)(nb * 128 + r) * p.ldx + g * 128 + 4 * c4);
        amax = fmaxf(amax, amax4(v[i]));
    }
    amax = group_max<64>(amax);
    if ((t & 63) == 0) wmax[t >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    if constexpr (FMT == 0) {
        const float sc = amax > 0.0f ? amax / 448.0f : 1.0f;
        if (t == 0) ((float*)p.s)[nb * p.s_sm + g] = sc;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int r = r0 + 8 * i;
            if (r < rows)
                *(uint32_t*)(p.q + (long long)(nb * 128 + r) * p.ldq + g * 128 + 4 * c4) =
                    f32_to_e4m3(v[i][0] / sc) | (f32_to_e4m3(v[i][1] / sc) << 8) |
                    (f32_to_e4m3(v[i][2] / sc) << 16) | (f32_to_e4m3(v[i][3] / sc) << 24);
        }
    } else {
        const int E = mx_exp(amax, 448.0f);
        if (t == 0) ((uint8_t*)p.s)[nb * p.s_sm + g] = (uint8_t)(E + 127);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int r = r0 + 8 * i;
            if (r < rows)
                *(uint32_t*)(p.q + (long long)(nb * 128 + r) * p.ldq + g * 128 + 4 * c4) =
                    f32_to_e4m3(__builtin_ldexpf(v[i][0], -E)) | (f32_to_e4m3(__builtin_ldexpf(v[i][1], -E)) << 8) |
                    (f32_to_e4m3(__builtin_ldexpf(v[i][2], -E)) << 16) |
                    (f32_to_e4m3(__builtin_ldexpf(v[i][3], -E)) << 24);
        }
    }
}

// bytes := 0x7F (E8M0 1.0), the padding value of e8m0_shuffle
__global__ __launch_bounds__(256) void fill_7f_kernel(uint8_t* dst, long long bytes) {
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < bytes; i += (long long)gridDim.x * 256)
        dst[i] = 0x7f;
}

// ---------------------------------------------------------------- layouts
// Every layout kernel walks its DESTINATION in order, one 16-byte unit per
// thread (coalesced stores), and gathers the source unit.
enum class Lay : int { KPANEL = 0, W16 = 1, FRAG = 2 };

template <Lay L>
__global__ __launch_bounds__(256) void relayout_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                       int n, int kbytes, long long ld) {
    const long long units = (L == Lay::FRAG ? (long long)((n + 15) / 16) * 16 : (long long)n) * (kbytes / 16);
    for (long long u = (long long)blockIdx.x * 256 + threadIdx.x; u < units; u += (long long)gridDim.x * 256) {
        long long so;
        bool zero = false;
        if constexpr (L == Lay::KPANEL) {            // dst [kt][n][8 chunks]
            const long long kt = u / ((long long)n * 8), rem = u - kt * n * 8;
            so = (rem >> 3) * ld + kt * 128 + (rem & 7) * 16;
        } else if constexpr (L == Lay::W16) {        // dst [n/16][kbytes/16][16 rows][16]
            const long long per_blk = (long long)(kbytes / 16) * 16;
            const long long nb = u / per_blk, rem = u - nb * per_blk;
            so = (nb * 16 + (rem & 15)) * ld + (rem >> 4) * 16;
        } else {                                     // dst [n/16][kbytes/128][h][lane][16]
            const int nkt = kbytes / 128;
            const int lane = (int)(u & 63), h = (int)((u >> 6) & 1);
            const long long blk = u >> 7, nb = blk / nkt, kt = blk - nb * nkt;
            const long long row = nb * 16 + (lane & 15);
            zero = row >= n;
            so = row * ld + kt * 128 + ((lane >> 4) + 4 * h) * 16;
        }
        i32x4 v = {0, 0, 0, 0};
        if (!zero) v = *(const i32x4*)(src + so);
        *(i32x4*)(dst + u * 16) = v;
    }
}

// e8m0_shuffle: one thread per destination byte; padding bytes are 0x7F.
__global__ __launch_bounds__(256) void e8m0_shuffle_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                           int rows, int kg, long long ld, int kg8, long long bytes) {
    for (long long o = (long long)blockIdx.x * 256 + threadIdx.x; o < bytes; o += (long long)gridDim.x * 256) {
        const long long blk = o >> 8;
        const int w = (int)(o & 255);
        const long long rb = blk / (kg8 >> 3), gb = blk - rb * (kg8 >> 3);
        const long long r = rb * 32 + (w & 1) * 16 + ((w & 63) >> 2);
        const long long g = gb * 8 + ((w & 3) >> 1) * 4 + (w >> 6);
        dst[o] = (r < rows && g < kg) ? src[r * ld + g] : (uint8_t)0x7f;
    }
}

// e8m0_shuffle of one or two operands (all batch entries) in one launch: a
// workgroup turns one 32-row block x 16 K-tiles (128 groups) of row-major
// E8M0 into 16 contiguous 256-byte shuffled blocks.  Each row's 128-byte run
// is read with dword loads (8 threads per row) into LDS, and every thread
// then gathers and writes 16 contiguous destination bytes.  Rows past
// `rows` and groups past kg read as 0x7F.  Source rows and pitches are
// dword aligned, destinations 16-byte aligned.
__global__ __launch_bounds__(256) void e8m0_shuffle_blocks_kernel(const ShuffleArgs a) {
    __shared__ uint8_t run[32][132];    // 33 dwords per row: the gathers spread over the banks
    int u = blockIdx.x, op = 0;
    if (u >= a.units[0]) {
        u -= a.units[0];
        op = 1;
    }
    const int kg = a.kg, kt8 = (kg + 7) / 8, chunks = (kt8 + 15) / 16;
    const int rb = u / chunks, ch = u - rb * chunks;
    const int rows = a.rows[op];
    const uint8_t* src = a.src[op] + (long long)blockIdx.y * a.src_batch[op];
    uint8_t* dst = a.dst[op] + (long long)blockIdx.y * a.dst_batch[op];
    const int t = threadIdx.x, rl = t >> 3, seg = t & 7, row = rb * 32 + rl;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const int g = ch * 128 + seg * 16 + 4 * d;
        uint32_t v = 0x7F7F7F7Fu;
        if (row < rows) {
            const uint8_t* q = src + (long long)row * a.ld[op] + g;
            if (g + 3 < kg) {
                v = *(const uint32_t*)q;
            } else {
                v = 0;
                for (int e = 0; e < 4; ++e) v |= (uint32_t)(g + e < kg ? q[e] : 0x7Fu) << (8 * e);
            }
        }
        *(uint32_t*)&run[rl][seg * 16 + 4 * d] = v;
    }
    __syncthreads();
    const int j = t >> 4, kt = ch * 16 + j, w0 = (t & 15) * 16;
    if (kt >= kt8) return;
    uint32_t o[4] = {0, 0, 0, 0};
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const int w = w0 + e;
        const int r = (w & 1) * 16 + ((w & 63) >> 2), g = j * 8 + ((w & 3) >> 1) * 4 + (w >> 6);
        o[e >> 2] |= (uint32_t)run[r][g] << (8 * (e & 3));
    }
    *(i32x4*)(dst + (long long)rb * 32 * (kt8 * 8) + (long long)kt * 256 + w0) =
        i32x4{(int)o[0], (int)o[1], (int)o[2], (int)o[3]};
}

unsigned grid_for(long long units) {
    const long long b = (units + 255) / 256;
    return (unsigned)(b < 8192 ? (b > 0 ? b : 1) : 8192);
}

}  // namespace

// ---------------------------------------------------------------- launchers
hipError_t launch_quant_rows(int fmt, int group, bool bf16in, bool shuffle, const void* x, long long ldx,
                             uint8_t* q, long long ldq, void* s, long long s_sm, long long s_sk, int rows, int k,
                             hipStream_t st) {
    QuantArgs p{};
    p.x = x;
    p.q = q;
    p.s = s;
    p.ldx = ldx;
    p.ldq = ldq;
    p.s_sm = s_sm;
    p.s_sk = s_sk;
    p.rows = rows;
    p.k = k;
    p.kg8 = (k / 32 + 7) / 8 * 8;
    const unsigned grid = grid_for((long long)rows * (k / 4));
    if (shuffle) {
        const long long bytes = (long long)(rows + 31) / 32 * 32 * p.kg8;
        if (rows % 32 || (k / 32) % 8) {
            fill_7f_kernel<<<grid_for(bytes), 256, 0, st>>>((uint8_t*)s, bytes);
            trace_launch("fill_7f");
        }
    }
#define QG_QUANT(F, G, B, S)                                                                            \
    if (fmt == F && group == G && bf16in == B && shuffle == S) {                                        \
        quant_rows_kernel<F, G, B, S><<<grid, 256, 0, st>>>(p);                                         \
        trace_launch("quant_rows<%s,g%d,%s%s>", F == 0 ? "e4m3,fp32" : F == 1 ? "e4m3,e8m0" : "e2m1,e8m0", G, \
                     B ? "bf16" : "fp32", S ? ",shuffled" : "");                                        \
        return hipGetLastError();                                                                       \
    }
    QG_QUANT(0, 128, false, false) QG_QUANT(0, 128, true, false)
    QG_QUANT(1, 128, false, false) QG_QUANT(1, 128, true, false)
    QG_QUANT(1, 32, false, false) QG_QUANT(1, 32, true, false) QG_QUANT(1, 32, false, true) QG_QUANT(1, 32, true, true)
    QG_QUANT(2, 32, false, false) QG_QUANT(2, 32, true, false) QG_QUANT(2, 32, false, true) QG_QUANT(2, 32, true, true)
#undef QG_QUANT
    return hipErrorInvalidValue;
}

hipError_t launch_quant_wgt_blocks(int fmt, bool bf16in, const void* w, long long ldw, uint8_t* q, long long ldq,
                                   void* s, long long ld_s, int n, int k, hipStream_t st) {
    QuantArgs p{};
    p.x = w;
    p.q = q;
    p.s = s;
    p.ldx = ldw;
    p.ldq = ldq;
    p.s_sm = ld_s;
    p.rows = n;
    p.k = k;
    const dim3 grid(k / 128, (n + 127) / 128);
#define QG_WQ(F, B)                                                                                      \
    if (fmt == F && bf16in == B) {                                                                       \
        quant_wgt_block_kernel<F, B><<<grid, 256, 0, st>>>(p);                                           \
        trace_launch("quant_wgt_block<%s,%s>", F == 0 ? "e4m3,fp32" : "e4m3,e8m0", B ? "bf16" : "fp32"); \
        return hipGetLastError();                                                                        \
    }
    QG_WQ(0, false) QG_WQ(0, true) QG_WQ(1, false) QG_WQ(1, true)
#undef QG_WQ
    return hipErrorInvalidValue;
}

hipError_t launch_relayout(int layout, const uint8_t* src, uint8_t* dst, int n, int kbytes, long long ld,
                           hipStream_t st) {
    const long long units = (layout == 2 ? (long long)((n + 15) / 16) * 16 : (long long)n) * (kbytes / 16);
    const unsigned grid = grid_for(units);
    switch (layout) {
        case 0: relayout_kernel<Lay::KPANEL><<<grid, 256, 0, st>>>(src, dst, n, kbytes, ld); trace_launch("relayout<KPANEL>"); break;
        case 1: relayout_kernel<Lay::W16><<<grid, 256, 0, st>>>(src, dst, n, kbytes, ld); trace_launch("relayout<W16>"); break;
        case 2: relayout_kernel<Lay::FRAG><<<grid, 256, 0, st>>>(src, dst, n, kbytes, ld); trace_launch("relayout<FRAG>"); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_e8m0_shuffle_blocks(const ShuffleArgs& a, int batch, hipStream_t st) {
    const dim3 grid(a.units[0] + a.units[1], batch);
    e8m0_shuffle_blocks_kernel<<<grid, 256, 0, st>>>(a);
    trace_launch("e8m0_shuffle_blocks<%d>", a.units[1] ? 2 : 1);
    return hipGetLastError();
}

hipError_t launch_e8m0_shuffle(const uint8_t* src, uint8_t* dst, int rows, int kg, long long ld, hipStream_t st) {
    const int kg8 = (kg + 7) / 8 * 8;
    const long long bytes = (long long)(rows + 31) / 32 * 32 * kg8;
    e8m0_shuffle_kernel<<<grid_for(bytes), 256, 0, st>>>(src, dst, rows, kg, ld, kg8, bytes);
    trace_launch("e8m0_shuffle");
    return hipGetLastError();
}

}  // namespace qg
