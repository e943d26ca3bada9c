// Scaled-MFMA and LDS-DMA layout probes: one wave64, known answers.
//
// Re-runs the reference's layout-pinning method (mfma_layout_probe/
// MMA_LAYOUT_PROBING_METHODOLOGY.md:322-334; known answers in
// probe_count.cu:45-59 and probe_scale_map.cu:74-81) with this library's
// own operand conventions.  Word map of the int32 output (64 lanes x 4
// accumulator registers per section, out[base + lane*4 + reg]):
//   [   0, 256) srcA row fingerprint: X[i][0] = i+1, Y[0][j] = 1  -> D = i+1
//   [ 256, 512) srcB col fingerprint: X[i][0] = 1, Y[0][j] = j+1  -> D = j+1
//   [ 512, 768) fp8 ones, scale_a byte0 = 127+L/16, op_sel 0       -> 480
//   [ 768,1024) same scale dword with byte1 = 127, op_sel 1        -> 128
//   [1024,1280) fp8 ones, lane 5 scale_a = 128 (x2)                -> 160 on row 5, else 128
//   [1280,1536) fp4 ones (E2M1 1.0 = 0x2 per nibble)               -> 128
//   [1536,1792) fp4 ones, lane 5 scale_a = 128                     -> 160 on row 5, else 128
//   [1792,2048) LDS image after one global_load_lds_dwordx4 in which lane L
//               fetched 16-byte chunk (5L+3)%64 of a 1 KB pattern whose byte
//               b is (7b+3)&255.
//   [2048,2080) fp8 K-block map: word 8*q0 + d0 is the scale block that the
//               element in byte 0 of dword d0 of lane group q0 (row 0)
//               belongs to (X has that single 1.0, Y is all 1.0, scale_a of
//               lane group q is 2^q, so D[0][0] = 2^block).
//   [2080,2096) same for fp4, dwords 0..3.
// v_mfma_scale_f32_32x32x64_f8f6f4 (64 lanes x 16 accumulator registers per
// section, out[base + lane*16 + reg]); every value is log2(D / 32), -1 for 0:
//   [2096,3120) fp8: X = 1.0 on lanes 0..31 only, scale_a of lane t = 2^t,
//               Y = 1.0 everywhere -> the srcA lane whose row lands in the slot
//   [3120,4144) same with X on lanes 32..63 (scale_a of lane t = 2^(t-32))
//   [4144,5168) fp8: Y = 1.0 on lanes 0..31 only, scale_b 2^t -> srcB lane
//   [5168,6192) same with Y on lanes 32..63
//   [6192,7216) fp4 version of [2096,3120)
//   [7216,8240) fp4 version of [4144,5168)
//   [8240,8256) fp8 K-block map: word 8*g0 + d0 = log2 of the scale applied
//               to byte 0 of dword d0 of lane group g0 (lane 32*g0, row 0)
//               when lane group g's scale is 2^g
//   [8256,8264) fp4 K-block map, dwords 0..3.
#include "launch.hpp"

namespace qg {

namespace {

__device__ int e4m3_small_int(int v) {  // exact E4M3 code of an integer 1..16
    int e = 31 - __clz(v);
    int m = ((v << 3) >> e) & 7;
    return ((e + 7) << 3) | m;
}

__global__ void probe_fill_kernel(int32_t* out) {
    uint8_t* p = (uint8_t*)(out + 1792);
    for (int b = threadIdx.x; b < 1024; b += blockDim.x) p[b] = (uint8_t)((7 * b + 3) & 255);
}

__global__ __launch_bounds__(64) void probe_kernel(int32_t* out, int s127) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds[1024];
    const int L = threadIdx.x;
    const int row = L & 15, q = L >> 4;
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    auto put = [&](int base, f32x4 d) {
        for (int r = 0; r < 4; ++r) out[base + L * 4 + r] = (int32_t)d[r];
    };
    const int one8 = 0x38;                     // E4M3 1.0
    const int ones8 = 0x38383838;
    const int ones4 = 0x22222222;              // E2M1 1.0 in both nibbles
    i32x8 X = {0, 0, 0, 0, 0, 0, 0, 0}, Y = {0, 0, 0, 0, 0, 0, 0, 0};

    if (q == 0) { X[0] = e4m3_small_int(row + 1); Y[0] = one8; }
    put(0, __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(X, Y, zero, kFmtFp8, kFmtFp8, 0, s127, 0, s127));

    X = i32x8{0, 0, 0, 0, 0, 0, 0, 0};
    Y = X;
    if (q == 0) { X[0] = one8; Y[0] = e4m3_small_int(row + 1); }
    put(256, __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(X, Y, zero, kFmtFp8, kFmtFp8, 0, s127, 0, s127));

    X = i32x8{ones8, ones8, ones8, ones8, ones8, ones8, ones8, ones8};
    Y = X;
    put(512, __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(X, Y, zero, kFmtFp8, kFmtFp8, 0, s127 + q, 0, s127));
    put(768, __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(X, Y, zero, kFmtFp8, kFmtFp8, 1,
                                                              (s127 + q) | (s127 << 8), 0, s127));
    put(1024, __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(X, Y, zero, kFmtFp8, kFmtFp8, 0,
                                                               L == 5 ? s127 + 1 : s127, 0, s127));

    X = i32x8{ones4, ones4, ones4, ones4, 0, 0, 0, 0};
    Y = X;
    put(1280, __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(X, Y, zero, kFmtFp4, kFmtFp4, 0, s127, 0, s127));
    put(1536, __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(X, Y, zero, kFmtFp4, kFmtFp4, 0,
                                                               L == 5 ? s127 + 1 : s127, 0, s127));

    // K-block map of the scale: one non-zero element at (lane group q0,
    // dword d0, byte 0) of row 0.
    for (int t = 0; t < 48; ++t) {
        const bool fp4 = t >= 32;
        const int q0 = fp4 ? (t - 32) / 4 : t / 8;
        const int d0 = fp4 ? (t - 32) % 4 : t % 8;
        i32x8 Xk = {0, 0, 0, 0, 0, 0, 0, 0};
        if (L == 16 * q0) Xk[d0] = fp4 ? 0x2 : one8;
        const i32x8 Yk = fp4 ? i32x8{ones4, ones4, ones4, ones4, 0, 0, 0, 0}
                             : i32x8{ones8, ones8, ones8, ones8, ones8, ones8, ones8, ones8};
        const f32x4 d = fp4 ? __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(Xk, Yk, zero, kFmtFp4, kFmtFp4, 0,
                                                                                s127 + q, 0, s127)
                            : __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(Xk, Yk, zero, kFmtFp8, kFmtFp8, 0,
                                                                                s127 + q, 0, s127);
        if (L == 0) out[2048 + t] = (int32_t)d[0];
    }

    // LDS DMA: lane L reads chunk (5L+3)%64 of the pattern written by
    // probe_fill_kernel; the LDS image shows where each lane's bytes land.
    const uint8_t* src = (const uint8_t*)(out + 1792);
    dma16(src + ((5 * L + 3) & 63) * 16, (QG_LDS uint8_t*)lds);
    wait_vmcnt<0>();
    __syncthreads();
    const i32x4 v = *(const i32x4*)(lds + L * 16);
    __syncthreads();
    for (int r = 0; r < 4; ++r) out[1792 + L * 4 + r] = v[r];
}

typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ int log2_or_neg(float v, int bias) {
    return v == 0.f ? -1 : (int)((__builtin_bit_cast(uint32_t, v) >> 23) & 255) - 127 - bias;
}

// 32x32x64 probes (word map in the header comment).
__global__ __launch_bounds__(64) void probe32_kernel(int32_t* out, int s127) {
    const int L = threadIdx.x;
    f32x16 z;
    for (int r = 0; r < 16; ++r) z[r] = 0.f;
    const int ones8 = 0x38383838, ones4 = 0x22222222;
    i32x8 all8, all4, none;
    for (int i = 0; i < 8; ++i) {
        all8[i] = ones8;
        all4[i] = i < 4 ? ones4 : 0;
        none[i] = 0;
    }
    const int sc = s127 + (L & 31);
    for (int half = 0; half < 2; ++half) {
        const bool mine = (L >> 5) == half;
        const f32x16 da = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(mine ? all8 : none, all8, z, kFmtFp8,
                                                                           kFmtFp8, 0, sc, 0, s127);
        const f32x16 db = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(all8, mine ? all8 : none, z, kFmtFp8,
                                                                           kFmtFp8, 0, s127, 0, sc);
        for (int r = 0; r < 16; ++r) {
            out[2096 + half * 1024 + L * 16 + r] = log2_or_neg(da[r], 5);
            out[4144 + half * 1024 + L * 16 + r] = log2_or_neg(db[r], 5);
        }
    }
    {
        const bool mine = L < 32;
        const f32x16 da = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(mine ? all4 : none, all4, z, kFmtFp4,
                                                                           kFmtFp4, 0, sc, 0, s127);
        const f32x16 db = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(all4, mine ? all4 : none, z, kFmtFp4,
                                                                           kFmtFp4, 0, s127, 0, sc);
        for (int r = 0; r < 16; ++r) {
            out[6192 + L * 16 + r] = log2_or_neg(da[r], 5);
            out[7216 + L * 16 + r] = log2_or_neg(db[r], 5);
        }
    }
}

// K-block map of the 32x32x64 scale: one launch per probed element.
__global__ __launch_bounds__(64) void probe32_kblock_kernel(int32_t* out, int s127, int t) {
    const int L = threadIdx.x;
    const bool fp4 = t >= 16;
    const int g0 = fp4 ? (t - 16) / 4 : t / 8;
    const int d0 = fp4 ? (t - 16) % 4 : t % 8;
    f32x16 z;
    for (int r = 0; r < 16; ++r) z[r] = 0.f;
    i32x8 X, Y;
    for (int i = 0; i < 8; ++i) {
        X[i] = 0;
        Y[i] = (fp4 && i >= 4) ? 0 : (fp4 ? 0x22222222 : 0x38383838);
    }
    if (L == 32 * g0) X[d0] = fp4 ? 0x2 : 0x38;
    const int sc = s127 + (L >> 5);
    const f32x16 d = fp4 ? __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(X, Y, z, kFmtFp4, kFmtFp4, 0, sc, 0, s127)
                         : __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(X, Y, z, kFmtFp8, kFmtFp8, 0, sc, 0, s127);
    if (L == 0) out[8240 + t] = log2_or_neg(d[0], 0);
}

}  // namespace

hipError_t launch_probe(int32_t* dev_out, hipStream_t s) {
    probe_fill_kernel<<<1, 256, 0, s>>>(dev_out);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    probe_kernel<<<1, 64, 0, s>>>(dev_out, 127);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    probe32_kernel<<<1, 64, 0, s>>>(dev_out, 127);
    for (int t = 0; t < 24 && e == hipSuccess; ++t) {
        probe32_kblock_kernel<<<1, 64, 0, s>>>(dev_out, 127, t);
        e = hipGetLastError();
    }
    return e;
}

}  // namespace qg
