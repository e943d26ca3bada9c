// Device-side building blocks shared by every gfx950 kernel of the library.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qg {

typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

#define QG_LDS __attribute__((address_space(3)))

// Operand format codes of v_mfma_scale_f32_16x16x128_f8f6f4 (cbsz/blgp).
enum : int { kFmtFp8 = 0, kFmtFp4 = 4 };

// s_waitcnt immediates for gfx9-family encoding: vmcnt in [3:0]+[15:14],
// expcnt [6:4], lgkmcnt [11:8]; all-ones means "do not wait".
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
template <int N>
__device__ __forceinline__ void wait_lgkmcnt() {
    static_assert(N >= 0 && N < 16, "lgkmcnt range");
    __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (N << 8) | (3 << 14));
}

// Global -> LDS DMA (global_load_lds_dword{,x4}): lane L of the wave writes
// its 4 or 16 bytes at lds_base + 4L or + 16L; lds_base must be wave-uniform.
// (Sub-dword sizes also occupy one dword slot per lane, so bytes are moved
// as aligned dwords.)
__device__ __forceinline__ void dma16(const void* gsrc, QG_LDS void* lds_base) {
    __builtin_amdgcn_global_load_lds(gsrc, lds_base, 16, 0, 0);
}
__device__ __forceinline__ void dma4(const void* gsrc, QG_LDS void* lds_base) {
    __builtin_amdgcn_global_load_lds(gsrc, lds_base, 4, 0, 0);
}

// fp32 -> bf16, round to nearest even, NaN quieted (the rounding the
// reference validates against: SNAP host.cc:185-193).
__device__ __forceinline__ uint32_t bf16_rne_bits(float x) {
    uint32_t u = __float_as_uint(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return bf16_rne_bits(lo) | (bf16_rne_bits(hi) << 16);
}

// Row swizzle of a 128-byte LDS row: logical 16-byte chunk c of row r lives
// at physical chunk c ^ swz(r), where swz depends on r mod 16 only.  Within
// any aligned group of 16 rows, the 16 lanes that read the same logical
// chunk of the 16 rows touch 16 distinct 16-byte bank groups (64 banks x 4 B)
// and each aligned 8-row half touches 8 distinct ones (32-bank view), so a
// ds_read_b128 of one MFMA operand block is conflict free.
__device__ __forceinline__ int swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

}  // namespace qg
