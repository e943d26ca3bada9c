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

// Buffer -> LDS DMA (buffer_load_dwordx4 ... lds): lane L writes its 16
// bytes at lds_base + 16L.  A lane whose offset falls outside the buffer
// descriptor's range writes zeros and reads no memory.  (Kept out of lambdas:
// the host pass of a kernel drops the kernel's launch stub when this builtin
// appears in a lambda body.)
__device__ __forceinline__ void dma16_buf(__amdgpu_buffer_rsrc_t r, QG_LDS void* lds_base, int voff, int soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds_base, 16, voff, soff, 0, 0);
}
// The same with the nontemporal cache policy, for data read exactly once
// (a decode GEMM's B): measured 4-7% faster than cached DMAs there, and
// 2.5-4% slower where other workgroups re-read the bytes from cache.
__device__ __forceinline__ void dma16_buf_nt(__amdgpu_buffer_rsrc_t r, QG_LDS void* lds_base, int voff, int soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds_base, 16, voff, soff, 0, 2);
}
__device__ __forceinline__ void dma4_buf(__amdgpu_buffer_rsrc_t r, QG_LDS void* lds_base, int voff, int soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds_base, 4, voff, soff, 0, 0);
}

// Split-K partial tiles cross workgroups that run on different XCDs, whose
// L2 caches are not coherent with each other.  An acquire/release counter
// would cost a write-back of the whole L2 before the atomic and an L2
// invalidate after it; instead the partials are written and read with
// device-coherent accesses (cache policy sc1: the instructions the compiler
// emits for relaxed agent-scope atomic stores and loads), the counter is a
// relaxed agent-scope atomic issued only after every partial store of the
// workgroup has completed (s_waitcnt vmcnt(0), then a barrier), and the
// last workgroup reads the partials only after its atomic has returned.
constexpr int kCoherent = 16;    // buffer-instruction cache policy: sc1
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ __amdgpu_buffer_rsrc_t partial_rsrc(const float* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, 0x7FFFFFFF, 0x00020000);
}
__device__ __forceinline__ void store_partial4(__amdgpu_buffer_rsrc_t r, int elem, f32x4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, elem * 4, 0, kCoherent);
}
__device__ __forceinline__ void store_partial1(__amdgpu_buffer_rsrc_t r, int elem, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), r, elem * 4, 0, kCoherent);
}
__device__ __forceinline__ f32x4 load_partial4(__amdgpu_buffer_rsrc_t r, int elem) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, elem * 4, 0, kCoherent));
}
__device__ __forceinline__ float load_partial1(__amdgpu_buffer_rsrc_t r, int elem) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, elem * 4, 0, kCoherent));
}

// The launch's claim on a tile's counter word, issued by every slice when it
// starts, long before any slice arrives: an atomic max with (epoch << 8)
// turns the re-armed word (zero, or an earlier epoch's count) into "this
// epoch, no arrivals" and leaves a word that already carries this epoch as
// it is, so the arrivals take split_arrive's one-atomic path.  Its result is
// not waited for.  A word above the tag (a wrapped epoch, garbage) keeps its
// value and the arrivals claim it by compare-and-swap instead.  Without the
// claim every slice of a tile arriving close together found an untagged word
// and went through the compare-and-swap loop: configs[0]'s five slices per
// tile measured 13.6 us a launch against 9.1 us.
__device__ __forceinline__ void split_claim(unsigned* ctr, unsigned epoch) {
    __hip_atomic_fetch_max(ctr, epoch << 8, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Split-K arrival counter of one output tile, tagged with the launch's
// epoch: bits 8..31 hold the epoch (a 24-bit number the host takes from a
// process-wide sequence, a new one per launch), bits 0..7 the slices of
// that epoch that have arrived.  A word carrying another epoch -- zero, a
// completed or interrupted earlier launch, or whatever a never-cleared
// workspace holds -- counts as zero arrivals, so the workspace needs no
// clearing between launches and a stale word cannot make a slice
// mistake itself for the last one.  (Only a word that already holds this
// very epoch, 2^-24 for arbitrary bytes, would be miscounted.)
// Fast path: one relaxed fetch_add, which lands on the tagged word for
// every slice after the first.  A slice whose add found a word of another
// epoch claims the word with a compare-and-swap (to this epoch, one
// arrival) or, when another slice claimed it first, counts itself into the
// claimed word; every failed swap means another slice's swap succeeded, so
// the loop ends within splitk rounds.  Called by one lane; true for the
// slice that completes the count.
__device__ __forceinline__ bool split_arrive(unsigned* ctr, unsigned epoch, int splitk) {
    const unsigned tag = epoch << 8;
    const unsigned old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if ((old & ~0xffu) == tag) return (int)(old & 0xffu) + 1 == splitk;
    unsigned expect = old + 1u;    // the word as this slice's add left it
    for (;;) {
        const unsigned want = (expect & ~0xffu) == tag ? expect + 1u : tag | 1u;
        if (__hip_atomic_compare_exchange_strong(ctr, &expect, want, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT))
            return (int)(want & 0xffu) == splitk;
    }
}

// fp32 -> bf16 with round-to-nearest-even (the rounding the reference
// validates against, SNAP host.cc:185-193): v_cvt_pk_bf16_f32 converts two
// values per instruction in hardware.
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    const bf16x2_t b = __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t);
    return __builtin_bit_cast(uint32_t, b);
}
__device__ __forceinline__ uint16_t bf16_bits(float x) { return (uint16_t)(pack_bf16x2(x, 0.f) & 0xffffu); }

// Row swizzle of a 128-byte LDS row: logical 16-byte chunk c of row r lives
// at physical chunk c ^ swz(r) (r taken mod 16).  Chosen per operand format
// from SQ_LDS_BANK_CONFLICT measurements of the exact ds_read_b128 patterns
// (16 rows x 4 lane groups per instruction, 256 B/clk LDS):
//   fp8 reads chunks q and q+4  -> swz(r) = r & 7                 0 conflicts
//   fp4 reads chunks 2q and 2q+1 -> swz(r) = (r & 7) ^ (r>>3 & 1) 0 conflicts
// (each of the two costs one extra cycle per access on the other format).
template <bool FP4>
__device__ __forceinline__ int swz(int r) {
    return FP4 ? ((r & 7) ^ ((r >> 3) & 1)) : (r & 7);
}

}  // namespace qg
