/*
 * qgemm.h -- C ABI of the MI355X (gfx950) quantized-GEMM library
 * (355_1_trans_amd/libqgemm.so).
 *
 * Every entry point is extern "C", takes plain pointers and sizes, launches
 * asynchronously on the given HIP stream and returns a hipError_t code:
 *   0  (hipSuccess)                     launched;
 *   1  (hipErrorInvalidValue)           null pointer, bad flag, bad shape or
 *                                       stride, int32 overflow, output
 *                                       overlapping an input, or a workspace
 *                                       that is too small;
 *   98 (hipErrorInvalidDeviceFunction)  current device is not gfx950;
 *   otherwise the launch status from hipGetLastError().
 * No entry point allocates device memory or preprocesses inputs; the caller
 * owns every buffer (reference contract:
 * trace_block_scale_latest_20260914_040021/source_snapshot/
 * gemm_a8w8_blockscale_bpreshuffle_launch.cc:29-30).
 *
 * Reference paths below are relative to /root/reference/:
 *   BPS  = block_scale_gemm_bpreshuffle/
 *   LBP  = block_scale_gemm_ldsbypass/
 *   MX8  = mxfp8_gemm/
 *   MX4  = mxfp4_gemm_4wave_20261112/
 *   SNAP = trace_block_scale_latest_20260914_040021/source_snapshot/
 */
#ifndef QGEMM_H
#define QGEMM_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * 96-byte kernel-argument block shared by every family. Field order and
 * size are the reference ABI (SNAP/gemm_a8w8_mxfp8_scale_common.h:12-38,
 * BPS/gemm_a8w8_blockscale_bpreshuffle_common.h:4-25,
 * MX8/gemm_a8w8_mxfp8_common.h:4-25, MX4/gemm_a4w4_mxfp4_4wave_traits.hpp:7-27).
 * Strides are in elements for FP8 operands and in bytes for packed FP4
 * operands; scale strides are in scale elements.
 */
typedef struct opus_gemm_scale_kargs {
    const void* ptr_a;
    const void* ptr_b;
    void* ptr_c;
    int m;
    int n;
    int k;
    int batch;
    int stride_a;
    int stride_b;
    int stride_c;
    int stride_a_batch;
    int stride_b_batch;
    int stride_c_batch;
    const void* ptr_sfa;
    const void* ptr_sfb;
    int stride_sfa;
    int stride_sfb;
    int stride_sfa_batch;
    int stride_sfb_batch;
} opus_gemm_scale_kargs;

/* The fp32-scale block-scale drivers name the same 96-byte block
 * opus_gemm_kargs (BPS/gemm_a8w8_blockscale_bpreshuffle_common.h:4-25). */
typedef opus_gemm_scale_kargs opus_gemm_kargs;

/* LDS-bypass variant: ptr_b_pp (B'' fragment order) follows ptr_b and
 * stride_b_pp_batch is appended (LBP/gemm_a8w8_blockscale_ldsbypass_common.h:4-27). */
typedef struct opus_gemm_ldsbypass_kargs {
    const void* ptr_a;
    const void* ptr_b;
    const void* ptr_b_pp;
    void* ptr_c;
    int m;
    int n;
    int k;
    int batch;
    int stride_a;
    int stride_b;
    int stride_c;
    int stride_a_batch;
    int stride_b_batch;
    int stride_c_batch;
    const void* ptr_sfa;
    const void* ptr_sfb;
    int stride_sfa;
    int stride_sfb;
    int stride_sfa_batch;
    int stride_sfb_batch;
    int stride_b_pp_batch;
} opus_gemm_ldsbypass_kargs;

/* Output dtype codes (the reference's output_bf16 flag: 1 = bf16, 0 = fp32). */
#define QGEMM_OUT_FP32 0
#define QGEMM_OUT_BF16 1

/* ------------------------------------------------------------------ */
/* Block-scale FP8, E8M0 scales: the reference's existing C ABI.        */
/* ------------------------------------------------------------------ */
/* Replaces SNAP/gemm_a8w8_blockscale_bpreshuffle_launch.cc:31-65 with the
 * identical signature and contract: A e4m3 [batch,M,K]; B e4m3 in
 * shuffle_weight(16,16) layout; SFA E8M0 bytes column-major [K/128,M]
 * (stride_sfa = M); SFB E8M0 [N/128,K/128]; C bf16 or fp32 [M,N].
 * M and N multiples of 256, K a multiple of 128, dense strides; `tiles`
 * must be 0 (auto) or 1. */
hipError_t launch_blockscale_bpreshuffle(const opus_gemm_scale_kargs* args, int output_bf16, int tiles,
                                  hipStream_t stream);

/* Physical layouts of C[M,N] = A[M,K] x B[K,N] with the E8M0 block scales
 * above: aiter's opus_gemm_mxfp8_{nn,tn,tt} (reference runner
 * opus_mxfp8_layouts_trace_8192_20261027T005846Z/capture.py:42-62).
 *   NT  A [M,K]; B shuffle_weight(16,16) of [N,K]  (= launch_blockscale_bpreshuffle)
 *   NN  A [M,K]; B [K,N] N-contiguous             (stride_b = N)
 *   TT  A [K,M] M-contiguous (stride_a = M); B [N,K] row-major (stride_b = K)
 *   TN  A [K,M]; B [K,N]
 * Scales, C, shape and density rules as launch_blockscale_bpreshuffle
 * (stride_a_batch = M*K, stride_b_batch = N*K). NN / TT / TN read the M- or
 * N-contiguous operands in place (K-major LDS stages, transposed on the
 * LDS read into the NT kernel's MFMA operands; results bit-identical to NT
 * on the same data). `workspace` is not used (may be NULL):
 * gemm_a8w8_blockscale_layout_workspace_bytes returns 0, kept so callers
 * written against a workspace-taking form keep working. */
#define QGEMM_LAYOUT_NT 0
#define QGEMM_LAYOUT_NN 1
#define QGEMM_LAYOUT_TT 2
#define QGEMM_LAYOUT_TN 3
hipError_t gemm_a8w8_blockscale_layout(const opus_gemm_scale_kargs* args, int layout, int output_bf16,
                                       void* workspace, size_t workspace_bytes, hipStream_t stream);
size_t gemm_a8w8_blockscale_layout_workspace_bytes(const opus_gemm_scale_kargs* args, int layout);

/* ------------------------------------------------------------------ */
/* Block-scale FP8, fp32 scales (1x128 activation, 128x128 weight).     */
/* ------------------------------------------------------------------ */
/* Replaces the launch in BPS/gemm_a8w8_blockscale_bpreshuffle_host.cc:275-284
 * (kernel declared :14-15). A e4m3 [batch,M,K] (stride_a >= K); B e4m3 in
 * K-panel layout [K/128][N][128] (stride_b = 128, BPS host.cc:92-111,263);
 * SFB fp32 [ceil(N/128)][K/128] (stride_sfb = K/128). SFA fp32 is either
 * the reference's column-major [K/128][M] (stride_sfa = M, BPS host.cc:270)
 * or BASELINE's row-major [M][K/128] (stride_sfa = 1). C bf16/fp32 [M,N].
 * Any M >= 1, N >= 1 (tails are masked), K a multiple of 128.
 * `workspace` (fp32 split-K partials) may be NULL; then no split-K is used.
 * Split-K workspace (every entry with a *_workspace_bytes query): at least
 * the queried bytes, 256-byte aligned, any contents; its first 2048 bytes
 * are arrival counters that each launch tags with a fresh epoch, so they
 * need no clearing (a completed call leaves them zero).  Calls that share a
 * workspace must be ordered (same stream).  The MX entries' plan, and so
 * the rounding of their last bits, also depends on workspace_bytes: the
 * four-wave kernel's K split is taken only when its planes fit (a workspace
 * of at least the scale-panel bytes but less than the query runs unsplit). */
hipError_t gemm_a8w8_blockscale_bpreshuffle(const opus_gemm_kargs* args, int out_dtype, void* workspace,
                                     size_t workspace_bytes, hipStream_t stream);
size_t gemm_a8w8_blockscale_bpreshuffle_workspace_bytes(const opus_gemm_kargs* args);

/* Replaces LBP/gemm_a8w8_blockscale_ldsbypass_host.cc:283-294 (main + repack
 * launches). Same math as the bpreshuffle entry; B'' = ptr_b_pp holds B in
 * this library's per-lane fragment order (qgemm_pack_b_ldsbypass), read
 * straight from global memory into registers. ptr_b may be NULL. */
hipError_t gemm_a8w8_blockscale_ldsbypass(const opus_gemm_ldsbypass_kargs* args, int out_dtype, void* workspace,
                                   size_t workspace_bytes, hipStream_t stream);
size_t gemm_a8w8_blockscale_ldsbypass_workspace_bytes(const opus_gemm_ldsbypass_kargs* args);
/* GPU repack B' (K-panel, ptr_b) -> B'' (ptr_b_pp); the reference's
 * gemm_a8w8_blockscale_ldsbypass_repack_kernel (LBP host.cc:289-294). */
hipError_t gemm_a8w8_blockscale_ldsbypass_repack(const opus_gemm_ldsbypass_kargs* args, hipStream_t stream);

/* Kernel selection for the two fp32 block-scale entries: the kernelId of
 * the reference's tuned dispatch (opus_a8w8_bpreshuffle_integration_and_
 * benchmark.md section 3-4: an explicit id skips the tuned-table lookup).
 * AUTO is the library's own plan (what the entries above run); the others
 * force one kernel family with that family's tile and K-split plan, and
 * return hipErrorInvalidValue for shapes the family cannot take (DECODE:
 * M <= 64 and the K-panel B' only; BURST: M <= 64, K <= 8192).  Workspace
 * contract as above, queried per id. */
#define QGEMM_KID_AUTO    0  /* library plan */
#define QGEMM_KID_TILE256 1  /* eight-wave 256x256 tiles */
#define QGEMM_KID_MID     2  /* four-wave 128x128 tiles, split-K */
#define QGEMM_KID_SKINNY  3  /* skinny-M tiles (16-64 rows), split-K */
#define QGEMM_KID_DECODE  4  /* decode kernel: waves split N, A shared through LDS */
#define QGEMM_KID_BURST   5  /* burst kernel: every load issued up front */
#define QGEMM_KID_STREAM  6  /* MX only: row-streaming kernel (M <= 8, N >= 256) */
#define QGEMM_KID_BAND    7  /* MX only: band kernel (M <= 64): 128-256 columns x a K slice, A in LDS */
#define QGEMM_KID_QUAD    8  /* MXFP4 only: one-by-four wave 256x256 tiles, B straight into registers
                                (row-major entries: the scales are shuffled into the workspace first) */
#define QGEMM_KID_RUNS    9  /* MX only: row-run decode kernel (M <= 64): B rows read in 512-byte runs,
                                32 columns per workgroup; 16-byte aligned A / B rows and scale rows */
#define QGEMM_KID_SLICE  10  /* MX only: slice decode kernel (M <= 64): A's K slice in LDS, B fragments
                                straight from memory, 32 / 64 / 128 columns per workgroup for M <= 16 /
                                32 / 64; row-major entries: 16-byte aligned A / B rows and scale rows;
                                also the aiter-format MXFP4 entry (W16 B, e8m0_shuffle scales) */
hipError_t gemm_a8w8_blockscale_bpreshuffle_kid(const opus_gemm_kargs* args, int out_dtype, int kernel_id,
                                                void* workspace, size_t workspace_bytes, hipStream_t stream);
size_t gemm_a8w8_blockscale_bpreshuffle_kid_workspace_bytes(const opus_gemm_kargs* args, int kernel_id);
hipError_t gemm_a8w8_blockscale_ldsbypass_kid(const opus_gemm_ldsbypass_kargs* args, int out_dtype, int kernel_id,
                                              void* workspace, size_t workspace_bytes, hipStream_t stream);
size_t gemm_a8w8_blockscale_ldsbypass_kid_workspace_bytes(const opus_gemm_ldsbypass_kargs* args, int kernel_id);

/* ------------------------------------------------------------------ */
/* MXFP8: e4m3 x e4m3 with one E8M0 scale per 32 K elements.            */
/* ------------------------------------------------------------------ */
/* Replaces the launch in MX8/gemm_a8w8_mxfp8_host.cc:287-296 (kernel
 * MX8/gemm_a8w8_mxfp8_kernel_template.hpp:300-432). TN layout: A [M,K],
 * B [N,K] K-contiguous; SFA [M,K/32], SFB [N,K/32] uint8 row-major
 * (stride_sfa/stride_sfb = row pitch, MX8 host.cc:282-285). C bf16/fp32.
 * Any M, N >= 1, K a multiple of 128. `workspace` (may be NULL;
 * gemm_a8w8_mxfp8_workspace_bytes; contract as above): split-K partials for
 * small and middle M (fewer than 128 256x256 tiles), reduced in the same
 * launch; at larger M a panel-major copy of both operands' E8M0 scales. */
hipError_t gemm_a8w8_mxfp8(const opus_gemm_scale_kargs* args, int out_dtype, void* workspace,
                    size_t workspace_bytes, hipStream_t stream);
size_t gemm_a8w8_mxfp8_workspace_bytes(const opus_gemm_scale_kargs* args);
/* The same with a kernel id (QGEMM_KID_*, as for the fp32 block-scale entries;
 * DECODE and BURST take M <= 64, STREAM M <= 8 with N >= 256 and needs the
 * workspace when its plan splits K; BAND M <= 64 with dword-aligned scale
 * rows, and the workspace when its plan splits K). */
hipError_t gemm_a8w8_mxfp8_kid(const opus_gemm_scale_kargs* args, int out_dtype, int kernel_id, void* workspace,
                               size_t workspace_bytes, hipStream_t stream);
size_t gemm_a8w8_mxfp8_kid_workspace_bytes(const opus_gemm_scale_kargs* args, int kernel_id);

/* ------------------------------------------------------------------ */
/* MXFP4 A4W4: packed e2m1 x e2m1, E8M0 per 32 K elements.             */
/* ------------------------------------------------------------------ */
/* Replaces the launch in MX4/gemm_a4w4_mxfp4_4wave_host.cc:201-216. A [M,K/2],
 * B [N,K/2] bytes (even k in the low nibble), strides in bytes; SFA [M,K/32],
 * SFB [N,K/32] uint8 row-major. C bf16/fp32. Any M, N >= 1; K a multiple of
 * 256. For small and middle M (fewer than 128 256x256 tiles) the call
 * splits K across workgroups when `workspace` is given
 * (gemm_a4w4_mxfp4_workspace_bytes; contract as above) and reduces the fp32
 * partials in the same launch; at larger M the workspace holds a
 * panel-major copy of both operands' E8M0 scales. */
hipError_t gemm_a4w4_mxfp4(const opus_gemm_scale_kargs* args, int out_dtype, void* workspace,
                    size_t workspace_bytes, hipStream_t stream);
size_t gemm_a4w4_mxfp4_workspace_bytes(const opus_gemm_scale_kargs* args);
/* The same with a kernel id (as gemm_a8w8_mxfp8_kid). */
hipError_t gemm_a4w4_mxfp4_kid(const opus_gemm_scale_kargs* args, int out_dtype, int kernel_id, void* workspace,
                               size_t workspace_bytes, hipStream_t stream);
size_t gemm_a4w4_mxfp4_kid_workspace_bytes(const opus_gemm_scale_kargs* args, int kernel_id);

/* MXFP4 with aiter's gemm_a4w4(..., bpreshuffle=True) operands: the
 * 96-byte block plus grid_blocks (MX4/candidate_m10/
 * gemm_a4w4_mxfp4_4wave_traits.hpp:9-30). */
typedef struct opus_gemm_mxfp4_scale_kargs {
    const void* ptr_a;
    const void* ptr_b;
    void* ptr_c;
    int m;
    int n;
    int k;
    int batch;
    int stride_a;
    int stride_b;
    int stride_c;
    int stride_a_batch;
    int stride_b_batch;
    int stride_c_batch;
    const void* ptr_sfa;
    const void* ptr_sfb;
    int stride_sfa;
    int stride_sfb;
    int stride_sfa_batch;
    int stride_sfb_batch;
    int grid_blocks;
} opus_gemm_mxfp4_scale_kargs;

/* Replaces the launch in MX4/candidate_m10/gemm_a4w4_mxfp4_4wave_host.cc:194-250
 * (kargs filled at host.cc:224-235). A [M,K/2] row-major bytes (stride_a);
 * B = shuffle_weight(16,16) of [N,K/2]: byte (n,kb) at
 * (n/16)*16*(K/2) + (kb/16)*256 + (n%16)*16 + kb%16, N a multiple of 16,
 * stride_b = K/2; SFA / SFB in e8m0_shuffle order (qgemm_e8m0_shuffle),
 * stride_sfa / stride_sfb = bytes per 32-row block (>= K, a multiple of
 * 16), stride_sf*_batch >= ceil(rows/32) * stride_sf*. K a multiple of 256,
 * any M. grid_blocks: 0 = one workgroup per 256x256 tile; > 0 = a persistent
 * grid of min(grid_blocks, tiles*batch) workgroups walking the tile list.
 * Needs no workspace. Every shape runs the 256x256 tile kernel (decode
 * shapes run faster through gemm_a4w4_mxfp4 with row-major operands). */
hipError_t gemm_a4w4_mxfp4_bpreshuffle(const opus_gemm_mxfp4_scale_kargs* args, int out_dtype, hipStream_t stream);
/* The same with a kernel id and an optional workspace: QGEMM_KID_AUTO (the
 * library's choice: M = 9-64 on the slice kernel where its plan is one round
 * of 7/10 to all of the CUs with full K slices, else M <= 64 on the burst
 * kernel where its plan takes the shape -- B's 16-row blocks are the
 * 16x16x128 MFMA's operand order, streamed as whole 1 KB loads -- with a K
 * split only when the workspace is given; otherwise the one-by-four wave
 * kernel, or the two-by-two wave kernel for grid_blocks > 0),
 * QGEMM_KID_TILE256 (the two-by-two wave 256x256 tile kernel, the only one
 * that takes grid_blocks > 0), QGEMM_KID_QUAD (one-by-four waves, B straight
 * from memory into registers), QGEMM_KID_BURST (M <= 64) or QGEMM_KID_SLICE
 * (M <= 64: A's K slice in LDS, B's W16 fragments straight into registers);
 * other ids, and shapes a forced id cannot take, are rejected.  The
 * workspace (size from the query below, 256-byte aligned, any contents)
 * carries a burst or slice plan's split-K counters and fp32 partials; the
 * plain entry above runs without one. */
hipError_t gemm_a4w4_mxfp4_bpreshuffle_kid(const opus_gemm_mxfp4_scale_kargs* args, int out_dtype, int kernel_id,
                                           void* workspace, size_t workspace_bytes, hipStream_t stream);
size_t gemm_a4w4_mxfp4_bpreshuffle_kid_workspace_bytes(const opus_gemm_mxfp4_scale_kargs* args, int kernel_id);

/* No counterpart in the reference.  gemm_a4w4_mxfp4 for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc): the same kernels and results,
 * with a static per-device scratch array of
 * gemm_a4w4_mxfp4_noalloc_max_workspace_bytes() bytes (32 MiB) inside the
 * library in place of `workspace`.  Returns hipErrorInvalidValue when the
 * call needs more (gemm_a4w4_mxfp4_workspace_bytes(args) above the limit).
 * Allocates nothing; each GPU keeps its array until the process ends.  All
 * calls on one GPU share that array: calls that overlap in time on one GPU
 * (different streams, or threads without stream order) race. */
hipError_t gemm_a4w4_mxfp4_noalloc(const opus_gemm_scale_kargs* args, int out_dtype, hipStream_t stream);
size_t gemm_a4w4_mxfp4_noalloc_max_workspace_bytes(void);

/* ------------------------------------------------------------------ */
/* Grouped decode GEMMs: several problems in one launch.                */
/* ------------------------------------------------------------------ */
/* The persistent scheduling across mixed decode batches that the
 * reference's split-K plan names next to its fused split-K reduce
 * (R/opus_gemm_splitk_and_interface_refactor.md:41-45; persistent tile walk
 * MX4/MULTITILE_DESIGN.md:78); the reference has no symbol for it.  `args`
 * points to `group_count` (1..16) kargs blocks, each a complete problem as
 * the family's single-problem entry takes it (same layouts, strides and
 * checks), with batch = 1 and 1 <= M <= 64; problems differ in M, N, K,
 * operands, scales and output.  No output may overlap any operand or output
 * of the call.  One grid walks every problem's (output tile, K slice) work
 * items; each split problem sums its slices in its own counters and fp32
 * planes inside the workspace (query: *_grouped_workspace_bytes; rules as
 * the single-problem workspace).  NULL runs every problem unsplit and is
 * refused (hipErrorInvalidValue) when a problem's K is past one workgroup's
 * reach (16 waves x 4-8 K-tiles of 128 bytes, 8 waves x 4 for M > 32).
 * grid_blocks: 0 = one workgroup per item; > 0 = a persistent grid of
 * min(grid_blocks, items) workgroups.  out_dtype applies to every problem. */
hipError_t gemm_a8w8_blockscale_bpreshuffle_grouped(const opus_gemm_kargs* args, int group_count, int out_dtype,
                                                    int grid_blocks, void* workspace, size_t workspace_bytes,
                                                    hipStream_t stream);
size_t gemm_a8w8_blockscale_bpreshuffle_grouped_workspace_bytes(const opus_gemm_kargs* args, int group_count);
hipError_t gemm_a8w8_blockscale_ldsbypass_grouped(const opus_gemm_ldsbypass_kargs* args, int group_count,
                                                  int out_dtype, int grid_blocks, void* workspace,
                                                  size_t workspace_bytes, hipStream_t stream);
size_t gemm_a8w8_blockscale_ldsbypass_grouped_workspace_bytes(const opus_gemm_ldsbypass_kargs* args,
                                                              int group_count);
hipError_t gemm_a8w8_mxfp8_grouped(const opus_gemm_scale_kargs* args, int group_count, int out_dtype, int grid_blocks,
                                   void* workspace, size_t workspace_bytes, hipStream_t stream);
size_t gemm_a8w8_mxfp8_grouped_workspace_bytes(const opus_gemm_scale_kargs* args, int group_count);
hipError_t gemm_a4w4_mxfp4_grouped(const opus_gemm_scale_kargs* args, int group_count, int out_dtype, int grid_blocks,
                                   void* workspace, size_t workspace_bytes, hipStream_t stream);
size_t gemm_a4w4_mxfp4_grouped_workspace_bytes(const opus_gemm_scale_kargs* args, int group_count);

/* ------------------------------------------------------------------ */
/* Whole-output verification.                                           */
/* ------------------------------------------------------------------ */
/* An independent GPU reference GEMM for checking every output of a
 * full-size launch: the role of the reference's gemm_ref_gpu
 * (MX4/gemm_a4w4_mxfp4_4wave_host.cc:66-94, used at :219-257).  Each code
 * is decoded and multiplied by its scale in fp64, the products are summed
 * in fp64 in K order and rounded once into fp32 C [M][N] (stride_c >= N).
 * No MFMA, no shuffled layouts: A [M][K] and B [N][K] row-major codes
 * (fp4: K/2 bytes, even k in the low nibble; strides in bytes), batch 1.
 * Scales: QGEMM_REF_BS_FP32 fp32, QGEMM_REF_BS_E8M0 E8M0 bytes, A per
 * (row, 128 K) row-major (stride_sfa = 1) or column-major [K/128][M]
 * (stride_sfa >= M), B per (128 rows, 128 K) [ceil(N/128)][stride_sfb];
 * QGEMM_REF_MXFP8 / _MXFP4 E8M0 per (row, 32 K), [rows][stride_sfa / _sfb].
 * K a multiple of 128 (block scales) or 32 (MX). */
#define QGEMM_REF_BS_FP32 0
#define QGEMM_REF_BS_E8M0 1
#define QGEMM_REF_MXFP8 2
#define QGEMM_REF_MXFP4 3
hipError_t qgemm_reference_gemm(int family, const opus_gemm_scale_kargs* args, hipStream_t stream);

/* ------------------------------------------------------------------ */
/* Offline layout helpers (host, CPU).                                  */
/* ------------------------------------------------------------------ */
/* K-panel pre-shuffle, BPS host.cc:92-111: dst[kt][n][ki] = src[n][kt*128+ki]. */
int qgemm_shuffle_b_kpanel(const uint8_t* src, uint8_t* dst, int n, int k_bytes);
/* shuffle_weight(16,16): SNAP host.cc:161-179 (fp8) and
 * MX4/candidate_m10 host.cc:215-225 (fp4, over bytes). */
int qgemm_shuffle_weight_16x16(const uint8_t* src, uint8_t* dst, int n, int k_bytes);
/* aiter e8m0_shuffle, MX4/candidate_m10 host.cc:194-206. */
size_t qgemm_e8m0_shuffle_bytes(int rows, int groups_k);
int qgemm_e8m0_shuffle(const uint8_t* src, uint8_t* dst, int rows, int groups_k);
/* B'' for gemm_a8w8_blockscale_ldsbypass from raw B [N][K] (host pack, the
 * role of LBP/gemm_a8w8_blockscale_ldsbypass_hostpack_host.cc:155-218). */
size_t qgemm_ldsbypass_b_bytes(int n, int k);
int qgemm_pack_b_ldsbypass(const uint8_t* b_raw, uint8_t* b_pp, int n, int k);

/* ------------------------------------------------------------------ */
/* Device-side quantizers (the step before the GEMM, on the GPU).       */
/* ------------------------------------------------------------------ */
/* Source: fp32 (in_dtype QGEMM_IN_FP32) or bf16 (QGEMM_IN_BF16) rows of K
 * elements, row pitch ldx >= K a multiple of 4 elements, base aligned to 16
 * (fp32) or 8 (bf16) bytes.  Codes are round-to-nearest-even, saturating,
 * bit-identical to the host recipes of BASELINE.json's configs.  Outputs
 * must not overlap the source or each other.  The reference quantizes with
 * aiter (not in the container; its MXFP4 path is quant(..., shuffle=True),
 * MX4/candidate_m9/README.md:6-12), so these replace that step; the recipes
 * themselves are the ones BASELINE.json configs[0-4] state. */
#define QGEMM_IN_FP32 0
#define QGEMM_IN_BF16 1

/* e4m3 [M,K] (pitch ldq bytes) + fp32 scale amax/448 per 1x128 block
 * (1.0 for an all-zero block): scale(m, g) = scale[m*scale_sm + g*scale_sk],
 * row-major [M][K/128] (scale_sm >= K/128, scale_sk = 1) or the BPS
 * column-major [K/128][M] (scale_sm = 1, scale_sk >= M, BPS host.cc:78,270).
 * K a multiple of 128.  Feeds gemm_a8w8_blockscale_bpreshuffle/_ldsbypass. */
hipError_t qgemm_quant_fp8_blockscale_act(const void* x, int in_dtype, int m, int k, int ldx, uint8_t* q, int ldq,
                                          float* scale, int scale_sm, int scale_sk, hipStream_t stream);
/* e4m3 [N,K] + fp32 scale per 128x128 block, scale [ceil(N/128)][ld_scale]. */
hipError_t qgemm_quant_fp8_blockscale_wgt(const void* w, int in_dtype, int n, int k, int ldw, uint8_t* q, int ldq,
                                          float* scale, int ld_scale, hipStream_t stream);
/* The same blocks with E8M0 scales 2^ceil(log2(amax/448)) (codes E+127):
 * the inputs of launch_blockscale_bpreshuffle (SNAP blockscale_bpreshuffle.py:3-4);
 * pass e_sm = 1, e_sk = M for its column-major SFA. */
hipError_t qgemm_quant_fp8_e8m0_act(const void* x, int in_dtype, int m, int k, int ldx, uint8_t* q, int ldq,
                                    uint8_t* e, int e_sm, int e_sk, hipStream_t stream);
hipError_t qgemm_quant_fp8_e8m0_wgt(const void* w, int in_dtype, int n, int k, int ldw, uint8_t* q, int ldq,
                                    uint8_t* e, int ld_e, hipStream_t stream);
/* MXFP8: e4m3 [rows,K] + E8M0 2^ceil(log2(amax/448)) per 32 K elements;
 * MXFP4: e2m1 [rows,K/2] bytes (even k in the low nibble) + E8M0
 * 2^ceil(log2(amax/6)).  Scales row-major [rows][lde] (shuffle = 0) or in
 * aiter's e8m0_shuffle order (shuffle = 1; qgemm_e8m0_shuffle_bytes bytes,
 * padding 0x7F; lde ignored).  K a multiple of 32. */
hipError_t qgemm_quant_mxfp8(const void* x, int in_dtype, int rows, int k, int ldx, uint8_t* q, int ldq, uint8_t* e,
                             int lde, int shuffle, hipStream_t stream);
hipError_t qgemm_quant_mxfp4(const void* x, int in_dtype, int rows, int k, int ldx, uint8_t* q, int ldq, uint8_t* e,
                             int lde, int shuffle, hipStream_t stream);

/* On-device twins of the offline layout helpers below (same byte maps);
 * src rows of k_bytes with pitch ld_src (multiple of 16), 16-byte aligned
 * buffers, dst packed. */
hipError_t qgemm_shuffle_b_kpanel_device(const uint8_t* src, uint8_t* dst, int n, int k_bytes, int ld_src,
                                         hipStream_t stream);
hipError_t qgemm_shuffle_weight_16x16_device(const uint8_t* src, uint8_t* dst, int n, int k_bytes, int ld_src,
                                             hipStream_t stream);
hipError_t qgemm_pack_b_ldsbypass_device(const uint8_t* b_raw, uint8_t* b_pp, int n, int k, int ld_src,
                                         hipStream_t stream);
hipError_t qgemm_e8m0_shuffle_device(const uint8_t* src, uint8_t* dst, int rows, int groups_k, int ld_src,
                                     hipStream_t stream);

/* ------------------------------------------------------------------ */
/* Layout probe (the reference's mfma_layout_probe/ known answers).     */
/* ------------------------------------------------------------------ */
/* Launches the one-wave scaled-MFMA and LDS-DMA probes on `stream`;
 * dev_out is device memory for qgemm_probe_words() int32 words (word map in
 * 355_1_trans_amd/csrc/probe.hip). The reference's probes are
 * mfma_layout_probe/probe_count.cu:1-63 and probe_scale_map.cu:1-86. */
int qgemm_probe_words(void);
hipError_t qgemm_probe_mfma_layout(int32_t* dev_out, hipStream_t stream);

/* Library identification: "gfx950" build string. */
const char* qgemm_version(void);

/* Diagnostics, no counterpart in the reference: the kernel instantiations
 * (name<template arguments>, joined by '+') that the calling thread's most
 * recent entry-point call launched, e.g.
 * "mx_scale_panels<pb16>+wide_gemm<fp8,MX,RAW,bf16,pb16>"; empty when that
 * call launched nothing (rejected arguments).  Tests and the benchmark use
 * it to name the exact kernel they check or time.  The string is owned by
 * the library and valid until the thread's next entry-point call. */
const char* qgemm_last_launch(void);

#ifdef __cplusplus
}
#endif
#endif
