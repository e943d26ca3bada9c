// Host-side launch wrappers shared between the kernel translation units and
// the C ABI layer (abi.hip).  Each wrapper launches exactly one kernel.
#pragma once
#include <hip/hip_runtime.h>
#include "tile_args.hpp"

namespace qg {

// Per-thread record of the kernels launched by the calling thread's most
// recent entry-point call (read back with qgemm_last_launch): the entry
// point resets it, every launcher appends its exact instantiation.
void trace_reset();
const char* g_trace_str();
void trace_launch(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

// kernels_bsf32.hip: eight-wave 256 x 256 tiles, fp32 block scales; B' (K-panel) or,
// with frag, B'' (the LDS-bypass entry's fragment order)
struct Bsf32Args;
// kernels_band.hip: band kernel (MX, row-major B, M <= 64): a workgroup owns
// 128 * cb columns and a K slice with A's slice in LDS; (mb, cb) in {(1,1),
// (1,2), (2,1), (4,1), (4,2)}
struct BandArgs;
hipError_t launch_band(const BandArgs& a, bool fp4, int mb, int cb, int batch, bool bf16, hipStream_t s);
hipError_t launch_bsf32(const Bsf32Args& a, int batch, bool bf16, bool frag, hipStream_t s);
// kernels_wide.hip: four-wave 256 x 256 tiles, accumulators in AGPRs
// panel_bytes: MX8 scale panel width, 16 or 4 bytes per row
hipError_t launch_wide_mx8_raw(const TileArgs& a, int batch, bool bf16, int panel_bytes, hipStream_t s);
// panel_bytes: MX4 scale panel width, 32, 16 or 8 bytes per row
hipError_t launch_wide_mx4_raw(const TileArgs& a, int batch, bool bf16, int panel_bytes, hipStream_t s);
// MXFP4 in aiter's bpreshuffle formats: B shuffle_weight(16,16), scales
// e8m0_shuffle (sfa_sm / sfb_sn = bytes per 32-row block, sfa_sk = sfb_sk =
// 256); panel_bytes 32 (K % 1024 == 0) or 8; persist_blocks > 0: persistent grid
hipError_t launch_wide_mx4_w16s(const TileArgs& a, int batch, bool bf16, int panel_bytes, int persist_blocks,
                                hipStream_t s);
hipError_t launch_wide_bs8_w16(const TileArgs& a, int batch, bool bf16, hipStream_t s);
// kernels_quad.hip: one-by-four wave 256 x 256 MXFP4 tiles, B straight into
// registers (W16 or row-major), scales in e8m0_shuffle order (sfa_sm / sfb_sn =
// bytes per 32-row block); every operand's bytes per batch entry below 2^31
hipError_t launch_quad_mx4(const TileArgs& a, int batch, bool w16, bool bf16, hipStream_t s);
// K-major operands: A [K][M] (a_km, lda = row pitch >= M) and/or B [K][N]
// (b_kn, ldb >= N); M and N multiples of 256
hipError_t launch_wide_bs8_kmajor(const TileArgs& a, int batch, bool bf16, bool a_km, bool b_kn, hipStream_t s);
// E8M0 scales of A and B into the wide kernel's panel-major layout
// [ngroups/pb][rows][pb] (pb = 16 or 32 bytes, ngroups % pb == 0)
struct ScalePanelArgs {
    const uint8_t* src[2];
    uint8_t* dst[2];
    int rows[2], ld[2];
    long long src_batch[2], dst_batch[2];
    int ngroups, pb;
};
hipError_t launch_mx_scale_panels(const ScalePanelArgs& a, int batch, hipStream_t s);

// kernels_mid.hip: four-wave 128 x 128 tiles, split-K; fp32 block scales
// with B' or B'', or MXFP8 / MXFP4 with row-major B
struct MidArgs;
enum class MidKind : int { BS_KPANEL, BS_FRAG, MX8, MX4 };
// stages: 2 (two workgroups per CU) or 4 (one, three K-tiles in flight)
hipError_t launch_mid(const MidArgs& a, int batch, bool bf16, MidKind kind, int stages, hipStream_t s);
// kernels_mid.hip: sum of fp32 split-K partial planes [splitk][batch][M][N] into C
struct SplitReduceArgs;
hipError_t launch_splitk_reduce(const SplitReduceArgs& r, bool bf16, hipStream_t s);
// skinny_*.hip: skinny-M / split-K kernel (mb = M-tile rows / 16, nb = N-tile columns / 16)
struct SkinnyArgs;
enum class SkinnyKind : int { MX8_RAW, MX4_RAW, BSF32_KPANEL, BSF32_FRAG };
hipError_t launch_skinny(SkinnyKind kind, const SkinnyArgs& a, int mb, int nb, int batch, bool bf16, hipStream_t s);
hipError_t launch_skinny_mx8(const SkinnyArgs& a, int mb, int nb, int batch, bool bf16, hipStream_t s);
hipError_t launch_skinny_mx4(const SkinnyArgs& a, int mb, int nb, int batch, bool bf16, hipStream_t s);
// kernels_decode.hip: decode kernel (M <= 64, mb row blocks, nw waves of 16 columns)
struct DecodeArgs;
hipError_t launch_decode(SkinnyKind kind, const DecodeArgs& a, int mb, int nw, int batch, bool bf16, hipStream_t s);
// kernels_stream.hip: row-streaming decode kernel (row-major MX B, M <= mb <= 8; wr rows
// of B per MFMA; (wr, mb) in {(1,1), (2,2), (4,4), (4,8)})
struct StreamArgs;
hipError_t launch_stream(const StreamArgs& a, bool fp4, int wr, int mb, int batch, bool bf16, hipStream_t s);
// kernels_burst.hip: burst kernel (fp8, fp32 block scales, M <= 64; mb row
// blocks, nb 16-column blocks and 4, 8 or 16 waves per workgroup; frag: B''
// instead of B')
struct BurstArgs;
hipError_t launch_burst(const BurstArgs& a, bool frag, int mb, int nb, int waves, int batch, bool bf16,
                        hipStream_t s);
// kernels_burst_mx.hip: the same for MXFP8 / MXFP4 (fp4) with row-major B and E8M0 scales
// kernels_burst_mx4s.hip: MXFP4 with W16 B (= B'' bytes) and e8m0_shuffle
// scales (sfa_sm / sfb_sn = bytes per 32-row block)
hipError_t launch_burst_mx4s(const BurstArgs& a, int mb, int nb, int waves, int batch, bool bf16, hipStream_t s);
hipError_t launch_burst_mx(const BurstArgs& a, bool fp4, int mb, int nb, int waves, int batch, bool bf16,
                           hipStream_t s);
// kernels_burst_grouped.hip / kernels_burst_mx_grouped.hip: the grouped form
// (several decode GEMMs, one grid over their work items; grid = the item
// count, or fewer workgroups for a persistent walk)
struct BurstGroup;
hipError_t launch_burst_grouped(const BurstGroup& g, bool frag, int mb, int nb, int waves, int grid, bool bf16,
                                hipStream_t s);
hipError_t launch_burst_mx_grouped(const BurstGroup& g, bool fp4, int mb, int nb, int waves, int grid, bool bf16,
                                   hipStream_t s);
// kernels_runs.hip: row-run decode kernel (MXFP8 / MXFP4, row-major B, M <= 16 mb,
// 32 columns per workgroup; 16-byte aligned rows and scale rows)
struct RunsArgs;
hipError_t launch_runs(const RunsArgs& a, bool fp4, int mb, int batch, bool bf16, hipStream_t s);
// kernels_slice.hip: slice decode kernel (the same operands and arguments; 16
// slice_nbw(mb) columns per workgroup, K slices of slice_kps(mb) K-tiles)
hipError_t launch_slice(const RunsArgs& a, bool fp4, int mb, int batch, bool bf16, hipStream_t s);
// the same for MXFP4 in aiter's formats: W16 B (b_bytes = N * K / 2) and
// e8m0_shuffle scales (sfa_sm / sfb_sn = bytes per 32-row block)
hipError_t launch_slice_mx4s(const RunsArgs& a, int mb, int batch, bool bf16, hipStream_t s);
// B' (K-panel) -> B'' (fragment order of the LDS-bypass path)
hipError_t launch_repack_frag(const uint8_t* bk, uint8_t* bpp, int n, int k, int batch, long long bk_batch,
                              long long bpp_batch, hipStream_t s);

// quant.hip: device-side quantizers and weight layouts.
// fmt 0: e4m3 + fp32 scale amax/448; 1: e4m3 + E8M0; 2: e2m1 + E8M0.
// group: 128 (1x128 blocks) or 32 (MX); scale(r, g) = s[r*s_sm + g*s_sk]
// unless shuffle (e8m0_shuffle order).
hipError_t launch_quant_rows(int fmt, int group, bool bf16in, bool shuffle, const void* x, long long ldx,
                             uint8_t* q, long long ldq, void* s, long long s_sm, long long s_sk, int rows, int k,
                             hipStream_t st);
// 128 x 128 weight blocks; scale(nb, g) = s[nb*ld_s + g]; fmt 0 or 1
hipError_t launch_quant_wgt_blocks(int fmt, bool bf16in, const void* w, long long ldw, uint8_t* q, long long ldq,
                                   void* s, long long ld_s, int n, int k, hipStream_t st);
// layout 0: K-panel, 1: shuffle_weight(16,16), 2: B'' (ldsbypass fragment order)
hipError_t launch_relayout(int layout, const uint8_t* src, uint8_t* dst, int n, int kbytes, long long ld,
                           hipStream_t st);
hipError_t launch_e8m0_shuffle(const uint8_t* src, uint8_t* dst, int rows, int kg, long long ld, hipStream_t st);
// e8m0_shuffle of one or two operands over a batch in one launch (quant.hip):
// operand i: rows[i] x kg row-major bytes at src[i] (pitch ld[i]; src and
// ld dword aligned) -> dst[i] (16-byte aligned, ceil(rows/32) * 32 *
// ceil(kg/8) * 8 bytes); units[i] = ceil(rows[i]/32) * ceil(ceil(kg/8)/16)
// workgroups per batch entry (units[1] = 0: one operand)
struct ShuffleArgs {
    const uint8_t* src[2];
    uint8_t* dst[2];
    int rows[2];
    long long ld[2];
    long long src_batch[2], dst_batch[2];
    int kg;
    int units[2];
};
hipError_t launch_e8m0_shuffle_blocks(const ShuffleArgs& a, int batch, hipStream_t st);

// ref_gemm.hip: the whole-output reference GEMM (fp64 sums of decoded,
// scaled products; row-major A [M][K] and B [N][K] codes, lda / ldb in
// bytes; fp32 C [M][N] with pitch ldc).  Scales: MX8 / MX4 sfa(m, g) =
// sfa[m * sfa_sm + g] (E8M0 per 32 K), sfb(n, g) = sfb[n * sfb_sm + g];
// BSF32 (fp32) / BS8 (E8M0) sfa(m, kg) = sfa[m * sfa_sm + kg * sfa_sk],
// sfb(nb, kg) = sfb[nb * sfb_sm + kg] per 128 K.
enum class RefFam : int { BSF32 = 0, BS8 = 1, MX8 = 2, MX4 = 3 };
struct RefArgs {
    const uint8_t* a;
    const uint8_t* b;
    const uint8_t* sfa;
    const uint8_t* sfb;
    float* c;
    int m, n, k;
    long long lda, ldb, ldc;
    long long sfa_sm, sfa_sk, sfb_sm;
};
hipError_t launch_ref_gemm(const RefArgs& a, RefFam fam, hipStream_t s);

// probe.hip
hipError_t launch_probe(int32_t* dev_out, hipStream_t s);
constexpr int kProbeWords = 8264;

}  // namespace qg
