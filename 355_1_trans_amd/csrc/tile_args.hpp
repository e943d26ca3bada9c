// Arguments, scale policies and B layouts shared by the tile kernels
// (wide_gemm.hpp, bsf32_gemm.hpp) and the skinny kernel (skinny_gemm.hpp).
//
// Scale policies (one K-tile = 128 bytes of K):
//   MX    one E8M0 per 32 K elements, row-major [rows][K/32] (MX8 host.cc:282-285,
//         MX4 host.cc:207-208).  A row's scales of one K-tile are 4 (fp8) or
//         8 (fp4) bytes of a different cache line per row, so the tile kernels
//         move them as 16-byte panels covering 4 (fp8) or 2 (fp4) K-tiles,
//         double buffered: one L1 request per row per panel instead of per
//         K-tile (narrow 4- or 8-byte panels when K % 512 != 0).
//   BS8   one E8M0 per 128 K elements: SFA column-major [K/128][M], SFB
//         [N/128][K/128] (SNAP gemm_a8w8_mxfp8_scale_common.h:28-35), broadcast
//         to the four 32-element lane groups in the matrix core.
//   MXS   the MX scales in aiter's e8m0_shuffle order (MX4 candidate_m10/
//         gemm_a4w4_mxfp4_4wave_host.cc:194-208): per 32-row block and 8-group
//         K-tile 256 contiguous bytes, byte (g%4)*64 + (r%16)*4 + (g/4)*2 + r/16,
//         so one dword read gives a lane the scales of two fp4 sub-tiles; the
//         blocks' K-tiles are contiguous, so the tile kernel DMAs them as they lie.
//   BSF32 fp32 scales per 1x128 (A) and 128x128 (B) block (BPS host.cc:66-90):
//         the MFMA runs unscaled (E8M0 127 = 1.0) into a fresh fp32 partial
//         and the VALU adds partial * (sfa*sfb) into the accumulator, the
//         reference's order of operations (scale each K-group, then sum).
// B layouts: RAW [N][Kbytes]; KPANEL [Kbytes/128][N][128] (BPS host.cc:92-111);
//            W16 shuffle_weight(16,16) [N/16][Kbytes/16][16][16] (SNAP host.cc:161-179);
//            FRAG this library's B'' for the LDS-bypass entry: per 16-row block and
//            128-byte K-tile, 2048 contiguous bytes in 16x16x128 operand order;
//            KN  [K][N] N-contiguous (row pitch ldb >= N): aiter's NN / TN B
//            (opus_mxfp8_layouts_trace_8192_20261027T005846Z/capture.py:42-62), fp8
//            only, read from LDS with the transposing ds_read_b64_tr_b8.
#pragma once
#include "common.hpp"

namespace qg {

enum class ScaleKind : int { MX = 0, BS8 = 1, BSF32 = 2, MXS = 3 };
enum class BLay : int { RAW = 0, KPANEL = 1, W16 = 2, FRAG = 3, KN = 4 };

constexpr const char* scale_name(ScaleKind k) {
    return k == ScaleKind::MX ? "MX" : k == ScaleKind::BS8 ? "BS8" : k == ScaleKind::MXS ? "MXS" : "BSF32";
}
constexpr const char* layout_name(BLay l) {
    return l == BLay::RAW ? "RAW" : l == BLay::KPANEL ? "KPANEL" : l == BLay::W16 ? "W16" : l == BLay::FRAG ? "FRAG" : "KN";
}

struct TileArgs {
    const uint8_t* a;
    const uint8_t* b;
    void* c;
    const uint8_t* sfa;
    const uint8_t* sfb;
    int m, n;
    int kbytes;          // bytes of K per row: K (fp8) or K/2 (fp4); multiple of 128
    int lda, ldb;        // row pitch in bytes (ldb: RAW only)
    int ldc;             // row pitch of C in elements
    int c_vec;           // elements per aligned C vector store (1, 2, 4 or 8): the largest
                         // power of two whose byte size divides ptr_c, ldc and c_batch (max 16 B)
    long long a_batch, b_batch, c_batch, sfa_batch, sfb_batch;  // batch strides (bytes / elements)
    // scale addressing (in scale elements):
    //   MX    : sfa(m, g) = sfa[m*sfa_sm + g], sfb(n, g) = sfb[n*sfb_sn + g]; the
    //           wide kernel also reads a panel-major copy (sfa_sk / sfb_sk below)
    //   BS8   : sfa(m, kt) = sfa[kt*sfa_sk + m], sfb(nb, kt) = sfb[nb*sfb_sn + kt]
    //   BSF32 : sfa(m, kt) = sfa[kt*sfa_sk + m*sfa_sm], sfb(nb, kt) = sfb[nb*sfb_sn + kt]
    //   MXS   : K-tile kt of 32-row block rb at sfa[rb*sfa_sm + 256*kt] (sfb: sfb_sn)
    int sfa_sm, sfa_sk, sfb_sn;
    // MX, wide kernel: bytes from one K-tile's scales to the next (KT_BYTES =
    // 4 (fp8) or 8 (fp4) row-major; rows * KT_BYTES in the panel-major copy
    // [K/32/PB][rows][PB], whose row pitch sfa_sm / sfb_sn is then PB)
    int sfb_sk;
    int tiles_m, tiles_n;
    int group_m;         // tile-rows per raster group
    int unit_scale;      // E8M0 127, passed at run time
    int batch;           // batch count (the persistent tile kernel walks batch x tiles)
    int persist;         // wide kernel: 1 = persistent grid (each workgroup walks the tile
                         // list with stride gridDim.x), 0 = one tile per workgroup
};

}  // namespace qg
