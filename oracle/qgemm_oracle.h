/*
 * CPU oracle for the quantized-GEMM hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library restates, in plain C, the CPU-side
 * semantics of the reference's host drivers (value codecs, data generation,
 * layout transforms and the CPU reference GEMMs). Only tests/, the smoke
 * check in __graft_entry__.py and the cpu_baseline leg of bench.py may load
 * it, and only as the checker or the reported CPU baseline. The product
 * library (355_1_trans_amd/) never links or calls it.
 *
 * Reference files followed (root /root/reference/):
 *   BPS  = block_scale_gemm_bpreshuffle/
 *   MX8  = mxfp8_gemm/
 *   MX4  = mxfp4_gemm_4wave_20261112/
 *   SNAP = trace_block_scale_latest_20260914_040021/source_snapshot/
 */
#ifndef QGEMM_ORACLE_H
#define QGEMM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- value codecs ---------------------------------------------------- */
float    ora_e4m3_to_f32(uint8_t v);          /* OCP E4M3FN decode            */
uint8_t  ora_f32_to_e4m3(float x);            /* RNE, saturate to +-448       */
float    ora_e8m0_to_f32(uint8_t e);          /* 2^(e-127)                    */
float    ora_e2m1_to_f32(unsigned code);      /* 4-bit E2M1 decode            */
unsigned ora_f32_to_e2m1(float x);            /* RNE onto E2M1 grid, sat +-6  */
uint16_t ora_f32_to_bf16(float x);            /* RNE, NaN quieted             */
float    ora_bf16_to_f32(uint16_t v);
void     ora_f32_to_bf16_array(const float* x, uint16_t* y, size_t n);
void     ora_bf16_to_f32_array(const uint16_t* x, float* y, size_t n);
void     ora_e4m3_decode_array(const uint8_t* x, float* y, size_t n);

/* ---- seeded data ----------------------------------------------------- */
uint64_t ora_mix_bits(uint64_t x);
/* N(0,1) fp32: counter-based splitmix64 + Box-Muller, element i depends only
 * on (seed, stream, i), so the draw is identical for any thread count. */
void ora_randn(float* out, size_t n, uint64_t seed, uint64_t stream);

/* ---- quantizers (BASELINE.json recipe) ------------------------------- */
/* 1 x 128 per-token: q [M][K] e4m3, s [M][K/128] fp32 row-major. */
void ora_quant_bs_act(const float* x, int m, int k, uint8_t* q, float* s);
/* 128 x 128 weight blocks: q [N][K] e4m3, s [ceil(N/128)][K/128] fp32. */
void ora_quant_bs_wgt(const float* w, int n, int k, uint8_t* q, float* s);
/* MXFP8: per 32-group scale 2^ceil(log2(amax/448)); e [R][K/32] uint8. */
void ora_quant_mx8(const float* x, int rows, int k, uint8_t* q, uint8_t* e);
/* MXFP4: per 32-group scale 2^ceil(log2(amax/6)); q [R][K/2], low nibble
 * holds the even element; e [R][K/32]. */
void ora_quant_mx4(const float* x, int rows, int k, uint8_t* q, uint8_t* e);
/* Block-scale FP8 with E8M0 scales 2^ceil(log2(amax/448)): per 1x128
 * activation block (e row-major [M][K/128]) or 128x128 weight block
 * (e [ceil(N/128)][K/128]); codes E + 127. */
void ora_quant_bs_e8m0_act(const float* x, int m, int k, uint8_t* q, uint8_t* e);
void ora_quant_bs_e8m0_wgt(const float* w, int n, int k, uint8_t* q, uint8_t* e);
/* Exponent helper: ceil(log2(v)) for v > 0. */
int  ora_ceil_log2(float v);

/* ---- layout transforms (pure byte permutations) ---------------------- */
/* K-panel: dst[kt][n][ki] = src[n][kt*128+ki]  (BPS host.cc:92-111). */
void ora_shuffle_b_kpanel(const uint8_t* src, uint8_t* dst, int n, int kbytes, int block_k);
/* shuffle_weight(16,16): dst[n/16][kb/16][n%16][kb%16] = src[n][kb] over
 * bytes (SNAP host.cc:161-179; MX4 candidate_m10 host.cc:215-225). */
void ora_shuffle_weight_16x16(const uint8_t* src, uint8_t* dst, int n, int kbytes);
/* aiter e8m0_shuffle (MX4 candidate_m10 host.cc:194-206); dst holds
 * ceil(rows/32)*32 * ceil(kg/8)*8 bytes, padding 0x7F. */
size_t ora_e8m0_shuffle_bytes(int rows, int kg);
void ora_e8m0_shuffle(const uint8_t* src, uint8_t* dst, int rows, int kg);

/* ---- CPU reference GEMMs --------------------------------------------- */
/* Block-scale FP8 with fp32 scales (BPS host.cc:66-90): sequential fp32
 * accumulation of (a*b)*(sa*sb) one K-group of 128 at a time.
 * sfa(m,kg) = sfa[kg*sfa_sk + m*sfa_sm]; sfb(n,kg) = sfb[(n/128)*sfb_sn + kg*sfb_sk].
 * a [M][lda], b [N][ldb] raw K-contiguous; c [M][ldc] fp32. */
void ora_gemm_bs_fp32(const uint8_t* a, const uint8_t* b, const float* sfa, const float* sfb,
                      float* c, int m, int n, int k, int lda, int ldb, int ldc,
                      int sfa_sm, int sfa_sk, int sfb_sn, int sfb_sk);
/* MXFP8 (MX8 host.cc:96-122): sum += a*b*(sa*sb) in fp32. sfa [M][sfa_ld],
 * sfb [N][sfb_ld] e8m0, one byte per 32 K elements. */
void ora_gemm_mx8(const uint8_t* a, const uint8_t* b, const uint8_t* sfa, const uint8_t* sfb,
                  float* c, int m, int n, int k, int lda, int ldb, int ldc, int sfa_ld, int sfb_ld);
/* MXFP4 (MX4 host.cc:96-115): exact fp64 accumulation, fp32 result.
 * a [M][lda bytes], b [N][ldb bytes]. */
void ora_gemm_mx4(const uint8_t* a, const uint8_t* b, const uint8_t* sfa, const uint8_t* sfb,
                  float* c, int m, int n, int k, int lda, int ldb, int ldc, int sfa_ld, int sfb_ld);
/* The same product in the grouped form of MX4 host.cc:66-94 (gemm_ref_gpu):
 * exact fp32 partial per 32-element group, fp64 sum of partial * scale.
 * Bit-identical to ora_gemm_mx4 whenever the fp64 sums are exact. */
void ora_gemm_mx4_grouped(const uint8_t* a, const uint8_t* b, const uint8_t* sfa, const uint8_t* sfb,
                          float* c, int m, int n, int k, int lda, int ldb, int ldc, int sfa_ld, int sfb_ld);
/* Block-scale FP8 with E8M0 scales (SNAP host.cc:219-248): fp64
 * accumulation; also returns sum|term| in mag (may be NULL).
 * sfa physical [K/128][M] (sfa(m,kg) = sfa[kg*sfa_sk + m]); sfb [N/128][sfb_sn]. */
void ora_gemm_bs_e8m0(const uint8_t* a, const uint8_t* b, const uint8_t* sfa, const uint8_t* sfb,
                      float* c, double* mag, int m, int n, int k, int lda, int ldb, int ldc,
                      int sfa_sk, int sfb_sn);

/* Point-sampled versions: out[i] = C[rows[i]][cols[i]] with the same
 * per-element arithmetic as the full GEMM. */
void ora_gemm_bs_fp32_points(const uint8_t* a, const uint8_t* b, const float* sfa, const float* sfb,
                             int k, int lda, int ldb, int sfa_sm, int sfa_sk, int sfb_sn, int sfb_sk,
                             const int32_t* rows, const int32_t* cols, size_t np, float* out);
void ora_gemm_mx8_points(const uint8_t* a, const uint8_t* b, const uint8_t* sfa, const uint8_t* sfb,
                         int k, int lda, int ldb, int sfa_ld, int sfb_ld,
                         const int32_t* rows, const int32_t* cols, size_t np, float* out);
void ora_gemm_bs_e8m0_points(const uint8_t* a, const uint8_t* b, const uint8_t* sfa, const uint8_t* sfb,
                             int k, int lda, int ldb, int sfa_sk, int sfb_sn,
                             const int32_t* rows, const int32_t* cols, size_t np, float* out);
void ora_gemm_mx4_points(const uint8_t* a, const uint8_t* b, const uint8_t* sfa, const uint8_t* sfb,
                         int k, int lda, int ldb, int sfa_ld, int sfb_ld,
                         const int32_t* rows, const int32_t* cols, size_t np, float* out);

/* ---- tolerance ---------------------------- */
/* Counts elements with |got-ref| > 2^-7*|ref| + 1e-3*rms(ref) (or any
 * non-finite got); writes the largest |got-ref|/bound ratio. rms is taken
 * over `ref` unless rms_override > 0. */
size_t ora_check_tolerance(const float* ref, const float* got, size_t n, double rms_override,
                           double* max_ratio, size_t* worst_index);
double ora_rms(const float* x, size_t n);

int ora_num_threads(void);

#ifdef __cplusplus
}
#endif
#endif
