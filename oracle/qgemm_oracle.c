/*
 * CPU oracle for the quantized-GEMM hot path -- TEST INFRASTRUCTURE ONLY.
 * See qgemm_oracle.h for the contract and the reference files followed.
 *
 * Build: gcc -O3 -fopenmp -ffp-contract=off -fPIC -shared (oracle/Makefile).
 * Contraction is off so the fp32 accumulation order and rounding follow the
 * reference drivers statement by statement (their x86-64 host builds have
 * no FMA instructions to contract into).
 */
#include "qgemm_oracle.h"

#include <math.h>
#include <string.h>
#include <stdlib.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ===================================================================== */
/* value codecs                                                           */
/* ===================================================================== */

/* OCP FP8 E4M3FN: bias 7, no infinities, 0x7F/0xFF are NaN, max 448.
 * Same value set as HIP's __hip_fp8_e4m3 (amd_hip_fp8.h) that the reference
 * drivers cast through (BPS host.cc:29, MX8 host.cc:30, SNAP host.cc:34). */
float ora_e4m3_to_f32(uint8_t v) {
    const int sign = v >> 7;
    const int e = (v >> 3) & 15;
    const int m = v & 7;
    float r;
    if (e == 15 && m == 7) return sign ? -NAN : NAN;
    if (e == 0) r = ldexpf((float)m, -9);                 /* subnormal m/8 * 2^-6 */
    else r = ldexpf(1.0f + (float)m / 8.0f, e - 7);
    return sign ? -r : r;
}

/* Round-to-nearest-even with saturation to the largest finite value, the
 * __HIP_SATFINITE default of HIP's float -> __hip_fp8_e4m3 conversion. */
uint8_t ora_f32_to_e4m3(float x) {
    uint8_t sign = signbit(x) ? 0x80 : 0x00;
    float a = fabsf(x);
    if (isnan(x)) return (uint8_t)(sign | 0x7F);
    if (a >= 448.0f) return (uint8_t)(sign | 0x7E);
    if (a < 0x1p-6f) {                                    /* subnormal range, step 2^-9 */
        float q = nearbyintf(a * 512.0f);                 /* 0..8; 8 is the first normal */
        return (uint8_t)(sign | (uint8_t)q);
    }
    int ex;
    frexpf(a, &ex);                                       /* a = f*2^ex, f in [0.5,1) */
    int E = ex - 1;                                       /* a in [2^E, 2^(E+1)) */
    float q = nearbyintf(ldexpf(a, 3 - E));               /* 8..16, exact scaling */
    if (q >= 16.0f) { q = 8.0f; E += 1; }
    int code = ((E + 7) << 3) | ((int)q - 8);
    if (code > 0x7E) code = 0x7E;
    return (uint8_t)(sign | code);
}

/* E8M0: 2^(e-127), 127 = 1.0 (MX8 host.cc:34-37, SNAP host.cc:181-183). */
float ora_e8m0_to_f32(uint8_t e) { return ldexpf(1.0f, (int)e - 127); }

/* E2M1 magnitudes {0,.5,1,1.5,2,3,4,6}, sign in bit 3 (MX4 host.cc:38-42). */
float ora_e2m1_to_f32(unsigned code) {
    static const float mag[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
    const float v = mag[code & 7];
    return (code & 8) ? -v : v;
}

/* RNE onto the E2M1 grid with saturation at 6. */
unsigned ora_f32_to_e2m1(float x) {
    unsigned sign = signbit(x) ? 8u : 0u;
    float a = fabsf(x);
    if (isnan(x)) return sign | 7u;
    if (a < 1.0f) {                                       /* subnormal: step 0.5 */
        float q = nearbyintf(a * 2.0f);                   /* 0,1,2 (2 == 1.0) */
        return sign | (unsigned)q;
    }
    int ex;
    frexpf(a, &ex);
    int E = ex - 1;                                       /* a in [2^E, 2^(E+1)) */
    float q = nearbyintf(ldexpf(a, 1 - E));               /* 2..4 */
    if (q >= 4.0f) { q = 2.0f; E += 1; }
    if (E > 2) return sign | 7u;
    return sign | (unsigned)(((E + 1) << 1) | ((int)q - 2));
}

/* RNE with NaN quieting (SNAP host.cc:185-193). */
uint16_t ora_f32_to_bf16(float x) {
    uint32_t bits;
    memcpy(&bits, &x, 4);
    if ((bits & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((bits >> 16) | 0x0040u);
    bits += 0x7fffu + ((bits >> 16) & 1u);
    return (uint16_t)(bits >> 16);
}

float ora_bf16_to_f32(uint16_t v) {
    uint32_t bits = (uint32_t)v << 16;
    float r;
    memcpy(&r, &bits, 4);
    return r;
}

void ora_f32_to_bf16_array(const float* x, uint16_t* y, size_t n) {
    #pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; ++i) y[i] = ora_f32_to_bf16(x[i]);
}

void ora_bf16_to_f32_array(const uint16_t* x, float* y, size_t n) {
    #pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; ++i) y[i] = ora_bf16_to_f32(x[i]);
}

static float g_e4m3_lut[256];
static int g_lut_ready = 0;

static void init_lut(void) {
    if (g_lut_ready) return;
    #pragma omp critical(ora_lut)
    {
        if (!g_lut_ready) {
            for (int i = 0; i < 256; ++i) g_e4m3_lut[i] = ora_e4m3_to_f32((uint8_t)i);
            __atomic_store_n(&g_lut_ready, 1, __ATOMIC_RELEASE);
        }
    }
}

void ora_e4m3_decode_array(const uint8_t* x, float* y, size_t n) {
    init_lut();
    #pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; ++i) y[i] = g_e4m3_lut[x[i]];
}

/* ===================================================================== */
/* seeded data                                                            */
/* ===================================================================== */

/* splitmix64 finalizer, as SNAP host.cc:139-144 uses for counter-based
 * initialisation that does not depend on the OpenMP thread count. */
uint64_t ora_mix_bits(uint64_t x) {
    x += 0x9e3779b97f4a7c15ull;
    x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
    x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
    return x ^ (x >> 31);
}

void ora_randn(float* out, size_t n, uint64_t seed, uint64_t stream) {
    const uint64_t base = ora_mix_bits(seed) ^ ora_mix_bits(0x5851f42d4c957f2dull + stream);
    const double two_pi = 6.283185307179586476925286766559;
    #pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; ++i) {
        const uint64_t h1 = ora_mix_bits(base + 2 * (uint64_t)i);
        const uint64_t h2 = ora_mix_bits(base + 2 * (uint64_t)i + 1);
        const double u1 = ((double)(h1 >> 11) + 1.0) * 0x1p-53;   /* (0,1] */
        const double u2 = (double)(h2 >> 11) * 0x1p-53;           /* [0,1) */
        out[i] = (float)(sqrt(-2.0 * log(u1)) * cos(two_pi * u2));
    }
}

/* ===================================================================== */
/* quantizers                                                             */
/* ===================================================================== */

int ora_ceil_log2(float v) {
    int ex;
    float f = frexpf(v, &ex);                             /* v = f*2^ex, f in [0.5,1) */
    return (f == 0.5f) ? ex - 1 : ex;
}

void ora_quant_bs_act(const float* x, int m, int k, uint8_t* q, float* s) {
    const int kg = k / 128;
    #pragma omp parallel for collapse(2) schedule(static)
    for (int r = 0; r < m; ++r) {
        for (int g = 0; g < kg; ++g) {
            const float* src = x + (size_t)r * k + (size_t)g * 128;
            float amax = 0.0f;
            for (int i = 0; i < 128; ++i) amax = fmaxf(amax, fabsf(src[i]));
            const float sc = amax > 0.0f ? amax / 448.0f : 1.0f;
            s[(size_t)r * kg + g] = sc;
            uint8_t* dst = q + (size_t)r * k + (size_t)g * 128;
            for (int i = 0; i < 128; ++i) dst[i] = ora_f32_to_e4m3(src[i] / sc);
        }
    }
}

void ora_quant_bs_wgt(const float* w, int n, int k, uint8_t* q, float* s) {
    const int kg = k / 128;
    const int nb = (n + 127) / 128;
    #pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < nb; ++b) {
        for (int g = 0; g < kg; ++g) {
            const int r0 = b * 128;
            const int r1 = (r0 + 128 < n) ? r0 + 128 : n;
            float amax = 0.0f;
            for (int r = r0; r < r1; ++r)
                for (int i = 0; i < 128; ++i)
                    amax = fmaxf(amax, fabsf(w[(size_t)r * k + (size_t)g * 128 + i]));
            const float sc = amax > 0.0f ? amax / 448.0f : 1.0f;
            s[(size_t)b * kg + g] = sc;
            for (int r = r0; r < r1; ++r)
                for (int i = 0; i < 128; ++i) {
                    const size_t idx = (size_t)r * k + (size_t)g * 128 + i;
                    q[idx] = ora_f32_to_e4m3(w[idx] / sc);
                }
        }
    }
}

/* Shared MX group step: the e8m0 byte and the exact power-of-two scaling.
 * amax == 0 gives the neutral byte 127 (all quanta are then 0). */
static int mx_exponent(float amax, float qmax) {
    if (!(amax > 0.0f)) return 0;
    const float v = amax / qmax;
    if (v == 0.0f) return -127;                           /* quotient underflows: the clamp */
    int e = ora_ceil_log2(v);
    if (e < -127) e = -127;
    if (e > 127) e = 127;
    return e;
}

void ora_quant_mx8(const float* x, int rows, int k, uint8_t* q, uint8_t* e) {
    const int kg = k / 32;
    #pragma omp parallel for collapse(2) schedule(static)
    for (int r = 0; r < rows; ++r) {
        for (int g = 0; g < kg; ++g) {
            const float* src = x + (size_t)r * k + (size_t)g * 32;
            float amax = 0.0f;
            for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(src[i]));
            const int E = mx_exponent(amax, 448.0f);
            e[(size_t)r * kg + g] = (uint8_t)(E + 127);
            uint8_t* dst = q + (size_t)r * k + (size_t)g * 32;
            for (int i = 0; i < 32; ++i) dst[i] = ora_f32_to_e4m3(ldexpf(src[i], -E));
        }
    }
}

void ora_quant_mx4(const float* x, int rows, int k, uint8_t* q, uint8_t* e) {
    const int kg = k / 32;
    #pragma omp parallel for collapse(2) schedule(static)
    for (int r = 0; r < rows; ++r) {
        for (int g = 0; g < kg; ++g) {
            const float* src = x + (size_t)r * k + (size_t)g * 32;
            float amax = 0.0f;
            for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(src[i]));
            const int E = mx_exponent(amax, 6.0f);
            e[(size_t)r * kg + g] = (uint8_t)(E + 127);
            uint8_t* dst = q + (size_t)r * (k / 2) + (size_t)g * 16;
            for (int i = 0; i < 16; ++i) {
                const unsigned lo = ora_f32_to_e2m1(ldexpf(src[2 * i], -E));
                const unsigned hi = ora_f32_to_e2m1(ldexpf(src[2 * i + 1], -E));
                dst[i] = (uint8_t)(lo | (hi << 4));
            }
        }
    }
}

/* Block-scale FP8 with E8M0 scales (the input format of the reference's
 * fastest block-scale kernel, SNAP blockscale_bpreshuffle.py:3-4,54-56):
 * one power-of-two scale 2^ceil(log2(amax/448)) per 1x128 activation block
 * or 128x128 weight block, the MX rule at block-scale granularity.
 * Codes: E + 127; the activation scales are written row-major [M][K/128]. */
void ora_quant_bs_e8m0_act(const float* x, int m, int k, uint8_t* q, uint8_t* e) {
    const int kg = k / 128;
    #pragma omp parallel for collapse(2) schedule(static)
    for (int r = 0; r < m; ++r) {
        for (int g = 0; g < kg; ++g) {
            const float* src = x + (size_t)r * k + (size_t)g * 128;
            float amax = 0.0f;
            for (int i = 0; i < 128; ++i) amax = fmaxf(amax, fabsf(src[i]));
            const int E = mx_exponent(amax, 448.0f);
            e[(size_t)r * kg + g] = (uint8_t)(E + 127);
            uint8_t* dst = q + (size_t)r * k + (size_t)g * 128;
            for (int i = 0; i < 128; ++i) dst[i] = ora_f32_to_e4m3(ldexpf(src[i], -E));
        }
    }
}

void ora_quant_bs_e8m0_wgt(const float* w, int n, int k, uint8_t* q, uint8_t* e) {
    const int kg = k / 128;
    const int nb = (n + 127) / 128;
    #pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < nb; ++b) {
        for (int g = 0; g < kg; ++g) {
            const int r0 = b * 128;
            const int r1 = (r0 + 128 < n) ? r0 + 128 : n;
            float amax = 0.0f;
            for (int r = r0; r < r1; ++r)
                for (int i = 0; i < 128; ++i)
                    amax = fmaxf(amax, fabsf(w[(size_t)r * k + (size_t)g * 128 + i]));
            const int E = mx_exponent(amax, 448.0f);
            e[(size_t)b * kg + g] = (uint8_t)(E + 127);
            for (int r = r0; r < r1; ++r)
                for (int i = 0; i < 128; ++i) {
                    const size_t idx = (size_t)r * k + (size_t)g * 128 + i;
                    q[idx] = ora_f32_to_e4m3(ldexpf(w[idx], -E));
                }
        }
    }
}

/* ===================================================================== */
/* layout transforms                                                      */
/* ===================================================================== */

void ora_shuffle_b_kpanel(const uint8_t* src, uint8_t* dst, int n, int kbytes, int block_k) {
    const int nkt = kbytes / block_k;
    #pragma omp parallel for schedule(static)
    for (int r = 0; r < n; ++r)
        for (int kt = 0; kt < nkt; ++kt)
            memcpy(dst + ((size_t)kt * n + r) * block_k, src + (size_t)r * kbytes + (size_t)kt * block_k,
                   (size_t)block_k);
}

void ora_shuffle_weight_16x16(const uint8_t* src, uint8_t* dst, int n, int kbytes) {
    const int nb = n / 16, kb = kbytes / 16;
    #pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < nb; ++b)
        for (int c = 0; c < kb; ++c)
            for (int ni = 0; ni < 16; ++ni)
                memcpy(dst + ((size_t)b * kb + c) * 256 + (size_t)ni * 16,
                       src + (size_t)(b * 16 + ni) * kbytes + (size_t)c * 16, 16);
}

size_t ora_e8m0_shuffle_bytes(int rows, int kg) {
    const size_t rows32 = (size_t)(rows + 31) / 32 * 32;
    const size_t kg8 = (size_t)(kg + 7) / 8 * 8;
    return rows32 * kg8;
}

void ora_e8m0_shuffle(const uint8_t* src, uint8_t* dst, int rows, int kg) {
    const int kg8 = (kg + 7) / 8 * 8;
    memset(dst, 0x7F, ora_e8m0_shuffle_bytes(rows, kg));
    for (int r = 0; r < rows; ++r)
        for (int g = 0; g < kg; ++g) {
            const size_t o = ((size_t)(r / 32) * (kg8 / 8) + g / 8) * 256 + (size_t)(g % 4) * 64 +
                             (size_t)(r % 16) * 4 + (size_t)((g % 8) / 4) * 2 + (size_t)((r % 32) / 16);
            dst[o] = src[(size_t)r * kg + g];
        }
}

/* ===================================================================== */
/* CPU reference GEMMs                                                    */
/* ===================================================================== */

static inline float bs_fp32_elem(const uint8_t* a_row, const uint8_t* b_row, const float* sfa,
                                 const float* sfb, int i, int j, int k, int sfa_sm, int sfa_sk,
                                 int sfb_sn, int sfb_sk) {
    const int n_group = j / 128;
    float sum = 0.0f;
    for (int g = 0; g < k / 128; ++g) {
        const float scale_a = sfa[(size_t)g * sfa_sk + (size_t)i * sfa_sm];
        const float scale_b = sfb[(size_t)n_group * sfb_sn + (size_t)g * sfb_sk];
        const float scale = scale_a * scale_b;
        for (int p = g * 128; p < (g + 1) * 128; ++p) {
            const float prod = g_e4m3_lut[a_row[p]] * g_e4m3_lut[b_row[p]];
            sum += prod * scale;
        }
    }
    return sum;
}

void ora_gemm_bs_fp32(const uint8_t* a, const uint8_t* b, const float* sfa, const float* sfb,
                      float* c, int m, int n, int k, int lda, int ldb, int ldc,
                      int sfa_sm, int sfa_sk, int sfb_sn, int sfb_sk) {
    init_lut();
    #pragma omp parallel for collapse(2) schedule(static)
    for (int i = 0; i < m; ++i)
        for (int j = 0; j < n; ++j)
            c[(size_t)i * ldc + j] = bs_fp32_elem(a + (size_t)i * lda, b + (size_t)j * ldb, sfa, sfb, i, j,
                                                  k, sfa_sm, sfa_sk, sfb_sn, sfb_sk);
}

void ora_gemm_bs_fp32_points(const uint8_t* a, const uint8_t* b, const float* sfa, const float* sfb,
                             int k, int lda, int ldb, int sfa_sm, int sfa_sk, int sfb_sn, int sfb_sk,
                             const int32_t* rows, const int32_t* cols, size_t np, float* out) {
    init_lut();
    #pragma omp parallel for schedule(static)
    for (size_t t = 0; t < np; ++t) {
        const int i = rows[t], j = cols[t];
        out[t] = bs_fp32_elem(a + (size_t)i * lda, b + (size_t)j * ldb, sfa, sfb, i, j, k, sfa_sm, sfa_sk,
                              sfb_sn, sfb_sk);
    }
}

static inline float mx8_elem(const uint8_t* a_row, const uint8_t* b_row, const uint8_t* sfa_row,
                             const uint8_t* sfb_row, int k) {
    float sum = 0.0f;
    for (int g = 0; g < k / 32; ++g) {
        const float scale = ora_e8m0_to_f32(sfa_row[g]) * ora_e8m0_to_f32(sfb_row[g]);
        for (int p = g * 32; p < (g + 1) * 32; ++p) {
            const float prod = g_e4m3_lut[a_row[p]] * g_e4m3_lut[b_row[p]];
            sum += prod * scale;
        }
    }
    return sum;
}

void ora_gemm_mx8(const uint8_t* a, const uint8_t* b, const uint8_t* sfa, const uint8_t* sfb,
                  float* c, int m, int n, int k, int lda, int ldb, int ldc, int sfa_ld, int sfb_ld) {
    init_lut();
    #pragma omp parallel for collapse(2) schedule(static)
    for (int i = 0; i < m; ++i)
        for (int j = 0; j < n; ++j)
            c[(size_t)i * ldc + j] = mx8_elem(a + (size_t)i * lda, b + (size_t)j * ldb,
                                              sfa + (size_t)i * sfa_ld, sfb + (size_t)j * sfb_ld, k);
}

void ora_gemm_mx8_points(const uint8_t* a, const uint8_t* b, const uint8_t* sfa, const uint8_t* sfb,
                         int k, int lda, int ldb, int sfa_ld, int sfb_ld,
                         const int32_t* rows, const int32_t* cols, size_t np, float* out) {
    init_lut();
    #pragma omp parallel for schedule(static)
    for (size_t t = 0; t < np; ++t) {
        const int i = rows[t], j = cols[t];
        out[t] = mx8_elem(a + (size_t)i * lda, b + (size_t)j * ldb, sfa + (size_t)i * sfa_ld,
                          sfb + (size_t)j * sfb_ld, k);
    }
}

static inline float mx4_elem(const uint8_t* a_row, const uint8_t* b_row, const uint8_t* sfa_row,
                             const uint8_t* sfb_row, int k) {
    double sum = 0.0;
    for (int p = 0; p < k; ++p) {
        const unsigned x = a_row[p / 2], y = b_row[p / 2];
        const unsigned xa = (p & 1) ? (x >> 4) : (x & 15);
        const unsigned yb = (p & 1) ? (y >> 4) : (y & 15);
        sum += (double)ora_e2m1_to_f32(xa) * ora_e2m1_to_f32(yb) *
               ldexp(1.0, (int)sfa_row[p / 32] - 127) * ldexp(1.0, (int)sfb_row[p / 32] - 127);
    }
    return (float)sum;
}

void ora_gemm_mx4(const uint8_t* a, const uint8_t* b, const uint8_t* sfa, const uint8_t* sfb,
                  float* c, int m, int n, int k, int lda, int ldb, int ldc, int sfa_ld, int sfb_ld) {
    #pragma omp parallel for collapse(2) schedule(static)
    for (int i = 0; i < m; ++i)
        for (int j = 0; j < n; ++j)
            c[(size_t)i * ldc + j] = mx4_elem(a + (size_t)i * lda, b + (size_t)j * ldb,
                                              sfa + (size_t)i * sfa_ld, sfb + (size_t)j * sfb_ld, k);
}

/* Grouped form of the same product, the reference's gemm_ref_gpu
 * (MX4 host.cc:66-94): per 32-element group an fp32 partial of the E2M1
 * products (at most 32 products of multiples of 1/4 up to 36, so the
 * partial is exact in fp32), then sum += partial * 2^(ea+eb-254) in fp64.
 * g_e2m1_pair[x][y] is one byte pair's two products, t0 + t1, in the
 * reference's statement order.  Whenever the fp64 sums are exact (scale
 * spreads below ~2^40, which covers every recipe here) the result is
 * bit-identical to the literal gemm_ref_cpu loop above. */
static float g_e2m1_pair[256 * 256];
static int g_pair_ready = 0;

static void init_pair_lut(void) {
    if (__atomic_load_n(&g_pair_ready, __ATOMIC_ACQUIRE)) return;
    #pragma omp critical(ora_pair_lut)
    {
        if (!g_pair_ready) {
            for (int x = 0; x < 256; ++x)
                for (int y = 0; y < 256; ++y) {
                    const float t0 = ora_e2m1_to_f32((unsigned)x & 15u) * ora_e2m1_to_f32((unsigned)y & 15u);
                    const float t1 = ora_e2m1_to_f32((unsigned)x >> 4) * ora_e2m1_to_f32((unsigned)y >> 4);
                    g_e2m1_pair[x * 256 + y] = t0 + t1;
                }
            __atomic_store_n(&g_pair_ready, 1, __ATOMIC_RELEASE);
        }
    }
}

static inline float mx4_elem_grouped(const uint8_t* a_row, const uint8_t* b_row, const uint8_t* sfa_row,
                                     const uint8_t* sfb_row, int k) {
    double sum = 0.0;
    for (int g = 0; g < k / 32; ++g) {
        float part = 0.0f;
        for (int p = 0; p < 16; ++p) part += g_e2m1_pair[(unsigned)a_row[g * 16 + p] * 256u + b_row[g * 16 + p]];
        sum += (double)part * ldexp(1.0, (int)sfa_row[g] + (int)sfb_row[g] - 254);
    }
    return (float)sum;
}

void ora_gemm_mx4_grouped(const uint8_t* a, const uint8_t* b, const uint8_t* sfa, const uint8_t* sfb,
                          float* c, int m, int n, int k, int lda, int ldb, int ldc, int sfa_ld, int sfb_ld) {
    init_pair_lut();
    #pragma omp parallel for collapse(2) schedule(static)
    for (int i = 0; i < m; ++i)
        for (int j = 0; j < n; ++j)
            c[(size_t)i * ldc + j] = mx4_elem_grouped(a + (size_t)i * lda, b + (size_t)j * ldb,
                                                      sfa + (size_t)i * sfa_ld, sfb + (size_t)j * sfb_ld, k);
}

void ora_gemm_mx4_points(const uint8_t* a, const uint8_t* b, const uint8_t* sfa, const uint8_t* sfb,
                         int k, int lda, int ldb, int sfa_ld, int sfb_ld,
                         const int32_t* rows, const int32_t* cols, size_t np, float* out) {
    init_pair_lut();
    #pragma omp parallel for schedule(static)
    for (size_t t = 0; t < np; ++t) {
        const int i = rows[t], j = cols[t];
        out[t] = mx4_elem_grouped(a + (size_t)i * lda, b + (size_t)j * ldb, sfa + (size_t)i * sfa_ld,
                                  sfb + (size_t)j * sfb_ld, k);
    }
}

static inline float bs_e8m0_elem(const uint8_t* a_row, const uint8_t* b_row, const uint8_t* sfa,
                                 const uint8_t* sfb, int i, int j, int k, int sfa_sk, int sfb_sn,
                                 double* mag_out) {
    double sum = 0.0, sum_abs = 0.0;
    for (int g = 0; g < k / 128; ++g) {
        const double scale = (double)ora_e8m0_to_f32(sfa[(size_t)g * sfa_sk + i]) *
                             (double)ora_e8m0_to_f32(sfb[(size_t)(j / 128) * sfb_sn + g]);
        for (int p = g * 128; p < (g + 1) * 128; ++p) {
            const double term = (double)g_e4m3_lut[a_row[p]] * (double)g_e4m3_lut[b_row[p]] * scale;
            sum += term;
            sum_abs += fabs(term);
        }
    }
    if (mag_out) *mag_out = sum_abs;
    return (float)sum;
}

void ora_gemm_bs_e8m0(const uint8_t* a, const uint8_t* b, const uint8_t* sfa, const uint8_t* sfb,
                      float* c, double* mag, int m, int n, int k, int lda, int ldb, int ldc,
                      int sfa_sk, int sfb_sn) {
    init_lut();
    #pragma omp parallel for collapse(2) schedule(static)
    for (int i = 0; i < m; ++i)
        for (int j = 0; j < n; ++j)
            c[(size_t)i * ldc + j] = bs_e8m0_elem(a + (size_t)i * lda, b + (size_t)j * ldb, sfa, sfb, i, j, k,
                                                  sfa_sk, sfb_sn, mag ? mag + (size_t)i * ldc + j : NULL);
}

void ora_gemm_bs_e8m0_points(const uint8_t* a, const uint8_t* b, const uint8_t* sfa, const uint8_t* sfb,
                             int k, int lda, int ldb, int sfa_sk, int sfb_sn,
                             const int32_t* rows, const int32_t* cols, size_t np, float* out) {
    init_lut();
    #pragma omp parallel for schedule(static)
    for (size_t t = 0; t < np; ++t) {
        const int i = rows[t], j = cols[t];
        out[t] = bs_e8m0_elem(a + (size_t)i * lda, b + (size_t)j * ldb, sfa, sfb, i, j, k, sfa_sk, sfb_sn, NULL);
    }
}

/* ===================================================================== */
/* tolerance                                                              */
/* ===================================================================== */

double ora_rms(const float* x, size_t n) {
    double acc = 0.0;
    #pragma omp parallel for reduction(+ : acc) schedule(static)
    for (size_t i = 0; i < n; ++i) acc += (double)x[i] * (double)x[i];
    return n ? sqrt(acc / (double)n) : 0.0;
}

size_t ora_check_tolerance(const float* ref, const float* got, size_t n, double rms_override,
                           double* max_ratio, size_t* worst_index) {
    const double rms = rms_override > 0.0 ? rms_override : ora_rms(ref, n);
    size_t bad = 0, worst = 0;
    double worst_ratio = 0.0;
    for (size_t i = 0; i < n; ++i) {
        const double r = ref[i], g = got[i];
        const double bound = 0x1p-7 * fabs(r) + 1e-3 * rms;
        const double d = fabs(g - r);
        double ratio;
        if (!isfinite(g) || !isfinite(r)) ratio = INFINITY;
        else ratio = bound > 0.0 ? d / bound : (d == 0.0 ? 0.0 : INFINITY);
        if (!(ratio <= 1.0)) ++bad;
        if (!(ratio <= worst_ratio)) { worst_ratio = ratio; worst = i; }
    }
    if (max_ratio) *max_ratio = worst_ratio;
    if (worst_index) *worst_index = worst;
    return bad;
}

int ora_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
