/*
 * CPU oracle for the quantized decode path — TEST INFRASTRUCTURE ONLY.
 * See qwn_oracle.h.  Built by oracle/Makefile with the reference's own
 * optimisation flags (c/Makefile:107-113) minus -march=native, so the same
 * shared object runs on any x86-64 host with AVX2/FMA/F16C; wider ISAs are
 * chosen at run time from CPUID.
 *
 * Floating-point order: every accumulation below is written with explicit
 * fmaf()/rounded products so that the result does not depend on the
 * compiler's contraction choices.  The order restates the reference as
 * compiled by GCC -O3 -mfma (which contracts `s += a*b` into one fma); the
 * tests compare the two bit for bit.
 */
#include "qwn_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#if defined(__x86_64__)
#include <cpuid.h>
#include <immintrin.h>
#endif

#if defined(_OPENMP)
#include <omp.h>
#endif

static int effective_threads(int threads) {
#if defined(_OPENMP)
    return threads > 0 ? threads : omp_get_max_threads();
#else
    (void)threads;
    return 1;
#endif
}

float qo_half_to_float(uint16_t h) {
    /* Rebuild the binary32 pattern field by field; a subnormal half is
     * normalised by shifting its mantissa up until the implicit bit
     * appears (c/qwanto_kernels.c:264-285). */
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exponent = (h >> 10) & 0x1fu;
    uint32_t mantissa = h & 0x3ffu;
    uint32_t bits;
    if (exponent == 0x1fu) {
        bits = sign | 0x7f800000u | (mantissa << 13);
    } else if (exponent != 0) {
        bits = sign | ((exponent + 112u) << 23) | (mantissa << 13);
    } else if (mantissa == 0) {
        bits = sign;
    } else {
        int e = 113; /* biased exponent of 2^-14 */
        while (!(mantissa & 0x400u)) {
            mantissa <<= 1;
            e--;
        }
        bits = sign | ((uint32_t)e << 23) | ((mantissa & 0x3ffu) << 13);
    }
    float out;
    memcpy(&out, &bits, sizeof(out));
    return out;
}

static inline float load_half(const uint8_t *p) {
    return qo_half_to_float((uint16_t)(p[0] | (p[1] << 8)));
}

/* ------------------------------------------------------------------ */
/* a1: per-token activation quantization                               */
/* ------------------------------------------------------------------ */

void qo_quantize_tokens(const float *x, int M, int K, int padded_k,
                        int8_t *q8, float *scales, int32_t *act_sums,
                        int sum_blocks) {
    for (int t = 0; t < M; t++) {
        const float *row = x + (size_t)t * K;
        int8_t *q = q8 + (size_t)t * padded_k;
        float amax = 0.0f;
        for (int k = 0; k < K; k++) {
            const float a = fabsf(row[k]);
            if (a > amax) amax = a;
        }
        /* division then reciprocal, as c/qwanto_kernels.c:385-386 */
        const float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
        const float inv = 1.0f / scale;
        scales[t] = scale;
        for (int k = 0; k < K; k++) {
            float v = row[k] * inv;
            v = v > 127.0f ? 127.0f : (v < -127.0f ? -127.0f : v);
            q[k] = (int8_t)lrintf(v); /* round-to-nearest-even */
        }
        for (int k = K; k < padded_k; k++) q[k] = 0;
        if (act_sums) {
            for (int b = 0; b < sum_blocks; b++) {
                int32_t s = 0;
                for (int i = b * 32; i < K && i < b * 32 + 32; i++) s += q[i];
                act_sums[(size_t)t * sum_blocks + b] = s;
            }
        }
    }
}

/* ------------------------------------------------------------------ */
/* a2/a3: Q4_0                                                          */
/* ------------------------------------------------------------------ */

int32_t qo_q4_0_block_raw(const uint8_t *blk, const int8_t *q8, int valid) {
    const uint8_t *nib = blk + 2;
    int32_t raw = 0;
    for (int i = 0; i < valid; i++) {
        const int code = (i & 1) ? (nib[i >> 1] >> 4) : (nib[i >> 1] & 0x0f);
        raw += (code - 8) * (int32_t)q8[i];
    }
    return raw;
}

#if defined(__x86_64__)
__attribute__((target("avx2")))
static int32_t q4_0_block_raw_avx2(const uint8_t *blk, const int8_t *q8) {
    /* nibbles -> 32 unsigned bytes in element order, then one maddubs with
     * the activations and one with ones; raw = sum(n*a) - 8*sum(a). */
    const __m128i packed = _mm_loadu_si128((const __m128i *)(blk + 2));
    const __m128i low_mask = _mm_set1_epi8(0x0f);
    const __m128i lo = _mm_and_si128(packed, low_mask);
    const __m128i hi = _mm_and_si128(_mm_srli_epi16(packed, 4), low_mask);
    const __m256i codes = _mm256_set_m128i(_mm_unpackhi_epi8(lo, hi),
                                           _mm_unpacklo_epi8(lo, hi));
    const __m256i act = _mm256_loadu_si256((const __m256i *)q8);
    const __m256i one16 = _mm256_set1_epi16(1);
    __m256i prod = _mm256_madd_epi16(_mm256_maddubs_epi16(codes, act), one16);
    __m256i asum = _mm256_madd_epi16(
        _mm256_maddubs_epi16(_mm256_set1_epi8(1), act), one16);
    __m256i diff = _mm256_sub_epi32(prod, _mm256_slli_epi32(asum, 3));
    __m128i s = _mm_add_epi32(_mm256_castsi256_si128(diff),
                              _mm256_extracti128_si256(diff, 1));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4e));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0xb1));
    return _mm_cvtsi128_si32(s);
}
#endif

static int cpu_has_avx2(void);

void qo_gemv_q4_0_q8(const uint8_t *w, const int8_t *q8, float x_scale,
                     int K, int N, float *y, int threads) {
    const int blocks = (K + 31) / 32;
    const size_t row_bytes = (size_t)blocks * 18;
    const int use_avx2 = cpu_has_avx2();
#if defined(_OPENMP)
    #pragma omp parallel for schedule(static) num_threads(effective_threads(threads)) if(N > 16)
#endif
    for (int n = 0; n < N; n++) {
        const uint8_t *row = w + (size_t)n * row_bytes;
        float sum = 0.0f;
        for (int b = 0; b < blocks; b++) {
            const int valid = K - b * 32 < 32 ? K - b * 32 : 32;
            const uint8_t *blk = row + (size_t)b * 18;
            int32_t raw;
#if defined(__x86_64__)
            if (use_avx2 && valid == 32) raw = q4_0_block_raw_avx2(blk, q8 + b * 32);
            else
#endif
                raw = qo_q4_0_block_raw(blk, q8 + b * 32, valid);
            /* dot = (float)raw * d is returned rounded by the block
             * function; the row loop then does sum += dot * x_scale. */
            const float dot = (float)raw * load_half(blk);
            sum = fmaf(dot, x_scale, sum);
        }
        y[n] = sum;
    }
}

int qo_matmul_q4_0(const uint8_t *w, const float *x, int M, int K, int N,
                   float *y, int threads) {
    if (!w || !x || !y || M < 1 || K < 1 || N < 1) return -1;
    const int padded = (K + 255) & ~255;
    int8_t *q8 = (int8_t *)calloc((size_t)M * padded, 1);
    float *scales = (float *)malloc((size_t)M * sizeof(float));
    if (!q8 || !scales) {
        free(q8);
        free(scales);
        return -1;
    }
    qo_quantize_tokens(x, M, K, padded, q8, scales, NULL, 0);
    for (int t = 0; t < M; t++)
        qo_gemv_q4_0_q8(w, q8 + (size_t)t * padded, scales[t], K, N,
                        y + (size_t)t * N, threads);
    free(q8);
    free(scales);
    return 0;
}

void qo_q4_0_block_sums(const uint8_t *w, const int8_t *q8, int K, int N,
                        int32_t *raw) {
    const int blocks = (K + 31) / 32;
    const size_t row_bytes = (size_t)blocks * 18;
    for (int n = 0; n < N; n++)
        for (int b = 0; b < blocks; b++) {
            const int valid = K - b * 32 < 32 ? K - b * 32 : 32;
            raw[(size_t)n * blocks + b] = qo_q4_0_block_raw(
                w + (size_t)n * row_bytes + (size_t)b * 18, q8 + b * 32, valid);
        }
}

/* ------------------------------------------------------------------ */
/* a4/a5: HyperVSQ-2                                                    */
/* ------------------------------------------------------------------ */

/* Block layout (c/qwanto_native.h:96-103): [0,2) fp16 d_base, [2,4) fp16
 * m_base, [4,8) eight 4-bit octant multipliers (low nibble = even octant),
 * [8,10) reserved, [10,74) codes: octant o at 10+8o, element i of the
 * octant in byte i/4 at bit 2*(i%4); weight = (code-1)*d*s/8 + m. */
static inline int hvsq2_code(const uint8_t *blk, int oct, int i) {
    return (blk[10 + oct * 8 + (i >> 2)] >> ((i & 3) * 2)) & 3;
}

static inline float hvsq2_eff_scale(const uint8_t *blk, int oct) {
    const uint8_t sb = blk[4 + (oct >> 1)];
    const int s = (oct & 1) ? (sb >> 4) : (sb & 0x0f);
    return load_half(blk) * ((float)s * (1.0f / 8.0f));
}

void qo_gemv_hvsq2_scalar(const uint8_t *w, const int8_t *q8,
                          const int32_t *act_sums, float x_scale, int K,
                          int N, size_t row_bytes, float *out) {
    const int blocks = (K + 255) / 256;
    for (int n = 0; n < N; n++) {
        const uint8_t *row = w + (size_t)n * row_bytes;
        float row_sum = 0.0f;
        for (int b = 0; b < blocks; b++) {
            const uint8_t *blk = row + (size_t)b * 74;
            const int valid = K - b * 256 < 256 ? K - b * 256 : 256;
            const float offset = load_half(blk + 2);
            for (int oct = 0; oct < 8 && oct * 32 < valid; oct++) {
                const int cap = valid - oct * 32 < 32 ? valid - oct * 32 : 32;
                const int base = b * 256 + oct * 32;
                int32_t sum_q = 0;
                int32_t sum_a = act_sums ? act_sums[b * 8 + oct] : 0;
                for (int i = 0; i < cap; i++) {
                    sum_q += (hvsq2_code(blk, oct, i) - 1) * (int32_t)q8[base + i];
                    if (!act_sums) sum_a += q8[base + i];
                }
                const float eff = hvsq2_eff_scale(blk, oct);
                /* row_sum += sq*(eff*xs) + sa*(off*xs): GCC forms
                 * fma(sq, eff*xs, sa*(off*xs)) and then adds row_sum. */
                row_sum += fmaf((float)sum_q, eff * x_scale,
                                (float)sum_a * (offset * x_scale));
            }
        }
        out[n] = row_sum;
    }
}

/* Per-lane integer partials of one full octant: lane j holds
 * sum_{e=4j..4j+3} (code_e - 1) * a_e (what dpbusd(codes, a) minus
 * dpbusd(1, a) leaves in each int32 lane). */
static inline void octant_lane_sums_c(const uint8_t *codes, const int8_t *a,
                                      int32_t lanes[8]) {
    for (int j = 0; j < 8; j++) {
        int32_t s = 0;
        for (int e = 4 * j; e < 4 * j + 4; e++)
            s += (((codes[e >> 2] >> ((e & 3) * 2)) & 3) - 1) * (int32_t)a[e];
        lanes[j] = s;
    }
}

#if defined(__x86_64__)
/* 8 code bytes -> 32 bytes holding one 2-bit code each, element order.
 * Code byte e>>2 is replicated into the 4 bytes of a dword; byte i of the
 * dword then takes bits 2i..2i+1 of it: four uniform shifts and masks. */
__attribute__((target("avx2")))
static inline __m256i expand_codes_avx2(const uint8_t *codes) {
    uint64_t raw;
    memcpy(&raw, codes, 8);
    const __m256i src = _mm256_set1_epi64x((long long)raw);
    const __m256i rep = _mm256_shuffle_epi8(
        src, _mm256_setr_epi8(0, 0, 0, 0, 1, 1, 1, 1, 2, 2, 2, 2, 3, 3, 3, 3,
                              4, 4, 4, 4, 5, 5, 5, 5, 6, 6, 6, 6, 7, 7, 7, 7));
    const __m256i s0 = rep;
    const __m256i s2 = _mm256_srli_epi16(rep, 2);
    const __m256i s4 = _mm256_srli_epi32(rep, 4);
    const __m256i s6 = _mm256_srli_epi32(rep, 6);
    const __m256i m0 = _mm256_set1_epi32(0x00000003);
    const __m256i m1 = _mm256_set1_epi32(0x00000300);
    const __m256i m2 = _mm256_set1_epi32(0x00030000);
    const __m256i m3 = _mm256_set1_epi32(0x03000000);
    return _mm256_or_si256(
        _mm256_or_si256(_mm256_and_si256(s0, m0), _mm256_and_si256(s2, m1)),
        _mm256_or_si256(_mm256_and_si256(s4, m2), _mm256_and_si256(s6, m3)));
}

/* codes x a minus a, per int32 lane; maddubs pairs stay far from int16
 * saturation because codes are at most 3 and |a| <= 127. */
__attribute__((target("avx2")))
static inline __m256i octant_lanes_avx2(const uint8_t *codes, const int8_t *a) {
    const __m256i c = expand_codes_avx2(codes);
    const __m256i act = _mm256_loadu_si256((const __m256i *)a);
    const __m256i one16 = _mm256_set1_epi16(1);
    const __m256i ca = _mm256_madd_epi16(_mm256_maddubs_epi16(c, act), one16);
    const __m256i aa = _mm256_madd_epi16(
        _mm256_maddubs_epi16(_mm256_set1_epi8(1), act), one16);
    return _mm256_sub_epi32(ca, aa);
}

__attribute__((target("avx2,avxvnni")))
static inline __m256i octant_lanes_avxvnni(const uint8_t *codes, const int8_t *a) {
    const __m256i c = expand_codes_avx2(codes);
    const __m256i act = _mm256_loadu_si256((const __m256i *)a);
    const __m256i zero = _mm256_setzero_si256();
    return _mm256_sub_epi32(_mm256_dpbusd_avx_epi32(zero, c, act),
                            _mm256_dpbusd_avx_epi32(zero, _mm256_set1_epi8(1), act));
}

__attribute__((target("avx2,avx512vnni,avx512vl")))
static inline __m256i octant_lanes_avx512vnni(const uint8_t *codes, const int8_t *a) {
    const __m256i c = expand_codes_avx2(codes);
    const __m256i act = _mm256_loadu_si256((const __m256i *)a);
    const __m256i zero = _mm256_setzero_si256();
    return _mm256_sub_epi32(_mm256_dpbusd_epi32(zero, c, act),
                            _mm256_dpbusd_epi32(zero, _mm256_set1_epi8(1), act));
}

#define DEFINE_DELAYED_SIMD(NAME, TARGET, LANES_FN)                                \
    __attribute__((target(TARGET))) static void NAME(                             \
        const uint8_t *w, const int8_t *q8, const int32_t *act_sums,              \
        float x_scale, int K, int N, size_t row_bytes, float *out) {              \
        const int blocks = (K + 255) / 256;                                       \
        for (int n = 0; n < N; n++) {                                             \
            const uint8_t *row = w + (size_t)n * row_bytes;                       \
            __m256 lanes = _mm256_setzero_ps();                                   \
            float offset_sum = 0.0f;                                              \
            for (int b = 0; b < blocks; b++) {                                    \
                const uint8_t *blk = row + (size_t)b * 74;                        \
                const int valid = K - b * 256 < 256 ? K - b * 256 : 256;          \
                const float offset = load_half(blk + 2);                          \
                const int full = valid / 32;                                      \
                for (int oct = 0; oct < full; oct++) {                            \
                    const int base = b * 256 + oct * 32;                          \
                    const __m256i d = LANES_FN(blk + 10 + oct * 8, q8 + base);    \
                    const __m256 es = _mm256_set1_ps(hvsq2_eff_scale(blk, oct) * x_scale); \
                    lanes = _mm256_fmadd_ps(_mm256_cvtepi32_ps(d), es, lanes);    \
                    int32_t sa;                                                   \
                    if (act_sums) sa = act_sums[b * 8 + oct];                     \
                    else {                                                        \
                        sa = 0;                                                   \
                        for (int i = 0; i < 32; i++) sa += q8[base + i];          \
                    }                                                             \
                    offset_sum = fmaf((float)sa, offset * x_scale, offset_sum);   \
                }                                                                 \
                for (int oct = full; oct < 8 && oct * 32 < valid; oct++) {        \
                    const int cap = valid - oct * 32 < 32 ? valid - oct * 32 : 32; \
                    const int base = b * 256 + oct * 32;                          \
                    int32_t sq = 0;                                               \
                    int32_t sa = act_sums ? act_sums[b * 8 + oct] : 0;            \
                    for (int i = 0; i < cap; i++) {                               \
                        sq += (hvsq2_code(blk, oct, i) - 1) * (int32_t)q8[base + i]; \
                        if (!act_sums) sa += q8[base + i];                        \
                    }                                                             \
                    offset_sum += fmaf((float)sq, hvsq2_eff_scale(blk, oct) * x_scale, \
                                       (float)sa * (offset * x_scale));           \
                }                                                                 \
            }                                                                     \
            float l[8];                                                           \
            _mm256_storeu_ps(l, lanes);                                           \
            out[n] = offset_sum + l[0] + l[1] + l[2] + l[3] + l[4] + l[5] + l[6] + l[7]; \
        }                                                                         \
    }

DEFINE_DELAYED_SIMD(delayed_avx2, "avx2,fma", octant_lanes_avx2)
DEFINE_DELAYED_SIMD(delayed_avxvnni, "avx2,fma,avxvnni", octant_lanes_avxvnni)
DEFINE_DELAYED_SIMD(delayed_avx512vnni, "avx2,fma,avx512vnni,avx512vl", octant_lanes_avx512vnni)
#endif

static void delayed_c(const uint8_t *w, const int8_t *q8,
                      const int32_t *act_sums, float x_scale, int K, int N,
                      size_t row_bytes, float *out) {
    const int blocks = (K + 255) / 256;
    for (int n = 0; n < N; n++) {
        const uint8_t *row = w + (size_t)n * row_bytes;
        float lanes[8] = {0};
        float offset_sum = 0.0f;
        for (int b = 0; b < blocks; b++) {
            const uint8_t *blk = row + (size_t)b * 74;
            const int valid = K - b * 256 < 256 ? K - b * 256 : 256;
            const float offset = load_half(blk + 2);
            const int full = valid / 32;
            for (int oct = 0; oct < full; oct++) {
                const int base = b * 256 + oct * 32;
                int32_t d[8];
                octant_lane_sums_c(blk + 10 + oct * 8, q8 + base, d);
                const float es = hvsq2_eff_scale(blk, oct) * x_scale;
                for (int j = 0; j < 8; j++) lanes[j] = fmaf((float)d[j], es, lanes[j]);
                int32_t sa = 0;
                if (act_sums) sa = act_sums[b * 8 + oct];
                else for (int i = 0; i < 32; i++) sa += q8[base + i];
                offset_sum = fmaf((float)sa, offset * x_scale, offset_sum);
            }
            for (int oct = full; oct < 8 && oct * 32 < valid; oct++) {
                const int cap = valid - oct * 32 < 32 ? valid - oct * 32 : 32;
                const int base = b * 256 + oct * 32;
                int32_t sq = 0;
                int32_t sa = act_sums ? act_sums[b * 8 + oct] : 0;
                for (int i = 0; i < cap; i++) {
                    sq += (hvsq2_code(blk, oct, i) - 1) * (int32_t)q8[base + i];
                    if (!act_sums) sa += q8[base + i];
                }
                offset_sum += fmaf((float)sq, hvsq2_eff_scale(blk, oct) * x_scale,
                                   (float)sa * (offset * x_scale));
            }
        }
        out[n] = offset_sum + lanes[0] + lanes[1] + lanes[2] + lanes[3] +
                 lanes[4] + lanes[5] + lanes[6] + lanes[7];
    }
}

/* ---- CPU feature detection (CPUID leaf 7 and XCR0) ---------------- */

static int g_features = -1; /* bit0 avx2+fma+f16c, bit1 avxvnni, bit2 avx512vnni+vl */

static int detect_features(void) {
    if (g_features >= 0) return g_features;
    int f = 0;
#if defined(__x86_64__)
    unsigned a, b, c, d;
    if (__get_cpuid(1, &a, &b, &c, &d)) {
        const int osxsave = (c >> 27) & 1, avx = (c >> 28) & 1;
        const int fma = (c >> 12) & 1, f16c = (c >> 29) & 1;
        unsigned xlo = 0, xhi = 0;
        if (osxsave) __asm__ volatile("xgetbv" : "=a"(xlo), "=d"(xhi) : "c"(0));
        const int ymm_ok = osxsave && avx && (xlo & 6u) == 6u;
        const int zmm_ok = ymm_ok && (xlo & 0xe0u) == 0xe0u;
        if (__get_cpuid_count(7, 0, &a, &b, &c, &d)) {
            const int avx2 = (b >> 5) & 1;
            const int avx512f = (b >> 16) & 1, avx512vl = (b >> 31) & 1;
            const int avx512vnni = (c >> 11) & 1;
            if (ymm_ok && avx2 && fma && f16c) f |= 1;
            if ((f & 1) && zmm_ok && avx512f && avx512vl && avx512vnni) f |= 4;
            if ((f & 1) && __get_cpuid_count(7, 1, &a, &b, &c, &d) && ((a >> 4) & 1))
                f |= 2;
        }
    }
#endif
    g_features = f;
    return f;
}

static int cpu_has_avx2(void) { return detect_features() & 1; }

int qo_hvsq2_best_variant(void) {
    const int f = detect_features();
    if (f & 2) return 2;
    if (f & 4) return 3;
    if (f & 1) return 1;
    return 0;
}

const char *qo_variant_name(int variant) {
    switch (variant) {
    case -2: return "scalar-golden";
    case 0: return "delayed-c";
    case 1: return "delayed-avx2";
    case 2: return "delayed-avxvnni";
    case 3: return "delayed-avx512vnni";
    default: return "unknown";
    }
}

void qo_gemv_hvsq2_delayed(const uint8_t *w, const int8_t *q8,
                           const int32_t *act_sums, float x_scale, int K,
                           int N, size_t row_bytes, float *out, int variant) {
    if (variant < 0) variant = qo_hvsq2_best_variant();
    const int f = detect_features();
#if defined(__x86_64__)
    if (variant == 2 && (f & 2)) {
        delayed_avxvnni(w, q8, act_sums, x_scale, K, N, row_bytes, out);
        return;
    }
    if (variant == 3 && (f & 4)) {
        delayed_avx512vnni(w, q8, act_sums, x_scale, K, N, row_bytes, out);
        return;
    }
    if (variant == 1 && (f & 1)) {
        delayed_avx2(w, q8, act_sums, x_scale, K, N, row_bytes, out);
        return;
    }
#endif
    (void)f;
    delayed_c(w, q8, act_sums, x_scale, K, N, row_bytes, out);
}

int qo_matmul_hvsq2(const uint8_t *w, const float *x, int M, int K, int N,
                    float *y, int threads, int variant) {
    if (!w || !x || !y || M < 1 || K < 1 || N < 1) return -1;
    const int padded = (K + 255) & ~255;
    const int sum_blocks = padded / 32;
    const int blocks = (K + 255) / 256;
    const size_t row_bytes = (size_t)blocks * 74;
    int8_t *q8 = (int8_t *)calloc((size_t)M * padded, 1);
    float *scales = (float *)malloc((size_t)M * sizeof(float));
    int32_t *sums = (int32_t *)malloc((size_t)M * sum_blocks * sizeof(int32_t));
    if (!q8 || !scales || !sums) {
        free(q8);
        free(scales);
        free(sums);
        return -1;
    }
    qo_quantize_tokens(x, M, K, padded, q8, scales, sums, sum_blocks);
    if (variant == -1) variant = qo_hvsq2_best_variant();
    for (int t = 0; t < M; t++) {
        const int8_t *qt = q8 + (size_t)t * padded;
        const int32_t *st = sums + (size_t)t * sum_blocks;
        float *yt = y + (size_t)t * N;
#if defined(_OPENMP)
        #pragma omp parallel for schedule(static) num_threads(effective_threads(threads)) if(N > 16)
#endif
        for (int n = 0; n < N; n += 64) {
            const int chunk = N - n < 64 ? N - n : 64;
            if (variant == -2)
                qo_gemv_hvsq2_scalar(w + (size_t)n * row_bytes, qt, st, scales[t], K,
                                     chunk, row_bytes, yt + n);
            else
                qo_gemv_hvsq2_delayed(w + (size_t)n * row_bytes, qt, st, scales[t], K,
                                      chunk, row_bytes, yt + n, variant);
        }
    }
    free(q8);
    free(scales);
    free(sums);
    return 0;
}

void qo_hvsq2_octant_sums(const uint8_t *w, const int8_t *q8, int K, int N,
                          int32_t *sum_q, int32_t *sum_a) {
    const int blocks = (K + 255) / 256;
    const size_t row_bytes = (size_t)blocks * 74;
    for (int b = 0; b < blocks; b++)
        for (int oct = 0; oct < 8; oct++) {
            int32_t s = 0;
            for (int i = 0; i < 32; i++) {
                const int e = b * 256 + oct * 32 + i;
                if (e < K) s += q8[e];
            }
            sum_a[b * 8 + oct] = s;
        }
    for (int n = 0; n < N; n++) {
        const uint8_t *row = w + (size_t)n * row_bytes;
        for (int b = 0; b < blocks; b++)
            for (int oct = 0; oct < 8; oct++) {
                int32_t s = 0;
                for (int i = 0; i < 32; i++) {
                    const int e = b * 256 + oct * 32 + i;
                    if (e < K) s += (hvsq2_code(row + (size_t)b * 74, oct, i) - 1) * (int32_t)q8[e];
                }
                sum_q[((size_t)n * blocks + b) * 8 + oct] = s;
            }
    }
}

/* ------------------------------------------------------------------ */
/* a6: F16 generic matmul                                              */
/* ------------------------------------------------------------------ */

float qo_bf16_to_float(uint16_t h) {
    const uint32_t bits = (uint32_t)h << 16;
    float f;
    memcpy(&f, &bits, sizeof(f));
    return f;
}

static void matmul_half(const uint16_t *w, int bf16, const float *x, int M, int K, int N, float *y,
                        int threads);

void qo_matmul_f16(const uint16_t *w, const float *x, int M, int K, int N,
                   float *y, int threads) {
    matmul_half(w, 0, x, M, K, N, y, threads);
}

void qo_matmul_bf16(const uint16_t *w, const float *x, int M, int K, int N,
                    float *y, int threads) {
    matmul_half(w, 1, x, M, K, N, y, threads);
}

/* Both 16-bit row formats: the row decoded to fp32, then the one loop. */
static void matmul_half(const uint16_t *w, int bf16, const float *x, int M, int K, int N, float *y,
                        int threads) {
#if defined(_OPENMP)
    #pragma omp parallel num_threads(effective_threads(threads))
#endif
    {
        float *row = (float *)malloc((size_t)K * sizeof(float));
#if defined(_OPENMP)
        #pragma omp for schedule(static)
#endif
        for (int n = 0; n < N; n++) {
            if (!row) continue;
            const uint16_t *src = w + (size_t)n * K;
            for (int k = 0; k < K; k++) row[k] = bf16 ? qo_bf16_to_float(src[k]) : qo_half_to_float(src[k]);
            for (int t = 0; t < M; t++) {
                const float *xr = x + (size_t)t * K;
                /* GCC vectorises the products (eight, then one four-wide
                 * step) and folds them in order without contraction, each
                 * product rounded first; the scalar remainder is
                 * contracted into fma. */
                float sum = 0.0f;
                int main_k = K & ~7;
                if (K - main_k >= 4) main_k += 4; /* one 4-wide epilogue step */
                for (int k = 0; k < main_k; k++) sum += xr[k] * row[k];
                for (int k = main_k; k < K; k++) sum = fmaf(xr[k], row[k], sum);
                y[(size_t)t * N + n] = sum;
            }
        }
        free(row);
    }
}

/* ------------------------------------------------------------------ */
/* a7: Q8 KV cache                                                      */
/* ------------------------------------------------------------------ */

static int8_t q8_round(float v) {
    if (!isfinite(v)) return 0;
    if (v >= 127.0f) return 127;
    if (v <= -127.0f) return -127;
    return (int8_t)lrintf(v);
}

void qo_q8_quantize_vector(const float *src, int8_t *dst, float *scales,
                           int n_channels) {
    const int groups = (n_channels + 63) / 64;
    for (int g = 0; g < groups; g++) {
        const int start = g * 64;
        const int count = n_channels - start < 64 ? n_channels - start : 64;
        float amax = 0.0f;
        for (int i = 0; i < count; i++)
            if (isfinite(src[start + i]) && fabsf(src[start + i]) > amax)
                amax = fabsf(src[start + i]);
        const float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
        scales[g] = scale;
        for (int i = 0; i < count; i++) dst[start + i] = q8_round(src[start + i] / scale);
    }
}

void qo_q8_attention_head(const float *query, const int8_t *keys,
                          const int8_t *values, const float *key_scales,
                          const float *value_scales, int n_channels,
                          int head_dim, int kv_head, int pos, float scale,
                          float *scores, float *ctx) {
    const int groups = (n_channels + 63) / 64;
    const int offset = kv_head * head_dim;
    for (int t = 0; t <= pos; t++) {
        const int8_t *k = keys + (size_t)t * n_channels;
        const float *ks = key_scales + (size_t)t * groups;
        float dot = 0.0f;
        for (int i = 0; i < head_dim; i++) {
            const int ch = offset + i;
            dot = fmaf(query[i], (float)k[ch] * ks[ch / 64], dot);
        }
        scores[t] = dot * scale;
    }
    float max_score = scores[0];
    for (int t = 1; t <= pos; t++)
        if (scores[t] > max_score) max_score = scores[t];
    float sum = 0.0f;
    for (int t = 0; t <= pos; t++) {
        scores[t] = expf(scores[t] - max_score);
        sum += scores[t];
    }
    const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
    for (int i = 0; i < head_dim; i++) ctx[i] = 0.0f;
    for (int t = 0; t <= pos; t++) {
        const int8_t *v = values + (size_t)t * n_channels;
        const float *vs = value_scales + (size_t)t * groups;
        const float p = scores[t] * inv;
        for (int i = 0; i < head_dim; i++) {
            const int ch = offset + i;
            ctx[i] = fmaf(p, (float)v[ch] * vs[ch / 64], ctx[i]);
        }
    }
}

void qo_q8_attention(const float *query, const int8_t *keys,
                     const int8_t *values, const float *key_scales,
                     const float *value_scales, int query_heads, int kv_heads,
                     int head_dim, int pos, float scale, float *out,
                     int threads) {
    const int n_channels = kv_heads * head_dim;
    const float ratio = (float)query_heads / (float)kv_heads;
#if defined(_OPENMP)
    #pragma omp parallel num_threads(effective_threads(threads))
#endif
    {
        float *scores = (float *)malloc((size_t)(pos + 1) * sizeof(float));
#if defined(_OPENMP)
        #pragma omp for schedule(static)
#endif
        for (int h = 0; h < query_heads; h++) {
            if (!scores) continue;
            const int kh = (int)((float)h / ratio);
            qo_q8_attention_head(query + (size_t)h * head_dim, keys, values,
                                 key_scales, value_scales, n_channels, head_dim,
                                 kh, pos, scale, scores, out + (size_t)h * head_dim);
        }
        free(scores);
    }
}

/* The GPU ABI's head mapping, kv_head = head * kv_heads / query_heads for
 * any ratio (c/cuda/qwn_hypervsq2_cuda_abi.cu:184); for query heads that
 * are a multiple of the KV heads it equals the decoder's mapping above. */
void qo_q8_attention_abi(const float *query, const int8_t *keys,
                         const int8_t *values, const float *key_scales,
                         const float *value_scales, int query_heads, int kv_heads,
                         int head_dim, int pos, float scale, float *out) {
    const int n_channels = kv_heads * head_dim;
    float *scores = (float *)malloc((size_t)(pos + 1) * sizeof(float));
    if (!scores) return;
    for (int h = 0; h < query_heads; h++) {
        const int kh = (int)(((long long)h * kv_heads) / query_heads);
        qo_q8_attention_head(query + (size_t)h * head_dim, keys, values,
                             key_scales, value_scales, n_channels, head_dim,
                             kh, pos, scale, scores, out + (size_t)h * head_dim);
    }
    free(scores);
}
