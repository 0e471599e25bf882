/*
 * TEST INFRASTRUCTURE ONLY -- never linked into, imported by, or called from
 * the product (intel_kivi_hybrid_amd/).  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load this library, and only as the
 * checker / CPU baseline.
 *
 * CPU restatement of the reference's KIVI 2-bit asymmetric codec, read as IEEE
 * fp32 (built with -ffp-contract=off, no fast-math):
 *
 *   min/max   : reference src/csrc/kernels/internal/quant_tile.hpp:35-49
 *               (init min=1e30f, max=-1e30f; fmin/fmax ignore NaN)
 *   scale/zero: src/csrc/kernels/quantize_kernels.cpp:46-48 and :98-100
 *               scale = (max-min)/3.0f + 1e-10f (stored with the epsilon),
 *               zero = min
 *   pack      : quant_tile.hpp:53-70
 *               q = clamp((int)round((x-min)/scale), 0, 3), round() is
 *               half-away-from-zero; element 4j+k -> byte j bits 2k..2k+1
 *   dequant   : src/csrc/kernels/dequantize_kernels.cpp:17-28
 *               x = (float)q * scale + zero, product and sum rounded
 *               separately (no fused multiply-add)
 *   round-trip: quant_tile.hpp:74-91, roundtrip_kernels.cpp:14-80
 *
 * Keys (per channel, grouped along tokens, quantize_kernels.cpp:24-54) and
 * values (per token, grouped along channels, quantize_kernels.cpp:69-106) both
 * reduce contiguous runs of `group_size` floats and write group g's packed
 * bytes at g*group_size/4 (values: out_base = token*D/4 + gi*G/4 = g*G/4), so
 * one flat-group routine covers both.
 *
 * Points the reference leaves open, fixed here and matched by the HIP kernels:
 *   - (int)round(NaN) is undefined in C++; a NaN quotient gives code 0.
 *   - fmin/fmax of -0.0 and +0.0 may return either; here -0.0 < +0.0.
 *   - indices are 64-bit (the reference uses int, kv_cache_ops.cpp:187).
 *
 * Parity pins (tests/test_oracle.py): known answers from the reference tests
 * (tests/integration/test_kivi.py:160-196 -> packed 228; test_kivi.py:256-278
 * and test_roundtrip_kernels.py:79-87 -> constant 5.0), the torch mirror of
 * tests/unit/test_manager_bookkeeping.py:54-66 on tie-free inputs, the tie
 * fixture [0,0.5,2.5,3] -> 244, exhaustive brute force over small groups,
 * and the bound |x - x_hat| <= scale/2.
 */
#include <math.h>
#include <stdint.h>
#include <stddef.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* fmin/fmax with NaN ignored and -0.0 ordered below +0.0. */
static inline float kv_min(float a, float b) {
    if (isnan(a)) return b;
    if (isnan(b)) return a;
    if (a == b) return signbit(a) ? a : b;
    return a < b ? a : b;
}

static inline float kv_max(float a, float b) {
    if (isnan(a)) return b;
    if (isnan(b)) return a;
    if (a == b) return signbit(a) ? b : a;
    return a > b ? a : b;
}

/* quant_tile.hpp:35-49: one group's min/max, float4 at a time. */
static void group_min_max(const float* x, int G, float* mn_out, float* mx_out) {
    float mn = 1e30f, mx = -1e30f;
    for (int i = 0; i < G; i += 4) {
        float lmax = kv_max(kv_max(x[i], x[i + 1]), kv_max(x[i + 2], x[i + 3]));
        float lmin = kv_min(kv_min(x[i], x[i + 1]), kv_min(x[i + 2], x[i + 3]));
        mx = kv_max(mx, lmax);
        mn = kv_min(mn, lmin);
    }
    *mn_out = mn;
    *mx_out = mx;
}

/* quantize_kernels.cpp:46 */
static inline float group_scale(float mn, float mx) {
    return (mx - mn) / 3.0f + 1e-10f;
}

/* quant_tile.hpp:63-66 */
static inline int code_of(float x, float mn, float scale) {
    float t = (x - mn) / scale;
    if (isnan(t)) return 0;
    int q = (int)roundf(t);
    if (q < 0) q = 0;
    if (q > 3) q = 3;
    return q;
}

/* dequantize_kernels.cpp:24 */
static inline float decode(int q, float scale, float zero) {
    return (float)q * scale + zero;   /* -ffp-contract=off: two roundings */
}

void kivi_oracle_quantize_groups(const float* in, uint8_t* packed, float* scales,
                                 float* zeros, int64_t n_groups, int32_t G) {
    #pragma omp parallel for schedule(static)
    for (int64_t g = 0; g < n_groups; ++g) {
        const float* x = in + g * (int64_t)G;
        float mn, mx;
        group_min_max(x, G, &mn, &mx);
        float s = group_scale(mn, mx);
        scales[g] = s;
        zeros[g] = mn;
        uint8_t* out = packed + g * (int64_t)(G / 4);
        for (int j = 0; j < G / 4; ++j) {
            unsigned b = 0;
            for (int k = 0; k < 4; ++k)
                b |= (unsigned)code_of(x[4 * j + k], mn, s) << (2 * k);
            out[j] = (uint8_t)b;
        }
    }
}

void kivi_oracle_dequantize_groups(const uint8_t* packed, const float* scales,
                                   const float* zeros, float* out,
                                   int64_t n_groups, int32_t G) {
    #pragma omp parallel for schedule(static)
    for (int64_t g = 0; g < n_groups; ++g) {
        const uint8_t* p = packed + g * (int64_t)(G / 4);
        float* o = out + g * (int64_t)G;
        for (int j = 0; j < G / 4; ++j)
            for (int k = 0; k < 4; ++k)
                o[4 * j + k] = decode((p[j] >> (2 * k)) & 3, scales[g], zeros[g]);
    }
}

void kivi_oracle_roundtrip_groups(const float* in, float* out, int64_t n_groups,
                                  int32_t G) {
    #pragma omp parallel for schedule(static)
    for (int64_t g = 0; g < n_groups; ++g) {
        const float* x = in + g * (int64_t)G;
        float mn, mx;
        group_min_max(x, G, &mn, &mx);
        float s = group_scale(mn, mx);
        for (int i = 0; i < G; ++i)
            out[g * (int64_t)G + i] = decode(code_of(x[i], mn, s), s, mn);
    }
}

/* Number of elements whose quotient (x-min)/scale is exactly k+0.5: there the
 * kernel's round-half-away and torch.round's half-to-even disagree. */
int64_t kivi_oracle_count_ties(const float* in, int64_t n_groups, int32_t G) {
    int64_t ties = 0;
    #pragma omp parallel for schedule(static) reduction(+:ties)
    for (int64_t g = 0; g < n_groups; ++g) {
        const float* x = in + g * (int64_t)G;
        float mn, mx;
        group_min_max(x, G, &mn, &mx);
        float s = group_scale(mn, mx);
        for (int i = 0; i < G; ++i) {
            float t = (x[i] - mn) / s;
            if (t == 0.5f || t == 1.5f || t == 2.5f) ++ties;
        }
    }
    return ties;
}

int kivi_oracle_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void kivi_oracle_set_num_threads(int n) {
#ifdef _OPENMP
    omp_set_num_threads(n);
#else
    (void)n;
#endif
}
