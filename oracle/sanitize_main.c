/*
 * TEST INFRASTRUCTURE ONLY: a driver that runs the C oracle
 * (kivi_oracle.c) under AddressSanitizer and UndefinedBehaviorSanitizer on
 * the host (`make -C oracle sanitize`, run by tests/test_oracle_sanitize.py).
 * It sweeps group sizes and group counts (ragged tails included) over
 * inputs with NaN, +-inf, denormals, +-0 and huge values, checks that every
 * buffer is written exactly within its bounds (guard words around each
 * output), and that the round-trip equals quantise followed by dequantise.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

void kivi_oracle_quantize_groups(const float* in, uint8_t* packed, float* scales, float* zeros,
                                 int64_t n_groups, int32_t G);
void kivi_oracle_dequantize_groups(const uint8_t* packed, const float* scales,
                                   const float* zeros, float* out, int64_t n_groups, int32_t G);
void kivi_oracle_roundtrip_groups(const float* in, float* out, int64_t n_groups, int32_t G);
int64_t kivi_oracle_count_ties(const float* in, int64_t n_groups, int32_t G);

static uint32_t rng_state = 12345u;
static uint32_t rnd(void) {
    rng_state ^= rng_state << 13;
    rng_state ^= rng_state >> 17;
    rng_state ^= rng_state << 5;
    return rng_state;
}

static float sample(void) {
    switch (rnd() % 16) {
        case 0: return NAN;
        case 1: return (rnd() & 1) ? INFINITY : -INFINITY;
        case 2: return (rnd() & 1) ? 1e-42f : -1e-42f;        /* denormal */
        case 3: return (rnd() & 1) ? 0.0f : -0.0f;
        case 4: return (rnd() & 1) ? 3e38f : -3e38f;
        default: return ((float)(rnd() % 2001) - 1000.0f) / 64.0f;
    }
}

int main(void) {
    static const int sizes[] = {4, 8, 12, 16, 20, 32, 64, 96, 128, 256};
    const uint32_t guard = 0xdeadbeefu;
    int failures = 0;
    for (size_t si = 0; si < sizeof(sizes) / sizeof(sizes[0]); ++si) {
        const int G = sizes[si];
        for (int64_t n = 1; n <= 37; n += 9) {
            const int64_t N = n * G;
            float* in = malloc(N * sizeof(float));
            /* one guard word after each output */
            uint8_t* packed = malloc(N / 4 + 4);
            float* scales = malloc((n + 1) * sizeof(float));
            float* zeros = malloc((n + 1) * sizeof(float));
            float* deq = malloc((N + 1) * sizeof(float));
            float* rt = malloc((N + 1) * sizeof(float));
            for (int64_t i = 0; i < N; ++i) in[i] = sample();
            memcpy(packed + N / 4, &guard, 4);
            memcpy(scales + n, &guard, 4);
            memcpy(zeros + n, &guard, 4);
            memcpy(deq + N, &guard, 4);
            memcpy(rt + N, &guard, 4);
            kivi_oracle_quantize_groups(in, packed, scales, zeros, n, G);
            kivi_oracle_dequantize_groups(packed, scales, zeros, deq, n, G);
            kivi_oracle_roundtrip_groups(in, rt, n, G);
            (void)kivi_oracle_count_ties(in, n, G);
            if (memcmp(packed + N / 4, &guard, 4) || memcmp(scales + n, &guard, 4) ||
                memcmp(zeros + n, &guard, 4) || memcmp(deq + N, &guard, 4) ||
                memcmp(rt + N, &guard, 4)) {
                printf("G=%d n=%lld: a guard word was overwritten\n", G, (long long)n);
                ++failures;
            }
            if (memcmp(deq, rt, N * sizeof(float))) {
                printf("G=%d n=%lld: round-trip differs from quantise + dequantise\n", G,
                       (long long)n);
                ++failures;
            }
            free(in); free(packed); free(scales); free(zeros); free(deq); free(rt);
        }
    }
    printf("%s\n", failures ? "FAILED" : "sanitized oracle run: ok");
    return failures != 0;
}
