/*
 * f16c_check.c — TEST INFRASTRUCTURE ONLY: pins the oracle's binary16
 * conversions against the host CPU's F16C instructions (vcvtps2ph with
 * round-to-nearest-even, vcvtph2ps), an implementation independent of
 * rq_oracle.c. Compiled with -mf16c on its own.
 */
#include <immintrin.h>
#include <stdint.h>
#include <string.h>

#include "rq_oracle.h"

/* Mismatches of orq_f32_to_f16 over the 2^32 f32 bit patterns in
 * [lo, hi) (hi <= 2^32); the first mismatching pattern goes to *first_bad. */
int64_t orq_check_f32_to_f16_range(uint64_t lo, uint64_t hi, int64_t* first_bad) {
    int64_t bad = 0;
    int64_t first = -1;
#pragma omp parallel for schedule(static) reduction(+ : bad)
    for (int64_t i = (int64_t)lo; i < (int64_t)hi; i++) {
        uint32_t u = (uint32_t)i;
        float f;
        memcpy(&f, &u, 4);
        const uint16_t want = (uint16_t)_cvtss_sh(f, _MM_FROUND_TO_NEAREST_INT);
        if (orq_f32_to_f16(f) != want) {
            bad++;
#pragma omp critical
            if (first < 0 || i < first) first = i;
        }
    }
    if (first_bad) *first_bad = first;
    return bad;
}

/* Mismatches of orq_f16_to_f32 (compared bitwise) over all 2^16 patterns. */
int64_t orq_check_f16_to_f32_all(int64_t* first_bad) {
    int64_t bad = 0;
    int64_t first = -1;
    for (uint32_t h = 0; h < 65536u; h++) {
        const float want = _cvtsh_ss((unsigned short)h);
        const float got = orq_f16_to_f32((uint16_t)h);
        uint32_t a, b;
        memcpy(&a, &want, 4);
        memcpy(&b, &got, 4);
        if (a != b) {
            if (first < 0) first = h;
            bad++;
        }
    }
    if (first_bad) *first_bad = first;
    return bad;
}
