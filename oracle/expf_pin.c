/* expf_pin.c — TEST INFRASTRUCTURE ONLY: compiles the library's device expf
 * (mynah-slm_amd/csrc/mynah_expf.h) for the host and compares it, bit for
 * bit, with the C library's expf (the one the reference's f32 operators
 * call) over ranges of floats, on several threads.
 *
 * SPDX-License-Identifier: MIT */
#define _GNU_SOURCE
#include "../mynah-slm_amd/csrc/mynah_expf.h"

#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <string.h>

float orc_mynah_expf(float x) { return mynah_expf(x); }

typedef struct {
    uint64_t lo, hi, step, bad, tested;
    uint32_t first_bad;
} span;

static void *sweep(void *arg) {
    span *s = (span *)arg;
    for (uint64_t u = s->lo; u < s->hi; u += s->step) {
        const uint32_t w = (uint32_t)u;
        float x, a, b;
        memcpy(&x, &w, 4);
        if (x != x) continue;
        a = mynah_expf(x);
        b = expf(x);
        s->tested++;
        if (memcmp(&a, &b, 4) != 0) {
            if (s->bad == 0) s->first_bad = w;
            s->bad++;
        }
    }
    return NULL;
}

/* Every step-th bit pattern in [lo, hi) (NaNs skipped), over `threads`
 * threads; returns the mismatch count, *first the first mismatching bits. */
uint64_t orc_expf_sweep(uint64_t lo, uint64_t hi, uint64_t step, int threads, uint64_t *tested,
                        uint32_t *first) {
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    span sp[64];
    pthread_t th[64];
    const uint64_t per = ((hi - lo) / step + (uint64_t)threads - 1) / (uint64_t)threads * step;
    for (int i = 0; i < threads; i++) {
        memset(&sp[i], 0, sizeof sp[i]);
        sp[i].lo = lo + per * (uint64_t)i;
        sp[i].hi = sp[i].lo + per < hi ? sp[i].lo + per : hi;
        sp[i].step = step;
        pthread_create(&th[i], NULL, sweep, &sp[i]);
    }
    uint64_t bad = 0, n = 0;
    *first = 0;
    for (int i = 0; i < threads; i++) {
        pthread_join(th[i], NULL);
        if (sp[i].bad && bad == 0) *first = sp[i].first_bad;
        bad += sp[i].bad;
        n += sp[i].tested;
    }
    *tested = n;
    return bad;
}

/* y[i] = the C library's expf(x[i]) (the host side of the GPU comparison). */
void orc_libm_expf_array(const float *x, float *y, size_t n) {
    for (size_t i = 0; i < n; i++) y[i] = expf(x[i]);
}
