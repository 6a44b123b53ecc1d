/* settle_pin.c — TEST INFRASTRUCTURE ONLY: the kernels' test of a
 * parallel-order double sum (mynah-slm_amd/csrc/sum_settle.h) compiled for
 * the host, so that tests/test_sum_settle.py can hold it against index-order
 * sums on the CPU.
 *
 * SPDX-License-Identifier: MIT */
#include "../mynah-slm_amd/csrc/sum_settle.h"

#include <stddef.h>
#include <stdint.h>
#include <string.h>

/* out[i] = the test for r[i] (n terms, k2). */
void orc_sum_settled(const double *r, size_t count, uint32_t n, uint32_t k2, uint8_t *out) {
    for (size_t i = 0; i < count; i++) {
        uint64_t b;
        memcpy(&b, &r[i], sizeof b);
        out[i] = (uint8_t)mynah_sum_settled((uint32_t)(b >> 32), (uint32_t)b, n, k2);
    }
}
