/* scratch.h — the size of the fixed device workspace of the
 * allocation-free entry point (mynah_hip_int8_product_noalloc_dev), shared
 * by the device array's definition (int8.hip) and the host checks (int8.c,
 * runtime.c). 8 MiB holds the int8 lane's quantised activations of
 * tokens * cols <= 7,354,396 values (1.140625 bytes per value: one int8,
 * a 4-byte scale per 256 and a 4-byte sum per 32), e.g. 512 tokens of 9728
 * or 3584 tokens of 2048.
 *
 * SPDX-License-Identifier: MIT */
#ifndef MYNAH_SCRATCH_H
#define MYNAH_SCRATCH_H

#define MYNAH_SCRATCH_BYTES (8u << 20)

#endif
