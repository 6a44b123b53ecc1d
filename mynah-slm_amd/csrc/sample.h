/* sample.h — the device sampler's state and sizes, shared by sample.hip
 * (kernels) and the host code (decode.c, sampler objects).
 *
 * SPDX-License-Identifier: MIT */
#ifndef MYNAH_SAMPLE_H
#define MYNAH_SAMPLE_H

#include <stdint.h>

#define SP_CH 2048u    /* logits per workgroup (penalties, exponentials) */
#define SP_T 256u      /* their threads */
#define SP_TK_CH 8192u /* probabilities per workgroup of the top_k launch */
#define SP_TK_T 1024u  /* its threads */
#define SP_TK_MAXWG 32u /* its workgroups: vocabulary up to 262,144 */
#define SP_KMAX 128u   /* largest top_k sampled on the device */
#define SP_WMAX 4096u  /* largest penalty window */
#define SP_FLAG_SEQ_SUM 1u /* always add the exponentials in index order */

/* src/sampler.c:16-25 (struct mynah_slm_sampler) without its work buffer:
 * the parameters (src/sampler.h:16-30, same order), the splitmix64 state
 * and the penalty window. */
typedef struct {
    float temp;
    uint32_t top_k;
    float top_p, min_p, repeat_penalty, freq_penalty, presence_penalty;
    uint32_t window;
    unsigned long long seed, rng;
    uint32_t head, n_recent, flags, pad;
    uint32_t ring[SP_WMAX];
} SampState;

#endif
