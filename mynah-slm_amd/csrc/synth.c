/* synth.c — the seeded synthetic-input generator (see include/mynah_synth.h).
 *
 * Compiled into the GPU library, the CPU oracle and the reference harness, so
 * all three consume identical bytes for a given seed.
 *
 * SPDX-License-Identifier: MIT */
#define _GNU_SOURCE
#include "mynah_synth.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#define GOLDEN 0x9E3779B97F4A7C15ull

static uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t mynah_synth_substream(uint64_t seed, uint64_t k) {
    return mix64(seed + (k + 1) * GOLDEN);
}

typedef struct {
    uint64_t state;
    uint64_t cur;
    int left;
} stream;

static void stream_init(stream *s, uint64_t state) {
    s->state = state;
    s->cur = 0;
    s->left = 0;
}

static uint64_t next_u64(stream *s) {
    s->state += GOLDEN;
    return mix64(s->state);
}

static unsigned next_byte(stream *s) {
    if (s->left == 0) {
        s->cur = next_u64(s);
        s->left = 8;
    }
    const unsigned b = (unsigned)(s->cur & 0xffu);
    s->cur >>= 8;
    s->left--;
    return b;
}

static double next_unit(stream *s) {
    return (double)(next_u64(s) >> 11) * 0x1.0p-53;
}

static double next_normal(stream *s) {
    const double u1 = next_unit(s);
    const double u2 = next_unit(s);
    const double r = sqrt(-2.0 * log(1.0 - u1));
    return r * cos(6.283185307179586476925286766559 * u2);
}

/* Uniform integer in [lo, hi] (span <= 256) by rejection on bytes. */
static int next_int8(stream *s, int lo, int hi) {
    const unsigned span = (unsigned)(hi - lo + 1);
    const unsigned limit = 256u - 256u % span;
    unsigned b;
    do { b = next_byte(s); } while (b >= limit);
    return lo + (int)(b % span);
}

uint16_t mynah_synth_f32_to_f16(float value) {
    uint32_t bits;
    memcpy(&bits, &value, sizeof bits);
    const uint32_t sign = (bits >> 16) & 0x8000u;
    const uint32_t mag = bits & 0x7fffffffu;
    if (mag >= 0x7f800000u)                       /* inf, nan */
        return (uint16_t)(sign | 0x7c00u | (mag > 0x7f800000u ? 0x0200u : 0u));
    if (mag >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 */
    if (mag < 0x38800000u) {                      /* below 2^-14: subnormal */
        const int e = (int)(mag >> 23);
        if (e < 102) return (uint16_t)sign;       /* below 2^-25 */
        const uint32_t m = (mag & 0x7fffffu) | 0x800000u;
        const int shift = 126 - e;                /* 14 .. 24 */
        uint32_t q = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = ((((mag >> 23) - 112u)) << 10) | ((mag & 0x7fffffu) >> 13);
    const uint32_t rem = mag & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

static void put_f16(unsigned char *p, double v) {
    const uint16_t h = mynah_synth_f32_to_f16((float)v);
    p[0] = (unsigned char)(h & 0xffu);
    p[1] = (unsigned char)(h >> 8);
}

static void gen_q4_k_row(stream *s, unsigned char *row, size_t blocks) {
    for (size_t b = 0; b < blocks; b++) {
        unsigned char *blk = row + b * 144;
        put_f16(blk, fabs(next_normal(s)) * 0.01);
        put_f16(blk + 2, fabs(next_normal(s)) * 0.01);
        for (int i = 0; i < 12; i++) blk[4 + i] = (unsigned char)next_byte(s);
        for (int i = 0; i < 128; i++) blk[16 + i] = (unsigned char)next_byte(s);
    }
}

static void gen_q5_k_row(stream *s, unsigned char *row, size_t blocks) {
    for (size_t b = 0; b < blocks; b++) {
        unsigned char *blk = row + b * 176;
        put_f16(blk, fabs(next_normal(s)) * 0.01);
        put_f16(blk + 2, fabs(next_normal(s)) * 0.01);
        for (int i = 0; i < 172; i++) blk[4 + i] = (unsigned char)next_byte(s);
    }
}

static void gen_q4_0_row(stream *s, unsigned char *row, size_t blocks) {
    for (size_t b = 0; b < blocks; b++) {
        unsigned char *blk = row + b * 18;
        put_f16(blk, fabs(next_normal(s)) * 0.01);
        for (int i = 0; i < 16; i++) blk[2 + i] = (unsigned char)next_byte(s);
    }
}

static void gen_q6_k_row(stream *s, unsigned char *row, size_t blocks) {
    for (size_t b = 0; b < blocks; b++) {
        unsigned char *blk = row + b * 210;
        for (int i = 0; i < 192; i++) blk[i] = (unsigned char)next_byte(s);
        for (int i = 0; i < 16; i++)
            blk[192 + i] = (unsigned char)(signed char)next_int8(s, -64, 63);
        put_f16(blk + 208, fabs(next_normal(s)) * 0.005);
    }
}

static void gen_q8_0_row(stream *s, unsigned char *row, size_t blocks) {
    for (size_t b = 0; b < blocks; b++) {
        unsigned char *blk = row + b * 34;
        put_f16(blk, fabs(next_normal(s)) * 0.01);
        for (int i = 0; i < 32; i++)
            blk[2 + i] = (unsigned char)(signed char)next_int8(s, -127, 127);
    }
}

typedef struct {
    int type;
    uint64_t seed;
    size_t row0, rows, cols, row_bytes, blocks;
    unsigned char *out;
    /* normal vectors */
    float *fout;
    size_t n;
    float mean, std;
    size_t begin, end;
} synth_job;

static void run_blocks(synth_job *j) {
    for (size_t r = j->begin; r < j->end; r++) {
        stream s;
        stream_init(&s, mynah_synth_substream(j->seed, j->row0 + r));
        unsigned char *row = j->out + r * j->row_bytes;
        if (j->type == 12) gen_q4_k_row(&s, row, j->blocks);
        else if (j->type == 13) gen_q5_k_row(&s, row, j->blocks);
        else if (j->type == 14) gen_q6_k_row(&s, row, j->blocks);
        else if (j->type == 2) gen_q4_0_row(&s, row, j->blocks);
        else gen_q8_0_row(&s, row, j->blocks);
    }
}

#define NORMAL_CHUNK 4096u

static void run_normal(synth_job *j) {
    for (size_t c = j->begin; c < j->end; c++) {
        stream s;
        stream_init(&s, mynah_synth_substream(j->seed, c));
        const size_t i0 = c * NORMAL_CHUNK;
        const size_t i1 = i0 + NORMAL_CHUNK < j->n ? i0 + NORMAL_CHUNK : j->n;
        for (size_t i = i0; i < i1; i++)
            j->fout[i] = (float)((double)j->mean + (double)j->std * next_normal(&s));
    }
}

static void *thread_main(void *arg) {
    synth_job *j = (synth_job *)arg;
    if (j->fout) run_normal(j);
    else run_blocks(j);
    return NULL;
}

static int thread_count(int threads, size_t units) {
    if (threads <= 0) {
        const long n = sysconf(_SC_NPROCESSORS_ONLN);
        threads = n > 0 ? (int)n : 1;
    }
    if (threads > 64) threads = 64;
    if ((size_t)threads > units) threads = (int)units;
    return threads < 1 ? 1 : threads;
}

/* Split [0, units) over threads; the calling thread takes the first share. */
static void run_split(synth_job base, size_t units, int threads) {
    const int nth = thread_count(threads, units);
    pthread_t tid[64];
    synth_job jobs[64];
    int started[64] = {0};
    const size_t per = (units + (size_t)nth - 1) / (size_t)nth;
    for (int t = 0; t < nth; t++) {
        jobs[t] = base;
        jobs[t].begin = (size_t)t * per < units ? (size_t)t * per : units;
        jobs[t].end = jobs[t].begin + per < units ? jobs[t].begin + per : units;
    }
    for (int t = 1; t < nth; t++)
        started[t] = pthread_create(&tid[t], NULL, thread_main, &jobs[t]) == 0;
    thread_main(&jobs[0]);
    for (int t = 1; t < nth; t++) {
        if (started[t]) pthread_join(tid[t], NULL);
        else thread_main(&jobs[t]);
    }
}

int mynah_synth_blocks(int type, uint64_t seed, size_t row0, size_t rows,
                       size_t cols, void *out, int threads) {
    size_t elems, bytes;
    switch (type) {
    case 12: elems = 256; bytes = 144; break;
    case 13: elems = 256; bytes = 176; break;
    case 14: elems = 256; bytes = 210; break;
    case 8:  elems = 32;  bytes = 34;  break;
    case 2:  elems = 32;  bytes = 18;  break;
    default: return -1;
    }
    if (out == NULL || rows == 0 || cols == 0 || cols % elems != 0) return -1;
    synth_job j;
    memset(&j, 0, sizeof j);
    j.type = type;
    j.seed = seed;
    j.row0 = row0;
    j.rows = rows;
    j.cols = cols;
    j.blocks = cols / elems;
    j.row_bytes = j.blocks * bytes;
    j.out = (unsigned char *)out;
    run_split(j, rows, threads);
    return 0;
}

int mynah_synth_normal(uint64_t seed, size_t n, float mean, float std,
                       float *out, int threads) {
    if (out == NULL || n == 0) return -1;
    synth_job j;
    memset(&j, 0, sizeof j);
    j.seed = seed;
    j.fout = out;
    j.n = n;
    j.mean = mean;
    j.std = std;
    run_split(j, (n + NORMAL_CHUNK - 1) / NORMAL_CHUNK, threads);
    return 0;
}

int mynah_synth_uniform_u32(uint64_t seed, size_t n, uint32_t bound,
                            uint32_t *out) {
    if (out == NULL || bound == 0) return -1;
    stream s;
    stream_init(&s, mynah_synth_substream(seed, 0));
    const uint64_t limit = UINT64_MAX - UINT64_MAX % bound;
    for (size_t i = 0; i < n; i++) {
        uint64_t v;
        do { v = next_u64(&s); } while (v >= limit);
        out[i] = (uint32_t)(v % bound);
    }
    return 0;
}
