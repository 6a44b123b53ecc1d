// sample.hip — the reference's token sampler (src/sampler.c:27-187) on the
// device, bit for bit: the same penalties, the same f32 exponentials and
// probabilities, the same candidates in the same order, the same splitmix64
// draw and walk. Four launches between the head GEMV and the step's
// mynah_argmax_advance, which then takes the sampled id as its only key.
//
//   mynah_samp_penalize  workgroup b owns logits 2048 b .. + 2047: applies
//                        the penalties of the window entries in its range
//                        (in place, as the reference does) and leaves the
//                        key of its first maximum (argmax_key).
//   mynah_samp_exp       (temp > 0) max of the keys; e_i = expf((l_i - max) /
//                        temp), f32 division and the C library's expf; the
//                        workgroup's exact-to-2^-100 sum of the e_i as a
//                        double-double.
//   mynah_samp_topk      the reference sums the e_i in double, in index order
//                        (src/sampler.c:131-141); every workgroup adds the
//                        double-double partials in one order and bounds that
//                        sequential sum: with n terms >= 0 it is within
//                        gamma_{n-1} = (n - 1) u / (1 - (n - 1) u), u = 2^-53, of
//                        the exact sum relative, and inv = (float)(1.0 / sum)
//                        is monotone in the sum, so when both ends of twice
//                        that interval give the same inv, it is the
//                        reference's inv. Otherwise (or with flag 1) thread 0
//                        adds the e_i in index order itself. p_i = e_i * inv;
//                        the workgroup's top_k keys (p, then the smaller id,
//                        as the reference's qsort orders them), 8192
//                        probabilities per workgroup.
//   mynah_samp_pick      one wave: greedy (temp <= 0) takes the largest
//                        penalised key; otherwise a k-way merge of the
//                        workgroups' sorted lists gives the global top_k in
//                        the reference's order, then min_p, top_p (crossing
//                        candidate kept), the double total, one splitmix64
//                        draw and the walk (src/sampler.c:145-186); with
//                        `accept` (the decoder's steps, where the loop
//                        accepts every id, src/generate.c:51-52) the id
//                        enters the window (mynah_slm_sampler_accept).
//
// The state (params, rng, window) lives in device memory, so a captured
// step replays with any parameters. top_k must be 1 .. SP_KMAX when
// temp > 0 (the host checks; a full sort of the vocabulary is not done
// here) and the window at most SP_WMAX.
//
// SPDX-License-Identifier: MIT
#include "common.hip.h"
#include "mynah_expf.h"
#include "sample.h"

// Inverse of argmax_key's value transform (a key's high word back to the
// f32 it orders).
MYNAH_DEV float key_value(unsigned long long key) {
    const uint32_t b = (uint32_t)(key >> 32);
    return __uint_as_float((b & 0x80000000u) ? (b & 0x7fffffffu) : ~b);
}

MYNAH_DEV uint32_t key_id(unsigned long long key) { return ~(uint32_t)(key & 0xffffffffull); }

// Error-free sum of two doubles (Knuth's TwoSum): a + b = s + e exactly.
MYNAH_DEV void two_sum(double a, double b, double &s, double &e) {
#pragma clang fp contract(off)
    s = a + b;
    const double bb = s - a;
    e = (a - (s - bb)) + (b - bb);
}

// Double-double addition (hi, lo) += (bh, bl), for non-negative terms.
MYNAH_DEV void dd_add(double &hi, double &lo, double bh, double bl) {
#pragma clang fp contract(off)
    double s, e;
    two_sum(hi, bh, s, e);
    e = e + (lo + bl);
    hi = s + e;
    lo = e - (hi - s);
}

// ── penalties and the first maximum ─────────────────────────────────────────
extern "C" __global__ __launch_bounds__(SP_T) void mynah_samp_penalize(
    float *__restrict__ logits, uint32_t vocab, const SampState *__restrict__ st,
    unsigned long long *__restrict__ wkey) {
#pragma clang fp contract(off)
    __shared__ float lg[SP_CH];
    __shared__ uint32_t ring[SP_WMAX];
    __shared__ unsigned long long wk[SP_T / 64u];
    __shared__ int changed;
    const uint32_t tid = threadIdx.x, c0 = blockIdx.x * SP_CH;
    const uint32_t n_recent = st->n_recent;
    const float rp = st->repeat_penalty, fp = st->freq_penalty, pp = st->presence_penalty;
    const bool active = n_recent > 0u && (rp != 1.0f || fp != 0.0f || pp != 0.0f);
    for (uint32_t i = tid; i < SP_CH; i += SP_T) lg[i] = c0 + i < vocab ? logits[c0 + i] : 0.0f;
    if (active)
        for (uint32_t i = tid; i < n_recent; i += SP_T) ring[i] = st->ring[i];
    if (tid == 0) changed = 0;
    __syncthreads();
    // src/sampler.c:72-94, the entries whose token this workgroup owns, in
    // the window's array order: each occurrence applies the transform once,
    // with the token's count.
    if (active && tid == 0) {
        for (uint32_t i = 0; i < n_recent; i++) {
            const uint32_t tok = ring[i];
            if (tok >= vocab || tok < c0 || tok - c0 >= SP_CH) continue;
            uint32_t count = 0;
            for (uint32_t k = 0; k < n_recent; k++) count += ring[k] == tok ? 1u : 0u;
            float l = lg[tok - c0];
            if (rp != 1.0f) l = (l > 0.0f) ? l / rp : l * rp;
            l -= fp * (float)count;
            l -= pp;
            lg[tok - c0] = l;
            changed = 1;
        }
    }
    __syncthreads();
    unsigned long long best = 0ull;
    for (uint32_t i = tid; i < SP_CH && c0 + i < vocab; i += SP_T) {
        const unsigned long long k = argmax_key(lg[i], c0 + i);
        best = k > best ? k : best;
        if (changed) logits[c0 + i] = lg[i];
    }
    best = wave_max_u64(best);
    if ((tid & 63u) == 0u) wk[tid >> 6] = best;
    __syncthreads();
    if (tid == 0) {
        for (uint32_t w = 1; w < SP_T / 64u; w++) best = wk[w] > best ? wk[w] : best;
        wkey[blockIdx.x] = best;
    }
}

// ── exponentials and their exact partial sums ───────────────────────────────
extern "C" __global__ __launch_bounds__(SP_T) void mynah_samp_exp(
    const float *__restrict__ logits, uint32_t vocab, const SampState *__restrict__ st,
    const unsigned long long *__restrict__ wkey, uint32_t nwg, float *__restrict__ e,
    double *__restrict__ wsum) {
#pragma clang fp contract(off)
    __shared__ unsigned long long wk[SP_T / 64u];
    __shared__ double sh[SP_T / 64u], sl[SP_T / 64u];
    const float temp = st->temp;
    if (!(temp > 0.0f)) return;
    const uint32_t tid = threadIdx.x, c0 = blockIdx.x * SP_CH;
    unsigned long long best = 0ull;
    for (uint32_t i = tid; i < nwg; i += SP_T) best = wkey[i] > best ? wkey[i] : best;
    best = wave_max_u64(best);
    if ((tid & 63u) == 0u) wk[tid >> 6] = best;
    __syncthreads();
    for (uint32_t w = 0; w < SP_T / 64u; w++) best = wk[w] > best ? wk[w] : best;
    const float mx = key_value(best);
    double hi = 0.0, lo = 0.0;
    for (uint32_t i = tid; i < SP_CH && c0 + i < vocab; i += SP_T) {
        const float v = mynah_expf((logits[c0 + i] - mx) / temp);
        e[c0 + i] = v;
        dd_add(hi, lo, (double)v, 0.0);
    }
    // Workgroup sum: lanes by xor butterfly, then the waves in order.
    for (int m = 32; m >= 1; m >>= 1) {
        const double oh = __shfl_xor(hi, m, 64), ol = __shfl_xor(lo, m, 64);
        dd_add(hi, lo, oh, ol);
    }
    if ((tid & 63u) == 0u) {
        sh[tid >> 6] = hi;
        sl[tid >> 6] = lo;
    }
    __syncthreads();
    if (tid == 0) {
        hi = sh[0];
        lo = sl[0];
        for (uint32_t w = 1; w < SP_T / 64u; w++) dd_add(hi, lo, sh[w], sl[w]);
        wsum[2u * blockIdx.x] = hi;
        wsum[2u * blockIdx.x + 1u] = lo;
    }
}

// ── probabilities and each workgroup's top_k ────────────────────────────────
// Descending compare-exchange of two keys.
MYNAH_DEV void cx(unsigned long long &a, unsigned long long &b) {
    const unsigned long long hi = a > b ? a : b, lo = a > b ? b : a;
    a = hi;
    b = lo;
}

// Workgroup b takes probabilities 8192 b .. + 8191, eight per thread
// (strided), sorted descending in registers by a 19-comparator network;
// each wave then pops its K largest keys by K rounds of a wave maximum over
// the lanes' first keys (keys are unique, so exactly one lane pops), and
// wave 0 merges the sixteen waves' lists the same way into cand[b].
extern "C" __global__ __launch_bounds__(SP_TK_T) void mynah_samp_topk(
    const float *__restrict__ e, uint32_t vocab, const SampState *__restrict__ st,
    const double *__restrict__ wsum, uint32_t nwg, unsigned long long *__restrict__ cand) {
#pragma clang fp contract(off)
    constexpr uint32_t NW = SP_TK_T / 64u;
    __shared__ unsigned long long wl[NW][SP_KMAX];
    __shared__ double ps[2u * SP_TK_MAXWG * (SP_TK_CH / SP_CH)];
    __shared__ float sinv;
    const float temp = st->temp;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t c0 = blockIdx.x * SP_TK_CH, K = st->top_k, flags = st->flags;
    // Every load goes out first: this workgroup's exponentials, the partial
    // sums (wave 0 then adds them by a fixed tree
    // (lane l: partials l and l + 64, then an xor butterfly), so every
    // workgroup gets the same sum).
    float ev[8];
#pragma unroll
    for (int q = 0; q < 8; q++) {
        const uint32_t i = c0 + tid + SP_TK_T * (uint32_t)q;
        ev[q] = i < vocab ? e[i] : 0.0f;
    }
    for (uint32_t i = tid; i < 2u * nwg; i += SP_TK_T) ps[i] = wsum[i];
    if (!(temp > 0.0f)) return;
    __syncthreads();
    double hi = 0.0, lo = 0.0;
    if (wave == 0) {
        for (uint32_t w = lane; w < nwg; w += 64u) dd_add(hi, lo, ps[2u * w], ps[2u * w + 1u]);
        for (int m = 1; m <= 32; m <<= 1) {
            const double oh = __shfl_xor(hi, m, 64), ol = __shfl_xor(lo, m, 64);
            dd_add(hi, lo, oh, ol);
        }
    }
    if (tid == 0) {
        const double x = hi + lo, u = 0x1p-53, n1 = (double)(vocab - 1u);
        const double gamma = n1 * u / (1.0 - n1 * u);
        const float a = (float)(1.0 / (x * (1.0 - 2.0 * gamma)));
        const float b = (float)(1.0 / (x * (1.0 + 2.0 * gamma)));
        float inv = a;
        if (a != b || (flags & SP_FLAG_SEQ_SUM) != 0u) {
            // The reference's own sum, src/sampler.c:133-141.
            double sum = 0.0;
            for (uint32_t i = 0; i < vocab; i++) sum += (double)e[i];
            inv = (float)(1.0 / sum);
        }
        sinv = inv;
    }
    __syncthreads();
    const float inv = sinv;
    unsigned long long k[8];
#pragma unroll
    for (int q = 0; q < 8; q++) {
        const uint32_t i = c0 + tid + SP_TK_T * (uint32_t)q;
        k[q] = i < vocab ? argmax_key(ev[q] * inv, i) : 0ull;
    }
    // Batcher's odd-even merge sort network for 8 (19 comparators).
    cx(k[0], k[1]); cx(k[2], k[3]); cx(k[4], k[5]); cx(k[6], k[7]);
    cx(k[0], k[2]); cx(k[1], k[3]); cx(k[4], k[6]); cx(k[5], k[7]);
    cx(k[1], k[2]); cx(k[5], k[6]);
    cx(k[0], k[4]); cx(k[1], k[5]); cx(k[2], k[6]); cx(k[3], k[7]);
    cx(k[2], k[4]); cx(k[3], k[5]);
    cx(k[1], k[2]); cx(k[3], k[4]); cx(k[5], k[6]);
    for (uint32_t r = 0; r < K; r++) {
        const unsigned long long m = wave_max_u64_dpp(k[0]);
        if (k[0] == m) {
#pragma unroll
            for (int q = 0; q < 7; q++) k[q] = k[q + 1];
            k[7] = 0ull;
        }
        if (lane == 0) wl[wave][r] = m;
    }
    __syncthreads();
    if (wave == 0) {
        uint32_t h = 0;
        for (uint32_t r = 0; r < K; r++) {
            const unsigned long long own = lane < NW && h < K ? wl[lane][h] : 0ull;
            const unsigned long long m = wave_max_u64_dpp(own);
            if (lane < NW && own == m) h++;
            if (lane == 0) cand[(size_t)blockIdx.x * SP_KMAX + r] = m;
        }
    }
}

// splitmix64 (src/sampler.c:40-46): a double in [0, 1).
MYNAH_DEV double rng_next(unsigned long long &state) {
    unsigned long long z = (state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z = z ^ (z >> 31);
    return (double)(z >> 11) * (1.0 / 9007199254740992.0);
}

// ── the pick ────────────────────────────────────────────────────────────────
extern "C" __global__ __launch_bounds__(64) void mynah_samp_pick(
    SampState *__restrict__ st, uint32_t vocab, const unsigned long long *__restrict__ wkey,
    const unsigned long long *__restrict__ cand, uint32_t nwg, uint32_t nwg_tk,
    unsigned long long *__restrict__ out_key, uint32_t accept) {
#pragma clang fp contract(off)
    __shared__ unsigned long long lc[SP_TK_MAXWG * SP_KMAX];
    const uint32_t lane = threadIdx.x;
    // The state's fields all at once (each later read would wait its own
    // round trip).
    const float temp = st->temp, min_p = st->min_p, top_p = st->top_p;
    const uint32_t K = st->top_k, w = st->window, head = st->head, n_recent = st->n_recent;
    unsigned long long rng = st->rng;
    uint32_t id = 0;
    if (!(temp > 0.0f)) {
        // src/sampler.c:122-129 on the penalised logits.
        unsigned long long best = 0ull;
        for (uint32_t i = lane; i < nwg; i += 64u) best = wkey[i] > best ? wkey[i] : best;
        id = key_id(wave_max_u64(best));
    } else {
        // The first K keys of each list (the merge reads no further).
#pragma unroll 4
        for (uint32_t i = lane; i < nwg_tk * K; i += 64u) {
            const uint32_t g = i / K, r = i - g * K;
            lc[g * SP_KMAX + r] = cand[(size_t)g * SP_KMAX + r];
        }
        __syncthreads();
        // K rounds of an nwg_tk-way merge of the sorted lists (lane g holds
        // list g's position); candidate r stays in lane r % 64 (t0, t1),
        // read back by readlane below.
        uint32_t h = 0;
        unsigned long long t0 = 0ull, t1 = 0ull;
        for (uint32_t r = 0; r < K; r++) {
            const unsigned long long own = lane < nwg_tk && h < K ? lc[lane * SP_KMAX + h] : 0ull;
            const unsigned long long m = wave_max_u64_dpp(own);
            if (lane < nwg_tk && own == m) h++;
            if (lane == (r & 63u)) {
                if (r < 64u) t0 = m;
                else t1 = m;
            }
        }
        // The walk runs in every lane alike (its indices are uniform, so the
        // candidates come back by readlane from registers every lane set).
        auto kr = [&](uint32_t r) -> unsigned long long {
            return r < 64u ? readlane_u64(t0, (int)r) : readlane_u64(t1, (int)(r - 64u));
        };
        auto pk = [&](uint32_t r) -> float { return key_value(kr(r)); };
        auto ik = [&](uint32_t r) -> uint32_t { return key_id(kr(r)); };
        {
            // src/sampler.c:145-186 over the sorted top K.
            uint32_t n = K;
            if (min_p > 0.0f && n > 0u) {
                const float floor_p = min_p * pk(0);
                uint32_t keep = 1;
                while (keep < n && pk(keep) >= floor_p) keep++;
                n = keep;
            }
            if (top_p < 1.0f && n > 0u) {
                double acc = 0.0;
                uint32_t keep = 0;
                while (keep < n) {
                    acc += (double)pk(keep);
                    keep++;
                    if (acc >= (double)top_p) break;
                }
                n = keep;
            }
            if (n == 0u) n = 1u;
            double total = 0.0;
            for (uint32_t i = 0; i < n; i++) total += (double)pk(i);
            double r = rng_next(rng) * total;
            if (lane == 0) st->rng = rng;
            id = ik(n - 1u);
            for (uint32_t i = 0; i < n; i++) {
                r -= (double)pk(i);
                if (r <= 0.0) {
                    id = ik(i);
                    break;
                }
            }
        }
    }
    if (lane == 0) {
        // src/sampler.c:73-78 (mynah_slm_sampler_accept).
        if (accept != 0u && w > 0u) {
            st->ring[head] = id;
            st->head = (head + 1u) % w;
            st->n_recent = n_recent < w ? n_recent + 1u : n_recent;
        }
        out_key[0] = argmax_key(0.0f, id);
    }
}
