/* kernels_hip.h — the MI355X (gfx950) drop-in for the reference's quantized
 * kernel ABI.
 *
 * Part 1 repeats ingot's kernel entry points with identical names, argument
 * meaning, layouts and return codes, so the reference's decoder
 * (src/arch_qwen3.c:46, :64, :175) links against this library unchanged:
 *   - `weights` is the row-major [rows][cols / block] array of GGUF blocks
 *     exactly as stored (never repacked);
 *   - matvec writes output[rows]; matmat reads input[tokens][cols] and writes
 *     output[tokens][rows]; dequant writes output[rows * cols] f32;
 *   - return 0 on success, -1 on a NULL pointer, rows == 0, cols == 0, a
 *     partial block, overflow or an unsupported type; nothing is printed.
 * The pointers are HOST pointers, as in the reference. Weights inside a range
 * handed to mynah_hip_register() are read from their resident HBM copy; any
 * other weights are staged to the device for the call. x and y cross PCIe on
 * every call, so a decoder that wants device speed uses part 2.
 *
 * Type ids are ggml's on-disk ids: Q4_0 = 2, Q8_0 = 8, Q4_K = 12, Q5_K = 13,
 * Q6_K = 14 (third_party/ingot/include/ingot/dtype.h:24-59).
 *
 * Part 2 is new API with no reference counterpart: device-pointer twins with a
 * stream argument (the stream is a hipStream_t passed as void *, NULL = the
 * library's own stream), host-range registration (the hook the reference's
 * ingot_gguf_mapping exists for, third_party/ingot/include/ingot/gguf.h:86-88),
 * plain device memory helpers, and a timing helper for the benchmark.
 *
 * Errors: every call returns 0 / -1 (or NULL); mynah_hip_last_error() gives
 * the message of the calling thread's last failure.
 *
 * Thread safety: calls may come from several threads; host-pointer calls are
 * serialised inside the library (one device, one staging area).
 *
 * SPDX-License-Identifier: MIT */
#ifndef MYNAH_KERNELS_HIP_H
#define MYNAH_KERNELS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ── part 1: ingot's kernel ABI ────────────────────────────────────────── */

/* third_party/ingot/include/ingot/quant.h:155-156 */
int ingot_matvec(int type, const void *weights, size_t rows, size_t cols,
                 const float *input, float *output);
/* quant.h:157-158. Exact f32 for every width unless the int8 lane is on
 * (mynah_hip_set_int8 below), which then takes Q4_K and Q5_K from two tokens
 * up, as the reference's AVX2 build does (kernels.c:1714-1751, 2573-2595). */
int ingot_matmat(int type, const void *weights, size_t rows, size_t cols,
                 const float *input, float *output, size_t tokens);
/* quant.h:159-160 — bit-identical to the reference decoders. */
int ingot_dequant_matrix(int type, const void *weights, size_t rows, size_t cols,
                         float *output);
/* quant.h:161 — 1 for Q4_K, Q5_K, Q6_K, Q8_0, Q4_0. */
int ingot_has_kernel(int type);
/* quant.h:149 (kernels.c:1714-1721): 1 when `tokens` takes the exact path —
 * always for tokens <= 1, otherwise unless the int8 lane is on. */
int ingot_matmat_is_exact(size_t tokens);

/* quant.h:64-73 */
int ingot_q4_k_matvec(const void *weights, size_t rows, size_t cols,
                      const float *input, float *output);
int ingot_q4_k_dequant(const void *weights, size_t rows, size_t cols, float *output);
int ingot_q4_k_matmat(const void *weights, size_t rows, size_t cols,
                      const float *input, float *output, size_t tokens);
/* quant.h:151-152: the exact batched order whatever the int8 lane's mode
 * (tokens == 1 is the matvec, kernels.c:1723-1726). */
int ingot_q4_k_matmat_exact(const void *weights, size_t rows, size_t cols,
                            const float *input, float *output, size_t tokens);
/* quant.h:74-75 (kernels.c:319-337): the scalar lane — the exact order —
 * whatever the int8 lane's mode. The as-built ingot_q4_k_matvec is that lane
 * too, so both give the same bits unless the int8 lane is on. */
int ingot_q4_k_matvec_scalar(const void *weights, size_t rows, size_t cols,
                             const float *input, float *output);
/* kernels.c:799-810 (exported by ingot's kernels, not declared in quant.h):
 * the int8 matvec whatever the mode — activations quantised per 256 values
 * (amax / 127, round half to even), integer dots per 32, the reference's f32
 * epilogue; bit-identical to an AVX2 + FMA build of ingot. */
int ingot_q4_k_matvec_int8(const void *weights, size_t rows, size_t cols,
                           const float *input, float *output);
/* quant.h:80-86. Q5_K: the matvec in the order of the scalar lane the
 * reference builds without -march (kernels.c:1785-1853), so the _scalar
 * entry point gives the same bits; matmat from two tokens up in its batched
 * core's order (kernels.c:2573-2606). */
int ingot_q5_k_matvec(const void *weights, size_t rows, size_t cols,
                      const float *input, float *output);
int ingot_q5_k_matvec_scalar(const void *weights, size_t rows, size_t cols,
                             const float *input, float *output);
int ingot_q5_k_dequant(const void *weights, size_t rows, size_t cols, float *output);
int ingot_q5_k_matmat(const void *weights, size_t rows, size_t cols,
                      const float *input, float *output, size_t tokens);
/* quant.h:152-153: the exact batched order whatever the int8 lane's mode. */
int ingot_q5_k_matmat_exact(const void *weights, size_t rows, size_t cols,
                            const float *input, float *output, size_t tokens);
/* quant.h:83-88 */
int ingot_q6_k_matvec(const void *weights, size_t rows, size_t cols,
                      const float *input, float *output);
int ingot_q6_k_dequant(const void *weights, size_t rows, size_t cols, float *output);
int ingot_q6_k_matmat(const void *weights, size_t rows, size_t cols,
                      const float *input, float *output, size_t tokens);
/* quant.h:108-110. Q4_0: one running sum over each whole row
 * (kernels.c:2467-2484); ingot_matmat(Q4_0, ...) runs that chain per token,
 * as the reference's generic path does (generic.c:76-93). cols % 32 == 0. */
int ingot_q4_0_matvec(const void *weights, size_t rows, size_t cols,
                      const float *input, float *output);
int ingot_q4_0_dequant(const void *weights, size_t rows, size_t cols, float *output);
/* quant.h:107-112 */
int ingot_q8_0_matvec(const void *weights, size_t rows, size_t cols,
                      const float *input, float *output);
int ingot_q8_0_dequant(const void *weights, size_t rows, size_t cols, float *output);
int ingot_q8_0_matmat(const void *weights, size_t rows, size_t cols,
                      const float *input, float *output, size_t tokens);

/* quant.h:179-183 (ingot_gguf_matvec / _matmat / _dequant_matrix,
 * generic.c:148-173). `g` and `t` are the reference's ingot_gguf /
 * ingot_tensor (third_party/ingot/include/ingot/gguf.h:41-50); the tensor's
 * bytes are located through the host process's ingot_gguf_data(), so these
 * entry points need ingot's GGUF reader linked in (they return -1
 * otherwise). rows = ne[1] (1 for rank 1), cols = ne[0]; rank 0, rank > 2
 * and zero dimensions return -1. */
int ingot_gguf_matvec(const void *g, const void *t, const float *input, float *output);
int ingot_gguf_matmat(const void *g, const void *t, const float *input, float *output,
                      size_t tokens);
int ingot_gguf_dequant_matrix(const void *g, const void *t, float *output);

/* ── part 2: device-resident API (no reference counterpart) ────────────── */

/* Select and initialise a device (default: device 0 on first use, or the
 * MYNAH_HIP_DEVICE environment variable). */
int mynah_hip_init(int device);
const char *mynah_hip_last_error(void);

/* Upload [host, host + bytes) unchanged into HBM; host pointers inside it
 * then resolve to the device copy (same address modulo 256). */
int mynah_hip_register(const void *host, size_t bytes);
int mynah_hip_unregister(const void *host);
/* Device address of a registered host pointer, or NULL. */
void *mynah_hip_device_ptr(const void *host);

/* Device-pointer twins. Weights 16-byte aligned for Q4_K / Q5_K and 2-byte
 * aligned for Q6_K / Q8_0 / Q4_0 (GGUF data and whole-row offsets satisfy
 * both); x 16-byte aligned. Asynchronous on `stream`. */
int mynah_hip_matvec_dev(int type, const void *w, size_t rows, size_t cols,
                         const float *x, float *y, void *stream);
int mynah_hip_matmat_dev(int type, const void *w, size_t rows, size_t cols,
                         const float *x, float *y, size_t tokens, void *stream);
int mynah_hip_dequant_dev(int type, const void *w, size_t rows, size_t cols,
                          float *y, void *stream);
/* Y[tokens][rows] = X[tokens][cols] · W^T summed in the MATVEC order: every
 * output bit-identical to mynah_hip_matvec_dev (and the reference's
 * ingot_matvec, kernels.c:94-115, 319-337, 2525-2551) of its own token, at
 * GEMM speed (the prompt prefill's projections). res (optional, may equal
 * y): y = res + W x, the reference's residual add (src/arch_qwen3.c:224).
 * No reference counterpart (the reference's batched product sums in its
 * own batched order). cols % 256 == 0 (Q4_0: cols % 32 == 0, its batched
 * order being the matvec's); device pointers; asynchronous. */
int mynah_hip_matmat_mv_dev(int type, const void *w, size_t rows, size_t cols,
                            const float *x, float *y, size_t tokens, const float *res,
                            void *stream);

/* Summation order of every GEMV (host and device entry points):
 *   MYNAH_GEMV_EXACT (default): the reference's own f32 order, so outputs are
 *     bit-identical to the as-built CPU kernels;
 *   MYNAH_GEMV_REORDERED: lane-parallel partial sums (fewer instructions per
 *     weight); differs from the reference by f32 rounding only. */
enum { MYNAH_GEMV_EXACT = 0, MYNAH_GEMV_REORDERED = 1 };
int mynah_hip_set_gemv_order(int order);
int mynah_hip_gemv_order(void);
/* The reference's double sums (RMSNorm's squares, src/kernels.c:118-121;
 * the softmax's exponentials, :213-218) are taken in a parallel order. Any
 * order lies within γ(n−1) of the exact sum, as does the reference's index
 * order, so where the f32 result (RMS scale, softmax reciprocal) is the same
 * over that whole interval it is the reference's (csrc/sum_settle.h);
 * otherwise the softmax and norm kernels add the terms again in index
 * order. The GEMV kernels' fused RMSNorm keeps its parallel sum unchecked
 * (by a rounding estimate its scale differs from the reference's about
 * once in 10^7 sums), as do the split attention's query/key norms.
 * on = 1 sends every checked sum through the index-order path (both paths
 * give the same bits; a test switch), 0 (default) restores the check. Takes
 * effect for launches after the call, on every initialised device. No
 * reference counterpart. */
int mynah_hip_set_index_order_sums(int on);
/* The code-object name of the kernel one matvec of this type and shape
 * launches in the given order (-1: the current one), from the same plan the
 * launch makes; NULL (reason in mynah_hip_last_error) when it cannot run.
 * No reference counterpart: it names what a profiler trace will show. */
const char *mynah_hip_gemv_kernel(int type, size_t rows, size_t cols, int order);

/* The int8 activation lane of Q4_K and Q5_K products (the reference's lane
 * of an AVX2 + FMA build of ingot, third_party/ingot/src/kernels.c:636-788,
 * 1120-1751, 2573-2595), bit-identical to that build:
 *   MYNAH_INT8_OFF (default, like the as-built reference, which has no int8
 *     lane): exact f32 everywhere;
 *   MYNAH_INT8_BATCHED: Q4_K and Q5_K matmat with tokens >= 2 quantise
 *     their input (that build's batched default);
 *   MYNAH_INT8_ALL: the Q4_K matvec too (that build with INGOT_SDOT=1; Q5_K
 *     has no int8 matvec there).
 * INGOT_SDOT=1 in the environment, read at the first call that needs the
 * mode, starts the library in MYNAH_INT8_ALL. Q6_K, Q8_0 and Q4_0 stay
 * exact, and the resident decode step (mynah_decode.h) always runs exact. */
enum { MYNAH_INT8_OFF = 0, MYNAH_INT8_BATCHED = 1, MYNAH_INT8_ALL = 2 };
int mynah_hip_set_int8(int mode);
int mynah_hip_int8(void);
/* The lane in two steps, for callers that reuse quantised activations:
 * x[tokens][cols] (cols % 256 == 0, 16-byte aligned) to xq[tokens][cols]
 * int8, xs[tokens][cols / 256] scales and xsum[tokens][cols / 32] int32 sums;
 * then y[tokens][rows] from them (16-byte aligned xq and xsum). tokens == 1
 * uses the matvec's epilogue, tokens >= 2 the batched one. Asynchronous. */
int mynah_hip_q8_quantize_dev(const float *x, size_t tokens, size_t cols, int8_t *xq,
                              float *xs, int32_t *xsum, void *stream);
int mynah_hip_q4k_int8_dev(const void *w, size_t rows, size_t cols, const int8_t *xq,
                           const float *xs, const int32_t *xsum, float *y, size_t tokens,
                           void *stream);

/* No counterpart in the reference. For callers that cannot allocate device
 * memory — code under HIP graph (stream) capture, serving loops that must
 * not allocate, harnesses that forbid hipMalloc: the int8 lane's product
 * (what mynah_hip_matmat_dev computes for Q4_K / Q5_K with the lane on:
 * activations quantised per 256 values, integer dots, the reference's
 * epilogue; tokens == 1 the Q4_K matvec epilogue, Q5_K needs tokens >= 2),
 * whatever the lane's mode, with its quantised activations in a fixed
 * device workspace of MYNAH_SCRATCH_BYTES (8 MiB, csrc/scratch.h) that each
 * GPU holds until the process ends. Allocates nothing and calls no
 * allocating routine. Refuses (-1, nothing launched) a workspace above the
 * limit: tokens * cols * 1.140625 bytes, about 7.35 M values. Calls that
 * overlap on one GPU share the workspace and race; serialise them (one
 * stream, or events). Device pointers; asynchronous on `stream`. */
int mynah_hip_int8_product_noalloc_dev(int type, const void *w, size_t rows, size_t cols,
                                       const float *x, float *y, size_t tokens, void *stream);

/* Plain device memory (256-byte aligned) and copies; *_async take a stream. */
void *mynah_hip_alloc(size_t bytes);
int   mynah_hip_free(void *p);
int   mynah_hip_h2d(void *dst, const void *src, size_t bytes);
int   mynah_hip_d2h(void *dst, const void *src, size_t bytes);
int   mynah_hip_memset(void *dst, int value, size_t bytes);
int   mynah_hip_sync(void *stream);
/* Device-to-device copy by a plain 16-byte-vector kernel (buffers 16-byte
 * aligned, bytes a multiple of 16); the yardstick of the HBM counters. */
int   mynah_hip_copy_dev(void *dst, const void *src, size_t bytes, void *stream);
/* A read-only stream over src (16-byte aligned, bytes a multiple of 16):
 * every byte loaded once, nothing written but (practically never) one word
 * of sink; the yardstick of what one launch reads at a size. No reference
 * counterpart. */
int   mynah_hip_read_dev(const void *src, size_t bytes, void *sink, void *stream);
/* The VALU yardstick (no reference counterpart): time per wave64 v_add_f32
 * per SIMD, in ns, with every SIMD issuing nothing but independent f32 adds
 * (eight waves per SIMD, `iters` x 8 adds per lane) — the price of one
 * product in the exact summation orders; *simds (optional) gets the
 * device's SIMD count. Synchronous; allocates 4 bytes. */
int   mynah_hip_valu_add_rate(uint32_t iters, float *ns_per_instr, uint32_t *simds);
/* The products of the exact GEMM's matrix-core instruction (no reference
 * counterpart; a test hook): per wave w < waves, a[64 w + l] and b[64 w + l]
 * feed lane l, c the accumulator; prod (zero accumulator), acc (c), mul (the
 * VALU's a * b) and fused (fmaf(a, b, c)) get 1024 w + 16 l + r for lane l,
 * register r: block r / 4, row 4 (l / 16) + r % 4, column l % 16. Device
 * buffers: a, b 64 * waves floats, the rest 1024 * waves. */
int   mynah_hip_mfma_probe(const float *a, const float *b, const float *c, float *prod,
                           float *acc, float *mul, float *fused, uint32_t waves, void *stream);
void *mynah_hip_stream(void);           /* the library's own stream */

/* y[i] = expf(x[i]) for i < n with the bits of the reference's C library
 * (glibc's expf, the exponential of the reference's softmax and sigmoid,
 * src/kernels.c:193-220), which the decode step's softmax and SwiGLU use.
 * Device pointers; asynchronous. */
int   mynah_hip_expf_dev(const float *x, float *y, size_t n, void *stream);

/* HIP events on a stream (NULL = the library's stream), for timing kernels
 * exactly where they are launched. Elapsed time in milliseconds. */
void *mynah_hip_event_create(void);
int   mynah_hip_event_record(void *event, void *stream);
int   mynah_hip_event_elapsed(void *start, void *end, float *ms);
int   mynah_hip_event_destroy(void *event);

/* Benchmark helper for a sweep of n matrices: `steps` passes, pass i
 * launching matrix m on weight copy w[m * copies + i % copies] (all copies of
 * one matrix share x[m] and y[m]). Launched from C on the library stream and
 * timed with HIP events: *ms_total for all passes, and *ms_timed the average
 * duration of matrix `timed`'s launch in every `every`-th pass (an event pair
 * around each of those: the markers lengthen a pass by a few µs, so a sample
 * of the passes carries them; every = 1: all). timed < 0: none. */
int mynah_hip_time_sweep(int n, const int *types, const void *const *w, int copies,
                         const size_t *rows, const size_t *cols, const float *const *x,
                         float *const *y, int steps, int timed, int every, float *ms_total,
                         float *ms_timed);

/* Benchmark helper: `iters` launches of the matvec, cycling through the
 * `n_copies` weight copies in w_copies[] (to stream from HBM rather than
 * cache), timed with HIP events on the launch stream. *ms = total time. */
int mynah_hip_time_matvec(int type, const void *const *w_copies, int n_copies,
                          size_t rows, size_t cols, const float *x, float *y,
                          int iters, float *ms);

#ifdef __cplusplus
}
#endif
#endif
