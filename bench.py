"""Benchmark: quantized GEMV throughput on one MI355X (BASELINE.json metric).

One "step" is one pass of the hot path over configs[1] of BASELINE.json: the
Q6_K and Q8_0 matvec sweep at the Qwen3-0.6B projection shapes plus the
151936 x 1024 Q6_K output head, synthetic inputs from seed 0, weights resident
in HBM. Each step reads a different one of several device copies of every
matrix (together > 2x the 256 MB MALL), so every launch streams from HBM.

`value` = algorithmic bytes per step (weights + x + y) / time per step.
`sweep` gives beside it the median and spread of 20 shorter trials of the
same sweep and the hot-cache figure (one weight copy, mostly held by the
MALL). `roofline` is the dominant kernel (the Q6_K head GEMV): algorithmic bytes per
launch over its average duration, timed with HIP events on the launch stream
inside the timed region. `traffic` is the HBM bytes per launch measured by
rocprofv3 PMC counters (profiles/traffic.json), when present.
`cpu_baseline` times the CPU oracle (the C11 restatement of the reference's
as-built kernels with the reference's 4*nth row-chunk threading, bit-identical
to it) on the same sweep on this host's cores, the median of five runs; beside
it the same sweep in the f32 lanes of an AVX2 + FMA ingot build (restated,
pinned to such a build by golden vectors), configs[0], the configs[2] and
configs[4] decode (tok/s, ids checked against the compiled reference's) and
configs[3]'s batched products, each the median of five runs.

Beside the metric line's value: `decode` (configs[2], Qwen3-0.6B greedy
decode tok/s in three numerics modes, tokens checked against the compiled
reference's, and `decode.sampled`: the generation loop with the front ends'
default sampler on the device), `prefill_gemm` (configs[3], the exact batched GEMM at 512
tokens), `prefill_gemm_int8` (the same with Q4_K on the int8 activation
lane, the batched default of the reference's AVX2 build),
`qwen3_4b_end_to_end` (configs[4]: 2048-token prompt prefill and 256
greedy steps on Qwen3-4B), `qwen3_4b_gemv_gbs` (each Qwen3-4B GEMV class),
`qwen3_4b_copy_ceiling_gbs` / `qwen3_4b_read_ceiling_gbs` (a plain copy and a
read-only stream moving the same HBM bytes per launch: what any kernel
launched back to back reaches at that size) and `valu` (the time per wave64
f32 add with every SIMD issuing adds only, and the exact GEMM's ceiling that
follows from one add per product).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "mynah-slm_amd"))

METRIC = "Q4_K/Q6_K GEMV HBM GB/s (% of peak); Qwen3 batch-1 decode tok/s, 1 GPU"
PEAK_HBM_GBS = 8000.0
PEAK_FP32_TFLOPS = 157.3
PEAK_INT8_TOPS = 5000.0
MALL_BYTES = 256 << 20
HEAD_EVERY = 10   # the roofline kernel's launch is timed in every tenth pass


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def algorithmic_bytes(m) -> int:
    import mynah_amd as M
    return m.rows * M.row_bytes(m.qtype, m.cols) + 4 * m.cols + 4 * m.rows


def upload_copies(M, w, copies: int):
    return [M.DeviceBuffer.from_array(w) for _ in range(copies)]


def warm_for(fn, ms: float = 100.0) -> None:
    """Run fn() until about `ms` of wall time has passed. The GPU's clocks
    rise under load; a short timed block right after an idle gap (the host
    making the next matrix) runs partly on low clocks (the 4B head class:
    4,131 GB/s so, 4,755 after 150 ms of launches)."""
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < ms:
        fn()


def gpu_sweep(M, CF, steps: int, warmup: int):
    """configs[1] sweep launched from C (no Python between launches)."""
    mats = CF.C2
    step_bytes = sum(algorithmic_bytes(m) for m in mats)
    copies = max(2, -(-2 * MALL_BYTES // step_bytes))
    ws, xs, ys = [], [], []
    for i, m in enumerate(mats):
        wseed, xseed = CF.matrix_seeds(M.substream, 0, i)
        ws.append(upload_copies(M, M.synth_blocks(m.qtype, wseed, m.rows, m.cols), copies))
        xs.append(M.DeviceBuffer.from_array(M.synth_normal(xseed, m.cols)))
        ys.append(M.DeviceBuffer(4 * m.rows))
    head = len(mats) - 1
    assert mats[head].rows == 151936
    w_ptrs = [b.ptr for copies_of in ws for b in copies_of]
    x_ptrs, y_ptrs = [b.ptr for b in xs], [b.ptr for b in ys]
    M.time_sweep(mats, w_ptrs, copies, x_ptrs, y_ptrs, max(1, warmup), -1)
    # The head's launch is bracketed by HIP events in every tenth pass of
    # the timed region (an event pair lengthens a pass by ~5.6 µs, so they
    # sample the passes rather than mark all of them).
    total_ms, head_ms = M.time_sweep(mats, w_ptrs, copies, x_ptrs, y_ptrs, steps, head,
                                     HEAD_EVERY)
    # Beside the timed block: 20 trials of the same sweep (median, spread),
    # and the hot-cache figure over one weight copy (144 MB: the MALL holds
    # most of it).
    trial_steps = max(1, steps // 20)
    trials = sorted(step_bytes * trial_steps / (M.time_sweep(mats, w_ptrs, copies, x_ptrs, y_ptrs,
                                                             trial_steps, -1)[0] * 1e-3) / 1e9
                    for _ in range(20))
    one = [ws[i][0].ptr for i in range(len(mats))]
    M.time_sweep(mats, one, 1, x_ptrs, y_ptrs, max(1, warmup), -1)
    hot_ms = M.time_sweep(mats, one, 1, x_ptrs, y_ptrs, steps, -1)[0] / steps
    extra = {"trials": {"count": 20, "steps_each": trial_steps,
                        "median_gbs": round(trials[10], 1), "min_gbs": round(trials[0], 1),
                        "max_gbs": round(trials[-1], 1)},
             "hot_cache_gbs": round(step_bytes / (hot_ms * 1e-3) / 1e9, 1)}

    # Per-matrix averages, each matrix alone over its rotating copies.
    per = {}
    for i, m in enumerate(mats):
        n = 8 * copies
        ms = M.time_matvec(m.qtype, [b.ptr for b in ws[i]], m.rows, m.cols, x_ptrs[i],
                           y_ptrs[i], n) / n
        per[m.name] = round(algorithmic_bytes(m) / (ms * 1e-3) / 1e9, 1)
    for b in [b for c in ws for b in c] + xs + ys:
        b.free()
    return step_bytes, copies, total_ms, head_ms, algorithmic_bytes(mats[head]), per, extra


def gpu_c1(M, CF, launches: int = 256):
    """the single Q4_K 1024 x 3072 matvec, weights rotated over
    enough device copies (> 2x MALL) that every launch streams from HBM;
    GB/s of algorithmic bytes over the average launch (HIP events around
    `launches` back-to-back launches)."""
    m = CF.C1[0]
    wseed, xseed = CF.matrix_seeds(M.substream, 0, 0)
    nbytes = algorithmic_bytes(m)
    copies = max(2, -(-2 * MALL_BYTES // nbytes))
    w = upload_copies(M, M.synth_blocks(m.qtype, wseed, m.rows, m.cols), copies)
    x = M.DeviceBuffer.from_array(M.synth_normal(xseed, m.cols))
    y = M.DeviceBuffer(4 * m.rows)
    ptrs = [b.ptr for b in w]
    n = max(launches, 2 * copies)
    warm_for(lambda: M.time_matvec(m.qtype, ptrs, m.rows, m.cols, x.ptr, y.ptr, copies))
    ms = M.time_matvec(m.qtype, ptrs, m.rows, m.cols, x.ptr, y.ptr, n) / n
    for b in w + [x, y]:
        b.free()
    return {"workload": "configs[0]: Q4_K 1024x3072 matvec, seed 0", "kernel":
            M.gemv_kernel(m.qtype, m.rows, m.cols), "bytes_per_launch": nbytes,
            "weight_copies": copies, "launches": n, "avg_launch_ms": round(ms, 5),
            "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "copy_ceiling_gbs": round(copy_ceiling(M, nbytes), 1),
            "read_ceiling_gbs": round(read_ceiling(M, nbytes), 1)}


def copy_ceiling(M, traffic: int, launches: int = 64) -> float:
    """GB/s of HBM traffic a plain device copy (mynah_copy16) reaches when
    each launch moves `traffic` bytes (reads traffic/2, writes traffic/2),
    launched back to back from rotating sources like the GEMVs: the
    practical per-launch ceiling at that size."""
    half = max(256, traffic // 2 // 256 * 256)
    copies = max(2, -(-2 * MALL_BYTES // half))
    src = [M.DeviceBuffer(half) for _ in range(copies)]
    dst = M.DeviceBuffer(half)
    for b in src:
        M.check(M.lib.mynah_hip_memset(b.ptr, 1, half), "memset")
    n = max(launches, 4 * copies)

    def one_pass():
        for i in range(copies):
            M.copy_dev(dst.ptr, src[i].ptr, half)
        M.sync()
    warm_for(one_pass)
    a, e = M.Event(), M.Event()
    a.record()
    for i in range(n):
        M.copy_dev(dst.ptr, src[i % copies].ptr, half)
    e.record()
    M.sync()
    ms = a.elapsed_ms(e) / n
    for b in src + [dst]:
        b.free()
    return 2 * half / (ms * 1e-3) / 1e9


def read_ceiling(M, nbytes: int, launches: int = 64) -> float:
    """GB/s a read-only stream (mynah_read16: every byte loaded once, nothing
    written) reaches when each launch reads `nbytes`, launched back to back
    from rotating sources (> 2x MALL) like the GEMVs: what one launch of a
    GEMV's size can read, whatever it computes."""
    size = max(256, nbytes // 256 * 256)
    copies = max(2, -(-2 * MALL_BYTES // size))
    src = [M.DeviceBuffer(size) for _ in range(copies)]
    sink = M.DeviceBuffer(256)
    for b in src:
        M.check(M.lib.mynah_hip_memset(b.ptr, 1, size), "memset")
    n = max(launches, 4 * copies)

    def one_pass():
        for i in range(copies):
            M.read_dev(src[i].ptr, size, sink.ptr)
        M.sync()
    warm_for(one_pass)
    a, e = M.Event(), M.Event()
    a.record()
    for i in range(n):
        M.read_dev(src[i % copies].ptr, size, sink.ptr)
    e.record()
    M.sync()
    ms = a.elapsed_ms(e) / n
    for b in src + [sink]:
        b.free()
    return size / (ms * 1e-3) / 1e9


def gpu_4b_classes(M, CF, launches: int = 64):
    """GB/s of each Qwen3-4B GEMV class, rotating copies totalling > 2x MALL,
    and beside it the copy and read-only ceilings for the same bytes per
    launch, and the kernel each class launches."""
    out, ceiling, rceiling, kernels = {}, {}, {}, {}
    for i, m in enumerate(CF.QWEN3_4B_GEMV):
        wseed, xseed = CF.matrix_seeds(M.substream, 4, i)
        nbytes = algorithmic_bytes(m)
        copies = max(2, -(-2 * MALL_BYTES // nbytes))
        w = upload_copies(M, M.synth_blocks(m.qtype, wseed, m.rows, m.cols), copies)
        x = M.DeviceBuffer.from_array(M.synth_normal(xseed, m.cols))
        y = M.DeviceBuffer(4 * m.rows)
        ptrs = [b.ptr for b in w]
        n = max(launches, 4 * copies)
        warm_for(lambda: M.time_matvec(m.qtype, ptrs, m.rows, m.cols, x.ptr, y.ptr, copies))
        ms = M.time_matvec(m.qtype, ptrs, m.rows, m.cols, x.ptr, y.ptr, n) / n
        out[m.name] = round(nbytes / (ms * 1e-3) / 1e9, 1)
        for b in w + [x, y]:
            b.free()
        ceiling[m.name] = round(copy_ceiling(M, nbytes, launches), 1)
        rceiling[m.name] = round(read_ceiling(M, nbytes, launches), 1)
        kernels[m.name] = M.gemv_kernel(m.qtype, m.rows, m.cols)
    return out, ceiling, rceiling, kernels


def forced_check(dec, g, k, v, npre):
    """The teacher-forced golden run of configs[2] (64 uniform-random inputs
    after the 512-position prefill, logits from the compiled reference)
    through the replayed step graphs: every step's greedy id, and the last
    step's logits (whole vector by SHA-256, the golden top-64 and every
    293rd logit by relative error)."""
    import hashlib
    import numpy as np
    dec.reset()
    dec.set_kv(k, v, npre)
    greedy, last = dec.forced([int(t) for t in g["inputs"]])
    ref = np.concatenate([g["top_vals"][-1], g["sample"][-1]]).astype(np.float64)
    got = np.concatenate([last[g["top_ids"][-1]], last[::293]]).astype(np.float64)
    err = float((np.abs(got - ref) / np.maximum(1.0, np.abs(ref))).max())
    return {"greedy_ids_match": greedy == [int(t) for t in g["greedy"]],
            "last_logits_bit_identical":
                hashlib.sha256(last.tobytes()).hexdigest() == str(g["logits_sha"][-1]),
            "last_logits_sample_max_rel_err": err,
            "sample": "the golden's top-64 ids and every 293rd id of the last step (0.4 % of "
                      "the vocabulary); the whole vector is compared by its SHA-256"}


def gpu_decode(M, CF):
    """Qwen3-0.6B batch-1 greedy decode, 512 prefilled positions,
    64 steps, in three numerics modes; the generated ids checked against the
    compiled reference's, and each mode run again teacher-forced over the
    golden's 64 random inputs (forced_check)."""
    import numpy as np
    shape, npre, steps = CF.QWEN3_06B, CF.C3_PREFILL, CF.C3_STEPS
    model = M.SynthQwen3(shape, 0)
    k, v = CF.kv_prefill(M.substream, M.synth_normal, shape, 0, npre)
    first = M.first_token(0, shape.vocab)
    golden = np.load(os.path.join(ROOT, "tests", "golden", "qwen3_06b.npz"), allow_pickle=False)
    forced = np.load(os.path.join(ROOT, "tests", "golden", "qwen3_06b_forced.npz"),
                     allow_pickle=False)
    want = [int(t) for t in golden["tokens"]]
    out = {"model": "Qwen3-0.6B random-init Q4_K_M mix", "prefill": npre, "steps": steps,
           "weight_bytes": model.weight_bytes()}
    old = M.lib.mynah_hip_gemv_order()
    try:
        for order, attn, name in ((0, M.ATTN_EXACT, "exact"),
                                  (0, M.ATTN_SPLIT, "exact_gemv_split_attention"),
                                  (1, M.ATTN_SPLIT, "reordered_gemv_split_attention")):
            M.check(M.lib.mynah_hip_set_gemv_order(order), "order")
            dec = M.Qwen3Decoder(model, npre + steps + 1)
            dec.set_attention(attn)
            dec.set_kv(k, v, npre)
            dec.generate(first, 4)                       # warm-up and graph capture
            dec.reset()
            dec.set_kv(k, v, npre)
            toks, ms = dec.generate(first, steps)
            out[name] = {"tok_s": round(steps / ms * 1e3, 1), "ms_per_token": round(ms / steps, 4),
                         "tokens_match_reference": toks == want, "graph": dec.uses_graph,
                         "teacher_forced": forced_check(dec, forced, k, v, npre)}
            dec.close()
        out["sampled"] = sampled_decode(M, model, k, v, npre, first, steps)
    finally:
        M.check(M.lib.mynah_hip_set_gemv_order(old), "order")
    head = out["exact"]
    out["headline"] = {"mode": "exact", "tok_s": head["tok_s"],
                       "target_tok_s": 1000.0, "meets_target": head["tok_s"] > 1000.0,
                       "tokens_match_reference": head["tokens_match_reference"],
                       "logits_bit_identical": head["teacher_forced"]["last_logits_bit_identical"],
                       "note": "every GEMV and the attention in the reference's operation order: "
                               "logits bit-identical to the compiled reference's (SHA-256 of the "
                               "whole vector). The split-attention modes take the softmax per "
                               "32-position chunk: outside the 1e-4 per-element bar on whole "
                               "vectors (up to 1.8e-4 at configs[2], 2.9e-4 at configs[4] in "
                               "tests/test_decode_forced_gpu.py), reported for comparison only"}
    return out


def sampled_decode(M, model, k, v, npre, first, steps):
    """The same workload through the generation loop (exact mode, chunks of
    eight steps per host round trip) with the front ends' default sampler
    (Qwen3's temp 0.6, top_k 20, top_p 0.95; src/sampler.c:27-36) on the
    device, beside greedy through the same loop. Its ids are the reference
    sampler's (tests/test_sampler_gpu.py); here only the rate."""
    params = dict(temp=0.6, top_k=20, top_p=0.95, seed=0)
    res = {"sampler": "temp 0.6, top_k 20, top_p 0.95, seed 0, on the device"}
    for name in ("greedy", "sampled"):
        dec = M.Qwen3Decoder(model, npre + steps + 1)
        dec.set_attention(M.ATTN_EXACT)
        for rep in range(2):                             # the first captures the graphs
            smp = M.DeviceSampler(model.shape.vocab, **params) if name == "sampled" else None
            dec.reset()
            dec.set_kv(k, v, npre)
            _, n, t = dec.generate_tokens([first], steps, device_sampler=smp)
            if smp is not None:
                smp.close()
        res[name + "_tok_s"] = round(n / t.decode_s, 1)
        dec.close()
    return res


def gpu_prefill_gemm(M, CF, reps: int = 20, int8: bool = False):
    """the prefill GEMMs at Qwen3-1.7B shapes, 512 tokens.
    int8=False: the exact batched order (bit-identical to the reference's
    exact matmat). int8=True: the Q4_K products take the int8 activation lane
    (bit-identical to the reference's AVX2 build, whose batched default it
    is), quantisation included in the time; Q6_K stays exact, as there."""
    out, tot_flop, tot_ms = {}, 0, 0.0
    M.set_int8(M.INT8_BATCHED if int8 else M.INT8_OFF)
    bufs = []
    try:
        # Every operand is made and resident before any GEMM runs, and the
        # six products run back to back for about 100 ms before the first
        # timed block: a prefill's GEMMs follow each other, and an idle gap
        # before a short timed block (the host making the next matrix) left
        # the GPU's clocks low for it (44 against 50 TFLOP/s measured).
        for i, m in enumerate(CF.C4):
            wseed, _ = CF.matrix_seeds(M.substream, 0, i)
            w = M.DeviceBuffer.from_array(M.synth_blocks(m.qtype, wseed, m.rows, m.cols))
            x = M.DeviceBuffer.from_array(M.synth_normal(M.substream(0, CF.PREFILL_X_INDEX + i),
                                                         CF.C4_TOKENS * m.cols))
            y = M.DeviceBuffer(4 * m.rows * CF.C4_TOKENS)
            bufs.append((m, w, x, y))
        run = lambda m, w, x, y: M.matmat_dev(m.qtype, w.ptr, m.rows, m.cols, x.ptr, y.ptr,
                                               CF.C4_TOKENS)
        a, b = M.Event(), M.Event()
        a.record()
        warm = 0
        while True:
            for args in bufs:
                run(*args)
            warm += 1
            b.record()
            M.sync()
            if a.elapsed_ms(b) >= 100.0 or warm >= 200:
                break
        for m, w, x, y in bufs:
            n = reps * (4 if int8 else 1)
            a, b = M.Event(), M.Event()
            a.record()
            for _ in range(n):
                run(m, w, x, y)
            b.record()
            M.sync()
            ms = a.elapsed_ms(b) / n
            flop = 2 * m.rows * m.cols * CF.C4_TOKENS
            tot_flop += flop
            tot_ms += ms
            lane = "int8" if (int8 and m.qtype == CF.Q4_K) else "exact"
            out[m.name] = {"ms": round(ms, 4), "tflop_s": round(flop / ms / 1e9, 2), "lane": lane}
    finally:
        for _, w, x, y in bufs:
            for buf in (w, x, y):
                buf.free()
        M.set_int8(M.INT8_OFF)
    res = {"workload": "configs[3]: Q4_K 4096/2048/2048/6144/6144 x 2048 and Q6_K 2048 x 6144, "
                       "512 tokens, " + ("Q4_K on the int8 activation lane" if int8
                                         else "exact batched order"),
           "total_ms": round(tot_ms, 4), "flop": tot_flop,
           "tflop_s": round(tot_flop / tot_ms / 1e9, 2), "per_matrix": out}
    if int8:
        q4 = [v for v in out.values() if v["lane"] == "int8"]
        q4_ms = sum(v["ms"] for v in q4)
        q4_flop = sum(2 * m.rows * m.cols * CF.C4_TOKENS for m in CF.C4 if m.qtype == CF.Q4_K)
        res.update({"q4k_int8_ms": round(q4_ms, 4),
                    "q4k_int8_top_s": round(q4_flop / q4_ms / 1e9, 2),
                    "peak_top_s_int8": PEAK_INT8_TOPS,
                    "frac_of_int8_peak": round(q4_flop / q4_ms / 1e9 / PEAK_INT8_TOPS, 4),
                    "note": "integer dots on v_mfma_i32_16x16x32_i8; the reference's f32 "
                            "epilogue (a convert and two fma per dot) bounds it on the VALU"})
    else:
        res.update({"peak_tflop_s_fp32": PEAK_FP32_TFLOPS,
                    "frac_of_fp32_peak": round(tot_flop / tot_ms / 1e9 / PEAK_FP32_TFLOPS, 4),
                    "note": "one mul and one add per product (the reference's roundings): the "
                            "non-packed VALU issue rate bounds this order near 40 TFLOP/s"})
    return res


def c5_golden_ids():
    """The 256 greedy ids of configs[4] from the compiled reference
    (tests/golden/qwen3_4b_c5.npz), or None when that golden is absent."""
    import numpy as np
    path = os.path.join(ROOT, "tests", "golden", "qwen3_4b_c5.npz")
    if not os.path.exists(path):
        return None
    return [int(t) for t in np.load(path, allow_pickle=False)["greedy"]]


def gpu_qwen3_4b(M, CF):
    """Qwen3-4B random-init Q4_K_M mix, a 2048-token prompt of
    uniform ids, then 256 greedy steps; tok/s as the reference's timing.c
    defines them (prompt tokens / prefill time, generated tokens / decode
    time). The prompt's 2047 cache-filling tokens are prefilled in batches
    (matvec-order GEMMs, per-query attention: the cache bit-identical to
    2047 decode steps without the head); the decode steps run in the mode
    named."""
    shape = CF.QWEN3_4B
    model = M.SynthQwen3(shape, 0)
    prompt = CF.c5_prompt(M.synth_uniform, M.substream, shape.vocab)
    want = c5_golden_ids()
    out = {"model": "Qwen3-4B random-init Q4_K_M mix", "prompt": int(prompt.size),
           "steps": CF.C5_STEPS, "weight_bytes": model.weight_bytes()}
    old = M.lib.mynah_hip_gemv_order()
    try:
        for order, attn, name in ((0, M.ATTN_EXACT, "exact"),
                                  (0, M.ATTN_SPLIT, "exact_gemv_split_attention"),
                                  (1, M.ATTN_SPLIT, "reordered_gemv_split_attention")):
            M.check(M.lib.mynah_hip_set_gemv_order(order), "order")
            dec = M.Qwen3Decoder(model, int(prompt.size) + CF.C5_STEPS + 1)
            dec.set_attention(attn)
            dec.prompt(prompt[:4], 4)                    # warm-up and graph captures
            dec.reset()
            toks, pre_ms, dec_ms = dec.prompt(prompt, CF.C5_STEPS)
            out[name] = {"prefill": "batched",
                         "prefill_tok_s": round(prompt.size / (pre_ms * 1e-3), 1),
                         "decode_tok_s": round(CF.C5_STEPS / (dec_ms * 1e-3), 1),
                         "prefill_ms": round(pre_ms, 2), "decode_ms": round(dec_ms, 2),
                         "first_tokens": toks[:4],
                         "tokens_match_reference": None if want is None else toks == want}
            dec.close()
    finally:
        M.check(M.lib.mynah_hip_set_gemv_order(old), "order")
    return out


def gpu_decode_4b(M, CF, steps: int):
    """configs[4]'s decode alone in the headline mode (exact: logits
    bit-identical to the reference's): the 2048-token prompt prefilled in
    batches, then `steps` greedy steps; one warm-up prompt first (graph
    captures)."""
    shape = CF.QWEN3_4B
    model = M.SynthQwen3(shape, 0)
    prompt = CF.c5_prompt(M.synth_uniform, M.substream, shape.vocab)
    dec = M.Qwen3Decoder(model, int(prompt.size) + steps + 1)
    dec.set_attention(M.ATTN_EXACT)
    dec.prompt(prompt[:4], 4)
    dec.reset()
    toks, pre_ms, dec_ms = dec.prompt(prompt, steps)
    dec.close()
    want = c5_golden_ids()
    return {"model": "Qwen3-4B random-init Q4_K_M mix", "mode": "exact",
            "prompt": int(prompt.size), "steps": steps, "decode_ms": round(dec_ms, 2),
            "decode_tok_s": round(steps / (dec_ms * 1e-3), 1), "first_tokens": toks[:4],
            "tokens_match_reference": None if want is None else
            toks[:len(want)] == want[:len(toks)]}


def gpu_prefill_4b(M, CF, reps: int = 3):
    """configs[4]'s prompt prefill alone: the 2047 cache-filling tokens of
    the 2048-token prompt through mynah_hip_qwen3_prefill (batched), best of
    `reps` after a warm-up; also the same prefill as 2047 decode steps."""
    shape = CF.QWEN3_4B
    model = M.SynthQwen3(shape, 0)
    prompt = CF.c5_prompt(M.synth_uniform, M.substream, shape.vocab)
    n = int(prompt.size) - 1
    dec = M.Qwen3Decoder(model, int(prompt.size) + 8)
    dec.prefill(prompt[:64])
    best = None
    for _ in range(reps):
        dec.reset()
        t0 = time.perf_counter()
        dec.prefill(prompt[:n])
        ms = (time.perf_counter() - t0) * 1e3
        best = ms if best is None else min(best, ms)
    dec.close()
    return {"model": "Qwen3-4B random-init Q4_K_M mix", "tokens": n, "ms": round(best, 2),
            "tok_s": round(n / (best * 1e-3), 1),
            "note": "batched prefill (mynah_hip_qwen3_prefill): K/V cache bit-identical to "
                    "token-by-token decode steps; wall time of the call, host sync included"}


def host_cpus() -> dict:
    """The host cores the CPU leg may use: every core of this process's
    affinity set (src/threads.c:27-41 starts the pool on all online cores),
    capped by the CPU share the host grants the job (a cgroup quota, or
    OMP_NUM_THREADS where the batch system sets it to that share)."""
    aff = sorted(os.sched_getaffinity(0))
    sockets = set()
    for c in aff:
        try:
            with open(f"/sys/devices/system/cpu/cpu{c}/topology/physical_package_id") as f:
                sockets.add(f.read().strip())
        except OSError:
            pass
    quota = None
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            q, period = f.read().split()[:2]
        if q != "max":
            quota = int(q) / int(period)
    except (OSError, ValueError):
        pass
    threads = len(aff)
    if quota is not None:
        threads = min(threads, max(1, int(quota)))
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        threads = min(threads, int(omp))
    return {"online": os.cpu_count(), "affinity": len(aff), "sockets": len(sockets) or None,
            "cgroup_quota_cpus": quota, "omp_num_threads": omp or None, "threads": threads}


RUNS = 5   # every CPU leg is measured this many times and reports the median


def _timed_passes(fn, seconds: float, min_reps: int = 1):
    reps, t0 = 0, time.perf_counter()
    while True:
        fn()
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds and reps >= min_reps:
            return reps, el


def _runs(rates):
    """The median of a leg's runs, with the spread beside it."""
    import statistics
    r = sorted(rates)
    return {"median": round(statistics.median(r), 2), "min": round(r[0], 2),
            "max": round(r[-1], 2), "runs": len(r)}


def cpu_sweep(O, CF, mats, seconds: float, avx2: bool = False):
    """GB/s of the oracle's threaded projection (4*nth row chunks, serial
    below 64 rows: src/arch_qwen3.c:52-83) over the matrices of a config:
    RUNS runs of about `seconds` each after one warm-up pass. avx2 takes the
    restated f32 lanes of an AVX2 + FMA ingot build instead of the as-built
    scalar ones."""
    data = []
    for i, m in enumerate(mats):
        ws, xs = CF.matrix_seeds(O.substream, 0, i)
        data.append((m, O.blocks(m.qtype, ws, m.rows, m.cols), O.normal(xs, m.cols)))
    step_bytes = sum(algorithmic_bytes(m) for m in mats)
    proj = O.project_avx2 if avx2 else O.project

    def one():
        for m, w, x in data:
            proj(m.qtype, w, m.rows, m.cols, x)
    one()                                      # warm-up pass
    rates, passes, total = [], 0, 0.0
    for _ in range(RUNS):
        reps, el = _timed_passes(one, seconds)
        rates.append(step_bytes * reps / el / 1e9)
        passes, total = passes + reps, total + el
    return step_bytes, rates, passes, total


def _greedy_runs(O, orc, tok, steps_per_run):
    """RUNS runs of `steps_per_run` greedy steps continuing one sequence
    (first-index argmax, src/sampler.c:124-129); decode tok/s as
    src/timing.c:52-54 defines it (generated ids / decode seconds)."""
    toks, rates, total = [], [], 0.0
    for _ in range(RUNS):
        t0 = time.perf_counter()
        for _ in range(steps_per_run):
            lg = orc.forward(tok)
            tok = int(O.orc.orc_argmax(O.ptr(lg), lg.size))
            toks.append(tok)
        el = time.perf_counter() - t0
        rates.append(steps_per_run / el)
        total += el
    return toks, rates, total


def cpu_decode(O, CF):
    """configs[2] on the CPU: the oracle decoder (the restated
    src/arch_qwen3.c:178-252 on the pool, bit-identical to the compiled
    reference) from the 512-position prefill, RUNS runs of 8 greedy steps;
    the 40 ids must match the golden run's."""
    import numpy as np
    shape, per = CF.QWEN3_06B, 8
    orc = O.OracleQwen3(O.SynthModel(shape, 0), CF.C3_PREFILL + RUNS * per + 1)
    k, v = O.kv_prefill(O.substream, shape, 0, CF.C3_PREFILL)
    orc.prefill_kv(k, v, CF.C3_PREFILL)
    del k, v
    want = [int(t) for t in np.load(os.path.join(ROOT, "tests", "golden", "qwen3_06b.npz"),
                                    allow_pickle=False)["tokens"]]
    toks, rates, total = _greedy_runs(O, orc, O.first_token(0, shape.vocab), per)
    del orc
    return {"tok_s": _runs(rates), "steps": len(toks), "seconds": round(total, 2),
            "context": f"{CF.C3_PREFILL}..{CF.C3_PREFILL + len(toks)}",
            "tokens_match_reference": toks == want[:len(toks)]}


def cpu_decode_4b(O, CF):
    """configs[4]'s decode on the CPU: the oracle decoder over the Qwen3-4B
    model with 2048 KV positions (filled with N(0, 1): a step's work depends
    on the context length only), RUNS runs of 2 greedy steps; the ids must
    match the compiled reference's on the same inputs."""
    import numpy as np
    shape, npre = CF.QWEN3_4B, CF.C5_CPU_KV
    per = CF.C5_CPU_STEPS // RUNS
    orc = O.OracleQwen3(O.SynthModel(shape, 0), npre + CF.C5_CPU_STEPS + 1)
    k, v = O.kv_prefill(O.substream, shape, 0, npre)
    orc.prefill_kv(k, v, npre)
    del k, v
    want = [int(t) for t in np.load(os.path.join(ROOT, "tests", "golden", "qwen3_4b_kv2048.npz"),
                                    allow_pickle=False)["tokens"]]
    toks, rates, total = _greedy_runs(O, orc, O.first_token(0, shape.vocab), per)
    del orc
    return {"tok_s": _runs(rates), "steps": len(toks), "seconds": round(total, 2),
            "context": f"{npre}..{npre + len(toks)}",
            "tokens_match_reference": toks == want[:len(toks)]}


def cpu_prefill_gemm(O, CF):
    """configs[3] on the CPU: the six exact batched products (the reference's
    ingot matmat order) with the pool injected over 8-row strips
    (third_party/ingot/src/cpu.c:217-230), 512 tokens; RUNS passes over the
    six, GFLOP/s of each pass."""
    data = []
    for i, m in enumerate(CF.C4):
        wseed, _ = CF.matrix_seeds(O.substream, 0, i)
        data.append((m, O.blocks(m.qtype, wseed, m.rows, m.cols),
                     O.normal(O.substream(0, CF.PREFILL_X_INDEX + i), CF.C4_TOKENS * m.cols)))
    flop = sum(2 * m.rows * m.cols * CF.C4_TOKENS for m in CF.C4)
    rates, total = [], 0.0
    for _ in range(RUNS):
        t0 = time.perf_counter()
        for m, w, x in data:
            O.matmat(m.qtype, w, m.rows, m.cols, x, CF.C4_TOKENS, threaded=True)
        el = time.perf_counter() - t0
        rates.append(flop / el / 1e9)
        total += el
    return {"gflop_s": _runs(rates), "seconds": round(total, 2)}


def cpu_baseline(CF, seconds: float = 10.0):
    """The CPU oracle (the C11 restatement of the reference's as-built
    kernels and decoder, bit-identical to it) on this host's cores, each leg
    the median of RUNS runs: the configs[1] sweep (the metric's value, about
    `seconds` in all) and the same sweep in the AVX2 + FMA lanes' order,
    configs[0], configs[2] and configs[4] decode, configs[3]'s batched
    products."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O
    cpus = host_cpus()
    threads = O.orc.orc_threads_init(cpus["threads"])
    try:
        step_bytes, rates, passes, el = cpu_sweep(O, CF, CF.C2, seconds / RUNS)
        _, a_rates, a_passes, a_el = cpu_sweep(O, CF, CF.C2, seconds / (2 * RUNS), avx2=True)
        c1_bytes, c1_rates, c1_passes, c1_el = cpu_sweep(O, CF, CF.C1, seconds / (4 * RUNS))
        decode = cpu_decode(O, CF)
        decode_4b = cpu_decode_4b(O, CF)
        gemm = cpu_prefill_gemm(O, CF)
    finally:
        O.orc.orc_threads_shutdown()
    sweep = _runs(rates)
    return {"value": sweep["median"], "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": f"median of {RUNS} runs (GB/s {sweep['min']}..{sweep['max']}), "
                      f"{passes} passes of the configs[1] sweep ({step_bytes / 1e6:.1f} MB "
                      f"each) in {el:.1f} s, oracle restatement (bit-identical to the "
                      f"as-built reference: ingot's scalar lanes) with 4*nth row chunks on "
                      f"{threads} threads",
            "host": cpus,
            "configs1_avx2_order_gbs": _runs(a_rates),
            "configs1_avx2_order_sample": f"{a_passes} passes in {a_el:.1f} s of the same sweep "
                                          "in the f32 lanes of an AVX2 + FMA ingot build "
                                          "(restated, bit-identical to such a build)",
            "configs0_gbs": _runs(c1_rates),
            "configs0_sample": f"{c1_passes} matvecs of Q4_K 1024x3072 in {c1_el:.1f} s",
            "configs2_decode": decode,
            "configs4_decode": decode_4b,
            "configs3_prefill_gemm": gemm}


def pmc_probe(M, CF, launches: int = 8) -> None:
    """A short program for rocprofv3 --pmc runs: `launches` head GEMVs over two
    weight copies in the current GEMV order, then four 256 MiB device copies
    (mynah_copy16) whose known bytes calibrate FETCH_SIZE / WRITE_SIZE."""
    m = CF.C2[-1]
    wseed, xseed = CF.matrix_seeds(M.substream, 0, len(CF.C2) - 1)
    w = upload_copies(M, M.synth_blocks(m.qtype, wseed, m.rows, m.cols), 2)
    x = M.DeviceBuffer.from_array(M.synth_normal(xseed, m.cols))
    y = M.DeviceBuffer(4 * m.rows)
    M.time_matvec(m.qtype, [b.ptr for b in w], m.rows, m.cols, x.ptr, y.ptr, launches)
    nbytes = 256 << 20
    a, b = M.DeviceBuffer(nbytes), M.DeviceBuffer(nbytes)
    M.check(M.lib.mynah_hip_memset(a.ptr, 1, nbytes), "memset")
    for _ in range(4):
        M.copy_dev(b.ptr, a.ptr, nbytes)
    M.sync()
    log(f"[pmc-probe] {launches} head launches ({algorithmic_bytes(m)} algorithmic bytes each), "
        f"4 copies of {nbytes} bytes (mynah_copy16)")


def valu_yardstick(M, prefill) -> dict:
    """The exact orders pay one non-packed v_add_f32 per product: the time per
    wave64 add (every SIMD issuing only adds) bounds the exact GEMM at
    2 flops x 64 lanes / t per SIMD. Measured twice, the faster kept."""
    ns, simds = min(M.valu_add_rate() for _ in range(2))
    ceiling = 2.0 * 64.0 / (ns * 1e-9) * simds / 1e12
    out = {"f32_add_ns_per_wave64_per_simd": round(ns, 4), "simds": simds,
           "exact_gemm_ceiling_tflop_s": round(ceiling, 1)}
    if prefill is not None:
        out["exact_gemm_frac_of_ceiling"] = round(prefill["tflop_s"] / ceiling, 3)
    return out


def traffic_for(name: str):
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        t = json.load(f)
    entry = t.get(name)
    return None if entry is None else entry.get("hbm_bytes_per_launch")


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-4b", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-4b-e2e", action="store_true")
    ap.add_argument("--decode-only", action="store_true",
                    help="only the configs[2] decode section, printed as one JSON line")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the configs[4] batched prompt prefill, printed as one JSON line")
    ap.add_argument("--decode-4b-only", action="store_true",
                    help="only configs[4]'s decode (2048-token prompt, then --steps greedy "
                         "steps, exact GEMV + split attention), printed as one JSON line")
    ap.add_argument("--gemm-only", action="store_true",
                    help="only the configs[3] GEMMs (exact, then the int8 lane), printed as "
                         "one JSON line")
    ap.add_argument("--classes-only", action="store_true",
                    help="only the Qwen3-4B GEMV classes with their copy and read-only "
                         "ceilings, printed as one JSON line")
    ap.add_argument("--pmc-probe", action="store_true",
                    help="only the head GEMV + calibration copies, for rocprofv3 --pmc")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported here "
              "(the multi-GPU sharding is a design note, not a measured path)", file=sys.stderr)
        return 2

    import configs as CF
    import mynah_amd as M
    M.check(M.lib.mynah_hip_init(0), "init")
    order = M.lib.mynah_hip_gemv_order()
    if args.pmc_probe:
        pmc_probe(M, CF)
        return 0
    if args.prefill_only:
        print(json.dumps({"prefill_4b": gpu_prefill_4b(M, CF)}), flush=True)
        return 0
    if args.decode_only:
        print(json.dumps({"decode": gpu_decode(M, CF)}), flush=True)
        return 0
    if args.gemm_only:
        pg = gpu_prefill_gemm(M, CF)
        print(json.dumps({"prefill_gemm": pg,
                          "prefill_gemm_int8": gpu_prefill_gemm(M, CF, int8=True),
                          "valu": valu_yardstick(M, pg)}), flush=True)
        return 0
    if args.classes_only:
        g, c, r, k = gpu_4b_classes(M, CF)
        print(json.dumps({"qwen3_4b_gemv_gbs": g, "copy_ceiling_gbs": c, "read_ceiling_gbs": r,
                          "kernels": k, "configs0": gpu_c1(M, CF)}), flush=True)
        return 0
    if args.decode_4b_only:
        print(json.dumps({"decode_4b": gpu_decode_4b(M, CF, args.steps)}), flush=True)
        return 0

    log("[bench] configs[1] sweep")
    step_bytes, copies, total_ms, head_ms, head_bytes, per, sweep_extra = gpu_sweep(
        M, CF, args.steps, args.warmup)
    ms_per_step = total_ms / args.steps
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    achieved = head_bytes / (head_ms * 1e-3) / 1e9

    log("[bench] configs[0] Q4_K matvec")
    c1 = gpu_c1(M, CF)

    decode = None
    if not args.no_decode:
        log("[bench] configs[2] decode")
        decode = gpu_decode(M, CF)

    prefill = prefill_int8 = None
    if not args.no_prefill:
        log("[bench] configs[3] prefill GEMM")
        prefill = gpu_prefill_gemm(M, CF)
        log("[bench] configs[3] prefill GEMM, int8 lane")
        prefill_int8 = gpu_prefill_gemm(M, CF, int8=True)

    e2e_4b = None
    if not args.no_4b_e2e:
        log("[bench] configs[4] Qwen3-4B end to end")
        e2e_4b = gpu_qwen3_4b(M, CF)

    extra_4b = ceiling_4b = rceiling_4b = kernels_4b = None
    if not args.no_4b:
        log("[bench] Qwen3-4B GEMV classes")
        extra_4b, ceiling_4b, rceiling_4b, kernels_4b = gpu_4b_classes(M, CF)

    log("[bench] VALU add rate")
    valu = valu_yardstick(M, prefill)

    cpu = None
    if not args.no_cpu:
        log("[bench] CPU baseline")
        cpu = cpu_baseline(CF, args.cpu_seconds)

    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "configs[1]: Q6_K + Q8_0 matvec at Qwen3-0.6B shapes (2048x1024, "
                        "1024x1024, 1024x2048, 3072x1024) + Q6_K 151936x1024 head, seed 0",
            "gemv_order": "exact (bit-identical to the reference)" if order == 0 else "reordered",
            "weight_copies": copies,
            "step_bytes": step_bytes,
        },
        "roofline": {
            "kernel": M.gemv_kernel(CF.Q6_K, 151936, 1024) + " (Q6_K 151936x1024 head)",
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": traffic_for("q6k_head_151936x1024"),
            "bytes_per_launch": head_bytes,
            "avg_launch_ms": round(head_ms, 5),
        },
        "cpu_baseline": cpu,
        "configs0": c1,
        "decode": decode,
        "prefill_gemm": prefill,
        "prefill_gemm_int8": prefill_int8,
        "qwen3_4b_end_to_end": e2e_4b,
        "sweep": sweep_extra,
        "per_matrix_gbs": per,
        "qwen3_4b_gemv_gbs": extra_4b,
        "qwen3_4b_copy_ceiling_gbs": ceiling_4b,
        "qwen3_4b_read_ceiling_gbs": rceiling_4b,
        "qwen3_4b_gemv_kernels": kernels_4b,
        "valu": valu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
