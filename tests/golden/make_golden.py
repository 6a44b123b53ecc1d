"""Write the golden vectors under tests/golden/ from the COMPILED REFERENCE.

Run in a container where /root/reference exists and `make -C oracle` has built
oracle/_ref/libref.so (the reference's own C sources, compiled unchanged). The
outputs are plain arrays (.npz without pickles) plus the ingot test fixtures
(data files of the reference's own test suite, copied as data).

    python tests/golden/make_golden.py

Cases (inputs are regenerated from seeds by the shared generator; the npz also
records a SHA-256 of the input bytes so generator drift is detected):
  kernels_small.npz  per type: matvec, exact matmat (3 tokens), dequant on
                     37 x 512 (Q8_0 also 37 x 96, a ragged block count)
  c1.npz             configs[0]: Q4_K 1024 x 3072 matvec, seed 0
  c2.npz             configs[1]: Q6_K / Q8_0 sweep; the 151936-row head as a
                     SHA-256 of its output bits plus every 97th row
  matmat.npz         batched exact order at prefill-like widths
  qwen3_tiny.npz     3-layer model: 32 greedy steps, first-step logits
  qwen3_06b.npz      configs[2]: 0.6B, KV prefill 512, 64 greedy steps,
                     first-step logits' top 64 and the SHA-256 of all of them
  qwen3_06b_forced.npz  configs[2]'s model and KV prefill, 64 teacher-forced
                     steps (uniform random inputs): every step's greedy id,
                     top-64 logits, every 293rd logit and SHA-256
                     (`--only forced` writes just this file)
  qwen3_4b_c5.npz    configs[4] end to end (2048-token prompt, 256 greedy
                     steps): every step's greedy id, the top-64 logits of
                     seven snapshot steps (`--only c5full`; not part of the
                     default run: about ten minutes of CPU)
  qwen3_4b_kv2048.npz  configs[4]'s model with 2048 N(0, 1) KV positions, the
                     greedy ids of 10 steps (the CPU baseline's 4B decode
                     leg checks its ids against them; `--only c5kv`)
  qwen3_4b_prompt.npz  configs[4]'s model (Qwen3-4B): the first 8 prompt ids,
                     prefill + 8 greedy steps, the first step's logits' top 64
                     (`--only c5` writes just this file)
  adjacent.npz       Q5_K and Q4_0 (configs.ADJACENT): matvec, batched
                     products and dequant of every shape (`--only adjacent`
                     writes just this file and those types' fixtures)
  int8.npz           the int8 activation lane of an AVX2 + FMA build of ingot
                     (oracle/_ref/libref_int8.so, INGOT_SDOT=1): Q4_K matvec
                     and batched outputs, incl. round-half-even ties, an
                     all-zero block and token counts around the token tile,
                     and Q5_K batched outputs
                     (`--only int8` writes just this file)
  generate_cases.json  the reference's generation loop (src/generate.c:13-86,
                     compiled, on the tiny model with a vocabulary): for each
                     case its prompt, limits, EOS ids, think markers, callback
                     stop and sampler, and what the loop did — the ids each
                     channel's callback saw, the count it returned, the
                     timing's generated count, the state's position
                     (`--only generate`)
  avx2.npz           the f32 AVX2 + FMA lanes of the same build (INGOT_SDOT=0,
                     in a process of its own): Q4_K, Q6_K and Q8_0 matvec on
                     small shapes, and configs[1]'s sweep as a SHA-256 of each
                     output plus every 97th row (`--only avx2`)
"""
from __future__ import annotations

import hashlib
import os
import shutil
import subprocess
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "tests"))
sys.path.insert(0, os.path.join(ROOT, "mynah-slm_amd"))

import configs as CF  # noqa: E402
import oracle_lib as O  # noqa: E402

REF_FIXTURES = "/root/reference/third_party/ingot/tests/fixtures"


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def ref_matvec(ref, t, w, rows, cols, x):
    y = np.empty(rows, np.float32)
    assert ref.ref_matvec(t, O.ptr(w), rows, cols, O.ptr(x), O.ptr(y)) == 0
    return y


def ref_matmat(ref, t, w, rows, cols, x, tokens):
    y = np.empty(rows * tokens, np.float32)
    assert ref.ref_matmat(t, O.ptr(w), rows, cols, O.ptr(x), O.ptr(y), tokens) == 0
    return y


def ref_dequant(ref, t, w, rows, cols):
    y = np.empty(rows * cols, np.float32)
    assert ref.ref_dequant_matrix(t, O.ptr(w), rows, cols, O.ptr(y)) == 0
    return y


def golden_c5(ref) -> None:
    shape = CF.QWEN3_4B
    model = O.SynthModel(shape, 0)
    prompt = CF.c5_prompt(O.uniform, O.substream, shape.vocab, CF.C5_GOLDEN_PROMPT)
    steps = CF.C5_GOLDEN_STEPS
    toks, lg = O.ref_prompt_greedy(ref, model, prompt, steps, CF.C5_GOLDEN_PROMPT + steps + 1)
    top = np.argsort(-lg, kind="stable")[:64]
    np.savez_compressed(os.path.join(HERE, "qwen3_4b_prompt.npz"), prompt=prompt.astype(np.uint32),
                        tokens=np.array(toks, np.uint32), top_ids=top.astype(np.uint32),
                        top_vals=lg[top], logits0_sha=np.array(sha(lg)),
                        blob_sha=np.array(sha(model.blob)))


def golden_c5_kv(ref) -> None:
    """configs[4]'s model with 2048 N(0, 1) KV positions, then the greedy ids
    of C5_CPU_STEPS steps: the check of the CPU baseline's 4B decode leg."""
    shape, npre, steps = CF.QWEN3_4B, CF.C5_CPU_KV, CF.C5_CPU_STEPS
    model = O.SynthModel(shape, 0)
    k, v = O.kv_prefill(O.substream, shape, 0, npre)
    first = O.first_token(0, shape.vocab)
    toks, lg = O.ref_greedy(ref, model, k, v, npre, first, steps, npre + steps + 1)
    np.savez_compressed(os.path.join(HERE, "qwen3_4b_kv2048.npz"), tokens=np.array(toks, np.uint32),
                        first=np.array(first), logits0_sha=np.array(sha(lg)),
                        blob_sha=np.array(sha(model.blob)))


def step_summary(lg: np.ndarray, stride: int):
    """Top-64 ids (stable, descending), their values, every `stride`-th
    logit and the SHA-256 of one step's logits."""
    top = np.argsort(-lg, kind="stable")[:64]
    return top.astype(np.uint32), lg[top], lg[::stride].copy(), sha(lg)


def golden_forced(ref) -> None:
    """configs[2]'s model, KV prefill and 64 teacher-forced steps with uniform
    random inputs: every step's logits summarised, and its greedy id."""
    shape, npre, steps = CF.QWEN3_06B, CF.C3_PREFILL, CF.C3_FORCED_STEPS
    model = O.SynthModel(shape, 0)
    k, v = O.kv_prefill(O.substream, shape, 0, npre)
    inputs = CF.forced_inputs(O.uniform, O.substream, shape.vocab, steps)
    greedy, lg = O.ref_run(ref, model, npre + steps + 1, steps, k=k, v=v, n_prefill=npre,
                           inputs=inputs)
    parts = [step_summary(lg[i], CF.FORCED_SAMPLE_STRIDE) for i in range(steps)]
    np.savez_compressed(os.path.join(HERE, "qwen3_06b_forced.npz"),
                        inputs=inputs.astype(np.uint32), greedy=np.array(greedy, np.uint32),
                        top_ids=np.stack([p[0] for p in parts]),
                        top_vals=np.stack([p[1] for p in parts]),
                        sample=np.stack([p[2] for p in parts]),
                        logits_sha=np.array([p[3] for p in parts]),
                        blob_sha=np.array(sha(model.blob)))


def golden_c5_full(ref) -> None:
    """configs[4] end to end: the 2048-token prompt and 256 greedy steps on
    Qwen3-4B, the greedy ids of every step and the top-64 logits (plus every
    293rd logit) of the snapshot steps."""
    shape = CF.QWEN3_4B
    model = O.SynthModel(shape, 0)
    prompt = CF.c5_prompt(O.uniform, O.substream, shape.vocab, CF.C5_PROMPT)
    steps = CF.C5_STEPS
    greedy, lg = O.ref_run(ref, model, CF.C5_PROMPT + steps + 1, steps, prompt=prompt)
    parts = [step_summary(lg[i], CF.FORCED_SAMPLE_STRIDE) for i in CF.C5_SNAPSHOT_STEPS]
    np.savez_compressed(os.path.join(HERE, "qwen3_4b_c5.npz"),
                        prompt_sha=np.array(sha(prompt.astype(np.uint32))),
                        greedy=np.array(greedy, np.uint32),
                        snapshot_steps=np.array(CF.C5_SNAPSHOT_STEPS, np.uint32),
                        top_ids=np.stack([p[0] for p in parts]),
                        top_vals=np.stack([p[1] for p in parts]),
                        sample=np.stack([p[2] for p in parts]),
                        logits_sha=np.array([p[3] for p in parts]),
                        blob_sha=np.array(sha(model.blob)))


def golden_adjacent(ref) -> None:
    fx = os.path.join(HERE, "ingot_fixtures")
    for name in ("Q5_K", "Q4_0"):
        for ext in ("bin", "ref"):
            shutil.copyfile(os.path.join(REF_FIXTURES, f"{name}.{ext}"),
                            os.path.join(fx, f"{name}.{ext}"))
    out = {}
    for t, rows, cols, token_counts in CF.ADJACENT:
        key = f"{CF.TYPE_NAME[t]}_{rows}x{cols}"
        w = O.blocks(t, 1000 + t + rows, rows, cols)
        x = O.normal(2000 + t + rows, max(token_counts) * cols)
        out[f"{key}_w_sha"] = np.array(sha(w))
        out[f"{key}_x_sha"] = np.array(sha(x))
        out[f"{key}_matvec"] = ref_matvec(ref, t, w, rows, cols, x)
        out[f"{key}_dequant"] = ref_dequant(ref, t, w, rows, cols)
        for n in token_counts:
            out[f"{key}_matmat{n}"] = ref_matmat(ref, t, w, rows, cols, x, n)
    np.savez_compressed(os.path.join(HERE, "adjacent.npz"), **out)


INT8_MATVEC = ((37, 512), (64, 3072))
# Q5_K on the int8 lane (batched only): token counts across the tile and the
# groups of four, ragged rows.
INT8_Q5K_MATMAT = ((40, 2048, 70), (9, 512, 130), (24, 1024, 5), (3, 256, 2))
INT8_MATMAT = ((16, 2048, 16), (24, 2048, 70), (9, 512, 130), (8, 6144, 5), (4, 9728, 110),
               (5, 512, 2), (3, 256, 3), (6, 1024, 1))


def int8_special_x() -> np.ndarray:
    """Three blocks that pin the quantiser: amax 127 with half-integer values
    (x * 127 / amax = k + 0.5 exactly: ties to even), all zeros (scale 0),
    and tiny values (a large finite inverse)."""
    x = np.zeros(768, np.float32)
    k = np.arange(256, dtype=np.float32)
    x[:256] = (k % 254) - 126.5
    x[0], x[1] = 127.0, -127.0
    x[512:] = O.normal(77, 256) * np.float32(1e-30)
    return x


def golden_int8(ref8) -> None:
    assert ref8.ingot_matmat_is_exact(2) == 0, "AVX2 build did not take the int8 lane"
    out = {}
    for rows, cols in INT8_MATVEC:
        w, x = O.blocks(CF.Q4_K, 500 + rows, rows, cols), O.normal(600 + rows, cols)
        y = np.empty(rows, np.float32)
        assert ref8.ingot_q4_k_matvec(O.ptr(w), rows, cols, O.ptr(x), O.ptr(y)) == 0
        out[f"mv_{rows}x{cols}_y"] = y
        out[f"mv_{rows}x{cols}_w_sha"] = np.array(sha(w))
        out[f"mv_{rows}x{cols}_x_sha"] = np.array(sha(x))
    w, x = O.blocks(CF.Q4_K, 700, 16, 768), int8_special_x()
    y = np.empty(16, np.float32)
    assert ref8.ingot_q4_k_matvec(O.ptr(w), 16, 768, O.ptr(x), O.ptr(y)) == 0
    out["mv_special_y"] = y
    out["mv_special_x"] = x
    for rows, cols, tokens in INT8_MATMAT:
        key = f"mm_{rows}x{cols}_t{tokens}"
        w, x = O.blocks(CF.Q4_K, 800 + rows, rows, cols), O.normal(900 + tokens, tokens * cols)
        y = np.empty(rows * tokens, np.float32)
        assert ref8.ingot_q4_k_matmat(O.ptr(w), rows, cols, O.ptr(x), O.ptr(y), tokens) == 0
        out[f"{key}_y"] = y
        out[f"{key}_w_sha"] = np.array(sha(w))
        out[f"{key}_x_sha"] = np.array(sha(x))
    for rows, cols, tokens in INT8_Q5K_MATMAT:
        key = f"q5k_mm_{rows}x{cols}_t{tokens}"
        w, x = O.blocks(CF.Q5_K, 1100 + rows, rows, cols), O.normal(1200 + tokens, tokens * cols)
        y = np.empty(rows * tokens, np.float32)
        assert ref8.ingot_q5_k_matmat(O.ptr(w), rows, cols, O.ptr(x), O.ptr(y), tokens) == 0
        out[f"{key}_y"] = y
        out[f"{key}_w_sha"] = np.array(sha(w))
        out[f"{key}_x_sha"] = np.array(sha(x))
    np.savez_compressed(os.path.join(HERE, "int8.npz"), **out)


def generate_cases(ref):
    """The cases of generate_cases.json, each run through the compiled loop."""
    shape = CF.QWEN3_TINY
    model = O.SynthModel(shape, 0)
    prompt = [int(t) for t in O.uniform(O.substream(6, 1), 9, shape.vocab)]
    pen = dict(repeat_penalty=1.5, penalty_window=16)
    temp = dict(temp=0.6, top_k=20, top_p=0.95, seed=7)
    base = dict(prompt=prompt, n_ctx=64, max_new=20, eos=[], think=[-1, -1], stop_after=0,
                sampler=None)
    cases = {"greedy": {}, "context_end": dict(n_ctx=16, max_new=30),
             "stop_after": dict(stop_after=7), "temperature": dict(sampler=temp),
             "penalty": dict(max_new=24, sampler=pen)}
    first = O.ref_generate(ref, model, 64, prompt, 1)["answer"][0]
    cases["eos_first"] = dict(eos=[5, first])
    seq = O.ref_generate(ref, model, 64, prompt, 24, sampler=pen)["answer"]
    k = next(i for i, t in enumerate(seq) if i >= 5 and t not in seq[:i])
    cases["penalty_eos"] = dict(max_new=24, sampler=pen, eos=[seq[k]])
    # Think markers: the first occurrences of two ids of the penalised run.
    a = next(i for i, t in enumerate(seq) if i >= 3 and t not in seq[:i])
    b = next(i for i, t in enumerate(seq) if i > a + 3 and t not in seq[:i] and t != seq[a])
    cases["think"] = dict(max_new=24, sampler=pen, think=[seq[a], seq[b]])
    # The answer callback stops on the first answer id after the block.
    cases["think_stop"] = dict(max_new=24, sampler=pen, think=[seq[a], seq[b]], stop_after=a + 1)
    out = {}
    for name, over in cases.items():
        c = dict(base, **over)
        got = O.ref_generate(ref, model, c["n_ctx"], c["prompt"], c["max_new"], eos=c["eos"],
                             think=tuple(c["think"]), stop_after=c["stop_after"],
                             sampler=c["sampler"])
        out[name] = dict(c, want=got)
    return out


def golden_generate(ref) -> None:
    import json
    with open(os.path.join(HERE, "generate_cases.json"), "w") as f:
        json.dump(generate_cases(ref), f, indent=1, sort_keys=True)
        f.write("\n")


AVX2_SHAPES = ((CF.Q4_K, 37, 512), (CF.Q4_K, 64, 2048), (CF.Q6_K, 37, 512),
               (CF.Q6_K, 16, 3072), (CF.Q8_0, 37, 96), (CF.Q8_0, 37, 512))


def golden_avx2(ref8) -> None:
    out = {}
    for t, rows, cols in AVX2_SHAPES:
        key = f"{CF.TYPE_NAME[t]}_{rows}x{cols}"
        w, x = O.blocks(t, 1300 + t, rows, cols), O.normal(1400 + t, cols)
        y = np.empty(rows, np.float32)
        assert ref8.ingot_matvec(t, O.ptr(w), rows, cols, O.ptr(x), O.ptr(y)) == 0
        out[f"{key}_y"] = y
        out[f"{key}_w_sha"] = np.array(sha(w))
        out[f"{key}_x_sha"] = np.array(sha(x))
    for i, m in enumerate(CF.C2):
        ws, xs = CF.matrix_seeds(O.substream, 0, i)
        w, x = O.blocks(m.qtype, ws, m.rows, m.cols), O.normal(xs, m.cols)
        y = np.empty(m.rows, np.float32)
        assert ref8.ingot_matvec(m.qtype, O.ptr(w), m.rows, m.cols, O.ptr(x), O.ptr(y)) == 0
        out[f"{m.name}_y_sha"] = np.array(sha(y))
        out[f"{m.name}_y_every97"] = y[::97].copy()
    np.savez_compressed(os.path.join(HERE, "avx2.npz"), **out)


def main() -> int:
    ref = O.load_ref()
    if ref is None:
        print("oracle/_ref/libref.so is not built (needs /root/reference): nothing written")
        return 1
    assert ref.ref_matmat_is_exact(2) == 1, "reference build took the int8 batched lane"

    # The reference's own fixtures, copied as data.
    fx = os.path.join(HERE, "ingot_fixtures")
    os.makedirs(fx, exist_ok=True)
    for name in ("Q4_K", "Q6_K", "Q8_0"):
        for ext in ("bin", "ref"):
            shutil.copyfile(os.path.join(REF_FIXTURES, f"{name}.{ext}"),
                            os.path.join(fx, f"{name}.{ext}"))
    for name in ("manifest.txt", "geometry.txt"):
        shutil.copyfile(os.path.join(REF_FIXTURES, name), os.path.join(fx, name))

    out = {}
    for t in (CF.Q4_K, CF.Q6_K, CF.Q8_0):
        shapes = [(37, 512)] + ([(37, 96)] if t == CF.Q8_0 else [])
        for rows, cols in shapes:
            key = f"{CF.TYPE_NAME[t]}_{rows}x{cols}"
            w = O.blocks(t, 100 + t, rows, cols)
            x = O.normal(200 + t, 3 * cols)
            out[f"{key}_w_sha"] = np.array(sha(w))
            out[f"{key}_x_sha"] = np.array(sha(x))
            out[f"{key}_matvec"] = ref_matvec(ref, t, w, rows, cols, x)
            if cols % 256 == 0:
                out[f"{key}_matmat3"] = ref_matmat(ref, t, w, rows, cols, x, 3)
                out[f"{key}_dequant"] = ref_dequant(ref, t, w, rows, cols)
            else:
                # The reference's batched core and matrix dequant work in
                # 256-wide units and refuse a ragged Q8_0 row (-1).
                y = np.empty(rows * cols * 3, np.float32)
                out[f"{key}_matmat3_rc"] = np.array(ref.ref_matmat(
                    t, O.ptr(w), rows, cols, O.ptr(x), O.ptr(y), 3))
                out[f"{key}_dequant_rc"] = np.array(ref.ref_dequant_matrix(
                    t, O.ptr(w), rows, cols, O.ptr(y)))
    np.savez_compressed(os.path.join(HERE, "kernels_small.npz"), **out)

    # configs[0]
    m = CF.C1[0]
    ws, xs = CF.matrix_seeds(O.substream, 0, 0)
    w, x = O.blocks(m.qtype, ws, m.rows, m.cols), O.normal(xs, m.cols)
    np.savez_compressed(os.path.join(HERE, "c1.npz"), w_sha=np.array(sha(w)),
                        x_sha=np.array(sha(x)), y=ref_matvec(ref, m.qtype, w, m.rows, m.cols, x))

    # configs[1]
    out = {}
    for i, m in enumerate(CF.C2):
        ws, xs = CF.matrix_seeds(O.substream, 0, i)
        w, x = O.blocks(m.qtype, ws, m.rows, m.cols), O.normal(xs, m.cols)
        y = ref_matvec(ref, m.qtype, w, m.rows, m.cols, x)
        out[f"{m.name}_w_sha"] = np.array(sha(w))
        out[f"{m.name}_y_sha"] = np.array(sha(y))
        out[f"{m.name}_y_every97"] = y[::97].copy()
        if m.rows <= 4096:
            out[f"{m.name}_y"] = y
    np.savez_compressed(os.path.join(HERE, "c2.npz"), **out)

    # batched exact order
    out = {}
    for t, rows, cols, tokens in ((CF.Q4_K, 64, 2048, 16), (CF.Q6_K, 32, 6144, 8),
                                  (CF.Q8_0, 40, 1024, 5)):
        key = f"{CF.TYPE_NAME[t]}_{rows}x{cols}_t{tokens}"
        w = O.blocks(t, 300 + t, rows, cols)
        x = O.normal(400 + t, tokens * cols)
        out[f"{key}_y"] = ref_matmat(ref, t, w, rows, cols, x, tokens)
        out[f"{key}_w_sha"] = np.array(sha(w))
    np.savez_compressed(os.path.join(HERE, "matmat.npz"), **out)

    # Qwen3: tiny (every step's logits) and the 0.6B config.
    shape, npre, steps = CF.QWEN3_TINY, 16, 32
    model = O.SynthModel(shape, 0)
    k, v = O.kv_prefill(O.substream, shape, 0, npre)
    first = O.first_token(0, shape.vocab)
    toks, lg = O.ref_greedy(ref, model, k, v, npre, first, steps, npre + steps + 1)
    np.savez_compressed(os.path.join(HERE, "qwen3_tiny.npz"), tokens=np.array(toks, np.uint32),
                        first=np.array(first), logits0=lg, blob_sha=np.array(sha(model.blob)))

    shape, npre, steps = CF.QWEN3_06B, CF.C3_PREFILL, CF.C3_STEPS
    model = O.SynthModel(shape, 0)
    k, v = O.kv_prefill(O.substream, shape, 0, npre)
    first = O.first_token(0, shape.vocab)
    toks, lg = O.ref_greedy(ref, model, k, v, npre, first, steps, npre + steps + 1)
    top = np.argsort(-lg, kind="stable")[:64]
    np.savez_compressed(os.path.join(HERE, "qwen3_06b.npz"), tokens=np.array(toks, np.uint32),
                        first=np.array(first), logits0_sha=np.array(sha(lg)),
                        top_ids=top.astype(np.uint32), top_vals=lg[top],
                        blob_sha=np.array(sha(model.blob)))
    golden_forced(ref)
    golden_adjacent(ref)
    golden_generate(ref)
    r8 = O.load_ref_int8()
    if r8 is not None:
        golden_int8(r8)
        # INGOT_SDOT is read once per process: the f32 lanes get their own.
        subprocess.run([sys.executable, os.path.abspath(__file__), "--only", "avx2"], check=True)
    print("golden vectors written to", HERE)
    return 0


if __name__ == "__main__":
    if sys.argv[1:] == ["--only", "avx2"]:
        r8 = O.load_ref_int8(sdot="0")
        assert r8 is not None, "oracle/_ref/libref_int8.so is missing: run make -C oracle"
        golden_avx2(r8)
        sys.exit(0)
    if sys.argv[1:] == ["--only", "int8"]:
        r8 = O.load_ref_int8()
        assert r8 is not None, "oracle/_ref/libref_int8.so is missing: run make -C oracle"
        golden_int8(r8)
        sys.exit(0)
    if sys.argv[1:] == ["--only", "adjacent"]:
        r = O.load_ref()
        assert r is not None, "oracle/_ref/libref.so is missing: run make -C oracle"
        golden_adjacent(r)
        sys.exit(0)
    if sys.argv[1:] == ["--only", "forced"]:
        r = O.load_ref()
        assert r is not None, "oracle/_ref/libref.so is missing: run make -C oracle"
        golden_forced(r)
        sys.exit(0)
    if sys.argv[1:] == ["--only", "c5full"]:
        r = O.load_ref()
        assert r is not None, "oracle/_ref/libref.so is missing: run make -C oracle"
        golden_c5_full(r)
        sys.exit(0)
    if sys.argv[1:] == ["--only", "generate"]:
        r = O.load_ref()
        assert r is not None, "oracle/_ref/libref.so is missing: run make -C oracle"
        golden_generate(r)
        sys.exit(0)
    if sys.argv[1:] == ["--only", "c5kv"]:
        r = O.load_ref()
        assert r is not None, "oracle/_ref/libref.so is missing: run make -C oracle"
        golden_c5_kv(r)
        sys.exit(0)
    if sys.argv[1:] == ["--only", "c5"]:
        r = O.load_ref()
        assert r is not None, "oracle/_ref/libref.so is missing: run make -C oracle"
        golden_c5(r)
        sys.exit(0)
    sys.exit(main())
