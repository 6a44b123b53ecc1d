"""Multi-step decode parity that a collapsed greedy trajectory cannot hide.

A random-init model's greedy ids settle on one token within a step or two,
so a token list says little about the later steps. Here every step's input
is drawn uniformly (teacher forcing), and the compiled reference's logits of
every step are the golden vectors (tests/golden/qwen3_06b_forced.npz,
configs[2]'s model and 512-position KV prefill, 64 steps):

  * step by step through forward(): every step's logits at the golden top-64
    ids and at every 293rd id within |gpu - ref| / max(1, |ref|) <= 1e-4 —
    and with exact attention bit for bit equal to the reference's — and
    every step's greedy id, in both attention modes;
  * through the replayed multi-step graphs (mynah_hip_qwen3_forced, eight
    steps per graph launch, the position and step counters advancing on the
    device): the greedy id of every step and the last step's logits against
    the golden, and the whole KV cache and last logits bit-identical to the
    step-by-step run;
  * greedy generate() (graph-replayed) against forward() fed the same ids:
    the KV cache and the next step's logits bit-identical.

configs[4] (Qwen3-4B): the batched prefill of a 2048-token prompt in one
2048-token chunk (the default chunk) against one decode step per token, K/V
and next logits bit-identical; and, when the golden exists, the whole
configs[4] run (2048-token prompt, 256 greedy steps) against the compiled
reference: every greedy id and the logits of seven snapshot steps.
"""
from __future__ import annotations

import hashlib
import os

import numpy as np
import pytest

import configs as CF
import oracle_lib as O

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TOL = 1e-4
MODES = {"exact": 0, "split": 1}


@pytest.fixture(scope="module")
def M():
    import mynah_amd
    mynah_amd.check(mynah_amd.lib.mynah_hip_init(0), "init")
    mynah_amd.check(mynah_amd.lib.mynah_hip_set_gemv_order(0), "order")
    return mynah_amd


@pytest.fixture(scope="module")
def g06():
    return np.load(os.path.join(GOLDEN, "qwen3_06b_forced.npz"), allow_pickle=False)


@pytest.fixture(scope="module")
def m06(M):
    return M.SynthQwen3(CF.QWEN3_06B, 0)


def rel_err(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float((np.abs(got - ref) / np.maximum(1.0, np.abs(ref))).max())


def check_step(lg, g, i, stride=CF.FORCED_SAMPLE_STRIDE, exact=False):
    """One step's logits against the golden summary of step i: within 1e-4,
    and in the exact modes bit for bit, the whole vocabulary by its SHA-256
    (the GEMVs keep the reference's order and the softmax / sigmoid
    exponential is the C library's)."""
    top, smp = lg[g["top_ids"][i]], lg[::stride]
    e_top = rel_err(top, g["top_vals"][i])
    e_smp = rel_err(smp, g["sample"][i])
    assert e_top <= TOL and e_smp <= TOL, f"step {i}: top {e_top:.2e}, sample {e_smp:.2e}"
    if exact:
        assert np.array_equal(top.view(np.uint32), g["top_vals"][i].view(np.uint32)), f"step {i}"
        assert np.array_equal(smp.view(np.uint32), g["sample"][i].view(np.uint32)), f"step {i}"
        assert hashlib.sha256(np.ascontiguousarray(lg).tobytes()).hexdigest() == \
            str(g["logits_sha"][i]), f"step {i}: whole logits vector"
    return max(e_top, e_smp)


def decoder_06b(M, model, mode):
    k, v = O.kv_prefill(O.substream, CF.QWEN3_06B, 0, CF.C3_PREFILL)
    dec = M.Qwen3Decoder(model, CF.C3_PREFILL + CF.C3_FORCED_STEPS + 1)
    dec.set_attention(mode)
    dec.set_kv(k, v, CF.C3_PREFILL)
    return dec


@pytest.mark.parametrize("mode", MODES)
def test_06b_forced_every_step_stepwise(M, m06, g06, mode):
    print(f"[case] 0.6B teacher-forced stepwise attention={mode}", flush=True)
    assert hashlib.sha256(m06.blob.tobytes()).hexdigest() == str(g06["blob_sha"])
    dec = decoder_06b(M, m06, MODES[mode])
    inputs = [int(t) for t in g06["inputs"]]
    assert inputs == [int(t) for t in CF.forced_inputs(M.synth_uniform, M.substream,
                                                       CF.QWEN3_06B.vocab, len(inputs))]
    worst = 0.0
    for i, tok in enumerate(inputs):
        lg = dec.forward(tok)
        worst = max(worst, check_step(lg, g06, i, exact=mode == "exact"))
        assert int(np.argmax(lg)) == int(g06["greedy"][i]), f"step {i}"
    print(f"0.6B forced ({mode}): worst logit error {worst:.2e} over {len(inputs)} steps")


@pytest.mark.parametrize("mode", MODES)
def test_06b_forced_graph_replay(M, m06, g06, mode):
    print(f"[case] 0.6B teacher-forced graph attention={mode}", flush=True)
    inputs = [int(t) for t in g06["inputs"]]
    n = len(inputs)
    dec = decoder_06b(M, m06, MODES[mode])
    greedy, last = dec.forced(inputs)
    assert dec.uses_graph
    assert greedy == [int(t) for t in g06["greedy"]]
    check_step(last, g06, n - 1, exact=mode == "exact")
    kg, vg = dec.get_kv(CF.C3_PREFILL + n)
    ref = decoder_06b(M, m06, MODES[mode])
    for tok in inputs:
        lg = ref.forward(tok)
    ks, vs = ref.get_kv(CF.C3_PREFILL + n)
    assert np.array_equal(kg.view(np.uint32), ks.view(np.uint32))
    assert np.array_equal(vg.view(np.uint32), vs.view(np.uint32))
    assert np.array_equal(last.view(np.uint32), lg.view(np.uint32))


@pytest.mark.parametrize("mode", MODES)
def test_06b_generate_state_equals_stepwise(M, m06, mode):
    """24 greedy steps as three 8-step graph launches, then the cache and
    the next step's logits against forward() fed the same ids."""
    print(f"[case] 0.6B generate state attention={mode}", flush=True)
    steps = 24
    first = O.first_token(0, CF.QWEN3_06B.vocab)
    dec = decoder_06b(M, m06, MODES[mode])
    toks, _ = dec.generate(first, steps)
    ref = decoder_06b(M, m06, MODES[mode])
    for tok in [first] + toks[:-1]:
        ref.forward(tok, want_logits=False)
    n = CF.C3_PREFILL + steps
    assert dec.n_past == ref.n_past == n
    kg, vg = dec.get_kv(n)
    ks, vs = ref.get_kv(n)
    assert np.array_equal(kg.view(np.uint32), ks.view(np.uint32))
    assert np.array_equal(vg.view(np.uint32), vs.view(np.uint32))
    a, b = dec.forward(toks[-1]), ref.forward(toks[-1])
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_qwen3_4b_prefill_2048_equals_stepwise(M):
    """configs[4]'s prompt through the batched prefill (one chunk of the
    default 2048) and through 2047 decode steps: K/V and the last prompt
    token's logits bit-identical."""
    print("[case] 4B 2048-token prefill vs steps", flush=True)
    shape = CF.QWEN3_4B
    model = M.SynthQwen3(shape, 0)
    prompt = [int(t) for t in CF.c5_prompt(M.synth_uniform, M.substream, shape.vocab)]
    n = len(prompt)
    a = M.Qwen3Decoder(model, n + 1)
    a.prefill(prompt[:-1])
    la = a.forward(prompt[-1])
    ka, va = a.get_kv(n)
    a.close()
    b = M.Qwen3Decoder(model, n + 1)
    for tok in prompt[:-1]:
        b.forward(tok, want_logits=False)
    lb = b.forward(prompt[-1])
    kb, vb = b.get_kv(n)
    b.close()
    assert np.array_equal(ka.view(np.uint32), kb.view(np.uint32))
    assert np.array_equal(va.view(np.uint32), vb.view(np.uint32))
    assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))


C5_GOLDEN = os.path.join(GOLDEN, "qwen3_4b_c5.npz")


@pytest.mark.skipif(not os.path.exists(C5_GOLDEN), reason="configs[4] golden not written")
@pytest.mark.parametrize("mode", MODES)
def test_qwen3_4b_configs4_against_reference(M, mode):
    """configs[4] end to end: the 2048-token prompt (batched prefill), 256
    greedy steps graph-replayed, every id against the compiled reference;
    then the same steps teacher-forced with those ids in segments ending at
    the snapshot steps, whose logits must match the reference's."""
    print(f"[case] 4B configs[4] attention={mode}", flush=True)
    g = np.load(C5_GOLDEN, allow_pickle=False)
    shape = CF.QWEN3_4B
    model = M.SynthQwen3(shape, 0)
    prompt = [int(t) for t in CF.c5_prompt(M.synth_uniform, M.substream, shape.vocab)]
    steps = CF.C5_STEPS
    dec = M.Qwen3Decoder(model, len(prompt) + steps + 1)
    dec.set_attention(MODES[mode])
    got, pre_ms, dec_ms = dec.prompt(prompt, steps)
    assert got == [int(t) for t in g["greedy"]]
    print(f"4B configs[4] ({mode}): prefill {pre_ms:.1f} ms, {steps / dec_ms * 1e3:.0f} tok/s")
    dec.reset()
    dec.prefill(prompt[:-1])
    inputs = [prompt[-1]] + got[:-1]
    done = 0
    for j, stop in enumerate(int(s) for s in g["snapshot_steps"]):
        ids, last = dec.forced(inputs[done:stop + 1])
        assert ids == got[done:stop + 1]
        check_step(last, g, j, exact=mode == "exact")
        done = stop + 1


# Split attention against the whole logit vector. The split mode rounds its
# per-chunk exponentials and sums differently from the reference (a few 1e-7
# of an attention output, tests/test_attention_gpu.py); 28 to 36 random-init
# layers amplify that. Measured whole-vector maxima of |gpu - ref| /
# max(1, |ref|) on one MI355X: configs[2], 64 teacher-forced steps, 1.79e-4
# (29 of the 64 steps above 1e-4, median 9.9e-5); configs[4], eight steps
# after the 2048-token prompt, 1.33e-4 rising to 2.90e-4. The bounds below
# are twice those: they hold the mode to what it does. It is outside the
# north star's 1e-4 per element, which the exact mode meets bit for bit.
TOL_SPLIT_C2 = 3.6e-4
TOL_SPLIT_C5 = 6e-4


def test_06b_split_whole_logits_against_oracle(M, m06, g06):
    """configs[2], split attention: every one of the 64 teacher-forced
    steps' whole logits vector against the oracle's (whose vectors are the
    compiled reference's: each step's SHA-256 is checked against the
    golden), and every greedy id."""
    print("[case] 0.6B split attention, whole logits vs oracle, 64 steps", flush=True)
    inputs = [int(t) for t in g06["inputs"]]
    k, v = O.kv_prefill(O.substream, CF.QWEN3_06B, 0, CF.C3_PREFILL)
    n_ctx = CF.C3_PREFILL + len(inputs) + 1
    O.orc.orc_threads_init(0)
    orc = O.OracleQwen3(O.SynthModel(CF.QWEN3_06B, 0), n_ctx)
    orc.prefill_kv(k, v, CF.C3_PREFILL)
    dec = decoder_06b(M, m06, MODES["split"])
    errs = []
    for i, tok in enumerate(inputs):
        a, b = dec.forward(tok), orc.forward(tok)
        assert hashlib.sha256(np.ascontiguousarray(b).tobytes()).hexdigest() == \
            str(g06["logits_sha"][i]), f"oracle step {i}"
        errs.append(rel_err(a, b))
        assert int(np.argmax(a)) == int(np.argmax(b)), f"step {i}"
    print(f"0.6B split: whole-vector max rel err per step: max {max(errs):.3e}, "
          f"median {float(np.median(errs)):.3e}, steps above 1e-4: "
          f"{sum(e > 1e-4 for e in errs)} of {len(errs)}")
    assert max(errs) <= TOL_SPLIT_C2


def test_4b_split_whole_logits_after_prompt(M):
    """configs[4], split attention: the exact mode's cache after the
    2048-token prompt (bit-identical to the reference's: the batched prefill
    equals stepwise decode, and the stepwise decode's logits the compiled
    reference's) seeds both the oracle and the split decoder; eight
    teacher-forced steps then compare whole logit vectors and greedy ids."""
    print("[case] 4B split attention, whole logits vs oracle after the prompt", flush=True)
    shape, steps = CF.QWEN3_4B, 8
    model = M.SynthQwen3(shape, 0)
    prompt = [int(t) for t in CF.c5_prompt(M.synth_uniform, M.substream, shape.vocab)]
    n = len(prompt) - 1
    inputs = [prompt[-1]] + [int(t) for t in CF.forced_inputs(M.synth_uniform, M.substream,
                                                              shape.vocab, steps - 1)]
    n_ctx = n + steps + 1
    ex = M.Qwen3Decoder(model, n_ctx)
    ex.prefill(prompt[:-1])
    k, v = ex.get_kv(n)
    ex.close()
    O.orc.orc_threads_init(0)
    orc = O.OracleQwen3(O.SynthModel(shape, 0), n_ctx)
    orc.prefill_kv(k, v, n)
    dec = M.Qwen3Decoder(model, n_ctx)
    dec.set_attention(MODES["split"])
    dec.set_kv(k, v, n)
    errs = []
    for i, tok in enumerate(inputs):
        a, b = dec.forward(tok), orc.forward(tok)
        errs.append(rel_err(a, b))
        assert int(np.argmax(a)) == int(np.argmax(b)), f"step {i}"
    dec.close()
    print(f"4B split after the prompt: whole-vector max rel err per step {['%.2e' % e for e in errs]}")
    assert max(errs) <= TOL_SPLIT_C5
