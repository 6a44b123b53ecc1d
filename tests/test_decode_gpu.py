"""GPU parity of the resident Qwen3 decode step (configs[2] and a tiny model).

The GEMVs are bit-exact and the f32 operators follow the reference operation
for operation, so the logits agree with the oracle (bit-identical to the
compiled reference decoder) to |gpu - ref| / max(1, |ref|) <= 1e-4 — the only
differences are last-bit expf results and the order of double sums — and
the greedy token ids equal the golden ids the compiled reference produced.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

import configs as CF
import oracle_lib as O

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TOL = 1e-4


@pytest.fixture(scope="module")
def M():
    import mynah_amd
    mynah_amd.check(mynah_amd.lib.mynah_hip_init(0), "init")
    mynah_amd.check(mynah_amd.lib.mynah_hip_set_gemv_order(0), "order")
    O.orc.orc_threads_init(0)
    return mynah_amd


def rel_err(got, ref):
    return float((np.abs(got.astype(np.float64) - ref) / np.maximum(1.0, np.abs(ref))).max())


def setup(M, shape, n_prefill, steps):
    print(f"[case] decode layers={shape.n_layers} d={shape.d_model} prefill={n_prefill}", flush=True)
    model = M.SynthQwen3(shape, 0)
    k, v = O.kv_prefill(O.substream, shape, 0, n_prefill)
    first = O.first_token(0, shape.vocab)
    n_ctx = n_prefill + steps + 1
    dec = M.Qwen3Decoder(model, n_ctx)
    dec.set_kv(k, v, n_prefill)
    return model, k, v, first, n_ctx, dec


def test_tiny_logits_and_tokens(M):
    g = np.load(os.path.join(GOLDEN, "qwen3_tiny.npz"), allow_pickle=False)
    shape, npre, steps = CF.QWEN3_TINY, 16, int(g["tokens"].size)
    model, k, v, first, n_ctx, dec = setup(M, shape, npre, steps)
    assert first == int(g["first"])
    lg = dec.forward(first)
    assert rel_err(lg, g["logits0"]) <= TOL
    assert int(np.argmax(lg)) == int(g["tokens"][0])
    dec.reset()
    dec.set_kv(k, v, npre)
    toks, _ = dec.generate(first, steps)
    assert toks == [int(t) for t in g["tokens"]]


def test_tiny_every_step_against_oracle(M):
    """Logits of every step, fed the same tokens, against the oracle."""
    shape, npre, steps = CF.QWEN3_TINY, 16, 12
    model, k, v, first, n_ctx, dec = setup(M, shape, npre, steps)
    orc_model = O.SynthModel(shape, 0)
    assert np.array_equal(orc_model.blob, model.blob)
    ref = O.OracleQwen3(orc_model, n_ctx)
    ref.prefill_kv(k, v, npre)
    tok = first
    for i in range(steps):
        a = dec.forward(tok)
        b = ref.forward(tok)
        err = rel_err(a, b)
        print(f"step {i}: max rel err {err:.2e}, bit-equal {np.array_equal(a.view(np.uint32), b.view(np.uint32))}")
        assert err <= TOL
        tok = int(np.argmax(b))


def test_graph_replay_equals_step_by_step(M):
    shape, npre, steps = CF.QWEN3_TINY, 8, 10
    model, k, v, first, n_ctx, dec = setup(M, shape, npre, steps)
    toks, _ = dec.generate(first, steps)
    dec.reset()
    dec.set_kv(k, v, npre)
    tok, stepwise = first, []
    for _ in range(steps):
        lg = dec.forward(tok)
        tok = int(np.argmax(lg))      # first maximum, like the reference sampler
        stepwise.append(tok)
    assert stepwise == toks


def test_context_exhaustion_returns_error(M):
    shape = CF.QWEN3_TINY
    model = M.SynthQwen3(shape, 0)
    dec = M.Qwen3Decoder(model, 3)
    for _ in range(3):
        dec.forward(1, want_logits=False)
    assert M.lib.mynah_hip_qwen3_forward(dec.h, 1, None) == -1
    assert b"context" in M.lib.mynah_hip_last_error()


def test_qwen3_06b_64_greedy_steps(M):
    g = np.load(os.path.join(GOLDEN, "qwen3_06b.npz"), allow_pickle=False)
    shape, npre, steps = CF.QWEN3_06B, CF.C3_PREFILL, CF.C3_STEPS
    model, k, v, first, n_ctx, dec = setup(M, shape, npre, steps)
    assert first == int(g["first"])
    lg = dec.forward(first)
    top = np.argsort(-lg, kind="stable")[:64]
    assert list(top[:8]) == [int(t) for t in g["top_ids"][:8]]
    assert rel_err(lg[g["top_ids"]], g["top_vals"]) <= TOL
    dec.reset()
    dec.set_kv(k, v, npre)
    toks, ms = dec.generate(first, steps)
    print(f"0.6B decode: {steps} steps in {ms:.2f} ms = {steps / ms * 1e3:.0f} tok/s, "
          f"graph={dec.uses_graph}")
    assert toks == [int(t) for t in g["tokens"]]


def test_fast_order_same_tokens(M):
    """The reordered GEMV order: logits differ from the reference only by f32
    rounding of the sums; the 64 greedy tokens are the reference's."""
    g = np.load(os.path.join(GOLDEN, "qwen3_06b.npz"), allow_pickle=False)
    shape, npre, steps = CF.QWEN3_06B, CF.C3_PREFILL, CF.C3_STEPS
    M.check(M.lib.mynah_hip_set_gemv_order(1), "order")
    try:
        model, k, v, first, n_ctx, dec = setup(M, shape, npre, steps)
        lg = dec.forward(first)
        err = rel_err(lg[g["top_ids"]], g["top_vals"])
        print(f"reordered: top-64 logits max rel err {err:.2e}")
        assert err <= 1e-3
        dec.reset()
        dec.set_kv(k, v, npre)
        toks, ms = dec.generate(first, steps)
        print(f"0.6B decode (reordered GEMVs): {steps / ms * 1e3:.0f} tok/s")
        assert toks == [int(t) for t in g["tokens"]]
    finally:
        M.check(M.lib.mynah_hip_set_gemv_order(0), "order")


@pytest.mark.parametrize("shape", [CF.QWEN3_TINY, CF.QWEN3_06B], ids=["tiny", "0.6B"])
def test_producer_consumer_gemv_decoder_bit_identical(M, monkeypatch, shape):
    """Every Q4_K projection launch in the producer/consumer layout (forced
    with MYNAH_GEMV_PC=1: q/k/v with the input RMSNorm, o and down with the
    residual, the gate/up pair with SwiGLU, K/V into the cache slot): each
    step's logits bit-identical to the default decoder's, stepwise and
    graph-replayed."""
    npre, steps = 40, 12
    print(f"[case] producer/consumer GEMV decoder d={shape.d_model}", flush=True)
    model = M.SynthQwen3(shape, 0)
    k, v = O.kv_prefill(O.substream, shape, 0, npre)
    first = O.first_token(0, shape.vocab)
    monkeypatch.setenv("MYNAH_GEMV_PC", "1")
    a = M.Qwen3Decoder(model, npre + steps + 1)
    a.set_kv(k, v, npre)
    la = [a.forward(t) for t in range(first, first + steps)]
    a.reset()
    a.set_kv(k, v, npre)
    ta, _ = a.generate(first, steps)
    monkeypatch.setenv("MYNAH_GEMV_PC", "0")
    b = M.Qwen3Decoder(model, npre + steps + 1)
    b.set_kv(k, v, npre)
    for i, t in enumerate(range(first, first + steps)):
        assert np.array_equal(la[i].view(np.uint32), b.forward(t).view(np.uint32)), f"step {i}"
    b.reset()
    b.set_kv(k, v, npre)
    assert b.generate(first, steps)[0] == ta


def _split_runs(M, model, shape, k, v, npre, first, steps):
    d = M.Qwen3Decoder(model, npre + steps + 1)
    d.set_attention(M.ATTN_SPLIT)
    d.set_kv(k, v, npre)
    logits = [d.forward(t) for t in range(first, first + steps)]
    d.reset()
    d.set_kv(k, v, npre)
    toks, _ = d.generate(first, steps)
    lg = d.forward(toks[-1])
    d.close()
    return logits, toks, lg


@pytest.mark.parametrize("shape,npre", [(CF.QWEN3_TINY, 60), (CF.QWEN3_06B, 500),
                                        (CF.QWEN3_TINY, 1000)],
                         ids=["tiny", "0.6B", "tiny-32ch"])
def test_one_wave_combine_bit_identical(M, monkeypatch, shape, npre):
    """The split attention's combine by one wave per query head (up to 32
    chunks, no barrier; the last case has exactly 32) against the four-wave
    combine (MYNAH_ATTN_COMBINE1=0): every step's logits bit-identical,
    stepwise and graph-replayed."""
    steps = 12
    print(f"[case] one-wave combine d={shape.d_model} npre={npre}", flush=True)
    model = M.SynthQwen3(shape, 0)
    k, v = O.kv_prefill(O.substream, shape, 0, npre)
    first = O.first_token(0, shape.vocab)
    monkeypatch.setenv("MYNAH_ATTN_COMBINE1", "1")
    la, ta, ga = _split_runs(M, model, shape, k, v, npre, first, steps)
    monkeypatch.setenv("MYNAH_ATTN_COMBINE1", "0")
    lb, tb, gb = _split_runs(M, model, shape, k, v, npre, first, steps)
    for i in range(steps):
        assert np.array_equal(la[i].view(np.uint32), lb[i].view(np.uint32)), f"step {i}"
    assert ta == tb
    assert np.array_equal(ga.view(np.uint32), gb.view(np.uint32))


@pytest.mark.parametrize("npre", [1500, 2105], ids=["48ch", "67ch"])
def test_four_wave_combine_wave0_sums_bit_identical(M, monkeypatch, npre):
    """The four-wave combine (past 32 chunks) finding the maximum and the
    double sum in wave 0 alone — up to 128 chunks, two per lane from the
    65th — against its all-waves form (MYNAH_COMBINE_WAVE0=0): every step's
    logits bit-identical, stepwise and graph-replayed, at 48 chunks and
    across the 67th chunk's boundary (tiny model)."""
    shape, steps = CF.QWEN3_TINY, 12
    print(f"[case] wave-0 combine sums npre={npre}", flush=True)
    model = M.SynthQwen3(shape, 0)
    k, v = O.kv_prefill(O.substream, shape, 0, npre)
    first = O.first_token(0, shape.vocab)
    monkeypatch.setenv("MYNAH_COMBINE_WAVE0", "1")
    la, ta, ga = _split_runs(M, model, shape, k, v, npre, first, steps)
    monkeypatch.setenv("MYNAH_COMBINE_WAVE0", "0")
    lb, tb, gb = _split_runs(M, model, shape, k, v, npre, first, steps)
    for i in range(steps):
        assert np.array_equal(la[i].view(np.uint32), lb[i].view(np.uint32)), f"step {i}"
    assert ta == tb
    assert np.array_equal(ga.view(np.uint32), gb.view(np.uint32))


@pytest.mark.parametrize("env", [{"MYNAH_PREFETCH_WGS": "128", "MYNAH_PREFETCH_BPW": "0"},
                                 {"MYNAH_PREFETCH_BPW": "8192"},
                                 {"MYNAH_PREFETCH_BPW": "1024", "MYNAH_PREFETCH_STEP": "6"},
                                 {"MYNAH_PREFETCH_BPW": "8192", "MYNAH_PREFETCH_MAX": "0",
                                  "MYNAH_PREFETCH_LAYER_MAX": "0"}],
                         ids=["ahead_wgs128", "ahead_bpw8192", "ahead_bpw1024_step64",
                              "next_bpw8192_all"])
def test_prefetching_decoder_bit_identical(M, monkeypatch, env):
    """Decode GEMVs carrying workgroups that prefetch weights into L2 — the
    same GEMV of the next layer (the 0.6B default: its layers fit the L2s)
    or, with MYNAH_PREFETCH_LAYER_MAX=0, the next GEMV (every one, no size
    cap) — by workgroup count or bytes per workgroup: logits and ids
    bit-identical to the decoder without them (MYNAH_PREFETCH_BPW=0; 0.6B,
    split attention, stepwise and graph-replayed)."""
    shape, npre, steps = CF.QWEN3_06B, 100, 8
    print(f"[case] prefetch {env}", flush=True)
    model = M.SynthQwen3(shape, 0)
    k, v = O.kv_prefill(O.substream, shape, 0, npre)
    first = O.first_token(0, shape.vocab)
    for e, val in env.items():
        monkeypatch.setenv(e, val)
    la, ta, ga = _split_runs(M, model, shape, k, v, npre, first, steps)
    for e in env:
        monkeypatch.delenv(e)
    monkeypatch.setenv("MYNAH_PREFETCH_BPW", "0")
    lb, tb, gb = _split_runs(M, model, shape, k, v, npre, first, steps)
    for i in range(steps):
        assert np.array_equal(la[i].view(np.uint32), lb[i].view(np.uint32)), f"step {i}"
    assert ta == tb
    assert np.array_equal(ga.view(np.uint32), gb.view(np.uint32))


def test_split_attention_every_step_against_oracle(M):
    """Split attention (per-chunk softmax partials, one launch per layer):
    logits within 1e-4 of the oracle on every step, over chunk boundaries."""
    shape, npre, steps = CF.QWEN3_TINY, 60, 12          # positions 60..71 cross 64
    model, k, v, first, n_ctx, dec = setup(M, shape, npre, steps)
    dec.set_attention(M.ATTN_SPLIT)
    orc_model = O.SynthModel(shape, 0)
    ref = O.OracleQwen3(orc_model, n_ctx)
    ref.prefill_kv(k, v, npre)
    tok = first
    worst = 0.0
    for i in range(steps):
        a = dec.forward(tok)
        b = ref.forward(tok)
        err = rel_err(a, b)
        worst = max(worst, err)
        assert err <= TOL, f"step {i}: {err:.2e}"
        tok = int(np.argmax(b))
    print(f"split attention: worst logit rel err {worst:.2e}")


def test_split_attention_graph_equals_stepwise(M):
    shape, npre, steps = CF.QWEN3_TINY, 30, 40
    model, k, v, first, n_ctx, dec = setup(M, shape, npre, steps)
    dec.set_attention(M.ATTN_SPLIT)
    toks, _ = dec.generate(first, steps)
    dec.reset()
    dec.set_kv(k, v, npre)
    tok, stepwise = first, []
    for _ in range(steps):
        lg = dec.forward(tok)
        tok = int(np.argmax(lg))
        stepwise.append(tok)
    assert stepwise == toks


def test_qwen3_06b_split_attention_same_tokens(M):
    g = np.load(os.path.join(GOLDEN, "qwen3_06b.npz"), allow_pickle=False)
    shape, npre, steps = CF.QWEN3_06B, CF.C3_PREFILL, CF.C3_STEPS
    model, k, v, first, n_ctx, dec = setup(M, shape, npre, steps)
    dec.set_attention(M.ATTN_SPLIT)
    lg = dec.forward(first)
    err = rel_err(lg[g["top_ids"]], g["top_vals"])
    print(f"split attention: top-64 logits max rel err {err:.2e}")
    assert err <= TOL
    dec.reset()
    dec.set_kv(k, v, npre)
    toks, ms = dec.generate(first, steps)
    print(f"0.6B decode (split attention): {steps / ms * 1e3:.0f} tok/s")
    assert toks == [int(t) for t in g["tokens"]]


def test_prompt_prefill_equals_stepwise(M):
    """Prompt prefill by decode steps (cache-filling steps without the head) then greedy
    steps gives the same ids as feeding the prompt through forward() and
    generating from its last token, and the oracle's greedy run."""
    shape, steps = CF.QWEN3_TINY, 12
    model = M.SynthQwen3(shape, 0)
    prompt = [int(t) for t in M.synth_uniform(M.substream(5, 1), 9, shape.vocab)]
    n_ctx = len(prompt) + steps + 2
    for attn in (M.ATTN_EXACT, M.ATTN_SPLIT):
        dec = M.Qwen3Decoder(model, n_ctx)
        dec.set_attention(attn)
        dec.set_prefill(M.PREFILL_STEPS)
        got, pre_ms, dec_ms = dec.prompt(prompt, steps)
        assert dec.n_past == len(prompt) - 1 + steps
        dec.reset()
        for t in prompt[:-1]:
            dec.forward(t, want_logits=False)
        ref, _ = dec.generate(prompt[-1], steps)
        assert got == ref
    orc_model = O.SynthModel(shape, 0)
    orc = O.OracleQwen3(orc_model, n_ctx)
    lg = None
    for t in prompt:
        lg = orc.forward(t)
    tok, want = int(np.argmax(lg)), []
    for _ in range(steps):
        want.append(tok)
        tok = int(np.argmax(orc.forward(tok)))
    assert got == want


def test_qwen3_4b_prompt_prefix(M):
    """configs[4]'s model (Qwen3-4B, 36 layers, group 4): the first 8 prompt
    ids, prefill + 8 greedy steps, against the compiled reference's run: the
    first step's top-64 logits within 1e-4 and the same ids, in both
    attention modes."""
    g = np.load(os.path.join(GOLDEN, "qwen3_4b_prompt.npz"), allow_pickle=False)
    shape = CF.QWEN3_4B
    print(f"[case] Qwen3-4B prompt prefix", flush=True)
    model = M.SynthQwen3(shape, 0)
    prompt = [int(t) for t in g["prompt"]]
    assert prompt == [int(t) for t in CF.c5_prompt(M.synth_uniform, M.substream, shape.vocab,
                                                   CF.C5_GOLDEN_PROMPT)]
    steps = int(g["tokens"].size)
    want = [int(t) for t in g["tokens"]]
    for attn in (M.ATTN_EXACT, M.ATTN_SPLIT):
        dec = M.Qwen3Decoder(model, len(prompt) + steps + 1)
        dec.set_attention(attn)
        for t in prompt[:-1]:
            dec.forward(t, want_logits=False)
        lg = dec.forward(prompt[-1])
        err = rel_err(lg[g["top_ids"]], g["top_vals"])
        print(f"4B attention mode {attn}: top-64 logits max rel err {err:.2e}")
        assert err <= TOL
        assert int(np.argmax(lg)) == want[0]
        dec.reset()
        got, _, _ = dec.prompt(prompt, steps)
        assert got == want
        dec.close()
