"""GPU parity of the generation loop (include/mynah_generate.h), the twin of
the reference's mynah_slm_generate (src/generate.c:13-86) that its CLI and
server drive.

The oracle is oracle_lib.oracle_generate: generate.c's loop restated over
the CPU decoder (itself bit-identical to the compiled reference decoder),
with greedy picks or the restated sampler (oracle/sampler.c, pinned bit for
bit against the compiled reference's sampler in test_sampler_oracle.py).
Checked: the generated ids, the count the loop returns, which ids reach the
token callback (an EOS id counts but is not shown), the stop on a callback
request in the middle of a device-side chunk (the position rewinds to just
after the stopping step, so the next step equals a fresh decoder's), the
end of the context, the host-sampling mode with penalties and with a
seeded temperature sampler, and the timing fields (src/timing.c:30-62).
Beside it, the record of the compiled reference's own loop
(tests/golden/generate_cases.json, written by tests/golden/make_golden.py
from src/generate.c built from its sources) is replayed through the GPU
loop with the channel-routing callback of a front end (think markers,
answer-callback stop).
"""
from __future__ import annotations

import json
import os

import numpy as np
import pytest

import configs as CF
import oracle_lib as O

pytestmark = pytest.mark.gpu
TOL = 1e-4


@pytest.fixture(scope="module")
def M():
    import mynah_amd
    mynah_amd.check(mynah_amd.lib.mynah_hip_init(0), "init")
    mynah_amd.check(mynah_amd.lib.mynah_hip_set_gemv_order(0), "order")
    O.orc.orc_threads_init(0)
    return mynah_amd


@pytest.fixture(scope="module")
def tiny(M):
    return M.SynthQwen3(CF.QWEN3_TINY, 0), O.SynthModel(CF.QWEN3_TINY, 0)


def prompt_of(M, seed, n=9):
    return [int(t) for t in M.synth_uniform(M.substream(seed, 1), n, CF.QWEN3_TINY.vocab)]


def oracle_ids(orc_model, prompt, max_new, n_ctx, **kw):
    return O.oracle_generate(O.OracleQwen3(orc_model, n_ctx), prompt, max_new, **kw)


@pytest.mark.parametrize("chunk", [1, 3, 8, 0])
def test_device_greedy_matches_the_loop(M, tiny, chunk):
    print(f"[case] generate greedy chunk={chunk}", flush=True)
    model, orc_model = tiny
    prompt, steps, n_ctx = prompt_of(M, 6), 20, 64
    want = oracle_ids(orc_model, prompt, steps, n_ctx)
    dec = M.Qwen3Decoder(model, n_ctx)
    seen, n, t = dec.generate_tokens(prompt, steps, chunk=chunk)
    assert n == steps and seen == want
    assert dec.n_past == len(prompt) - 1 + steps
    assert t.n_prompt == len(prompt) and t.n_gen == steps
    assert t.prefill_s > 0 and t.decode_s > 0 and t.prefill_s <= t.ttft_s <= t.prefill_s + t.decode_s


def test_eos_counts_but_is_not_shown(M, tiny):
    model, orc_model = tiny
    prompt = prompt_of(M, 6)
    first = oracle_ids(orc_model, prompt, 1, 64)[0]
    dec = M.Qwen3Decoder(model, 64)
    seen, n, t = dec.generate_tokens(prompt, 20, eos=(5, first))
    assert n == 1 and seen == [] and t.n_gen == 1
    assert dec.n_past == len(prompt)


def test_eos_mid_run_with_host_sampling(M, tiny):
    """Penalties make the ids vary; EOS = the id of step 5 stops there."""
    model, orc_model = tiny
    prompt = prompt_of(M, 5)
    par = dict(repeat_penalty=1.5, penalty_window=16)
    want = oracle_ids(orc_model, prompt, 24, 64, sampler=O.OracleSampler(4096, **par))
    assert len(set(want)) > 6, want
    k = next(i for i, t in enumerate(want) if i >= 5 and t not in want[:i])
    dec = M.Qwen3Decoder(model, 64)
    seen, n, _ = dec.generate_tokens(prompt, 24, eos=(want[k],),
                                     sampler=O.OracleSampler(4096, **par))
    assert n == k + 1 and seen == want[:k]
    assert dec.n_past == len(prompt) - 1 + k + 1


@pytest.mark.parametrize("par", [dict(repeat_penalty=1.5, penalty_window=16),
                                 dict(temp=0.6, top_k=20, top_p=0.95, seed=7),
                                 dict(temp=1.2, min_p=0.02, freq_penalty=0.3,
                                      presence_penalty=0.2, penalty_window=8, seed=3)],
                         ids=["penalty", "qwen3-defaults", "penalised-temperature"])
def test_host_sampling_matches_the_loop(M, tiny, par):
    print(f"[case] generate host sampler {par}", flush=True)
    model, orc_model = tiny
    prompt, steps = prompt_of(M, 5), 24
    want = oracle_ids(orc_model, prompt, steps, 64, sampler=O.OracleSampler(4096, **par))
    dec = M.Qwen3Decoder(model, 64)
    seen, n, _ = dec.generate_tokens(prompt, steps, sampler=O.OracleSampler(4096, **par))
    assert n == steps and seen == want


def test_callback_stop_inside_a_chunk_rewinds(M, tiny):
    """Stop after 5 ids while the device runs chunks of 8: the position is
    the stopping step's, and the next step's logits equal those of a
    decoder that ran exactly those steps, bit for bit."""
    model, orc_model = tiny
    prompt = prompt_of(M, 7)
    want = oracle_ids(orc_model, prompt, 5, 64, stop_after=5)
    dec = M.Qwen3Decoder(model, 64)
    seen, n, _ = dec.generate_tokens(prompt, 30, chunk=8, stop_after=5)
    assert n == 5 and seen == want
    assert dec.n_past == len(prompt) - 1 + 5
    after = dec.forward(seen[-1])
    ref = M.Qwen3Decoder(model, 64)
    for tok in prompt[:-1]:
        ref.forward(tok, want_logits=False)
    for tok in [prompt[-1]] + seen[:-1]:
        ref.forward(tok, want_logits=False)
    assert np.array_equal(after.view(np.uint32), ref.forward(seen[-1]).view(np.uint32))


@pytest.mark.parametrize("sampled", [False, True])
def test_context_end_stops_the_loop(M, tiny, sampled):
    model, orc_model = tiny
    prompt, n_ctx = prompt_of(M, 5), 14
    par = dict(repeat_penalty=1.5, penalty_window=16)
    want = oracle_ids(orc_model, prompt, 50, n_ctx,
                      sampler=O.OracleSampler(4096, **par) if sampled else None)
    assert len(want) == n_ctx - (len(prompt) - 1)
    dec = M.Qwen3Decoder(model, n_ctx)
    seen, n, _ = dec.generate_tokens(prompt, 50,
                                     sampler=O.OracleSampler(4096, **par) if sampled else None)
    assert n == len(want) and seen == want and dec.n_past == n_ctx


def test_qwen3_06b_generate_matches_golden(M):
    """configs[2]'s model from an empty cache: the prompt of the golden
    teacher-forced run's first 9 inputs, 32 greedy ids through the loop,
    against the oracle's loop."""
    print("[case] generate 0.6B", flush=True)
    g = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                             "qwen3_06b_forced.npz"), allow_pickle=False)
    prompt = [int(t) for t in g["inputs"][:9]]
    model = M.SynthQwen3(CF.QWEN3_06B, 0)
    orc_model = O.SynthModel(CF.QWEN3_06B, 0)
    want = oracle_ids(orc_model, prompt, 32, 64)
    dec = M.Qwen3Decoder(model, 64)
    seen, n, t = dec.generate_tokens(prompt, 32)
    assert n == 32 and seen == want
    print(f"0.6B generate: prefill {t.prefill_s * 1e3:.2f} ms, TTFT {t.ttft_s * 1e3:.2f} ms, "
          f"{t.n_gen / t.decode_s:.0f} tok/s")


GEN_CASES = json.load(open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                                        "generate_cases.json")))


@pytest.mark.parametrize("name", sorted(GEN_CASES))
def test_loop_against_the_compiled_reference_loop(M, tiny, name):
    """The compiled src/generate.c:13-86's record (tests/golden/
    generate_cases.json) replayed through mynah_hip_qwen3_generate_tokens
    with the channel-routing callback a front end binds (think markers,
    answer-callback stop): each channel's ids, the count returned, the
    timing's generated count and the position afterwards."""
    c, want = GEN_CASES[name], GEN_CASES[name]["want"]
    print(f"[case] generate vs compiled loop: {name}", flush=True)
    model, _ = tiny
    router = O.ChannelRouter(c["think"][0], c["think"][1], c["stop_after"])
    sampler = O.OracleSampler(CF.QWEN3_TINY.vocab, **c["sampler"]) if c["sampler"] else None
    dec = M.Qwen3Decoder(model, c["n_ctx"])
    _, n, t = dec.generate_tokens(c["prompt"], c["max_new"], eos=tuple(c["eos"]),
                                  sampler=sampler, on_token=router)
    assert router.answer == want["answer"] and router.think == want["think"]
    assert n == want["produced"] and t.n_gen == want["n_gen"]
    assert dec.n_past == want["n_past"]
