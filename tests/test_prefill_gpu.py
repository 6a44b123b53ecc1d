"""GPU parity of the batched prompt prefill through the C ABI.

mynah_hip_qwen3_prefill fills the cache T tokens at a time with GEMMs that
sum in the matvec order, per-row RMSNorm / SwiGLU, and per-query attention
in the decode kernels' arithmetic. Its contract is BIT-IDENTITY with feeding
the same tokens one decode step at a time (mynah_hip_qwen3_forward without
logits, exact GEMV order, exact attention), which is itself within the
reference's 1e-4 metric of the compiled reference and gives its greedy ids
(test_decode_gpu.py). Checked here: the matvec-order GEMM against the oracle
matvec of every token (bit-exact, Q4_K / Q6_K / Q8_0 / Q4_0, with and without the
residual epilogue); the whole K/V cache and the next step's logits after a
batched prefill against the step-by-step fill (bit-exact), for the tiny
model across chunk sizes 1, 7, 64 and 512 and a prefill starting after a
synthetic cache, for Qwen3-0.6B, and the prompt() loop's greedy ids (the
Qwen3-4B 2048-token prefill at the default chunk is in
test_decode_forced_gpu.py).
"""
from __future__ import annotations

import os

import numpy as np
import pytest

import configs as CF
import oracle_lib as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def M():
    import mynah_amd
    mynah_amd.check(mynah_amd.lib.mynah_hip_init(0), "init")
    mynah_amd.check(mynah_amd.lib.mynah_hip_set_gemv_order(0), "order")
    O.orc.orc_threads_init(0)
    return mynah_amd


@pytest.fixture
def chunk():
    saved = os.environ.get("MYNAH_PREFILL_CHUNK")

    def set_(n):
        os.environ["MYNAH_PREFILL_CHUNK"] = str(n)

    yield set_
    if saved is None:
        os.environ.pop("MYNAH_PREFILL_CHUNK", None)
    else:
        os.environ["MYNAH_PREFILL_CHUNK"] = saved


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.mark.parametrize("qtype", [12, 14, 8, 2])
@pytest.mark.parametrize("rows,cols,tokens", [(96, 1024, 5), (130, 2048, 64), (64, 512, 131)])
def test_matmat_mv_equals_matvec(M, qtype, rows, cols, tokens):
    print(f"[case] matmat_mv type={qtype} {rows}x{cols} tokens={tokens}", flush=True)
    w = M.synth_blocks(qtype, 3, rows, cols)
    x = M.synth_normal(4, tokens * cols)
    y = M.matmat_mv(qtype, w, rows, cols, x, tokens).reshape(tokens, rows)
    for t in range(tokens):
        ref = O.matvec(qtype, w, rows, cols, x[t * cols:(t + 1) * cols])
        assert np.array_equal(bits(y[t]), bits(ref)), f"token {t}"
    res = M.synth_normal(5, tokens * rows)
    y2 = M.matmat_mv(qtype, w, rows, cols, x, tokens, res=res)
    assert np.array_equal(bits(y2), bits((res + y.reshape(-1)).astype(np.float32)))


def fill_both(M, model, prompt, n_ctx, kv=None):
    """Decoder A fed token by token, decoder B prefilled in batches; both
    optionally start from the same synthetic cache."""
    a = M.Qwen3Decoder(model, n_ctx)
    b = M.Qwen3Decoder(model, n_ctx)
    if kv is not None:
        k, v, n0 = kv
        a.set_kv(k, v, n0)
        b.set_kv(k, v, n0)
    for t in prompt:
        a.forward(int(t), want_logits=False)
    b.prefill(prompt)
    assert a.n_past == b.n_past
    return a, b


def assert_same_state(a, b, nxt):
    n = a.n_past
    ka, va = a.get_kv(n)
    kb, vb = b.get_kv(n)
    for l in range(ka.shape[0]):
        assert np.array_equal(bits(ka[l]), bits(kb[l])), f"K of layer {l}"
        assert np.array_equal(bits(va[l]), bits(vb[l])), f"V of layer {l}"
    la, lb = a.forward(nxt), b.forward(nxt)
    assert np.array_equal(bits(la), bits(lb))


@pytest.mark.parametrize("chunk_size", [1, 7, 64, 512])
def test_tiny_prefill_equals_steps(M, chunk, chunk_size):
    chunk(chunk_size)
    shape = CF.QWEN3_TINY
    print(f"[case] tiny prefill chunk={chunk_size}", flush=True)
    model = M.SynthQwen3(shape, 0)
    prompt = M.synth_uniform(M.substream(7, 2), 70, shape.vocab)
    a, b = fill_both(M, model, prompt, 80)
    assert_same_state(a, b, int(prompt[3]))


def test_tiny_prefill_after_cache(M, chunk):
    """Prefill from position 16 of a synthetic cache, chunks crossing the
    64-token GEMM tiles and the 16-position score chunks."""
    chunk(33)
    shape = CF.QWEN3_TINY
    model = M.SynthQwen3(shape, 0)
    k, v = O.kv_prefill(O.substream, shape, 0, 16)
    prompt = M.synth_uniform(M.substream(7, 3), 81, shape.vocab)
    a, b = fill_both(M, model, prompt, 100, kv=(k, v, 16))
    assert_same_state(a, b, int(prompt[0]))


@pytest.mark.parametrize("group", [3, 5, 6, 7, 8])
def test_prefill_equals_steps_every_group(M, chunk, group):
    """Query heads per key head 3 .. 8 (Qwen3-14B has 5): the batched
    prefill (its PV tiles compiled per group) leaves K/V and the next
    logits bit-identical to token-by-token steps."""
    chunk(40)
    shape = CF.Qwen3Shape(2, 512, 768, 2 * group, 2, 128, 4096)
    print(f"[case] prefill group={group}", flush=True)
    model = M.SynthQwen3(shape, 0)
    prompt = M.synth_uniform(M.substream(7, 5), 75, shape.vocab)
    a, b = fill_both(M, model, prompt, 80)
    assert_same_state(a, b, int(prompt[2]))


def test_prefill_after_cache_crosses_score_tiles(M, chunk):
    """Group 8 (the scores tile's largest query block in LDS), prefill of
    100 tokens from position 200 of a synthetic cache: the queries' rows
    cross the 256-position score tiles, and the last 16-query tile holds 4."""
    chunk(100)
    shape = CF.Qwen3Shape(2, 512, 768, 16, 2, 128, 4096)
    print("[case] prefill group=8 from position 200", flush=True)
    model = M.SynthQwen3(shape, 0)
    k, v = O.kv_prefill(O.substream, shape, 0, 200)
    prompt = M.synth_uniform(M.substream(7, 6), 100, shape.vocab)
    a, b = fill_both(M, model, prompt, 320, kv=(k, v, 200))
    assert_same_state(a, b, int(prompt[4]))


def test_qwen3_06b_prefill_equals_steps(M):
    shape = CF.QWEN3_06B
    print("[case] Qwen3-0.6B prefill of 100 tokens", flush=True)
    model = M.SynthQwen3(shape, 0)
    prompt = M.synth_uniform(M.substream(7, 4), 100, shape.vocab)
    a, b = fill_both(M, model, prompt, 104)
    assert_same_state(a, b, int(prompt[1]))


def test_prompt_batched_equals_steps(M):
    """prompt(): batched prefill then greedy steps gives the same ids and
    position as the decode-step prefill."""
    shape, steps = CF.QWEN3_TINY, 12
    model = M.SynthQwen3(shape, 0)
    prompt = M.synth_uniform(M.substream(7, 5), 40, shape.vocab)
    out = []
    for mode in (M.PREFILL_BATCHED, M.PREFILL_STEPS):
        dec = M.Qwen3Decoder(model, len(prompt) + steps + 1)
        dec.set_prefill(mode)
        toks, _, _ = dec.prompt(prompt, steps)
        assert dec.n_past == len(prompt) - 1 + steps
        out.append(toks)
    assert out[0] == out[1]


def test_prefill_refuses_overflow(M):
    shape = CF.QWEN3_TINY
    model = M.SynthQwen3(shape, 0)
    dec = M.Qwen3Decoder(model, 8)
    with pytest.raises(M.HipError):
        dec.prefill(np.arange(9, dtype=np.uint32))
    with pytest.raises(M.HipError):
        dec.prefill(np.array([shape.vocab], dtype=np.uint32))
    assert dec.n_past == 0
    dec.prefill(np.arange(8, dtype=np.uint32))
    assert dec.n_past == 8
