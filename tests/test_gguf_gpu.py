"""The decoder built from a GGUF checkpoint (mynah_hip_qwen3_from_gguf).

The tiny Qwen3's golden tokens (tests/golden/qwen3_tiny.npz) are what the
compiled reference decoded after loading this very file (the test writer's
bytes equal the reference writer's, test_gguf.py), so loading the GGUF here
and decoding must give the same ids, and the first logits within the decode
tolerance. Built from the file or from the synthetic tensor table, the
decoder holds the same bytes and must give bit-identical logits; an untied
head holding the embedding's bytes must equal the tied one.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

import configs as CF
import gguf_writer as GW
import oracle_lib as O

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TOL = 1e-4
N_PRE, STEPS = 16, 32
N_CTX = N_PRE + STEPS + 1          # the context_length the golden file was written with


@pytest.fixture(scope="module")
def M():
    import mynah_amd
    mynah_amd.check(mynah_amd.lib.mynah_hip_init(0), "init")
    mynah_amd.check(mynah_amd.lib.mynah_hip_set_gemv_order(0), "order")
    return mynah_amd


@pytest.fixture(scope="module")
def tiny(M):
    model = M.SynthQwen3(CF.QWEN3_TINY, 0)
    k, v = O.kv_prefill(O.substream, CF.QWEN3_TINY, 0, N_PRE)
    return model, k, v, O.first_token(0, CF.QWEN3_TINY.vocab)


def rel_err(got, ref):
    return float((np.abs(got.astype(np.float64) - ref) / np.maximum(1.0, np.abs(ref))).max())


def write(tmp_path, name, w: GW.GgufWriter) -> str:
    p = str(tmp_path / f"{name}.gguf")
    with open(p, "wb") as f:
        f.write(w.to_bytes())
    return p


def tiny_writer(model, n_ctx=N_CTX):
    return GW.qwen3_writer(model.shape, model.table, model.count, model.blob, n_ctx)


def test_tiny_gguf_decodes_the_golden_tokens(M, tiny, tmp_path):
    print("[case] tiny GGUF -> from_gguf, 32 greedy steps", flush=True)
    g = np.load(os.path.join(GOLDEN, "qwen3_tiny.npz"), allow_pickle=False)
    model, k, v, first = tiny
    assert first == int(g["first"])
    dec = M.Qwen3Decoder.from_gguf(write(tmp_path, "tiny", tiny_writer(model)))
    assert dec.model.shape.vocab == CF.QWEN3_TINY.vocab
    dec.set_kv(k, v, N_PRE)
    lg = dec.forward(first)
    assert rel_err(lg, g["logits0"]) <= TOL
    dec.reset()
    dec.set_kv(k, v, N_PRE)
    toks, _ = dec.generate(first, STEPS)
    assert toks == [int(t) for t in g["tokens"]]
    # The context is the file's context_length: one more step than it holds fails.
    assert dec.n_past == N_PRE + STEPS
    dec.forward(toks[-1], want_logits=False)
    assert M.lib.mynah_hip_qwen3_forward(dec.h, 1, None) == -1


@pytest.mark.parametrize("ask,have", [(10 * N_CTX, N_CTX), (N_PRE + 3, N_PRE + 3)])
def test_context_clamped_to_context_length(M, tiny, tmp_path, ask, have):
    """src/arch_qwen3.c:94: a context above the file's context_length is cut
    to it, a smaller one is kept; the step after the last position fails."""
    print(f"[case] from_gguf n_ctx {ask} on context_length {N_CTX}", flush=True)
    model, k, v, first = tiny
    dec = M.Qwen3Decoder.from_gguf(write(tmp_path, "ctx", tiny_writer(model)), ask)
    dec.set_kv(k, v, N_PRE)
    tok = first
    for _ in range(have - N_PRE):
        tok = int(np.argmax(dec.forward(tok)))
    assert dec.n_past == have
    assert M.lib.mynah_hip_qwen3_forward(dec.h, tok, None) == -1


def test_file_and_table_decoders_bit_identical(M, tiny, tmp_path):
    print("[case] GGUF decoder vs synthetic-table decoder, 6 steps", flush=True)
    model, k, v, first = tiny
    a = M.Qwen3Decoder.from_gguf(write(tmp_path, "t", tiny_writer(model)), 24)
    b = M.Qwen3Decoder(model, 24)
    for dec in (a, b):
        dec.set_kv(k, v, N_PRE)
    tok = first
    for _ in range(6):
        la, lb = a.forward(tok), b.forward(tok)
        assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
        tok = int(np.argmax(la))


def test_untied_head_equals_tied(M, tiny, tmp_path):
    print("[case] output.weight = token_embd bytes vs tied head", flush=True)
    model, k, v, first = tiny
    w = tiny_writer(model)
    embed = next(t for t in w.tensors if t[0] == "token_embd.weight")
    w.tensor("output.weight", embed[1], embed[2], embed[3])
    a = M.Qwen3Decoder.from_gguf(write(tmp_path, "untied", w), 20)
    b = M.Qwen3Decoder.from_gguf(write(tmp_path, "tied", tiny_writer(model)), 20)
    for dec in (a, b):
        dec.set_kv(k, v, N_PRE)
    assert np.array_equal(a.forward(first).view(np.uint32), b.forward(first).view(np.uint32))


def test_prompt_through_gguf_equals_table(M, tiny, tmp_path):
    print("[case] prompt (batched prefill) via GGUF vs table", flush=True)
    model, _, _, _ = tiny
    prompt = O.uniform(11, 20, CF.QWEN3_TINY.vocab)
    a = M.Qwen3Decoder.from_gguf(write(tmp_path, "p", tiny_writer(model)), 40)
    b = M.Qwen3Decoder(model, 40)
    assert a.prompt(prompt, 8)[0] == b.prompt(prompt, 8)[0]


def test_refusals(M, tiny, tmp_path):
    print("[case] GGUF refusals (no kernel launches)", flush=True)
    model, _, _, _ = tiny
    w = tiny_writer(model)
    w.tensors = [t for t in w.tensors if t[0] != "blk.1.ffn_up.weight"]
    with pytest.raises(M.HipError, match="missing tensor"):
        M.Qwen3Decoder.from_gguf(write(tmp_path, "missing", w))
    w = tiny_writer(model)
    w.tensors = [(n, t, ne[::-1] if n == "blk.0.ffn_gate.weight" else ne, d)
                 for n, t, ne, d in w.tensors]
    with pytest.raises(M.HipError, match="wrong shape"):
        M.Qwen3Decoder.from_gguf(write(tmp_path, "shape", w))
    # An 8-byte tensor first and alignment 8: every later tensor sits 8 bytes
    # off a 16-byte boundary, which the kernels cannot read.
    w = tiny_writer(model)
    w.alignment = 8
    w.tensors.insert(0, ("pad.weight", 0, [2], bytes(8)))
    with pytest.raises(M.HipError, match="16-byte aligned"):
        M.Qwen3Decoder.from_gguf(write(tmp_path, "align8", w))
    # A context up to 2^20 positions is taken; a file whose context_length
    # asks for more is refused.
    with pytest.raises(M.HipError, match="unsupported shape"):
        M.Qwen3Decoder.from_gguf(write(tmp_path, "ctx", tiny_writer(model, (1 << 20) + 1)))
    with pytest.raises(M.HipError):
        M.Qwen3Decoder.from_gguf(str(tmp_path / "absent.gguf"))


def test_split_checkpoint_decodes_like_the_single_file(M, tiny, tmp_path):
    """The tiny model as a three-shard checkpoint (its tensors spread in
    order, the later shards with their own alignments, 64 and 16) opened
    through its second shard's name: the same logits bit for bit as the
    single file, step after step (src/model.c:183 opens both the same way)."""
    print("[case] split GGUF (3 shards) vs single file, 6 steps", flush=True)
    model, k, v, first = tiny
    w = tiny_writer(model)
    d = tmp_path / "split"
    d.mkdir()
    for i, s in enumerate(GW.split_writers(w, 3, alignments=[32, 64, 16])):
        (d / GW.split_name("tiny", i, 3)).write_bytes(s.to_bytes())
    a = M.Qwen3Decoder.from_gguf(str(d / GW.split_name("tiny", 1, 3)), 24)
    b = M.Qwen3Decoder.from_gguf(write(tmp_path, "one", w), 24)
    for dec in (a, b):
        dec.set_kv(k, v, N_PRE)
    tok = first
    for _ in range(6):
        la, lb = a.forward(tok), b.forward(tok)
        assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
        tok = int(np.argmax(la))
