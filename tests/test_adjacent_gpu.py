"""GPU parity of the adjacent block types, Q5_K and Q4_0, through the C ABI.

Every output is BIT-IDENTICAL to the oracle, itself bit-identical to the
compiled reference (test_oracle_adjacent.py): the Q5_K matvec in the order of
the reference's scalar lane (grouped kernel, both the one-lane and the
split-quad layouts), its batched product in the batched core's order, the
Q4_0 matvec and batched product as one running sum per (row, token), and
both dequants. The decoder takes Q5_K and Q4_0 tensors (embedding, tied
head, paired gate/up, K/V, residual projections): its logits match the
oracle decoder within the decode tolerance, its greedy ids equal, and its
batched prefill (Q4_0 through the token chains, whose batched order is the
matvec's) leaves the step-by-step cache bit for bit. Misaligned or ragged
operands are refused by the ABI.
"""
from __future__ import annotations

import ctypes as C
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


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def rel_err(got, ref):
    return float((np.abs(got.astype(np.float64) - ref) / np.maximum(1.0, np.abs(ref))).max())


@pytest.mark.parametrize("case", CF.ADJACENT, ids=lambda c: f"{CF.TYPE_NAME[c[0]]}_{c[1]}x{c[2]}")
def test_golden(M, case):
    t, rows, cols, token_counts = case
    print(f"[case] golden type={t} {rows}x{cols} tokens={token_counts}", flush=True)
    g = np.load(os.path.join(GOLDEN, "adjacent.npz"), allow_pickle=False)
    key = f"{CF.TYPE_NAME[t]}_{rows}x{cols}"
    w = M.synth_blocks(t, 1000 + t + rows, rows, cols)
    x = M.synth_normal(2000 + t + rows, max(token_counts) * cols)
    assert np.array_equal(bits(M.matvec(t, w, rows, cols, x)), bits(g[f"{key}_matvec"]))
    assert np.array_equal(bits(M.dequant(t, w, rows, cols)), bits(g[f"{key}_dequant"]))
    for n in token_counts:
        assert np.array_equal(bits(M.matmat(t, w, rows, cols, x, n)), bits(g[f"{key}_matmat{n}"]))


@pytest.mark.parametrize("qtype,rows,cols", [(13, 4096, 4096), (13, 40000, 1024), (13, 64, 9728),
                                             (2, 4096, 4096), (2, 1000, 2080), (2, 65, 32),
                                             (2, 130, 96), (2, 64, 288), (2, 3, 4160),
                                             (2, 33000, 96)])
def test_matvec_against_oracle(M, qtype, rows, cols):
    """Small and large launches (split quads vs one lane per super-block for
    Q5_K; long and short chains for Q4_0)."""
    print(f"[case] matvec type={qtype} {rows}x{cols}", flush=True)
    w, x = M.synth_blocks(qtype, 7, rows, cols), M.synth_normal(8, cols)
    got, ref = M.matvec(qtype, w, rows, cols, x), O.project(qtype, w, rows, cols, x)
    assert np.array_equal(bits(got), bits(ref)) and rel_err(got, ref) <= TOL


@pytest.mark.parametrize("cols", [32, 96, 2080, 4096])
def test_q40_one_wave_matvec_against_oracle(M, monkeypatch, cols):
    """The matvec's other kernel (MYNAH_Q40_PC=0: one wave decodes and adds)."""
    monkeypatch.setenv("MYNAH_Q40_PC", "0")
    rows = 200
    print(f"[case] Q4_0 one-wave matvec {rows}x{cols}", flush=True)
    w, x = M.synth_blocks(2, 20, rows, cols), M.synth_normal(21, cols)
    assert np.array_equal(bits(M.matvec(2, w, rows, cols, x)), bits(O.matvec(2, w, rows, cols, x)))


@pytest.mark.parametrize("qtype,rows,cols,tokens", [(13, 1024, 2048, 130), (13, 70, 512, 2),
                                                    (2, 512, 2080, 64), (2, 33, 4096, 9),
                                                    # Q4_0 token chains per lane: 8, 4 (ragged), 4
                                                    (2, 4096, 64, 256), (2, 4100, 64, 130),
                                                    (2, 4096, 96, 128)])
def test_matmat_against_oracle(M, qtype, rows, cols, tokens):
    print(f"[case] matmat type={qtype} {rows}x{cols} tokens={tokens}", flush=True)
    w, x = M.synth_blocks(qtype, 9, rows, cols), M.synth_normal(10, tokens * cols)
    got = M.matmat(qtype, w, rows, cols, x, tokens)
    ref = O.matmat(qtype, w, rows, cols, x, tokens, threaded=True)
    assert np.array_equal(bits(got), bits(ref))


def test_q5k_ignores_the_reordered_gemv_switch(M):
    """Q5_K has only the exact kernel: with the reordered order selected its
    matvec stays the reference's."""
    rows, cols = 1024, 2048
    w, x = M.synth_blocks(13, 11, rows, cols), M.synth_normal(12, cols)
    M.check(M.lib.mynah_hip_set_gemv_order(1), "order")
    try:
        got = M.matvec(13, w, rows, cols, x)
    finally:
        M.check(M.lib.mynah_hip_set_gemv_order(0), "order")
    assert np.array_equal(bits(got), bits(O.matvec(13, w, rows, cols, x)))


def test_per_type_entry_points(M):
    lib, P = M.lib, M.ptr
    assert all(lib.ingot_has_kernel(t) == 1 for t in (2, 8, 12, 13, 14))
    assert lib.ingot_has_kernel(3) == 0
    rows, cols, tokens = 96, 1024, 5
    w5, w4 = M.synth_blocks(13, 13, rows, cols), M.synth_blocks(2, 14, rows, cols)
    x = M.synth_normal(15, tokens * cols)
    y = np.empty(rows * tokens, np.float32)
    for f, want in ((lib.ingot_q5_k_matvec, O.matvec(13, w5, rows, cols, x)),
                    (lib.ingot_q5_k_matvec_scalar, O.matvec(13, w5, rows, cols, x))):
        assert f(P(w5), rows, cols, P(x), P(y)) == 0
        assert np.array_equal(bits(y[:rows]), bits(want))
    mm = O.matmat(13, w5, rows, cols, x, tokens)
    for f in (lib.ingot_q5_k_matmat, lib.ingot_q5_k_matmat_exact):
        assert f(P(w5), rows, cols, P(x), P(y), tokens) == 0
        assert np.array_equal(bits(y), bits(mm))
    assert lib.ingot_q4_0_matvec(P(w4), rows, cols, P(x), P(y)) == 0
    assert np.array_equal(bits(y[:rows]), bits(O.matvec(2, w4, rows, cols, x)))
    dq = np.empty(rows * cols, np.float32)
    for f, w, t in ((lib.ingot_q5_k_dequant, w5, 13), (lib.ingot_q4_0_dequant, w4, 2)):
        assert f(P(w), rows, cols, P(dq)) == 0
        assert np.array_equal(bits(dq), bits(O.dequant(t, w, rows, cols)))


def test_device_twins_and_refusals(M):
    rows, cols, tokens = 200, 2048, 3
    for t in (13, 2):
        print(f"[case] device twins type={t}", flush=True)
        w, x = M.synth_blocks(t, 16, rows, cols), M.synth_normal(17, tokens * cols)
        wd, xd = M.DeviceBuffer.from_array(w), M.DeviceBuffer.from_array(x)
        yd = M.DeviceBuffer(4 * rows * cols)
        try:
            M.matvec_dev(t, wd.ptr, rows, cols, xd.ptr, yd.ptr)
            M.sync()
            assert np.array_equal(bits(yd.download(np.float32, rows)),
                                  bits(O.matvec(t, w, rows, cols, x)))
            M.matmat_dev(t, wd.ptr, rows, cols, xd.ptr, yd.ptr, tokens)
            M.sync()
            assert np.array_equal(bits(yd.download(np.float32, rows * tokens)),
                                  bits(O.matmat(t, w, rows, cols, x, tokens)))
            M.dequant_dev(t, wd.ptr, rows, cols, yd.ptr)
            M.sync()
            assert np.array_equal(bits(yd.download(np.float32, rows * cols)),
                                  bits(O.dequant(t, w, rows, cols)))
            # Refused before any launch: misaligned weights, ragged rows.
            bad = 8 if t == 13 else 1
            assert M.lib.mynah_hip_matvec_dev(t, wd.ptr + bad, rows - 1, cols, xd.ptr, yd.ptr,
                                              None) == -1
            assert M.lib.mynah_hip_matvec_dev(t, wd.ptr, rows, cols - 16, xd.ptr, yd.ptr,
                                              None) == -1
            if t == 2:
                # Q4_0's matvec-order GEMM is its batched product.
                M.check(M.lib.mynah_hip_matmat_mv_dev(2, wd.ptr, rows, cols, xd.ptr, yd.ptr,
                                                      tokens, None, None), "matmat_mv")
                M.sync()
                assert np.array_equal(bits(yd.download(np.float32, rows * tokens)),
                                      bits(O.matmat(t, w, rows, cols, x, tokens)))
        finally:
            for b in (wd, xd, yd):
                b.free()
    y = np.empty(16, np.float32)
    w = M.synth_blocks(13, 1, 2, 512)
    x = M.synth_normal(2, 512)
    assert M.lib.ingot_matvec(13, M.ptr(w), 2, 300, M.ptr(x), M.ptr(y)) == -1
    assert M.lib.ingot_dequant_matrix(2, M.ptr(w), 2, 100, M.ptr(y)) == -1


def test_q5k_matmat_mv_equals_matvec(M):
    rows, cols, tokens = 130, 2048, 67
    w, x = M.synth_blocks(13, 18, rows, cols), M.synth_normal(19, tokens * cols)
    y = M.matmat_mv(13, w, rows, cols, x, tokens).reshape(tokens, rows)
    for t in range(tokens):
        assert np.array_equal(bits(y[t]), bits(O.matvec(13, w, rows, cols, x[t * cols:])))


# ── the decoder with Q5_K tensors ─────────────────────────────────────────

Q5K_TENSORS = ("token_embd.weight", "blk.0.attn_q.weight", "blk.0.ffn_gate.weight",
               "blk.0.ffn_up.weight", "blk.1.ffn_down.weight", "blk.2.attn_v.weight",
               "blk.2.attn_k.weight", "blk.1.attn_output.weight")


class Variant:
    """The tiny synthetic Qwen3 with some tensors re-drawn as `qtype`, in
    the attribute layout both the GPU binding and the oracle read."""

    def __init__(self, M, convert, qtype=13, seed=0):
        base = O.SynthModel(CF.QWEN3_TINY, seed)
        self.shape = base.shape
        self.c_shape = M.Qwen3Shape(*[getattr(base.c_shape, n) for n, _ in M.Qwen3Shape._fields_])
        rows = []
        off = 0
        for i in range(base.count):
            t = base.table[i]
            name = t.name.decode()
            if name in convert:
                data = O.blocks(qtype, 5000 + i, t.rows, t.cols)
                typ = qtype
            else:
                data = base.blob[t.offset:t.offset + t.nbytes]
                typ = t.type
            off = (off + 255) & ~255
            rows.append((name, typ, t.rank, t.rows, t.cols, off, data))
            off += data.size
        self.blob = np.zeros(off, np.uint8)
        self.count = len(rows)
        self.table = (M.SynthTensor * self.count)()
        self.by_name = {}
        for i, (name, typ, rank, r, c, o, data) in enumerate(rows):
            self.blob[o:o + data.size] = data
            self.table[i] = M.SynthTensor(name.encode(), typ, rank, r, c, o, data.size)
            self.by_name[name] = self.table[i]

    def tensor(self, name):
        t = self.by_name[name]
        return O.OrcTensor(t.type, t.rows, t.cols, O.ptr(self.blob) + t.offset)


# Q5_K and Q4_0 tensors in the step: the embedding row, single matrices with
# and without the residual, the gate/up pair, and grouped q/k/v launches that
# mix the type with the model's Q4_K / Q6_K matrices.
DECODER_TYPES = [pytest.param(13, id="Q5_K"), pytest.param(2, id="Q4_0")]


@pytest.mark.parametrize("qtype", DECODER_TYPES)
def test_decoder_with_block_type(M, qtype):
    print(f"[case] tiny decoder with type {qtype} tensors vs the oracle, 12 steps", flush=True)
    model = Variant(M, Q5K_TENSORS, qtype=qtype)
    shape, npre, steps = CF.QWEN3_TINY, 16, 12
    k, v = O.kv_prefill(O.substream, shape, 0, npre)
    first = O.first_token(0, shape.vocab)
    n_ctx = npre + steps + 1
    dec = M.Qwen3Decoder(model, n_ctx)
    ref = O.OracleQwen3(model, n_ctx)
    dec.set_kv(k, v, npre)
    ref.prefill_kv(k, v, npre)
    tok, ids = first, []
    for _ in range(steps):
        a, b = dec.forward(tok), ref.forward(tok)
        assert rel_err(a, b) <= TOL
        tok = int(np.argmax(b))
        assert int(np.argmax(a)) == tok
        ids.append(tok)
    dec.reset()
    dec.set_kv(k, v, npre)
    assert dec.generate(first, steps)[0] == ids


@pytest.mark.parametrize("qtype", DECODER_TYPES)
def test_decoder_batched_prefill_is_bit_identical(M, qtype):
    """The batched prefill of a model with Q5_K or Q4_0 projections: the
    cache and the next logits equal the per-token path's bits."""
    print(f"[case] type {qtype} decoder: batched prefill vs steps", flush=True)
    model = Variant(M, Q5K_TENSORS, qtype=qtype)
    prompt = O.uniform(21, 40, CF.QWEN3_TINY.vocab)
    a, b = M.Qwen3Decoder(model, 64), M.Qwen3Decoder(model, 64)
    for t in prompt:
        a.forward(int(t), want_logits=False)
    b.prefill(prompt)
    ka, va = a.get_kv(prompt.size)
    kb, vb = b.get_kv(prompt.size)
    assert np.array_equal(bits(ka), bits(kb)) and np.array_equal(bits(va), bits(vb))
    assert np.array_equal(bits(a.forward(3)), bits(b.forward(3)))


ALL_PROJECTIONS = tuple(["token_embd.weight", "output.weight"] + [
    f"blk.{l}.{n}.weight" for l in range(CF.QWEN3_TINY.n_layers)
    for n in ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down")])


def test_decoder_all_q40_projections(M):
    """Every projection and the embedding/head Q4_0 (a Q4_0 checkpoint's
    layout): greedy ids equal the oracle's."""
    print("[case] tiny decoder, all projections Q4_0, 10 steps", flush=True)
    model = Variant(M, ALL_PROJECTIONS, qtype=2)
    shape, npre, steps = CF.QWEN3_TINY, 8, 10
    k, v = O.kv_prefill(O.substream, shape, 0, npre)
    first = O.first_token(0, shape.vocab)
    dec = M.Qwen3Decoder(model, npre + steps + 1)
    ref = O.OracleQwen3(model, npre + steps + 1)
    dec.set_kv(k, v, npre)
    ref.prefill_kv(k, v, npre)
    tok = first
    for _ in range(steps):
        a, b = dec.forward(tok), ref.forward(tok)
        assert rel_err(a, b) <= TOL
        tok = int(np.argmax(b))
        assert int(np.argmax(a)) == tok


@pytest.mark.parametrize("chunk", ["2048", "16"])
def test_all_q40_batched_prefill(M, monkeypatch, chunk):
    """Every projection Q4_0: a 70-token prompt prefilled in batches (one
    chunk, and 16-token chunks) leaves the per-token cache and next logits
    bit for bit; the chains take 8, 4 or 2 tokens per lane by batch size."""
    monkeypatch.setenv("MYNAH_PREFILL_CHUNK", chunk)
    print(f"[case] all-Q4_0 tiny decoder: batched prefill (chunk {chunk}) vs steps", flush=True)
    model = Variant(M, ALL_PROJECTIONS, qtype=2)
    prompt = O.uniform(23, 70, CF.QWEN3_TINY.vocab)
    a, b = M.Qwen3Decoder(model, 80), M.Qwen3Decoder(model, 80)
    for t in prompt:
        a.forward(int(t), want_logits=False)
    b.prefill(prompt)
    ka, va = a.get_kv(prompt.size)
    kb, vb = b.get_kv(prompt.size)
    assert np.array_equal(bits(ka), bits(kb)) and np.array_equal(bits(va), bits(vb))
    assert np.array_equal(bits(a.forward(5)), bits(b.forward(5)))


@pytest.mark.parametrize("qtype", DECODER_TYPES)
def test_checkpoint_from_gguf(M, qtype, tmp_path):
    """The all-`qtype` model written as a GGUF file: mynah_hip_qwen3_from_gguf
    gives the table-built decoder's bits, and greedy ids equal the oracle's."""
    import gguf_writer as GW
    print(f"[case] all-type-{qtype} GGUF -> from_gguf vs table vs oracle, 6 steps", flush=True)
    model = Variant(M, ALL_PROJECTIONS, qtype=qtype)
    shape, npre, n_ctx = CF.QWEN3_TINY, 8, 24
    path = tmp_path / f"t{qtype}.gguf"
    path.write_bytes(GW.qwen3_writer(model.shape, model.table, model.count, model.blob,
                                     n_ctx).to_bytes())
    a, b = M.Qwen3Decoder.from_gguf(str(path), n_ctx), M.Qwen3Decoder(model, n_ctx)
    ref = O.OracleQwen3(model, n_ctx)
    k, v = O.kv_prefill(O.substream, shape, 0, npre)
    for dec in (a, b):
        dec.set_kv(k, v, npre)
    ref.prefill_kv(k, v, npre)
    tok = O.first_token(0, shape.vocab)
    for _ in range(6):
        la, lb, lr = a.forward(tok), b.forward(tok), ref.forward(tok)
        assert np.array_equal(bits(la), bits(lb))
        assert rel_err(la, lr) <= TOL
        tok = int(np.argmax(lr))
        assert int(np.argmax(la)) == tok
