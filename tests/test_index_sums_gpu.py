"""The reference's double sums through their index-order path.

RMSNorm's sum of squares (/root/reference/src/kernels.c:118-121) and the
softmax's sum of exponentials (:207-220) are double sums in index order. The
kernels outside the GEMVs take them in a parallel order — the query and key
norms of the exact attention's score kernel, the softmax of the exact PV
kernels, of the long-context softmax and of the prefill softmax, the
prefill's row norms and query/key norms, the final-norm kernel — and keep
the f32 result only where it is the same over the whole interval the
reference's sum can lie in (csrc/sum_settle.h); elsewhere they take the
index-order sum (the score kernel normalises again and rewrites its scores,
the PV kernel's chain wave rewrites the probabilities).
mynah_hip_set_index_order_sums(1) sends every such sum through that path
(the score kernel's second pass and the PV kernel's rewrite included), and
these tests hold it to the same bits as the checked path and the reference:

* one layer's exact attention (both PV kernels; n_kv 513 .. 8003, the
  probabilities in LDS and through memory) bit-identical to the oracle's;
* configs[2]'s 64 teacher-forced steps through the replayed graphs: every
  greedy id and the last step's whole logits vector (SHA-256) equal to the
  compiled reference's golden;
* a 0.6B 300-token batched prefill: K/V and the next step's logits
  bit-identical to the same prefill with the checked sums.
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

ONE_LAYER = {
    2: CF.Qwen3Shape(1, 1024, 3072, 16, 8, 128, 2048),
    4: CF.Qwen3Shape(1, 2560, 9728, 32, 8, 128, 2048),
}


@pytest.fixture(scope="module")
def M():
    import mynah_amd
    mynah_amd.check(mynah_amd.lib.mynah_hip_init(0), "init")
    mynah_amd.check(mynah_amd.lib.mynah_hip_set_gemv_order(0), "order")
    O.orc.orc_threads_init(0)
    return mynah_amd


@pytest.fixture
def index_order(M):
    M.check(M.lib.mynah_hip_set_index_order_sums(1), "index-order sums on")
    yield
    M.check(M.lib.mynah_hip_set_index_order_sums(0), "index-order sums off")


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def test_switch_refuses_other_values(M):
    with pytest.raises(M.HipError, match="index-order"):
        M.check(M.lib.mynah_hip_set_index_order_sums(2), "index-order sums")


@pytest.mark.parametrize("group", [2, 4])
@pytest.mark.parametrize("n_pre,n_ctx", [(512, 520), (8002, 8010)])
def test_attention_index_order_against_oracle(M, index_order, monkeypatch, group, n_pre, n_ctx):
    shape = ONE_LAYER[group]
    print(f"[case] index-order sums, one layer, group {group}, n_kv {n_pre + 1}", flush=True)
    model = M.SynthQwen3(shape, 0)
    k, v = O.kv_prefill(O.substream, shape, 0, n_pre)
    tok = O.first_token(0, shape.vocab)
    orc = O.OracleQwen3(O.SynthModel(shape, 0), n_ctx)
    orc.prefill_kv(k, v, n_pre)
    want_logits = orc.forward(tok)
    want = orc.last_attn()
    del orc
    for pv in ("1", "0"):
        monkeypatch.setenv("MYNAH_ATTN_PV", pv)
        dec = M.Qwen3Decoder(model, n_ctx)
        monkeypatch.delenv("MYNAH_ATTN_PV")
        dec.set_attention(M.ATTN_EXACT)
        dec.set_kv(k, v, n_pre)
        lg = dec.forward(tok)
        got = dec.read_attn()
        dec.close()
        assert np.array_equal(bits(got), bits(want)), f"MYNAH_ATTN_PV={pv}"
        assert np.array_equal(bits(lg), bits(want_logits)), f"MYNAH_ATTN_PV={pv}"


def test_06b_forced_graph_index_order_against_golden(M, index_order):
    print("[case] index-order sums, 0.6B teacher-forced graph replay", flush=True)
    g = np.load(os.path.join(GOLDEN, "qwen3_06b_forced.npz"), allow_pickle=False)
    model = M.SynthQwen3(CF.QWEN3_06B, 0)
    assert hashlib.sha256(model.blob.tobytes()).hexdigest() == str(g["blob_sha"])
    inputs = [int(t) for t in g["inputs"]]
    k, v = O.kv_prefill(O.substream, CF.QWEN3_06B, 0, CF.C3_PREFILL)
    dec = M.Qwen3Decoder(model, CF.C3_PREFILL + CF.C3_FORCED_STEPS + 1)
    dec.set_attention(M.ATTN_EXACT)
    dec.set_kv(k, v, CF.C3_PREFILL)
    greedy, last = dec.forced(inputs)
    assert dec.uses_graph
    dec.close()
    assert greedy == [int(t) for t in g["greedy"]]
    assert hashlib.sha256(np.ascontiguousarray(last).tobytes()).hexdigest() == \
        str(g["logits_sha"][len(inputs) - 1])


def test_06b_prefill_index_order_equals_checked(M):
    print("[case] index-order sums, 0.6B 300-token batched prefill", flush=True)
    shape = CF.QWEN3_06B
    model = M.SynthQwen3(shape, 0)
    prompt = [int(t) for t in M.synth_uniform(M.substream(11, 3), 300, shape.vocab)]
    out = []
    for on in (0, 1):
        M.check(M.lib.mynah_hip_set_index_order_sums(on), "index-order sums")
        try:
            dec = M.Qwen3Decoder(model, len(prompt) + 1)
            dec.prefill(prompt[:-1])
            lg = dec.forward(prompt[-1])
            kv = dec.get_kv(len(prompt))
            dec.close()
        finally:
            M.check(M.lib.mynah_hip_set_index_order_sums(0), "index-order sums off")
        out.append((lg, kv))
    (la, (ka, va)), (lb, (kb, vb)) = out
    assert np.array_equal(bits(ka), bits(kb))
    assert np.array_equal(bits(va), bits(vb))
    assert np.array_equal(bits(la), bits(lb))
