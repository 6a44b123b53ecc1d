"""Context buckets: a step's attention launches sized for the positions it
reaches, not for the whole context.

A decoder replays one graph per bucket (capacities 256, 512, 1024, 2048,
3072, 4096, then doubling, each clamped to n_ctx); the attention grids, the
split chunk size and the exact PV kernel (probabilities in LDS up to 4096
positions, from the scores rows past that) follow the bucket. The result may
not depend on it: the tiny model, 1100 teacher-forced steps in pieces that
cross the 256, 512 and 1024 boundaries (single and eight-step graphs on both
sides), decoded with n_ctx 40960 by buckets, with n_ctx 40960 as one bucket
(MYNAH_CTX_BUCKETS=0: the whole-context grids and the PV kernel that reads
the probabilities from memory) and with n_ctx 1101. Exact attention: every
piece's greedy ids and last logits bit for bit equal across the three, and
the last logits against the oracle decoder (the restated reference) within
|gpu - ref| / max(1, |ref|) <= 1e-4. The same across the largest buckets
(32,760 cached positions, steps past 32,768, where the probabilities come
from memory). Split attention: the buckets below 32768 positions take
32-position chunks at both context sizes, so n_ctx 40960 and 1101 agree bit
for bit.
"""
from __future__ import annotations

import numpy as np
import pytest

import configs as CF
import oracle_lib as O

pytestmark = pytest.mark.gpu
TOL = 1e-4
N_BIG, N_SMALL = 40960, 1101
PIECES = (0, 250, 259, 600, 1100)


@pytest.fixture(scope="module")
def M():
    import mynah_amd
    mynah_amd.check(mynah_amd.lib.mynah_hip_init(0), "init")
    mynah_amd.check(mynah_amd.lib.mynah_hip_set_gemv_order(0), "order")
    return mynah_amd


@pytest.fixture(scope="module")
def inputs(M):
    shape = CF.QWEN3_TINY
    return [int(t) for t in CF.forced_inputs(M.synth_uniform, M.substream, shape.vocab,
                                             PIECES[-1])]


def run(M, n_ctx, mode, inputs, monkeypatch, buckets=True):
    if buckets:
        monkeypatch.delenv("MYNAH_CTX_BUCKETS", raising=False)
    else:
        monkeypatch.setenv("MYNAH_CTX_BUCKETS", "0")
    model = M.SynthQwen3(CF.QWEN3_TINY, 0)
    dec = M.Qwen3Decoder(model, n_ctx)
    monkeypatch.delenv("MYNAH_CTX_BUCKETS", raising=False)
    dec.set_attention(mode)
    out = []
    for a, b in zip(PIECES[:-1], PIECES[1:]):
        ids, lg = dec.forced(inputs[a:b])
        out.append((ids, lg))
    assert dec.uses_graph and dec.n_past == PIECES[-1]
    # After a reset the first bucket's graph replays from position 0 again.
    dec.reset()
    again = dec.forced(inputs[: PIECES[1]])
    assert again[0] == out[0][0]
    assert np.array_equal(again[1].view(np.uint32), out[0][1].view(np.uint32))
    dec.close()
    return out


def same(a, b):
    for (ia, la), (ib, lb) in zip(a, b):
        assert ia == ib
        assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))


def test_exact_attention_independent_of_buckets(M, inputs, monkeypatch):
    print(f"[case] tiny exact attention, {PIECES[-1]} forced steps, n_ctx {N_BIG} by buckets, "
          f"as one bucket, and n_ctx {N_SMALL}", flush=True)
    by_bucket = run(M, N_BIG, M.ATTN_EXACT, inputs, monkeypatch)
    whole = run(M, N_BIG, M.ATTN_EXACT, inputs, monkeypatch, buckets=False)
    small = run(M, N_SMALL, M.ATTN_EXACT, inputs, monkeypatch)
    same(by_bucket, whole)
    same(by_bucket, small)
    O.orc.orc_threads_init(0)
    orc = O.OracleQwen3(O.SynthModel(CF.QWEN3_TINY, 0), N_SMALL)
    for tok in inputs[:-1]:
        orc.forward(tok)
    want = orc.forward(inputs[-1]).astype(np.float64)
    got = by_bucket[-1][1].astype(np.float64)
    err = float((np.abs(got - want) / np.maximum(1.0, np.abs(want))).max())
    print(f"last step against the oracle: max rel err {err:.2e}")
    assert err <= TOL


def test_exact_attention_across_the_top_buckets(M, monkeypatch):
    """Past 4096 positions the exact PV kernel reads the probabilities from
    memory and the grids grow with the bucket: the tiny model with n_ctx
    33,000 and 32,760 cached positions of N(0, 1), then 12 forced steps
    across the 32,768-position boundary (the last bucket is the context
    itself), by buckets and as one bucket: ids and last logits bit for bit
    equal, and the last logits against the oracle within 1e-4."""
    shape, n_ctx, n_pre, steps = CF.QWEN3_TINY, 33000, 32760, 12
    print(f"[case] tiny exact attention, n_ctx {n_ctx}, {n_pre} cached, {steps} steps "
          f"across 32768", flush=True)
    k, v = O.kv_prefill(O.substream, shape, 0, n_pre)
    inputs = [int(t) for t in CF.forced_inputs(M.synth_uniform, M.substream, shape.vocab, steps)]
    model = M.SynthQwen3(shape, 0)
    out = []
    for buckets in ("1", "0"):
        monkeypatch.setenv("MYNAH_CTX_BUCKETS", buckets)
        dec = M.Qwen3Decoder(model, n_ctx)
        monkeypatch.delenv("MYNAH_CTX_BUCKETS")
        dec.set_kv(k, v, n_pre)
        out.append(dec.forced(inputs))
        dec.close()
    assert out[0][0] == out[1][0]
    assert np.array_equal(out[0][1].view(np.uint32), out[1][1].view(np.uint32))
    O.orc.orc_threads_init(0)
    orc = O.OracleQwen3(O.SynthModel(shape, 0), n_ctx)
    orc.prefill_kv(k, v, n_pre)
    for tok in inputs[:-1]:
        orc.forward(tok)
    want = orc.forward(inputs[-1]).astype(np.float64)
    got = out[0][1].astype(np.float64)
    err = float((np.abs(got - want) / np.maximum(1.0, np.abs(want))).max())
    print(f"last step against the oracle: max rel err {err:.2e}")
    assert err <= TOL


def test_split_attention_independent_of_context_size(M, inputs, monkeypatch):
    print(f"[case] tiny split attention, {PIECES[-1]} forced steps, n_ctx {N_BIG} and {N_SMALL}",
          flush=True)
    same(run(M, N_BIG, M.ATTN_SPLIT, inputs, monkeypatch),
         run(M, N_SMALL, M.ATTN_SPLIT, inputs, monkeypatch))
