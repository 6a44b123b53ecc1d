"""The reference's sampler on the device (include/mynah_generate.h,
mynah_hip_sampler_*, csrc/sample.hip) against the oracle's restatement of
mynah_slm_sample (oracle/sampler.c, pinned bit for bit against the compiled
reference's sampler in test_sampler_oracle.py).

Checked bit for bit: the picked ids and the logits the penalties leave in
place, over streams of logits with exact ties at the top (the lower id must
win) and extra window entries between draws, at a 3,000-entry vocabulary
(two workgroups) and Qwen3's 151,936 (75), for greedy with penalties, the
Qwen3 defaults, min_p, top_p with frequency and presence penalties, top_k 1
and 128, a hot temperature, seed 0's fixed state, temperatures 0.01 and 100,
a top_p below the best candidate's probability, min_p 1 and a window of 4096
entries; the index-order double sum forced on (MYNAH_SAMPLE_SEQ_SUM=1) gives
the same ids. Then the
generation loop with the device sampler against the same loop with the
oracle sampler on the host (the decoder's logits are bit-identical, so the
sampler is the only difference): ids, count, a stop in the middle of a
device chunk, and the sampler's state after the call (its next draw). The
settings the device sampler does not take (temp > 0 with top_k 0, above
128 or not below the vocabulary, a window over 4096, an empty vocabulary or
one above 32 x 8192) are refused when the sampler is made; the largest
vocabulary taken (32 x 8192, the most lists the merge takes) draws as the
oracle does.
"""
from __future__ import annotations

import numpy as np
import pytest

import configs as CF
import oracle_lib as O

pytestmark = pytest.mark.gpu

CASES = [
    dict(repeat_penalty=1.3, penalty_window=16),                              # greedy + penalty
    dict(temp=0.6, top_k=20, top_p=0.95, seed=7),                             # Qwen3 defaults
    dict(temp=1.0, top_k=40, min_p=0.05, seed=3),
    dict(temp=0.8, top_k=50, top_p=0.5, freq_penalty=0.2, presence_penalty=0.1,
         penalty_window=8, seed=11),
    dict(temp=1.5, top_k=128, seed=0),                                        # the fixed default state
    dict(temp=0.7, top_k=1, seed=5),
    dict(temp=3.0, top_k=100, top_p=0.99, repeat_penalty=0.9, penalty_window=64, seed=9),
    dict(temp=0.01, top_k=20, top_p=0.95, seed=2),                          # nearly greedy
    dict(temp=100.0, top_k=128, min_p=0.5, seed=4),                          # nearly flat
    dict(temp=0.6, top_k=20, top_p=0.01, seed=6),                            # top_p below the best
    dict(temp=1.0, top_k=64, min_p=1.0, seed=8),                             # min_p keeps the best
    dict(temp=0.9, top_k=30, repeat_penalty=1.1, freq_penalty=0.05, presence_penalty=0.2,
         penalty_window=4096, seed=10),                                      # the largest window
]


@pytest.fixture(scope="module")
def M():
    import mynah_amd
    mynah_amd.check(mynah_amd.lib.mynah_hip_init(0), "init")
    mynah_amd.check(mynah_amd.lib.mynah_hip_set_gemv_order(0), "order")
    O.orc.orc_threads_init(0)
    return mynah_amd


def logits_stream(seed, steps, vocab):
    x = O.normal(seed, steps * vocab).reshape(steps, vocab) * np.float32(3.0)
    x[:, 17] = x[:, 5]               # exact ties: the lower id must win
    top = np.argmax(x, axis=1)
    x[np.arange(steps), (top + 1) % vocab] = x[np.arange(steps), top]   # ties at the top
    return x


def draws(sampler, vocab, steps=30, seed=1):
    ids, after = [], []
    for i, row in enumerate(logits_stream(seed, steps, vocab)):
        lg = np.ascontiguousarray(row)
        t = sampler.sample(lg)
        ids.append(t)
        after.append(lg.copy())
        sampler.accept(t)
        if i % 3 == 0:
            sampler.accept((t * 7 + 1) % vocab)
    return ids, np.stack(after)


@pytest.mark.parametrize("vocab", [3000, 151936])
@pytest.mark.parametrize("params", CASES, ids=[str(i) for i in range(len(CASES))])
def test_device_sampler_matches_the_reference_sampler(M, params, vocab):
    print(f"[case] device sampler {params} vocab {vocab}", flush=True)
    want = draws(O.OracleSampler(vocab, **params), vocab)
    dev = M.DeviceSampler(vocab, **params)
    got = draws(dev, vocab)
    dev.close()
    assert got[0] == want[0]
    assert np.array_equal(got[1].view(np.uint32), want[1].view(np.uint32))


def test_index_order_sum_gives_the_same_draws(M, monkeypatch):
    """The inverse of the double sum taken from the reference's own
    index-order sum (the path a sum too close to a rounding boundary takes)
    against the bounded double-double sum."""
    params, vocab = CASES[1], 151936
    print("[case] device sampler, index-order sum forced", flush=True)
    a = M.DeviceSampler(vocab, **params)
    monkeypatch.setenv("MYNAH_SAMPLE_SEQ_SUM", "1")
    b = M.DeviceSampler(vocab, **params)
    monkeypatch.delenv("MYNAH_SAMPLE_SEQ_SUM")
    ga, gb = draws(a, vocab, steps=12), draws(b, vocab, steps=12)
    a.close()
    b.close()
    assert ga[0] == gb[0]
    assert ga[0] == draws(O.OracleSampler(vocab, **params), vocab, steps=12)[0]


@pytest.mark.parametrize("params,error", [
    (dict(temp=0.6, top_k=0), "top_k"),
    (dict(temp=0.6, top_k=129), "top_k"),
    (dict(temp=0.6, top_k=20, penalty_window=5000), "window"),
])
def test_unsupported_settings_are_refused(M, params, error):
    with pytest.raises(M.HipError, match=error):
        M.DeviceSampler(3000, **params)


@pytest.mark.parametrize("vocab,params,error", [
    (0, dict(), "empty vocabulary"),
    (32 * 8192 + 1, dict(), "exceeds"),          # more top-k workgroups than the merge takes
    (100, dict(temp=0.6, top_k=100), "top_k"),   # top_k not below the vocabulary
])
def test_unsupported_vocabularies_are_refused(M, vocab, params, error):
    with pytest.raises(M.HipError, match=error):
        M.DeviceSampler(vocab, **params)


def test_largest_vocabulary_taken(M):
    """32 top-k workgroups of 8,192 probabilities: the largest vocabulary the
    merge takes, against the oracle sampler."""
    vocab, params = 32 * 8192, CASES[1]
    print(f"[case] device sampler {params} vocab {vocab}", flush=True)
    want = draws(O.OracleSampler(vocab, **params), vocab, steps=6)
    dev = M.DeviceSampler(vocab, **params)
    got = draws(dev, vocab, steps=6)
    dev.close()
    assert got[0] == want[0]
    assert np.array_equal(got[1].view(np.uint32), want[1].view(np.uint32))


@pytest.mark.parametrize("params", CASES[:5], ids=[str(i) for i in range(5)])
def test_generation_loop_with_the_device_sampler(M, params):
    """generate_tokens(device_sampler=...) against the same loop with the
    oracle sampler on the host: two calls in a row on each side (the second
    stopped by the callback in the middle of an eight-step chunk), then one
    more draw from each sampler on the same logits."""
    shape = CF.QWEN3_TINY
    print(f"[case] generation loop, device sampler {params}", flush=True)
    model = M.SynthQwen3(shape, 0)
    prompt = [int(t) for t in M.synth_uniform(M.substream(6, 1), 9, shape.vocab)]
    results = []
    for side in ("host", "device"):
        smp = (O.OracleSampler(shape.vocab, **params) if side == "host"
               else M.DeviceSampler(shape.vocab, **params))
        dec = M.Qwen3Decoder(model, 96)
        kw = dict(sampler=smp) if side == "host" else dict(device_sampler=smp)
        s1, n1, _ = dec.generate_tokens(prompt, 20, **kw)
        dec.reset()
        s2, n2, _ = dec.generate_tokens(prompt[:5], 30, stop_after=11, **kw)
        lg = np.ascontiguousarray(logits_stream(4, 1, shape.vocab)[0])
        last = smp.sample(lg)
        results.append((s1, n1, s2, n2, last, dec.n_past))
        dec.close()
    host, device = results
    print(f"host {host[:4]}\ndevice {device[:4]}")
    assert device == host
    assert host[1] == 20 and host[3] == 11
