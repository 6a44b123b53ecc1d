"""The restated generation loop (oracle_lib.oracle_generate with the
ChannelRouter callback) against the compiled reference's own loop.

tests/golden/generate_cases.json holds what src/generate.c:13-86, compiled
from the reference's sources (oracle/_ref/libref.so, ref_generate_record),
did on the tiny model with a vocabulary: greedy and sampled runs, an EOS id
first and mid-run (it counts but reaches no callback), the answer callback
stopping the loop, the context running out, and the think markers (each
switches the channel and reaches neither callback; the answer callback's
stop also works after a think block). Per case: the ids each channel saw,
the count the loop returned, the timing's generated count and the state's
position. The sampled cases use the restated sampler (oracle/sampler.c,
pinned to the compiled one in test_sampler_oracle.py).
"""
from __future__ import annotations

import json
import os

import pytest

import configs as CF
import oracle_lib as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
CASES = json.load(open(os.path.join(GOLDEN, "generate_cases.json")))


@pytest.fixture(scope="module")
def model():
    O.orc.orc_threads_init(0)
    return O.SynthModel(CF.QWEN3_TINY, 0)


@pytest.mark.parametrize("name", sorted(CASES))
def test_restated_loop_against_the_compiled_one(model, name):
    c, want = CASES[name], CASES[name]["want"]
    orc = O.OracleQwen3(model, c["n_ctx"])
    router = O.ChannelRouter(c["think"][0], c["think"][1], c["stop_after"])
    sampler = O.OracleSampler(CF.QWEN3_TINY.vocab, **c["sampler"]) if c["sampler"] else None
    ids = O.oracle_generate(orc, c["prompt"], c["max_new"], eos=tuple(c["eos"]),
                            sampler=sampler, on_token=router)
    assert router.answer == want["answer"] and router.think == want["think"]
    assert len(ids) == want["produced"] == want["n_gen"]
    assert O.orc.orc_qwen3_n_past(orc.h) == want["n_past"]


def test_cases_cover_the_loops_exits():
    """Each exit of the loop is in the goldens: max_new, EOS, the callback's
    stop, the context's end; and the think split."""
    got = {n: c["want"] for n, c in CASES.items()}
    assert got["greedy"]["produced"] == CASES["greedy"]["max_new"]
    assert got["eos_first"]["produced"] == 1 and got["eos_first"]["answer"] == []
    assert got["penalty_eos"]["produced"] == len(got["penalty_eos"]["answer"]) + 1
    assert got["stop_after"]["produced"] == CASES["stop_after"]["stop_after"]
    assert got["context_end"]["n_past"] == CASES["context_end"]["n_ctx"]
    # Every marker counts as generated and reaches no callback.
    assert got["think"]["think"] and got["think"]["produced"] >= \
        len(got["think"]["answer"]) + len(got["think"]["think"]) + 2
