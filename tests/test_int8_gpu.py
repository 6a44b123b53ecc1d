"""GPU parity of the int8 activation lane of Q4_K and Q5_K products (int8.hip).

Bar: BIT-IDENTICAL outputs to the oracle's int8 restatement, which is itself
bit-identical to an AVX2 + FMA build of the reference's own sources
(test_int8_oracle.py); the quantiser's int8 values, scales and sums are
compared exactly; the integer dots are read out directly (weights whose one
non-zero scale makes each output one dot) and compared exactly with an
independent numpy unpacking.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

import configs as CF
import oracle_lib as O

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def M():
    import mynah_amd
    mynah_amd.check(mynah_amd.lib.mynah_hip_init(0), "init")
    yield mynah_amd
    mynah_amd.set_int8(mynah_amd.INT8_OFF)


@pytest.fixture(scope="module")
def gold():
    return np.load(os.path.join(GOLDEN, "int8.npz"), allow_pickle=False)


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def say(*a):
    print("[case]", *a, flush=True)


def orc_matmat_int8(w, rows, cols, x, tokens):
    y = np.empty(rows * tokens, np.float32)
    assert O.orc.orc_q4k_matmat_int8(O.ptr(w), rows, cols, O.ptr(x), O.ptr(y), tokens) == 0
    return y


def orc_q5k_matmat_int8(w, rows, cols, x, tokens):
    y = np.empty(rows * tokens, np.float32)
    assert O.orc.orc_q5k_matmat_int8(O.ptr(w), rows, cols, O.ptr(x), O.ptr(y), tokens) == 0
    return y


def orc_matvec_int8(w, rows, cols, x):
    y = np.empty(rows, np.float32)
    assert O.orc.orc_q4k_matvec_int8(O.ptr(w), rows, cols, O.ptr(x), O.ptr(y)) == 0
    return y


# ── quantiser ──────────────────────────────────────────────────────────────

@pytest.mark.parametrize("tokens,cols", [(1, 256), (3, 1024), (17, 3072)])
def test_quantiser_bit_exact(M, tokens, cols):
    say("quantize", tokens, cols)
    x = M.synth_normal(5 + tokens, tokens * cols).reshape(tokens, cols)
    x[0, :256] = 0.0                       # scale 0
    if cols >= 512:
        x[0, 256:512] = np.arange(256, dtype=np.float32) % 254 - 126.5   # ties
        x[0, 256] = 127.0
    nb = cols // 256
    xd = M.DeviceBuffer.from_array(x)
    xq = M.DeviceBuffer(tokens * cols)
    xs = M.DeviceBuffer(tokens * nb * 4)
    xsum = M.DeviceBuffer(tokens * nb * 32)
    M.q8_quantize_dev(xd.ptr, tokens, cols, xq.ptr, xs.ptr, xsum.ptr)
    M.sync()
    q, sc, sums = O.q8_quantize(x)
    np.testing.assert_array_equal(xq.download(np.int8, tokens * cols).reshape(tokens, cols), q)
    np.testing.assert_array_equal(bits(xs.download(np.float32, tokens * nb)), bits(sc.ravel()))
    np.testing.assert_array_equal(xsum.download(np.int32, tokens * nb * 8), sums.ravel())


# ── integer dots, read out directly ────────────────────────────────────────

def dot_readout_weights(M, rows, cols, seed):
    """Q4_K rows whose every super-block has d = 1, dmin = 0 and a single
    non-zero scale (1) at sub-block j = row % 8: the row's output on one
    super-block is then exactly that sub-block's integer dot."""
    w = M.synth_blocks(CF.Q4_K, seed, rows, cols).copy()
    wb = w.view(np.uint8).reshape(rows, cols // 256, 144)
    wb[:, :, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    wb[:, :, 2:4] = 0
    wb[:, :, 4:16] = 0
    for r in range(rows):
        j = r % 8
        wb[r, :, 4 + (j if j < 4 else j + 4)] = 1
    return w


@pytest.mark.parametrize("rows,tokens", [(16, 1), (40, 2), (64, 37), (130, 70)])
def test_integer_dots_exact(M, rows, tokens):
    say("dots", rows, tokens)
    cols = 256
    w = dot_readout_weights(M, rows, cols, 61)
    x = M.synth_normal(62, tokens * cols).reshape(tokens, cols)
    q, sc, sums = O.q8_quantize(x)
    want = O.q4k_int8_dots(w, rows, cols, q)            # [rows][tokens][8]
    expect = np.array([[want[r, t, r % 8] for r in range(rows)] for t in range(tokens)],
                      np.float32)
    wd = M.DeviceBuffer.from_array(w)
    xq = M.DeviceBuffer.from_array(q)
    xs = M.DeviceBuffer.from_array(np.ones(tokens, np.float32))
    xsum = M.DeviceBuffer.from_array(np.zeros((tokens, 8), np.int32))
    y = M.DeviceBuffer(tokens * rows * 4)
    M.q4k_int8_dev(wd.ptr, rows, cols, xq.ptr, xs.ptr, xsum.ptr, y.ptr, tokens)
    M.sync()
    got = y.download(np.float32, tokens * rows).reshape(tokens, rows)
    np.testing.assert_array_equal(got, expect)


# ── golden vectors of the AVX2 reference build ─────────────────────────────

def test_matvec_int8_golden(M, gold):
    for rows, cols in ((37, 512), (64, 3072)):
        say("golden matvec", rows, cols)
        w, x = M.synth_blocks(CF.Q4_K, 500 + rows, rows, cols), M.synth_normal(600 + rows, cols)
        np.testing.assert_array_equal(bits(M.matvec_int8(w, rows, cols, x)),
                                      bits(gold[f"mv_{rows}x{cols}_y"]))
    w = M.synth_blocks(CF.Q4_K, 700, 16, 768)
    np.testing.assert_array_equal(bits(M.matvec_int8(w, 16, 768, gold["mv_special_x"])),
                                  bits(gold["mv_special_y"]))


@pytest.mark.parametrize("rows,cols,tokens", [(16, 2048, 16), (24, 2048, 70), (9, 512, 130),
                                              (8, 6144, 5), (4, 9728, 110), (5, 512, 2),
                                              (3, 256, 3), (6, 1024, 1)])
def test_matmat_int8_golden(M, gold, rows, cols, tokens):
    say("golden matmat", rows, cols, tokens)
    M.set_int8(M.INT8_ALL)
    try:
        w = M.synth_blocks(CF.Q4_K, 800 + rows, rows, cols)
        x = M.synth_normal(900 + tokens, tokens * cols)
        got = M.matmat(CF.Q4_K, w, rows, cols, x, tokens)
    finally:
        M.set_int8(M.INT8_OFF)
    np.testing.assert_array_equal(bits(got), bits(gold[f"mm_{rows}x{cols}_t{tokens}_y"]))


@pytest.mark.parametrize("rows,cols,tokens", [(40, 2048, 70), (9, 512, 130), (24, 1024, 5),
                                              (3, 256, 2)])
def test_q5k_matmat_int8_golden(M, gold, rows, cols, tokens):
    say("golden q5k matmat", rows, cols, tokens)
    w = M.synth_blocks(CF.Q5_K, 1100 + rows, rows, cols)
    x = M.synth_normal(1200 + tokens, tokens * cols)
    M.set_int8(M.INT8_BATCHED)
    try:
        got = M.matmat(CF.Q5_K, w, rows, cols, x, tokens)
    finally:
        M.set_int8(M.INT8_OFF)
    np.testing.assert_array_equal(bits(got), bits(gold[f"q5k_mm_{rows}x{cols}_t{tokens}_y"]))


# ── larger shapes against the oracle ───────────────────────────────────────

@pytest.mark.parametrize("rows,cols", [(1024, 3072), (333, 1024), (2560, 9728), (9728, 2560)])
def test_matvec_int8_against_oracle(M, rows, cols):
    say("matvec int8", rows, cols)
    w, x = M.synth_blocks(CF.Q4_K, 71, rows, cols), M.synth_normal(72, cols)
    np.testing.assert_array_equal(bits(M.matvec_int8(w, rows, cols, x)),
                                  bits(orc_matvec_int8(w, rows, cols, x)))


@pytest.mark.parametrize("rows,cols,tokens", [(100, 2048, 70), (64, 16384, 66), (2048, 2048, 512),
                                              (6144, 2048, 128), (77, 9728, 213)])
def test_matmat_int8_against_oracle(M, rows, cols, tokens):
    say("matmat int8", rows, cols, tokens)
    w, x = M.synth_blocks(CF.Q4_K, 73, rows, cols), M.synth_normal(74, tokens * cols)
    M.set_int8(M.INT8_BATCHED)
    try:
        got = M.matmat(CF.Q4_K, w, rows, cols, x, tokens)
    finally:
        M.set_int8(M.INT8_OFF)
    np.testing.assert_array_equal(bits(got), bits(orc_matmat_int8(w, rows, cols, x, tokens)))


@pytest.mark.parametrize("i", [i for i, m in enumerate(CF.C4) if m.qtype == CF.Q4_K])
def test_matmat_int8_configs3_against_oracle(M, i):
    """The five Q4_K products of configs[3] at 512 tokens, on the inputs
    bench.py times (weights and activations from the config's seeds)."""
    m = CF.C4[i]
    say("matmat int8 configs[3]", m.rows, m.cols, CF.C4_TOKENS)
    wseed, _ = CF.matrix_seeds(M.substream, 0, i)
    w = M.synth_blocks(m.qtype, wseed, m.rows, m.cols)
    x = M.synth_normal(M.substream(0, CF.PREFILL_X_INDEX + i), CF.C4_TOKENS * m.cols)
    M.set_int8(M.INT8_BATCHED)
    try:
        got = M.matmat(CF.Q4_K, w, m.rows, m.cols, x, CF.C4_TOKENS)
    finally:
        M.set_int8(M.INT8_OFF)
    np.testing.assert_array_equal(bits(got),
                                  bits(orc_matmat_int8(w, m.rows, m.cols, x, CF.C4_TOKENS)))


@pytest.mark.parametrize("rows,cols,tokens", [(100, 2048, 70), (2048, 2048, 512), (77, 9728, 213),
                                              (1027, 4096, 33)])
def test_q5k_matmat_int8_against_oracle(M, rows, cols, tokens):
    say("q5k matmat int8", rows, cols, tokens)
    w, x = M.synth_blocks(CF.Q5_K, 77, rows, cols), M.synth_normal(78, tokens * cols)
    M.set_int8(M.INT8_BATCHED)
    try:
        got = M.matmat(CF.Q5_K, w, rows, cols, x, tokens)
    finally:
        M.set_int8(M.INT8_OFF)
    np.testing.assert_array_equal(bits(got), bits(orc_q5k_matmat_int8(w, rows, cols, x, tokens)))


def test_q5k_lane_modes(M):
    """Q5_K: the batched product follows the lane; the matvec, the one-token
    product and the explicit exact entry stay exact in every mode."""
    rows, cols, tokens = 48, 1024, 9
    say("q5k modes", rows, cols, tokens)
    w, x = M.synth_blocks(CF.Q5_K, 85, rows, cols), M.synth_normal(86, tokens * cols)
    exact = np.empty(rows * tokens, np.float32)
    assert O.orc.orc_matmat(CF.Q5_K, O.ptr(w), rows, cols, O.ptr(x), O.ptr(exact), tokens) == 0
    exact_mv = np.empty(rows, np.float32)
    assert O.orc.orc_matvec(CF.Q5_K, O.ptr(w), rows, cols, O.ptr(x), O.ptr(exact_mv)) == 0
    int8 = orc_q5k_matmat_int8(w, rows, cols, x, tokens)
    assert not np.array_equal(bits(int8), bits(exact))
    y = np.empty(rows * tokens, np.float32)
    try:
        for mode in (M.INT8_OFF, M.INT8_BATCHED, M.INT8_ALL):
            M.set_int8(mode)
            want = exact if mode == M.INT8_OFF else int8
            assert np.array_equal(bits(M.matmat(CF.Q5_K, w, rows, cols, x, tokens)), bits(want))
            assert np.array_equal(bits(M.matvec(CF.Q5_K, w, rows, cols, x)), bits(exact_mv))
            assert np.array_equal(bits(M.matmat(CF.Q5_K, w, rows, cols, x, 1)), bits(exact_mv))
            M.check(M.lib.ingot_q5_k_matmat_exact(M.ptr(w), rows, cols, M.ptr(x), M.ptr(y),
                                                  tokens), "q5_k_matmat_exact")
            assert np.array_equal(bits(y), bits(exact))
    finally:
        M.set_int8(M.INT8_OFF)


def test_device_twin_int8(M):
    rows, cols, tokens = 256, 2048, 96
    say("device twin", rows, cols, tokens)
    w, x = M.synth_blocks(CF.Q4_K, 75, rows, cols), M.synth_normal(76, tokens * cols)
    wd, xd = M.DeviceBuffer.from_array(w), M.DeviceBuffer.from_array(x)
    yd = M.DeviceBuffer(rows * tokens * 4)
    M.set_int8(M.INT8_BATCHED)
    try:
        M.matmat_dev(CF.Q4_K, wd.ptr, rows, cols, xd.ptr, yd.ptr, tokens)
        M.sync()
    finally:
        M.set_int8(M.INT8_OFF)
    np.testing.assert_array_equal(bits(yd.download(np.float32, rows * tokens)),
                                  bits(orc_matmat_int8(w, rows, cols, x, tokens)))


# ── the lane switch ────────────────────────────────────────────────────────

def test_modes_and_exact_paths(M):
    rows, cols, tokens = 48, 1024, 9
    w, x = M.synth_blocks(CF.Q4_K, 81, rows, cols), M.synth_normal(82, tokens * cols)
    exact = np.empty(rows * tokens, np.float32)
    assert O.orc.orc_matmat(CF.Q4_K, O.ptr(w), rows, cols, O.ptr(x), O.ptr(exact), tokens) == 0
    exact_mv = np.empty(rows, np.float32)
    assert O.orc.orc_matvec(CF.Q4_K, O.ptr(w), rows, cols, O.ptr(x), O.ptr(exact_mv)) == 0
    int8 = orc_matmat_int8(w, rows, cols, x, tokens)
    int8_mv = orc_matvec_int8(w, rows, cols, x)
    w6 = M.synth_blocks(CF.Q6_K, 83, rows, cols)
    exact6 = np.empty(rows * tokens, np.float32)
    assert O.orc.orc_matmat(CF.Q6_K, O.ptr(w6), rows, cols, O.ptr(x), O.ptr(exact6), tokens) == 0
    try:
        M.set_int8(M.INT8_OFF)
        assert M.lib.ingot_matmat_is_exact(1) == 1 and M.lib.ingot_matmat_is_exact(2) == 1
        assert np.array_equal(bits(M.matmat(CF.Q4_K, w, rows, cols, x, tokens)), bits(exact))
        assert np.array_equal(bits(M.matvec(CF.Q4_K, w, rows, cols, x)), bits(exact_mv))
        # The explicit int8 matvec is int8 whatever the mode.
        assert np.array_equal(bits(M.matvec_int8(w, rows, cols, x)), bits(int8_mv))

        M.set_int8(M.INT8_BATCHED)
        assert M.lib.ingot_matmat_is_exact(1) == 1 and M.lib.ingot_matmat_is_exact(2) == 0
        assert np.array_equal(bits(M.matmat(CF.Q4_K, w, rows, cols, x, tokens)), bits(int8))
        assert np.array_equal(bits(M.matvec(CF.Q4_K, w, rows, cols, x)), bits(exact_mv))
        assert np.array_equal(bits(M.matmat_exact(w, rows, cols, x, tokens)), bits(exact))
        assert np.array_equal(bits(M.matmat(CF.Q6_K, w6, rows, cols, x, tokens)), bits(exact6))

        M.set_int8(M.INT8_ALL)
        assert M.lib.ingot_matmat_is_exact(1) == 1 and M.lib.ingot_matmat_is_exact(2) == 0
        assert np.array_equal(bits(M.matvec(CF.Q4_K, w, rows, cols, x)), bits(int8_mv))
        assert np.array_equal(bits(M.matmat(CF.Q4_K, w, rows, cols, x, 1)), bits(int8_mv))
        assert np.array_equal(bits(M.matmat_exact(w, rows, cols, x, tokens)), bits(exact))
        assert M.lib.mynah_hip_set_int8(7) == -1
    finally:
        M.set_int8(M.INT8_OFF)


def test_int8_argument_guards(M):
    w, x = M.synth_blocks(CF.Q4_K, 1, 4, 512), M.synth_normal(1, 1024)
    y = np.empty(8, np.float32)
    assert M.lib.ingot_q4_k_matvec_int8(None, 4, 512, M.ptr(x), M.ptr(y)) == -1
    assert M.lib.ingot_q4_k_matvec_int8(M.ptr(w), 0, 512, M.ptr(x), M.ptr(y)) == -1
    assert M.lib.ingot_q4_k_matvec_int8(M.ptr(w), 4, 500, M.ptr(x), M.ptr(y)) == -1
    assert M.lib.mynah_hip_q8_quantize_dev(None, 1, 256, None, None, None, None) == -1
