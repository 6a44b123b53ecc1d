"""CPU tests of the oracle's int8 activation lane (oracle/int8.c).

The reference's int8 lane (third_party/ingot/src/kernels.c:636-788 for the
Q4_K matvec, 1120-1751 for the batched form, which Q5_K also takes through
kernels.c:2573-2595) exists only in an AVX2 + FMA build of ingot. The restatement is pinned by:
  * golden vectors written by such a build of the reference's own sources
    (tests/golden/int8.npz, tests/golden/make_golden.py --only int8), matched
    bit for bit, including round-half-even ties, an all-zero block and token
    counts on both sides of the token tile and its groups of four;
  * the quantiser against numpy's float32 arithmetic (np.rint is
    round-half-even) and its invariants (|q| <= 127, the sums);
  * the integer dots against an independent numpy unpacking of the nibbles;
  * the f32 epilogue against the same expression in float64 (a dropped or
    sign-flipped term moves the result by far more than f32 rounding);
  * the compiled AVX2 reference directly, when it was built on this machine.
"""
from __future__ import annotations

import hashlib
import os

import numpy as np
import pytest

import configs as CF
import oracle_lib as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def sha(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def gold():
    return np.load(os.path.join(GOLDEN, "int8.npz"), allow_pickle=False)


def orc_matvec_int8(w, rows, cols, x):
    y = np.empty(rows, np.float32)
    assert O.orc.orc_q4k_matvec_int8(O.ptr(w), rows, cols, O.ptr(x), O.ptr(y)) == 0
    return y


def orc_matmat_int8(w, rows, cols, x, tokens):
    y = np.empty(rows * tokens, np.float32)
    assert O.orc.orc_q4k_matmat_int8(O.ptr(w), rows, cols, O.ptr(x), O.ptr(y), tokens) == 0
    return y


def orc_q5k_matmat_int8(w, rows, cols, x, tokens):
    y = np.empty(rows * tokens, np.float32)
    assert O.orc.orc_q5k_matmat_int8(O.ptr(w), rows, cols, O.ptr(x), O.ptr(y), tokens) == 0
    return y


# ── golden vectors of the AVX2 reference build ─────────────────────────────

@pytest.mark.parametrize("rows,cols", [(37, 512), (64, 3072)])
def test_matvec_int8_golden(gold, rows, cols):
    w, x = O.blocks(CF.Q4_K, 500 + rows, rows, cols), O.normal(600 + rows, cols)
    assert sha(w) == str(gold[f"mv_{rows}x{cols}_w_sha"])
    assert sha(x) == str(gold[f"mv_{rows}x{cols}_x_sha"])
    np.testing.assert_array_equal(bits(orc_matvec_int8(w, rows, cols, x)),
                                  bits(gold[f"mv_{rows}x{cols}_y"]))


def test_matvec_int8_special_blocks_golden(gold):
    w, x = O.blocks(CF.Q4_K, 700, 16, 768), gold["mv_special_x"]
    np.testing.assert_array_equal(bits(orc_matvec_int8(w, 16, 768, x)),
                                  bits(gold["mv_special_y"]))


@pytest.mark.parametrize("rows,cols,tokens", [(16, 2048, 16), (24, 2048, 70), (9, 512, 130),
                                              (8, 6144, 5), (4, 9728, 110), (5, 512, 2),
                                              (3, 256, 3), (6, 1024, 1)])
def test_matmat_int8_golden(gold, rows, cols, tokens):
    key = f"mm_{rows}x{cols}_t{tokens}"
    w, x = O.blocks(CF.Q4_K, 800 + rows, rows, cols), O.normal(900 + tokens, tokens * cols)
    assert sha(w) == str(gold[f"{key}_w_sha"])
    assert sha(x) == str(gold[f"{key}_x_sha"])
    np.testing.assert_array_equal(bits(orc_matmat_int8(w, rows, cols, x, tokens)),
                                  bits(gold[f"{key}_y"]))


@pytest.mark.parametrize("rows,cols,tokens", [(40, 2048, 70), (9, 512, 130), (24, 1024, 5),
                                              (3, 256, 2)])
def test_q5k_matmat_int8_golden(gold, rows, cols, tokens):
    key = f"q5k_mm_{rows}x{cols}_t{tokens}"
    w, x = O.blocks(CF.Q5_K, 1100 + rows, rows, cols), O.normal(1200 + tokens, tokens * cols)
    assert sha(w) == str(gold[f"{key}_w_sha"])
    assert sha(x) == str(gold[f"{key}_x_sha"])
    got = orc_q5k_matmat_int8(w, rows, cols, x, tokens)
    np.testing.assert_array_equal(bits(got), bits(gold[f"{key}_y"]))
    # The lane is not the exact product: a restatement that fell back to the
    # exact order would still match nothing above but must not pass here.
    assert not np.array_equal(bits(got), bits(O.matmat(CF.Q5_K, w, rows, cols, x, tokens)))


# ── the quantiser ──────────────────────────────────────────────────────────

def test_quantiser_against_numpy_float32():
    x = np.concatenate([O.normal(1, 256 * 6), np.zeros(256, np.float32),
                        O.normal(2, 256) * np.float32(1e-30)]).reshape(1, -1)
    q, sc, sums = O.q8_quantize(x)
    for b in range(x.shape[1] // 256):
        blk = x[0, 256 * b:256 * b + 256]
        amax = np.float32(np.abs(blk).max())
        if amax == 0:
            assert sc[0, b] == 0 and not q[0, 256 * b:256 * b + 256].any()
            assert not sums[0, 8 * b:8 * b + 8].any()
            continue
        assert sc[0, b] == np.float32(amax / np.float32(127))
        r = np.rint(blk * (np.float32(127) / amax)).astype(np.int32)
        assert np.abs(r).max() == 127
        np.testing.assert_array_equal(q[0, 256 * b:256 * b + 256], r.astype(np.int8))
        np.testing.assert_array_equal(sums[0, 8 * b:8 * b + 8], r.reshape(8, 32).sum(axis=1))


def test_quantiser_ties_to_even():
    x = np.zeros(256, np.float32)
    x[0] = 127.0
    x[1:9] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -126.5]
    q, sc, _ = O.q8_quantize(x.reshape(1, -1))
    assert sc[0, 0] == 1.0
    assert list(q[0, :9]) == [127, 0, 2, 2, 0, -2, -2, 126, -126]


# ── integer dots and the epilogue ──────────────────────────────────────────

def test_int8_dots_against_numpy_unpacking():
    rows, cols = 5, 768
    w, x = O.blocks(CF.Q4_K, 31, rows, cols), O.normal(32, cols)
    q, _, _ = O.q8_quantize(x.reshape(1, -1))
    dots = O.q4k_int8_dots(w, rows, cols, q)
    wb = w.view(np.uint8).reshape(rows, cols // 256, 144)
    for r in range(rows):
        for b in range(cols // 256):
            for j in range(8):
                d = O.orc.orc_q4k_int8_dot(wb[r, b].ctypes.data, q[0, 256 * b:].ctypes.data, j)
                assert d == dots[r, 0, 8 * b + j]


def _epilogue_f64(w, rows, cols, x):
    """Σ_b xscale_b Σ_j (d·sc_j·dot_j − dmin·m_j·sum_j), in float64."""
    q, sc, sums = O.q8_quantize(x.reshape(1, -1))
    dots = O.q4k_int8_dots(w, rows, cols, q)[:, 0, :]
    nb = cols // 256
    wb = w.view(np.uint8).reshape(rows, nb, 144)
    d = wb[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float64)
    dmin = wb[:, :, 2:4].copy().view(np.float16)[..., 0].astype(np.float64)
    s12 = wb[:, :, 4:16].astype(np.int64)
    scl = np.empty((rows, nb, 8)); mn = np.empty((rows, nb, 8))
    for j in range(8):
        if j < 4:
            scl[..., j] = s12[..., j] & 63
            mn[..., j] = s12[..., j + 4] & 63
        else:
            scl[..., j] = (s12[..., j + 4] & 15) | ((s12[..., j - 4] >> 6) << 4)
            mn[..., j] = (s12[..., j + 4] >> 4) | ((s12[..., j] >> 6) << 4)
    per = (d[..., None] * scl * dots.reshape(rows, nb, 8)
           - dmin[..., None] * mn * sums[0].reshape(nb, 8)[None].astype(np.float64))
    return (per.sum(axis=2) * sc[0][None].astype(np.float64)).sum(axis=1)


@pytest.mark.parametrize("rows,cols", [(32, 1024), (8, 4096)])
def test_matvec_int8_epilogue_f64(rows, cols):
    w, x = O.blocks(CF.Q4_K, 41, rows, cols), O.normal(42, cols)
    y = orc_matvec_int8(w, rows, cols, x).astype(np.float64)
    want = _epilogue_f64(w, rows, cols, x)
    scale = np.maximum(1.0, np.abs(want))
    assert (np.abs(y - want) / scale).max() < 2e-5


def test_matmat_int8_columns_equal_f64_epilogue():
    rows, cols, tokens = 8, 1024, 6
    w, x = O.blocks(CF.Q4_K, 43, rows, cols), O.normal(44, tokens * cols)
    y = orc_matmat_int8(w, rows, cols, x, tokens).reshape(tokens, rows).astype(np.float64)
    for t in range(tokens):
        want = _epilogue_f64(w, rows, cols, x[t * cols:(t + 1) * cols])
        assert (np.abs(y[t] - want) / np.maximum(1.0, np.abs(want))).max() < 2e-5


def _q5k_sub_quants(w, rows, cols):
    """Q5_K quants 0..31 by an independent numpy unpacking: sub-block j of a
    super-block takes nibble (j & 1) of qs bytes 32*(j//2) .. +32 and bit j of
    the 32 qh bytes as its fifth bit."""
    wb = w.view(np.uint8).reshape(rows, cols // 256, 176)
    qh, qs = wb[:, :, 16:48], wb[:, :, 48:176]
    out = np.empty((rows, cols // 256, 8, 32), np.int64)
    for j in range(8):
        nib = qs[:, :, 32 * (j // 2):32 * (j // 2) + 32]
        nib = (nib >> 4) if j & 1 else (nib & 15)
        out[:, :, j] = nib.astype(np.int64) + (((qh >> j) & 1).astype(np.int64) << 4)
    return out


def test_q5k_int8_dots_against_numpy_unpacking():
    rows, cols = 4, 768
    w, x = O.blocks(CF.Q5_K, 33, rows, cols), O.normal(34, cols)
    q, _, _ = O.q8_quantize(x.reshape(1, -1))
    quants = _q5k_sub_quants(w, rows, cols)
    wb = w.view(np.uint8).reshape(rows, cols // 256, 176)
    for r in range(rows):
        for b in range(cols // 256):
            for j in range(8):
                want = int((quants[r, b, j] * q[0, 256 * b + 32 * j:256 * b + 32 * j + 32]
                            .astype(np.int64)).sum())
                assert O.orc.orc_q5k_int8_dot(wb[r, b].ctypes.data,
                                              q[0, 256 * b:].ctypes.data, j) == want


def test_int8_near_exact_matvec():
    """Quantising the activations costs ~1e-3 relative, not more."""
    rows, cols = 64, 2048
    w, x = O.blocks(CF.Q4_K, 45, rows, cols), O.normal(46, cols)
    y8 = orc_matvec_int8(w, rows, cols, x)
    y = np.empty(rows, np.float32)
    assert O.orc.orc_matvec(CF.Q4_K, O.ptr(w), rows, cols, O.ptr(x), O.ptr(y)) == 0
    rel = np.abs(y8 - y).max() / np.abs(y).max()
    assert 1e-6 < rel < 2e-2


def test_int8_guards():
    w, x = O.blocks(CF.Q4_K, 1, 2, 256), O.normal(1, 512)
    y = np.empty(4, np.float32)
    assert O.orc.orc_q4k_matvec_int8(O.ptr(w), 2, 255, O.ptr(x), O.ptr(y)) == -1
    assert O.orc.orc_q4k_matvec_int8(O.ptr(w), 0, 256, O.ptr(x), O.ptr(y)) == -1
    assert O.orc.orc_q4k_matmat_int8(O.ptr(w), 2, 256, O.ptr(x), O.ptr(y), 0) == -1
    assert O.orc.orc_q5k_matmat_int8(O.ptr(w), 2, 255, O.ptr(x), O.ptr(y), 2) == -1


# ── the compiled AVX2 reference, where it was built ────────────────────────

@pytest.mark.parametrize("rows,cols,tokens", [(7, 1536, 1), (7, 1536, 4), (11, 768, 37),
                                              (3, 16384, 66)])
def test_int8_against_compiled_reference(rows, cols, tokens):
    ref8 = O.load_ref_int8()
    if ref8 is None:
        pytest.skip("oracle/_ref/libref_int8.so not built (needs /root/reference)")
    w, x = O.blocks(CF.Q4_K, 51, rows, cols), O.normal(52, tokens * cols)
    y = np.empty(rows * tokens, np.float32)
    assert ref8.ingot_q4_k_matmat(O.ptr(w), rows, cols, O.ptr(x), O.ptr(y), tokens) == 0
    np.testing.assert_array_equal(bits(orc_matmat_int8(w, rows, cols, x, tokens)), bits(y))


@pytest.mark.parametrize("rows,cols,tokens", [(5, 1536, 4), (11, 768, 37), (2, 4096, 66)])
def test_q5k_int8_against_compiled_reference(rows, cols, tokens):
    ref8 = O.load_ref_int8()
    if ref8 is None:
        pytest.skip("oracle/_ref/libref_int8.so not built (needs /root/reference)")
    w, x = O.blocks(CF.Q5_K, 53, rows, cols), O.normal(54, tokens * cols)
    y = np.empty(rows * tokens, np.float32)
    assert ref8.ingot_q5_k_matmat(O.ptr(w), rows, cols, O.ptr(x), O.ptr(y), tokens) == 0
    np.testing.assert_array_equal(bits(orc_q5k_matmat_int8(w, rows, cols, x, tokens)), bits(y))
