"""CPU tests of the oracle's AVX2-order lanes (orc_matvec_avx2, oracle/kernels.c).

The secondary CPU baseline times the f32 lanes an AVX2 + FMA build of ingot
takes: third_party/ingot/src/kernels.c:455-506 (Q4_K, eight FMA lanes over the
unpacked nibbles) and :2062-2081 (qk_dot_avx2, four 8-lane accumulators, the
dot of Q6_K and Q8_0 after the block decode). The restatement is pinned by:
  * golden vectors written by such a build of the reference's own sources
    (tests/golden/avx2.npz, tests/golden/make_golden.py --only avx2, with
    INGOT_SDOT=0 so the Q4_K matvec keeps its f32 lanes), matched bit for bit
    on small shapes and on configs[1]'s whole sweep (SHA-256 of each output);
  * the lanes against float64 (a dropped term or a wrong nibble moves the
    result by far more than the f32 reassociation does);
  * the discrimination of the goldens: the scalar lane's order differs from
    the AVX2 order in the last bits, so matching the goldens says which order
    was restated.
"""
from __future__ import annotations

import hashlib
import os

import numpy as np
import pytest

import configs as CF
import oracle_lib as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
SHAPES = ((CF.Q4_K, 37, 512), (CF.Q4_K, 64, 2048), (CF.Q6_K, 37, 512),
          (CF.Q6_K, 16, 3072), (CF.Q8_0, 37, 96), (CF.Q8_0, 37, 512))


def sha(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def gold():
    return np.load(os.path.join(GOLDEN, "avx2.npz"))


def case(t, rows, cols):
    return O.blocks(t, 1300 + t, rows, cols), O.normal(1400 + t, cols)


@pytest.mark.parametrize("t,rows,cols", SHAPES)
def test_matvec_avx2_golden(gold, t, rows, cols):
    key = f"{CF.TYPE_NAME[t]}_{rows}x{cols}"
    w, x = case(t, rows, cols)
    assert sha(w) == str(gold[f"{key}_w_sha"]) and sha(x) == str(gold[f"{key}_x_sha"])
    y = O.matvec_avx2(t, w, rows, cols, x)
    assert np.array_equal(bits(y), bits(gold[f"{key}_y"]))
    # The threaded form splits rows only: the same bits.
    assert np.array_equal(bits(O.project_avx2(t, w, rows, cols, x)), bits(y))


@pytest.mark.parametrize("t,rows,cols", SHAPES)
def test_matvec_avx2_against_f64(t, rows, cols):
    w, x = case(t, rows, cols)
    y = O.matvec_avx2(t, w, rows, cols, x).astype(np.float64)
    if t == CF.Q8_0:
        # An independent decode (a block: f16 scale, 32 int8 quants); the
        # matrix dequant refuses a ragged row of 96 values.
        blk = np.frombuffer(w.tobytes(), np.uint8).reshape(-1, 34)
        d = blk[:, :2].copy().view(np.float16).astype(np.float64)
        deq = (blk[:, 2:].view(np.int8).astype(np.float64) * d).reshape(rows, cols)
    else:
        deq = O.dequant(t, w, rows, cols).astype(np.float64).reshape(rows, cols)
    want = deq @ x.astype(np.float64)
    scale = np.abs(deq) @ np.abs(x.astype(np.float64))
    assert np.all(np.abs(y - want) <= 1e-5 * scale + 1e-30)


def test_goldens_tell_the_orders_apart(gold):
    differs = 0
    for t, rows, cols in SHAPES:
        w, x = case(t, rows, cols)
        differs += int(not np.array_equal(bits(O.matvec(t, w, rows, cols, x)),
                                          bits(gold[f"{CF.TYPE_NAME[t]}_{rows}x{cols}_y"])))
    assert differs >= 4


@pytest.mark.parametrize("i", range(len(CF.C2)))
def test_c2_sweep_avx2_golden(gold, i):
    m = CF.C2[i]
    ws, xs = CF.matrix_seeds(O.substream, 0, i)
    w, x = O.blocks(m.qtype, ws, m.rows, m.cols), O.normal(xs, m.cols)
    O.orc.orc_threads_init(0)
    y = O.project_avx2(m.qtype, w, m.rows, m.cols, x)
    assert np.array_equal(bits(y[::97]), bits(gold[f"{m.name}_y_every97"]))
    assert sha(y) == str(gold[f"{m.name}_y_sha"])
