"""The oracle's Q5_K and Q4_0 (oracle/kernels.c), pinned on the CPU.

  * ingot's own llama.cpp-derived fixtures for both formats (copied as data
    into tests/golden/ingot_fixtures) and its geometry table;
  * golden vectors of the COMPILED reference (tests/golden/adjacent.npz:
    matvec, batched products and dequant of configs.ADJACENT), bit for bit;
  * an independent numpy restatement of each format (decoded from the byte
    layout) and of each summation order (f32 numpy operations, one rounding
    each), so a swapped nibble, a wrong fifth-bit index or a reordered sum in
    the C restatement fails here even without the golden file;
  * the f64 closed form of every matvec with the recursive-summation bound.
"""
from __future__ import annotations

import hashlib
import os

import numpy as np
import pytest

import configs as CF
import oracle_lib as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FIX = os.path.join(GOLDEN, "ingot_fixtures")


def sha(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


# ── the formats, restated in numpy from the byte layout ───────────────────

def f16(b):
    return b.copy().view(np.float16).astype(np.float32)


def k_scales(sc):
    """The eight 6-bit (scale, min) pairs of a Q4_K / Q5_K scale field
    (ggml get_scale_min_k4), for blocks along axis 0; shape (n, 8) each."""
    sc = sc.astype(np.uint32)
    s = np.empty((sc.shape[0], 8), np.uint32)
    m = np.empty_like(s)
    for j in range(8):
        if j < 4:
            s[:, j] = sc[:, j] & 63
            m[:, j] = sc[:, j + 4] & 63
        else:
            s[:, j] = (sc[:, j + 4] & 15) | ((sc[:, j - 4] >> 6) << 4)
            m[:, j] = (sc[:, j + 4] >> 4) | ((sc[:, j] >> 6) << 4)
    return s.astype(np.float32), m.astype(np.float32)


def np_q5k(w, rows, cols):
    """(rows, cols) f32 weights: block = d, dmin, scales[12], qh[32], qs[128];
    value 64g + i = (d*sc[2g])*(lo_i + 16*bit_2g(qh[i])) - dmin*m[2g],
    value 64g + 32 + i likewise with the high nibble and bit 2g + 1."""
    blk = w.reshape(-1, 176)
    d, dmin = f16(blk[:, 0:2])[:, 0], f16(blk[:, 2:4])[:, 0]
    s, m = k_scales(blk[:, 4:16])
    qh, qs = blk[:, 16:48].astype(np.uint32), blk[:, 48:176].astype(np.uint32)
    out = np.empty((blk.shape[0], 256), np.float32)
    for g in range(4):
        q = qs[:, 32 * g:32 * g + 32]
        lo = (q & 15) + (((qh >> (2 * g)) & 1) << 4)
        hi = (q >> 4) + (((qh >> (2 * g + 1)) & 1) << 4)
        for half, v in ((0, lo), (1, hi)):
            j = 2 * g + half
            dd = (d * s[:, j])[:, None]
            mm = (dmin * m[:, j])[:, None]
            out[:, 64 * g + 32 * half:64 * g + 32 * half + 32] = dd * v.astype(np.float32) - mm
    return out.reshape(rows, cols)


def np_q40(w, rows, cols):
    """(rows, cols) f32 weights: block = d, qs[16]; value i = d*((qs[i] & 15) - 8),
    value 16 + i = d*((qs[i] >> 4) - 8)."""
    blk = w.reshape(-1, 18)
    d = f16(blk[:, 0:2])[:, 0][:, None]
    q = blk[:, 2:18].astype(np.int32)
    out = np.concatenate([d * ((q & 15) - 8).astype(np.float32),
                          d * ((q >> 4) - 8).astype(np.float32)], axis=1)
    return out.reshape(rows, cols)


def np_decode(t, w, rows, cols):
    return np_q5k(w, rows, cols) if t == CF.Q5_K else np_q40(w, rows, cols)


def np_matvec(t, w, rows, cols, x):
    """The reference's matvec order in f32 numpy steps: Q5_K per super-block
    the low then the high weight of each i of each group, the block sum added
    to the row; Q4_0 one running sum over the row."""
    wf = np_decode(t, w, rows, cols)
    x = x[:cols].astype(np.float32)
    total = np.zeros(rows, np.float32)
    if t == CF.Q4_0:
        for i in range(cols):
            total = total + wf[:, i] * x[i]
        return total
    for b in range(cols // 256):
        acc = np.zeros(rows, np.float32)
        for g in range(4):
            for i in range(32):
                a, c = 256 * b + 64 * g + i, 256 * b + 64 * g + 32 + i
                acc = acc + wf[:, a] * x[a]
                acc = acc + wf[:, c] * x[c]
        total = total + acc
    return total


def np_matmat_q5k(w, rows, cols, x, tokens):
    """The batched core's order: per super-block a natural-order sum from 0,
    added to the (row, token) accumulator."""
    wf = np_q5k(w, rows, cols)
    out = np.empty((tokens, rows), np.float32)
    for t in range(tokens):
        xt = x[t * cols:(t + 1) * cols]
        total = np.zeros(rows, np.float32)
        for b in range(cols // 256):
            acc = np.zeros(rows, np.float32)
            for i in range(256 * b, 256 * b + 256):
                acc = acc + wf[:, i] * xt[i]
            total = total + acc
        out[t] = total
    return out.reshape(-1)


# ── fixtures and geometry ────────────────────────────────────────────────

def test_geometry_matches_ggml_table():
    table = {}
    for line in open(os.path.join(FIX, "geometry.txt")):
        name, tid, elems, nbytes = line.split()
        table[name] = (int(tid), int(elems), int(nbytes))
    for name, t in (("Q5_K", 13), ("Q4_0", 2)):
        assert table[name][0] == t
        assert O.BLOCK[t] == (table[name][1], table[name][2])


@pytest.mark.parametrize("name,qtype", [("Q5_K", 13), ("Q4_0", 2)])
def test_dequant_matches_llama_cpp_fixture(name, qtype):
    raw = np.fromfile(os.path.join(FIX, f"{name}.bin"), dtype=np.uint8)
    ref = np.fromfile(os.path.join(FIX, f"{name}.ref"), dtype=np.float32)
    elems, nbytes = O.BLOCK[qtype]
    values = raw.size // nbytes * elems
    rows, cols = values // 256, 256
    got = O.dequant(qtype, raw, rows, cols)
    assert np.array_equal(bits(got), bits(ref)), f"{name}: decode differs from llama.cpp"
    assert np.array_equal(bits(np_decode(qtype, raw, rows, cols).reshape(-1)), bits(ref))


# ── golden vectors of the compiled reference ─────────────────────────────

@pytest.mark.parametrize("case", CF.ADJACENT, ids=lambda c: f"{CF.TYPE_NAME[c[0]]}_{c[1]}x{c[2]}")
def test_adjacent_golden(case):
    t, rows, cols, token_counts = case
    g = np.load(os.path.join(GOLDEN, "adjacent.npz"), allow_pickle=False)
    key = f"{CF.TYPE_NAME[t]}_{rows}x{cols}"
    w = O.blocks(t, 1000 + t + rows, rows, cols)
    x = O.normal(2000 + t + rows, max(token_counts) * cols)
    assert sha(w) == str(g[f"{key}_w_sha"]) and sha(x) == str(g[f"{key}_x_sha"])
    assert np.array_equal(bits(O.matvec(t, w, rows, cols, x)), bits(g[f"{key}_matvec"]))
    assert np.array_equal(bits(O.dequant(t, w, rows, cols)), bits(g[f"{key}_dequant"]))
    for n in token_counts:
        assert np.array_equal(bits(O.matmat(t, w, rows, cols, x, n)), bits(g[f"{key}_matmat{n}"]))
        assert np.array_equal(bits(O.matmat(t, w, rows, cols, x, n, threaded=True)),
                              bits(g[f"{key}_matmat{n}"]))


# ── independent restatement of the orders ────────────────────────────────

@pytest.mark.parametrize("qtype,rows,cols", [(13, 64, 512), (2, 64, 256), (2, 16, 96)])
def test_matvec_order_restated_in_numpy(qtype, rows, cols):
    w, x = O.blocks(qtype, 31, rows, cols), O.normal(32, cols)
    assert np.array_equal(bits(O.dequant(qtype, w, rows, cols)),
                          bits(np_decode(qtype, w, rows, cols).reshape(-1)))
    assert np.array_equal(bits(O.matvec(qtype, w, rows, cols, x)),
                          bits(np_matvec(qtype, w, rows, cols, x)))


def test_q5k_batched_order_restated_in_numpy():
    rows, cols, tokens = 24, 512, 3
    w, x = O.blocks(13, 33, rows, cols), O.normal(34, tokens * cols)
    got = O.matmat(13, w, rows, cols, x, tokens)
    assert np.array_equal(bits(got), bits(np_matmat_q5k(w, rows, cols, x, tokens)))
    # ...which is not the matvec's order: the two differ in the last bits.
    assert not np.array_equal(bits(got[:rows]), bits(O.matvec(13, w, rows, cols, x)))


def test_q40_batched_is_the_matvec_chain_per_token():
    rows, cols, tokens = 40, 2080, 4
    w, x = O.blocks(2, 35, rows, cols), O.normal(36, tokens * cols)
    got = O.matmat(2, w, rows, cols, x, tokens).reshape(tokens, rows)
    for t in range(tokens):
        assert np.array_equal(bits(got[t]), bits(O.matvec(2, w, rows, cols, x[t * cols:])))


@pytest.mark.parametrize("qtype,cols", [(13, 1024), (2, 1024), (2, 96)])
def test_matvec_equals_f64_dot_of_dequant(qtype, cols):
    rows = 64
    w, x = O.blocks(qtype, 37, rows, cols), O.normal(38, cols)
    y = O.matvec(qtype, w, rows, cols, x)
    dq = np_decode(qtype, w, rows, cols).astype(np.float64)
    ref = dq @ x.astype(np.float64)
    mag = np.abs(dq) @ np.abs(x.astype(np.float64))
    assert (np.abs(y - ref) <= (cols + 1) * 2.0 ** -24 * mag).all()


def test_argument_guards():
    x = O.normal(2, 512)
    y = np.empty(4 * 512, np.float32)
    w5 = O.blocks(13, 1, 2, 512)
    w4 = O.blocks(2, 1, 2, 96)
    assert O.orc.orc_matvec(13, O.ptr(w5), 2, 300, O.ptr(x), O.ptr(y)) == -1   # partial block
    assert O.orc.orc_matvec(2, O.ptr(w4), 2, 100, O.ptr(x), O.ptr(y)) == -1
    assert O.orc.orc_matmat(13, O.ptr(w5), 2, 0, O.ptr(x), O.ptr(y), 2) == -1
    # Q4_0's batched product and dequant take any multiple of 32.
    assert O.orc.orc_matmat(2, O.ptr(w4), 2, 96, O.ptr(x), O.ptr(y), 2) == 0
    assert O.orc.orc_dequant_matrix(2, O.ptr(w4), 2, 96, O.ptr(y)) == 0
