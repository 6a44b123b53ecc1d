"""CPU tests of the oracle (the C11 restatement under oracle/).

The restatement is pinned by:
  * the reference's own llama.cpp-derived fixtures (ingot tests/fixtures,
    copied as data into tests/golden/ingot_fixtures) and its geometry table;
  * golden vectors written by the COMPILED reference (tests/golden/*.npz, see
    tests/golden/make_golden.py) — matched bit for bit;
  * closed forms: matvec against an f64 dot of the decoded weights; a
    hand-packed Q4_K / Q6_K block with known values; f16 conversion against
    numpy; threading invariance.
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


def golden(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


@pytest.fixture(scope="module", autouse=True)
def threads():
    O.orc.orc_threads_init(0)
    yield


# ── formats ────────────────────────────────────────────────────────────────

def test_geometry_matches_ggml_table():
    table = {}
    for line in open(os.path.join(FIX, "geometry.txt")):
        name, tid, elems, nbytes = line.split()
        table[name] = (int(tid), int(elems), int(nbytes))
    for name, t in (("Q4_K", 12), ("Q6_K", 14), ("Q8_0", 8)):
        assert table[name][0] == t
        assert O.BLOCK[t] == (table[name][1], table[name][2])


@pytest.mark.parametrize("name,qtype", [("Q4_K", 12), ("Q6_K", 14), ("Q8_0", 8)])
def test_dequant_matches_llama_cpp_fixture(name, qtype):
    raw = np.fromfile(os.path.join(FIX, f"{name}.bin"), dtype=np.uint8)
    ref = np.fromfile(os.path.join(FIX, f"{name}.ref"), dtype=np.float32)
    elems, nbytes = O.BLOCK[qtype]
    nblocks = raw.size // nbytes
    # Lay the 64 blocks out as rows of 256 values (the matrix API's unit).
    cols = 256
    rows = nblocks * elems // cols
    got = O.dequant(qtype, raw, rows, cols)
    assert got.size == ref.size
    assert np.array_equal(bits(got), bits(ref)), f"{name}: decode differs from llama.cpp"


def test_f16_encoder_matches_numpy():
    rng = np.random.default_rng(7)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(0.01),
        np.abs(rng.standard_normal(2000)).astype(np.float32) * np.float32(1e-6),   # subnormal f16
        np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e9, -1e9, 2.0 ** -24, 2.0 ** -25,
                  3 * 2.0 ** -26, 5.960464477539063e-08, np.inf, -np.inf], np.float32),
        (np.arange(0, 4096, dtype=np.float32) + np.float32(0.5)),                  # ties
    ])
    ours = np.array([O.orc.mynah_synth_f32_to_f16(float(v)) for v in vals], np.uint16)
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, want)


def test_f16_decoder_exact_on_all_finite_halves():
    h = np.arange(0, 1 << 16, dtype=np.uint32)
    h = h[(h & 0x7C00) != 0x7C00]                      # finite values
    sample = h[::37]
    got = np.array([O.orc.orc_f16_to_f32(int(v)) for v in sample], np.float32)
    assert np.array_equal(bits(got), bits(sample.astype(np.uint16).view(np.float16).astype(np.float32)))


def _pack_q4k_scales(sc, m):
    """Inverse of the 6-bit (scale, min) packing: 12 bytes from 8 pairs."""
    s = [0] * 12
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (m[j] & 63) | ((m[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((m[j + 4] & 15) << 4)
    return bytes(s)


def test_q4k_known_block():
    sc = [1, 7, 13, 63, 32, 17, 44, 5]
    m = [0, 3, 60, 11, 63, 1, 20, 33]
    q = [(i * 7 + 3) % 16 for i in range(256)]          # weight e's 4-bit quant
    qs = bytearray(128)
    for g in range(4):
        for i in range(32):
            qs[32 * g + i] = q[64 * g + i] | (q[64 * g + 32 + i] << 4)
    d, dmin = np.float16(0.125), np.float16(0.0625)
    blk = (d.tobytes() + dmin.tobytes() + _pack_q4k_scales(sc, m) + bytes(qs))
    w = np.frombuffer(blk, np.uint8).copy()
    got = O.dequant(12, w, 1, 256)
    want = np.array([0.125 * sc[e // 32] * q[e] - 0.0625 * m[e // 32] for e in range(256)],
                    np.float32)
    assert np.array_equal(got, want)
    x = np.zeros(256, np.float32)
    x[77] = 1.0
    assert O.matvec(12, w, 1, 256, x)[0] == want[77]


def test_q6k_known_block():
    q = [(i * 11 + 5) % 64 for i in range(256)]          # 6-bit quant of weight e
    sc = [(-64 + 9 * j) for j in range(16)]
    ql, qh = bytearray(128), bytearray(64)
    for h in range(2):
        for i in range(32):
            e = [128 * h + 32 * k + i for k in range(4)]
            ql[64 * h + i] = (q[e[0]] & 15) | ((q[e[2]] & 15) << 4)
            ql[64 * h + 32 + i] = (q[e[1]] & 15) | ((q[e[3]] & 15) << 4)
            qh[32 * h + i] = sum(((q[e[k]] >> 4) & 3) << (2 * k) for k in range(4))
    d = np.float16(0.25)
    blk = bytes(ql) + bytes(qh) + bytes(np.array(sc, np.int8).tobytes()) + d.tobytes()
    w = np.frombuffer(blk, np.uint8).copy()
    got = O.dequant(14, w, 1, 256)
    want = np.array([np.float32(0.25) * np.float32(sc[e // 16]) * np.float32(q[e] - 32)
                     for e in range(256)], np.float32)
    assert np.array_equal(got, want)


# ── the golden vectors of the compiled reference ───────────────────────────

def test_kernels_small_golden():
    g = golden("kernels_small.npz")
    for t in (CF.Q4_K, CF.Q6_K, CF.Q8_0):
        shapes = [(37, 512)] + ([(37, 96)] if t == CF.Q8_0 else [])
        for rows, cols in shapes:
            key = f"{CF.TYPE_NAME[t]}_{rows}x{cols}"
            w = O.blocks(t, 100 + t, rows, cols)
            x = O.normal(200 + t, 3 * cols)
            assert sha(w) == str(g[f"{key}_w_sha"]) and sha(x) == str(g[f"{key}_x_sha"])
            assert np.array_equal(bits(O.matvec(t, w, rows, cols, x)), bits(g[f"{key}_matvec"]))
            if cols % 256 == 0:
                assert np.array_equal(bits(O.matmat(t, w, rows, cols, x, 3)),
                                      bits(g[f"{key}_matmat3"]))
                assert np.array_equal(bits(O.dequant(t, w, rows, cols)), bits(g[f"{key}_dequant"]))
            else:
                y = np.empty(rows * cols * 3, np.float32)
                assert int(g[f"{key}_matmat3_rc"]) == -1 and int(g[f"{key}_dequant_rc"]) == -1
                assert O.orc.orc_matmat(t, O.ptr(w), rows, cols, O.ptr(x), O.ptr(y), 3) == -1
                assert O.orc.orc_dequant_matrix(t, O.ptr(w), rows, cols, O.ptr(y)) == -1


def test_c1_golden():
    g = golden("c1.npz")
    m = CF.C1[0]
    ws, xs = CF.matrix_seeds(O.substream, 0, 0)
    w, x = O.blocks(m.qtype, ws, m.rows, m.cols), O.normal(xs, m.cols)
    assert sha(w) == str(g["w_sha"]) and sha(x) == str(g["x_sha"])
    assert np.array_equal(bits(O.matvec(m.qtype, w, m.rows, m.cols, x)), bits(g["y"]))


def test_c2_golden():
    g = golden("c2.npz")
    for i, m in enumerate(CF.C2):
        ws, xs = CF.matrix_seeds(O.substream, 0, i)
        w, x = O.blocks(m.qtype, ws, m.rows, m.cols), O.normal(xs, m.cols)
        assert sha(w) == str(g[f"{m.name}_w_sha"])
        y = O.project(m.qtype, w, m.rows, m.cols, x)     # threaded == serial
        assert sha(y) == str(g[f"{m.name}_y_sha"]), m.name


def test_matmat_golden():
    g = golden("matmat.npz")
    for t, rows, cols, tokens in ((CF.Q4_K, 64, 2048, 16), (CF.Q6_K, 32, 6144, 8),
                                  (CF.Q8_0, 40, 1024, 5)):
        key = f"{CF.TYPE_NAME[t]}_{rows}x{cols}_t{tokens}"
        w, x = O.blocks(t, 300 + t, rows, cols), O.normal(400 + t, tokens * cols)
        assert sha(w) == str(g[f"{key}_w_sha"])
        assert np.array_equal(bits(O.matmat(t, w, rows, cols, x, tokens)), bits(g[f"{key}_y"]))
        assert np.array_equal(bits(O.matmat(t, w, rows, cols, x, tokens, threaded=True)),
                              bits(g[f"{key}_y"]))


def test_qwen3_tiny_golden():
    g = golden("qwen3_tiny.npz")
    shape, npre = CF.QWEN3_TINY, 16
    steps = int(g["tokens"].size)
    model = O.SynthModel(shape, 0)
    assert sha(model.blob) == str(g["blob_sha"])
    k, v = O.kv_prefill(O.substream, shape, 0, npre)
    first = O.first_token(0, shape.vocab)
    assert first == int(g["first"])
    dec = O.OracleQwen3(model, npre + steps + 1)
    dec.prefill_kv(k, v, npre)
    toks, lg0 = dec.greedy(first, steps)
    assert np.array_equal(bits(lg0), bits(g["logits0"]))
    assert toks == [int(t) for t in g["tokens"]]


def test_qwen3_06b_golden():
    g = golden("qwen3_06b.npz")
    shape, npre, steps = CF.QWEN3_06B, CF.C3_PREFILL, CF.C3_STEPS
    model = O.SynthModel(shape, 0)
    assert sha(model.blob) == str(g["blob_sha"])
    k, v = O.kv_prefill(O.substream, shape, 0, npre)
    first = O.first_token(0, shape.vocab)
    dec = O.OracleQwen3(model, npre + steps + 1)
    dec.prefill_kv(k, v, npre)
    toks, lg0 = dec.greedy(first, steps)
    assert sha(lg0) == str(g["logits0_sha"])
    assert toks == [int(t) for t in g["tokens"]]


# ── closed forms and invariants ────────────────────────────────────────────

@pytest.mark.parametrize("qtype,cols", [(12, 1024), (14, 1024), (8, 1024), (8, 96)])
def test_matvec_equals_f64_dot_of_dequant(qtype, cols):
    rows = 64
    w, x = O.blocks(qtype, 5, rows, cols), O.normal(6, cols)
    y = O.matvec(qtype, w, rows, cols, x)
    if cols % 256 == 0:
        dq = O.dequant(qtype, w, rows, cols).reshape(rows, cols).astype(np.float64)
    else:   # ragged Q8_0: decode block by block from the format definition
        blk = w.reshape(rows, cols // 32, 34)
        d = blk[:, :, :2].copy().view(np.float16).astype(np.float64)
        dq = (blk[:, :, 2:].view(np.int8).astype(np.float64) * d).reshape(rows, cols)
    ref = dq @ x.astype(np.float64)
    mag = np.abs(dq) @ np.abs(x.astype(np.float64))
    # Recursive f32 summation of n products: |error| <= ~(n + 1) u sum |w x|.
    assert (np.abs(y - ref) <= (cols + 1) * 2.0 ** -24 * mag).all()
    # ... and far tighter in practice (the reference's own budget is 1e-5 relative
    # on max(1, |y|) for its test data; these blocks reach larger |y|).
    assert (np.abs(y - ref) / np.maximum(1.0, np.abs(ref))).max() < 5e-5


def test_project_threaded_is_bit_identical():
    rows, cols = 1000, 2048
    for t in (12, 14, 8):
        w, x = O.blocks(t, 9, rows, cols), O.normal(10, cols)
        assert np.array_equal(bits(O.project(t, w, rows, cols, x)),
                              bits(O.matvec(t, w, rows, cols, x)))


def test_argument_guards():
    w = O.blocks(12, 1, 2, 256)
    x = O.normal(2, 256)
    y = np.empty(2, np.float32)
    f = O.orc.orc_matvec
    assert f(12, None, 2, 256, O.ptr(x), O.ptr(y)) == -1
    assert f(12, O.ptr(w), 2, 256, None, O.ptr(y)) == -1
    assert f(12, O.ptr(w), 0, 256, O.ptr(x), O.ptr(y)) == -1
    assert f(12, O.ptr(w), 2, 0, O.ptr(x), O.ptr(y)) == -1
    assert f(12, O.ptr(w), 2, 100, O.ptr(x), O.ptr(y)) == -1
    assert f(99, O.ptr(w), 2, 256, O.ptr(x), O.ptr(y)) == -1


def test_qwen3_4b_prompt_golden():
    """The oracle's forward at Qwen3-4B scale (36 layers, 4 query heads per
    key head) against the compiled reference's prompt prefill + greedy run:
    the first step's top-64 logits bit for bit, then the greedy ids."""
    g = np.load(os.path.join(GOLDEN, "qwen3_4b_prompt.npz"), allow_pickle=False)
    O.orc.orc_threads_init(0)
    model = O.SynthModel(CF.QWEN3_4B, 0)
    prompt = [int(t) for t in g["prompt"]]
    steps = int(g["tokens"].size)
    orc = O.OracleQwen3(model, len(prompt) + steps + 1)
    for t in prompt[:-1]:
        orc.forward(t)
    lg = orc.forward(prompt[-1])
    assert np.array_equal(lg[g["top_ids"]].view(np.uint32), g["top_vals"].view(np.uint32))
    tok, out = int(np.argmax(lg)), []
    for _ in range(steps):
        out.append(tok)
        tok = int(np.argmax(orc.forward(tok)))
    assert out == [int(t) for t in g["tokens"]]


def test_qwen3_4b_kv2048_golden():
    """The oracle's forward at configs[4]'s context (2048 cached positions, the
    CPU baseline's 4B decode leg) against the compiled reference on the same
    inputs: the first step's logits by SHA-256, its greedy id."""
    g = np.load(os.path.join(GOLDEN, "qwen3_4b_kv2048.npz"), allow_pickle=False)
    O.orc.orc_threads_init(0)
    shape, npre = CF.QWEN3_4B, CF.C5_CPU_KV
    model = O.SynthModel(shape, 0)
    assert sha(model.blob) == str(g["blob_sha"])
    orc = O.OracleQwen3(model, npre + 2)
    k, v = O.kv_prefill(O.substream, shape, 0, npre)
    orc.prefill_kv(k, v, npre)
    del k, v
    first = O.first_token(0, shape.vocab)
    assert first == int(g["first"])
    lg = orc.forward(first)
    assert sha(lg) == str(g["logits0_sha"])
    assert int(O.orc.orc_argmax(O.ptr(lg), lg.size)) == int(g["tokens"][0])
