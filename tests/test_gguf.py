"""The GGUF reader (include/mynah_gguf.h) against the reference's reader and
loader, on the CPU.

Pinned three ways:
  * the test writer (tests/gguf_writer.py) produces the bytes of the
    reference's writer for the tiny Qwen3 (SHA-256 in
    tests/golden/gguf_cases.json; byte-for-byte with the compiled reference
    where oracle/_ref/libref.so is built);
  * for every file of tests/gguf_cases.py, this reader accepts exactly what
    ingot_gguf_open accepts and reads the same header, tensor table and
    metadata values; the config matches mynah_slm_load's, refusals included
    (verdicts recorded from the compiled reference in gguf_cases.json, and
    re-derived live where the reference is built);
  * truncations at every byte of a small file never crash and are refused
    exactly where the reference refuses them.
"""
from __future__ import annotations

import ctypes as C
import hashlib
import json
import os

import numpy as np
import pytest

import configs as CF
import gguf_cases as GC
import gguf_writer as GW
import oracle_lib as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
CASES = json.load(open(os.path.join(GOLDEN, "gguf_cases.json")))
MINI_KEYS = [k for k, *_ in GC.mini_writer().kvs] + ["general.alignment", "absent.key"]


@pytest.fixture(scope="module")
def M():
    import mynah_amd
    return mynah_amd


@pytest.fixture(scope="module")
def ref():
    return O.load_ref()


def write(tmp_path, name: str, data: bytes) -> str:
    p = str(tmp_path / f"{name}.gguf")
    with open(p, "wb") as f:
        f.write(data)
    return p


def ours_read(M, path: str, keys=()):
    """This reader's view of the file, in ref_gguf_read's form."""
    try:
        g = M.GgufFile(path)
    except M.HipError as e:
        assert str(e).split(":", 1)[1].strip(), "refusal without a message"
        return None
    with g:
        out = {"version": g.version, "n_kv": g.n_kv, "alignment": g.alignment,
               "data_base": os.path.getsize(path) - g.data_bytes(), "tensors": [], "kv": {}}
        assert g.n_tensors == len(g.tensors())
        for name, t, rank, rows, cols, off, nb in g.tensors():
            out["tensors"].append([name, t, rank, rows, cols, off, nb])
        for key in keys:
            u, f, s, n = g.get_int(key), g.get_float(key), g.get_str(key), g.array_len(key)
            out["kv"][key] = None if (u, f, s, n) == (None, None, None, None) else \
                {"u64": u, "f64": f, "str": s, "arr_len": n}
        return out


def as_table(ref_tensors):
    """The reference's [name, type, rank, ne, offset, nbytes] rows in the form
    this reader reports them (rows = product of ne[1..], cols = ne[0])."""
    out = []
    for name, t, rank, ne, off, nb in ref_tensors:
        cols = ne[0] if rank >= 1 else 1
        rows = int(np.prod(ne[1:], dtype=np.uint64)) if rank >= 2 else 1
        out.append([name, t, rank, rows, cols, off, nb])
    return out


def same_reading(ours, theirs):
    if theirs is None or ours is None:
        return ours is None and theirs is None
    for k in ("version", "n_kv", "alignment", "data_base"):
        assert ours[k] == theirs[k], k
    assert ours["tensors"] == as_table(theirs["tensors"])
    for key, want in theirs["kv"].items():
        got = ours["kv"][key]
        if want is None:
            assert got is None, key
            continue
        assert got is not None, key
        assert got["u64"] == want["u64"], key
        assert got["arr_len"] == want["arr_len"], key
        assert got["str"] == want["str"], key
        if want["f64"] is None or np.isnan(want["f64"]):
            assert (got["f64"] is None) == (want["f64"] is None), key
        else:
            assert got["f64"] == want["f64"], key
    return True


# ── the writer ────────────────────────────────────────────────────────────

def tiny_bytes():
    m = O.SynthModel(CF.QWEN3_TINY, 0)
    return GW.qwen3_gguf(m.shape, m.table, m.count, m.blob, CASES["qwen3_tiny"]["n_ctx"]), m


def test_writer_matches_the_reference_writer(ref, tmp_path):
    data, m = tiny_bytes()
    want = CASES["qwen3_tiny"]
    assert len(data) == want["bytes"]
    assert hashlib.sha256(data).hexdigest() == want["sha256"]
    if ref is not None:
        p = str(tmp_path / "ref.gguf").encode()
        err = C.create_string_buffer(512)
        assert ref.ref_write_qwen3_gguf(p, C.byref(m.c_shape), m.table, m.count, O.ptr(m.blob),
                                        want["n_ctx"], err, 512) == 0, err.value
        assert open(p, "rb").read() == data


# ── the container ─────────────────────────────────────────────────────────

@pytest.mark.parametrize("case", sorted(GC.OPEN_CASES))
def test_open_case_agrees_with_reference(M, ref, tmp_path, case):
    path = write(tmp_path, case, GC.OPEN_CASES[case]())
    ours = ours_read(M, path, MINI_KEYS)
    assert same_reading(ours, CASES["open"][case]), (case, ours is None)
    if ref is not None:
        assert same_reading(ours, O.ref_gguf_read(ref, path, MINI_KEYS))


def test_recorded_verdicts_cover_every_case():
    assert set(CASES["open"]) == set(GC.OPEN_CASES)
    assert set(CASES["config"]) == set(GC.CONFIG_CASES)
    # The reference's own malformations (ingot tests/test_gguf.c:345-410)
    # are all refused; the valid layouts are all read.
    for bad in ("bad_magic", "version_1", "version_9", "truncated_40", "alignment_value_33",
                "tensor_type_99", "huge_key_length", "tensor_count_max", "offset_past_eof"):
        assert CASES["open"][bad] is None, bad
    for good in ("valid_v3", "valid_v2", "no_alignment_key", "alignment_16"):
        assert CASES["open"][good] is not None, good


def test_valid_file_values(M, tmp_path):
    """Independent of any recorded answer: the values the writer put in."""
    w = GC.mini_writer()
    path = write(tmp_path, "mini", w.to_bytes())
    with M.GgufFile(path) as g:
        assert (g.version, g.n_kv, g.n_tensors, g.alignment) == (3, len(w.kvs) + 1, 7, 32)
        assert g.get_str("general.architecture") == "mini"
        assert g.get_int("mini.u8") == 200 and g.get_int("mini.i8") == (1 << 64) - 3
        assert g.get_int("mini.u32") == 4000000000 and g.get_float("mini.i32") == -100000.0
        assert g.get_float("mini.f32") == 0.5 and g.get_int("mini.f32") == 0
        assert g.get_int("mini.bool") == 1 and g.get_int("mini.u64") == 1 << 40
        assert g.get_int("mini.f64") == 2750000000 and g.get_int("mini.neg_f64") == 0
        assert g.get_int("mini.big_f32") == (1 << 64) - 1          # saturates
        assert g.array_len("mini.tokens") == 4 and g.array_len("mini.empty") == 0
        assert g.get_int("mini.tokens") is None and g.get_str("mini.u8") is None
        assert g.get_int("absent.key") is None and g.array_len("mini.u8") is None
        for (name, t, rank, rows, cols, off, nb), (wn, wt, ne, data) in zip(g.tensors(), w.tensors):
            assert (name, t, rank, cols) == (wn, wt, len(ne), ne[0])
            assert rows == int(np.prod(ne[1:])) and nb == len(data)
            assert off % 32 == 0 and g.tensor_data(off, nb) == data


def test_tiny_model_table_and_bytes(M, tmp_path):
    data, m = tiny_bytes()
    path = write(tmp_path, "tiny", data)
    with M.GgufFile(path) as g:
        shape, n_ctx = g.qwen3_shape()
        for name, _ in M.Qwen3Shape._fields_:
            assert getattr(shape, name) == pytest.approx(getattr(m.c_shape, name), rel=0), name
        assert n_ctx == CASES["qwen3_tiny"]["n_ctx"]
        table = g.tensors()
        assert len(table) == m.count
        for (name, t, rank, rows, cols, off, nb), st in zip(table, m.table[:m.count]):
            assert (name, t, rank, rows, cols, nb) == (st.name.decode(), st.type, st.rank, st.rows,
                                                       st.cols, st.nbytes)
            assert g.tensor_data(off, nb) == m.blob[st.offset:st.offset + nb].tobytes()


def test_truncation_sweep(M, ref, tmp_path):
    """Every prefix of a small file: no crash, and accepted from the end of
    the last payload on (the trailing pad is optional), like the reference."""
    w = GC.mini_writer()
    data = w.to_bytes()
    last = w.tensors[-1]
    end = w.pos[("data", last[0])] + len(last[3])
    path = str(tmp_path / "cut.gguf")
    for n in range(len(data) + 1):
        with open(path, "wb") as f:
            f.write(data[:n])
        ok = ours_read(M, path) is not None
        assert ok == (n >= end), n
        if ref is not None and (n < 600 or n % 7 == 0 or n >= end - 2):
            assert ok == (O.ref_gguf_read(ref, path) is not None), n


def test_open_errors(M, tmp_path):
    for path in (str(tmp_path / "does-not-exist.gguf"), str(tmp_path)):
        with pytest.raises(M.HipError):
            M.GgufFile(path)
    err = C.create_string_buffer(64)
    assert not M.lib.mynah_gguf_open(None, err, 64) and err.value
    assert M.lib.mynah_gguf_version(None) == 0 and M.lib.mynah_gguf_n_tensors(None) == 0
    M.lib.mynah_gguf_close(None)


def test_flipped_bytes_never_crash(M, tmp_path):
    """Random single-byte corruptions of the header and tables: either read
    or refused with a message, never a crash (what the reference's
    fuzz_mutate.c exercises on its reader)."""
    w = GC.mini_writer()
    data = w.to_bytes()
    limit = w.pos["data"]                            # header, metadata, tensor table
    rng = np.random.default_rng(7)
    path = str(tmp_path / "flip.gguf")
    for i in range(400):
        b = bytearray(data)
        for _ in range(1 + i % 3):
            b[int(rng.integers(0, limit))] = int(rng.integers(0, 256))
        with open(path, "wb") as f:
            f.write(bytes(b))
        ours_read(M, path, MINI_KEYS)


# ── the Qwen3 config ──────────────────────────────────────────────────────

def ours_config(M, path: str):
    try:
        with M.GgufFile(path) as g:
            shape, n_ctx = g.qwen3_shape()
    except M.HipError:
        return None
    out = {n: getattr(shape, n) for n in GC.CONFIG_FIELDS if n not in ("n_ctx",)}
    out["n_ctx"] = n_ctx
    out["rms_eps"], out["rope_theta"] = float(np.float32(out["rms_eps"])), \
        float(np.float32(out["rope_theta"]))
    return out


@pytest.mark.parametrize("case", sorted(GC.CONFIG_CASES))
def test_config_case_agrees_with_reference(M, ref, tmp_path, case):
    path = write(tmp_path, case.replace(".", "_"), GC.CONFIG_CASES[case]())
    ours = ours_config(M, path)
    want = CASES["config"][case]
    assert ours == want, (case, ours, want)
    if ref is not None:
        assert ours == O.ref_qwen3_config(ref, path)


def test_config_refusals_name_the_key(M, tmp_path):
    path = write(tmp_path, "nokey", GC.CONFIG_CASES["missing_rope.freq_base"]())
    with M.GgufFile(path) as g, pytest.raises(M.HipError, match="qwen3.rope.freq_base"):
        g.qwen3_shape()
    path = write(tmp_path, "vlen", GC.CONFIG_CASES["value_length_64"]())
    with M.GgufFile(path) as g, pytest.raises(M.HipError, match="value_length"):
        g.qwen3_shape()
