"""Split GGUF checkpoints (include/mynah_gguf.h mynah_gguf_open_split, the
twin of ingot_gguf_open_split: third_party/ingot/include/ingot/gguf.h:62-66,
src/gguf.c:466-570; the reference's loader opens every checkpoint through it,
src/model.c:183).

Every case of tests/gguf_cases.py SPLIT_CASES — three- and two-shard
checkpoints opened through any shard's name, per-shard alignments (a later
shard's missing or zero general.alignment meaning 32), and one shard broken
or missing at a time — is read by this library and compared with what the
compiled reference's reader made of it (tests/golden/gguf_cases.json, and
live where oracle/_ref/libref.so is built): the same verdict, header, merged
tensor table (each tensor's shard and offset within that shard's data
section) and metadata reads. Accepted checkpoints also give back every
payload the writer put in, byte for byte.
"""
from __future__ import annotations

import json
import os
import re

import numpy as np
import pytest

import gguf_cases as GC
import oracle_lib as O

HERE = os.path.dirname(os.path.abspath(__file__))
CASES = json.load(open(os.path.join(HERE, "golden", "gguf_cases.json")))
KEYS = [k for k, *_ in GC.mini_writer().kvs] + ["general.alignment", "absent.key"]


@pytest.fixture(scope="module")
def M():
    import mynah_amd
    return mynah_amd


@pytest.fixture(scope="module")
def ref():
    return O.load_ref()


def materialise(tmp_path, case):
    files, opened = GC.SPLIT_CASES[case]()
    d = tmp_path / case
    d.mkdir()
    for name, data in files:
        (d / name).write_bytes(data)
    return str(d / opened), files


def ours_split(M, path):
    """This library's reading in ref_gguf_read(split=True)'s form."""
    try:
        g = M.GgufFile(path, split=True)
    except M.HipError as e:
        assert str(e).split(":", 1)[1].strip(), "refusal without a message"
        return None
    with g:
        shard0 = re.sub(r"-\d{5}-of-(\d{5})\.gguf$", r"-00001-of-\1.gguf", path) \
            if g.n_shards > 1 else path
        out = {"version": g.version, "n_kv": g.n_kv, "alignment": g.alignment,
               "data_base": os.path.getsize(shard0) - g.shard_size(0), "tensors": [], "kv": {}}
        for (name, t, rank, rows, cols, _, nb), (sh, off) in zip(g.tensors(), g.places()):
            out["tensors"].append([name, t, rank, rows, cols, off, nb, sh])
        for key in KEYS:
            u, f, s, n = g.get_int(key), g.get_float(key), g.get_str(key), g.array_len(key)
            out["kv"][key] = None if (u, f, s, n) == (None, None, None, None) else \
                {"u64": u, "f64": f, "str": s, "arr_len": n}
        return out


def as_ours(ref_read):
    """ref_gguf_read(split=True) rows -> [name, type, rank, rows, cols,
    offset, nbytes, shard]."""
    if ref_read is None:
        return None
    out = dict(ref_read)
    rows = []
    for name, t, rank, ne, off, nb, sh in ref_read["tensors"]:
        cols = ne[0] if rank >= 1 else 1
        r = int(np.prod(ne[1:], dtype=np.uint64)) if rank >= 2 else 1
        rows.append([name, t, rank, r, cols, off, nb, sh])
    out["tensors"] = rows
    return out


def same(ours, want):
    if ours is None or want is None:
        return ours is None and want is None
    for k in ("version", "n_kv", "alignment", "data_base", "tensors"):
        if ours[k] != want[k]:
            return False
    for key in KEYS:
        a, b = ours["kv"].get(key), want["kv"].get(key)
        if (a is None) != (b is None):
            return False
        if a is None:
            continue
        for f in ("u64", "str", "arr_len"):
            if a[f] != b[f]:
                return False
        if (a["f64"] is None) != (b["f64"] is None) or (
                a["f64"] is not None and not np.isnan(b["f64"]) and a["f64"] != b["f64"]):
            return False
    return True


@pytest.mark.parametrize("case", sorted(GC.SPLIT_CASES))
def test_split_case_agrees_with_reference(M, ref, tmp_path, case):
    path, _ = materialise(tmp_path, case)
    ours = ours_split(M, path)
    assert same(ours, as_ours(CASES["split"][case])), (case, ours is None)
    if ref is not None:
        assert same(ours, as_ours(O.ref_gguf_read(ref, path, KEYS, split=True)))


def test_recorded_split_verdicts_cover_every_case():
    assert set(CASES["split"]) == set(GC.SPLIT_CASES)
    for good in ("three_shards", "open_via_second", "open_via_last", "two_shards_v2",
                 "later_alignment_64", "later_alignment_0", "later_no_alignment_key",
                 "one_of_one_is_plain", "plain_name"):
        assert CASES["split"][good] is not None, good
    for bad in ("missing_shard", "duplicate_across_shards", "later_bad_kv_type",
                "later_version_1", "later_truncated", "later_payload_past_eof",
                "later_alignment_48"):
        assert CASES["split"][bad] is None, bad
    assert CASES["open"]["duplicate_tensor_name"] is None


@pytest.mark.parametrize("case", ["three_shards", "later_alignment_64", "two_shards_v2"])
def test_split_payloads_and_placement(M, tmp_path, case):
    """Independent of any recorded answer: each tensor in the shard it was
    written to, its bytes the payload, the merged order the writer's."""
    path, files = materialise(tmp_path, case)
    w = GC.mini_writer(version=2) if case == "two_shards_v2" else GC.mini_writer()
    n = len(files)
    per = -(-len(w.tensors) // n)
    with M.GgufFile(path, split=True) as g:
        assert g.n_shards == n and g.n_tensors == len(w.tensors)
        for i, ((name, t, rank, rows, cols, _, nb), (sh, off)) in enumerate(
                zip(g.tensors(), g.places())):
            wn, wt, ne, data = w.tensors[i]
            assert (name, t, cols, nb, sh) == (wn, wt, ne[0], len(data), i // per)
            assert g.shard_bytes(sh, off, nb) == data
        assert g.get_str("general.architecture") == "mini"


def test_single_open_refuses_split_only_through_split(M, tmp_path):
    """The plain open reads one shard as the file it is; the split open
    reads the checkpoint."""
    path, _ = materialise(tmp_path, "three_shards")
    with M.GgufFile(path) as g:
        assert g.n_shards == 1 and g.n_tensors < 7
    with M.GgufFile(path, split=True) as g:
        assert g.n_shards == 3 and g.n_tensors == 7
