"""CPU tests of the C ABI library: it loads, exports every symbol the public
headers declare, rejects bad arguments without touching a device (the
reference's guard cases, third_party/ingot/tests/test_quant.c:298-309), and its
built-in generator matches the oracle's copy byte for byte."""
from __future__ import annotations

import ctypes as C
import os
import re

import numpy as np

import mynah_amd as M
import oracle_lib as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions(header: str):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^[A-Za-z_][\w \*]*?\b([a-z_][a-z0-9_]*)\s*\(", text, flags=re.M)
    return sorted(set(n for n in names if n not in ("defined",)))


def test_every_declared_symbol_is_exported():
    for header in sorted(f for f in os.listdir(os.path.join(ROOT, "include")) if f.endswith(".h")):
        names = declared_functions(header)
        assert len(names) > 5, header
        for n in names:
            assert hasattr(M.lib, n), f"{header}: {n} not exported"


def test_has_kernel_and_exactness():
    # The reference's specialised kernels (generic.c:24-37) for the five
    # types built here; Q4_1 has none there either.
    assert [M.lib.ingot_has_kernel(t) for t in (8, 12, 14, 2, 13)] == [1, 1, 1, 1, 1]
    assert [M.lib.ingot_has_kernel(t) for t in (3, 99)] == [0, 0]
    assert M.lib.ingot_matmat_is_exact(1) == 1 and M.lib.ingot_matmat_is_exact(512) == 1


def test_guards_fail_without_a_device():
    w = np.zeros(144 * 2, np.uint8)
    x = np.zeros(256, np.float32)
    y = np.zeros(2, np.float32)
    P = M.ptr
    f = M.lib.ingot_matvec
    assert f(12, None, 2, 256, P(x), P(y)) == -1
    assert f(12, P(w), 2, 256, None, P(y)) == -1
    assert f(12, P(w), 2, 256, P(x), None) == -1
    assert f(12, P(w), 0, 256, P(x), P(y)) == -1
    assert f(12, P(w), 2, 0, P(x), P(y)) == -1
    assert f(12, P(w), 2, 100, P(x), P(y)) == -1
    assert f(99, P(w), 2, 256, P(x), P(y)) == -1
    assert M.lib.ingot_matmat(12, P(w), 2, 256, P(x), P(y), 0) == -1
    assert M.lib.ingot_dequant_matrix(12, None, 2, 256, P(y)) == -1
    assert M.lib.mynah_hip_last_error()


def test_gguf_matvec_needs_the_reader():
    # No ingot GGUF reader in this process: a clean -1, not a crash.
    buf = C.create_string_buffer(128)
    assert M.lib.ingot_gguf_matvec(C.addressof(buf), C.addressof(buf), None, None) == -1


def test_generator_identical_in_both_builds():
    for t, rows, cols in ((12, 5, 512), (14, 3, 768), (8, 7, 96)):
        assert np.array_equal(M.synth_blocks(t, 123, rows, cols), O.blocks(t, 123, rows, cols))
    assert np.array_equal(M.synth_normal(9, 10000), O.normal(9, 10000))


def test_generator_row_offset_is_a_substream():
    full = M.synth_blocks(14, 77, 10, 512)
    part = M.synth_blocks(14, 77, 4, 512, row0=6)
    rb = M.row_bytes(14, 512)
    assert np.array_equal(full[6 * rb:], part)
