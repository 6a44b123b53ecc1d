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
    text = re.sub(r"^typedef [^;]*;", "", text, flags=re.M)   # function-pointer types
    names = re.findall(r"^[A-Za-z_][\w \*]*?\b([a-z_][a-z0-9_]*)\s*\(", text, flags=re.M)
    return sorted(set(n for n in names if n not in ("defined",)))


def test_every_declared_symbol_is_exported():
    for header in sorted(f for f in os.listdir(os.path.join(ROOT, "include")) if f.endswith(".h")):
        names = declared_functions(header)
        assert names, header
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
    for call in (lambda: M.lib.ingot_gguf_matvec(C.addressof(buf), C.addressof(buf), None, None),
                 lambda: M.lib.ingot_gguf_matmat(C.addressof(buf), C.addressof(buf), None, None, 1),
                 lambda: M.lib.ingot_gguf_dequant_matrix(C.addressof(buf), C.addressof(buf), None)):
        assert call() == -1
    assert b"ingot_gguf_data" in M.lib.mynah_hip_last_error()


# The refusals of the GGUF-tensor entry points (generic.c:148-173) happen
# before any device work, so they run here, in a child process that loads a
# stand-in reader (oracle/gguf_shim.c) ahead of the library.
GGUF_REFUSALS = r"""
import ctypes as C, sys
sys.path[:0] = [sys.argv[1], sys.argv[2]]
C.CDLL(sys.argv[3], mode=C.RTLD_GLOBAL)
import gguf_shim_lib as S
lib = S.load_library()
blob = (C.c_ubyte * 4096)()
g = S.Handle(C.cast(blob, C.c_void_p), 4096, 0)
x = (C.c_float * 512)()
y = (C.c_float * 512)()
def call(t):
    return lib.ingot_gguf_matvec(C.byref(g), C.byref(t), x, y)
out = []
out.append(call(S.tensor(12, 3, (256, 2, 1), 0, 288)))    # rank 3
out.append(call(S.tensor(12, 0, (256,), 0, 144)))         # rank 0
out.append(call(S.tensor(12, 2, (256, 0), 0, 0)))         # a zero row count
out.append(call(S.tensor(12, 2, (0, 2), 0, 0)))           # a zero width
out.append(call(S.tensor(12, 2, (256, 2), 4000, 288)))    # bytes outside the mapping
out.append(lib.ingot_gguf_matvec(None, C.byref(S.tensor(12, 1, (256,), 0, 144)), x, y))
out.append(lib.ingot_gguf_dequant_matrix(C.byref(g), C.byref(S.tensor(12, 3, (256, 1, 1), 0, 144)), y))
out.append(lib.ingot_gguf_matmat(C.byref(g), C.byref(S.tensor(12, 2, (256, 2), 4000, 288)), x, y, 2))
print(out)
print(lib.mynah_hip_last_error().decode())
"""


def test_gguf_entry_points_refuse_like_the_reference():
    import subprocess
    import sys
    shim = os.path.join(ROOT, "oracle", "libgguf_shim.so")
    r = subprocess.run([sys.executable, "-c", GGUF_REFUSALS, os.path.join(ROOT, "tests"),
                        os.path.join(ROOT, "mynah-slm_amd"), shim],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    lines = r.stdout.strip().splitlines()
    assert lines[0] == str([-1] * 8), r.stdout
    # The stand-in reader was bound (the last refusal is its NULL, not a
    # missing reader).
    assert lines[-1] == "tensor data not found", r.stdout


def _called_names(path: str):
    """(receiver, name) of every `<lib>.<entry point>` in a Python source."""
    text = open(path).read()
    pat = r"\b(lib|orc|ref8|ref)\.((?:mynah|ingot|orc|ref)_[a-z0-9_]+)\b"
    return set(re.findall(pat, text))


def test_every_called_entry_point_has_a_ctypes_signature():
    """ctypes passes an argument of an undeclared function as a C int: a
    64-bit pointer loses its upper half and the library dereferences the
    truncated address. Every library function that the tests, the benchmark
    and the driver entry call must have its argtypes declared."""
    sources = [os.path.join(ROOT, "bench.py"), os.path.join(ROOT, "__graft_entry__.py"),
               os.path.join(ROOT, "mynah-slm_amd", "mynah_amd.py")]
    for d in (os.path.join(ROOT, "tests"), os.path.join(ROOT, "tests", "golden")):
        sources += [os.path.join(d, f) for f in sorted(os.listdir(d)) if f.endswith(".py")]
    ref, ref8 = O.load_ref(), O.load_ref_int8()
    libs = {"lib": M.lib, "orc": O.orc, "ref": ref, "ref8": ref8}
    missing = []
    for path in sources:
        for recv, name in sorted(_called_names(path)):
            target = libs[recv]
            if recv == "lib" and os.path.basename(path) == "oracle_lib.py":
                continue        # there `lib` is the library being declared
            if recv == "ref" and name.startswith(("mynah_hip", "mynah_synth")):
                target = M.lib  # a GPU-side object named ref in a test
            if target is None:
                continue        # the compiled reference is not built here
            if getattr(target, name).argtypes is None:
                missing.append(f"{os.path.relpath(path, ROOT)}: {recv}.{name}")
    assert not missing, "undeclared ctypes signatures:\n" + "\n".join(missing)


def test_generator_identical_in_both_builds():
    for t, rows, cols in ((12, 5, 512), (14, 3, 768), (8, 7, 96)):
        assert np.array_equal(M.synth_blocks(t, 123, rows, cols), O.blocks(t, 123, rows, cols))
    assert np.array_equal(M.synth_normal(9, 10000), O.normal(9, 10000))


def test_generator_row_offset_is_a_substream():
    full = M.synth_blocks(14, 77, 10, 512)
    part = M.synth_blocks(14, 77, 4, 512, row0=6)
    rb = M.row_bytes(14, 512)
    assert np.array_equal(full[6 * rb:], part)
