"""The working path of the GGUF-tensor entry points on the GPU.

The reference's decoder calls ingot_gguf_matvec for every projection when it
runs on one thread or a matrix has fewer than 64 rows
(/root/reference/src/arch_qwen3.c:52-64). The entry point maps a tensor's
shape the ggml way, rows = ne[1] and cols = ne[0], rank 1 being one row, and
finds the bytes through the process's ingot_gguf_data
(/root/reference/third_party/ingot/src/generic.c:148-173).

Here the process's reader is the stand-in of oracle/gguf_shim.c (loaded
RTLD_GLOBAL ahead of libmynah_hip.so, so in a child process). Each case puts
a Q4_K, Q6_K or Q8_0 tensor of rank 1 or 2 into a mapping at a non-zero data
offset and calls ingot_gguf_matvec, ingot_gguf_matmat (1 and 5 tokens) and
ingot_gguf_dequant_matrix, once with the mapping staged per call and once with
it registered (mynah_hip_register, resident in HBM). Every output must be
bit-identical to ingot_matvec / ingot_matmat / ingot_dequant_matrix on the
same bytes and to the oracle's restatement of the reference.
"""
from __future__ import annotations

import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

CHILD = r"""
import ctypes as C, sys
sys.path[:0] = [sys.argv[1], sys.argv[2]]
C.CDLL(sys.argv[3], mode=C.RTLD_GLOBAL)
import numpy as np
import gguf_shim_lib as S
import oracle_lib as O
import mynah_amd as M

lib = M.lib
M.check(lib.mynah_hip_init(0), "init")
M.check(lib.mynah_hip_set_gemv_order(0), "order")

def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)

def ptr(a):
    return a.ctypes.data

# (type, rank, rows, cols, skew): each tensor starts at the next 256-byte
# boundary of the data section plus its skew. A skew of 2 or 6 leaves a Q4_K
# tensor off 16 bytes; the registered copy keeps the host address's skew, so
# such a tensor reaches the kernels through the staged path.
CASES = [(12, 2, 96, 1024, 0), (12, 1, 1, 2048, 32), (12, 2, 7, 512, 2),
         (14, 2, 80, 768, 16), (14, 1, 1, 1536, 2), (14, 2, 33, 256, 6),
         (8, 2, 64, 512, 32), (8, 1, 1, 1024, 34), (8, 2, 9, 256, 6)]
TOKENS = 5
DATA_BASE = 96

blob = np.zeros(1 << 20, np.uint8)
g = S.Handle(ptr(blob), blob.nbytes, DATA_BASE)
cursor = 256
for i, (qt, rank, rows, cols, skew) in enumerate(CASES):
    w = M.synth_blocks(qt, 40 + i, rows, cols)
    off = cursor + skew
    cursor = (off + w.nbytes + 255) // 256 * 256
    start = DATA_BASE + off
    assert start + w.nbytes <= blob.nbytes
    blob[start:start + w.nbytes] = w
    ne = (cols, rows) if rank == 2 else (cols,)
    t = S.tensor(qt, rank, ne, off, w.nbytes)
    x = M.synth_normal(60 + i, TOKENS * cols)
    view = blob[start:start + w.nbytes]
    mv_ref = O.matvec(qt, view, rows, cols, x[:cols])
    mm_ref = O.matmat(qt, view, rows, cols, x, TOKENS)
    dq_ref = O.dequant(qt, view, rows, cols)

    def run(tag):
        y1 = np.full(rows, np.nan, np.float32)
        y5 = np.full(rows * TOKENS, np.nan, np.float32)
        ym = np.full(rows, np.nan, np.float32)
        dq = np.full(rows * cols, np.nan, np.float32)
        assert lib.ingot_gguf_matvec(C.byref(g), C.byref(t), ptr(x), ptr(y1)) == 0, \
            lib.mynah_hip_last_error()
        assert lib.ingot_gguf_matmat(C.byref(g), C.byref(t), ptr(x), ptr(y5), TOKENS) == 0, \
            lib.mynah_hip_last_error()
        assert lib.ingot_gguf_matmat(C.byref(g), C.byref(t), ptr(x), ptr(ym), 1) == 0, \
            lib.mynah_hip_last_error()
        assert lib.ingot_gguf_dequant_matrix(C.byref(g), C.byref(t), ptr(dq)) == 0, \
            lib.mynah_hip_last_error()
        # The same bytes through the plain entry points.
        p1 = np.empty(rows, np.float32)
        p5 = np.empty(rows * TOKENS, np.float32)
        pd = np.empty(rows * cols, np.float32)
        assert lib.ingot_matvec(qt, ptr(view), rows, cols, ptr(x), ptr(p1)) == 0
        assert lib.ingot_matmat(qt, ptr(view), rows, cols, ptr(x), ptr(p5), TOKENS) == 0
        assert lib.ingot_dequant_matrix(qt, ptr(view), rows, cols, ptr(pd)) == 0
        for name, got, plain, ref in (("matvec", y1, p1, mv_ref), ("matmat1", ym, p1, mv_ref),
                                      ("matmat5", y5, p5, mm_ref), ("dequant", dq, pd, dq_ref)):
            assert np.array_equal(bits(got), bits(plain)), (tag, name, "vs plain entry point")
            assert np.array_equal(bits(got), bits(ref)), (tag, name, "vs oracle")
        print(f"PASS {tag} type={qt} rank={rank} rows={rows} cols={cols} off={off}", flush=True)

    print(f"[case] type={qt} rank={rank} rows={rows} cols={cols} off={off}", flush=True)
    run("staged")
    assert lib.mynah_hip_register(ptr(blob), blob.nbytes) == 0, lib.mynah_hip_last_error()
    assert lib.mynah_hip_device_ptr(ptr(view)) is not None
    run("registered")
    assert lib.mynah_hip_unregister(ptr(blob)) == 0, lib.mynah_hip_last_error()
print("ALL OK", flush=True)
"""


def test_gguf_entry_points_compute_like_the_plain_ones():
    shim = os.path.join(ROOT, "oracle", "libgguf_shim.so")
    r = subprocess.run([sys.executable, "-u", "-c", CHILD, os.path.join(ROOT, "tests"),
                        os.path.join(ROOT, "mynah-slm_amd"), shim],
                       capture_output=True, text=True, timeout=110)
    print(r.stdout)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    assert r.stdout.strip().splitlines()[-1] == "ALL OK"
    assert r.stdout.count("PASS ") == 18
