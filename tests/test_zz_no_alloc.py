"""The allocation-free int8 product (mynah_hip_int8_product_noalloc_dev)
against the allocating entry point it mirrors (mynah_hip_matmat_dev with the
int8 lane on, itself bit-exact against the AVX2 build of the reference in
test_int8_gpu.py): bit-identical outputs on two calls in a row, the second
smaller than the first, so the fixed workspace is reused with stale contents
from the first call; a workspace above the fixed limit refused before any
launch; and a call after the refusal still right.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle_lib as O

pytestmark = pytest.mark.gpu

SCRATCH = 8 << 20


@pytest.fixture(scope="module")
def M():
    import mynah_amd
    mynah_amd.check(mynah_amd.lib.mynah_hip_init(0), "init")
    return mynah_amd


def workspace_bytes(tokens, cols):
    nb = cols // 256
    up = lambda n: (n + 255) & ~255  # noqa: E731
    return up(tokens * cols) + up(tokens * nb * 4) + tokens * nb * 32


class Case:
    def __init__(self, M, qtype, rows, cols, max_tokens, seed):
        self.M, self.qtype, self.rows, self.cols = M, qtype, rows, cols
        self.w = M.DeviceBuffer.from_array(M.synth_blocks(qtype, seed, rows, cols))
        self.x_host = M.synth_normal(seed + 1, max_tokens * cols)
        self.x = M.DeviceBuffer.from_array(self.x_host)
        self.y = M.DeviceBuffer(4 * rows * max_tokens)

    def noalloc(self, tokens):
        rc = self.M.lib.mynah_hip_int8_product_noalloc_dev(
            self.qtype, self.w.ptr, self.rows, self.cols, self.x.ptr, self.y.ptr, tokens, None)
        self.M.check(rc, "int8_product_noalloc")
        self.M.sync()
        return self.y.download(np.float32, self.rows * tokens)

    def allocating(self, tokens):
        M = self.M
        M.check(M.lib.mynah_hip_set_int8(M.INT8_ALL), "set_int8")
        try:
            M.matmat_dev(self.qtype, self.w.ptr, self.rows, self.cols, self.x.ptr, self.y.ptr,
                         tokens)
            M.sync()
        finally:
            M.check(M.lib.mynah_hip_set_int8(M.INT8_OFF), "set_int8")
        return self.y.download(np.float32, self.rows * tokens)


def bits(a):
    return a.view(np.uint32)


@pytest.mark.parametrize("qtype,rows,cols,first,second",
                         [(12, 1024, 2048, 512, 37), (12, 300, 4096, 3, 1),
                          (13, 256, 4096, 130, 2), (12, 96, 9728, 700, 5)])
def test_noalloc_equals_the_allocating_entry_point(M, qtype, rows, cols, first, second):
    print(f"[case] int8 no-alloc type={qtype} {rows}x{cols} tokens {first} then {second}",
          flush=True)
    assert workspace_bytes(first, cols) <= SCRATCH
    c = Case(M, qtype, rows, cols, first, seed=rows + cols)
    for tokens in (first, second):
        got = c.noalloc(tokens)
        want = c.allocating(tokens)
        assert np.array_equal(bits(got), bits(want)), f"tokens={tokens}"
    if qtype == 12 and second == 1:
        # the one-token epilogue is the reference's int8 matvec
        ref = np.empty(rows, np.float32)
        wh = M.synth_blocks(qtype, rows + cols, rows, cols)
        assert O.orc.orc_q4k_matvec_int8(O.ptr(wh), rows, cols, O.ptr(c.x_host), O.ptr(ref)) == 0
        assert np.array_equal(bits(c.noalloc(1)), bits(ref))


def test_noalloc_refuses_beyond_the_workspace(M):
    cols, rows = 9728, 64
    too_many = 800
    assert workspace_bytes(too_many, cols) > SCRATCH
    c = Case(M, 12, rows, cols, too_many, seed=5)
    rc = M.lib.mynah_hip_int8_product_noalloc_dev(12, c.w.ptr, rows, cols, c.x.ptr, c.y.ptr,
                                                  too_many, None)
    assert rc == -1
    assert b"exceeds the fixed" in M.lib.mynah_hip_last_error()
    # a call that fits still gives the allocating entry point's bits
    assert np.array_equal(bits(c.noalloc(9)), bits(c.allocating(9)))
    # bad arguments are refused too
    assert M.lib.mynah_hip_int8_product_noalloc_dev(14, c.w.ptr, rows, cols, c.x.ptr, c.y.ptr,
                                                    2, None) == -1
    assert M.lib.mynah_hip_int8_product_noalloc_dev(13, c.w.ptr, rows, cols, c.x.ptr, c.y.ptr,
                                                    1, None) == -1
