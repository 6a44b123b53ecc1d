"""GPU parity of the streaming exact GEMV (gemv_stream.hip) through the C ABI.

Single large Q4_K / Q6_K matrices (>= 131,072 super-blocks, rows of >= 8
super-blocks; here any row length) take the persistent streaming kernel; its
outputs must be BIT-IDENTICAL to the oracle
(itself bit-identical to the compiled reference, test_oracle.py), in both
weight-value forms (v_cvt_f32_ubyte, the default, and v_fma_mix_f32 on
f16-subnormal quant codes, MYNAH_GEMV_MIX=1), for every row partition
(MYNAH_STREAM_WGS), odd super-block counts per row, and blocks of random
bytes (subnormal, negative and zero f16 scales, every 6-bit scale code).
"""
from __future__ import annotations

import os

import numpy as np
import pytest

import oracle_lib as O

pytestmark = pytest.mark.gpu

TOL = 1e-4
BLOCK = {12: (256, 144), 14: (256, 210)}


@pytest.fixture(scope="module")
def M():
    import mynah_amd
    mynah_amd.check(mynah_amd.lib.mynah_hip_init(0), "init")
    mynah_amd.check(mynah_amd.lib.mynah_hip_set_gemv_order(0), "order")
    O.orc.orc_threads_init(0)
    return mynah_amd


@pytest.fixture(autouse=True)
def env():
    """Environment switches of the launch, restored after each test. Every
    test here routes single large matrices to the streaming kernel whatever
    their row length (by default only rows of >= 8 super-blocks take it)."""
    saved = {}

    def set_(name, value):
        if name not in saved:
            saved[name] = os.environ.get(name)
        os.environ[name] = str(value)

    set_("MYNAH_STREAM_MIN_ROW_UNITS", 1)
    yield set_
    for name, value in saved.items():
        if value is None:
            os.environ.pop(name, None)
        else:
            os.environ[name] = value


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def same(got, ref) -> bool:
    err = float((np.abs(got.astype(np.float64) - ref) / np.maximum(1.0, np.abs(ref))).max())
    return np.array_equal(bits(got), bits(ref)) and err <= TOL


def random_blocks(qtype: int, rows: int, cols: int, seed: int) -> np.ndarray:
    """Blocks of uniformly random bytes with every f16 field finite: d / dmin
    (Q4_K) and d (Q6_K) take any sign, subnormals and zero included."""
    e, b = BLOCK[qtype]
    rng = np.random.default_rng(seed)
    w = rng.integers(0, 256, size=(rows * (cols // e), b), dtype=np.uint8)
    offs = (0, 2) if qtype == 12 else (208,)
    for o in offs:
        h = w[:, o:o + 2].copy().view(np.uint16)
        inf_nan = (h & 0x7C00) == 0x7C00
        h[inf_nan] &= 0xBFFF                        # clear an exponent bit
        w[:, o:o + 2] = h.view(np.uint8).reshape(-1, 2)
    return w.reshape(-1)


def run(M, qtype, w, rows, cols, x):
    print(f"[stream] type={qtype} rows={rows} cols={cols} "
          f"mix={os.environ.get('MYNAH_GEMV_MIX', '0')} "
          f"wgs={os.environ.get('MYNAH_STREAM_WGS', 'default')}", flush=True)
    return M.matvec(qtype, w, rows, cols, x)


@pytest.mark.parametrize("mix", [1, 0])
@pytest.mark.parametrize("qtype,rows,cols", [(12, 32768, 1024), (14, 65537, 512),
                                             (14, 50001, 768), (12, 12289, 2816)])
def test_stream_synthetic(M, env, mix, qtype, rows, cols):
    env("MYNAH_GEMV_MIX", mix)
    assert rows * (cols // 256) >= 131072
    w = M.synth_blocks(qtype, 21, rows, cols)
    x = M.synth_normal(22, cols)
    assert same(run(M, qtype, w, rows, cols, x), O.project(qtype, w, rows, cols, x))


@pytest.mark.parametrize("mix", [1, 0])
@pytest.mark.parametrize("qtype", [12, 14])
def test_stream_random_bytes(M, env, mix, qtype):
    env("MYNAH_GEMV_MIX", mix)
    rows, cols = 40000, 1024
    w = random_blocks(qtype, rows, cols, 5 + qtype)
    x = M.synth_normal(31, cols)
    assert same(run(M, qtype, w, rows, cols, x), O.project(qtype, w, rows, cols, x))


@pytest.mark.parametrize("wgs", [64, 256, 513, 1024, 4096])
def test_stream_partitions(M, env, wgs):
    env("MYNAH_STREAM_WGS", wgs)
    rows, cols = 33333, 1024
    for qtype in (12, 14):
        w = M.synth_blocks(qtype, 41, rows, cols)
        x = M.synth_normal(42, cols)
        assert same(run(M, qtype, w, rows, cols, x), O.project(qtype, w, rows, cols, x))


def test_stream_long_rows_default_route(M, env):
    """Rows of 10 super-blocks take the streaming kernel with no override."""
    os.environ.pop("MYNAH_STREAM_MIN_ROW_UNITS", None)
    rows, cols = 16384, 2560
    for qtype in (12, 14):
        w = M.synth_blocks(qtype, 51, rows, cols)
        x = M.synth_normal(52, cols)
        assert same(run(M, qtype, w, rows, cols, x), O.project(qtype, w, rows, cols, x))


def test_stream_matches_grouped_kernel(M, env):
    """The same matrix through the streaming and the grouped kernel."""
    rows, cols = 151936, 1024
    w = M.synth_blocks(14, 3, rows, cols)
    x = M.synth_normal(4, cols)
    y_stream = run(M, 14, w, rows, cols, x)
    env("MYNAH_GEMV_STREAM", 0)
    y_group = run(M, 14, w, rows, cols, x)
    assert np.array_equal(bits(y_stream), bits(y_group))
