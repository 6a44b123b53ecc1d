"""GPU parity of the gfx950 GEMV / dequant / matmat kernels through the C ABI.

The default (exact-order) GEMVs must be BIT-IDENTICAL to the oracle, which is
itself bit-identical to the compiled reference (test_oracle.py). That is
stricter than the reference's 1e-4 metric (|gpu - ref| / max(1, |ref|),
third_party/ingot/tests/test_quant.c:143-152), which the tests also assert.
The reordered GEMVs are held to the f32 summation error bound against an f64
dot of the exactly decoded weights. Dequant is bit-identical; layout
invariance is checked with memcmp.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

import configs as CF
import oracle_lib as O

pytestmark = pytest.mark.gpu

TOL = 1e-4
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def M():
    import mynah_amd
    mynah_amd.check(mynah_amd.lib.mynah_hip_init(0), "init")
    mynah_amd.check(mynah_amd.lib.mynah_hip_set_gemv_order(0), "order")
    O.orc.orc_threads_init(0)
    return mynah_amd


def same(got, ref) -> bool:
    """Bit-identical, and (redundantly) within the reference's 1e-4 metric."""
    return np.array_equal(bits(got), bits(ref)) and rel_err(got, ref) <= TOL


def rel_err(got, ref):
    return float((np.abs(got.astype(np.float64) - ref) / np.maximum(1.0, np.abs(ref))).max())


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def case(M, qtype, rows, cols, seed=1):
    print(f"[case] type={qtype} rows={rows} cols={cols} seed={seed}", flush=True)
    w = M.synth_blocks(qtype, seed, rows, cols)
    x = M.synth_normal(seed + 1, cols)
    return w, x


def test_c1_q4k_config(M):
    g = np.load(os.path.join(GOLDEN, "c1.npz"), allow_pickle=False)
    m = CF.C1[0]
    ws, xs = CF.matrix_seeds(M.substream, 0, 0)
    w, x = M.synth_blocks(m.qtype, ws, m.rows, m.cols), M.synth_normal(xs, m.cols)
    y = M.matvec(m.qtype, w, m.rows, m.cols, x)
    assert same(y, g["y"])


def test_c2_sweep_against_oracle(M):
    g = np.load(os.path.join(GOLDEN, "c2.npz"), allow_pickle=False)
    for i, m in enumerate(CF.C2):
        print(f"[case] {m.name}", flush=True)
        ws, xs = CF.matrix_seeds(M.substream, 0, i)
        w, x = M.synth_blocks(m.qtype, ws, m.rows, m.cols), M.synth_normal(xs, m.cols)
        y = M.matvec(m.qtype, w, m.rows, m.cols, x)
        ref = O.project(m.qtype, w, m.rows, m.cols, x)
        assert same(y, ref), m.name
        assert same(y[::97], g[f"{m.name}_y_every97"])


@pytest.mark.parametrize("qtype", [12, 14, 8])
@pytest.mark.parametrize("rows,cols", [(1, 256), (7, 512), (37, 1024), (64, 2048), (333, 3072),
                                       (1025, 4096), (2049, 2560), (100, 9728)])
def test_shapes_against_oracle(M, qtype, rows, cols):
    w, x = case(M, qtype, rows, cols)
    y = M.matvec(qtype, w, rows, cols, x)
    assert same(y, O.matvec(qtype, w, rows, cols, x))


def test_q80_ragged_rows(M):
    for cols in (32, 96, 224, 1056):
        w, x = case(M, 8, 19, cols)
        assert same(M.matvec(8, w, 19, cols, x), O.matvec(8, w, 19, cols, x))


@pytest.mark.parametrize("m", CF.QWEN3_4B_GEMV, ids=lambda m: m.name)
def test_qwen3_4b_shapes(M, m):
    w, x = case(M, m.qtype, m.rows, m.cols, seed=11)
    y = M.matvec(m.qtype, w, m.rows, m.cols, x)
    assert same(y, O.project(m.qtype, w, m.rows, m.cols, x))


PC_SHAPES = [(4096, 2560), (1024, 2560), (2560, 4096), (9728, 2560), (2560, 9728),
             (1000, 256), (37, 256 * 40), (130, 256 * 33), (3, 2560)]


@pytest.mark.parametrize("rows,cols", PC_SHAPES)
def test_producer_consumer_layout_bit_exact(M, monkeypatch, rows, cols):
    """The producer/consumer Q4_K GEMV (gemv_pc.hip, forced on with
    MYNAH_GEMV_PC=1): the Qwen3-4B shapes, one-unit rows (64 rows per
    workgroup), rows of 40 and 33 units (one row per workgroup) and a
    ragged last workgroup, against the oracle bit for bit."""
    monkeypatch.setenv("MYNAH_GEMV_PC", "1")
    assert M.gemv_kernel(12, rows, cols, 0) == "mynah_gemv_pc_q4k"
    w, x = case(M, 12, rows, cols, seed=13)
    ref = O.project(12, w, rows, cols, x)
    assert same(M.matvec(12, w, rows, cols, x), ref)


@pytest.mark.parametrize("qtype", [12, 14, 8])
def test_dequant_bit_exact(M, qtype):
    rows, cols = 77, 1536
    w, _ = case(M, qtype, rows, cols)
    assert np.array_equal(bits(M.dequant(qtype, w, rows, cols)), bits(O.dequant(qtype, w, rows, cols)))


def test_dequant_matches_llama_cpp_fixtures(M):
    fx = os.path.join(GOLDEN, "ingot_fixtures")
    for name, t in (("Q4_K", 12), ("Q6_K", 14), ("Q8_0", 8)):
        raw = np.fromfile(os.path.join(fx, f"{name}.bin"), dtype=np.uint8)
        ref = np.fromfile(os.path.join(fx, f"{name}.ref"), dtype=np.float32)
        rows = ref.size // 256
        assert np.array_equal(bits(M.dequant(t, raw, rows, 256)), bits(ref)), name


def test_ragged_q80_refused_like_reference(M):
    w, x = case(M, 8, 4, 96)
    y = np.empty(4 * 96 * 3, np.float32)
    assert M.lib.ingot_dequant_matrix(8, M.ptr(w), 4, 96, M.ptr(y)) == -1
    assert M.lib.ingot_matmat(8, M.ptr(w), 4, 96, M.ptr(np.zeros(288, np.float32)),
                              M.ptr(y), 3) == -1


@pytest.mark.parametrize("qtype", [12, 14, 8])
def test_matmat_against_oracle(M, qtype):
    rows, cols, tokens = 96, 1024, 5
    w, _ = case(M, qtype, rows, cols)
    x = M.synth_normal(3, tokens * cols)
    y = M.matmat(qtype, w, rows, cols, x, tokens)
    assert same(y, O.matmat(qtype, w, rows, cols, x, tokens))
    # tokens == 1 is the matvec, bit for bit (test_quant.c:199-203)
    assert np.array_equal(bits(M.matmat(qtype, w, rows, cols, x, 1)),
                          bits(M.matvec(qtype, w, rows, cols, x[:cols])))


@pytest.mark.parametrize("qtype,rows,cols,tokens", [(12, 100, 2048, 70), (14, 72, 1536, 65),
                                                    (8, 130, 512, 3), (12, 64, 256, 64),
                                                    (14, 1, 256, 2)])
def test_gemm_ragged_tiles(M, qtype, rows, cols, tokens):
    """The tiled batched GEMM on shapes that leave partial row and token
    tiles, bit-identical to the batched reference order."""
    w, _ = case(M, qtype, rows, cols, seed=rows + tokens)
    x = M.synth_normal(7 + tokens, tokens * cols)
    assert same(M.matmat(qtype, w, rows, cols, x, tokens), O.matmat(qtype, w, rows, cols, x, tokens))


@pytest.mark.parametrize("name", [m.name for m in CF.C4])
def test_gemm_configs3_shapes(M, name):
    """All six configs[3] prefill GEMMs (512 tokens) against the oracle's
    threaded batched path, bit for bit."""
    print(f"[case] configs[3] GEMM {name}", flush=True)
    m = next(m for m in CF.C4 if m.name == name)
    i = CF.C4.index(m)
    ws, xs = CF.matrix_seeds(M.substream, 0, i)
    w, _ = case(M, m.qtype, m.rows, m.cols, seed=ws)
    x = M.synth_normal(M.substream(0, CF.PREFILL_X_INDEX + i), CF.C4_TOKENS * m.cols)
    O.orc.orc_threads_init(0)
    ref = O.matmat(m.qtype, w, m.rows, m.cols, x, CF.C4_TOKENS, threaded=True)
    assert same(M.matmat(m.qtype, w, m.rows, m.cols, x, CF.C4_TOKENS), ref)


def test_matmat_golden(M):
    g = np.load(os.path.join(GOLDEN, "matmat.npz"), allow_pickle=False)
    for t, rows, cols, tokens in ((12, 64, 2048, 16), (14, 32, 6144, 8), (8, 40, 1024, 5)):
        key = f"{CF.TYPE_NAME[t]}_{rows}x{cols}_t{tokens}"
        w, x = M.synth_blocks(t, 300 + t, rows, cols), M.synth_normal(400 + t, tokens * cols)
        assert same(M.matmat(t, w, rows, cols, x, tokens), g[f"{key}_y"]), key


@pytest.mark.parametrize("qtype,shifts", [(12, (0, 16, 32, 48, 256)), (14, (0, 2, 4, 6, 210)),
                                          (8, (0, 2, 4, 6, 34))])
def test_address_invariance(M, qtype, shifts):
    """Same bytes at different HBM offsets give identical outputs (memcmp)."""
    rows, cols = 130, 2048
    w, x = case(M, qtype, rows, cols)
    buf = M.DeviceBuffer(w.nbytes + 512)
    xd = M.DeviceBuffer.from_array(x)
    yd = M.DeviceBuffer(rows * 4)
    outs = []
    for s in shifts:
        buf.upload(w, offset=s)
        M.matvec_dev(qtype, buf.ptr + s, rows, cols, xd.ptr, yd.ptr)
        M.sync()
        outs.append(yd.download(np.float32, rows))
    for o in outs[1:]:
        assert np.array_equal(bits(o), bits(outs[0]))
    assert np.array_equal(bits(outs[0]), bits(M.matvec(qtype, w, rows, cols, x)))


def test_registered_weights_are_used_in_place(M):
    rows, cols = 512, 1024
    w, x = case(M, 12, rows, cols)
    y0 = M.matvec(12, w, rows, cols, x)
    M.check(M.lib.mynah_hip_register(M.ptr(w), w.nbytes), "register")
    try:
        dev = M.lib.mynah_hip_device_ptr(M.ptr(w))
        assert dev and (dev - M.ptr(w)) % 256 == 0
        # a row chunk inside the registered range, as project() passes it
        half = rows // 2
        rb = M.row_bytes(12, cols)
        y1 = np.empty(half, np.float32)
        M.check(M.lib.ingot_matvec(12, M.ptr(w) + half * rb, half, cols, M.ptr(x), M.ptr(y1)))
        assert np.array_equal(bits(y1), bits(y0[half:]))
    finally:
        M.check(M.lib.mynah_hip_unregister(M.ptr(w)), "unregister")


def test_misaligned_x_is_refused(M):
    xd = M.DeviceBuffer(4096 + 64)
    wd = M.DeviceBuffer(144 * 4)
    yd = M.DeviceBuffer(64)
    assert M.lib.mynah_hip_matvec_dev(12, wd.ptr, 1, 1024, xd.ptr + 4, yd.ptr, None) == -1
    assert b"aligned" in M.lib.mynah_hip_last_error()


@pytest.mark.parametrize("qtype", [12, 14, 8])
def test_reordered_order_within_f32_bound(M, qtype):
    rows, cols = 777, 2560
    w, x = case(M, qtype, rows, cols, seed=21)
    M.check(M.lib.mynah_hip_set_gemv_order(1), "order")
    try:
        y = M.matvec(qtype, w, rows, cols, x).astype(np.float64)
    finally:
        M.check(M.lib.mynah_hip_set_gemv_order(0), "order")
    dq = O.dequant(qtype, w, rows, cols).reshape(rows, cols).astype(np.float64)
    exact = dq @ x.astype(np.float64)
    mag = np.abs(dq) @ np.abs(x.astype(np.float64))
    assert (np.abs(y - exact) <= (cols + 1) * 2.0 ** -24 * mag).all()


def test_kernel_query_names_the_planned_kernel(M):
    """mynah_hip_gemv_kernel answers from the launch's own plan: the exact
    order's flat or streaming kernels, the reordered kernel, Q4_0's chains;
    refused geometry gives NULL with the reason."""
    exact = {"mynah_gemv_flat_q4k", "mynah_gemv_flat_q6k", "mynah_gemv_group", "mynah_gemv_pc_q4k",
             "mynah_gemv_group_q4k", "mynah_gemv_group_q6k", "mynah_gemv_stream",
             "mynah_gemv_stream_cvt"}
    for qtype, rows, cols in ((12, 1024, 3072), (14, 151936, 1024), (14, 151936, 2560),
                              (12, 9728, 2560), (8, 1024, 2048)):
        assert M.gemv_kernel(qtype, rows, cols, 0) in exact
        assert M.gemv_kernel(qtype, rows, cols, 1) == "mynah_gemv_fast_group"
    assert M.gemv_kernel(2, 1024, 1024).startswith("mynah_q40_chain")
    assert M.lib.mynah_hip_gemv_kernel(12, 1024, 100, 0) is None
    assert b"geometry" in M.lib.mynah_hip_last_error()


@pytest.mark.parametrize("qtype", [12, 13, 14, 8])
@pytest.mark.parametrize("mv", [False, True])
def test_mfma_gemm_equals_valu_gemm(M, qtype, mv):
    """The exact GEMM with its products on MFMA (the default) against the
    VALU kernels (MYNAH_GEMM_MFMA=0), bit for bit, with and without the
    split over super-blocks (forced 3 ways, and off) and, in the matvec
    order, the residual epilogue; ragged rows and token counts around the
    64-token tile. The products of v_mfma_f32_16x16x1_4b_f32 with a zero
    accumulator are v_mul_f32's (a -0 comes out +0, which no sum here can
    see)."""
    keys = ("MYNAH_GEMM_MFMA", "MYNAH_GEMM_SPLIT", "MYNAH_GEMM_WGS_PER_CU")
    saved = {k: os.environ.get(k) for k in keys}

    def run(env, rows, cols, tokens, res):
        for k in keys:
            os.environ.pop(k, None)
        os.environ.update(env)
        w = M.DeviceBuffer.from_array(M.synth_blocks(qtype, 5, rows, cols))
        x = M.DeviceBuffer.from_array(M.synth_normal(9, tokens * cols))
        y = M.DeviceBuffer(4 * rows * tokens)
        r = M.DeviceBuffer.from_array(M.synth_normal(11, tokens * rows)) if res else None
        try:
            if mv:
                M.check(M.lib.mynah_hip_matmat_mv_dev(qtype, w.ptr, rows, cols, x.ptr, y.ptr,
                                                      tokens, r.ptr if r else None, None), "mv")
            else:
                M.check(M.lib.mynah_hip_matmat_dev(qtype, w.ptr, rows, cols, x.ptr, y.ptr,
                                                   tokens, None), "matmat")
            M.sync()
            return y.download(np.float32, rows * tokens)
        finally:
            for b in (w, x, y, r):
                if b is not None:
                    b.free()

    try:
        for rows, cols, tokens in ((100, 512, 2), (64, 256, 65), (300, 1024, 130),
                                   (2048, 2048, 512)):
            for res in ((False, True) if mv else (False,)):
                print(f"[case] type={qtype} mv={mv} {rows}x{cols} tokens={tokens} res={res}",
                      flush=True)
                ref = run({"MYNAH_GEMM_MFMA": "0"}, rows, cols, tokens, res)
                for env in ({}, {"MYNAH_GEMM_SPLIT": "0"}, {"MYNAH_GEMM_SPLIT": "3"}):
                    got = run(env, rows, cols, tokens, res)
                    assert np.array_equal(bits(got), bits(ref)), (rows, cols, tokens, res, env)
    finally:
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


def test_valu_add_yardstick(M):
    """The VALU yardstick runs and reports a plausible time per wave64 add
    (a non-packed f32 add takes 4 cycles of a 16-lane SIMD: 1.6-2.5 ns at the
    MI355X's clocks) and the device's SIMD count."""
    ns, simds = M.valu_add_rate(2000)
    assert 0.5 < ns < 10.0 and simds % 4 == 0 and simds >= 4
