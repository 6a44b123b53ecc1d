"""The exact GEMM's products on the matrix cores, over edge operands.

mynah_*_gemm_exact_mfma (csrc/gemm_mfma.hip) takes every product w[i] * x[i]
from v_mfma_f32_16x16x1_4b_f32 with a zero accumulator and adds it with its
own v_add_f32, where the reference (third_party/ingot/src/kernels.c:1017-1039,
2635-2648) multiplies and adds as two IEEE single roundings. That rests on:

* the zero-accumulator product equals the IEEE product a * b (numpy's float32
  multiply, what the reference's mulss gives) bit for bit, except that a -0
  product may come out +0 — a running sum that starts at +0 cannot tell the
  two apart (x + (+0) == x + (-0) for every x but -0, which such a sum never
  holds);
* the accumulate form D = A B + C is fused (it equals fmaf(a, b, c), one
  rounding) and so could not carry the reference's sums.

4096 waves of 1024 products each (4.2 million operand pairs): specials (zeros
of both signs, subnormals, the smallest and largest normals, infinities,
NaN), random bit patterns, pairs whose product lands at the subnormal and
overflow boundaries, and N(0, 1) values.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

WAVES = 4096
GROUP = WAVES // 4


def f32(bits):
    return np.asarray(bits, np.uint32).view(np.float32)


SPECIALS = np.concatenate([
    f32([0x00000000, 0x80000000,                      # +0, -0
         0x00000001, 0x80000001, 0x007FFFFF, 0x807FFFFF, 0x00400000,  # subnormals
         0x00800000, 0x80800000, 0x7F7FFFFF, 0xFF7FFFFF,  # min normal, max finite
         0x7F800000, 0xFF800000, 0x7FC00000]),        # +inf, -inf, NaN
    np.array([1.0, -1.0, 1.0 + 2.0 ** -23, 0.5, 3.0, 1e-20, -1e-20, 1e-30, 1e20, -1e20,
              2.0 ** 64, 2.0 ** -64, 1.5 * 2.0 ** -75, 2.0 ** 127], np.float32),
])


def operands(seed: int = 0):
    rng = np.random.default_rng(seed)
    n = 64 * GROUP
    # 1: specials against specials.
    a1, b1 = rng.choice(SPECIALS, n), rng.choice(SPECIALS, n)
    # 2: any bit pattern.
    a2 = f32(rng.integers(0, 1 << 32, n, dtype=np.uint64).astype(np.uint32))
    b2 = f32(rng.integers(0, 1 << 32, n, dtype=np.uint64).astype(np.uint32))
    # 3: products near the subnormal range and near overflow.
    ea = rng.integers(-80, 80, n)
    eb = np.where(rng.random(n) < 0.5, -140 - ea + rng.integers(-12, 14, n),
                  127 - ea + rng.integers(-2, 2, n))
    ma, mb = rng.uniform(1.0, 2.0, n), rng.uniform(1.0, 2.0, n)
    sa, sb = rng.choice([-1.0, 1.0], n), rng.choice([-1.0, 1.0], n)
    a3 = (sa * np.ldexp(ma, ea)).astype(np.float32)
    b3 = (sb * np.ldexp(mb, np.clip(eb, -149, 127))).astype(np.float32)
    # 4: the GEMM's own kind of operands.
    a4 = rng.standard_normal(n).astype(np.float32)
    b4 = rng.standard_normal(n).astype(np.float32)
    a = np.concatenate([a1, a2, a3, a4]).astype(np.float32)
    b = np.concatenate([b1, b2, b3, b4]).astype(np.float32)
    c = rng.standard_normal(1024 * WAVES).astype(np.float32)
    c[: 1024 * GROUP] = rng.choice(SPECIALS, 1024 * GROUP)
    return a, b, c


def pairs(a, b):
    """The operand pair of every output in the instruction's layout."""
    l = np.arange(64)[:, None]
    r = np.arange(16)[None, :]
    blk, row, col = r // 4, 4 * (l // 16) + r % 4, l % 16
    ia = (np.arange(WAVES)[:, None, None] * 64 + (16 * blk + row)[None]).reshape(-1)
    ib = (np.arange(WAVES)[:, None, None] * 64 + (16 * blk + col)[None]).reshape(-1)
    return a[ia], b[ib]


def run(M, a, b, c):
    bufs = [M.DeviceBuffer.from_array(v) for v in (a, b, c)]
    outs = [M.DeviceBuffer(4 * 1024 * WAVES) for _ in range(4)]
    M.check(M.lib.mynah_hip_mfma_probe(*[x.ptr for x in bufs], *[o.ptr for o in outs],
                                       WAVES, None), "mfma_probe")
    M.sync()
    res = [o.download(np.float32, 1024 * WAVES) for o in outs]
    for x in bufs + outs:
        x.free()
    return res


def same(got, want):
    """Equal bits, or both NaN."""
    gb, wb = got.view(np.uint32), want.view(np.uint32)
    return (gb == wb) | (np.isnan(got) & np.isnan(want))


def test_mfma_products_equal_ieee_products():
    import mynah_amd as M
    M.check(M.lib.mynah_hip_init(0), "init")
    print(f"[case] v_mfma_f32_16x16x1_4b_f32 on {WAVES} waves x 1024 products", flush=True)
    a, b, c = operands()
    prod, acc, mul, fused = run(M, a, b, c)
    x, y = pairs(a, b)
    with np.errstate(all="ignore"):
        want = x * y                                   # IEEE single products
        sep = (x * y) + c                              # multiply, then add
    # The VALU's product is the IEEE one (subnormals kept).
    assert same(mul, want).all()
    ok = same(prod, want)
    zeros = (prod == 0) & (want == 0)
    sign_only = ~ok & zeros
    print(f"zero-accumulator products: {int(ok.sum())} equal, {int(sign_only.sum())} zeros of "
          f"the other sign, {int((~ok & ~zeros).sum())} different; subnormal products "
          f"{int(((want != 0) & (np.abs(want) < np.float32(2.0 ** -126))).sum())}, "
          f"infinite {int(np.isinf(want).sum())}, NaN {int(np.isnan(want).sum())}", flush=True)
    assert (ok | sign_only).all()
    # Only a -0 product turns +0, never the other way.
    assert (want[sign_only].view(np.uint32) == 0x80000000).all()
    # The accumulate form is fused: fmaf's bits, and not multiply-then-add.
    fok = same(acc, fused) | ((acc == 0) & (fused == 0))
    differs = ~same(acc, sep) & np.isfinite(sep)
    print(f"accumulate form: {int(fok.sum())} of {fok.size} equal to fmaf; "
          f"{int(differs.sum())} differ from a * b + c", flush=True)
    assert fok.all()
    assert differs.sum() > fok.size // 20
