"""The kernels' test of a parallel-order double sum (mynah-slm_amd/csrc/
sum_settle.h, compiled for the host by oracle/settle_pin.c) against
index-order sums, on the CPU.

The reference's softmax reciprocal (float)(1 / sum) and RMSNorm scale
(float)(1 / sqrt(sum / n + eps)) come from double sums in index order
(/root/reference/src/kernels.c:207-220, 118-121). A kernel keeps the sum it
took in another order only where the test says every sum the reference's
order can give rounds to the same f32; otherwise it adds the terms again in
index order. Held here:

* the decision boundary: r at an f32 rounding midpoint plus m double ulps
  fails the test for |m| <= t and passes beyond, t = k2 (n - 1) plus its
  slack;
* soundness where the orders differ most: term sets whose index-order sum
  drops every small term (each below half an ulp of the running sum) while
  numpy's pairwise sum keeps most of them, with r placed within about t
  ulps of a midpoint. Whenever the two sums' f32 results differ, the test
  failed; such differences occur, and the orders' distance reaches a good
  part of t (so an interval much narrower than the bound would be caught);
* ordinary sums (normal scores' exponentials, squares of normal values):
  the test passes for all but a small fraction.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PIN = C.CDLL(os.path.join(ROOT, "oracle", "libsettle_pin.so"))
PIN.orc_sum_settled.restype = None
PIN.orc_sum_settled.argtypes = [C.c_void_p, C.c_size_t, C.c_uint32, C.c_uint32, C.c_void_p]
EPS = 1e-6


def settled(r, n, k2):
    r = np.ascontiguousarray(r, dtype=np.float64)
    out = np.empty(r.size, np.uint8)
    PIN.orc_sum_settled(r.ctypes.data, r.size, n, k2, out.ctypes.data)
    return out.astype(bool)


def slack(n, k2):
    w = k2 * (n - 1)
    return w + (w >> 18) + 13


def recip(s):
    return 1.0 / s


def rms(n):
    return lambda s: 1.0 / np.sqrt(s / n + EPS)


def midpoints(rng, count):
    """Doubles halfway between adjacent normal f32 values in [2^-8, 2^8)."""
    f = (rng.uniform(-8, 8, count).astype(np.float64))
    f = np.exp2(f).astype(np.float32)
    up = np.nextafter(f, np.float32(np.inf))
    return (f.astype(np.float64) + up.astype(np.float64)) / 2.0


@pytest.mark.parametrize("n", [2, 128, 1000, 2560, 8003])
@pytest.mark.parametrize("k2", [1, 2])
def test_boundary(n, k2):
    rng = np.random.default_rng(n * 7 + k2)
    m = midpoints(rng, 64).view(np.uint64)
    t = slack(n, k2)
    for off, want in ((0, False), (t, False), (-t, False), (t + 1, True), (-(t + 1), True),
                      (t + 1000, True), (1 << 27, True)):
        r = (m.astype(np.int64) + off).astype(np.uint64).view(np.float64)
        assert (settled(r, n, k2) == want).all(), (off, want)
        if want:
            # Passing means the f32 rounding is the same t ulps either way.
            lo = (m.astype(np.int64) + off - t).astype(np.uint64).view(np.float64)
            hi = (m.astype(np.int64) + off + t).astype(np.uint64).view(np.float64)
            assert (lo.astype(np.float32) == hi.astype(np.float32)).all()


def test_special_values():
    r = np.array([0.0, -1.0, np.inf, np.nan, 2.0 ** -126, 2.0 ** 127, 1.5, 2.0 ** -124])
    assert settled(r, 100, 2).tolist() == [False, False, False, False, False, False, True, True]
    assert not settled(np.array([1.5]), (1 << 20) + 1, 2)[0]


def floor_f32(x):
    """The largest f32 <= x (x >= 0, double)."""
    f = np.float32(x)
    return np.nextafter(f, np.float32(0)) if float(f) > x else f


def split_f32(x):
    """Non-negative f32 parts whose sum is x exactly in any order."""
    parts, rest = [], x
    while rest > 0.0 and len(parts) < 4:
        p = floor_f32(rest)
        parts.append(p)
        rest = rest - float(p)
    assert rest == 0.0
    return parts


def adversarial(rng, n, k2, trials):
    """(r from numpy's pairwise sum, r from the index-order sum) of term sets
    built to separate the two orders, r near an f32 midpoint."""
    fn = recip if k2 == 2 else rms(n)
    t = slack(n, k2)
    out_par, out_seq = [], []
    for mid in midpoints(rng, trials):
        target_r = float((np.array([mid]).view(np.uint64).astype(np.int64)
                          + int(rng.integers(-t, t + 1))).astype(np.uint64).view(np.float64)[0])
        s = 1.0 / target_r if k2 == 2 else n * (1.0 / (target_r * target_r) - EPS)
        big = split_f32(s)
        ulp = np.spacing(s)
        tiny = floor_f32(0.45 * ulp)
        m = n - len(big)
        terms = np.array(big + [tiny] * m, dtype=np.float32).astype(np.float64)
        out_par.append(fn(np.sum(terms)))
        out_seq.append(fn(np.cumsum(terms)[-1]))
    return np.array(out_par), np.array(out_seq)


@pytest.mark.parametrize("n", [128, 1000, 2560, 8003])
@pytest.mark.parametrize("k2", [1, 2])
def test_sound_where_orders_differ(n, k2):
    rng = np.random.default_rng(1000 + n + k2)
    r_par, r_seq = adversarial(rng, n, k2, 300)
    ok = settled(r_par, n, k2)
    differ = r_par.astype(np.float32) != r_seq.astype(np.float32)
    assert not (ok & differ).any()
    assert differ.sum() >= 3, "no near-midpoint difference produced"
    dist = np.abs(r_par.view(np.int64) - r_seq.view(np.int64))
    assert dist.max() >= 0.1 * slack(n, k2), (dist.max(), slack(n, k2))
    print(f"n {n} k2 {k2}: {differ.sum()} of {r_par.size} differ, all refused; "
          f"order distance up to {dist.max()} ulps of t = {slack(n, k2)}; "
          f"passed {ok.sum()}")


def test_ordinary_sums_mostly_pass():
    rng = np.random.default_rng(5)
    n, rows = 2080, 2000
    sc = rng.normal(0.0, 3.0, (rows, n)).astype(np.float32)
    e = np.exp(sc - sc.max(axis=1, keepdims=True)).astype(np.float64)
    ok_soft = settled(1.0 / e.sum(axis=1), n, 2)
    x = rng.normal(0.0, 1.0, (rows, 2560)).astype(np.float32).astype(np.float64)
    ok_rms = settled(1.0 / np.sqrt((x * x).sum(axis=1) / 2560 + EPS), 2560, 1)
    assert ok_soft.mean() > 0.995 and ok_rms.mean() > 0.995
