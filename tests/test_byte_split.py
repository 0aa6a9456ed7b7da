"""The byte-split form of 16-bit convolutions (int8 matrix cores): the
weight packer, the decomposition the kernel sums and the epilogue's float64
requantization, checked on the CPU.

A stored activation x (int16) is 256 xh + xl + 128 with xh = x >> 8 and
xl = (x & 255) - 128, both int8; a centred weight w likewise. Over the
positions of one output (zero weights where the packed layout has no
weight, the stored zero point -x_add outside the image):

    sum (x + x_add) w = 65536 Hh + 256 (Hl + Lh) + Ll + 128 U
                        + (128 + x_add) W

with Hh = sum xh wh, ..., U = sum (256 xh + xl), W = sum w. The identity is
checked against the direct int64 sum (the reference's 16-bit convolution
accumulates exactly: qa_kernels.cpp:281-284), on random and extreme int16
values, so that a dropped term, a wrong sign or a wrong offset fails."""

import ctypes

import numpy as np
import pytest

from quantanything_amd import native


def _lib():
    if not native.available():
        pytest.skip(f"library not built: {native.load_error()}")
    return native.library()


def _split(v):
    v = np.asarray(v, np.int64)
    return v >> 8, (v & 255) - 128


@pytest.mark.parametrize("cout,cg,kh,kw,g", [
    (20, 32, 3, 3, 1),   # rows and k-groups padded
    (8, 16, 1, 1, 2),    # two groups
    (5, 48, 2, 3, 1),    # 3 channel blocks a tap
])
def test_pack_planes_reconstruct_the_weights(cout, cg, kh, kw, g):
    lib = _lib()
    rng = np.random.default_rng(cout * 100 + cg)
    w = rng.integers(-32768, 32768, size=(cout, cg, kh, kw)).astype(np.int32)
    w.flat[0], w.flat[1] = -32768, 32767  # the int16 extremes
    kgp, rows = ctypes.c_int64(0), ctypes.c_int64(0)
    n = lib.qa_pack_weights_i8_size(cout, cg, kh, kw, g, 0,
                                    ctypes.byref(kgp), ctypes.byref(rows))
    wp = np.empty(2 * n, np.int8)
    wsum = np.empty(cout, np.int64)
    assert lib.qa_pack_weights_i16s(w.ctypes.data, cout, cg, kh, kw, g,
                                    wp.ctypes.data, wsum.ctypes.data) == 0
    kgp, rows = kgp.value, rows.value
    cb = -(-cg // 16)
    hi = wp[:n].astype(np.int64).reshape(g, rows, kgp * 16)
    lo = wp[n:].astype(np.int64).reshape(g, rows, kgp * 16)
    full = hi * 256 + lo + 128  # the weight each position stands for
    want = np.zeros_like(full)
    cog = cout // g
    for co in range(cout):
        for c in range(cg):
            for ky in range(kh):
                for kx in range(kw):
                    at = ((ky * kw + kx) * cb + c // 16) * 16 + c % 16
                    want[co // cog, co % cog, at] = w[co, c, ky, kx]
    np.testing.assert_array_equal(full, want)  # zero where no weight sits
    np.testing.assert_array_equal(
        wsum, w.reshape(cout, -1).astype(np.int64).sum(1))


def test_pack_rejects_weights_outside_int16():
    lib = _lib()
    w = np.array([[[[32768]]]], np.int32)
    kgp, rows = ctypes.c_int64(0), ctypes.c_int64(0)
    n = lib.qa_pack_weights_i8_size(1, 1, 1, 1, 1, 0, ctypes.byref(kgp),
                                    ctypes.byref(rows))
    wp = np.empty(2 * n, np.int8)
    wsum = np.empty(1, np.int64)
    assert lib.qa_pack_weights_i16s(w.ctypes.data, 1, 1, 1, 1, 1,
                                    wp.ctypes.data, wsum.ctypes.data) == 1


@pytest.mark.parametrize("seed", range(6))
def test_decomposition_equals_the_direct_sum(seed):
    rng = np.random.default_rng(seed)
    kp = 16 * int(rng.integers(1, 40))      # K' positions of one output
    x_add = int(rng.integers(-32767, 32769))
    x = rng.integers(-32768, 32768, size=kp)
    w = rng.integers(-32768, 32768, size=kp)
    if seed % 2:  # extremes
        x[: kp // 4] = rng.choice([-32768, 32767], size=kp // 4)
        w[: kp // 4] = rng.choice([-32768, 32767], size=kp // 4)
    # positions without a weight (any x), and image padding (x = -x_add)
    nw = rng.random(kp) < 0.2
    w[nw] = 0
    pad = rng.random(kp) < 0.1
    x[pad & ~nw] = -x_add
    want = int(((x + x_add) * w).sum())
    xh, xl = _split(x)
    wh, wl = _split(w)
    hh = int((xh * wh).sum())
    mid = int((xh * wl).sum() + (xl * wh).sum())
    lo = int((xl * wl).sum())
    u = int((256 * xh + xl).sum())
    wsum = int(w.sum())
    got = 65536 * hh + 256 * mid + lo + 128 * u + (128 + x_add) * wsum
    assert got == want
    # the int8 sums stay inside int32 for K' < 2^16
    assert max(abs(hh), abs(mid), abs(lo)) < 2 ** 31
    assert ((xh >= -128) & (xh <= 127) & (xl >= -128) & (xl <= 127)).all()


def _mbqm(x, m, s):
    """The reference's fixed-point multiply (qa_kernels.cpp:188-205):
    round half up of x m 2^-(31+s), exact in Python integers."""
    ts = 31 + s
    p = x * m
    if ts > 0:
        ts = min(ts, 120)
        return (p + (1 << (ts - 1))) >> ts
    return p << min(-ts, 60)


def _fma_double(a, b, c):
    """fma(a, b, c) on doubles: the exact a b + c rounded once to the
    nearest double (Python's float() of a Fraction rounds correctly)."""
    from fractions import Fraction
    return float(Fraction(a) * Fraction(b) + Fraction(c))


@pytest.mark.parametrize("seed", range(4))
def test_float64_requantize_form_is_exact(seed):
    """The 16-bit epilogue's float64 requantization: y = fma(x, m 2^-ts,
    1/2 + zp), floor(y) clipped, except where frac(y) lies within 2^-30 of
    0 or 1 below |y| = 2^20 (those take the 128-bit form). Every value the
    guard lets through equals the exact clip(mbqm(x) + zp); exact ties (x m
    a multiple of 2^(ts-1)) are all flagged."""
    import math
    rng = np.random.default_rng(100 + seed)
    flagged = 0
    for _ in range(3000):
        m = int(rng.integers(1 << 29, 1 << 31)) * int(rng.choice([1, -1]))
        s = int(rng.integers(-30, 40))
        ts = 31 + s
        if not 1 <= ts <= 120:
            continue
        zp = int(rng.integers(-32768, 32768))
        lo, hi = -32768, 32767
        if rng.random() < 0.3:  # an exact tie: x m = (2k + 1) 2^(ts-1)
            if ts - 1 > 62:
                continue
            # x = (2k + 1) 2^(ts-1) / m needs m | ...: use m a power of two
            m = (1 << int(rng.integers(0, 31))) * int(rng.choice([1, -1]))
            k = int(rng.integers(-4000, 4000))
            num = (2 * k + 1) << (ts - 1)
            if num % m:
                continue
            x = num // m
        else:
            x = int(rng.integers(-(1 << 45), 1 << 45))
        if abs(x) >= 1 << 53:
            continue
        md = math.ldexp(float(m), -ts)  # exact: |m| < 2^31
        y = _fma_double(float(x), md, 0.5 + zp)
        f = math.floor(y)
        fr = y - f
        near = (fr < 2.0 ** -30 or fr > 1 - 2.0 ** -30) and abs(y) < 2.0 ** 20
        want = min(max(_mbqm(x, m, s) + zp, lo), hi)
        if near:
            flagged += 1
            continue
        assert min(max(f, lo), hi) == want, (x, m, s, zp)
        # an exact tie never passes the guard
        assert (x * m) % (1 << (ts - 1)) or (x * m) % (1 << ts) == 0 \
            or abs(y) >= 2.0 ** 20, (x, m, s)
    assert flagged > 0
