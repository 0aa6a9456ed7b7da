"""Pins of the oracle's host-side parameter maths (``oracle/pipeline.py``).

Known answers are those the reference's own test-suite asserts
(``quantization/tests/test_utils.py:16-114``,
``quantization/tests/test_native.py:83-86``); closed forms use exact rational
arithmetic, so that a dropped rounding step, a wrong sign or an off-by-one
exponent fails here. The product's host maths (``quantanything_amd.utils``)
must agree with the pinned oracle.
"""

from fractions import Fraction

import numpy as np
import pytest

from oracle import pipeline as P
from quantanything_amd import utils as U


def test_quant_type_ranges():
    assert P.quant_type_info("int8") == (8, True, -128, 127)
    assert P.quant_type_info("uint8") == (8, False, 0, 255)
    assert P.quant_type_info("int9") == (9, True, -256, 255)
    assert P.quant_type_info("uint12") == (12, False, 0, 4095)
    assert P.quant_type_info("int16") == (16, True, -32768, 32767)


def test_scale_zp_known_answers():
    s, z = P.scale_zp(-10.0, 10.0, "int8")
    assert z == 0 and s == pytest.approx(10.0 / 127.0)
    s, z = P.scale_zp(-2.0, 8.0, "uint8")
    assert s == pytest.approx(10.0 / 255.0) and z == int(np.round(2.0 / s))
    s, z = P.scale_zp(2.0, 10.0, "uint8")  # range widened to contain 0
    assert z == 0 and s == pytest.approx(10.0 / 255.0)
    s, z = P.scale_zp(-100.0, 50.0, "int9")
    assert z == 0 and s == pytest.approx(100.0 / 255.0)
    assert P.scale_zp(0.0, 0.0, "int8") == (1.0, 0)
    assert P.scale_zp(0.0, 0.0, "uint8") == (1.0, 0)


def test_quantize_known_answers():
    x = np.array([0.5, 1.5, 2.5, -0.5, -1.5], np.float32)
    np.testing.assert_array_equal(P.quantize_np(x, 1.0, 0, -128, 127),
                                  [0, 2, 2, 0, -2])  # half to even
    np.testing.assert_array_equal(
        P.quantize_np(np.array([1e6, -1e6], np.float32), 0.1, 0, -128, 127),
        [127, -128])
    np.testing.assert_array_equal(
        P.quantize_np(np.ones((2, 3), np.float32), np.array([[0.5], [0.25]]),
                      np.array([[0], [0]]), -128, 127),
        [[2] * 3, [4] * 3])


def _exact_multiplier(real):
    """(M0, shift) from exact rationals: M0 = round_half_even(f * 2^31)
    for real = f * 2^e with f in [0.5, 1), renormalised when it reaches
    2^31; shift = -e."""
    if real == 0:
        return 0, 0
    sign = -1 if real < 0 else 1
    r = Fraction(abs(real))
    e = 0
    while r >= 1:
        r /= 2
        e += 1
    while r < Fraction(1, 2):
        r *= 2
        e -= 1
    m = round(r * (1 << 31))  # Fraction rounds half to even
    if m == 1 << 31:
        m //= 2
        e += 1
    return sign * m, -e


@pytest.mark.parametrize("real", [1e-5, 0.0123, 0.5, 1.0, 3.7, 250.0, -0.3,
                                  1 - 2.0**-40, 0.75 + 2.0**-33, 2.0**-60])
def test_multiplier_closed_form(real):
    m, s = P.multiplier(real)
    assert (m, s) == _exact_multiplier(real)
    assert 2**30 <= abs(m) < 2**31
    assert m * 2.0 ** -(31 + s) == pytest.approx(real, rel=1e-8)
    assert U.quantize_multiplier(real) == (m, s)


def test_multiplier_zero_and_renormalisation():
    assert P.multiplier(0.0) == (0, 0)
    # the significand of 1 - 2^-40 rounds up to 2^31: halved, exponent + 1
    assert P.multiplier(1 - 2.0**-40) == (1 << 30, -1)


def test_accumulator_width_rule():
    assert not P.wide_accumulator(8, 3 * 3 * 256)
    assert P.wide_accumulator(8, 1 << 20)
    assert P.wide_accumulator(16, 1)
    # boundary: (2^8)^2 * K >= 2^31  <=>  K >= 32768
    assert not P.wide_accumulator(8, 32767)
    assert P.wide_accumulator(8, 32768)


def test_product_host_maths_agree_with_oracle():
    rng = np.random.default_rng(11)
    for qt in ("int8", "uint8", "int16", "uint16", "int9"):
        for _ in range(50):
            lo, hi = sorted(rng.normal(0, 3, 2))
            s_o, z_o = P.scale_zp(lo, hi, qt)
            s_p, z_p, qmin, qmax = U.calculate_scale_zp(lo, hi, qt)
            assert (s_p, z_p) == (s_o, z_o)
            x = rng.normal(0, 3, 64).astype(np.float32)
            np.testing.assert_array_equal(
                U.quantize(x, s_o, z_o, qmin, qmax),
                P.quantize_np(x, s_o, z_o, qmin, qmax))
