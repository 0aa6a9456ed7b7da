"""Pins of the oracle's parameter derivations that no golden vector covers:
activation tables (quant_layers.py:461-468 over float_ops.py:225-227,
:251-253, :230-232), the GlobalAveragePool multiplier (quant_layers.py:
575-577) and the BatchNorm branch (quant_layers.py:411-422, :424-441).

Each check is fixed by the mathematics, not by retyping the oracle's
formula: tables against an exact decimal evaluation of the reference's
float pipeline (float64 sigmoid rounded to float32, float32 product, float64
quotient rounded half to even) away from rounding ties, their values at the
zero point and in the saturated tails, SiLU's monotonicity, GAP of a
constant image, and BatchNorm on small integers with an exactly
representable scale."""

import decimal
from decimal import Decimal
from fractions import Fraction

import numpy as np
import pytest

from oracle.pipeline import OraclePipeline, quant_type_info
from quantanything_amd import graph as G

decimal.getcontext().prec = 60
TIE = Decimal(2) ** -40


def _qj(quant_type, qp):
    return {"quant_type": quant_type, "per_channel": True,
            "qparams": {k: dict(scale=s, zp=z, qmin=lo, qmax=hi)
                        for k, (s, z, lo, hi) in qp.items()}}


def _range(quant_type):
    return quant_type_info(quant_type)[2:]


def _activation_graph(op):
    b = G.GraphBuilder(seed=0)
    if op == "SiLU":
        y = b.silu("x")
    else:
        y = b.op(op, ["x"])
    return b.build("x", [None, 1, 4, 4], y)


def _table(op, quant_type, s_in, z_in, s_out, z_out):
    g = _activation_graph(op)
    lo, hi = _range(quant_type)
    qj = _qj(quant_type, {"x": (s_in, z_in, lo, hi),
                          g.outputs[0]: (s_out, z_out, lo, hi)})
    (step,) = OraclePipeline(g, qj).plan
    assert step["kind"] == "lut" and step["offset"] == lo
    assert step["node"].op_type == ("FusedElementwise" if op == "SiLU"
                                    else op)
    return step["table"].astype(np.int64)


def _dequantized(q, z, s):
    """float32((q - z) * s) with the product in float64 (utils.dequantize
    -> qa_dequantize_f32)."""
    return np.float32(float(q - z) * s)


def _nearest_f32(v):
    """Round-to-nearest float32 of the Decimal v > 0, or None within 2^-40
    (relative) of a midpoint between two float32 values."""
    f = np.float32(float(v))
    cands = [np.nextafter(f, np.float32(-np.inf)), f,
             np.nextafter(f, np.float32(np.inf))]
    for a, b_ in zip(cands, cands[1:]):
        mid = (Decimal(float(a)) + Decimal(float(b_))) / 2
        if abs(v - mid) <= TIE * v:
            return None
    return min(cands, key=lambda c: abs(Decimal(float(c)) - v))


def _quantize_exact(y, s, z, lo, hi):
    """round_half_even(y / s) + z clipped, with y / s exact, or None within
    2^-40 of a tie."""
    t = Decimal(float(y)) / Decimal(s)
    frac = t - t.to_integral_value(rounding=decimal.ROUND_FLOOR)
    if abs(frac - Decimal("0.5")) <= TIE * max(abs(t), 1):
        return None
    q = int(t.to_integral_value(rounding=decimal.ROUND_HALF_EVEN)) + z
    return min(max(q, lo), hi)


def _silu_exact(x32):
    """SiLU as the reference evaluates it: sigma = float32(1 / (1 +
    exp(-x))) (float64 then cast, float_ops.py:225-227), y = float32(x *
    sigma) (float32 Mul); None near a float32 rounding midpoint."""
    x = Decimal(float(x32))
    sig = 1 / (1 + (-x).exp())
    s32 = _nearest_f32(sig)
    if s32 is None:
        return None
    return np.float32(x32 * s32)


SILU_CASES = [
    # quant type, input (scale, zp), output (scale, zp)
    ("int8", (0.05, 0), (0.04, 0)),
    ("uint8", (0.035, 131), (0.021, 13)),
    ("int16", (3.2e-4, 0), (2.9e-4, 0)),
    ("uint16", (1.7e-4, 40000), (1.3e-4, 2200)),
]


@pytest.mark.parametrize("quant_type, inp, out", SILU_CASES)
def test_silu_table_matches_exact_evaluation(quant_type, inp, out):
    """Every entry equals the decimal evaluation except within 2^-40 of a
    rounding midpoint. A sigmoid evaluated in float32, a Mul in float64 or a
    truncating quantizer changes entries of the 16-bit tables."""
    lo, hi = _range(quant_type)
    table = _table("SiLU", quant_type, inp[0], inp[1], out[0], out[1])
    assert len(table) == hi - lo + 1
    checked = 0
    step = 1 if hi - lo < 1024 else 7  # every 7th entry of 16-bit tables
    for q in range(lo, hi + 1, step):
        x32 = _dequantized(q, inp[1], inp[0])
        y = _silu_exact(x32)
        if y is None:
            continue
        want = _quantize_exact(y, out[0], out[1], lo, hi)
        if want is None:
            continue
        assert table[q - lo] == want, (q, float(x32))
        checked += 1
    assert checked > 0.99 * len(range(lo, hi + 1, step))


@pytest.mark.parametrize("quant_type, inp, out", SILU_CASES)
def test_activation_tables_at_the_zero_point(quant_type, inp, out):
    """f(0) = 0 for SiLU, HardSwish and Relu: the entry at the input zero
    point is the output zero point."""
    lo, _ = _range(quant_type)
    for op in ("SiLU", "HardSwish", "Relu"):
        table = _table(op, quant_type, inp[0], inp[1], out[0], out[1])
        assert table[inp[1] - lo] == out[1], op


def test_silu_saturated_tails():
    """Where float32(sigmoid(x)) is exactly 1.0 (x >= 17.33) SiLU is the
    identity, so the entry is the plain requantization of x; where it is
    exactly 0.0 (x < -103.3) the product is -0.0 and the entry is the output
    zero point."""
    quant_type, s_in, s_out, z_out = "int8", 1.25, 0.75, 0
    lo, hi = _range(quant_type)
    table = _table("SiLU", quant_type, s_in, 0, s_out, z_out)
    n_one = n_zero = 0
    for q in range(lo, hi + 1):
        x32 = _dequantized(q, 0, s_in)
        sig = np.float32(1.0 / (1.0 + np.exp(-np.float64(x32))))
        if sig == np.float32(1.0):
            assert x32 >= 17.0
            want = _quantize_exact(x32, s_out, z_out, lo, hi)
            assert table[q - lo] == want, q
            n_one += 1
        elif sig == np.float32(0.0):
            assert x32 < -100.0
            assert table[q - lo] == z_out, q
            n_zero += 1
    assert n_one > 10 and n_zero > 10


def test_hardswish_linear_and_zero_regions():
    """HardSwish(x) = x for x >= 3 and 0 for x <= -3."""
    quant_type, s_in, s_out = "int16", 2.5e-4, 2.0e-4
    lo, hi = _range(quant_type)
    table = _table("HardSwish", quant_type, s_in, 0, s_out, 0)
    for q in range(lo, hi + 1, 13):
        x32 = _dequantized(q, 0, s_in)
        if x32 >= 3.0:
            want = _quantize_exact(x32, s_out, 0, lo, hi)
            if want is not None:
                assert table[q - lo] == want, q
        elif x32 <= -3.0:
            assert table[q - lo] == 0, q


def test_silu_table_is_monotone_either_side_of_its_minimum():
    """SiLU decreases on (-inf, x*) and increases on (x*, inf), x* =
    -1.2785; the table (an order-preserving quantization of it) is
    non-increasing, then non-decreasing."""
    quant_type, s_in, z_in, s_out, z_out = "uint16", 1.5e-4, 30000, 1.1e-4, \
        3000
    lo, hi = _range(quant_type)
    table = _table("SiLU", quant_type, s_in, z_in, s_out, z_out)
    x = np.array([_dequantized(q, z_in, s_in) for q in range(lo, hi + 1)])
    left = table[x < -1.30]
    right = table[x > -1.26]
    assert (np.diff(left) <= 0).all() and (np.diff(right) >= 0).all()
    assert table.min() < z_out  # the dip below zero is resolved


# ------------------------------------------------------------------ GAP --
def _gap_graph():
    b = G.GraphBuilder(seed=0)
    return b.build("x", [None, 3, 7, 5], b.op("GlobalAveragePool", ["x"]))


@pytest.mark.parametrize("quant_type, zp", [("int8", 0), ("uint8", 117)])
def test_gap_of_a_constant_image(quant_type, zp):
    """The mean of a constant image is the constant: with equal input and
    output parameters GAP returns the input integer exactly, for every
    value of the type. An area taken from one axis, or a multiplier of
    scale_out * area / scale_in, breaks this."""
    g = _gap_graph()
    lo, hi = _range(quant_type)
    qp = (0.0371, zp, lo, hi)
    pipe = OraclePipeline(g, _qj(quant_type, {"x": qp,
                                              g.outputs[0]: qp}))
    vals = np.arange(lo, hi + 1, dtype=np.int32)
    x = np.broadcast_to(vals[:, None, None, None], (len(vals), 3, 7, 5))
    ints, _ = pipe.run_integers({"x": np.ascontiguousarray(x)})
    got = ints[g.outputs[0]]
    assert got.shape == (len(vals), 3, 1, 1)
    np.testing.assert_array_equal(got[:, :, 0, 0],
                                  np.repeat(vals[:, None], 3, axis=1))


def test_gap_of_a_constant_image_rescaled():
    """With out_scale = in_scale / 2 (an exact binary ratio) the mean of a
    constant image q is exactly 2 (q - z_in) + z_out, clipped: this fixes
    the direction of the multiplier, not only the area."""
    g = _gap_graph()
    lo, hi = _range("uint8")
    s_in, z_in, z_out = 0.0371, 117, 31
    pipe = OraclePipeline(g, _qj("uint8", {
        "x": (s_in, z_in, lo, hi), g.outputs[0]: (s_in / 2, z_out, lo, hi)}))
    vals = np.arange(lo, hi + 1, dtype=np.int32)
    x = np.broadcast_to(vals[:, None, None, None], (len(vals), 3, 7, 5))
    ints, _ = pipe.run_integers({"x": np.ascontiguousarray(x)})
    want = np.clip(2 * (vals.astype(np.int64) - z_in) + z_out, lo, hi)
    np.testing.assert_array_equal(ints[g.outputs[0]][:, :, 0, 0],
                                  np.repeat(want[:, None], 3, axis=1))


def test_gap_multiplier_is_the_exact_ratio():
    """M0 * 2^-(31 + shift) equals in_scale / (out_scale * H * W) within the
    2^-31 relative rounding of a 31-bit mantissa."""
    from oracle.pipeline import multiplier

    s_in, s_out, area = 0.0371, 0.0123, 7 * 5
    m, sh = multiplier(s_in / (s_out * area))
    got = Fraction(m, 2 ** (31 + sh))
    want = Fraction(s_in) / (Fraction(s_out) * area)
    assert abs(got - want) <= want * Fraction(1, 2 ** 31)
    assert 2 ** 30 <= m < 2 ** 31


# ------------------------------------------------------------ BatchNorm --
def test_batchnorm_on_small_integers():
    """gamma = (1, 3), var = (4, 1), epsilon = 0 make the per-channel scale
    a = (1/2, 3) exact; with equal input and output scales the integer BN
    is y = round_half_up((x - zp) * a) + round((beta - a * mean) / s) + zp,
    clipped: a hand-computed affine map."""
    b = G.GraphBuilder(seed=0)
    gamma = b.const(np.array([1.0, 3.0], np.float32))
    beta = b.const(np.array([0.25, -0.5], np.float32))
    mean = b.const(np.array([1.0, 0.125], np.float32))
    var = b.const(np.array([4.0, 1.0], np.float32))
    y = b.op("BatchNormalization", ["x", gamma, beta, mean, var],
             epsilon=0.0)
    g = b.build("x", [None, 2, 3, 3], y)
    s, zp, lo, hi = 0.125, 100, 0, 255
    qj = _qj("uint8", {"x": (s, zp, lo, hi), g.outputs[0]: (s, zp, lo, hi)})
    pipe = OraclePipeline(g, qj)
    (step,) = pipe.plan
    assert step["kind"] == "bn"
    # qB = round((beta - a * mean) / s): (0.25 - 0.5) / 0.125 = -2,
    # (-0.5 - 0.375) / 0.125 = -7
    np.testing.assert_array_equal(step["qB"], [-2, -7])
    x = np.arange(lo, hi + 1, dtype=np.int32)[:18 * 14].reshape(14, 2, 3, 3)
    ints, _ = pipe.run_integers({"x": x})
    got = ints[g.outputs[0]]
    a2, qb = np.array([1, 6]), np.array([-2, -7])  # 2 * a and qB
    t = (x.astype(np.int64) - zp) * a2[None, :, None, None]
    want = np.floor_divide(t + 1, 2) + qb[None, :, None, None] + zp
    np.testing.assert_array_equal(got, np.clip(want, lo, hi))
