"""Quantization maths of the host side (reference: ``quantization/utils.py``).

Everything here is host-side parameter derivation on small arrays (scales,
zero points, weight quantization, multiplier decomposition, lookup tables);
activation tensors are quantized on the GPU by the executor
(``qa_d_quantize_f32``). The functions keep the reference's names, argument
meaning and numerics:

* symmetric signed / asymmetric unsigned ranges (``utils.py:66-90``),
* quantize = clip(round_half_even(double(x) / scale) + zp) with the
  scale == 0 special case (``utils.py:97-114``),
* dequantize = float32((q - zp) * scale) (``utils.py:117-124``),
* ``quantize_multiplier``: frexp significand rounded half-even to 31 bits,
  |M0| in [2^30, 2^31), sign carried, 0 -> (0, 0) (``utils.py:132-149``),
* ``multiply_by_quantized_multiplier``: round(x * M0 * 2^-(31+shift)),
  round half up, exact beyond int64 (``utils.py:162-167``).
"""

from dataclasses import dataclass

import numpy as np

_INT32_MIN, _INT32_MAX = -(2**31), 2**31 - 1


@dataclass
class QParams:
    """Affine parameters of one tensor: ``real = (q - zp) * scale``,
    ``qmin <= q <= qmax``."""

    scale: float
    zp: int
    qmin: int
    qmax: int

    def to_dict(self):
        return {"scale": float(self.scale), "zp": int(self.zp),
                "qmin": int(self.qmin), "qmax": int(self.qmax)}

    @classmethod
    def from_dict(cls, d):
        return cls(float(d["scale"]), int(d["zp"]), int(d["qmin"]),
                   int(d["qmax"]))


def parse_quant_type(quant_type):
    """``'int8'`` -> ``(8, True)``, ``'uint12'`` -> ``(12, False)``."""
    for prefix, signed in (("uint", False), ("int", True)):
        if quant_type.startswith(prefix):
            return int(quant_type[len(prefix):]), signed
    raise ValueError(f"Unknown quant_type: {quant_type}")


def quant_range(quant_type):
    """``(qmin, qmax)`` of a quantization type."""
    bits, signed = parse_quant_type(quant_type)
    if signed:
        return -(1 << (bits - 1)), (1 << (bits - 1)) - 1
    return 0, (1 << bits) - 1


def calculate_scale_zp(min_val, max_val, quant_type="int8"):
    """``(scale, zp, qmin, qmax)`` of a calibrated range: symmetric
    (``zp = 0``) for signed types, asymmetric over a range containing 0 for
    unsigned ones; a degenerate range gives ``(1.0, 0)``."""
    qmin, qmax = quant_range(quant_type)
    _, signed = parse_quant_type(quant_type)
    lo, hi = float(min_val), float(max_val)
    if signed:
        peak = max(abs(lo), abs(hi))
        return (1.0 if peak == 0 else peak / qmax), 0, qmin, qmax
    lo, hi = min(lo, 0.0), max(hi, 0.0)
    if lo == hi:
        return 1.0, 0, qmin, qmax
    scale = (hi - lo) / qmax
    zp = int(np.clip(np.round(-lo / scale), qmin, qmax))
    return scale, zp, qmin, qmax


def int_dtype(qmin, qmax):
    """int32 when the range fits, else int64."""
    return np.int32 if _INT32_MIN <= qmin and qmax <= _INT32_MAX else np.int64


def quantize(x, scale, zp, qmin, qmax):
    """Float -> integer on the host, per-tensor or broadcast per-channel."""
    x = np.asarray(x)
    dtype = int_dtype(qmin, qmax)
    scale_a = np.asarray(scale, dtype=np.float64)
    zp_a = np.asarray(zp)
    if scale_a.ndim == 0 and zp_a.ndim == 0 and float(scale_a) == 0.0:
        return np.full(x.shape, int(zp_a), dtype=dtype)
    safe = np.where(scale_a == 0, 1.0, scale_a)
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        q = np.round(x.astype(np.float64) / safe) + zp_a
    q = np.where(scale_a == 0, zp_a, q)
    return np.clip(q, qmin, qmax).astype(dtype)


def dequantize(q, scale, zp):
    """Integer -> float32: ``(q - zp) * scale`` (double product)."""
    q = np.asarray(q)
    return ((q.astype(np.int64) - zp)
            * np.asarray(scale, dtype=np.float64)).astype(np.float32)


def fake_quantize(x, scale, zp, qmin, qmax):
    """Quantize then dequantize (quantization noise on float data)."""
    return dequantize(quantize(x, scale, zp, qmin, qmax), scale, zp)


def quantize_multiplier(real_multiplier):
    """``(M0, shift)`` with ``real = M0 * 2^-(31+shift)``."""
    real = float(real_multiplier)
    if real == 0.0:
        return 0, 0
    sign = -1 if real < 0 else 1
    significand, exponent = np.frexp(abs(real))
    m0 = int(np.round(significand * 2.0**31))
    if m0 >= 1 << 31:  # the significand rounded up to 1.0
        m0 //= 2
        exponent += 1
    return sign * m0, int(-exponent)


def quantize_multipliers(real_multipliers):
    """Element-wise :func:`quantize_multiplier` -> two int64 arrays."""
    real = np.asarray(real_multipliers, dtype=np.float64)
    pairs = [quantize_multiplier(v) for v in real.reshape(-1)]
    mult = np.array([m for m, _ in pairs], dtype=np.int64).reshape(real.shape)
    shift = np.array([s for _, s in pairs], dtype=np.int64).reshape(real.shape)
    return mult, shift


def multiply_by_quantized_multiplier(accum, q_multiplier, shift):
    """``round(accum * M0 * 2^-(31+shift))``, round half up, on the host.

    Uses int64 arithmetic while ``|accum| * |M0| < 2^62`` and exact Python
    integers beyond (results clipped to +-2^62), like the reference's NumPy
    twin (``native.py:177-203``)."""
    x = np.asarray(accum, dtype=np.int64)
    m = np.asarray(q_multiplier, dtype=np.int64)
    t = 31 + np.asarray(shift, dtype=np.int64)
    bound = (int(np.abs(x).max()) if x.size else 0) * (
        int(np.abs(m).max()) if m.size else 0)
    if bound < 1 << 62:
        p = x * m
        t_r = np.maximum(t, 1)
        right = (p + np.left_shift(np.int64(1), t_r - 1)) >> t_r
        left = np.left_shift(p, np.clip(-t, 0, 60))
        return np.where(t > 0, right, left).astype(np.int64)
    xb, mb, tb = np.broadcast_arrays(x, m, t)
    out = []
    for xi, mi, ti in zip(xb.ravel().tolist(), mb.ravel().tolist(),
                          tb.ravel().tolist()):
        p = xi * mi
        out.append((p + (1 << (ti - 1))) >> ti if ti > 0 else p << -ti)
    big = np.array(out, dtype=object).reshape(xb.shape)
    return np.clip(big, -(1 << 62), 1 << 62).astype(np.int64)
