"""Seeded synthetic workloads for the quantized Conv/Gemm path.

All randomness comes from a counter-based SplitMix64 stream implemented here in
NumPy, so every consumer (benchmark, tests, fixture scripts) regenerates the
same bytes from the same seed independent of the NumPy version.

Workloads (integer data in the "raw" quantized domain):

* ``gemm_workload``: standalone integer GEMM + requantize, M=4096 K=576 N=64;
  uint8 activations uniform in [0,255] with zero point 128, int8 symmetric
  per-output-channel weights round(N(0,40)) clipped to [-127,127], int32
  bias uniform in [-2^16, 2^16], M0 uniform in [2^30, 2^31), shift in 1..15,
  uint8 output with zero point 128.
* ``conv_workload``: one int8 Conv2d, batch 32, 64->64 channels, 3x3, stride
  1, pad 1, 56x56 NCHW, uint8 input with a seeded zero point, per-channel
  symmetric int8 weights, int32 bias, followed by requantize and a 256-entry
  SiLU lookup table.
"""

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed, n, offset=0):
    """``n`` 64-bit words of the SplitMix64 sequence of ``seed``."""
    with np.errstate(over="ignore"):
        i = np.arange(offset + 1, offset + n + 1, dtype=np.uint64)
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + i * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


class Stream:
    """A seeded stream; every draw advances a private counter."""

    def __init__(self, seed):
        self.seed = int(seed)
        self.pos = 0

    def _words(self, n):
        w = splitmix64(self.seed, n, self.pos)
        self.pos += n
        return w

    def integers(self, lo, hi, shape):
        """Integers uniform in ``[lo, hi]`` (inclusive), int64."""
        n = int(np.prod(shape, dtype=np.int64))
        span = np.uint64(hi - lo + 1)
        return (self._words(n) % span).astype(np.int64).reshape(shape) + lo

    def uniform(self, shape, lo=0.0, hi=1.0):
        """Float64 uniform in ``[lo, hi)``."""
        n = int(np.prod(shape, dtype=np.int64))
        u = (self._words(n) >> np.uint64(11)).astype(np.float64) * 2.0**-53
        return (lo + (hi - lo) * u).reshape(shape)

    def normal(self, shape, sigma=1.0):
        """Float64 normals (Box-Muller)."""
        n = int(np.prod(shape, dtype=np.int64))
        u1 = 1.0 - self.uniform((n,))  # (0, 1]
        u2 = self.uniform((n,))
        z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
        return (sigma * z).reshape(shape)


def _requant_params(s, channels):
    mult = s.integers(1 << 30, (1 << 31) - 1, (channels,))
    shift = s.integers(1, 15, (channels,))
    return mult, shift


def gemm_workload(seed=1, M=4096, K=576, N=64):
    """Integer GEMM + requantize workload (dict of arrays and scalars)."""
    s = Stream(seed)
    a = s.integers(0, 255, (M, K)).astype(np.uint8)
    w = np.clip(np.round(s.normal((K, N), 40.0)), -127, 127).astype(np.int8)
    bias = s.integers(-(1 << 16), 1 << 16, (N,))
    mult, shift = _requant_params(s, N)
    return dict(a=a, w=w, bias=bias, mult=mult, shift=shift, zp_in=128,
                zp_out=128, qmin=0, qmax=255, M=M, K=K, N=N)


def silu_lut(in_scale, in_zp, out_scale, out_zp, qmin=0, qmax=255):
    """256-entry SiLU table in the reference's float semantics: dequantize to
    float32 (double product), Sigmoid in float64 cast to float32, float32
    multiply, quantize with a double division and half-to-even rounding
    (quant_layers.py:461-468, float_ops.py:225-227, utils.py:97-124)."""
    q = np.arange(qmin, qmax + 1, dtype=np.int64)
    x = ((q - in_zp) * float(in_scale)).astype(np.float32)
    sig = (1.0 / (1.0 + np.exp(-x.astype(np.float64)))).astype(np.float32)
    y = x * sig
    out = np.round(y.astype(np.float64) / out_scale) + out_zp
    return np.clip(out, qmin, qmax).astype(np.int32)


def conv_workload(seed=2, batch=32, cin=64, cout=64, hw=56, k=3, stride=1,
                  pad=1):
    """Single int8 Conv2d + requantize + SiLU LUT workload."""
    s = Stream(seed)
    zp_in = int(s.integers(0, 255, (1,))[0])
    x = s.integers(0, 255, (batch, cin, hw, hw)).astype(np.uint8)
    wf = s.normal((cout, cin, k, k), 1.0)
    max_abs = np.abs(wf.reshape(cout, -1)).max(axis=1)
    w = np.clip(np.round(wf / (max_abs / 127.0).reshape(-1, 1, 1, 1)),
                -127, 127).astype(np.int8)
    bias = s.integers(-(1 << 16), 1 << 16, (cout,))
    mult, shift = _requant_params(s, cout)
    zp_out = int(s.integers(0, 255, (1,))[0])
    lut = silu_lut(0.05, zp_out, 0.03, 10)
    return dict(x=x, w=w, bias=bias, mult=mult, shift=shift, zp_in=zp_in,
                zp_out=zp_out, qmin=0, qmax=255, lut=lut, lut_offset=0,
                stride=stride, pad=pad, k=k)
