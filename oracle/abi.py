"""ctypes binding of a ``qa_*`` C-ABI library for the oracle (test only).

The declaration table restates the one the reference loader applies
(``quantization/native.py:104-128``): every pointer is ``c_void_p``, every
size / integer scalar ``c_int64``, scales ``c_double``, thread counts
``c_int``. The wrappers restate the reference wrapper semantics
(``native.py:207-556``): operand dtypes per path, int16 operands on the
narrow path and int32 on the wide one, broadcast of scalar multipliers to the
channel count, optional pre/post bias.
"""

import ctypes
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_LIB = HERE / "libqa_oracle.so"
REF_LIB = HERE / "_ref" / "libqa_ref.so"

ABI_SIGNATURES = {
    "qa_num_threads": (ctypes.c_int, []),
    "qa_set_num_threads": (None, [ctypes.c_int]),
    "qa_has_openmp": (ctypes.c_int, []),
}


def _table():
    p, i64, f64 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_double
    sigs = dict(ABI_SIGNATURES)
    for name in ("qa_gemm_f32", "qa_gemm_i16_i32", "qa_gemm_i32_i64"):
        sigs[name] = (None, [i64, i64, i64, p, p, p])
    for name in ("qa_conv_f32", "qa_conv_i32_i16_i32", "qa_conv_i32_i32_i64"):
        sigs[name] = (None, [p, p, p] + [i64] * 16)
    for name in ("qa_requantize_i32", "qa_requantize_i64"):
        sigs[name] = (None, [p, p, i64, i64, i64, p, p, p, p, i64, i64, i64])
    sigs["qa_rescale"] = (None, [p, p] + [i64] * 7)
    sigs["qa_add"] = (None, [p, p, p] + [i64] * 11)
    sigs["qa_mul"] = (None, [p, p, p] + [i64] * 8)
    sigs["qa_lut"] = (None, [p, p, i64, i64, p, i64])
    sigs["qa_quantize_f32"] = (None, [p, p, i64, f64, i64, i64, i64])
    sigs["qa_dequantize_f32"] = (None, [p, p, i64, f64, i64])
    return sigs


ABI_TABLE = _table()


def declare(lib):
    """Binds every ``qa_*`` export; raises AttributeError when one is missing."""
    for name, (restype, argtypes) in ABI_TABLE.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    return lib


def _ptr(a):
    return ctypes.c_void_p(a.ctypes.data) if a is not None else None


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def conv_output_size(size, k, stride, pad_begin, pad_end, dilation):
    """Spatial output size along one axis (``native.py:239-241``)."""
    return (size + pad_begin + pad_end - dilation * (k - 1) - 1) // stride + 1


def conv_geometry(x_shape, w_shape, strides, pads, dilations, groups):
    """Validates conv shapes like ``native.py:244-257``; raises ValueError."""
    n, c, h, wd = x_shape
    cout, cg, kh, kw = w_shape
    if c != cg * groups or cout % groups:
        raise ValueError(
            f"conv shape mismatch: input C={c}, weight={tuple(w_shape)}, "
            f"groups={groups}"
        )
    sh, sw = strides
    dh, dw = dilations
    pt, pl, pb, pr = pads
    oh = conv_output_size(h, kh, sh, pt, pb, dh)
    ow = conv_output_size(wd, kw, sw, pl, pr, dw)
    return n, c, h, wd, cout, kh, kw, sh, sw, pt, pl, dh, dw, oh, ow


class QaLib:
    """Wrappers over one loaded ``qa_*`` library (reference or oracle)."""

    def __init__(self, path):
        self.path = Path(path)
        self.lib = declare(ctypes.CDLL(str(self.path)))

    # ------------------------------------------------------------ threads --
    def set_num_threads(self, n):
        self.lib.qa_set_num_threads(int(n))

    def num_threads(self):
        return int(self.lib.qa_num_threads())

    # --------------------------------------------------------------- GEMM --
    def gemm_f32(self, a, b):
        a, b = _c(a, np.float32), _c(b, np.float32)
        out = np.empty((a.shape[0], b.shape[1]), dtype=np.float32)
        self.lib.qa_gemm_f32(a.shape[0], b.shape[1], a.shape[1],
                             _ptr(a), _ptr(b), _ptr(out))
        return out

    def gemm_int(self, a, b, wide=False):
        m, k = a.shape
        n = b.shape[1]
        if wide:
            a, b = _c(a, np.int32), _c(b, np.int32)
            out = np.empty((m, n), dtype=np.int64)
            self.lib.qa_gemm_i32_i64(m, n, k, _ptr(a), _ptr(b), _ptr(out))
        else:
            a, b = _c(a, np.int16), _c(b, np.int16)
            out = np.empty((m, n), dtype=np.int32)
            self.lib.qa_gemm_i16_i32(m, n, k, _ptr(a), _ptr(b), _ptr(out))
        return out

    # --------------------------------------------------------------- conv --
    def _conv(self, fn, x, w, out_dtype, strides, pads, dilations, groups):
        geo = conv_geometry(x.shape, w.shape, strides, pads, dilations, groups)
        n, c, h, wd, cout, kh, kw, sh, sw, pt, pl, dh, dw, oh, ow = geo
        out = np.empty((n, cout, oh, ow), dtype=out_dtype)
        fn(_ptr(x), _ptr(w), _ptr(out), n, c, h, wd, cout, kh, kw, sh, sw,
           pt, pl, dh, dw, groups, oh, ow)
        return out

    def conv2d_f32(self, x, w, strides=(1, 1), pads=(0, 0, 0, 0),
                   dilations=(1, 1), groups=1):
        return self._conv(self.lib.qa_conv_f32, _c(x, np.float32),
                          _c(w, np.float32), np.float32, strides, pads,
                          dilations, groups)

    def conv2d_int(self, x, w, strides=(1, 1), pads=(0, 0, 0, 0),
                   dilations=(1, 1), groups=1, wide=False):
        x = _c(x, np.int32)
        if wide:
            return self._conv(self.lib.qa_conv_i32_i32_i64, x,
                              _c(w, np.int32), np.int64, strides, pads,
                              dilations, groups)
        return self._conv(self.lib.qa_conv_i32_i16_i32, x, _c(w, np.int16),
                          np.int32, strides, pads, dilations, groups)

    # --------------------------------------------------------- requantize --
    def requantize(self, acc, outer, channels, inner, mult, shift, zp, qmin,
                   qmax, pre_bias=None, post_bias=None):
        mult = _c(np.broadcast_to(np.asarray(mult, np.int64), (channels,)),
                  np.int64)
        shift = _c(np.broadcast_to(np.asarray(shift, np.int64), (channels,)),
                   np.int64)
        wide = acc.dtype == np.int64
        acc = _c(acc, np.int64 if wide else np.int32)
        out = np.empty(acc.shape, dtype=np.int32)
        pre = None if pre_bias is None else _c(
            np.broadcast_to(np.asarray(pre_bias, np.int64), (channels,)),
            np.int64)
        post = None if post_bias is None else _c(
            np.broadcast_to(np.asarray(post_bias, np.int64), (channels,)),
            np.int64)
        fn = self.lib.qa_requantize_i64 if wide else self.lib.qa_requantize_i32
        fn(_ptr(acc), _ptr(out), int(outer), int(channels), int(inner),
           _ptr(mult), _ptr(shift), _ptr(pre), _ptr(post), int(zp),
           int(qmin), int(qmax))
        return out

    # ------------------------------------------------------- element-wise --
    def rescale(self, x, zp_in, mult, shift, zp_out, qmin, qmax):
        x = _c(x, np.int32)
        out = np.empty_like(x)
        self.lib.qa_rescale(_ptr(x), _ptr(out), x.size, int(zp_in), int(mult),
                            int(shift), int(zp_out), int(qmin), int(qmax))
        return out

    def add(self, a, b, za, ma, sa, zb, mb, sb, zp_out, qmin, qmax, sign=1):
        a, b = np.broadcast_arrays(a, b)
        a, b = _c(a, np.int32), _c(b, np.int32)
        out = np.empty_like(a)
        self.lib.qa_add(_ptr(a), _ptr(b), _ptr(out), a.size, int(za), int(ma),
                        int(sa), int(zb), int(mb), int(sb), int(sign),
                        int(zp_out), int(qmin), int(qmax))
        return out

    def mul(self, a, b, za, zb, mult, shift, zp_out, qmin, qmax):
        a, b = np.broadcast_arrays(a, b)
        a, b = _c(a, np.int32), _c(b, np.int32)
        out = np.empty_like(a)
        self.lib.qa_mul(_ptr(a), _ptr(b), _ptr(out), a.size, int(za), int(zb),
                        int(mult), int(shift), int(zp_out), int(qmin),
                        int(qmax))
        return out

    def lut(self, x, table, offset):
        table = _c(table, np.int32)
        x = _c(x, np.int32)
        out = np.empty_like(x)
        self.lib.qa_lut(_ptr(x), _ptr(out), x.size, int(offset), _ptr(table),
                        len(table))
        return out

    # ---------------------------------------------------- float <-> int --
    def quantize_f32(self, x, scale, zp, qmin, qmax):
        x = _c(x, np.float32)
        out = np.empty(x.shape, dtype=np.int32)
        self.lib.qa_quantize_f32(_ptr(x), _ptr(out), x.size, float(scale),
                                 int(zp), int(qmin), int(qmax))
        return out

    def dequantize_f32(self, q, scale, zp):
        q = _c(q, np.int32)
        out = np.empty(q.shape, dtype=np.float32)
        self.lib.qa_dequantize_f32(_ptr(q), _ptr(out), q.size, float(scale),
                                   int(zp))
        return out


_CACHE = {}


def load(kind="oracle"):
    """Loads ``"oracle"`` (the C restatement) or ``"ref"`` (the compiled
    reference). Raises FileNotFoundError when the library was not built."""
    if kind not in _CACHE:
        path = {"oracle": ORACLE_LIB, "ref": REF_LIB}[kind]
        if not path.exists():
            raise FileNotFoundError(
                f"{path} is missing; build it with `make -C oracle`")
        _CACHE[kind] = QaLib(path)
    return _CACHE[kind]


def ref_available():
    """True when the compiled reference library exists (it travels with the
    tree to wherever the tests run)."""
    return REF_LIB.exists() and os.access(REF_LIB, os.R_OK)
