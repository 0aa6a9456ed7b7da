"""ctypes boundary of the MI355X library ``libqa_hip.so``.

Mirrors the wrapper API of QuantAnything's ``quantization/native.py``
(``gemm_f32``, ``gemm_int``, ``conv2d_f32``, ``conv2d_int``,
``accumulator_is_wide``, ``requantize``, ``rescale``, ``add``, ``mul``,
``lut``, ``quantize_f32``, ``dequantize_f32``, ``mbqm_np``) with the same
argument meaning, dtypes and error behaviour (``ValueError`` on a conv shape
mismatch), so callers written against the reference run unchanged.

Differences from the reference, on purpose:

* There is no NumPy fallback. The library is found at ``$QA_LIB`` or next to
  this file; if it is missing, or a GPU call fails, the wrapper raises
  ``RuntimeError`` naming the reason. Silent CPU execution would hide a
  broken GPU path.
* ``backend()`` returns the loaded library's backend string (``hip-gfx950``)
  so tests can assert which code ran.

Environment variables: ``QA_LIB`` (path of the library to load).
"""

import ctypes
import os
from pathlib import Path

import numpy as np

_PKG = Path(__file__).resolve().parent
DEFAULT_LIB = _PKG / "libqa_hip.so"

_lib = None
_load_error = None


# --------------------------------------------------------------- loading ----
def _declare(lib):
    c = ctypes
    p, i64, f64, i32 = c.c_void_p, c.c_int64, c.c_double, c.c_int
    sigs = {
        # the reference ABI (native.py:104-128)
        "qa_num_threads": (i32, []),
        "qa_set_num_threads": (None, [i32]),
        "qa_has_openmp": (i32, []),
        "qa_gemm_f32": (None, [i64, i64, i64, p, p, p]),
        "qa_gemm_i16_i32": (None, [i64, i64, i64, p, p, p]),
        "qa_gemm_i32_i64": (None, [i64, i64, i64, p, p, p]),
        "qa_requantize_i32": (None, [p, p] + [i64] * 3 + [p] * 4 + [i64] * 3),
        "qa_requantize_i64": (None, [p, p] + [i64] * 3 + [p] * 4 + [i64] * 3),
        "qa_rescale": (None, [p, p] + [i64] * 7),
        "qa_add": (None, [p, p, p] + [i64] * 11),
        "qa_mul": (None, [p, p, p] + [i64] * 8),
        "qa_lut": (None, [p, p, i64, i64, p, i64]),
        "qa_quantize_f32": (None, [p, p, i64, f64, i64, i64, i64]),
        "qa_dequantize_f32": (None, [p, p, i64, f64, i64]),
        # additional surface
        "qa_backend": (c.c_char_p, []),
        "qa_last_error": (c.c_char_p, []),
        "qa_clear_error": (None, []),
        "qa_device_count": (i32, []),
        "qa_device_arch": (i32, [c.c_char_p, i64]),
        "qa_stream": (p, []),
        "qa_synchronize": (i32, []),
        "qa_pack_weights_i8_size": (i64, [i64] * 6 + [p, p]),
        "qa_pack_weights_i8": (i32, [p] + [i64] * 7 + [p, p, p, p]),
        "qa_pack_weights_f64_size": (i64, [i64] * 5 + [p, p]),
        "qa_pack_weights_f64": (i32, [p] + [i64] * 6 + [p]),
        "qa_pack_weights_i16s": (i32, [p] + [i64] * 5 + [p, p]),
        "qa_d_conv": (i32, [p, p]),
        "qa_d_quantize_conv": (i32, [p, p, f64, i64, i64, i64, p]),
        "qa_d_conv_pool": (i32, [p, p, p]),
        "qa_conv_pw_pool_supported": (i32, [p, p]),
        "qa_d_conv_pw_pool": (i32, [p, p, p, p]),
        "qa_fragments_i8_size": (i64, [i64, i64]),
        "qa_d_pack_fragments_i8": (i32, [p, i64, i64, p, p]),
        "qa_conv_pair_supported": (i32, [p, p]),
        "qa_conv_pair_tail_supported": (i32, [p, p, p]),
        "qa_d_conv_pair_tail": (i32, [p, p, p, p]),
        "qa_d_conv_pair": (i32, [p, p, p]),
        "qa_conv_chain_supported": (i32, [p, p]),
        "qa_d_conv_chain": (i32, [p, p, p]),
        "qa_d_copy_nd": (i32, [p, p]),
        "qa_d_layernorm": (i32, [p, i32, i64, i64, i64, f64, i64, i64, p, p,
                                 f64, p, i32, i64, f64, i64, i64, i64, i64,
                                 p]),
        "qa_d_matmul_act": (i32, [p, p]),
        "qa_attention_supported": (i32, [p]),
        "qa_d_attention": (i32, [p, p]),
        "qa_epi_plan_bytes": (i64, [i64]),
        "qa_plan_epilogue_i8": (i32, [p, p]),
        "qa_d_requantize": (i32, [p, i32, p, i32] + [i64] * 3 + [p] * 4
                            + [i64] * 5 + [p]),
        "qa_d_rescale": (i32, [p, i32, i64, p, i32] + [i64] * 11 + [p]),
        "qa_d_add": (i32, [p, i64, p, i64, i32, p, i32] + [i64] * 16 + [p]),
        "qa_d_mul": (i32, [p, i64, p, i64, i32, p, i32] + [i64] * 13 + [p]),
        "qa_d_lut": (i32, [p, i32, i64, p, i32, i64, i64, i64, i64, p, i64,
                           i64, i64, p]),
        "qa_d_gap": (i32, [p, i32] + [i64] * 13 + [p, i32, i64, i64, p]),
        "qa_d_quantize_nhwc": (i32, [p, i64, i64, i64, p, i32, i64, f64, i64,
                                     i64, i64, i64, p]),
        "qa_d_quantize_patches": (i32, [p] + [i64] * 6 + [p, f64] +
                                  [i64] * 4 + [p]),
        "qa_d_softmax": (i32, [p, i32, i64, i64, f64, i64, i64, p, i32, f64]
                         + [i64] * 4 + [p]),
        "qa_d_softmax_table": (i32, [f64, i64, i64, p, p]),
        "qa_d_softmax_lut": (i32, [p, i64, i64, p, p, f64, i64, i64, i64, i64,
                                   p]),
        "qa_d_softmax_lut_f32": (i32, [p, i64, i64, p, p, f64, i64, i64, i64,
                                       i64, p, p]),
        "qa_d_softmax_f32": (i32, [p, i32, i64, i64, f64, i64, i64, p, i32,
                                   f64] + [i64] * 4 + [p, p]),
        "qa_d_quantize_f32": (i32, [p, p, i32, i64, f64, i64, i64, i64, i64,
                                    p]),
        "qa_d_dequantize_f32": (i32, [p, i32, p, i64, f64, i64, i64, p]),
        "qa_d_pad_nd": (i32, [p, p]),
        "qa_d_maxpool": (i32, [p, p]),
        "qa_d_fb_binary": (i32, [p, p]),
        "qa_d_binary_nd": (i32, [p, p]),
        "qa_d_fb_reduce_mean": (i32, [p, p]),
        "qa_d_fb_softmax": (i32, [p, p]),
        "qa_d_fb_avgpool": (i32, [p, p]),
        "qa_d_fb_pad": (i32, [p, p]),
        "qa_d_fb_gather": (i32, [p, p]),
        "qa_noalloc_scratch_bytes": (i64, []),
        "qa_gemm_i16_i32_noalloc_need": (i64, [i64] * 3),
        "qa_gemm_i16_i32_noalloc": (i32, [i64] * 3 + [p] * 4),
    }
    for name in ("qa_conv_f32", "qa_conv_i32_i16_i32", "qa_conv_i32_i32_i64"):
        sigs[name] = (None, [p, p, p] + [i64] * 16)
    for name, (restype, argtypes) in sigs.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    return sigs


SYMBOLS = None


def _single_hip_runtime():
    """PyTorch-ROCm ships its own ``libamdhip64.so`` with the same soname
    (``libamdhip64.so.7``) as the system one the library was linked against.
    Loading torch first makes the library bind to that already-loaded
    runtime, so the process has ONE HIP runtime (device pointers and streams
    are shared with torch); loading the library first would pull in a second
    runtime that then fails to see the GPU."""
    try:
        import torch  # noqa: F401
    except ImportError:
        pass


def _load():
    global _lib, _load_error, SYMBOLS
    path = os.environ.get("QA_LIB") or str(DEFAULT_LIB)
    _single_hip_runtime()
    try:
        lib = ctypes.CDLL(path)
        SYMBOLS = _declare(lib)
        _lib = lib
    except Exception as exc:  # missing file, missing symbol, bad ELF
        _load_error = f"{path}: {exc}"


_load()


def available():
    """True when ``libqa_hip.so`` is loaded (a GPU is still needed to run)."""
    return _lib is not None


def load_error():
    """Why the library is not loaded (None when it is)."""
    return _load_error


def library():
    """The loaded ``ctypes.CDLL``; raises when missing."""
    if _lib is None:
        raise RuntimeError(
            "libqa_hip.so is not loaded (build it with "
            f"`python -m quantanything_amd.build`): {_load_error}")
    return _lib


def backend():
    return library().qa_backend().decode()


def require():
    """Raises unless the HIP library is loaded and a GPU is visible."""
    lib = library()
    if lib.qa_device_count() < 1:
        raise RuntimeError("libqa_hip.so is loaded but no GPU is visible")
    return lib


def _check(what):
    err = _lib.qa_last_error()
    if err is not None:
        _lib.qa_clear_error()
        raise RuntimeError(f"{what} failed on the GPU: {err.decode()}")


def set_num_threads(n):
    """Accepted for API compatibility; the GPU library ignores it."""
    library().qa_set_num_threads(int(n))


def _ptr(a):
    return ctypes.c_void_p(a.ctypes.data)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def _as_i64(v):
    return np.asarray(v, dtype=np.int64)


# --------------------------------------------------- fixed-point multiply ----
def mbqm_np(x, mult, shift):
    """Host ``round(x * mult * 2**-(31+shift))`` (reference name kept; the
    implementation is :func:`quantanything_amd.utils.
    multiply_by_quantized_multiplier`)."""
    from quantanything_amd.utils import multiply_by_quantized_multiplier

    return multiply_by_quantized_multiplier(x, mult, shift)


# ------------------------------------------------------------------ GEMM ----
def gemm_f32(a, b):
    """Float32 matrix product of host arrays, computed by the GPU
    library (reference wrapper: ``native.py:207-217``)."""
    lib = library()
    a, b = _c(a, np.float32), _c(b, np.float32)
    out = np.empty((a.shape[0], b.shape[1]), dtype=np.float32)
    lib.qa_gemm_f32(a.shape[0], b.shape[1], a.shape[1], _ptr(a), _ptr(b),
                    _ptr(out))
    _check("qa_gemm_f32")
    return out


def gemm_int(a, b, wide=False):
    """Exact integer matrix product of host arrays: int16 operands summed
    in int32, or int32 operands in int64 with ``wide``
    (``native.py:219-235``)."""
    lib = library()
    m, k = a.shape
    n = b.shape[1]
    if wide:
        a, b = _c(a, np.int32), _c(b, np.int32)
        out = np.empty((m, n), dtype=np.int64)
        lib.qa_gemm_i32_i64(m, n, k, _ptr(a), _ptr(b), _ptr(out))
    else:
        a, b = _c(a, np.int16), _c(b, np.int16)
        out = np.empty((m, n), dtype=np.int32)
        lib.qa_gemm_i16_i32(m, n, k, _ptr(a), _ptr(b), _ptr(out))
    _check("gemm_int")
    return out


# ----------------------------------------------------------- convolution ----
def conv_output_size(size, k, stride, pad_begin, pad_end, dilation):
    """Output extent along H or W: (size + both pads - dilated kernel) //
    stride + 1 (``native.py:239-241``)."""
    return (size + pad_begin + pad_end - dilation * (k - 1) - 1) // stride + 1


def conv_geometry(x_shape, w_shape, strides, pads, dilations, groups):
    """``(n, c, h, w, cout, kh, kw, sh, sw, pt, pl, dh, dw, oh, ow)``;
    raises ValueError on a channel / group mismatch."""
    n, c, h, wd = x_shape
    cout, cg, kh, kw = w_shape
    if c != cg * groups or cout % groups:
        raise ValueError(
            f"conv shape mismatch: input C={c}, weight={tuple(w_shape)}, "
            f"groups={groups}")
    sh, sw = strides
    dh, dw = dilations
    pt, pl, pb, pr = pads
    oh = conv_output_size(h, kh, sh, pt, pb, dh)
    ow = conv_output_size(wd, kw, sw, pl, pr, dw)
    return n, c, h, wd, cout, kh, kw, sh, sw, pt, pl, dh, dw, oh, ow


def conv2d_f32(x, w, strides=(1, 1), pads=(0, 0, 0, 0), dilations=(1, 1),
               groups=1):
    """Float32 convolution of an NCHW host array with OIHW weights
    (``[Cout, C / groups, KH, KW]``) on the GPU (``native.py:282-313``)."""
    lib = library()
    x, w = _c(x, np.float32), _c(w, np.float32)
    n, c, h, wd, cout, kh, kw, sh, sw, pt, pl, dh, dw, oh, ow = conv_geometry(
        x.shape, w.shape, strides, pads, dilations, groups)
    out = np.empty((n, cout, oh, ow), dtype=np.float32)
    lib.qa_conv_f32(_ptr(x), _ptr(w), _ptr(out), n, c, h, wd, cout, kh, kw,
                    sh, sw, pt, pl, dh, dw, groups, oh, ow)
    _check("qa_conv_f32")
    return out


def conv2d_int(x, w, strides=(1, 1), pads=(0, 0, 0, 0), dilations=(1, 1),
               groups=1, wide=False):
    """Integer NCHW convolution of zero-point-centred operands; int32
    accumulators, int64 when ``wide`` (reference ``native.py:315-360``)."""
    lib = library()
    x = _c(x, np.int32)
    n, c, h, wd, cout, kh, kw, sh, sw, pt, pl, dh, dw, oh, ow = conv_geometry(
        x.shape, w.shape, strides, pads, dilations, groups)
    args = (n, c, h, wd, cout, kh, kw, sh, sw, pt, pl, dh, dw, groups, oh, ow)
    if wide:
        w = _c(w, np.int32)
        out = np.empty((n, cout, oh, ow), dtype=np.int64)
        lib.qa_conv_i32_i32_i64(_ptr(x), _ptr(w), _ptr(out), *args)
    else:
        w = _c(w, np.int16)
        out = np.empty((n, cout, oh, ow), dtype=np.int32)
        lib.qa_conv_i32_i16_i32(_ptr(x), _ptr(w), _ptr(out), *args)
    _check("conv2d_int")
    return out


def accumulator_is_wide(num_bits, reduction_size):
    """Whether a dot product needs the int64 accumulator (int16 operands are
    only safe when ``num_bits <= 15`` and ``(2^bits)^2 * K < 2^31``;
    reference ``native.py:363-373``)."""
    if num_bits > 15:
        return True
    return ((1 << num_bits) ** 2) * int(reduction_size) >= (1 << 31)


# -------------------------------------------------------- requantisation ----
def requantize(acc, outer, channels, inner, mult, shift, zp, qmin, qmax,
               pre_bias=None, post_bias=None):
    """``clip(mbqm(acc + pre_bias[c], mult[c], shift[c]) + post_bias[c] +
    zp)`` over the ``[outer, channels, inner]`` view; int32 result."""
    lib = library()
    mult = _c(np.broadcast_to(_as_i64(mult), (channels,)), np.int64)
    shift = _c(np.broadcast_to(_as_i64(shift), (channels,)), np.int64)
    wide = acc.dtype == np.int64
    acc = _c(acc, np.int64 if wide else np.int32)
    out = np.empty(acc.shape, dtype=np.int32)
    pre = None if pre_bias is None else _c(
        np.broadcast_to(_as_i64(pre_bias), (channels,)), np.int64)
    post = None if post_bias is None else _c(
        np.broadcast_to(_as_i64(post_bias), (channels,)), np.int64)
    fn = lib.qa_requantize_i64 if wide else lib.qa_requantize_i32
    fn(_ptr(acc), _ptr(out), int(outer), int(channels), int(inner),
       _ptr(mult), _ptr(shift), _ptr(pre) if pre is not None else None,
       _ptr(post) if post is not None else None, int(zp), int(qmin),
       int(qmax))
    _check("requantize")
    return out


def rescale(x, zp_in, mult, shift, zp_out, qmin, qmax):
    """Each value moved from the input grid to the output grid:
    mbqm(x - zp_in) + zp_out, clipped (``native.py:444-462``)."""
    lib = library()
    x = _c(x, np.int32)
    out = np.empty_like(x)
    lib.qa_rescale(_ptr(x), _ptr(out), x.size, int(zp_in), int(mult),
                   int(shift), int(zp_out), int(qmin), int(qmax))
    _check("rescale")
    return out


def add(a, b, za, ma, sa, zb, mb, sb, zp_out, qmin, qmax, sign=1):
    """Integer Add / Sub: each operand brought to the output scale by its
    own fixed-point multiplier, summed with the sign, offset by the output
    zero point and clipped (``native.py:465-493``)."""
    lib = library()
    a, b = np.broadcast_arrays(a, b)
    a, b = _c(a, np.int32), _c(b, np.int32)
    out = np.empty_like(a)
    lib.qa_add(_ptr(a), _ptr(b), _ptr(out), a.size, int(za), int(ma),
               int(sa), int(zb), int(mb), int(sb), int(sign), int(zp_out),
               int(qmin), int(qmax))
    _check("add")
    return out


def mul(a, b, za, zb, mult, shift, zp_out, qmin, qmax):
    """Integer Mul: the centred product requantized by one fixed-point
    multiplier, offset and clipped (``native.py:496-518``)."""
    lib = library()
    a, b = np.broadcast_arrays(a, b)
    a, b = _c(a, np.int32), _c(b, np.int32)
    out = np.empty_like(a)
    lib.qa_mul(_ptr(a), _ptr(b), _ptr(out), a.size, int(za), int(zb),
               int(mult), int(shift), int(zp_out), int(qmin), int(qmax))
    _check("mul")
    return out


def lut(x, table, offset):
    """Lookup-table activation: the entry at x - offset, the index held
    inside the table (``native.py:521-532``)."""
    lib = library()
    table = _c(table, np.int32)
    x = _c(x, np.int32)
    out = np.empty_like(x)
    lib.qa_lut(_ptr(x), _ptr(out), x.size, int(offset), _ptr(table),
               len(table))
    _check("lut")
    return out


# ------------------------------------------------- float <-> integer ----
def quantize_f32(x, scale, zp, qmin, qmax):
    """float32 -> int32 with one scale and zero point: the double quotient
    rounded half to even, clipped (``native.py:536-546``)."""
    lib = library()
    x = _c(x, np.float32)
    out = np.empty(x.shape, dtype=np.int32)
    lib.qa_quantize_f32(_ptr(x), _ptr(out), x.size, float(scale), int(zp),
                        int(qmin), int(qmax))
    _check("quantize_f32")
    return out


def dequantize_f32(q, scale, zp):
    """int32 -> float32 with one scale and zero point, (q - zp) * scale in
    double (``native.py:549-556``)."""
    lib = library()
    q = _c(q, np.int32)
    out = np.empty(q.shape, dtype=np.float32)
    lib.qa_dequantize_f32(_ptr(q), _ptr(out), q.size, float(scale), int(zp))
    _check("dequantize_f32")
    return out
