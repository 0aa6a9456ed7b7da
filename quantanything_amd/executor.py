"""Device-resident integer executor.

Turns a calibrated container into a fixed sequence of GPU launches over
preallocated device buffers, so a whole inference pass runs without a host
round trip per node (the reference crosses Python -> C per node with host
NumPy arrays, ``quant_container.py:135-193``). The sequence can be captured
once into a HIP graph and replayed.

Storage: every quantized tensor lives on the device as int8 (types of at most
8 bits) or int16 (9-16 bits) holding ``q - so``, ``so`` = 0 for signed types
and 2^(bits-1) for unsigned ones. 4-D tensors are channels-last: element
(n, c, pix) at ``offset + n*sn + c*sc + pix*sp`` with ``sc = 1`` and a pixel
stride ``sp`` of the channel count rounded up to 16 for int8 (4 for tensors
of at most 4 channels), which keeps every 16-channel group of a pixel one
aligned 16-byte load for the MFMA kernel. ``Split`` outputs are channel views
into their input's buffer (no copy).

Fusion: a Conv / Gemm whose output feeds only a lookup-table activation runs
the table in its epilogue; if that result feeds only an Add whose other
operand already exists, the Add runs in the same epilogue; if the final
result (or the Split views of it) is a Concat input, the epilogue also writes
the rescaled copy straight into the Concat buffer. Every fused step applies
the same integer operations, in the same order, as the separate layers.

torch is used for device memory, the stream and graph capture only; all
arithmetic is in ``libqa_hip.so``.
"""

import ctypes

import numpy as np
import torch

from quantanything_amd import float_ops, native

_I64 = ctypes.c_int64
_P = ctypes.c_void_p
IDENTITY = (1 << 30, -1)  # multiplier exactly 1.0
TAIL = 64  # slack bytes after every buffer (16-byte group over-reads)


class ConvDesc(ctypes.Structure):
    """``qa_conv_desc`` of ``include/qa_hip.h`` (all fields 8 bytes)."""

    _fields_ = (
        [("x", _P)] + [(n, _I64) for n in ("x_code", "x_sn", "x_sc", "x_sp",
                                          "x_add")]
        + [(n, _I64) for n in ("N", "C", "H", "W", "Cout", "KH", "KW", "SH",
                               "SW", "PH", "PW", "DH", "DW", "G", "OH", "OW")]
        + [("w", _P)] + [(n, _I64) for n in ("w_code", "w_layout", "w_kgp",
                                            "w_rows", "wide", "needs_rowsum")]
        + [(n, _P) for n in ("epi_plan", "corr", "boff", "pre_bias", "mult",
                             "shift")]
        + [(n, _I64) for n in ("zp", "qmin", "qmax")]
        + [("lut", _P), ("lut_offset", _I64), ("lut_len", _I64)]
        + [("res", _P)] + [(n, _I64) for n in ("res_sn", "res_sc", "res_sp",
                                              "res_so", "res_first")]
        + [(n, _I64) for n in ("za", "ma", "sa", "zb", "mb", "sb", "add_sign",
                               "add_zp", "add_qmin", "add_qmax")]
        + [("y", _P)] + [(n, _I64) for n in ("y_code", "y_sn", "y_sc", "y_sp",
                                            "y_so")]
        + [("y2", _P)] + [(n, _I64) for n in ("y2_sn", "y2_sc", "y2_sp",
                                             "r2_zp_in", "r2_m", "r2_s",
                                             "r2_zp_out", "r2_qmin",
                                             "r2_qmax")]
        + [("tile", _I64), ("wsplit", _P), ("wsplit_k", _P),
           ("w_frag", _P)])


def storage_of(bits, signed):
    """``(code, torch dtype, storage offset)`` of a quantization type."""
    if bits <= 8:
        return 1, torch.int8, 0 if signed else 128
    if bits <= 16:
        return 2, torch.int16, 0 if signed else 32768
    raise NotImplementedError(f"{bits}-bit tensors are not supported on the "
                              "device")


class DeviceTensor:
    """A quantized tensor (or view) resident in device memory.

    ``shape`` is the logical (NCHW / [N, F] / N-D) shape. 4-D and 2-D
    tensors: element (n, c, pix) is at element offset ``offset + n*sn +
    c*sc + pix*sp``. Any tensor: element index i at ``offset + sum
    i_k * nd_strides[k]``; ``strides`` is given for views that are not of
    the (n, c, pix) form (``nhwc`` is then False)."""

    def __init__(self, buf, offset, shape, sn, sc, sp, code, so, qp,
                 strides=None):
        self.buf, self.offset = buf, int(offset)
        self.shape = tuple(int(s) for s in shape)
        self.sn, self.sc, self.sp = int(sn), int(sc), int(sp)
        self.code, self.so, self.qp = code, int(so), qp
        self._strides = None if strides is None else \
            tuple(int(v) for v in strides)
        self.nhwc = True

    @staticmethod
    def nd(buf, offset, shape, strides, code, so, qp):
        """View with explicit N-D element strides."""
        shape, strides = tuple(shape), tuple(strides)
        t = DeviceTensor(buf, offset, shape, strides[0] if strides else 0,
                         strides[1] if len(strides) > 1 else 1, 0, code, so,
                         qp, strides)
        if len(shape) == 4 and (shape[3] == 1 or shape[2] == 1 or
                                strides[2] == shape[3] * strides[3]):
            t.sp = strides[3] if shape[3] > 1 else strides[2] // max(
                shape[3], 1)
        elif len(shape) == 4:
            t.nhwc = False
        elif len(shape) != 2:
            t.nhwc = False
        return t

    @property
    def nd_strides(self):
        if self._strides is not None:
            return self._strides
        if len(self.shape) == 4:
            return (self.sn, self.sc, self.shape[3] * self.sp, self.sp)
        if len(self.shape) == 2:
            return (self.sn, self.sc)
        raise NotImplementedError(f"{len(self.shape)}-D tensor without "
                                  "strides")

    def meta(self):
        """A storage-free torch tensor of this view's shape and strides
        (storage offset 0), for computing the strides of derived views."""
        return torch.empty_strided(self.shape, self.nd_strides,
                                   dtype=self.buf.dtype, device="meta")

    def derived(self, m):
        """The view of this tensor's buffer that the meta tensor ``m``
        (derived from :meth:`meta`) describes."""
        return DeviceTensor.nd(self.buf, self.offset + m.storage_offset(),
                               tuple(m.shape), tuple(m.stride()), self.code,
                               self.so, self.qp)

    @property
    def ptr(self):
        return self.buf.data_ptr() + self.offset * self.buf.element_size()

    @property
    def channels(self):
        return self.shape[1]

    @property
    def pixels(self):
        return int(np.prod(self.shape[2:], dtype=np.int64))

    def rows_view(self):
        """``(rows, cols, row_stride)`` of the tensor as a strided matrix
        (4-D: rows = N*pixels, cols = channels; N-D: rows = all but the last
        axis, cols = the last axis), or None when not expressible."""
        if self._strides is not None and (len(self.shape) != 2 or
                                          self._strides[1] != 1):
            sh, st = self.shape, self._strides
            if not sh:
                return 1, 1, 1  # a scalar
            if st[-1] != 1 and sh[-1] > 1:
                return None
            dims = [(n, v) for n, v in zip(sh[:-1], st[:-1]) if n > 1]
            for (n0, s0), (n1, s1) in zip(dims, dims[1:]):
                if s0 != n1 * s1:
                    return None
            rs = dims[-1][1] if dims else sh[-1]
            return int(np.prod(sh[:-1], dtype=np.int64)), sh[-1], rs
        if len(self.shape) == 2:
            return self.shape[0], self.shape[1], self.sn
        if len(self.shape) == 4 and self.sc == 1 and self.pixels == 1:
            return self.shape[0], self.channels, self.sn  # e.g. [N, C, 1, 1]
        if len(self.shape) == 4 and self.sc == 1 and \
                self.sn == self.pixels * self.sp:
            return self.shape[0] * self.pixels, self.channels, self.sp
        return None

    def row_major(self):
        """True when the elements are dense in row-major logical order."""
        st = self.nd_strides
        want = 1
        for n, v in zip(reversed(self.shape), reversed(st)):
            if n > 1 and v != want:
                return False
            want *= n
        return True

    def contiguous_2d(self):
        return len(self.shape) == 2 and self.sn == self.shape[1] and \
            self.sc == 1

    def to_host(self):
        """Quantized values ``q`` as an int32 NumPy array (logical shape)."""
        if self._strides is not None:
            v = torch.as_strided(self.buf, self.shape, self._strides,
                                 self.offset)
        elif len(self.shape) == 4:
            n, c, h, w = self.shape
            v = torch.as_strided(self.buf, (n, c, h, w),
                                 (self.sn, self.sc, w * self.sp, self.sp),
                                 self.offset)
        else:
            v = torch.as_strided(self.buf, self.shape, (self.sn, self.sc),
                                 self.offset)
        return v.to(torch.int32).cpu().numpy() + self.so


class NdCopy(ctypes.Structure):
    """``qa_nd_copy`` of ``include/qa_hip.h``."""

    _fields_ = ([("x", _P), ("x_code", _I64), ("x_so", _I64), ("y", _P),
                 ("y_code", _I64), ("y_so", _I64), ("ndim", _I64),
                 ("shape", _I64 * 6), ("xs", _I64 * 6), ("ys", _I64 * 6)]
                + [(n, _I64) for n in ("mode", "zp_in", "m", "s", "zp_out",
                                       "qmin", "qmax")]
                + [("in_scale", ctypes.c_double), ("in_zp", _I64),
                   ("out_scale", ctypes.c_double)])


class PadDesc(ctypes.Structure):
    """``qa_nd_pad`` of ``include/qa_hip.h``."""

    _fields_ = ([("x", _P), ("code", _I64), ("y", _P), ("ndim", _I64)]
                + [(n, _I64 * 6) for n in ("shape", "lo", "xshape", "xs",
                                           "ys")]
                + [("fill", _I64)])


class MaxPoolDesc(ctypes.Structure):
    """``qa_maxpool_desc`` of ``include/qa_hip.h``."""

    _fields_ = ([("x", _P)]
                + [(n, _I64) for n in ("code", "x_sn", "x_sc", "x_sh", "x_sw",
                                       "N", "C", "H", "W", "KH", "KW", "SH",
                                       "SW", "DH", "DW", "PT", "PL", "OH",
                                       "OW", "pad")]
                + [("y", _P)]
                + [(n, _I64) for n in ("y_sn", "y_sc", "y_sh", "y_sw")])


_D = ctypes.c_double


class FbBinary(ctypes.Structure):
    """``qa_fb_binary`` of ``include/qa_hip.h``."""

    _fields_ = ([("a", _P)] + [(n, _I64) for n in ("a_code", "a_so", "a_zp")]
                + [("a_scale", _D), ("as_", _I64 * 6), ("b", _P)]
                + [(n, _I64) for n in ("b_code", "b_so", "b_zp")]
                + [("b_scale", _D), ("bs", _I64 * 6), ("y", _P)]
                + [(n, _I64) for n in ("y_code", "y_so")]
                + [("ys", _I64 * 6), ("ndim", _I64), ("shape", _I64 * 6),
                   ("op", _I64), ("out_scale", _D)]
                + [(n, _I64) for n in ("out_zp", "qmin", "qmax")])


class BinaryNd(ctypes.Structure):
    """``qa_binary_nd`` of ``include/qa_hip.h``."""

    _fields_ = ([("a", _P), ("b", _P), ("y", _P)]
                + [(n, _I64) for n in ("a_code", "b_code", "y_code", "a_so",
                                       "b_so", "y_so", "ndim")]
                + [("shape", _I64 * 6), ("as_", _I64 * 6), ("bs", _I64 * 6),
                   ("ys", _I64 * 6)]
                + [(n, _I64) for n in ("op", "za", "ma", "sa", "zb", "mb",
                                       "sb", "sign", "zp_out", "qmin",
                                       "qmax")])


class FbReduce(ctypes.Structure):
    """``qa_fb_reduce`` of ``include/qa_hip.h``."""

    _fields_ = ([("x", _P)] + [(n, _I64) for n in ("x_code", "x_so", "x_zp")]
                + [("x_scale", _D), ("nkeep", _I64), ("keep", _I64 * 6),
                   ("xks", _I64 * 6), ("nred", _I64), ("red", _I64 * 6),
                   ("xrs", _I64 * 6), ("y", _P)]
                + [(n, _I64) for n in ("y_code", "y_so")]
                + [("out_scale", _D)]
                + [(n, _I64) for n in ("out_zp", "qmin", "qmax")])


class FbSoftmax(ctypes.Structure):
    """``qa_fb_softmax`` of ``include/qa_hip.h``."""

    _fields_ = ([("x", _P)] + [(n, _I64) for n in ("x_code", "x_so", "x_zp")]
                + [("x_scale", _D)]
                + [(n, _I64) for n in ("outer", "len", "inner", "xs_o",
                                       "xs_k", "xs_i")]
                + [("y", _P)]
                + [(n, _I64) for n in ("y_code", "y_so", "ys_o", "ys_k",
                                       "ys_i", "log")]
                + [("out_scale", _D)]
                + [(n, _I64) for n in ("out_zp", "qmin", "qmax")])


class FbAvgPool(ctypes.Structure):
    """``qa_fb_avgpool`` of ``include/qa_hip.h``."""

    _fields_ = ([("x", _P)] + [(n, _I64) for n in ("x_code", "x_so", "x_zp")]
                + [("x_scale", _D)]
                + [(n, _I64) for n in ("x_sn", "x_sc", "x_sh", "x_sw", "N",
                                       "C", "H", "W", "KH", "KW", "SH", "SW",
                                       "PT", "PL", "OH", "OW", "count_pad")]
                + [("y", _P)]
                + [(n, _I64) for n in ("y_code", "y_so", "y_sn", "y_sc",
                                       "y_sh", "y_sw")]
                + [("out_scale", _D)]
                + [(n, _I64) for n in ("out_zp", "qmin", "qmax")])


class FbPad(ctypes.Structure):
    """``qa_fb_pad`` of ``include/qa_hip.h``."""

    _fields_ = ([("x", _P)] + [(n, _I64) for n in ("x_code", "x_so", "x_zp")]
                + [("x_scale", _D), ("y", _P)]
                + [(n, _I64) for n in ("y_code", "y_so", "ndim")]
                + [(n, _I64 * 6) for n in ("shape", "lo", "xshape", "xs",
                                           "ys")]
                + [("mode", _I64), ("value", _D), ("out_scale", _D)]
                + [(n, _I64) for n in ("out_zp", "qmin", "qmax")])


class FbGather(ctypes.Structure):
    """``qa_fb_gather`` of ``include/qa_hip.h``."""

    _fields_ = ([("x", _P)] + [(n, _I64) for n in ("x_code", "x_so", "x_zp")]
                + [("x_scale", _D), ("idx", _P)]
                + [(n, _I64) for n in ("nidx", "axis", "cast_to")]
                + [("y", _P)]
                + [(n, _I64) for n in ("y_code", "y_so", "ndim")]
                + [(n, _I64 * 6) for n in ("shape", "xs", "ys")]
                + [("out_scale", _D)]
                + [(n, _I64) for n in ("out_zp", "qmin", "qmax")])


# ONNX element types a Cast fallback handles on the device (qa_fb_gather)
CAST_CODES = frozenset({1, 2, 3, 4, 5, 6, 7, 9, 10, 11})


def _collapse(shape, strides, lo, hi):
    """The element stride of axes lo..hi-1 taken as one index (row-major
    order), or None when their strides do not allow it; 0 for no axes."""
    dims = [(n, s) for n, s in zip(shape[lo:hi], strides[lo:hi]) if n > 1]
    for (n0, s0), (n1, s1) in zip(dims, dims[1:]):
        if s0 != n1 * s1:
            return None
    return dims[-1][1] if dims else 0


class MatmulDesc(ctypes.Structure):
    """``qa_matmul_desc`` of ``include/qa_hip.h``."""

    _fields_ = ([("a", _P)] + [(n, _I64) for n in ("a_code", "a_so", "a_zp")]
                + [("a_scale", ctypes.c_double)]
                + [(n, _I64) for n in ("a_s0", "a_s1", "a_sm", "a_sk")]
                + [("b", _P)] + [(n, _I64) for n in ("b_code", "b_so", "b_zp")]
                + [("b_scale", ctypes.c_double)]
                + [(n, _I64) for n in ("b_s0", "b_s1", "b_sn", "b_sk", "B0",
                                       "B1", "M", "N", "K")]
                + [("y", _P)] + [(n, _I64) for n in ("y_code", "y_so", "y_s0",
                                                     "y_s1", "y_sm", "y_sn")]
                + [("out_scale", ctypes.c_double)]
                + [(n, _I64) for n in ("out_zp", "qmin", "qmax")])


class AttentionDesc(ctypes.Structure):
    """``qa_attention_desc`` of ``include/qa_hip.h``."""

    _fields_ = ([("qk", MatmulDesc), ("table", _P),
                 ("p_scale", ctypes.c_double)]
                + [(n, _I64) for n in ("p_zp", "p_qmin", "p_qmax", "p_so")]
                + [("av", MatmulDesc)])


class PoolParams(ctypes.Structure):
    """``qa_pool_params`` of ``include/qa_hip.h``."""

    _fields_ = ([(n, _I64) for n in ("in_zp", "mult", "shift", "zp", "qmin",
                                     "qmax")]
                + [("out", _P), ("out_sn", _I64), ("out_so", _I64)])


class EpiParams(ctypes.Structure):
    """``qa_epi_params`` of ``include/qa_hip.h`` (all fields 8 bytes)."""

    _fields_ = (
        [("cout", _I64)] + [(n, _P) for n in ("mult", "shift", "pre_bias")]
        + [(n, _I64) for n in ("zp", "qmin", "qmax")]
        + [("lut", _P), ("lut_offset", _I64), ("lut_len", _I64)]
        + [(n, _I64) for n in ("has_res", "res_first", "res_so", "za", "ma",
                               "sa", "zb", "mb", "sb", "add_sign", "add_zp",
                               "add_qmin", "add_qmax", "has_y2", "r2_zp_in",
                               "r2_m", "r2_s", "r2_zp_out", "r2_qmin",
                               "r2_qmax", "y_so")])


def plan_epilogue(lib, d, mult, shift, pre=None, lut=None):
    """Host plan of the int8 table epilogue for the parameters held in the
    conv descriptor ``d`` (per-channel ``mult`` / ``shift`` / ``pre`` and the
    activation table ``lut`` as host arrays). Returns the plan bytes (NumPy
    uint8) or None when the parameters need the 128-bit epilogue."""
    cout = int(d.Cout)
    mult = np.ascontiguousarray(np.broadcast_to(mult, (cout,)), np.int64)
    shift = np.ascontiguousarray(np.broadcast_to(shift, (cout,)), np.int64)
    e = EpiParams()
    e.cout, e.mult, e.shift = cout, mult.ctypes.data, shift.ctypes.data
    keep = [mult, shift]
    if pre is not None:
        pre = np.ascontiguousarray(np.broadcast_to(pre, (cout,)), np.int64)
        keep.append(pre)
        e.pre_bias = pre.ctypes.data
    e.zp, e.qmin, e.qmax = d.zp, d.qmin, d.qmax
    if lut is not None:
        lut = np.ascontiguousarray(lut, np.int32)
        keep.append(lut)
        e.lut, e.lut_offset, e.lut_len = lut.ctypes.data, d.lut_offset, \
            len(lut)
    if d.res:
        e.has_res, e.res_first, e.res_so = 1, d.res_first, d.res_so
        (e.za, e.ma, e.sa, e.zb, e.mb, e.sb, e.add_sign, e.add_zp,
         e.add_qmin, e.add_qmax) = (d.za, d.ma, d.sa, d.zb, d.mb, d.sb,
                                    d.add_sign, d.add_zp, d.add_qmin,
                                    d.add_qmax)
    if d.y2:
        e.has_y2 = 1
        (e.r2_zp_in, e.r2_m, e.r2_s, e.r2_zp_out, e.r2_qmin, e.r2_qmax) = (
            d.r2_zp_in, d.r2_m, d.r2_s, d.r2_zp_out, d.r2_qmin, d.r2_qmax)
    e.y_so = d.y_so
    plan = np.zeros(lib.qa_epi_plan_bytes(cout), np.uint8)
    rc = lib.qa_plan_epilogue_i8(ctypes.byref(e), plan.ctypes.data)
    if rc < 0:
        raise ValueError("qa_plan_epilogue_i8: bad arguments")
    return plan if rc == 1 else None


# Tiles of the FP64 matrix-core path (qa_conv_f64.hip): 16-channel groups
# wm | 16-pixel tiles per wave tm << 4 | K split over the work-group << 8.
F64_TILES = (0x11, 0x12, 0x41, 0x111, 0x112, 0x114)
# Band heights (output rows a work-group) timed for the band kernels, beside
# the library's own choice.
BAND_ROWS = (1, 2, 3, 4, 6, 8, 12)
# Element types tried, in order, for that path's packed weights.
F64_WEIGHT_TYPES = (np.int16, np.int32)


def _dev(a, dtype):
    return torch.from_numpy(np.array(a, dtype=dtype, copy=True)).cuda()


def _ok(rc, what):
    if rc != 0:
        err = native.library().qa_last_error()
        native.library().qa_clear_error()
        raise RuntimeError(f"{what} failed: {err.decode() if err else rc}")


class DeviceExecutor:
    """Plans and runs one integer inference pass for fixed input shapes.
    ``fuse_attention``: q k^T -> Softmax -> . v as one launch where it
    applies (identical results; the scores and probabilities are then not
    kept as tensors)."""

    def __init__(self, container, input_shapes, fuse_attention=True):
        self.lib = native.require()
        self.fuse_attention = fuse_attention
        self.c = container
        self.graph = container.graph
        bits, signed = container.layers[0].bits, \
            container.layers[0].signed
        self.code, self.dtype, self.so = storage_of(bits, signed)
        self.launches = []  # (name, fn(stream))
        self.keep = []  # host objects that launches point into
        self.tensors = {}
        self.epi = {}  # tensor -> (desc, first channel) written by an epilogue
        self.mfma_descs = []  # (desc, host params, host table, launch name)
        self.inputs_f32 = {}
        self.input_q = {}  # graph input -> (float buffer, int8 tensor, qp)
        self.softmax_of = {}  # Softmax output -> (launch name, arguments)
        # activation MatMul output -> (launch name, desc, first operand)
        self.matmul_act = {}
        # table Softmax output -> (launch name, input, table, out qp, so)
        self.softmax_lut = {}
        self.gap_info = {}  # pool launch -> layer, input, output, parameters
        self.pair_descs = {}  # fused pair launch -> (first, second desc)
        self.pool_descs = {}  # fused conv + pool launch -> (desc, params)
        self.tunables = []  # (launch name, desc, tile codes, fn(stream))
        self.f64_descs = []  # (desc, None, None, launch name), FP64 path
        self.outputs_f32 = {}
        self.cuda_graph = None
        self._plan(input_shapes)

    # -------------------------------------------------------------- utils --
    def _new(self, shape, qp, dense=False):
        """Fresh channels-last (4-D, unless ``dense``) or row-major tensor
        (``dense``: row-major in the logical order, for the N-D operators
        of transformers). Buffers start zeroed once, at planning: no kernel
        writes the padding channels of a channels-last pixel, and the int8
        MFMA path's pixel sums (weight rows with an offset) read them."""
        shape = tuple(int(s) for s in shape)
        if len(shape) == 4 and not dense:
            n, c, h, w = shape
            if c <= 4:
                cs = 4
            elif self.code == 1:
                cs = -(-c // 16) * 16
            else:
                cs = c
            numel = n * h * w * cs
            buf = torch.zeros(numel + TAIL, dtype=self.dtype, device="cuda")
            return DeviceTensor(buf, 0, shape, h * w * cs, 1, cs, self.code,
                                self.so, qp)
        if len(shape) == 2 and not dense:
            numel = shape[0] * shape[1]
            buf = torch.zeros(numel + TAIL, dtype=self.dtype, device="cuda")
            return DeviceTensor(buf, 0, shape, shape[1], 1, 0, self.code,
                                self.so, qp)
        if len(shape) > 6:
            raise NotImplementedError(f"{len(shape)}-D tensors on the device")
        numel = int(np.prod(shape, dtype=np.int64))  # 1 for a scalar
        buf = torch.zeros(numel + TAIL, dtype=self.dtype, device="cuda")
        strides = tuple(int(np.prod(shape[k + 1:], dtype=np.int64))
                        for k in range(len(shape)))
        return DeviceTensor.nd(buf, 0, shape, strides, self.code, self.so, qp)

    def _copy(self, name, x, y, mode=0, rescale=None, requant=None):
        """Launch copying x into the view y (same logical shape): mode 0
        unchanged, 1 integer rescale ``(zp_in, m, s, zp_out, qmin, qmax)``,
        2 float requantization ``(in_scale, in_zp, out_scale, zp_out, qmin,
        qmax)``."""
        d = NdCopy()
        d.x, d.x_code, d.x_so = x.ptr, x.code, x.so
        d.y, d.y_code, d.y_so = y.ptr, y.code, y.so
        shape = x.shape or (1,)
        d.ndim = len(shape)
        xs, ys = x.nd_strides or (0,), y.nd_strides or (0,)
        for k in range(len(shape)):
            d.shape[k], d.xs[k], d.ys[k] = shape[k], xs[k], ys[k]
        d.mode = mode
        d.qmin, d.qmax = -(1 << 62), 1 << 62
        if mode == 1:
            d.zp_in, d.m, d.s, d.zp_out, d.qmin, d.qmax = rescale
        elif mode == 2:
            (d.in_scale, d.in_zp, d.out_scale, d.zp_out, d.qmin,
             d.qmax) = requant
        self.keep.extend([d, x.buf, y.buf])  # the launch's raw pointers
        self._add(name, lambda s, d=d: _ok(self.lib.qa_d_copy_nd(
            ctypes.byref(d), s), "qa_d_copy_nd"))

    def _new_for_users(self, name, shape, qp):
        """A dense output, laid out in the order its only consumer, a
        Transpose, reads it (so that the Transpose and a following Reshape
        are views rather than copies)."""
        users = self._cons.get(name, [])
        if name not in self.graph.outputs and len(users) == 1 and \
                users[0].node.op_type == "Transpose" and \
                users[0].kind == "shape":
            perm = users[0].node.attr("perm") or \
                list(range(len(shape)))[::-1]
            t = self._new([shape[p] for p in perm], qp, dense=True)
            return t.derived(t.meta().permute(*np.argsort(perm).tolist()))
        return self._new(shape, qp, dense=True)

    def _contiguous(self, name, x):
        """x itself when row-major dense, else a dense copy."""
        if x.row_major():
            return x
        y = self._new(x.shape, x.qp, dense=True)
        self._copy(name, x, y)
        return y

    def _add(self, name, fn):
        self.launches.append((name, fn))

    @staticmethod
    def _params(layer):
        if getattr(layer, "_dev_params", None) is None:
            layer._dev_params = {}
        return layer._dev_params

    # ------------------------------------------------------------ planning --
    def _plan(self, input_shapes):
        c, g = self.c, self.graph
        for name, shape in input_shapes.items():
            qp = c.qparams[name]
            shape = tuple(shape)
            xf = torch.empty(shape, dtype=torch.float32, device="cuda")
            self.inputs_f32[name] = xf
            if len(shape) == 4:
                t = self._new(shape, qp)
                self.input_q[name] = (xf, t, qp)
                n, ch, h, w = shape
                self._add(f"quantize:{name}", lambda s, xf=xf, t=t, n=n,
                          ch=ch, hw=h * w, qp=qp: _ok(
                              self.lib.qa_d_quantize_nhwc(
                                  xf.data_ptr(), n, ch, hw, t.ptr, t.code,
                                  t.sp, qp.scale, qp.zp, qp.qmin, qp.qmax,
                                  t.so, s), "quantize"))
            else:
                t = self._new(shape, qp)
                numel = xf.numel()
                self._add(f"quantize:{name}", lambda s, xf=xf, t=t,
                          numel=numel, qp=qp: _ok(
                              self.lib.qa_d_quantize_f32(
                                  xf.data_ptr(), t.ptr, t.code, numel,
                                  qp.scale, qp.zp, qp.qmin, qp.qmax, t.so, s),
                              "quantize"))
            self.tensors[name] = t
        for name in c.const_names:
            # quantized constant operands (e.g. a position embedding),
            # uploaded once, stored as q - so
            q = np.asarray(c.const_q[name], dtype=np.int64)
            t = self._new(q.shape, c.qparams[name], dense=True)
            host = torch.from_numpy((q - t.so).astype(
                np.int8 if self.code == 1 else np.int16).reshape(-1))
            t.buf[:host.numel()].copy_(host)
            self.tensors[name] = t

        layers = c.layers
        producer = g.producer_index()
        cons = {}
        for l in layers:
            for i in l.data_inputs:
                cons.setdefault(i, []).append(l)
        self._cons = cons
        absorbed = set()
        for layer in layers:
            if layer.name in absorbed:
                continue
            layer.check_ready()
            ins = [self.tensors[n] for n in layer.data_inputs]
            if layer.kind in ("conv", "gemm"):
                lut_layer = add_layer = res = None
                out_name = layer.node.outputs[0]
                users = cons.get(out_name, [])
                if out_name not in g.outputs and len(users) == 1 and \
                        users[0].kind == "table":
                    lut_layer = users[0]
                    out_name = lut_layer.node.outputs[0]
                    users = cons.get(out_name, [])
                if out_name not in g.outputs and len(users) == 1 and \
                        users[0].kind == "add" and \
                        len(users[0].data_inputs) == 2:
                    a = users[0]
                    others = [i for i in a.data_inputs if i != out_name]
                    if len(others) == 1 and others[0] in self.tensors and \
                            producer.get(others[0], -1) < \
                            producer.get(layer.node.outputs[0], 0):
                        add_layer = a
                        res = (others[0], a.data_inputs[0] == others[0])
                final = add_layer or lut_layer or layer
                y = self._plan_weighted(layer, ins[0], lut_layer, add_layer,
                                        res)
                for l in (lut_layer, add_layer):
                    if l is not None:
                        absorbed.add(l.name)
                self.tensors[final.node.outputs[0]] = y
                continue
            outs = getattr(self, "_plan_" + layer.kind)(layer, ins)
            for name, t in zip(layer.node.outputs, outs):
                self.tensors[name] = t
        self._plan_epilogues()
        self._fuse_patch_input(cons)
        self._fuse_input_quantization(cons)
        self._fuse_pools(cons)
        self._fuse_pool_heads(cons)
        self._fuse_pairs(cons)
        self._fuse_pair_tails(cons)
        self._fuse_chains(cons)
        if self.fuse_attention:
            self._fuse_attention(cons)
        live = dict(self.launches)
        for d, _, _, name in self.mfma_descs:
            # the narrow-GEMM kernel's weights in fragment order
            if name in live and self.narrow_ok(d):
                self._frag_weights(d)
        for d, _, _, name in self.mfma_descs + self.f64_descs:
            if name in dict(self.launches):
                self.tunables.append(
                    (name, d, self.tile_candidates(d),
                     lambda s, d=d: _ok(self.lib.qa_d_conv(ctypes.byref(d), s),
                                        "qa_d_conv")))
        for name in g.outputs:
            t = self.tensors[name]
            if not (t.contiguous_2d() or (t._strides is not None and
                                          t.row_major())):
                # a dense copy that the dequantization reads
                t = self._contiguous(f"copy:{name}", DeviceTensor.nd(
                    t.buf, t.offset, t.shape, t.nd_strides, t.code, t.so,
                    t.qp))
                self.tensors[name] = t
            yf = torch.empty(t.shape, dtype=torch.float32, device="cuda")
            self.outputs_f32[name] = yf
            sm = self.softmax_of.get(name)
            if sm is not None:  # the Softmax writes the float copy too
                lname, with_f32 = sm
                fused = (lname, lambda s, f=with_f32, yf=yf: f(s, yf))
                self.launches = [fused if n == lname else (n, f)
                                 for n, f in self.launches]
                continue
            n = yf.numel()
            self._add(f"dequantize:{name}", lambda s, t=t, yf=yf, n=n:
                      _ok(self.lib.qa_d_dequantize_f32(
                          t.ptr, t.code, yf.data_ptr(), n, t.qp.scale,
                          t.qp.zp, t.so, s), "dequantize"))

    # ---------------------------------------------------- conv and gemm --
    def _mfma_ok(self, layer, x, layout, groups, cg, k_real):
        if self.code != 1 or layer.wide or k_real >= 131072:
            return False
        off_bytes = x.offset  # int8 elements are bytes
        if layout == 1:
            return groups == 1 and x.sp % 4 == 0 and x.sn % 4 == 0 and \
                off_bytes % 4 == 0
        pix = x.pixels if len(x.shape) == 4 else 1
        return off_bytes % 16 == 0 and x.sn % 16 == 0 and \
            (pix == 1 or x.sp % 16 == 0) and (groups == 1 or cg % 16 == 0)

    @staticmethod
    def _f64_ok(x, a_off):
        """16-bit activations the FP64 matrix-core path takes: channels
        contiguous, centred values within 2^17."""
        return x.code == 2 and x.sc == 1 and -65536 <= a_off <= 65536

    def _weights_dev(self, layer, x, layout, use_mfma):
        p = self._params(layer)
        a_off = x.so - layer.in_zp
        key = ("w", a_off, self.code, layout, use_mfma)
        if key in p:
            return p[key]
        if layer.kind == "gemm":
            w = np.ascontiguousarray(layer.w_centered.T)[:, :, None, None]
            groups = 1
        else:
            w = layer.w_centered
            groups = layer.geometry(x.shape)[3]
        cout, cg, kh, kw = w.shape
        w32 = np.ascontiguousarray(w, dtype=np.int32)
        info = None
        if use_mfma:
            kgp, rows = _I64(0), _I64(0)
            size = self.lib.qa_pack_weights_i8_size(
                cout, cg, kh, kw, groups, layout, ctypes.byref(kgp),
                ctypes.byref(rows))
            wp = np.empty(size, np.int8)
            corr = np.empty(cout, np.int64)
            boff = np.empty(cout, np.int32)
            need = ctypes.c_int32(0)
            rc = self.lib.qa_pack_weights_i8(
                w32.ctypes.data, cout, cg, kh, kw, groups, a_off, layout,
                wp.ctypes.data, corr.ctypes.data, boff.ctypes.data,
                ctypes.byref(need))
            if rc == 0:
                info = dict(w=_dev(wp, np.int8), w_code=1, layout=layout,
                            kgp=kgp.value, rows=rows.value,
                            corr=_dev(corr, np.int64),
                            boff=_dev(boff, np.int32), rowsum=need.value,
                            wide=0)
        if info is None and self._f64_ok(x, a_off):
            ck, rows = _I64(0), _I64(0)
            size = self.lib.qa_pack_weights_f64_size(
                cout, cg, kh, kw, groups, ctypes.byref(ck), ctypes.byref(rows))
            for dt in F64_WEIGHT_TYPES:  # the narrowest element that fits
                wf = np.empty(size, dt)
                if self.lib.qa_pack_weights_f64(
                        w32.ctypes.data, cout, cg, kh, kw, groups,
                        wf.itemsize, wf.ctypes.data) == 0:
                    info = dict(w=_dev(wf, dt), w_code=8, layout=wf.itemsize,
                                kgp=ck.value, rows=rows.value, corr=None,
                                boff=None, rowsum=0, wide=1)
                    if dt == np.int16 and (cg % 16 == 0 or
                                           (cg <= 4 and groups == 1)):
                        # the same weights as two int8 planes: the library
                        # may run the byte-split form on the int8 cores
                        kgp8, rows8 = _I64(0), _I64(0)
                        n8 = self.lib.qa_pack_weights_i8_size(
                            cout, cg, kh, kw, groups, 0, ctypes.byref(kgp8),
                            ctypes.byref(rows8))
                        ws = np.empty(2 * n8, np.int8)
                        wsum = np.empty(cout, np.int64)
                        if self.lib.qa_pack_weights_i16s(
                                w32.ctypes.data, cout, cg, kh, kw, groups,
                                ws.ctypes.data, wsum.ctypes.data) == 0:
                            info["wsplit"] = _dev(ws, np.int8)
                            info["wsum"] = wsum
                    break
        if info is None:  # exact VALU path, int64 accumulation
            info = dict(w=_dev(w32, np.int32), w_code=4, layout=0, kgp=0,
                        rows=0, corr=None, boff=None, rowsum=0, wide=1)
        mult = np.broadcast_to(layer.q_mult, (cout,)).astype(np.int64)
        shift = np.broadcast_to(layer.shift, (cout,)).astype(np.int64)
        info["mult"] = _dev(mult, np.int64)
        info["shift"] = _dev(shift, np.int64)
        info["pre"] = (None if layer.bias_int is None
                       else _dev(layer.bias_int, np.int64))
        info["host"] = (mult, shift, layer.bias_int)
        p[key] = info
        return info

    def _plan_weighted(self, layer, x, lut_layer, add_layer, res):
        d = ConvDesc()
        if layer.kind == "conv":
            if len(x.shape) != 4:
                raise NotImplementedError("only 2-D convolution")
            strides, pads, dil, groups = layer.geometry(x.shape)
            n, cin, h, w = x.shape
            cout, cg, kh, kw = layer.w_centered.shape
            if cin != cg * groups or cout % groups:
                raise ValueError(f"conv shape mismatch: input C={cin}, "
                                 f"weight={layer.w_centered.shape}, "
                                 f"groups={groups}")
            oh = (h + pads[0] + pads[2] - dil[0] * (kh - 1) - 1) // \
                strides[0] + 1
            ow = (w + pads[1] + pads[3] - dil[1] * (kw - 1) - 1) // \
                strides[1] + 1
            out_shape = (n, cout, oh, ow)
            geo = (n, cin, h, w, cout, kh, kw, strides[0], strides[1],
                   pads[0], pads[1], dil[0], dil[1], groups, oh, ow)
            layout = 1 if (groups == 1 and cg <= 4 and kw <= 16 and
                           x.sp == 4) else 0
        else:
            k, ncol = layer.w_centered.shape
            xv = x.rows_view()
            if x.shape[-1] != k or xv is None or \
                    (len(x.shape) == 4 and x._strides is None):
                raise NotImplementedError(
                    f"gemm input {x.shape} x {layer.w_centered.shape}")
            m = xv[0]
            out_shape = layer.out_shape(x.shape)
            geo = (m, k, 1, 1, ncol, 1, 1, 1, 1, 0, 0, 1, 1, 1, 1, 1)
            groups, cg, kh, kw, cout = 1, k, 1, 1, ncol
            layout = 0
            # rows of the input as images of one pixel
            x = DeviceTensor(x.buf, x.offset, (m, k), xv[2], 1, 0, x.code,
                             x.so, x.qp)
        if layer.kind == "conv" and (not x.nhwc or x.sc != 1):
            # rows and columns strided apart (a Slice with a step) or
            # channels not contiguous (a dense copy): the view copied into
            # a channels-last tensor, the layout the kernels read
            xc = self._new(x.shape, x.qp)
            self._copy(f"copy:{layer.name}", x, xc)
            x = xc
        use_mfma = self._mfma_ok(layer, x, layout, groups, cg, cg * kh * kw)
        info = self._weights_dev(layer, x, layout, use_mfma)
        (d.N, d.C, d.H, d.W, d.Cout, d.KH, d.KW, d.SH, d.SW, d.PH, d.PW,
         d.DH, d.DW, d.G, d.OH, d.OW) = geo
        d.x, d.x_code = x.ptr, x.code
        d.x_sn, d.x_sc, d.x_sp = x.sn, x.sc, x.sp
        d.x_add = x.so - layer.in_zp
        d.w = info["w"].data_ptr()
        d.w_code, d.w_layout = info["w_code"], info["layout"]
        d.w_kgp, d.w_rows = info["kgp"], info["rows"]
        d.wide, d.needs_rowsum = info["wide"], info["rowsum"]
        if info.get("wsplit") is not None:
            kc = _dev((128 + int(d.x_add)) * info["wsum"], np.int64)
            self.keep.append(kc)
            d.wsplit = info["wsplit"].data_ptr()
            d.wsplit_k = kc.data_ptr()
        d.corr = info["corr"].data_ptr() if info["corr"] is not None else None
        d.boff = info["boff"].data_ptr() if info["boff"] is not None else None
        d.pre_bias = info["pre"].data_ptr() if info["pre"] is not None \
            else None
        d.mult = info["mult"].data_ptr()
        d.shift = info["shift"].data_ptr()
        d.zp, d.qmin, d.qmax = layer.out_zp, layer.out_qmin, layer.out_qmax
        final_qp = layer.out_qp[0]
        if lut_layer is not None:
            p = self._params(lut_layer)
            if "lut" not in p:
                p["lut"] = _dev(lut_layer.lut, np.int32)
            d.lut = p["lut"].data_ptr()
            d.lut_offset = lut_layer.lut_offset
            d.lut_len = len(lut_layer.lut)
            final_qp = lut_layer.out_qp[0]
        y = self._new(out_shape, final_qp,
                      dense=layer.kind == "gemm" and len(out_shape) != 2)
        if add_layer is not None:
            rname, first = res
            r = self.tensors[rname]
            if r.shape != tuple(out_shape) or r.code != self.code:
                raise NotImplementedError("residual shape mismatch")
            (ma, sa), (mb, sb) = add_layer.mults
            qa_, qb_ = add_layer.in_qp
            o = add_layer.out_qp[0]
            d.res = r.ptr
            d.res_sn, d.res_sc, d.res_sp, d.res_so = r.sn, r.sc, r.sp, r.so
            if layer.kind == "gemm":
                rv = r.rows_view()
                if rv is None:
                    raise NotImplementedError("residual of a strided view")
                d.res_sn, d.res_sc, d.res_sp = rv[2], 1, 0
            d.res_first = 1 if first else 0
            d.za, d.ma, d.sa = qa_.zp, ma, sa
            d.zb, d.mb, d.sb = qb_.zp, mb, sb
            d.add_sign = add_layer.sign
            d.add_zp, d.add_qmin, d.add_qmax = o.zp, o.qmin, o.qmax
            y.qp = o
        d.y, d.y_code = y.ptr, y.code
        d.y_sn, d.y_sc, d.y_sp, d.y_so = y.sn, y.sc, y.sp, y.so
        if layer.kind == "gemm":
            d.y_sn, d.y_sc, d.y_sp = y.rows_view()[2], 1, 0
        self.keep.append(d)
        if d.w_code == 1 and d.y_code == 1:
            self.mfma_descs.append(
                (d, info["host"],
                 None if lut_layer is None else lut_layer.lut,
                 f"conv:{layer.name}"))
        if d.w_code == 8:
            self.f64_descs.append((d, None, None, f"conv:{layer.name}"))
        name = add_layer or lut_layer or layer
        self.epi[name.node.outputs[0]] = (d, 0, cout)
        self._add(f"conv:{layer.name}", lambda s, d=d:
                  _ok(self.lib.qa_d_conv(ctypes.byref(d), s), "qa_d_conv"))
        return y

    def _plan_epilogues(self):
        """Table-epilogue plans of the int8 MFMA convolutions, built once the
        descriptors are final (a later Concat may add the rescaled copy)."""
        for d, (mult, shift, pre), lut, _ in self.mfma_descs:
            plan = plan_epilogue(self.lib, d, mult, shift, pre, lut)
            if plan is not None:
                dev = _dev(plan, np.uint8)
                self.keep.append(dev)
                d.epi_plan = dev.data_ptr()

    def _fuse_patch_input(self, cons):
        """A 4-D graph input read only by an int8 convolution whose stride
        is its kernel (no padding, KW a multiple of 4, layout-1 weights: a
        transformer's patch embedding) is quantized straight into that
        convolution's im2col rows (``qa_d_quantize_patches``: the bytes of
        the channels-last tensor, permuted), and the convolution runs as a
        1x1 convolution over N*OH*OW one-pixel images of KH*KW*4 channels
        (the large-GEMM kernels), its weights in the same order."""
        for name, (xf, t, qp) in list(self.input_q.items()):
            users = cons.get(name, [])
            if name in self.graph.outputs or len(users) != 1 or \
                    users[0].kind != "conv" or t.code != 1 or t.offset:
                continue
            ln = f"conv:{users[0].name}"
            hits = [e for e in self.mfma_descs
                    if e[0].x == t.ptr and e[3] == ln]
            if len(hits) != 1:
                continue
            d, host, lut, _ = hits[0]
            if not (d.w_layout == 1 and d.G == 1 and d.KH == d.SH and
                    d.KW == d.SW and d.PH == 0 and d.PW == 0 and
                    d.DH == 1 and d.DW == 1 and d.KW % 4 == 0 and
                    d.H == d.OH * d.KH and d.W == d.OW * d.KW and
                    1 <= d.C <= 4 and d.x_sp == 4 and d.x_sc == 1 and
                    d.x_sn == d.H * d.W * 4 and d.y_sc == 1 and
                    d.y_sn == d.OH * d.OW * d.y_sp and not d.res and
                    d.y_code == 1 and d.epi_plan):
                continue
            layer = users[0]
            n, c, h, w = t.shape
            kh, kw = d.KH, d.KW
            kc = kh * kw * 4
            wc = np.asarray(layer.w_centered, np.int64)
            cout = wc.shape[0]
            # channel (ky * KW + kx) * 4 + ci of the 1x1 convolution
            w2 = np.zeros((cout, kh, kw, 4), np.int32)
            w2[..., :c] = wc.transpose(0, 2, 3, 1)
            w2 = np.ascontiguousarray(w2.reshape(cout, kc, 1, 1))
            kgp, rows = _I64(0), _I64(0)
            size = self.lib.qa_pack_weights_i8_size(
                cout, kc, 1, 1, 1, 0, ctypes.byref(kgp), ctypes.byref(rows))
            wp = np.empty(size, np.int8)
            corr = np.empty(cout, np.int64)
            boff = np.empty(cout, np.int32)
            need = ctypes.c_int32(0)
            if self.lib.qa_pack_weights_i8(
                    w2.ctypes.data, cout, kc, 1, 1, 1, int(d.x_add), 0,
                    wp.ctypes.data, corr.ctypes.data, boff.ctypes.data,
                    ctypes.byref(need)) != 0:
                continue
            dev = [_dev(wp, np.int8), _dev(corr, np.int64),
                   _dev(boff, np.int32)]
            self.keep.extend(dev)
            pix = d.y_sp
            (d.N, d.C, d.H, d.W, d.KH, d.KW, d.SH, d.SW, d.PH, d.PW, d.DH,
             d.DW, d.OH, d.OW) = (n * d.OH * d.OW, kc, 1, 1, 1, 1, 1, 1, 0,
                                  0, 1, 1, 1, 1)
            d.x_sn, d.x_sc, d.x_sp = kc, 1, 0
            d.y_sn, d.y_sc, d.y_sp = pix, 1, 0
            d.w, d.w_layout = dev[0].data_ptr(), 0
            d.w_kgp, d.w_rows = kgp.value, rows.value
            d.corr, d.boff = dev[1].data_ptr(), dev[2].data_ptr()
            d.needs_rowsum = need.value
            d.tile = 0
            plan = plan_epilogue(self.lib, d, *host, lut)
            if plan is None:
                raise RuntimeError(f"{ln}: no epilogue plan as a 1x1 "
                                   "convolution")
            pdev = _dev(plan, np.uint8)
            self.keep.append(pdev)
            d.epi_plan = pdev.data_ptr()
            qname = f"quantize:{name}"

            def fn(s, xf=xf, t=t, n=n, c=c, h=h, w=w, kh=kh, kw=kw, qp=qp):
                _ok(self.lib.qa_d_quantize_patches(
                    xf.data_ptr(), n, c, h, w, kh, kw, t.ptr, qp.scale,
                    qp.zp, qp.qmin, qp.qmax, t.so, s),
                    "qa_d_quantize_patches")

            self.launches = [(f"patches:{name}", fn) if nm == qname
                             else (nm, f) for nm, f in self.launches]
            self.keep.append(t)
            del self.tensors[name]  # holds the rows, not the image

    def _fuse_input_quantization(self, cons):
        """A 4-D graph input read only by a layout-1 (<= 4 channel) int8
        convolution with a table plan is quantized inside that convolution
        (``qa_d_quantize_conv``): the int8 input tensor is never written."""
        for name, (xf, t, qp) in self.input_q.items():
            users = cons.get(name, [])
            if name in self.graph.outputs or len(users) != 1:
                continue
            hits = [(d, ln) for d, _, _, ln in self.mfma_descs
                    if d.x == t.ptr and ln == f"conv:{users[0].name}"]
            if len(hits) != 1:
                continue
            d, ln = hits[0]
            if not (d.w_layout == 1 and d.G == 1 and d.epi_plan and
                    1 <= d.KH <= 4 and 1 <= d.KW <= 4 and not d.res and
                    not d.y2 and d.y_sc == 1 and d.y_sp % 4 == 0):
                continue
            qname = f"quantize:{name}"
            fused = f"qconv:{users[0].name}"

            def fn(s, d=d, xf=xf, qp=qp):
                _ok(self.lib.qa_d_quantize_conv(
                    ctypes.byref(d), xf.data_ptr(), qp.scale, qp.zp, qp.qmin,
                    qp.qmax, s), "qa_d_quantize_conv")

            self.launches = [(fused, fn) if n == ln else (n, f)
                             for n, f in self.launches if n != qname]
            self.keep.append(t)
            del self.tensors[name]  # never materialized
            rows = [0] + [0x10000 | r for r in (1, 2, 4, 8, 16)
                          if r <= d.OH]
            self.tunables.append((fused, d, rows, fn))

    def _fuse_pools(self, cons):
        """An int8 MFMA convolution (one group, table plan, no residual or
        second output) whose output only feeds a global average pool runs
        with the pool fused (``qa_d_conv_pool``): its output is never
        written and the pool has no launch of its own."""
        for gname, gi in list(self.gap_info.items()):
            x, layer = gi["x"], gi["layer"]
            xname = layer.data_inputs[0]
            if xname in self.graph.outputs or \
                    [l.name for l in cons.get(xname, [])] != [layer.name]:
                continue
            hits = [(d, ln) for d, _, _, ln in self.mfma_descs
                    if d.y == x.ptr and ln in dict(self.launches)]
            if len(hits) != 1:
                continue
            d, ln = hits[0]
            if not (d.epi_plan and d.G == 1 and d.w_layout == 0 and
                    not d.res and not d.y2 and d.y_code == 1 and
                    self.tensors[xname].buf.data_ptr() == x.buf.data_ptr()):
                continue
            o, y = gi["out"], gi["y"]
            pp = PoolParams()
            pp.in_zp, pp.mult, pp.shift = layer.in_zp, gi["mult"], gi["shift"]
            pp.zp, pp.qmin, pp.qmax = o.zp, o.qmin, o.qmax
            pp.out, pp.out_sn, pp.out_so = y.ptr, y.sn, y.so
            self.keep.append(pp)
            fused = f"convpool:{ln[5:]}"

            def fn(s, d=d, pp=pp):
                _ok(self.lib.qa_d_conv_pool(ctypes.byref(d), ctypes.byref(pp),
                                            s), "qa_d_conv_pool")

            self.launches = [(fused, fn) if n == ln else (n, f)
                             for n, f in self.launches if n != gname]
            codes = [0, 0x10001] + ([0x10002] if d.Cout > 64 else [])
            self.tunables.append((fused, d, codes, fn))
            self.pool_descs[fused] = (d, pp)
            self.tensors.pop(xname, None)  # never materialized

    def _frag_weights(self, d):
        """Sets ``d.w_frag``: the descriptor's int8 weights in fragment order
        (made once, on the current stream, kept with the plan)."""
        if d.w_frag:
            return
        size = self.lib.qa_fragments_i8_size(d.w_rows, d.w_kgp)
        if size <= 0:
            return
        buf = torch.empty(size, dtype=torch.int8, device="cuda")
        _ok(self.lib.qa_d_pack_fragments_i8(
            d.w, d.w_rows, d.w_kgp, buf.data_ptr(),
            torch.cuda.current_stream().cuda_stream),
            "qa_d_pack_fragments_i8")
        self.keep.append(buf)
        d.w_frag = buf.data_ptr()

    def _fuse_pool_heads(self, cons):
        """A 1x1 convolution whose output only feeds a pooled 1x1
        convolution runs in the pool's launch (``qa_d_conv_pw_pool``): the
        two layers of a classifier head before its pool in one launch, the
        intermediate kept in LDS and never written."""
        for fused, (d2, pp) in list(self.pool_descs.items()):
            live = dict(self.launches)
            if fused not in live:
                continue
            firsts = [(d, ln) for d, _, _, ln in self.mfma_descs
                      if d.y == d2.x and ln in live]
            if len(firsts) != 1:
                continue
            d1, ln1 = firsts[0]
            mids = [n for n, t in self.tensors.items() if t.ptr == d1.y]
            if len(mids) != 1 or mids[0] in self.graph.outputs or \
                    [l.name for l in cons.get(mids[0], [])] != \
                    [fused[len("convpool:"):]]:
                continue
            if not self.lib.qa_conv_pw_pool_supported(ctypes.byref(d1),
                                                      ctypes.byref(d2)):
                continue
            name = f"convpool:{ln1[5:]}+{fused[len('convpool:'):]}"
            for d in (d1, d2):  # both weight sets in fragment order
                self._frag_weights(d)

            def fn(s, d1=d1, d2=d2, pp=pp):
                _ok(self.lib.qa_d_conv_pw_pool(ctypes.byref(d1),
                                               ctypes.byref(d2),
                                               ctypes.byref(pp), s),
                    "qa_d_conv_pw_pool")

            self.launches = [(name, fn) if n == fused else (n, f)
                             for n, f in self.launches if n != ln1]
            self.tunables = [t for t in self.tunables if t[0] != fused]
            self.tensors.pop(mids[0], None)  # never materialized

    def _fuse_attention(self, cons):
        """MatMul(q, k^T) -> Softmax over its rows -> MatMul(., v), int8,
        the scores and the probabilities read by nothing else, run as one
        launch (``qa_d_attention``): both stay on chip and are never
        written; the results are those of the three launches."""
        g = self.graph
        for pname, (sm_ln, sname, x_ptr, tab, o, p_so) in \
                self.softmax_lut.items():
            qk = self.matmul_act.get(sname)
            avs = [(ln, d) for ln, d, a_name in self.matmul_act.values()
                   if a_name == pname]
            if qk is None or len(avs) != 1 or qk[1].y != x_ptr or \
                    sname in g.outputs or pname in g.outputs or \
                    len(cons.get(sname, [])) != 1 or \
                    len(cons.get(pname, [])) != 1:
                continue
            qk_ln, qkd, _ = qk
            av_ln, avd = avs[0]
            live = dict(self.launches)
            if not all(n in live for n in (qk_ln, sm_ln, av_ln)):
                continue
            ad = AttentionDesc()
            ad.qk, ad.av = qkd, avd
            ad.table = tab.data_ptr()
            ad.p_scale, ad.p_zp, ad.p_qmin, ad.p_qmax, ad.p_so = \
                o.scale, o.zp, o.qmin, o.qmax, p_so
            if not self.lib.qa_attention_supported(ctypes.byref(ad)):
                continue
            self.keep.append(ad)
            fused = f"attention:{qk_ln[7:]}+{av_ln[7:]}"

            def fn(s, ad=ad):
                _ok(self.lib.qa_d_attention(ctypes.byref(ad), s),
                    "qa_d_attention")

            self.launches = [(fused, fn) if n == av_ln else (n, f)
                             for n, f in self.launches
                             if n not in (qk_ln, sm_ln)]
            self.tensors.pop(sname, None)  # never materialized
            self.tensors.pop(pname, None)

    def _fuse_pairs(self, cons):
        """Two int8 3x3 stride-1 convolutions C -> C (C 16 to 128), the
        second the only reader of the first's output (a C2f bottleneck), run
        as one launch (``qa_d_conv_pair``): the intermediate tensor stays in
        LDS and is never written."""
        for d2, _, _, ln2 in self.mfma_descs:
            live = dict(self.launches)
            if ln2 not in live:
                continue
            firsts = [(d, ln) for d, _, _, ln in self.mfma_descs
                      if d.y == d2.x and ln in live and ln != ln2]
            if len(firsts) != 1:
                continue
            d1, ln1 = firsts[0]
            mids = [n for n, t in self.tensors.items() if t.ptr == d1.y]
            if len(mids) != 1 or mids[0] in self.graph.outputs or \
                    [l.name for l in cons.get(mids[0], [])] != [ln2[5:]]:
                continue
            if not self.lib.qa_conv_pair_supported(ctypes.byref(d1),
                                                   ctypes.byref(d2)):
                continue
            fused = f"pair:{ln1[5:]}+{ln2[5:]}"

            def fn(s, d1=d1, d2=d2):
                _ok(self.lib.qa_d_conv_pair(ctypes.byref(d1),
                                            ctypes.byref(d2), s),
                    "qa_d_conv_pair")

            if d2.Cout == 128:  # the channel-split form loads fragments
                self._frag_weights(d1)
                self._frag_weights(d2)
            self.launches = [(fused, fn) if n == ln2 else (n, f)
                             for n, f in self.launches if n != ln1]
            # band heights to time (0: the library's cost model)
            rows = [0] + [0x10000 | r for r in range(1, min(d2.OH, 16) + 1)]
            self.tunables.append((fused, d2, rows, fn))
            self.pair_descs[fused] = (d1, d2)
            self.tensors.pop(mids[0], None)  # never materialized

    def _fuse_pair_tails(self, cons):
        """A C2f block's last 1x1 convolution (cv2) whose input, the block's
        Concat, ends with the last bottleneck pair's output runs inside that
        pair's launch (``qa_d_conv_pair_tail``). The fused launch takes
        cv2's place, after every launch that writes the Concat's other
        channels, so the pair's outputs and the Concat may have no reader
        but the Concat and cv2 respectively."""
        g = self.graph
        layer_of = {l.name: l for l in self.c.layers}
        made_by = {o: l for l in self.c.layers for o in l.node.outputs}
        for fused, (d1, d2) in list(self.pair_descs.items()):
            live = dict(self.launches)
            if fused not in live:
                continue
            for d3, _, _, ln3 in self.mfma_descs:
                if ln3 not in live or d3.KH != 1 or d3.KW != 1 or \
                        not self.lib.qa_conv_pair_tail_supported(
                            ctypes.byref(d1), ctypes.byref(d2),
                            ctypes.byref(d3)):
                    continue
                cv2 = layer_of.get(ln3[5:])
                if cv2 is None:
                    continue
                cname = cv2.data_inputs[0]
                cat = made_by.get(cname)
                if cat is None or cname in g.outputs or \
                        [l.name for l in cons.get(cname, [])] != [cv2.name]:
                    continue
                outs = [n for n, t in self.tensors.items()
                        if t.ptr in (d2.y, d2.y2) and n != cname]
                if not outs or any(
                        n in g.outputs or
                        {l.name for l in cons.get(n, [])} != {cat.name}
                        for n in outs):
                    continue
                tname = f"pairtail:{fused[5:]}+{cv2.name}"

                def fn(s, d1=d1, d2=d2, d3=d3):
                    _ok(self.lib.qa_d_conv_pair_tail(
                        ctypes.byref(d1), ctypes.byref(d2), ctypes.byref(d3),
                        s), "qa_d_conv_pair_tail")

                self.launches = [(tname, fn) if n == ln3 else (n, f)
                                 for n, f in self.launches if n != fused]
                rows = next(t[2] for t in self.tunables if t[0] == fused)
                self.tunables = [t for t in self.tunables if t[0] != fused]
                self.tunables.append((tname, d2, rows, fn))
                break

    def _fuse_chains(self, cons):
        """An int8 convolution of 16, 32 or 64 output channels whose output
        only feeds a 1x1 convolution of the same width runs with it as one
        launch (``qa_d_conv_chain``): the intermediate never leaves the
        work-group."""
        for d2, _, _, ln2 in self.mfma_descs:
            live = dict(self.launches)
            if ln2 not in live or d2.KH != 1 or d2.KW != 1:
                continue
            firsts = [(d, ln) for d, _, _, ln in self.mfma_descs
                      if d.y == d2.x and ln in live and ln != ln2]
            if len(firsts) != 1:
                continue
            d1, ln1 = firsts[0]
            mids = [n for n, t in self.tensors.items() if t.ptr == d1.y]
            if len(mids) != 1 or mids[0] in self.graph.outputs or \
                    [l.name for l in cons.get(mids[0], [])] != [ln2[5:]]:
                continue
            # the narrow chain kernel reads both weight sets in fragment
            # order
            narrow = self.narrow_ok(d1) and d1.Cout <= 256 and \
                d2.Cout <= 256 and self.code == 1
            if narrow:
                self._frag_weights(d1)
                self._frag_weights(d2)
            if not self.lib.qa_conv_chain_supported(ctypes.byref(d1),
                                                    ctypes.byref(d2)):
                continue
            fused = f"chain:{ln1[5:]}+{ln2[5:]}"
            rows = [0] + [0x10000 | r for r in BAND_ROWS if r <= d1.OH]
            if narrow:  # the narrow chain, 1, 2 or 4 row tiles a group
                rows += [0x12000, 0x12010, 0x12030]

            def fn(s, d1=d1, d2=d2):
                _ok(self.lib.qa_d_conv_chain(ctypes.byref(d1),
                                             ctypes.byref(d2), s),
                    "qa_d_conv_chain")

            self.launches = [(fused, fn) if n == ln2 else (n, f)
                             for n, f in self.launches if n != ln1]
            self.tunables.append((fused, d2, rows, fn))
            self.tensors.pop(mids[0], None)  # never materialized

    # ------------------------------------------------------- element-wise --
    def _plan_table(self, layer, ins):
        x = ins[0]
        p = self._params(layer)
        if "lut" not in p:
            p["lut"] = _dev(layer.lut, np.int32)
        if x.rows_view() is None:  # e.g. a Slice with a step: copy it dense
            x = self._contiguous(f"copy:{layer.name}", x)
        y = self._new(x.shape, layer.out_qp[0], dense=x._strides is not None)
        xv, yv = x.rows_view(), y.rows_view()
        if xv is None or yv is None:
            raise NotImplementedError("table on a non-matrix view")
        rows, cols, xs = xv
        lut = p["lut"]
        self._add(f"lut:{layer.name}", lambda s: _ok(self.lib.qa_d_lut(
            x.ptr, x.code, xs, y.ptr, y.code, yv[2], rows, cols,
            layer.lut_offset, lut.data_ptr(), len(layer.lut), x.so, y.so, s),
            "qa_d_lut"))
        return [y]

    def _binary_views(self, a, b, y):
        """Row views ``(rows, cols, row stride)`` of a, b and y; an operand
        of batch size 1 broadcast over the batch gets row stride 0 (then
        rows = batch, cols = one item)."""
        if a.shape != b.shape:
            big = a if b.shape[0] == 1 else b
            one = b if big is a else a
            if len(a.shape) != len(b.shape) or one.shape[0] != 1 or \
                    one.shape[1:] != big.shape[1:]:
                raise NotImplementedError("broadcasting element-wise op")
            item = int(np.prod(big.shape[1:], dtype=np.int64))
            views = []
            for t in (a, b, y):
                if not t.row_major() and t.shape[0] > 1:
                    raise NotImplementedError("broadcast of a strided view")
                views.append((big.shape[0], item,
                              0 if t is one else t.nd_strides[0]))
            if not one.row_major():
                raise NotImplementedError("broadcast of a strided view")
            return tuple(views)
        av, bv, yv = a.rows_view(), b.rows_view(), y.rows_view()
        if None in (av, bv, yv):
            raise NotImplementedError("element-wise op on strided views")
        return av, bv, yv

    @staticmethod
    def _rows_pair(a, b):
        """Whether the row kernels cover a (op) b: one storage code and equal
        shapes as row views, or one operand of batch 1 repeated over the
        other's batch (both row-major)."""
        if a.code != b.code:
            return False
        if a.shape == b.shape:
            av, bv = a.rows_view(), b.rows_view()
            if av is None or bv is None:
                return False
            if a._strides is None and b._strides is None:
                return True  # one default layout (and so the output's)
            # the output is dense row-major: rows must be the leading axes
            want = (int(np.prod(a.shape[:-1], dtype=np.int64)), a.shape[-1])
            return tuple(av[:2]) == want and tuple(bv[:2]) == want
        if not a.shape or not b.shape:  # a scalar: the broadcasting kernel
            return False
        one, big = (b, a) if b.shape[0] == 1 else (a, b)
        return len(a.shape) == len(b.shape) and one.shape[0] == 1 and \
            one.shape[1:] == big.shape[1:] and one.row_major() and \
            (big.row_major() or big.shape[0] == 1)

    def _plan_binary_nd(self, layer, ins, op):
        """Add / Sub (op 0) or Mul (op 1) with NumPy broadcasting of any two
        operand shapes and strides (``qa_d_binary_nd``)."""
        a, b = ins
        out = tuple(np.broadcast_shapes(a.shape, b.shape))
        nd = len(out)
        if not 1 <= nd <= 6:
            raise NotImplementedError(f"{layer.node.op_type} of rank {nd}")
        o = layer.out_qp[0]
        y = self._new(out, o, dense=nd not in (2, 4))
        d = BinaryNd()
        for side, t in (("a", a), ("b", b)):
            st = t.nd_strides
            arr = d.as_ if side == "a" else d.bs
            for j in range(1, len(t.shape) + 1):  # right-aligned
                arr[nd - j] = 0 if t.shape[-j] == 1 else st[-j]
            setattr(d, side, t.ptr)
            setattr(d, side + "_code", t.code)
            setattr(d, side + "_so", t.so)
        d.y, d.y_code, d.y_so, d.ndim, d.op = y.ptr, y.code, y.so, nd, op
        for j, (n_, s_) in enumerate(zip(out, y.nd_strides)):
            d.shape[j], d.ys[j] = n_, s_
        qa_, qb_ = layer.in_qp
        d.za, d.zb = int(qa_.zp), int(qb_.zp)
        if op == 0:
            (d.ma, d.sa), (d.mb, d.sb) = layer.mults
            d.sign = layer.sign
        else:
            d.ma, d.sa = layer.mult, layer.shift
        d.zp_out, d.qmin, d.qmax = int(o.zp), int(o.qmin), int(o.qmax)
        self.keep.extend([a.buf, b.buf, y.buf, d])
        self._add(f"{('add', 'mul')[op]}:{layer.name}", lambda s: _ok(
            self.lib.qa_d_binary_nd(ctypes.byref(d), s), "qa_d_binary_nd"))
        return [y]

    def _plan_add(self, layer, ins):
        a, b = ins
        if not self._rows_pair(a, b):
            return self._plan_binary_nd(layer, ins, 0)
        o = layer.out_qp[0]
        y = self._new(a.shape if a.shape[0] >= b.shape[0] else b.shape, o,
                      dense=a._strides is not None or b._strides is not None)
        av, bv, yv = self._binary_views(a, b, y)
        (ma, sa), (mb, sb) = layer.mults
        qa_, qb_ = layer.in_qp
        self._add(f"add:{layer.name}", lambda s: _ok(self.lib.qa_d_add(
            a.ptr, av[2], b.ptr, bv[2], a.code, y.ptr, y.code, yv[2], av[0],
            av[1], qa_.zp, ma, sa, qb_.zp, mb, sb, layer.sign, o.zp, o.qmin,
            o.qmax, a.so, b.so, y.so, s), "qa_d_add"))
        return [y]

    def _plan_mul(self, layer, ins):
        a, b = ins
        if not self._rows_pair(a, b):
            return self._plan_binary_nd(layer, ins, 1)
        o = layer.out_qp[0]
        y = self._new(a.shape if a.shape[0] >= b.shape[0] else b.shape, o,
                      dense=a._strides is not None or b._strides is not None)
        av, bv, yv = self._binary_views(a, b, y)
        qa_, qb_ = layer.in_qp
        self._add(f"mul:{layer.name}", lambda s: _ok(self.lib.qa_d_mul(
            a.ptr, av[2], b.ptr, bv[2], a.code, y.ptr, y.code, yv[2], av[0],
            av[1], qa_.zp, qb_.zp, layer.mult, layer.shift, o.zp, o.qmin,
            o.qmax, a.so, b.so, y.so, s), "qa_d_mul"))
        return [y]

    def _plan_concat_nd(self, layer, ins, axis):
        """Concat along any axis: each part copied (rescaled when its
        parameters differ) into its slice of a dense output."""
        o = layer.out_qp[0]
        shape = list(ins[0].shape)
        shape[axis] = sum(t.shape[axis] for t in ins)
        y = self._new(tuple(shape), o, dense=True)
        ym, off = y.meta(), 0
        for t, qp, (m, s_) in zip(ins, layer.in_qp, layer.mults):
            part = y.derived(ym.narrow(axis, off, t.shape[axis]))
            if qp.scale == o.scale and qp.zp == o.zp:
                self._copy(f"concat:{layer.name}", t, part, mode=1,
                           rescale=(qp.zp, *IDENTITY, o.zp, o.qmin, o.qmax))
            else:
                self._copy(f"concat:{layer.name}", t, part, mode=1,
                           rescale=(qp.zp, m, s_, o.zp, o.qmin, o.qmax))
            off += t.shape[axis]
        return [y]

    def _plan_concat(self, layer, ins):
        axis = layer.node.attr("axis")
        nd = len(ins[0].shape)
        axis = axis + nd if axis < 0 else axis
        if axis != 1 or nd != 4 or any(t._strides is not None for t in ins):
            return self._plan_concat_nd(layer, ins, axis)
        o = layer.out_qp[0]
        shape = list(ins[0].shape)
        shape[1] = sum(t.shape[1] for t in ins)
        y = self._new(tuple(shape), o)
        names = layer.data_inputs
        k, off = 0, 0
        while k < len(ins):
            t, qp, (m, s_) = ins[k], layer.in_qp[k], layer.mults[k]
            if qp.scale == o.scale and qp.zp == o.zp:
                m, s_ = IDENTITY
            # Parts written by one epilogue (its whole output, possibly as
            # consecutive Split views) get the copy from that epilogue.
            e = self.epi.get(names[k])
            if e is not None and e[1] == 0:
                d, _, cout = e
                span, j = 0, k
                while j < len(ins) and span < cout:
                    ej = self.epi.get(names[j])
                    if ej is None or ej[0] is not d or ej[1] != span or \
                            layer.in_qp[j] != qp:
                        break
                    span += ins[j].shape[1]
                    j += 1
                if span == cout and not d.y2:
                    d.y2 = y.ptr + off * y.buf.element_size()
                    d.y2_sn, d.y2_sc, d.y2_sp = y.sn, y.sc, y.sp
                    d.r2_zp_in, d.r2_m, d.r2_s = qp.zp, m, s_
                    d.r2_zp_out, d.r2_qmin, d.r2_qmax = o.zp, o.qmin, o.qmax
                    off += span
                    k = j
                    continue
            tv = t.rows_view()
            yv = (y.shape[0] * y.pixels, t.shape[1], y.sp) \
                if len(y.shape) == 4 else (y.shape[0], t.shape[1], y.sn)
            if tv is None:
                raise NotImplementedError("Concat of a non-matrix view")
            dst = y.ptr + off * y.buf.element_size()
            self._add(f"concat:{layer.name}", lambda st, t=t, tv=tv, qp=qp,
                      m=m, s_=s_, dst=dst, yv=yv: _ok(self.lib.qa_d_rescale(
                          t.ptr, t.code, tv[2], dst, y.code, yv[2], tv[0],
                          tv[1], qp.zp, m, s_, o.zp, o.qmin, o.qmax, t.so,
                          y.so, st), "qa_d_rescale"))
            off += t.shape[1]
            k += 1
        return [y]

    def _plan_gap(self, layer, ins):
        x = ins[0]
        n, ch = x.shape[:2]
        area = x.pixels
        mult, shift = layer.multiplier(area)
        o = layer.out_qp[0]
        y = self._new((n, ch), o)
        self.gap_info[f"gap:{layer.name}"] = dict(layer=layer, x=x, y=y,
                                                  mult=mult, shift=shift,
                                                  out=o)
        self._add(f"gap:{layer.name}", lambda s: _ok(self.lib.qa_d_gap(
            x.ptr, x.code, x.sn, x.sc, x.sp, n, ch, area, layer.in_zp, x.so,
            mult, shift, o.zp, o.qmin, o.qmax, y.ptr, y.code, y.sn, y.so, s),
            "qa_d_gap"))
        # keep the ONNX shape [N, C, 1, 1] as a view of the [N, C] buffer
        return [DeviceTensor(y.buf, 0, (n, ch) + (1,) * (len(x.shape) - 2),
                             y.sn, 1, 0, y.code, y.so, o)]

    def _plan_bn(self, layer, ins):
        x = ins[0]
        xv = x.rows_view()
        if xv is None or xv[2] != xv[1]:
            raise NotImplementedError("BatchNorm on a padded or strided view")
        p = self._params(layer)
        if "mult" not in p:
            p["mult"] = _dev(layer.q_mult, np.int64)
            p["shift"] = _dev(layer.shift, np.int64)
            p["post"] = _dev(layer.q_B, np.int64)
        o = layer.out_qp[0]
        y = self._new(x.shape, o)
        rows, ch = xv[0], xv[1]
        self._add(f"bn:{layer.name}", lambda s: _ok(self.lib.qa_d_requantize(
            x.ptr, x.code, y.ptr, y.code, rows, ch, 1, p["mult"].data_ptr(),
            p["shift"].data_ptr(), None, p["post"].data_ptr(), o.zp, o.qmin,
            o.qmax, layer.in_zp - x.so, y.so, s), "qa_d_requantize"))
        return [y]

    def _const_list(self, node, index, attr):
        if len(node.inputs) > index and node.inputs[index]:
            return [int(v) for v in np.asarray(
                self.graph.initializers[node.inputs[index]]).reshape(-1)]
        v = node.attr(attr)
        return None if v is None else [int(a) for a in np.asarray(v).reshape(
            -1)]

    def _plan_shape_nd(self, layer, x):
        """Layout operators on N-D views (no copy unless a Reshape of a
        non-dense view needs one)."""
        node, op = layer.node, layer.node.op_type
        m = x.meta()
        nd = len(x.shape)
        if op == "Reshape":
            shape = self._const_list(node, 1, "shape")
            if not node.attr("allowzero", 0):
                shape = [x.shape[i] if v == 0 else v
                         for i, v in enumerate(shape)]
            try:
                return [x.derived(m.view(shape))]
            except RuntimeError:
                xc = self._contiguous(f"copy:{layer.name}", x)
                return [xc.derived(xc.meta().view(shape))]
        if op == "Flatten":
            ax = node.attr("axis", 1)
            ax = ax + nd if ax < 0 else ax
            shape = [int(np.prod(x.shape[:ax], dtype=np.int64)), -1]
            try:
                return [x.derived(m.view(shape))]
            except RuntimeError:
                xc = self._contiguous(f"copy:{layer.name}", x)
                return [xc.derived(xc.meta().view(shape))]
        if op == "Transpose":
            perm = node.attr("perm") or list(range(nd))[::-1]
            return [x.derived(m.permute(*perm))]
        if op in ("Squeeze", "Unsqueeze"):
            axes = self._const_list(node, 1, "axes")
            if op == "Squeeze":
                if axes is None:
                    axes = [i for i, n in enumerate(x.shape) if n == 1]
                axes = sorted(a + nd if a < 0 else a for a in axes)
                for a in reversed(axes):
                    m = m.squeeze(a)
            else:
                out_nd = nd + len(axes)
                for a in sorted(a + out_nd if a < 0 else a for a in axes):
                    m = m.unsqueeze(a)
            return [x.derived(m)]
        if op == "Split":
            ax = node.attr("axis", 0)
            ax = ax + nd if ax < 0 else ax
            sizes = self._const_list(node, 1, "split") or \
                [x.shape[ax] // len(node.outputs)] * len(node.outputs)
            return [x.derived(v) for v in torch.split(m, sizes, dim=ax)]
        if op == "Slice":
            return [self._slice_view(layer, x)]
        raise NotImplementedError(f"{op} on the device")

    def _slice_view(self, layer, x):
        """Slice as Python slicing (``float_ops.py:469-481``: bounds at or
        beyond 2^62 open, others clamped, negative indices from the end):
        per axis, offset += first * stride, stride *= step. A negative step
        gives negative strides, which only the strided copy reads, so that
        view is copied to a dense tensor."""
        node = layer.node
        nd = len(x.shape)
        starts = self._const_list(node, 1, "starts")
        ends = self._const_list(node, 2, "ends")
        axes = self._const_list(node, 3, "axes") or list(range(len(starts)))
        steps = self._const_list(node, 4, "steps") or [1] * len(starts)
        shape, strides = list(x.shape), list(x.nd_strides)
        offset = x.offset
        for b, e, a, step in zip(starts, ends, axes, steps):
            if step == 0:
                raise ValueError(f"{layer.name}: Slice step 0")
            a = a + nd if a < 0 else a
            r = range(*slice(None if b >= 2**62 else b,
                             None if abs(e) >= 2**62 else e,
                             step).indices(shape[a]))
            if len(r) == 0:
                raise NotImplementedError(f"{layer.name}: empty Slice")
            offset += r.start * strides[a]
            shape[a], strides[a] = len(r), strides[a] * step
        v = DeviceTensor.nd(x.buf, offset, shape, strides, x.code, x.so,
                            x.qp)
        if any(st < 0 for st in strides):
            return self._contiguous(f"copy:{layer.name}", v)
        return v

    def _plan_shape(self, layer, ins):
        x = ins[0]
        op = layer.node.op_type
        if op == "Split" and len(x.shape) == 4 and x._strides is None and \
                (layer.node.attr("axis", 0) in (1, -3)):
            node = layer.node
            if len(node.inputs) > 1 and node.inputs[1]:
                sizes = self.graph.initializers[node.inputs[1]].astype(
                    np.int64).tolist()
            else:
                sizes = node.attr("split") or \
                    [x.shape[1] // len(node.outputs)] * len(node.outputs)
            outs, c0 = [], 0
            src = self.epi.get(node.inputs[0])
            for name, sz in zip(node.outputs, sizes):
                shape = (x.shape[0], sz) + x.shape[2:]
                outs.append(DeviceTensor(x.buf, x.offset + c0 * x.sc, shape,
                                         x.sn, x.sc, x.sp, x.code, x.so,
                                         x.qp))
                if src is not None:
                    self.epi[name] = (src[0], src[1] + c0, src[2])
                c0 += sz
            return outs
        if op == "Flatten" and len(x.shape) == 4 and x._strides is None \
                and layer.node.attr("axis", 1) == 1 and x.pixels == 1:
            return [DeviceTensor(x.buf, x.offset, (x.shape[0], x.channels),
                                 x.sn, x.sc, 0, x.code, x.so, x.qp)]
        if op == "Pad":
            return self._plan_pad(layer, x)
        if op in ("MaxPool", "GlobalMaxPool"):
            return self._plan_maxpool(layer, x)
        return self._plan_shape_nd(layer, x)

    def _plan_pad(self, layer, x):
        """Pad with the input zero point (constant mode; any rank <= 6)."""
        node = layer.node
        nd = len(x.shape)
        pads = self._const_list(node, 1, "pads")
        if pads is None or len(pads) != 2 * nd:
            raise NotImplementedError("Pad without 2 * rank constant pads")
        if min(pads) < 0:
            raise NotImplementedError("Pad with negative pads (cropping)")
        shape = tuple(x.shape[k] + pads[k] + pads[k + nd] for k in range(nd))
        iq = layer.in_qp[0]
        y = self._new(shape, layer.out_qp[0])
        d = PadDesc()
        d.x, d.code, d.y, d.ndim = x.ptr, x.code, y.ptr, nd
        for k in range(nd):
            d.shape[k], d.lo[k], d.xshape[k] = shape[k], pads[k], x.shape[k]
            d.xs[k], d.ys[k] = x.nd_strides[k], y.nd_strides[k]
        d.fill = int(iq.zp) - x.so
        self.keep.extend([x.buf, y.buf, d])
        self._add(f"pad:{layer.name}", lambda s: _ok(
            self.lib.qa_d_pad_nd(ctypes.byref(d), s), "qa_d_pad_nd"))
        return [y]

    def _plan_maxpool(self, layer, x):
        """MaxPool with the input qmin as padding value (auto_pad, ceil_mode
        and dilations resolved on the host); GlobalMaxPool as the window of
        the whole image."""
        node = layer.node
        if len(x.shape) != 4:
            raise NotImplementedError(f"{node.op_type} of a "
                                      f"{len(x.shape)}-D tensor")
        n, c, h, w = x.shape
        if node.op_type == "GlobalMaxPool":
            k, s, dl, p = (h, w), (1, 1), (1, 1), (0, 0, 0, 0)
        else:
            k, s, dl, p = float_ops.pool_geometry(node, (h, w))
            if len(k) != 2:
                raise NotImplementedError("MaxPool that is not 2-D")
        oh = (h + p[0] + p[2] - (dl[0] * (k[0] - 1) + 1)) // s[0] + 1
        ow = (w + p[1] + p[3] - (dl[1] * (k[1] - 1) + 1)) // s[1] + 1
        if oh < 1 or ow < 1:
            raise NotImplementedError("MaxPool window larger than the input")
        iq = layer.in_qp[0]
        y = self._new((n, c, oh, ow), layer.out_qp[0])
        d = MaxPoolDesc()
        d.x, d.code, d.y = x.ptr, x.code, y.ptr
        d.x_sn, d.x_sc, d.x_sh, d.x_sw = x.nd_strides
        d.y_sn, d.y_sc, d.y_sh, d.y_sw = y.nd_strides
        d.N, d.C, d.H, d.W, d.OH, d.OW = n, c, h, w, oh, ow
        d.KH, d.KW, d.SH, d.SW, d.DH, d.DW = k[0], k[1], s[0], s[1], dl[0], \
            dl[1]
        d.PT, d.PL = p[0], p[1]
        d.pad = int(iq.qmin) - x.so
        self.keep.extend([x.buf, y.buf, d])
        self._add(f"maxpool:{layer.name}", lambda s_: _ok(
            self.lib.qa_d_maxpool(ctypes.byref(d), s_), "qa_d_maxpool"))
        return [y]

    def _plan_float(self, layer, ins):
        op = layer.node.op_type
        x = ins[0]
        if op == "Softmax":
            ax = layer.node.attr("axis", -1 if self.graph.opset >= 13 else 1)
            ax = ax + len(x.shape) if ax < 0 else ax
            if ax != len(x.shape) - 1:
                return self._plan_fb_softmax(layer, x, log=False)
            x = self._contiguous(f"copy:{layer.name}", x)
            o = layer.out_qp[0]
            y = self._new(x.shape, o, dense=True)
            rows, cols, _ = x.rows_view()
            self.keep.extend([x.buf, y.buf])
            iq = layer.in_qp[0]
            args = (x.ptr, x.code, rows, cols, iq.scale, iq.zp, x.so, y.ptr,
                    y.code, o.scale, o.zp, o.qmin, o.qmax, y.so)
            lname = f"softmax:{layer.name}"
            # for a graph output: the same launch writing the float copy too
            self.softmax_of[layer.node.outputs[0]] = (
                lname, lambda s, yf: _ok(self.lib.qa_d_softmax_f32(
                    *args, yf.data_ptr(), s), "qa_d_softmax_f32"))
            if x.code == 1 and y.code == 1 and cols <= 1024:
                # int8: exponentials from a table built once per layer
                tab = torch.empty(65536, dtype=torch.float64, device="cuda")
                _ok(self.lib.qa_d_softmax_table(
                    iq.scale, iq.zp, x.so, tab.data_ptr(),
                    torch.cuda.current_stream().cuda_stream),
                    "qa_d_softmax_table")
                torch.cuda.synchronize()
                self.keep.append(tab)
                largs = (x.ptr, rows, cols, tab.data_ptr(), y.ptr, o.scale,
                         o.zp, o.qmin, o.qmax, y.so)
                self.softmax_lut[layer.node.outputs[0]] = (
                    lname, layer.data_inputs[0], x.ptr, tab, o, y.so)
                self._add(lname, lambda s: _ok(
                    self.lib.qa_d_softmax_lut(*largs, s), "qa_d_softmax_lut"))
                self.softmax_of[layer.node.outputs[0]] = (
                    lname, lambda s, yf: _ok(self.lib.qa_d_softmax_lut_f32(
                        *largs, yf.data_ptr(), s), "qa_d_softmax_lut_f32"))
            else:
                self._add(lname, lambda s: _ok(
                    self.lib.qa_d_softmax(*args, s), "qa_d_softmax"))
            return [y]
        if op == "LayerNormalization":
            return self._plan_layernorm(layer, x)
        if op == "MatMul" and len(ins) == 2:
            return self._plan_matmul_act(layer, ins[0], ins[1])
        if op == "Gather":
            return self._plan_gather(layer, x)
        if op in ("Div", "Max", "Min", "Pow"):
            return self._plan_fb_binary(layer, ins)
        if op == "ReduceMean":
            return self._plan_fb_reduce(layer, x)
        if op == "LogSoftmax":
            return self._plan_fb_softmax(layer, x, log=True)
        if op == "AveragePool":
            return self._plan_fb_avgpool(layer, x)
        if op == "Expand" or (op == "Cast" and layer.node.attr("to") == 1):
            return self._plan_fb_copy(layer, x)
        if op == "Cast":
            return self._plan_fb_gather(layer, x, None, -1,
                                        int(layer.node.attr("to")))
        if op == "Pad":
            return self._plan_fb_pad(layer, x)
        raise NotImplementedError(f"float fallback of {op} on the device")

    def _plan_fb_pad(self, layer, x):
        """Pad in reflect / edge mode or with a non-zero constant: the
        float fallback, each output value requantized (the padding value
        quantized from its float32 value)."""
        node = layer.node
        nd = len(x.shape)
        pads = self._const_list(node, 1, "pads")
        if pads is None or len(pads) != 2 * nd:
            raise NotImplementedError("Pad without 2 * rank constant pads")
        if min(pads) < 0:
            raise NotImplementedError("Pad with negative pads (cropping)")
        if not 1 <= nd <= 6:
            raise NotImplementedError(f"Pad of rank {nd}")
        mode = node.attr("mode", "constant")
        if mode not in ("constant", "reflect", "edge"):
            raise NotImplementedError(f"Pad mode {mode}")
        value = 0.0
        if mode == "constant":
            init = self.graph.initializers
            value = (np.asarray(init[node.inputs[2]]).reshape(()).item()
                     if len(node.inputs) > 2 and node.inputs[2]
                     else node.attr("value", 0.0))
        shape = tuple(x.shape[k] + pads[k] + pads[k + nd] for k in range(nd))
        o, iq = layer.out_qp[0], layer.in_qp[0]
        y = self._new(shape, o, dense=nd not in (2, 4))
        d = FbPad()
        d.x, d.x_code, d.x_so = x.ptr, x.code, x.so
        d.x_zp, d.x_scale = int(iq.zp), float(iq.scale)
        d.y, d.y_code, d.y_so, d.ndim = y.ptr, y.code, y.so, nd
        for k in range(nd):
            d.shape[k], d.lo[k], d.xshape[k] = shape[k], pads[k], x.shape[k]
            d.xs[k], d.ys[k] = x.nd_strides[k], y.nd_strides[k]
        d.mode = ("constant", "reflect", "edge").index(mode)
        d.value = float(np.float32(value))  # np.pad casts it to float32
        d.out_scale, d.out_zp, d.qmin, d.qmax = self._qargs(o)
        self.keep.extend([x.buf, y.buf, d])
        self._add(f"fallback:{layer.name}", lambda s: _ok(
            self.lib.qa_d_fb_pad(ctypes.byref(d), s), "qa_d_fb_pad"))
        return [y]

    def _plan_fb_gather(self, layer, x, idx, axis, cast_to):
        """Gather of an index array along ``axis`` (``idx``: the indices,
        any shape) and / or Cast to ``cast_to``: the selected values
        dequantized, cast, and requantized with the output parameters."""
        if cast_to not in CAST_CODES:
            raise NotImplementedError(f"Cast to element type {cast_to}")
        nd = len(x.shape)
        shape = list(x.shape)
        out = tuple(x.shape)
        if axis >= 0:
            n = x.shape[axis]
            idx = np.asarray(idx).astype(np.int64)
            if idx.size == 0:
                raise NotImplementedError("Gather of an empty index array")
            if idx.min() < -n or idx.max() >= n:
                raise IndexError(f"{layer.name}: Gather index out of range "
                                 f"for an axis of {n}")
            idx = np.where(idx < 0, idx + n, idx)
            shape[axis] = idx.size
            out = x.shape[:axis] + idx.shape + x.shape[axis + 1:]
        if not 1 <= nd <= 6 or len(out) > 6:
            raise NotImplementedError(f"{layer.node.op_type} of rank "
                                      f"{len(out)}")
        o, iq = layer.out_qp[0], layer.in_qp[0]
        if len(out) == nd:  # coordinates map one to one: any layout
            y = self._new(out, o, dense=nd not in (2, 4))
            ys = list(y.nd_strides)
        else:  # the index dimensions, dense in y, taken as one axis
            y = self._new(out, o, dense=True)
            ys = [int(np.prod(shape[k + 1:], dtype=np.int64))
                  for k in range(nd)]
        d = FbGather()
        d.x, d.x_code, d.x_so = x.ptr, x.code, x.so
        d.x_zp, d.x_scale = int(iq.zp), float(iq.scale)
        if axis >= 0:
            t = _dev(idx.reshape(-1), np.int64)
            self.keep.append(t)
            d.idx, d.nidx = t.data_ptr(), idx.size
        d.axis, d.cast_to = axis, cast_to
        d.y, d.y_code, d.y_so, d.ndim = y.ptr, y.code, y.so, nd
        for k in range(nd):
            d.shape[k], d.xs[k], d.ys[k] = shape[k], x.nd_strides[k], ys[k]
        d.out_scale, d.out_zp, d.qmin, d.qmax = self._qargs(o)
        self.keep.extend([x.buf, y.buf, d])
        self._add(f"fallback:{layer.name}", lambda s: _ok(
            self.lib.qa_d_fb_gather(ctypes.byref(d), s), "qa_d_fb_gather"))
        return [y]

    @staticmethod
    def _qargs(qp):
        return float(qp.scale), int(qp.zp), int(qp.qmin), int(qp.qmax)

    def _plan_fb_binary(self, layer, ins):
        """Div / Max / Min / Pow of two operands, either quantized
        activations or float constants, with NumPy broadcasting."""
        node = layer.node
        init = self.graph.initializers
        data = dict(zip(layer.inputs, ins))
        qps = dict(zip(layer.inputs, layer.in_qp))
        ops = []
        for name in node.inputs[:2]:
            if name in data:
                ops.append((data[name], qps[name]))
            else:  # a float constant, read as float32 (code 0)
                v = np.ascontiguousarray(init[name], np.float32)
                t = _dev(v, np.float32)
                st = tuple(int(np.prod(v.shape[k + 1:], dtype=np.int64))
                           for k in range(v.ndim))
                ops.append((t, v.shape, st))
        shapes = [o[0].shape if len(o) == 2 else o[1] for o in ops]
        out = tuple(np.broadcast_shapes(*shapes))
        nd = len(out)
        if not 1 <= nd <= 6:
            raise NotImplementedError(f"{node.op_type} of rank {nd}")
        o = layer.out_qp[0]
        y = self._new(out, o, dense=len(out) not in (2, 4))
        d = FbBinary()
        for k, (side, src) in enumerate(zip(("a", "b"), ops)):
            if len(src) == 2:
                t, qp = src
                shp, st = t.shape, t.nd_strides
                ptr, code, so, zp, sc = t.ptr, t.code, t.so, qp.zp, qp.scale
                self.keep.append(t.buf)
            else:
                t, shp, st = src
                ptr, code, so, zp, sc = t.data_ptr(), 0, 0, 0, 1.0
                self.keep.append(t)
            strides = [0] * nd
            for j in range(1, len(shp) + 1):  # right-aligned broadcasting
                if shp[-j] != 1:
                    strides[-j] = st[-j]
            setattr(d, side, ptr)
            setattr(d, side + "_code", code)
            setattr(d, side + "_so", so)
            setattr(d, side + "_zp", int(zp))
            setattr(d, side + "_scale", float(sc))
            arr = d.as_ if side == "a" else d.bs
            for j in range(nd):
                arr[j] = strides[j]
        d.y, d.y_code, d.y_so = y.ptr, y.code, y.so
        for j, (n_, s_) in enumerate(zip(out, y.nd_strides)):
            d.shape[j], d.ys[j] = n_, s_
        d.ndim = nd
        d.op = ("Div", "Max", "Min", "Pow").index(node.op_type)
        d.out_scale, d.out_zp, d.qmin, d.qmax = self._qargs(o)
        self.keep.extend([y.buf, d])
        self._add(f"fallback:{layer.name}", lambda s: _ok(
            self.lib.qa_d_fb_binary(ctypes.byref(d), s), "qa_d_fb_binary"))
        return [y]

    def _plan_fb_reduce(self, layer, x):
        node = layer.node
        nd = len(x.shape)
        axes = self._const_list(node, 1, "axes")
        axes = sorted({a + nd if a < 0 else a for a in axes}) if axes \
            else list(range(nd))
        keep = [k for k in range(nd) if k not in axes]
        keepdims = bool(node.attr("keepdims", 1))
        shape = tuple(1 if k in axes else x.shape[k] for k in range(nd)) \
            if keepdims else tuple(x.shape[k] for k in keep)
        o = layer.out_qp[0]
        y = self._new(shape or (1,), o, dense=True)
        st = x.nd_strides
        d = FbReduce()
        d.x, d.x_code, d.x_so = x.ptr, x.code, x.so
        d.x_zp, d.x_scale = int(layer.in_qp[0].zp), float(layer.in_qp[0].scale)
        d.nkeep, d.nred = len(keep), len(axes)
        for j, k in enumerate(keep):
            d.keep[j], d.xks[j] = x.shape[k], st[k]
        for j, k in enumerate(axes):
            d.red[j], d.xrs[j] = x.shape[k], st[k]
        d.y, d.y_code, d.y_so = y.ptr, y.code, y.so
        d.out_scale, d.out_zp, d.qmin, d.qmax = self._qargs(o)
        self.keep.extend([x.buf, y.buf, d])
        self._add(f"fallback:{layer.name}", lambda s: _ok(
            self.lib.qa_d_fb_reduce_mean(ctypes.byref(d), s),
            "qa_d_fb_reduce_mean"))
        if not shape:
            y = DeviceTensor.nd(y.buf, y.offset, (), (), y.code, y.so, y.qp)
        return [y]

    def _plan_fb_softmax(self, layer, x, log):
        """Softmax / LogSoftmax over any axis, float64 rows."""
        node = layer.node
        nd = len(x.shape)
        ax = node.attr("axis", -1 if self.graph.opset >= 13 else 1)
        ax = ax + nd if ax < 0 else ax

        def form(t):
            st = t.nd_strides
            so_, si = _collapse(t.shape, st, 0, ax), \
                _collapse(t.shape, st, ax + 1, nd)
            return None if so_ is None or si is None else (so_, st[ax], si)

        if form(x) is None:
            x = self._contiguous(f"copy:{layer.name}", x)
        o = layer.out_qp[0]
        y = self._new(x.shape, o, dense=nd not in (2, 4))
        if form(y) is None:
            y = self._new(x.shape, o, dense=True)
        (xo, xk, xi), (yo, yk, yi) = form(x), form(y)
        d = FbSoftmax()
        d.x, d.x_code, d.x_so = x.ptr, x.code, x.so
        d.x_zp, d.x_scale = int(layer.in_qp[0].zp), float(layer.in_qp[0].scale)
        d.outer = int(np.prod(x.shape[:ax], dtype=np.int64))
        d.len = x.shape[ax]
        d.inner = int(np.prod(x.shape[ax + 1:], dtype=np.int64))
        d.xs_o, d.xs_k, d.xs_i = xo, xk, xi
        d.y, d.y_code, d.y_so = y.ptr, y.code, y.so
        d.ys_o, d.ys_k, d.ys_i = yo, yk, yi
        d.log = int(log)
        d.out_scale, d.out_zp, d.qmin, d.qmax = self._qargs(o)
        self.keep.extend([x.buf, y.buf, d])
        self._add(f"fallback:{layer.name}", lambda s: _ok(
            self.lib.qa_d_fb_softmax(ctypes.byref(d), s), "qa_d_fb_softmax"))
        return [y]

    def _plan_fb_avgpool(self, layer, x):
        node = layer.node
        if len(x.shape) != 4:
            raise NotImplementedError("AveragePool that is not 2-D")
        n, c, h, w = x.shape
        k, s_, _, p = float_ops.pool_geometry(node, (h, w))
        oh = (h + p[0] + p[2] - k[0]) // s_[0] + 1
        ow = (w + p[1] + p[3] - k[1]) // s_[1] + 1
        o = layer.out_qp[0]
        y = self._new((n, c, oh, ow), o)
        d = FbAvgPool()
        d.x, d.x_code, d.x_so = x.ptr, x.code, x.so
        d.x_zp, d.x_scale = int(layer.in_qp[0].zp), float(layer.in_qp[0].scale)
        d.x_sn, d.x_sc, d.x_sh, d.x_sw = x.nd_strides
        d.N, d.C, d.H, d.W, d.OH, d.OW = n, c, h, w, oh, ow
        d.KH, d.KW, d.SH, d.SW, d.PT, d.PL = k[0], k[1], s_[0], s_[1], p[0], \
            p[1]
        d.count_pad = int(node.attr("count_include_pad", 0))
        d.y, d.y_code, d.y_so = y.ptr, y.code, y.so
        d.y_sn, d.y_sc, d.y_sh, d.y_sw = y.nd_strides
        d.out_scale, d.out_zp, d.qmin, d.qmax = self._qargs(o)
        self.keep.extend([x.buf, y.buf, d])
        self._add(f"fallback:{layer.name}", lambda s: _ok(
            self.lib.qa_d_fb_avgpool(ctypes.byref(d), s), "qa_d_fb_avgpool"))
        return [y]

    def _plan_fb_copy(self, layer, x):
        """Expand (a broadcast copy) and Cast to float: the values move, and
        are requantized with the output parameters."""
        node = layer.node
        shape = x.shape
        if node.op_type == "Expand":
            tgt = tuple(self._const_list(node, 1, "shape"))
            shape = tuple(np.broadcast_shapes(x.shape, tgt))
        o, iq = layer.out_qp[0], layer.in_qp[0]
        y = self._new(shape, o, dense=len(shape) not in (2, 4))
        nd = len(shape)
        st = x.nd_strides
        xs = [0] * nd
        for j in range(1, len(x.shape) + 1):
            if x.shape[-j] != 1:
                xs[-j] = st[-j]
        xv = DeviceTensor.nd(x.buf, x.offset, shape, xs, x.code, x.so, x.qp)
        self._copy(f"fallback:{layer.name}", xv, y, mode=2,
                   requant=(float(iq.scale), int(iq.zp), float(o.scale),
                            int(o.zp), int(o.qmin), int(o.qmax)))
        return [y]

    def _plan_layernorm(self, layer, x):
        """LayerNormalization over the last axis (float fallback)."""
        node = layer.node
        ax = node.attr("axis", -1)
        ax = ax + len(x.shape) if ax < 0 else ax
        out_shape = x.shape
        if ax != len(x.shape) - 1:
            # the trailing axes as one row of a dense row-major view
            x = self._contiguous(f"copy:{layer.name}", x)
            cols = int(np.prod(x.shape[ax:], dtype=np.int64))
            rows = int(np.prod(x.shape[:ax], dtype=np.int64))
            x = DeviceTensor.nd(x.buf, x.offset, (rows, cols), (cols, 1),
                                x.code, x.so, x.qp)
        init = self.graph.initializers
        p = self._params(layer)
        if "gamma" not in p:
            p["gamma"] = _dev(init[node.inputs[1]].reshape(-1), np.float32)
            p["beta"] = (_dev(init[node.inputs[2]].reshape(-1), np.float32)
                         if len(node.inputs) > 2 and node.inputs[2] else None)
        xv = x.rows_view()
        if xv is None:
            x = self._contiguous(f"copy:{layer.name}", x)
            xv = x.rows_view()
        rows, cols, xrs = xv
        if p["gamma"].numel() != cols:
            raise NotImplementedError("LayerNorm gain of another length")
        o, iq = layer.out_qp[0], layer.in_qp[0]
        y = self._new(x.shape, o, dense=True)
        yrs = y.rows_view()[2]
        eps = float(node.attr("epsilon", 1e-5))
        g, b = p["gamma"], p["beta"]
        self.keep.extend([x.buf, y.buf])
        self._add(f"layernorm:{layer.name}", lambda s: _ok(
            self.lib.qa_d_layernorm(
                x.ptr, x.code, xrs, rows, cols, iq.scale, iq.zp, x.so,
                g.data_ptr(), None if b is None else b.data_ptr(), eps,
                y.ptr, y.code, yrs, o.scale, o.zp, o.qmin, o.qmax, y.so, s),
            "qa_d_layernorm"))
        if y.shape != out_shape:  # back to the operator's shape (dense)
            st = tuple(int(np.prod(out_shape[k + 1:], dtype=np.int64))
                       for k in range(len(out_shape)))
            y = DeviceTensor.nd(y.buf, y.offset, out_shape, st, y.code, y.so,
                                y.qp)
        return [y]

    def _plan_matmul_act(self, layer, a, b):
        """MatMul of two activations (float fallback): [.., M, K] x
        [.., K, N] with up to two equal batch axes."""
        if len(a.shape) != len(b.shape) or not 2 <= len(a.shape) <= 4 or \
                a.shape[:-2] != b.shape[:-2] or a.shape[-1] != b.shape[-2]:
            raise NotImplementedError(
                f"MatMul of {a.shape} and {b.shape} on the device")
        if a.code != b.code:
            raise NotImplementedError("MatMul of mixed storage")
        # any strides: the kernel stages both operands through LDS; B is
        # described transposed ([.., N, K])
        bt = b.derived(b.meta().transpose(-1, -2))
        lead = a.shape[:-2]
        batch = (1,) * (2 - len(lead)) + tuple(lead)
        M, K = a.shape[-2:]
        N = b.shape[-1]
        o = layer.out_qp[0]
        y = self._new_for_users(layer.node.outputs[0],
                                tuple(lead) + (M, N), o)

        def bstr(t):
            st = t.nd_strides[:-2]
            return (0,) * (2 - len(st)) + tuple(st)
        qa_, qb_ = layer.in_qp
        d = MatmulDesc()
        d.a, d.a_code, d.a_so, d.a_zp, d.a_scale = a.ptr, a.code, a.so, \
            qa_.zp, qa_.scale
        (d.a_s0, d.a_s1), d.a_sm, d.a_sk = bstr(a), a.nd_strides[-2], \
            a.nd_strides[-1]
        d.b, d.b_code, d.b_so, d.b_zp, d.b_scale = bt.ptr, bt.code, bt.so, \
            qb_.zp, qb_.scale
        (d.b_s0, d.b_s1), d.b_sn, d.b_sk = bstr(bt), bt.nd_strides[-2], \
            bt.nd_strides[-1]
        d.B0, d.B1, d.M, d.N, d.K = batch[0], batch[1], M, N, K
        d.y, d.y_code, d.y_so = y.ptr, y.code, y.so
        (d.y_s0, d.y_s1), d.y_sm, d.y_sn = bstr(y), y.nd_strides[-2], \
            y.nd_strides[-1]
        d.out_scale, d.out_zp, d.qmin, d.qmax = o.scale, o.zp, o.qmin, o.qmax
        self.keep.extend([d, a.buf, bt.buf, y.buf])
        self.matmul_act[layer.node.outputs[0]] = (
            f"matmul:{layer.name}", d, layer.data_inputs[0])
        self._add(f"matmul:{layer.name}", lambda s, d=d: _ok(
            self.lib.qa_d_matmul_act(ctypes.byref(d), s), "qa_d_matmul_act"))
        return [y]

    def _plan_gather(self, layer, x):
        """Gather of constant indices (float fallback: the selected values
        are requantized to the output's parameters)."""
        node = layer.node
        idx = np.asarray(self.graph.initializers[node.inputs[1]])
        ax = node.attr("axis", 0)
        ax = ax + len(x.shape) if ax < 0 else ax
        m = x.meta()
        if idx.ndim == 0:
            v = x.derived(m.select(ax, int(idx)))
        else:
            return self._plan_fb_gather(layer, x, idx, ax, 1)
        o, iq = layer.out_qp[0], layer.in_qp[0]
        y = self._new(v.shape, o, dense=True)
        self._copy(f"gather:{layer.name}", v, y, mode=2,
                   requant=(iq.scale, iq.zp, o.scale, o.zp, o.qmin, o.qmax))
        return [y]

    # ------------------------------------------------------------ tiling --
    @staticmethod
    def narrow_ok(d):
        """Whether the narrow-GEMM kernel takes an int8 descriptor (a 1x1
        convolution or GEMM, or a k x k convolution as a GEMM over its
        im2col rows)."""
        k = d.C * d.KH * d.KW  # K of the GEMM (of the im2col rows)
        return d.G == 1 and d.w_layout == 0 and d.Cout >= 16 and \
            d.Cout % 4 == 0 and (d.Cout > 64 or d.Cout % 16 == 0) and \
            d.C % 64 == 0 and (k <= 576 or (k <= 1280 and d.Cout >= 64)) \
            and bool(d.epi_plan) and not d.res

    @staticmethod
    def tile_candidates(d):
        """``qa_conv_desc.tile`` codes worth timing for one MFMA
        convolution. FP64 path: 0 (the library's choice), then each of its
        tiles (16-channel groups, 16-pixel tiles per wave, K split over the
        work-group). int8: 0, then every channel-block
        width up to the output channels per group, K-split (channel-blocked
        weight layout only) and weights in LDS (where 16 rows per channel
        group of K bytes fit in the 3 KiB-chunk staging budget; the library
        re-checks the LDS size), the large-GEMM kernel and the narrow-GEMM
        kernel where their shapes apply."""
        cog = d.Cout // d.G
        if d.w_code == 8:  # FP64 path: wm | tm << 4 | split << 8
            wm_max = 1 if cog <= 16 else 2 if cog <= 32 else 4
            out = [0] + [0x10000 | c for c in F64_TILES if c & 15 <= wm_max]
            if d.wsplit:  # byte split: 0x1000 | wm | tm << 4
                out += [0x11000 | wm | tm << 4 for tm in (1, 2)
                        for wm in (1, 2, 4) if wm <= wm_max]
            return out
        wm_max = 1 if cog <= 16 else 2 if cog <= 32 else 4 if cog <= 64 else 8
        out = [0]
        if d.H == d.W == d.KH == d.KW == 1 and d.G == 1 and \
                d.w_layout == 0 and d.C % 64 == 0:
            # the large-GEMM kernel (128 x 128 blocks): K steps staged
            # through registers, or through 3 / 4 LDS stages of direct loads
            out += [0x10400, 0x10403, 0x10404]
        if DeviceExecutor.narrow_ok(d):
            # narrow GEMM: a 16 x 16 block a wave, 1, 2 or 4 row tiles a
            # wave with the same weights
            out += [0x12000, 0x12010, 0x12030]
        if d.w_layout == 0 and d.G == 1 and d.C % 16 == 0 and \
                d.OW <= 256 and d.epi_plan and (d.H > 1 or d.W > 1):
            # bands of output rows, operands in LDS (the library checks the
            # LDS size and falls back when the band does not fit)
            out += [0x10800 | wm for wm in (1, 2, 4) if wm <= wm_max]
            # weights held in registers (K up to 36 / wm steps of 64 bytes;
            # the library checks the rest and falls back)
            out += [0x11000 | wm | r << 4 for wm in (1, 2, 4)
                    if wm <= wm_max and d.w_kgp // 4 <= 36 // wm
                    for r in (0,) + BAND_ROWS if r <= d.OH]
        for wm in (1, 2, 4, 8):
            if wm > wm_max:
                break
            for split in ((0, 1) if d.w_layout == 0 else (0,)):
                for lds in ((0, 1) if wm * d.w_kgp <= 192 else (0,)):
                    out.append(0x10000 | wm | split << 8 | lds << 9)
        return out

    def tune(self, launches=8, reps=3):
        """Times every tile code of every int8 MFMA convolution in place
        (captured graphs of ``launches`` back-to-back launches, HIP events
        over ``reps`` replays) and keeps the fastest per layer. Inputs must
        hold a pass's data (call once after ``launch``); results do not
        depend on the tiles. Returns ``{launch name: (code, best ms,
        library-choice ms)}``."""
        if self.cuda_graph is not None:
            raise RuntimeError("tune() before the pass is captured")
        report = {}
        torch.cuda.synchronize()
        for name, d, codes, fn in self.tunables:
            times = {}
            for code in codes:
                d.tile = code
                times[code] = self._time_launch(fn, launches, reps)
            best = min(times, key=times.get)
            d.tile = best
            report[name] = (best, times[best], times[0])
        return report

    @staticmethod
    def _time_launch(fn, launches, reps):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            s = torch.cuda.current_stream().cuda_stream
            for _ in range(launches):
                fn(s)
        g.replay()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            g.replay()
        e1.record()
        e1.synchronize()
        ms = e0.elapsed_time(e1) / (reps * launches)
        del g
        return ms

    # ------------------------------------------------------------ running --
    def launch(self, stream=None):
        """Queues every launch on ``stream`` (default: torch's current)."""
        s = stream if stream is not None else \
            torch.cuda.current_stream().cuda_stream
        for _, fn in self.launches:
            fn(s)

    def capture(self):
        """Captures the launch sequence into a HIP graph (once)."""
        if self.cuda_graph is None:
            self.launch()  # warm-up outside capture
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self.launch()
            self.cuda_graph = g
        return self.cuda_graph

    def replay(self):
        if self.cuda_graph is None:
            self.capture()
        self.cuda_graph.replay()

    def run(self, feeds, use_graph=False):
        """Copies float inputs in, runs the pass, returns float outputs."""
        for name, x in feeds.items():
            self.inputs_f32[name].copy_(torch.as_tensor(
                np.ascontiguousarray(x, dtype=np.float32)))
        if use_graph:
            self.replay()
        else:
            self.launch()
        torch.cuda.synchronize()
        return {k: v.cpu().numpy() for k, v in self.outputs_f32.items()}

    def integer_outputs(self):
        return {k: self.tensors[k].to_host() for k in self.graph.outputs}


class InFlight:
    """Several batches in flight: the passes of ``executors`` (one per
    batch, each with its own buffers, e.g. consecutive batches of a stream
    of requests) captured as parallel branches of ONE HIP graph, forked from
    and joined to the replaying stream. The GPU then runs one batch's
    launches while another's wait on a launch gap or leave CUs idle: a
    late-stage launch of a classifier covers a few hundred work-groups and
    runs for a few microseconds, so a single pass leaves most of the chip
    idle most of the time. Graphs replayed from two streams did not overlap
    here; branches of one graph do. Each executor's results are those of
    its own pass (``DeviceExecutor.replay``): the branches share no memory.
    ``replay()`` runs every batch once."""

    def __init__(self, executors):
        if not executors:
            raise ValueError("InFlight needs at least one executor")
        self.executors = list(executors)
        for ex in self.executors:  # warm-up outside capture
            ex.launch()
        torch.cuda.synchronize()
        # one side stream a branch past the first, default priority
        self.streams = [torch.cuda.Stream() for _ in self.executors[1:]]
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            cur = torch.cuda.current_stream()
            for s in self.streams:
                s.wait_stream(cur)
            self.executors[0].launch(cur.cuda_stream)
            for ex, s in zip(self.executors[1:], self.streams):
                with torch.cuda.stream(s):
                    ex.launch(s.cuda_stream)
            for s in self.streams:
                cur.wait_stream(s)
        self.cuda_graph = g

    def replay(self):
        self.cuda_graph.replay()


def tune_in_flight(executors, sweeps=2, reps=60, rounds=3, keep=()):
    """Chooses each launch's tile code with the batches of ``executors``
    in flight (``InFlight``; the executors of one graph and input shape,
    planned alike): for every tunable launch in turn, every code is set on
    all executors and the two-branch graph is captured and timed (best of
    ``rounds`` runs of ``reps`` replays); a code replaces the current one
    when it is at least 0.5% faster. ``sweeps`` passes over the launches;
    launches named in ``keep`` stay as they are. With the GPU shared, bands
    of more rows (fewer work-groups, less halo work) tend to win over the
    fastest code of a launch timed alone. Returns ``{launch name: code}``;
    results do not depend on the codes."""
    import time

    def setcode(i, code):
        for e in executors:
            e.tunables[i][1].tile = code

    def rate():
        fl = InFlight(executors)
        for _ in range(5):
            fl.replay()
        torch.cuda.synchronize()
        best = None
        for _ in range(rounds):
            t0 = time.perf_counter()
            for _ in range(reps):
                fl.replay()
            torch.cuda.synchronize()
            dt = time.perf_counter() - t0
            best = dt if best is None else min(best, dt)
        return reps / best

    for _ in range(sweeps):
        for i, (name, d, codes, _) in enumerate(executors[0].tunables):
            if name in keep:
                continue
            cur = d.tile
            res = {}
            for code in codes:
                setcode(i, code)
                res[code] = rate()
            best = max(res, key=res.get)
            setcode(i, best if res[best] > res[cur] * 1.005 else cur)
    return {name: d.tile for name, d, _, _ in executors[0].tunables}
