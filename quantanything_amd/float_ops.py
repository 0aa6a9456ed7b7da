"""Float semantics of the graph's operators (reference: ``float_ops.py``).

Used for calibration (min/max of every tensor), for building activation
lookup tables (``prepare`` of LUT layers evaluates the op on every quantized
input value) and by the float fallback of the integer path. The element-wise
numerics follow the reference exactly where they feed integer parameters:
Sigmoid / Exp / Softplus in float64 cast to float32 (``float_ops.py:225-227``
and around), HardSwish / HardSigmoid / LeakyRelu / Elu formulas, the
Abramowitz-Stegun ``erf`` (``float_ops.py:289-304``), float64 Softmax and
LayerNorm (``:336-347``, ``:380-385``).

Conv and Gemm run on the GPU through ``native.conv2d_f32`` /
``native.gemm_f32`` (the float entries of the same library).
"""

import numpy as np
from numpy.lib.stride_tricks import sliding_window_view

from quantanything_amd import native

# op_type -> evaluator(node, inputs, opset, **kw) returning the list of the
# node's outputs; UNARY: the element-wise ops that tabulate (f(node, x)).
OPS = {}
UNARY = {}


class UnsupportedOp(NotImplementedError):
    """An operator without a float implementation here."""


def operator(*names, multi=False):
    """Registers an evaluator under ONNX op names. Single-output evaluators
    (``multi`` False) return one array, which is wrapped into the list that
    every entry of :data:`OPS` returns."""
    def register(fn):
        entry = fn if multi else \
            (lambda node, ins, opset, **kw: [fn(node, ins, opset, **kw)])
        OPS.update(dict.fromkeys(names, entry))
        return fn
    return register


def tabulated(name):
    """Registers an element-wise ``f(node, x)`` that integer passes turn
    into a lookup table over every quantized input value."""
    def register(fn):
        UNARY[name] = fn
        OPS[name] = lambda node, ins, opset, **kw: [fn(node, ins[0])]
        return fn
    return register


def run_node(node, inputs, opset=13, **kw):
    """The node's outputs (a list) on float (or integer) NumPy inputs."""
    try:
        evaluate = OPS[node.op_type]
    except KeyError:
        raise UnsupportedOp(f"operator {node.op_type} ({node.name}) has no "
                            "float implementation") from None
    return evaluate(node, inputs, opset, **kw)


def feed_dict(graph, feeds):
    """``{input name: float32 array}`` from a dict, or from one array when
    the graph has a single input."""
    names = graph.input_names
    if isinstance(feeds, dict):
        pairs = feeds.items()
    elif len(names) == 1:
        pairs = [(names[0], feeds)]
    else:
        raise ValueError(f"the graph has {len(names)} inputs "
                         f"({', '.join(names)}): feed a dict of them")
    return {name: np.asarray(v, dtype=np.float32) for name, v in pairs}


def run_float(graph, feeds, keep_all=False):
    """The float32 pass: graph outputs (one array, or a list), or every
    tensor of the pass with ``keep_all``."""
    env = {**graph.initializers, **feed_dict(graph, feeds)}
    for node in graph.nodes:
        args = [env[i] if i else None for i in node.inputs]
        env.update(zip(node.outputs, run_node(node, args, graph.opset)))
    if keep_all:
        return env
    outs = [env[o] for o in graph.outputs]
    return outs if len(outs) > 1 else outs[0]


def conv_pads(node, in_hw, kernel, strides, dilations):
    """``pads`` / ``auto_pad`` -> ``(top, left, bottom, right)``
    (``float_ops.py:132-146``)."""
    auto = node.attr("auto_pad", "NOTSET")
    if auto in ("SAME_UPPER", "SAME_LOWER"):
        res = []
        for size, k, s, d in zip(in_hw, kernel, strides, dilations):
            out = -(-size // s)
            total = max((out - 1) * s + d * (k - 1) + 1 - size, 0)
            lo, hi = total // 2, total - total // 2
            res.append((lo, hi) if auto == "SAME_UPPER" else (hi, lo))
        return (res[0][0], res[1][0], res[0][1], res[1][1])
    if auto == "VALID":
        return (0, 0, 0, 0)
    p = node.attr("pads", [0] * 4)
    return (p[0], p[1], p[2], p[3])


def conv_geometry(node, x_shape, w_shape):
    strides = tuple(node.attr("strides", [1, 1]))
    dilations = tuple(node.attr("dilations", [1, 1]))
    pads = conv_pads(node, x_shape[2:], w_shape[2:], strides, dilations)
    return strides, pads, dilations, node.attr("group", 1)


# ------------------------------------------------------------- linear ----
@operator("Conv")
def _conv(node, ins, opset, **kw):
    x, w = ins[0], ins[1]
    if x.ndim != 4:
        raise UnsupportedOp("only 2-D convolution is supported")
    y = native.conv2d_f32(x, w, *conv_geometry(node, x.shape, w.shape))
    if len(ins) > 2 and ins[2] is not None:
        y = y + ins[2].reshape(1, -1, 1, 1)
    return y


@operator("Gemm")
def _gemm(node, ins, opset, **kw):
    a, b = ins[0], ins[1]
    if node.attr("transA", 0):
        a = a.T
    if node.attr("transB", 0):
        b = b.T
    y = np.float32(node.attr("alpha", 1.0)) * native.gemm_f32(a, b)
    if len(ins) > 2 and ins[2] is not None:
        y = y + np.float32(node.attr("beta", 1.0)) * ins[2]
    return y.astype(np.float32)


@operator("MatMul")
def _matmul(node, ins, opset, **kw):
    y = np.matmul(ins[0], ins[1]).astype(np.float32)
    if len(ins) > 2 and ins[2] is not None:
        y = y + ins[2]
    return y


@operator("FusedElementwise")
def _fused(node, ins, opset, **kw):
    env = dict(node.attrs["consts"])
    env[node.inputs[0]] = ins[0]
    for sub in node.attrs["nodes"]:
        env[sub.outputs[0]] = run_node(
            sub, [env[i] if i else None for i in sub.inputs], opset)[0]
    return env[node.outputs[0]]


@operator("BatchNormalization")
def _bn(node, ins, opset, **kw):
    x, gamma, beta, mean, var = ins[:5]
    shape = [1, -1] + [1] * (x.ndim - 2)
    a = gamma / np.sqrt(var + node.attr("epsilon", 1e-5))
    return (x * a.reshape(shape) + (beta - a * mean).reshape(shape)).astype(
        np.float32)


# ------------------------------------------------------- element-wise ----
def _binary(ufunc):
    return lambda node, ins, opset, **kw: ufunc(ins[0], ins[1])


for _op, _ufunc in {"Add": np.add, "Sub": np.subtract, "Mul": np.multiply,
                    "Div": np.divide, "Max": np.maximum,
                    "Min": np.minimum}.items():
    operator(_op)(_binary(_ufunc))


@tabulated("Sigmoid")
def _sigmoid(node, x):
    return (1.0 / (1.0 + np.exp(-x.astype(np.float64)))).astype(np.float32)


@tabulated("Relu")
def _relu(node, x):
    return np.maximum(x, 0)


@tabulated("LeakyRelu")
def _leaky(node, x):
    return np.where(x >= 0, x, node.attr("alpha", 0.01) * x).astype(
        np.float32)


@tabulated("Tanh")
def _tanh(node, x):
    return np.tanh(x).astype(np.float32)


@tabulated("HardSigmoid")
def _hsig(node, x):
    a, b = node.attr("alpha", 0.2), node.attr("beta", 0.5)
    return np.clip(a * x + b, 0, 1).astype(np.float32)


@tabulated("HardSwish")
def _hswish(node, x):
    return (x * np.clip(x / 6.0 + 0.5, 0, 1)).astype(np.float32)


@tabulated("Elu")
def _elu(node, x):
    a = node.attr("alpha", 1.0)
    return np.where(x > 0, x, a * np.expm1(np.minimum(x, 0))).astype(
        np.float32)


@tabulated("Softplus")
def _softplus(node, x):
    return np.logaddexp(0, x.astype(np.float64)).astype(np.float32)


@tabulated("Abs")
def _abs(node, x):
    return np.abs(x)


@tabulated("Neg")
def _neg(node, x):
    return -x


@tabulated("Sqrt")
def _sqrt(node, x):
    return np.sqrt(x).astype(np.float32)


@tabulated("Exp")
def _exp(node, x):
    return np.exp(x.astype(np.float64)).astype(np.float32)


def erf(x):
    """Abramowitz-Stegun 7.1.26 in float64 (the reference's ``_erf``)."""
    x = x.astype(np.float64)
    ax = np.abs(x)
    t = 1.0 / (1.0 + 0.3275911 * ax)
    poly = t * (0.254829592 + t * (-0.284496736 + t * (
        1.421413741 + t * (-1.453152027 + t * 1.061405429))))
    return np.sign(x) * (1.0 - poly * np.exp(-ax * ax))


@tabulated("Erf")
def _erf(node, x):
    return erf(x).astype(np.float32)


@tabulated("Gelu")
def _gelu(node, x):
    x64 = x.astype(np.float64)
    if node.attr("approximate", "none") == "tanh":
        inner = np.sqrt(2 / np.pi) * (x64 + 0.044715 * x64**3)
        return (0.5 * x64 * (1 + np.tanh(inner))).astype(np.float32)
    return (0.5 * x64 * (1 + erf(x64 / np.sqrt(2)))).astype(np.float32)


@operator("Pow")
def _pow(node, ins, opset, **kw):
    return np.power(ins[0].astype(np.float64),
                    np.asarray(ins[1]).astype(np.float64)).astype(np.float32)


@operator("Clip")
def _clip(node, ins, opset, **kw):
    lo = ins[1] if len(ins) > 1 and ins[1] is not None else node.attr("min")
    hi = ins[2] if len(ins) > 2 and ins[2] is not None else node.attr("max")
    return np.clip(ins[0], lo, hi)


def _axis(axis, ndim):
    return axis + ndim if axis < 0 else axis


@operator("Softmax")
def _softmax(node, ins, opset, **kw):
    x = ins[0].astype(np.float64)
    ax = _axis(node.attr("axis", -1 if opset >= 13 else 1), x.ndim)
    e = np.exp(x - x.max(axis=ax, keepdims=True))
    return (e / e.sum(axis=ax, keepdims=True)).astype(np.float32)


@operator("LogSoftmax")
def _log_softmax(node, ins, opset, **kw):
    x = ins[0].astype(np.float64)
    ax = _axis(node.attr("axis", -1 if opset >= 13 else 1), x.ndim)
    z = x - x.max(axis=ax, keepdims=True)
    return (z - np.log(np.exp(z).sum(axis=ax, keepdims=True))).astype(
        np.float32)


@operator("LayerNormalization")
def _layer_norm(node, ins, opset, **kw):
    x = ins[0].astype(np.float64)
    axes = tuple(range(_axis(node.attr("axis", -1), x.ndim), x.ndim))
    mean = x.mean(axis=axes, keepdims=True)
    var = ((x - mean) ** 2).mean(axis=axes, keepdims=True)
    y = (x - mean) / np.sqrt(var + node.attr("epsilon", 1e-5)) * ins[1]
    if len(ins) > 2 and ins[2] is not None:
        y = y + ins[2]
    return y.astype(np.float32)


# ------------------------------------------------------------- shapes ----
@operator("Identity", "Dropout")
def _identity(node, ins, opset, **kw):
    return ins[0]


@operator("Flatten")
def _flatten(node, ins, opset, **kw):
    x = ins[0]
    ax = _axis(node.attr("axis", 1), x.ndim)
    return x.reshape(int(np.prod(x.shape[:ax])), -1)


@operator("Reshape")
def _reshape(node, ins, opset, **kw):
    x = ins[0]
    shape = [int(s) for s in np.asarray(ins[1]).reshape(-1)]
    if not node.attr("allowzero", 0):
        shape = [x.shape[i] if s == 0 else s for i, s in enumerate(shape)]
    return x.reshape(shape)


@operator("Transpose")
def _transpose(node, ins, opset, **kw):
    perm = node.attr("perm")
    return np.transpose(ins[0], perm if perm else None)


def _axes(node, ins, index, attr):
    if len(ins) > index and ins[index] is not None:
        return [int(a) for a in np.asarray(ins[index]).reshape(-1)]
    v = node.attr(attr)
    return None if v is None else [int(a) for a in v]


@operator("Squeeze")
def _squeeze(node, ins, opset, **kw):
    axes = _axes(node, ins, 1, "axes")
    x = ins[0]
    if axes is None:
        return np.squeeze(x)
    return np.squeeze(x, axis=tuple(_axis(a, x.ndim) for a in axes))


@operator("Unsqueeze")
def _unsqueeze(node, ins, opset, **kw):
    axes = _axes(node, ins, 1, "axes")
    x = ins[0]
    out_nd = x.ndim + len(axes)
    for a in sorted(_axis(a, out_nd) for a in axes):
        x = np.expand_dims(x, a)
    return x


@operator("Gather")
def _gather(node, ins, opset, **kw):
    return np.take(ins[0], np.asarray(ins[1]).astype(np.int64),
                   axis=node.attr("axis", 0))


@operator("Slice")
def _slice(node, ins, opset, **kw):
    x = ins[0]
    starts = _axes(node, ins, 1, "starts")
    ends = _axes(node, ins, 2, "ends")
    axes = _axes(node, ins, 3, "axes") or list(range(len(starts)))
    steps = _axes(node, ins, 4, "steps") or [1] * len(starts)
    index = [slice(None)] * x.ndim
    for st, en, a, sp in zip(starts, ends, axes, steps):
        index[_axis(a, x.ndim)] = slice(None if st >= 2**62 else st,
                                        None if abs(en) >= 2**62 else en, sp)
    return x[tuple(index)]


@operator("Concat")
def _concat(node, ins, opset, **kw):
    return np.concatenate(ins, axis=node.attr("axis"))


@operator("Split", multi=True)
def _split(node, ins, opset, **kw):
    x = ins[0]
    ax = _axis(node.attr("axis", 0), x.ndim)
    if len(ins) > 1 and ins[1] is not None:
        sizes = np.asarray(ins[1]).astype(np.int64).tolist()
    else:
        sizes = node.attr("split")
    n_out = len(node.outputs)
    if not sizes:
        sizes = [x.shape[ax] // n_out] * n_out
    return list(np.split(x, np.cumsum(sizes)[:-1], axis=ax))


@operator("GlobalAveragePool")
def _gap(node, ins, opset, **kw):
    x = ins[0]
    return x.mean(axis=tuple(range(2, x.ndim)), keepdims=True).astype(
        np.float32)


@operator("GlobalMaxPool")
def _gmp(node, ins, opset, **kw):
    x = ins[0]
    return x.max(axis=tuple(range(2, x.ndim)), keepdims=True)


@operator("Pad")
def _pad(node, ins, opset, pad_value=None, **kw):
    """Constant padding with ``pad_value`` (the integer path's zero point),
    else the value input or attribute; reflect (mirrored without repeating
    the border) and edge (border repeated) modes (``float_ops.py:499-513``).
    """
    x = ins[0]
    pads = (np.asarray(ins[1]).astype(np.int64).tolist()
            if len(ins) > 1 and ins[1] is not None else node.attr("pads"))
    width = list(zip(pads[:x.ndim], pads[x.ndim:]))
    mode = node.attr("mode", "constant")
    if mode in ("reflect", "edge"):
        return np.pad(x, width, mode=mode)
    if mode != "constant":
        raise UnsupportedOp(f"Pad mode {mode}")
    if pad_value is None:
        pad_value = (np.asarray(ins[2]).reshape(()).item()
                     if len(ins) > 2 and ins[2] is not None
                     else node.attr("value", 0))
    return np.pad(x, width, mode="constant", constant_values=pad_value)


def pool_geometry(node, in_hw):
    """``(kernel, strides, dilations, (top, left, bottom, right))`` of a 2-D
    pooling node: pads from ``auto_pad`` / ``pads``, then the end pads grown
    under ``ceil_mode`` so the last partial window is included
    (``float_ops.py:518-531``)."""
    kernel = tuple(node.attr("kernel_shape"))
    strides = tuple(node.attr("strides", [1] * len(kernel)))
    dil = tuple(node.attr("dilations", [1] * len(kernel)))
    pads = list(conv_pads(node, in_hw, kernel, strides, dil))
    if node.attr("ceil_mode", 0):
        for ax in range(2):
            size = in_hw[ax] + pads[ax] + pads[ax + 2]
            ek = dil[ax] * (kernel[ax] - 1) + 1
            out = -(-(size - ek) // strides[ax]) + 1
            pads[ax + 2] += max((out - 1) * strides[ax] + ek - size, 0)
    return kernel, strides, dil, tuple(pads)


@operator("MaxPool")
def _maxpool(node, ins, opset, pad_value=None, **kw):
    x = ins[0]
    kernel, strides, dil, pads = pool_geometry(node, x.shape[2:])
    if pad_value is None:
        pad_value = (-np.inf if np.issubdtype(x.dtype, np.floating)
                     else np.iinfo(x.dtype).min)
    xp = np.pad(x, ((0, 0), (0, 0), (pads[0], pads[2]), (pads[1], pads[3])),
                constant_values=pad_value)
    ek = [d * (k - 1) + 1 for k, d in zip(kernel, dil)]
    win = sliding_window_view(xp, tuple(ek), axis=(2, 3))
    win = win[:, :, ::strides[0], ::strides[1], ::dil[0], ::dil[1]]
    return win.max(axis=(4, 5))


# ------------------------------------------------- model-file operators ----
# Constant's value fields and the NumPy type their value takes
_CONSTANT_FIELDS = (("value", None), ("value_float", np.float32),
                    ("value_int", np.int64), ("value_floats", None),
                    ("value_ints", np.int64))


def constant_value(node):
    """The value of an ONNX ``Constant`` node (``float_ops.py:101-118``):
    its tensor, or its scalar / list field as float32 / int64."""
    field = next(((f, t) for f, t in _CONSTANT_FIELDS if f in node.attrs),
                 None)
    if field is None:
        raise UnsupportedOp(f"Constant node '{node.name}' has no supported "
                            "value")
    v = np.asarray(node.attrs[field[0]])
    return v if field[1] is None else v.astype(field[1])


@operator("Constant")
def _constant(node, ins, opset, **kw):
    return constant_value(node)


@operator("Shape")
def _shape(node, ins, opset, **kw):
    shape = np.array(np.shape(ins[0]), np.int64)
    return shape[node.attr("start", 0):node.attr("end", None)]


def _per_axis(v, x, axis):
    """A per-axis parameter shaped to broadcast along ``axis`` of x."""
    v = np.asarray(v)
    if v.ndim == 0 or x.ndim == 0:
        return v
    shape = [1] * x.ndim
    shape[axis % x.ndim] = -1
    return v.reshape(shape)


@operator("QuantizeLinear")
def _quantize_linear(node, ins, opset, **kw):
    """y = saturate(round_half_even(x / scale) + zero_point) in the zero
    point's type (uint8 without one), float32 arithmetic."""
    x = np.asarray(ins[0], np.float32)
    axis = node.attr("axis", 1)
    scale = _per_axis(np.asarray(ins[1], np.float32), x, axis)
    zp = ins[2] if len(ins) > 2 and ins[2] is not None else \
        np.zeros((), np.uint8)
    info = np.iinfo(np.asarray(zp).dtype)
    y = np.rint(x / scale) + _per_axis(np.asarray(zp), x, axis).astype(
        np.float32)
    return np.clip(y, info.min, info.max).astype(np.asarray(zp).dtype)


@operator("DequantizeLinear")
def _dequantize_linear(node, ins, opset, **kw):
    """x = (q - zero_point) * scale in float32."""
    q = np.asarray(ins[0])
    axis = node.attr("axis", 1)
    zp = ins[2] if len(ins) > 2 and ins[2] is not None else 0
    zpf = _per_axis(np.asarray(zp), q, axis).astype(np.float32)
    scale = _per_axis(np.asarray(ins[1], np.float32), q, axis)
    return ((q.astype(np.float32) - zpf) * scale).astype(np.float32)


@operator("Expand")
def _expand(node, ins, opset, **kw):
    shape = tuple(int(v) for v in np.asarray(ins[1]).reshape(-1))
    return np.broadcast_to(ins[0], np.broadcast_shapes(ins[0].shape,
                                                       shape)).copy()


# ONNX TensorProto data types of Cast's "to"
CAST_TYPES = {1: np.float32, 2: np.uint8, 3: np.int8, 4: np.uint16,
              5: np.int16, 6: np.int32, 7: np.int64, 9: np.bool_,
              10: np.float16, 11: np.float64}


@operator("Cast")
def _cast(node, ins, opset, **kw):
    to = node.attr("to")
    if to not in CAST_TYPES:
        raise UnsupportedOp(f"Cast to data type {to}")
    return ins[0].astype(CAST_TYPES[to])


@operator("AveragePool")
def _avgpool(node, ins, opset, **kw):
    """Window sums of the zero-padded input over the window's element count
    (or the whole window with count_include_pad), float32."""
    x = ins[0].astype(np.float32)
    kernel, strides, _, pads = pool_geometry(node, x.shape[2:])
    pad = ((0, 0), (0, 0), (pads[0], pads[2]), (pads[1], pads[3]))
    win = sliding_window_view(np.pad(x, pad), tuple(kernel), axis=(2, 3))
    total = win[:, :, ::strides[0], ::strides[1]].sum(axis=(4, 5))
    if node.attr("count_include_pad", 0):
        return (total / (kernel[0] * kernel[1])).astype(np.float32)
    ones = np.pad(np.ones_like(x[:1, :1]), pad)
    cnt = sliding_window_view(ones, tuple(kernel), axis=(2, 3))[
        :, :, ::strides[0], ::strides[1]].sum(axis=(4, 5))
    return (total / cnt).astype(np.float32)


@operator("ReduceMean")
def _reduce_mean(node, ins, opset, **kw):
    x = ins[0]
    axes = (np.asarray(ins[1]).astype(np.int64).tolist()
            if len(ins) > 1 and ins[1] is not None else node.attr("axes"))
    axes = tuple(_axis(a, x.ndim) for a in axes) if axes else None
    return x.mean(axis=axes, keepdims=bool(node.attr("keepdims", 1))).astype(
        np.float32)
