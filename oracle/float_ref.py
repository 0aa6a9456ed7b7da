"""Float operator semantics needed by the oracle pipeline (test only).

Restated from the reference's ``quantization/float_ops.py`` for the ops that
feed integer parameters (lookup tables are built by evaluating these on every
quantized input value) or run as float fallbacks:
Sigmoid / Exp / Softplus in float64 cast to float32 (``float_ops.py:225-227``
and neighbours), HardSwish / HardSigmoid / LeakyRelu / Elu / Tanh / Relu,
Abramowitz-Stegun erf and Gelu (``:289-320``), binary element-wise ops in
NumPy's promotion, Softmax and LayerNorm in float64 (``:336-347``,
``:380-385``), the float32 MatMul of two activations (``:181-186``), Gather
(``:490-496``) and the integer-safe shaping ops.
"""

import numpy as np
from numpy.lib.stride_tricks import sliding_window_view


def _f32(a):
    return np.asarray(a).astype(np.float32)


def _erf(x):
    x = x.astype(np.float64)
    a = np.abs(x)
    t = 1.0 / (1.0 + 0.3275911 * a)
    p = t * (0.254829592 + t * (-0.284496736 + t * (1.421413741 + t * (
        -1.453152027 + t * 1.061405429))))
    return np.sign(x) * (1.0 - p * np.exp(-a * a))


UNARY = {
    "Sigmoid": lambda n, x: _f32(1.0 / (1.0 + np.exp(-x.astype(np.float64)))),
    "Relu": lambda n, x: np.maximum(x, 0),
    "LeakyRelu": lambda n, x: _f32(np.where(x >= 0, x,
                                            n.attr("alpha", 0.01) * x)),
    "Tanh": lambda n, x: _f32(np.tanh(x)),
    "HardSigmoid": lambda n, x: _f32(np.clip(
        n.attr("alpha", 0.2) * x + n.attr("beta", 0.5), 0, 1)),
    "HardSwish": lambda n, x: _f32(x * np.clip(x / 6.0 + 0.5, 0, 1)),
    "Elu": lambda n, x: _f32(np.where(
        x > 0, x, n.attr("alpha", 1.0) * np.expm1(np.minimum(x, 0)))),
    "Softplus": lambda n, x: _f32(np.logaddexp(0, x.astype(np.float64))),
    "Abs": lambda n, x: np.abs(x),
    "Neg": lambda n, x: -x,
    "Sqrt": lambda n, x: _f32(np.sqrt(x)),
    "Exp": lambda n, x: _f32(np.exp(x.astype(np.float64))),
    "Erf": lambda n, x: _f32(_erf(x)),
}


def _gelu(node, x):
    x = x.astype(np.float64)
    if node.attr("approximate", "none") == "tanh":
        return _f32(0.5 * x * (1 + np.tanh(np.sqrt(2 / np.pi) * (
            x + 0.044715 * x**3))))
    return _f32(0.5 * x * (1 + _erf(x / np.sqrt(2))))


UNARY["Gelu"] = _gelu

BINARY = {"Add": np.add, "Sub": np.subtract, "Mul": np.multiply,
          "Div": np.divide, "Max": np.maximum, "Min": np.minimum}


def softmax(x, axis):
    x = x.astype(np.float64)
    e = np.exp(x - x.max(axis=axis, keepdims=True))
    return _f32(e / e.sum(axis=axis, keepdims=True))


def layer_norm(x, gamma, beta, axis, eps):
    x = x.astype(np.float64)
    axes = tuple(range(axis, x.ndim))
    m = x.mean(axis=axes, keepdims=True)
    v = ((x - m) ** 2).mean(axis=axes, keepdims=True)
    y = (x - m) / np.sqrt(v + eps) * gamma
    return _f32(y + beta if beta is not None else y)


def conv_pads(node, in_hw, kernel, strides, dilations):
    """``(top, left, bottom, right)`` of a convolution or pooling window:
    ``auto_pad`` SAME_UPPER / SAME_LOWER (the output is ceil(size / stride)
    and the padding that needs is split with the odd pixel at the end or at
    the start), VALID (none) or the ``pads`` attribute
    (``float_ops.py:132-146``)."""
    auto = node.attr("auto_pad", "NOTSET")
    if auto in ("SAME_UPPER", "SAME_LOWER"):
        lo, hi = [], []
        for size, k, s, d in zip(in_hw, kernel, strides, dilations):
            out = -(-size // s)
            total = max((out - 1) * s + d * (k - 1) + 1 - size, 0)
            small, big = total // 2, total - total // 2
            lo.append(small if auto == "SAME_UPPER" else big)
            hi.append(big if auto == "SAME_UPPER" else small)
        return (lo[0], lo[1], hi[0], hi[1])
    if auto == "VALID":
        return (0, 0, 0, 0)
    p = node.attr("pads", [0, 0, 0, 0])
    return (p[0], p[1], p[2], p[3])


def pool_pads(node, in_hw, kernel, strides, dilations):
    """:func:`conv_pads`, then, under ``ceil_mode``, the end pads grown so
    that the last partial window is included (``float_ops.py:518-531``)."""
    pads = list(conv_pads(node, in_hw, kernel, strides, dilations))
    if node.attr("ceil_mode", 0):
        for ax in range(2):
            size = in_hw[ax] + pads[ax] + pads[ax + 2]
            ek = dilations[ax] * (kernel[ax] - 1) + 1
            out = -(-(size - ek) // strides[ax]) + 1
            pads[ax + 2] += max((out - 1) * strides[ax] + ek - size, 0)
    return tuple(pads)


def _ints(args, index, node, attr, default=None):
    """An integer list from input ``index`` when given (opset >= 10 / 13
    form), else from attribute ``attr`` (``float_ops.py:125-129``)."""
    if len(args) > index and args[index] is not None:
        return np.asarray(args[index]).astype(np.int64).reshape(-1).tolist()
    return node.attr(attr, default)


# ONNX TensorProto element types of Cast's "to" and their NumPy types, as
# onnx.helper.tensor_dtype_to_np_dtype maps them (float_ops.py:398-402)
CAST_TYPES = {1: np.float32, 2: np.uint8, 3: np.int8, 4: np.uint16,
              5: np.int16, 6: np.int32, 7: np.int64, 9: np.bool_,
              10: np.float16, 11: np.float64}


def eval_node(node, args, opset=13, pad_value=None):
    """Evaluates one node on NumPy arrays; returns the list of outputs."""
    op = node.op_type
    if op in UNARY:
        return [UNARY[op](node, args[0])]
    if op in BINARY:
        return [BINARY[op](args[0], args[1])]
    if op == "Pow":
        return [_f32(np.power(args[0].astype(np.float64),
                              np.asarray(args[1]).astype(np.float64)))]
    if op == "Clip":
        lo = args[1] if len(args) > 1 and args[1] is not None \
            else node.attr("min")
        hi = args[2] if len(args) > 2 and args[2] is not None \
            else node.attr("max")
        return [np.clip(args[0], lo, hi)]
    if op == "FusedElementwise":
        env = dict(node.attrs["consts"])
        env[node.inputs[0]] = args[0]
        for sub in node.attrs["nodes"]:
            env[sub.outputs[0]] = eval_node(
                sub, [env[i] if i else None for i in sub.inputs], opset)[0]
        return [env[node.outputs[0]]]
    if op == "Softmax":
        ax = node.attr("axis", -1 if opset >= 13 else 1)
        return [softmax(args[0], ax + args[0].ndim if ax < 0 else ax)]
    if op == "LogSoftmax":  # float_ops.py:388-395
        ax = node.attr("axis", -1 if opset >= 13 else 1)
        x = args[0].astype(np.float64)
        ax = ax + x.ndim if ax < 0 else ax
        z = x - x.max(axis=ax, keepdims=True)
        return [_f32(z - np.log(np.exp(z).sum(axis=ax, keepdims=True)))]
    if op == "ReduceMean":  # float_ops.py:594-601
        x = args[0]
        axes = (np.asarray(args[1]).astype(np.int64).tolist()
                if len(args) > 1 and args[1] is not None
                else node.attr("axes"))
        axes = tuple(a + x.ndim if a < 0 else a for a in axes) if axes \
            else None
        return [_f32(x.mean(axis=axes,
                            keepdims=bool(node.attr("keepdims", 1))))]
    if op == "Expand":  # float_ops.py:328-333
        shape = tuple(int(v) for v in np.asarray(args[1]).reshape(-1))
        return [np.broadcast_to(args[0], np.broadcast_shapes(
            args[0].shape, shape)).copy()]
    if op == "Cast":  # float_ops.py:398-402
        return [args[0].astype(CAST_TYPES[node.attr("to")])]
    if op == "Slice":  # float_ops.py:469-481: NumPy slicing, 2^62 = open
        x = args[0]
        starts = _ints(args, 1, node, "starts")
        ends = _ints(args, 2, node, "ends")
        axes = _ints(args, 3, node, "axes", list(range(len(starts))))
        steps = _ints(args, 4, node, "steps", [1] * len(starts))
        index = [slice(None)] * x.ndim
        for b, e, a, st in zip(starts, ends, axes, steps):
            index[a + x.ndim if a < 0 else a] = slice(
                None if b >= 2**62 else b, None if abs(e) >= 2**62 else e, st)
        return [x[tuple(index)]]
    if op == "AveragePool":  # float_ops.py:563-577
        x = args[0].astype(np.float32)
        k = tuple(node.attr("kernel_shape"))
        s = tuple(node.attr("strides", [1] * len(k)))
        p = pool_pads(node, x.shape[2:], k, s, (1, 1))
        pad = ((0, 0), (0, 0), (p[0], p[2]), (p[1], p[3]))
        win = sliding_window_view(np.pad(x, pad), k, axis=(2, 3))
        total = win[:, :, ::s[0], ::s[1]].sum(axis=(4, 5))
        if node.attr("count_include_pad", 0):
            return [_f32(total / (k[0] * k[1]))]
        ones = np.pad(np.ones_like(x[:1, :1]), pad)
        cnt = sliding_window_view(ones, k, axis=(2, 3))[
            :, :, ::s[0], ::s[1]].sum(axis=(4, 5))
        return [_f32(total / cnt)]
    if op == "LayerNormalization":
        ax = node.attr("axis", -1)
        return [layer_norm(args[0], args[1], args[2] if len(args) > 2
                           else None, ax + args[0].ndim if ax < 0 else ax,
                           node.attr("epsilon", 1e-5))]
    if op == "Split":
        x = args[0]
        ax = node.attr("axis", 0)
        ax = ax + x.ndim if ax < 0 else ax
        sizes = (np.asarray(args[1]).astype(np.int64).tolist()
                 if len(args) > 1 and args[1] is not None
                 else node.attr("split"))
        if not sizes:
            sizes = [x.shape[ax] // len(node.outputs)] * len(node.outputs)
        return list(np.split(x, np.cumsum(sizes)[:-1], axis=ax))
    if op == "Flatten":
        x = args[0]
        ax = node.attr("axis", 1)
        ax = ax + x.ndim if ax < 0 else ax
        return [x.reshape(int(np.prod(x.shape[:ax])), -1)]
    if op == "Reshape":
        shape = [int(s) for s in np.asarray(args[1]).reshape(-1)]
        if not node.attr("allowzero", 0):
            shape = [args[0].shape[i] if s == 0 else s
                     for i, s in enumerate(shape)]
        return [args[0].reshape(shape)]
    if op == "Transpose":
        perm = node.attr("perm")
        return [np.transpose(args[0], perm if perm else None)]
    if op in ("Squeeze", "Unsqueeze"):
        x = args[0]
        axes = (np.asarray(args[1]).astype(np.int64).reshape(-1).tolist()
                if len(args) > 1 and args[1] is not None
                else node.attr("axes"))
        if op == "Squeeze":
            if axes is None:
                return [np.squeeze(x)]
            return [np.squeeze(x, axis=tuple(a + x.ndim if a < 0 else a
                                             for a in axes))]
        nd = x.ndim + len(axes)
        for a in sorted(a + nd if a < 0 else a for a in axes):
            x = np.expand_dims(x, a)
        return [x]
    if op == "Gather":
        return [np.take(args[0], np.asarray(args[1]).astype(np.int64),
                        axis=node.attr("axis", 0))]
    if op == "MatMul":
        # float32 operands, float32 result (float_ops.py:181-186)
        y = np.matmul(args[0], args[1]).astype(np.float32)
        if len(args) > 2 and args[2] is not None:
            y = y + args[2]
        return [y]
    if op == "Concat":
        return [np.concatenate(args, axis=node.attr("axis"))]
    if op == "GlobalAveragePool":
        x = args[0]
        return [_f32(x.mean(axis=tuple(range(2, x.ndim)), keepdims=True))]
    if op == "Pad":  # float_ops.py:499-513
        x = args[0]
        pads = _ints(args, 1, node, "pads")
        value = pad_value
        if value is None:
            value = (np.asarray(args[2]).reshape(()).item()
                     if len(args) > 2 and args[2] is not None
                     else node.attr("value", 0))
        n = x.ndim
        width = [(pads[i], pads[i + n]) for i in range(n)]
        mode = node.attr("mode", "constant")
        if mode == "constant":
            return [np.pad(x, width, constant_values=value)]
        return [np.pad(x, width, mode={"reflect": "reflect",
                                       "edge": "edge"}[mode])]
    if op == "MaxPool":
        # float_ops.py:518-560: pads from auto_pad / pads, the end pads
        # grown under ceil_mode, then the max over dilated windows
        x = args[0]
        k = tuple(node.attr("kernel_shape"))
        s = tuple(node.attr("strides", [1] * len(k)))
        d = tuple(node.attr("dilations", [1] * len(k)))
        p = list(pool_pads(node, x.shape[2:], k, s, d))
        value = pad_value if pad_value is not None else (
            -np.inf if x.dtype.kind == "f" else np.iinfo(x.dtype).min)
        xp = np.pad(x, ((0, 0), (0, 0), (p[0], p[2]), (p[1], p[3])),
                    constant_values=value)
        ek = tuple(dd * (kk - 1) + 1 for kk, dd in zip(k, d))
        win = sliding_window_view(xp, ek, axis=(2, 3))
        win = win[:, :, ::s[0], ::s[1], ::d[0], ::d[1]]
        return [win.max(axis=(4, 5))]
    if op == "BatchNormalization":  # float_ops.py:200-206, float32
        x, gamma, beta, mean, var = args[:5]
        shape = [1, -1] + [1] * (x.ndim - 2)
        a = gamma / np.sqrt(var + node.attr("epsilon", 1e-5))
        b = beta - a * mean
        return [_f32(x * a.reshape(shape) + b.reshape(shape))]
    if op == "GlobalMaxPool":  # float_ops.py:586-589
        x = args[0]
        return [x.max(axis=tuple(range(2, x.ndim)), keepdims=True)]
    raise NotImplementedError(f"oracle has no float semantics for {op}")
