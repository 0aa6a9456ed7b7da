"""Quantized layers: one per graph node (reference: ``quant_layers.py``).

Each layer records its calibration range, derives its quantization
parameters and precomputes every integer parameter on the host
(``prepare``); the device executor (``executor.py``) turns the prepared
layers into GPU launches. Class roles, ``data_inputs`` selection, output
parameter rules and the parameter formulas restate the reference:

* weighted layers (Conv / Gemm / MatMul): per-channel (or per-tensor) weight
  scale / zero point, ``w_centered``, ``bias_int = clip(round(b / (s_in *
  s_w)))`` in the int32 (<= 8 bits) or int64 range, ``real = s_in * s_w /
  s_out`` -> (M0, shift), accumulator width (``quant_layers.py:209-402``);
* BatchNorm as a per-channel affine requantize (``:405-441``);
* activations as lookup tables over every input value (``:445-472``);
* Add / Mul / Concat multipliers (``:476-560``), GAP (``:563-590``),
  scale-preserving shaping ops (``:593-650``) and the dequantize -> float ->
  quantize fallback for everything else (``:195-205``).
"""

import numpy as np

from quantanything_amd import float_ops
from quantanything_amd.float_ops import run_node
from quantanything_amd.native import accumulator_is_wide
from quantanything_amd.utils import (
    QParams,
    calculate_scale_zp,
    dequantize,
    parse_quant_type,
    quantize,
    quantize_multiplier,
    quantize_multipliers,
)

MAX_LUT_BITS = 16


def _bias_range(num_bits):
    return ((-(1 << 63), (1 << 63) - 1) if num_bits > 8
            else (-(1 << 31), (1 << 31) - 1))


def _weight_qparams(w, axis, quant_type, per_channel):
    """Per-slice ``(scale float64[], zp int64[])`` along ``axis``; every entry
    equal when not ``per_channel`` (``quant_layers.py:50-67``)."""
    rows = np.moveaxis(w, axis, 0).reshape(w.shape[axis], -1)
    if per_channel:
        pairs = [calculate_scale_zp(r.min(), r.max(), quant_type)[:2]
                 for r in rows]
    else:
        pairs = [calculate_scale_zp(rows.min(), rows.max(),
                                    quant_type)[:2]] * rows.shape[0]
    return (np.array([p[0] for p in pairs], dtype=np.float64),
            np.array([p[1] for p in pairs], dtype=np.int64))


class QuantLayer:
    """Generic quantized node: float op sandwiched between dequantize and
    quantize on the integer path."""

    kind = "fallback"

    def __init__(self, node, graph, quant_type="int8", per_channel=True):
        self.node = node
        self.graph = graph
        self.name = node.name
        self.quant_type = quant_type
        self.per_channel = per_channel
        self.num_bits, self.signed = parse_quant_type(quant_type)
        self.data_inputs = self._select_data_inputs()
        self.out_min = [None] * len(node.outputs)
        self.out_max = [None] * len(node.outputs)
        self.in_qp = []
        self.out_qp = []

    def _select_data_inputs(self):
        return [i for i in self.node.inputs
                if i and not self.graph.is_constant(i)]

    def _qp(self, qps, field):
        return getattr(qps[0], field) if qps else None

    in_scale = property(lambda s: s._qp(s.in_qp, "scale"))
    in_zp = property(lambda s: s._qp(s.in_qp, "zp"))
    in_qmin = property(lambda s: s._qp(s.in_qp, "qmin"))
    in_qmax = property(lambda s: s._qp(s.in_qp, "qmax"))
    out_scale = property(lambda s: s._qp(s.out_qp, "scale"))
    out_zp = property(lambda s: s._qp(s.out_qp, "zp"))
    out_qmin = property(lambda s: s._qp(s.out_qp, "qmin"))
    out_qmax = property(lambda s: s._qp(s.out_qp, "qmax"))

    # ------------------------------------------------------------ float ----
    def _full_args(self, data_args):
        data = dict(zip(self.data_inputs, data_args))
        return [None if not n else data[n] if n in data
                else self.graph.initializers[n] for n in self.node.inputs]

    def run_float(self, data_args, **kw):
        return run_node(self.node, self._full_args(data_args),
                        self.graph.opset, **kw)

    def calibrate(self, inputs):
        outs = self.run_float(inputs)
        for i, o in enumerate(outs):
            lo, hi = float(np.min(o)), float(np.max(o))
            if self.out_min[i] is None:
                self.out_min[i], self.out_max[i] = lo, hi
            else:
                self.out_min[i] = min(self.out_min[i], lo)
                self.out_max[i] = max(self.out_max[i], hi)
        return outs

    # ---------------------------------------------------------- finalize ----
    def _default_out_qparams(self):
        qps = []
        for i, name in enumerate(self.node.outputs):
            if self.out_min[i] is None:
                raise ValueError(f"Layer {self.name}: output '{name}' was "
                                 "never observed; run calibrate() first")
            qps.append(QParams(*calculate_scale_zp(
                self.out_min[i], self.out_max[i], self.quant_type)))
        return qps

    def finalize_calibration(self, container):
        self.in_qp = [container.qparams[n] for n in self.data_inputs]
        self.out_qp = self._default_out_qparams()
        for name, qp in zip(self.node.outputs, self.out_qp):
            container.qparams[name] = qp
        self.prepare()

    def load_qparams(self, container):
        self.in_qp = [container.qparams[n] for n in self.data_inputs]
        self.out_qp = [container.qparams[n] for n in self.node.outputs]
        self.prepare()

    def prepare(self):
        """Precomputes the integer parameters once qparams are known."""

    def check_ready(self):
        if not self.out_qp or (self.data_inputs and not self.in_qp):
            raise ValueError(f"Layer {self.name} is not calibrated.")


class WeightedLayer(QuantLayer):
    """Shared weight / bias quantization of Conv and Gemm layers."""

    weight_axis = 0

    def __init__(self, node, graph, quant_type="int8", per_channel=True):
        super().__init__(node, graph, quant_type, per_channel)
        bits = self.num_bits
        self.w_qmin, self.w_qmax = ((-(1 << (bits - 1)), (1 << (bits - 1)) - 1)
                                    if self.signed else (0, (1 << bits) - 1))
        self.b_qmin, self.b_qmax = _bias_range(bits)
        self.bias_int = None

    def _select_data_inputs(self):
        return [self.node.inputs[0]]

    def weights(self):
        """Float ``(weight, bias or None)`` laid out for this layer."""
        raise NotImplementedError

    def prepare(self):
        w, bias = self.weights()
        scale_c, zp_c = _weight_qparams(w, self.weight_axis, self.quant_type,
                                        self.per_channel)
        bshape = [1] * w.ndim
        bshape[self.weight_axis] = -1
        if self.per_channel:
            self.w_scale, self.w_zp = scale_c, zp_c
        else:
            self.w_scale, self.w_zp = float(scale_c[0]), int(zp_c[0])
        self.reduction = int(np.prod(w.shape) // w.shape[self.weight_axis])
        self.wide = accumulator_is_wide(self.num_bits, self.reduction)
        self.w_q = quantize(w, scale_c.reshape(bshape), zp_c.reshape(bshape),
                            self.w_qmin, self.w_qmax)
        self.w_centered = (self.w_q.astype(np.int64) - zp_c.reshape(bshape)
                           ).astype(np.int32 if self.wide else np.int16)
        self.b_scale = self.in_scale * self.w_scale
        if bias is not None:
            self.bias_int = np.clip(np.round(bias / (self.in_scale * scale_c)),
                                    self.b_qmin, self.b_qmax).astype(np.int64)
        else:
            self.bias_int = None
        self.q_mult, self.shift = quantize_multipliers(
            self.in_scale * scale_c / self.out_scale)
        if not self.per_channel:
            self.q_mult, self.shift = self.q_mult[:1], self.shift[:1]


class ConvLayer(WeightedLayer):
    """2-D convolution with constant weights (grouped / depthwise)."""

    kind = "conv"

    def weights(self):
        init = self.graph.initializers
        w = init[self.node.inputs[1]].astype(np.float32)
        bias = None
        if len(self.node.inputs) > 2 and self.node.inputs[2]:
            bias = init[self.node.inputs[2]].astype(np.float32)
        return w, bias

    def geometry(self, x_shape):
        strides, pads, dil, groups = float_ops.conv_geometry(
            self.node, x_shape, self.w_q.shape)
        return strides, pads, dil, groups


class GemmLayer(WeightedLayer):
    """``Gemm`` / ``MatMul`` against a constant ``[K, N]`` matrix."""

    kind = "gemm"
    weight_axis = 1

    def weights(self):
        node, init = self.node, self.graph.initializers
        b = init[node.inputs[1]].astype(np.float32)
        bias = None
        if node.op_type == "Gemm":
            if node.attr("transB", 0):
                b = b.T
            b = b * np.float32(node.attr("alpha", 1.0))
            if len(node.inputs) > 2 and node.inputs[2]:
                c = init[node.inputs[2]].astype(np.float32)
                bias = np.broadcast_to(c.reshape(-1), (b.shape[1],)).astype(
                    np.float32) * np.float32(node.attr("beta", 1.0))
        elif len(node.inputs) > 2 and node.inputs[2]:
            bias = np.ascontiguousarray(
                init[node.inputs[2]].astype(np.float32).reshape(-1))
        return np.ascontiguousarray(b), bias

    def out_shape(self, x_shape):
        if self.node.op_type == "Gemm":
            return (x_shape[0], self.w_q.shape[1])
        return tuple(x_shape[:-1]) + (self.w_q.shape[1],)


class BatchNormLayer(QuantLayer):
    """Inference BatchNorm as a per-channel integer affine map."""

    kind = "bn"

    def _select_data_inputs(self):
        return [self.node.inputs[0]]

    def prepare(self):
        init = self.graph.initializers
        gamma, beta, mean, var = (init[n].astype(np.float64)
                                  for n in self.node.inputs[1:5])
        a = gamma / np.sqrt(var + self.node.attr("epsilon", 1e-5))
        self.q_mult, self.shift = quantize_multipliers(
            self.in_scale * a / self.out_scale)
        self.q_B = np.round((beta - a * mean) / self.out_scale).astype(
            np.int64)


class ActivationLayer(QuantLayer):
    """Element-wise unary function (or fused element-wise region) as a
    lookup table over every input integer."""

    kind = "lut"

    @staticmethod
    def supports(node, graph, quant_type):
        bits, _ = parse_quant_type(quant_type)
        if bits > MAX_LUT_BITS:
            return False
        if node.op_type == "Clip":
            return all(graph.is_constant(i) for i in node.inputs[1:] if i)
        return node.op_type in float_ops.UNARY or \
            node.op_type == "FusedElementwise"

    def _select_data_inputs(self):
        return [self.node.inputs[0]]

    def prepare(self):
        qp, o = self.in_qp[0], self.out_qp[0]
        q_in = np.arange(qp.qmin, qp.qmax + 1, dtype=np.int64)
        y = self.run_float([dequantize(q_in.astype(np.int32), qp.scale,
                                       qp.zp)])[0]
        self.lut = quantize(y, o.scale, o.zp, o.qmin, o.qmax).astype(np.int32)
        self.lut_offset = qp.qmin


class MultiInputLayer(QuantLayer):
    """Layers whose constant operands are quantized like activations."""

    def _select_data_inputs(self):
        return [i for i in self.node.inputs if i]


class AddLayer(MultiInputLayer):
    kind = "add"

    def prepare(self):
        self.mults = [quantize_multiplier(qp.scale / self.out_scale)
                      for qp in self.in_qp]
        self.sign = -1 if self.node.op_type == "Sub" else 1


class MulLayer(MultiInputLayer):
    kind = "mul"

    def prepare(self):
        self.mult, self.shift = quantize_multiplier(
            self.in_qp[0].scale * self.in_qp[1].scale / self.out_scale)


class ConcatLayer(MultiInputLayer):
    kind = "concat"

    def prepare(self):
        self.mults = [quantize_multiplier(qp.scale / self.out_scale)
                      for qp in self.in_qp]


class GlobalAveragePoolLayer(QuantLayer):
    kind = "gap"

    def _select_data_inputs(self):
        return [self.node.inputs[0]]

    def multiplier(self, area):
        return quantize_multiplier(self.in_scale / (self.out_scale * area))


class ShapingLayer(QuantLayer):
    """Scale-preserving layout / selection operators (output parameters are
    the input's)."""

    kind = "shape"
    SUPPORTED = {"Reshape", "Flatten", "Squeeze", "Unsqueeze", "Transpose",
                 "Split", "Slice", "Pad", "MaxPool", "GlobalMaxPool"}

    def _select_data_inputs(self):
        return [self.node.inputs[0]]

    @classmethod
    def supports(cls, node, graph):
        if node.op_type not in cls.SUPPORTED:
            return False
        if not all(graph.is_constant(i) for i in node.inputs[1:] if i):
            return False
        if node.op_type == "Pad":
            if node.attr("mode", "constant") != "constant":
                return False
            value = (graph.initializers[node.inputs[2]]
                     if len(node.inputs) > 2 and node.inputs[2]
                     else node.attr("value", 0))
            return float(np.asarray(value)) == 0.0
        return True

    def _default_out_qparams(self):
        return [self.in_qp[0]] * len(self.node.outputs)


def map_node_to_quant(node, graph, quant_type="int8", per_channel=True):
    """Chooses the layer implementation (``quant_layers.py:653-691``)."""
    op, const = node.op_type, graph.is_constant
    args = (node, graph, quant_type, per_channel)
    if op == "Conv" and len(node.inputs) > 1 and const(node.inputs[1]):
        w = graph.initializers[node.inputs[1]]
        bias_ok = (len(node.inputs) < 3 or not node.inputs[2]
                   or const(node.inputs[2]))
        if w.ndim == 4 and bias_ok:
            return ConvLayer(*args)
    if op in ("Gemm", "MatMul") and len(node.inputs) > 1 and \
            const(node.inputs[1]):
        b = graph.initializers[node.inputs[1]]
        ok = b.ndim == 2 and not (op == "Gemm" and node.attr("transA", 0))
        if len(node.inputs) > 2 and node.inputs[2]:
            ok = ok and const(node.inputs[2])
        if ok and not const(node.inputs[0]):
            return GemmLayer(*args)
    if op == "BatchNormalization" and all(const(i) for i in node.inputs[1:5]):
        return BatchNormLayer(*args)
    if ActivationLayer.supports(node, graph, quant_type):
        return ActivationLayer(*args)
    if op in ("Add", "Sub") and not all(const(i) for i in node.inputs):
        return AddLayer(*args)
    if op == "Mul" and not all(const(i) for i in node.inputs):
        return MulLayer(*args)
    if op == "Concat":
        return ConcatLayer(*args)
    if op == "GlobalAveragePool":
        return GlobalAveragePoolLayer(*args)
    if ShapingLayer.supports(node, graph):
        return ShapingLayer(*args)
    return QuantLayer(*args)
