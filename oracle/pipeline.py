"""Oracle of the integer-only inference path (test only).

Given a graph, its q.json parameters and an input batch, computes the integer
outputs on the CPU the way the reference does, as a second implementation
independent of the product package:

* integer parameter derivation restated from ``quant_layers.py``
  (``_weight_qparams`` :50-67, ``_WeightedLayer.prepare`` :241-287,
  ``BatchNormalizationQuantize.prepare`` :411-422,
  ``ActivationQuantize.prepare`` :461-468, Add / Mul / Concat multipliers
  :489-547, GAP multiplier :575-577) with ``utils.py`` maths
  (``calculate_scale_zp`` :66-90, ``quantize`` :97-114,
  ``quantize_multiplier`` :132-149);
* per-layer integer execution restated from the ``quantized_infer_integer``
  methods (``quant_layers.py:195-205``, :320-341, :384-402, :424-441,
  :470-472, :493-590, :642-650) and the container loop
  (``quant_container.py:135-193``), every integer kernel running in the
  oracle C library (``qa_oracle.c``) or the compiled reference
  (``_ref/libqa_ref.so``) through the same ABI.

Parity pins: the kernels by ``tests/test_oracle.py``; the parameter maths by
the reference test-suite's known answers (``tests/test_host_maths.py``).
"""

import json

import numpy as np

from oracle import abi
from oracle.float_ref import UNARY, conv_pads, eval_node

INT32 = (-(2**31), 2**31 - 1)


# ---------------------------------------------------------------- maths --
def quant_type_info(quant_type):
    signed = not quant_type.startswith("uint")
    bits = int(quant_type[3 if signed else 4:])
    if signed:
        return bits, True, -(1 << (bits - 1)), (1 << (bits - 1)) - 1
    return bits, False, 0, (1 << bits) - 1


def scale_zp(lo, hi, quant_type):
    bits, signed, qmin, qmax = quant_type_info(quant_type)
    lo, hi = float(lo), float(hi)
    if signed:
        m = max(abs(lo), abs(hi))
        return (1.0 if m == 0 else m / qmax), 0
    lo, hi = min(lo, 0.0), max(hi, 0.0)
    if lo == hi:
        return 1.0, 0
    s = (hi - lo) / qmax
    return s, int(np.clip(np.round(-lo / s), qmin, qmax))


def quantize_np(x, scale, zp, qmin, qmax):
    scale = np.asarray(scale, dtype=np.float64)
    q = np.round(np.asarray(x).astype(np.float64) / scale) + zp
    return np.clip(q, qmin, qmax)


def multiplier(real):
    real = float(real)
    if real == 0:
        return 0, 0
    if real < 0:
        m, s = multiplier(-real)
        return -m, s
    frac, exp = np.frexp(real)
    m = int(np.round(frac * (1 << 31)))
    if m >= 1 << 31:
        m //= 2
        exp += 1
    return m, int(-exp)


def wide_accumulator(bits, k):
    return bits > 15 or ((1 << bits) ** 2) * int(k) >= 1 << 31


# ------------------------------------------------------------- pipeline --
class OraclePipeline:
    """Integer inference of ``graph`` with the parameters of a q.json."""

    def __init__(self, graph, qjson, lib="oracle"):
        if not isinstance(qjson, dict):
            qjson = json.loads(open(qjson).read())
        self.g = graph
        self.lib = abi.load(lib)
        self.quant_type = qjson["quant_type"]
        self.per_channel = qjson["per_channel"]
        self.qp = {k: (float(v["scale"]), int(v["zp"]), int(v["qmin"]),
                       int(v["qmax"])) for k, v in qjson["qparams"].items()}
        self.bits = quant_type_info(self.quant_type)[0]
        self.plan = [self._prepare(n) for n in graph.nodes]

    # ----------------------------------------------------------- prepare --
    def _kind(self, node):
        g, op = self.g, node.op_type
        const = g.is_constant
        if op == "Conv" and len(node.inputs) > 1 and const(node.inputs[1]) \
                and g.initializers[node.inputs[1]].ndim == 4 and (
                    len(node.inputs) < 3 or not node.inputs[2]
                    or const(node.inputs[2])):
            return "conv"
        if op in ("Gemm", "MatMul") and len(node.inputs) > 1 and \
                const(node.inputs[1]) and \
                g.initializers[node.inputs[1]].ndim == 2 and \
                not (op == "Gemm" and node.attr("transA", 0)) and \
                (len(node.inputs) < 3 or not node.inputs[2]
                 or const(node.inputs[2])) and not const(node.inputs[0]):
            return "gemm"
        if op == "BatchNormalization" and all(const(i)
                                              for i in node.inputs[1:5]):
            return "bn"
        if self.bits <= 16 and (
                op in UNARY or op == "FusedElementwise" or
                (op == "Clip" and all(const(i) for i in node.inputs[1:]
                                      if i))):
            return "lut"
        if op in ("Add", "Sub") and not all(const(i) for i in node.inputs):
            return "add"
        if op == "Mul" and not all(const(i) for i in node.inputs):
            return "mul"
        if op == "Concat":
            return "concat"
        if op == "GlobalAveragePool":
            return "gap"
        if op in ("Reshape", "Flatten", "Squeeze", "Unsqueeze", "Transpose",
                  "Split", "Slice", "Pad", "MaxPool", "GlobalMaxPool") and \
                all(const(i) for i in node.inputs[1:] if i):
            # ShapingQuantize.supports (quant_layers.py:617-633): a Pad is
            # scale-preserving only in constant mode with a zero pad value
            if op != "Pad":
                return "shape"
            if node.attr("mode", "constant") == "constant":
                value = (g.initializers[node.inputs[2]]
                         if len(node.inputs) > 2 and node.inputs[2]
                         else node.attr("value", 0))
                if float(np.asarray(value)) == 0.0:
                    return "shape"
        return "fallback"

    def _data_inputs(self, node, kind):
        if kind in ("conv", "gemm", "bn", "lut", "gap", "shape"):
            return [node.inputs[0]]
        if kind in ("add", "mul", "concat"):
            return [i for i in node.inputs if i]
        return [i for i in node.inputs if i and not self.g.is_constant(i)]

    def _weighted(self, node, kind, in_scale, out_scale):
        init = self.g.initializers
        if kind == "conv":
            w = init[node.inputs[1]].astype(np.float32)
            bias = (init[node.inputs[2]].astype(np.float32)
                    if len(node.inputs) > 2 and node.inputs[2] else None)
            axis = 0
        else:
            w = init[node.inputs[1]].astype(np.float32)
            bias = None
            if node.op_type == "Gemm":
                if node.attr("transB", 0):
                    w = w.T
                w = w * np.float32(node.attr("alpha", 1.0))
                if len(node.inputs) > 2 and node.inputs[2]:
                    c = init[node.inputs[2]].astype(np.float32).reshape(-1)
                    bias = np.broadcast_to(c, (w.shape[1],)).astype(
                        np.float32) * np.float32(node.attr("beta", 1.0))
            elif len(node.inputs) > 2 and node.inputs[2]:
                bias = init[node.inputs[2]].astype(np.float32).reshape(-1)
            w = np.ascontiguousarray(w)
            axis = 1
        bits, signed, _, _ = quant_type_info(self.quant_type)
        wmin, wmax = ((-(1 << (bits - 1)), (1 << (bits - 1)) - 1) if signed
                      else (0, (1 << bits) - 1))
        rows = np.moveaxis(w, axis, 0).reshape(w.shape[axis], -1)
        if self.per_channel:
            sz = [scale_zp(r.min(), r.max(), self.quant_type) for r in rows]
        else:
            sz = [scale_zp(rows.min(), rows.max(), self.quant_type)] * len(rows)
        sc = np.array([s for s, _ in sz], dtype=np.float64)
        zp = np.array([z for _, z in sz], dtype=np.int64)
        shape = [1] * w.ndim
        shape[axis] = -1
        wq = quantize_np(w, sc.reshape(shape), zp.reshape(shape), wmin, wmax)
        k = w.size // w.shape[axis]
        wide = wide_accumulator(bits, k)
        wc = (wq.astype(np.int64) - zp.reshape(shape)).astype(
            np.int32 if wide else np.int16)
        bias_int = None
        if bias is not None:
            lo, hi = ((-(1 << 63), (1 << 63) - 1) if bits > 8 else INT32)
            bias_int = np.clip(np.round(bias / (in_scale * sc)), lo, hi
                               ).astype(np.int64)
        # fake quantization (quant_layers.py:264-279): dequantized weights,
        # the integer bias back on the float grid
        fake_w = ((wq.astype(np.int64) - zp.reshape(shape)) *
                  sc.reshape(shape)).astype(np.float32)
        fake_b = (None if bias_int is None else
                  (bias_int * (in_scale * sc)).astype(np.float32))
        pairs = [multiplier(v) for v in in_scale * sc / out_scale]
        mult = np.array([p[0] for p in pairs], dtype=np.int64)
        shift = np.array([p[1] for p in pairs], dtype=np.int64)
        if not self.per_channel:
            mult, shift = mult[:1], shift[:1]
        return dict(wc=wc, wide=wide, bias=bias_int, mult=mult, shift=shift,
                    fake_w=fake_w, fake_b=fake_b)

    def _prepare(self, node):
        kind = self._kind(node)
        ins = self._data_inputs(node, kind)
        step = dict(node=node, kind=kind, ins=ins)
        in_qp = [self.qp[n] for n in ins]
        out_qp = [self.qp[n] for n in node.outputs]
        step.update(in_qp=in_qp, out_qp=out_qp)
        if kind in ("conv", "gemm"):
            step.update(self._weighted(node, kind, in_qp[0][0],
                                       out_qp[0][0]))
        elif kind == "bn":
            init = self.g.initializers
            gamma, beta, mean, var = (init[n].astype(np.float64)
                                      for n in node.inputs[1:5])
            a = gamma / np.sqrt(var + node.attr("epsilon", 1e-5))
            pairs = [multiplier(v) for v in in_qp[0][0] * a / out_qp[0][0]]
            step.update(mult=np.array([p[0] for p in pairs], np.int64),
                        shift=np.array([p[1] for p in pairs], np.int64),
                        qB=np.round((beta - a * mean) / out_qp[0][0]).astype(
                            np.int64))
        elif kind == "lut":
            s, z, lo, hi = in_qp[0]
            q = np.arange(lo, hi + 1, dtype=np.int64)
            x = ((q - z) * s).astype(np.float32)
            args = [x] + [self.g.initializers[i] if i else None
                          for i in node.inputs[1:]]
            y = eval_node(node, args, self.g.opset)[0]
            os_, oz, olo, ohi = out_qp[0]
            step.update(table=quantize_np(y, os_, oz, olo, ohi).astype(
                np.int32), offset=lo)
        elif kind in ("add", "concat"):
            step["mults"] = [multiplier(q[0] / out_qp[0][0]) for q in in_qp]
        elif kind == "mul":
            step["mult"] = multiplier(in_qp[0][0] * in_qp[1][0] /
                                      out_qp[0][0])
        return step

    # --------------------------------------------------------------- run --
    def _run_step(self, st, args):
        L = self.lib
        node, kind = st["node"], st["kind"]
        if kind == "conv":
            x = args[0]
            zp = st["in_qp"][0][1]
            w = st["wc"]
            strides, p, dil = self._conv_geometry(node, x, w)
            acc = L.conv2d_int(x.astype(np.int64) - zp, w, strides, p, dil,
                               node.attr("group", 1), st["wide"])
            n, co, oh, ow = acc.shape
            o = st["out_qp"][0]
            return [L.requantize(acc, n, co, oh * ow, st["mult"],
                                 st["shift"], o[1], o[2], o[3], st["bias"])]
        if kind == "gemm":
            x = args[0]
            k = st["wc"].shape[0]
            acc = L.gemm_int(x.reshape(-1, k).astype(np.int64)
                             - st["in_qp"][0][1], st["wc"], st["wide"])
            m, n = acc.shape
            o = st["out_qp"][0]
            out = L.requantize(acc, m, n, 1, st["mult"], st["shift"], o[1],
                               o[2], o[3], st["bias"])
            shape = ((x.shape[0], n) if node.op_type == "Gemm"
                     else x.shape[:-1] + (n,))
            return [out.reshape(shape)]
        if kind == "bn":
            x = args[0]
            o = st["out_qp"][0]
            c = (x.astype(np.int64) - st["in_qp"][0][1]).astype(np.int32)
            out = L.requantize(c, x.shape[0], x.shape[1],
                               int(np.prod(x.shape[2:])), st["mult"],
                               st["shift"], o[1], o[2], o[3],
                               post_bias=st["qB"])
            return [out.reshape(x.shape)]
        if kind == "lut":
            return [L.lut(args[0], st["table"], st["offset"])]
        if kind == "add":
            (ma, sa), (mb, sb) = st["mults"]
            a, b = st["in_qp"]
            o = st["out_qp"][0]
            return [L.add(args[0], args[1], a[1], ma, sa, b[1], mb, sb, o[1],
                          o[2], o[3], -1 if node.op_type == "Sub" else 1)]
        if kind == "mul":
            a, b = st["in_qp"]
            o = st["out_qp"][0]
            return [L.mul(args[0], args[1], a[1], b[1], *st["mult"], o[1],
                          o[2], o[3])]
        if kind == "concat":
            o = st["out_qp"][0]
            parts = []
            for x, q, (m, s) in zip(args, st["in_qp"], st["mults"]):
                if q[0] == o[0] and q[1] == o[1]:
                    parts.append(np.clip(x, o[2], o[3]).astype(np.int32))
                else:
                    parts.append(L.rescale(x, q[1], m, s, o[1], o[2], o[3]))
            return [np.concatenate(parts, axis=node.attr("axis"))]
        if kind == "gap":
            x = args[0]
            i, o = st["in_qp"][0], st["out_qp"][0]
            area = int(np.prod(x.shape[2:]))
            acc = (x.astype(np.int64) - i[1]).sum(
                axis=tuple(range(2, x.ndim)), keepdims=True)
            m, s = multiplier(i[0] / (o[0] * area))
            return [L.requantize(acc, x.shape[0], x.shape[1], 1, m, s, o[1],
                                 o[2], o[3])]
        if kind == "shape":
            i = st["in_qp"][0]
            pad = i[1] if node.op_type == "Pad" else (
                i[2] if node.op_type == "MaxPool" else None)
            full = [args[0]] + [self.g.initializers[n] if n else None
                                for n in node.inputs[1:]]
            outs = eval_node(node, full, self.g.opset, pad_value=pad)
            return [np.ascontiguousarray(o, dtype=np.int32) for o in outs]
        # float fallback: dequantize -> float op -> quantize
        data = dict(zip(st["ins"], args))
        full = []
        qmap = dict(zip(st["ins"], st["in_qp"]))
        for n in node.inputs:
            if not n:
                full.append(None)
            elif n in data:
                s, z = qmap[n][0], qmap[n][1]
                full.append(L.dequantize_f32(data[n], s, z))
            else:
                full.append(self.g.initializers[n])
        outs = eval_node(node, full, self.g.opset)
        return [self._quantize(y, q) for y, q in zip(outs, st["out_qp"])]

    def _quantize(self, y, qp):
        """``utils.quantize`` (utils.py:97-114) of a fallback output: float32
        and float64 values through the float32 ABI entry (the wrapper casts
        them to float32 first), values of any other type (the integer, bool
        and float16 results of a Cast) divided in float64 and rounded half
        to even."""
        s, z, lo, hi = qp
        y = np.asarray(y)
        if s == 0:
            return np.full(y.shape, z, np.int32)
        if y.dtype in (np.float32, np.float64):
            return self.lib.quantize_f32(y, s, z, lo, hi)
        q = np.round(y.astype(np.float64) / s) + z
        return np.clip(q, lo, hi).astype(np.int32)

    @staticmethod
    def _conv_geometry(node, x, w):
        """Strides, ``(top, left, bottom, right)`` pads with ``auto_pad``
        resolved (``quant_layers.py:302-309`` through ``float_ops.py:132-146``)
        and dilations of a convolution."""
        strides = tuple(node.attr("strides", [1, 1]))
        dil = tuple(node.attr("dilations", [1, 1]))
        return strides, conv_pads(node, x.shape[2:], w.shape[2:], strides,
                                  dil), dil

    def run(self, x, keep=False, overrides=None):
        """Returns ``{output name: int32 quantized array}`` and the
        dequantized float32 outputs in graph-output order; ``keep`` leaves
        every tensor of the pass in ``self.env``. ``overrides`` maps tensor
        names to values used in place of the computed ones (the computed
        values are kept in ``self.computed``), so that layers after a float
        fallback can be checked on the same inputs as another
        implementation's."""
        feeds = x if isinstance(x, dict) else {self.g.input_names[0]: x}
        env = {}
        for name, v in feeds.items():
            s, z, lo, hi = self.qp[name]
            env[name] = self.lib.quantize_f32(np.asarray(v, np.float32), s, z,
                                              lo, hi)
        return self.run_integers(env, keep, overrides)

    def run_integers(self, env, keep=False, overrides=None):
        """:meth:`run` from already quantized graph inputs ``{name: int32
        array}``."""
        env = {k: np.asarray(v, np.int32) for k, v in env.items()}
        self.computed = {}
        for st in self.plan:
            args = [env[n] if n in env else self._const(n) for n in st["ins"]]
            outs = dict(zip(st["node"].outputs, self._run_step(st, args)))
            for name in list(outs):
                if overrides and name in overrides:
                    self.computed[name] = outs[name]
                    outs[name] = np.asarray(overrides[name]).reshape(
                        outs[name].shape).astype(np.int32)
            env.update(outs)
        if keep:
            self.env = env
        ints = {o: env[o] for o in self.g.outputs}
        floats = [self.lib.dequantize_f32(env[o], *self.qp[o][:2])
                  for o in self.g.outputs]
        return ints, floats

    # ------------------------------------------------ fake quantization --
    def _fq(self, x, qp):
        s, z, lo, hi = qp
        return self.lib.dequantize_f32(
            self.lib.quantize_f32(np.asarray(x, np.float32), s, z, lo, hi),
            s, z)

    def fake_step(self, st, args):
        """One layer of the fake-quantized pass (``quant_layers.py:178-193``;
        Conv :311-318 and Gemm :376-382 with dequantized weights and the
        bias on the float grid; shaping ops :638-640 without output
        quantization) on float inputs ``args`` (constants given as
        floats)."""
        node, kind = st["node"], st["kind"]
        xs = [self._fq(a, q) for a, q in zip(args, st["in_qp"])]
        if kind == "conv":
            x = xs[0]
            strides, p, dil = self._conv_geometry(node, x, st["fake_w"])
            y = self.lib.conv2d_f32(x, st["fake_w"], strides, p, dil,
                                    node.attr("group", 1))
            if st["fake_b"] is not None:
                y = y + st["fake_b"].reshape(1, -1, 1, 1)
            outs = [y]
        elif kind == "gemm":
            x = xs[0]
            y = self.lib.gemm_f32(x.reshape(-1, x.shape[-1]), st["fake_w"])
            if st["fake_b"] is not None:
                y = y + st["fake_b"]
            n = st["fake_w"].shape[1]
            outs = [y.reshape((x.shape[0], n) if node.op_type == "Gemm"
                              else x.shape[:-1] + (n,))]
        else:
            data = dict(zip(st["ins"], xs))
            full = [None if not n else data[n] if n in data
                    else self.g.initializers[n] for n in node.inputs]
            outs = eval_node(node, full, self.g.opset)
            if kind == "shape":
                return outs
        return [self._fq(o, q) for o, q in zip(outs, st["out_qp"])]

    def run_fake(self, x):
        """The fake-quantized pass (``quant_container.py:150-160``):
        ``{tensor: float32}`` for every tensor of the pass."""
        feeds = x if isinstance(x, dict) else {self.g.input_names[0]: x}
        env = {k: self._fq(v, self.qp[k]) for k, v in feeds.items()}
        for st in self.plan:
            args = [env[n] if n in env else
                    self.g.initializers[n].astype(np.float32)
                    for n in st["ins"]]
            env.update(zip(st["node"].outputs, self.fake_step(st, args)))
        return env

    def _const(self, name):
        v = self.g.initializers[name].astype(np.float32)
        s, z, lo, hi = self.qp[name]
        return quantize_np(v, s, z, lo, hi).astype(np.int32)
