"""Quantization container: calibration, q.json persistence, fake-quantized
and integer inference (reference: ``quantization/quant_container.py``).

``QuantContainer(graph, quant_type, per_channel)`` keeps one quantization
record (:class:`~quantanything_amd.qnodes.QNode`) per graph node.
``calibrate`` runs float batches and widens every tensor's observed range;
``finalize`` turns the ranges into QParams and each record's integer
parameters. ``run_graph(x, mode)`` runs one of the reference's four modes
(``quant_container.py:19``, ``:115-193``):

* ``"float"``: the float32 graph;
* ``"calibrate"``: one calibration batch (ranges only);
* ``"quantize"`` (the default, as in the reference): fake quantization,
  every record's float evaluation between quantize-dequantize steps;
* ``"integer"``: the integer-only pass, on the device
  (:class:`~quantanything_amd.executor.DeviceExecutor`), outputs dequantized
  to float32.

``save`` / ``load`` write and read the reference's q.json (``:226-267``):
``{"quant_type", "per_channel", "qparams": {tensor: {scale, zp, qmin,
qmax}}}``; graph plus q.json fully determine the integer model.
"""

import json
from pathlib import Path

import numpy as np

from quantanything_amd import float_ops
from quantanything_amd.qnodes import QNode
from quantanything_amd.utils import (
    QParams,
    calculate_scale_zp,
    fake_quantize,
    quantize,
)

MODES = ("float", "calibrate", "quantize", "integer")


def _batches(x):
    """One batch (array or dict of arrays) as a list, or the iterable of
    batches itself."""
    return [x] if isinstance(x, (np.ndarray, dict)) else x


class QuantContainer:
    """Post-training static quantization of a graph, executed on the GPU."""

    def __init__(self, graph, quant_type="int8", per_channel=True):
        self.graph = graph
        self.quant_type = quant_type
        self.per_channel = per_channel
        self.records = {node.name: QNode(node, graph, quant_type, per_channel)
                        for node in graph.nodes}
        self.qparams = {}
        self.ranges = {}  # graph input -> observed (lo, hi)
        # constants consumed as quantized operands (e.g. Add of a bias)
        self.const_names = list(dict.fromkeys(
            n for r in self.records.values() for n in r.inputs
            if graph.is_constant(n)))
        self.const_q = {}
        self.calibrated = False
        self._executors = {}

    @property
    def layers(self):
        """The records in execution order."""
        return list(self.records.values())

    # -------------------------------------------------------- calibration --
    def calibrate(self, x_calib, verbose=False):
        """Runs calibration batches, then :meth:`finalize`."""
        count = 0
        for batch in _batches(x_calib):
            self._observe(batch)
            count += 1
        if count == 0:
            raise ValueError("no calibration data provided")
        self.finalize()
        if verbose:
            print(f"Calibrated on {count} batch(es).")

    def _observe(self, batch):
        env = dict(float_ops.feed_dict(self.graph, batch))
        for name, v in env.items():
            lo, hi = float(v.min()), float(v.max())
            old = self.ranges.get(name, (lo, hi))
            self.ranges[name] = (min(old[0], lo), max(old[1], hi))
        env.update((n, self.graph.initializers[n]) for n in self.const_names)
        for r in self.records.values():
            env.update(zip(r.node.outputs, r.observe([env[n]
                                                      for n in r.inputs])))

    def finalize(self):
        """Derives qparams from the observed ranges and every record's
        integer parameters."""
        self.qparams = {n: QParams(*calculate_scale_zp(lo, hi,
                                                       self.quant_type))
                        for n, (lo, hi) in self.ranges.items()}
        for n in self.const_names:
            v = self.graph.initializers[n].astype(np.float32)
            self.qparams[n] = QParams(*calculate_scale_zp(v.min(), v.max(),
                                                          self.quant_type))
        self._quantize_constants()
        for r in self.records.values():
            r.settle(self.qparams, derive_outputs=True)
        self.calibrated = True
        self._executors = {}

    def _quantize_constants(self):
        self.const_q = {}
        for n in self.const_names:
            qp = self.qparams[n]
            self.const_q[n] = quantize(
                self.graph.initializers[n].astype(np.float32), qp.scale,
                qp.zp, qp.qmin, qp.qmax)

    # ---------------------------------------------------------- execution --
    def _require_calibration(self):
        if not self.calibrated:
            raise ValueError("Container is not calibrated; call calibrate().")

    def executor(self, input_shapes, fuse_attention=True):
        """The (cached) device executor for these input shapes
        (``fuse_attention``: see ``DeviceExecutor``)."""
        self._require_calibration()
        from quantanything_amd.executor import DeviceExecutor

        key = tuple(sorted((k, tuple(v)) for k, v in input_shapes.items())) \
            + (bool(fuse_attention),)
        if key not in self._executors:
            self._executors[key] = DeviceExecutor(
                self, dict(input_shapes), fuse_attention=fuse_attention)
        return self._executors[key]

    def run_graph(self, x, mode="quantize", use_graph=False):
        """Runs one pass in ``mode`` (see the module docstring); returns the
        graph output (a list when there are several). ``use_graph`` replays
        a captured HIP graph in integer mode."""
        if mode not in MODES:
            raise ValueError(f"Unknown graph mode: {mode}")
        if mode == "float":
            return float_ops.run_float(self.graph, x)
        if mode == "calibrate":
            self._observe(x)
            return None
        self._require_calibration()
        feeds = float_ops.feed_dict(self.graph, x)
        if mode == "quantize":
            res = self._fake_pass(feeds)
        else:
            ex = self.executor({k: v.shape for k, v in feeds.items()})
            outs = ex.run(feeds, use_graph=use_graph)
            res = [outs[o] for o in self.graph.outputs]
        return res[0] if len(res) == 1 else res

    def quantized_infer(self, x, mode="quantize"):
        """Quantized pass: ``"quantize"`` (fake) or ``"integer"``."""
        return self.run_graph(x, mode=mode)

    def _fake_pass(self, feeds):
        """Fake quantization (``quant_container.py:150-160``): graph inputs
        fake-quantized, constant operands as floats, every record through its
        fake-quantized float evaluation; tensors are dropped after their last
        reader."""
        env = {}
        for name, v in feeds.items():
            qp = self.qparams[name]
            env[name] = fake_quantize(v, qp.scale, qp.zp, qp.qmin, qp.qmax)
        env.update((n, self.graph.initializers[n]) for n in self.const_names)
        last = {}
        for i, r in enumerate(self.records.values()):
            for n in r.inputs:
                last[n] = i
        keep = set(self.graph.outputs)
        for i, r in enumerate(self.records.values()):
            env.update(zip(r.node.outputs, r.fake([env[n]
                                                   for n in r.inputs])))
            for n in r.inputs:
                if last.get(n) == i and n not in keep:
                    env.pop(n, None)
        return [env[o] for o in self.graph.outputs]

    def integer_outputs(self, x):
        """Runs the integer pass and returns the graph outputs as quantized
        integers (int32 arrays), before dequantization."""
        feeds = float_ops.feed_dict(self.graph, x)
        ex = self.executor({k: v.shape for k, v in feeds.items()})
        ex.run(feeds)
        return ex.integer_outputs()

    # -------------------------------------------------------- persistence --
    def save(self, path):
        """Writes q.json (quantization parameters, not the weights)."""
        payload = {"quant_type": self.quant_type,
                   "per_channel": self.per_channel,
                   "qparams": {k: v.to_dict()
                               for k, v in self.qparams.items()}}
        Path(path).write_text(json.dumps(payload, indent=2))

    @classmethod
    def load(cls, graph, path):
        """Rebuilds a calibrated container from ``graph`` and a q.json."""
        payload = json.loads(Path(path).read_text())
        c = cls(graph, payload["quant_type"], payload["per_channel"])
        c.qparams = {k: QParams.from_dict(v)
                     for k, v in payload["qparams"].items()}
        missing = [n for n in graph.input_names + c.const_names
                   if n not in c.qparams]
        if missing:
            raise ValueError(f"saved parameters do not match model: {missing}")
        c._quantize_constants()
        for r in c.records.values():
            r.settle(c.qparams, derive_outputs=False)
        c.calibrated = True
        return c
