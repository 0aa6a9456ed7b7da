"""Quantization container: calibration, q.json persistence and integer
inference on the GPU (reference: ``quantization/quant_container.py``).

``QuantContainer(graph, quant_type, per_channel)`` builds one quantized layer
per node, ``calibrate`` runs float batches and records ranges, ``finalize``
derives every tensor's QParams and each layer's integer parameters, and
``run_graph(x, "integer")`` executes the integer-only pass on the device
(``executor.DeviceExecutor``) and returns dequantized float outputs, like the
reference's integer mode (``quant_container.py:119-193``). ``save`` / ``load``
write and read the reference's q.json format (``:226-267``):
``{"quant_type", "per_channel", "qparams": {tensor: {scale, zp, qmin,
qmax}}}``; the graph plus q.json fully determine the integer model.
"""

import json
from pathlib import Path

import numpy as np

from quantanything_amd import float_ops
from quantanything_amd.layers import map_node_to_quant
from quantanything_amd.utils import QParams, calculate_scale_zp, quantize

MODES = ("float", "calibrate", "integer")


def _is_batches(x):
    return not isinstance(x, (np.ndarray, dict))


class QuantContainer:
    """Post-training static quantization of a graph, executed on the GPU."""

    def __init__(self, graph, quant_type="int8", per_channel=True):
        self.graph = graph
        self.quant_type = quant_type
        self.per_channel = per_channel
        self.quant_layers = {
            node.name: map_node_to_quant(node, graph, quant_type, per_channel)
            for node in graph.nodes}
        self.qparams = {}
        self._input_range = {}
        self.const_names = []
        for layer in self.quant_layers.values():
            for n in layer.data_inputs:
                if graph.is_constant(n) and n not in self.const_names:
                    self.const_names.append(n)
        self.const_q = {}
        self.calibrated = False
        self._executors = {}

    @property
    def layers(self):
        return list(self.quant_layers.values())

    # -------------------------------------------------------- calibration --
    def calibrate(self, x_calib, verbose=False):
        """Runs calibration batches, then :meth:`finalize`."""
        batches = x_calib if _is_batches(x_calib) else [x_calib]
        count = 0
        for batch in batches:
            self._calibrate_batch(batch)
            count += 1
        if count == 0:
            raise ValueError("no calibration data provided")
        self.finalize()
        if verbose:
            print(f"Calibrated on {count} batch(es).")

    def _calibrate_batch(self, batch):
        feeds = float_ops.normalize_feeds(self.graph, batch)
        env = {}
        for name, value in feeds.items():
            lo, hi = float(value.min()), float(value.max())
            cur = self._input_range.get(name)
            self._input_range[name] = (lo, hi) if cur is None else (
                min(cur[0], lo), max(cur[1], hi))
            env[name] = value
        for name in self.const_names:
            env[name] = self.graph.initializers[name]
        for layer in self.layers:
            outs = layer.calibrate([env[n] for n in layer.data_inputs])
            env.update(zip(layer.node.outputs, outs))

    def finalize(self):
        """Derives qparams from the collected ranges and prepares layers."""
        self.qparams = {name: QParams(*calculate_scale_zp(lo, hi,
                                                          self.quant_type))
                        for name, (lo, hi) in self._input_range.items()}
        self._quantize_constants(from_values=True)
        for layer in self.layers:
            layer.finalize_calibration(self)
        self.calibrated = True
        self._executors = {}

    def _quantize_constants(self, from_values):
        self.const_q = {}
        for name in self.const_names:
            value = self.graph.initializers[name].astype(np.float32)
            if from_values:
                self.qparams[name] = QParams(*calculate_scale_zp(
                    value.min(), value.max(), self.quant_type))
            qp = self.qparams[name]
            self.const_q[name] = quantize(value, qp.scale, qp.zp, qp.qmin,
                                          qp.qmax)

    # ---------------------------------------------------------- execution --
    def executor(self, input_shapes):
        """The (cached) device executor for these input shapes."""
        if not self.calibrated:
            raise ValueError("Container is not calibrated; call calibrate().")
        from quantanything_amd.executor import DeviceExecutor

        key = tuple(sorted((k, tuple(v)) for k, v in input_shapes.items()))
        if key not in self._executors:
            self._executors[key] = DeviceExecutor(self, dict(input_shapes))
        return self._executors[key]

    def run_graph(self, x, mode="integer", use_graph=False):
        """``"float"``: float32 reference pass; ``"integer"``: integer-only
        pass on the GPU, outputs dequantized to float32."""
        if mode not in MODES:
            raise ValueError(f"Unknown graph mode: {mode}")
        if mode == "float":
            return float_ops.run_float(self.graph, x)
        if mode == "calibrate":
            self._calibrate_batch(x)
            return None
        if not self.calibrated:
            raise ValueError("Container is not calibrated; call calibrate().")
        feeds = float_ops.normalize_feeds(self.graph, x)
        ex = self.executor({k: v.shape for k, v in feeds.items()})
        outs = ex.run(feeds, use_graph=use_graph)
        res = [outs[o] for o in self.graph.outputs]
        return res[0] if len(res) == 1 else res

    def quantized_infer(self, x, mode="integer"):
        return self.run_graph(x, mode=mode)

    def integer_outputs(self, x):
        """Runs the integer pass and returns the graph outputs as quantized
        integers (int32 arrays), before dequantization."""
        feeds = float_ops.normalize_feeds(self.graph, x)
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
        c._quantize_constants(from_values=False)
        for layer in c.layers:
            layer.load_qparams(c)
        c.calibrated = True
        return c
