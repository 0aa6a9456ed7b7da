"""Slice with any step, Pad in reflect / edge mode or with a non-zero
constant, Gather with an index array and Cast on the device, inside graphs,
vs the oracle pipeline on the same q.json (int8, uint8, int16).

* Slice is scale-preserving (``quant_layers.py:593-650``): the output keeps
  the input's parameters and the values move unchanged, following Python
  slicing (``float_ops.py:469-481``: negative steps, clamped and negative
  bounds, 2^62 as an open end).
* The Pads that ``ShapingQuantize.supports`` declines (``quant_layers.py:
  617-633``), Gather (``float_ops.py:490-496``) and Cast (``:398-402``) are
  float fallbacks (``quant_layers.py:195-205``): each value is dequantized,
  moved (or cast) and quantized with the output's own parameters. The
  device does the oracle's arithmetic on the same values, so every tensor
  is compared bit for bit."""

import numpy as np
import pytest

from oracle.pipeline import OraclePipeline
from quantanything_amd import graph as G
from quantanything_amd.container import QuantContainer
from quantanything_amd.synth import Stream

pytestmark = pytest.mark.gpu

SHAPE = (2, 6, 9, 11)
BIG = 2**62
I64 = np.int64


def _slice(b, x, starts, ends, axes, steps):
    return b.op("Slice", [x, b.const(np.array(starts, I64)),
                          b.const(np.array(ends, I64)),
                          b.const(np.array(axes, I64)),
                          b.const(np.array(steps, I64))])


def _graph(kind):
    b = G.GraphBuilder(29, opset=13)
    x = "x"
    if kind == "slice_pos":  # channels 1..4, every second column
        y = _slice(b, x, [1, 0], [5, BIG], [1, 3], [1, 2])
    elif kind == "slice_rev_c":  # all channels reversed
        y = _slice(b, x, [-1], [-BIG], [1], [-1])
    elif kind == "slice_rev_hw":  # rows 7, 5, 3 and columns from 9 down
        y = _slice(b, x, [7, BIG], [1, 2], [2, -1], [-2, -1])
    elif kind == "slice_clamped":  # bounds far outside the axes
        y = _slice(b, x, [-100, 2], [100, 1000], [2, 3], [3, 1])
    elif kind == "slice_into_conv":  # a strided view consumed by a conv
        s = _slice(b, x, [BIG, 1], [-BIG, 10], [2, 3], [-1, 2])
        y = b.conv(s, SHAPE[1], 8, k=3)
    elif kind == "pad_reflect":
        y = b.op("Pad", [x, b.const(np.array([0, 0, 2, 3, 0, 1, 1, 2], I64))],
                 mode="reflect")
    elif kind == "pad_reflect_wide":  # pads longer than the axes
        y = b.op("Pad", [x, b.const(np.array([0, 0, 10, 1, 0, 0, 9, 25],
                                             I64))], mode="reflect")
    elif kind == "pad_edge":
        y = b.op("Pad", [x, b.const(np.array([0, 1, 3, 0, 0, 2, 1, 4], I64))],
                 mode="edge")
    elif kind == "pad_value":  # a non-zero constant is not the zero point
        y = b.op("Pad", [x, b.const(np.array([0, 0, 1, 2, 0, 0, 2, 1], I64)),
                         b.const(np.float32(0.75))])
    elif kind == "pad_value_3d":
        r = b.op("Reshape", [x, b.const(np.array([2, 6, 99], I64))])
        y = b.op("Pad", [r, b.const(np.array([0, 2, 3, 1, 0, 4], I64)),
                         b.const(np.float32(-1.25))])
    elif kind == "gather_c":  # repeated and negative indices
        y = b.op("Gather", [x, b.const(np.array([5, -1, 0, 2, 2], I64))],
                 axis=1)
    elif kind == "gather_2d":  # a 2-D index array on the rows
        r = b.op("Reshape", [x, b.const(np.array([2, 54, 11], I64))])
        g = b.op("Gather", [r, b.const(np.array([[3, 50, -2], [0, 7, 7]],
                                                I64))], axis=1)
        y = b.op("Reshape", [g, b.const(np.array([2, 6, 11], I64))])
    elif kind == "gather_w":
        y = b.op("Gather", [x, b.const(np.array([10, 0, 4], I64))], axis=-1)
    elif kind.startswith("cast_"):
        to = {"i32": 6, "i8": 3, "u8": 2, "bool": 9, "f16": 10, "i64": 7,
              "f64": 11, "i16": 5, "u16": 4}[kind[5:]]
        y = b.op("Cast", [b.op("Mul", [x, b.const(np.float32(40.0))])],
                 to=to)
    else:
        raise ValueError(kind)
    y = b.op("Relu", [y])  # an integer layer after the operator
    return b.build(x, [None] + list(SHAPE[1:]), y)


SLICES = ["slice_pos", "slice_rev_c", "slice_rev_hw", "slice_clamped",
          "slice_into_conv"]
FALLBACKS = ["pad_reflect", "pad_reflect_wide", "pad_edge", "pad_value",
             "pad_value_3d", "gather_c", "gather_2d", "gather_w", "cast_i32",
             "cast_i8", "cast_u8", "cast_bool", "cast_f16", "cast_i64",
             "cast_f64", "cast_i16", "cast_u16"]


@pytest.mark.parametrize("quant_type", ["int8", "uint8", "int16"])
@pytest.mark.parametrize("kind", SLICES + FALLBACKS)
def test_index_ops_bit_exact(hip, tmp_path, quant_type, kind):
    print(f"case {kind} {quant_type}", flush=True)
    g = _graph(kind)
    calib = [Stream(90 + i).normal(SHAPE).astype(np.float32)
             for i in range(2)]
    c = QuantContainer(g, quant_type, True)
    c.calibrate(calib)
    op = "Slice" if kind.startswith("slice") else \
        {"pad": "Pad", "gat": "Gather", "cas": "Cast"}[kind[:3]]
    role = {r.node.op_type: r.kind for r in c.layers}[op]
    assert role == ("shape" if op == "Slice" else "float"), role
    x = Stream(99).normal(SHAPE).astype(np.float32) * np.float32(1.2)
    ex = c.executor({"x": x.shape})
    ex.run({"x": x})
    path = tmp_path / "q.json"
    c.save(path)
    o = OraclePipeline(g, path)
    o.run(x, keep=True)
    checked = 0
    for n, t in ex.tensors.items():
        if n in o.env:
            got = t.to_host()
            want = o.env[n]
            assert got.shape == want.shape, (n, got.shape, want.shape)
            np.testing.assert_array_equal(got, want, err_msg=n)
            checked += 1
    assert checked >= 3
    out = g.outputs[0]
    np.testing.assert_array_equal(c.integer_outputs(x)[out], o.env[out])
