"""Generic float fallbacks of the integer pass on the device (the
reference's dequantize -> float operator -> quantize for operators with no
integer form, ``quant_layers.py:195-205``): Div / Max / Min / Pow of two
activations or of an activation and a float constant (with broadcasting),
ReduceMean, Softmax and LogSoftmax over any axis, AveragePool, Expand,
Cast to float and LayerNormalization over several trailing axes. Each
single-operator graph runs on the GPU and through the oracle pipeline on
the same q.json; the oracle is given the device's fallback outputs, so every
integer layer around a fallback must be bit-exact, and the fallback itself
within one quantization step of the oracle (float32 / float64 evaluation
order) for at least 99% exact elements."""

import numpy as np
import pytest

from oracle.pipeline import OraclePipeline
from quantanything_amd import graph as G
from quantanything_amd.container import QuantContainer
from quantanything_amd.synth import Stream

pytestmark = pytest.mark.gpu

SHAPE = (2, 6, 9, 11)


def _graph(kind, shape=SHAPE):
    b = G.GraphBuilder(23, opset=13)
    x = "x"
    c = shape[-1]

    def positive(*s):  # a float constant in [0.5, 1.5)
        return b.const((np.abs(b.rng.normal(s, 0.5)) + 0.5).astype(
            np.float32))

    def mix():  # a second activation: a 1x1 convolution of x
        return b.conv(x, shape[1], shape[1], k=1, w_scale=0.5)

    # (element-wise functions of x alone, or of x and a scalar, become one
    # integer table; the operands here keep each operator a fallback)

    if kind == "div":
        den = b.op("Add", [b.op("Sigmoid", [x]), positive(c)])
        y = b.op("Div", [x, den])
    elif kind == "div_const":
        y = b.op("Div", [x, positive(c)])
    elif kind == "rdiv_const":  # the constant as the numerator
        den = b.op("Add", [b.op("Sigmoid", [x]), positive(c)])
        y = b.op("Div", [positive(c), den])
    elif kind == "max":
        y = b.op("Max", [x, mix()])
    elif kind == "max_bcast":  # [N, C, H, W] against [N, C, 1, 1]
        y = b.op("Max", [x, b.op("GlobalAveragePool", [x])])
    elif kind == "min":
        y = b.op("Min", [b.op("Tanh", [x]), mix()])
    elif kind == "min_const":
        y = b.op("Min", [x, b.const(np.linspace(-0.5, 0.5, c).astype(
            np.float32))])
    elif kind == "pow_const":  # integer exponents: negative bases allowed
        y = b.op("Pow", [x, b.const((np.arange(c) % 3 + 1).astype(
            np.float32))])
    elif kind == "pow":
        y = b.op("Pow", [b.op("Sigmoid", [x]), b.op("Tanh", [mix()])])
    elif kind == "mean_hw":
        y = b.op("ReduceMean", [x], axes=[2, 3], keepdims=1)
    elif kind == "mean_c":
        y = b.op("ReduceMean", [x], axes=[1], keepdims=0)
    elif kind == "mean_all":
        y = b.op("ReduceMean", [x], keepdims=0)
    elif kind == "softmax_axis1":
        y = b.op("Softmax", [x], axis=1)
    elif kind == "logsoftmax":
        y = b.op("LogSoftmax", [x], axis=-1)
    elif kind == "logsoftmax_axis2":
        y = b.op("LogSoftmax", [x], axis=2)
    elif kind == "avgpool":
        y = b.op("AveragePool", [x], kernel_shape=[3, 3], strides=[2, 2],
                 pads=[1, 1, 1, 1], count_include_pad=0)
    elif kind == "avgpool_countpad":
        y = b.op("AveragePool", [x], kernel_shape=[3, 2], strides=[2, 1],
                 pads=[1, 0, 1, 1], count_include_pad=1, ceil_mode=1)
    elif kind == "expand":
        y = b.op("Expand", [b.op("GlobalAveragePool", [x]),
                            b.const(np.array([1, 1, 4, 5], np.int64))])
    elif kind == "cast":
        y = b.op("Cast", [x], to=1)
    elif kind == "layernorm_2axes":
        y = b.op("LayerNormalization",
                 [x, b.weight(*shape[2:], scale=0.5),
                  b.weight(*shape[2:], scale=0.2)], axis=-2, epsilon=1e-5)
    else:
        raise ValueError(kind)
    y = b.op("Relu", [y])  # an integer layer after the fallback
    return b.build(x, [None] + list(shape[1:]), y)


KINDS = ["div", "div_const", "rdiv_const", "max", "max_bcast", "min",
         "min_const", "pow_const", "pow", "mean_hw", "mean_c", "mean_all",
         "softmax_axis1", "logsoftmax", "logsoftmax_axis2", "avgpool",
         "avgpool_countpad", "expand", "cast", "layernorm_2axes"]


@pytest.mark.parametrize("quant_type", ["int8", "uint8", "int16"])
@pytest.mark.parametrize("kind", KINDS)
def test_fallback_within_one_step(hip, tmp_path, quant_type, kind):
    g = _graph(kind)
    calib = [Stream(70 + i).normal(SHAPE).astype(np.float32)
             for i in range(2)]
    c = QuantContainer(g, quant_type, True)
    c.calibrate(calib)
    fb = [r.node.outputs[0] for r in c.layers if r.kind == "float"]
    assert fb, f"{kind}: no float fallback in the graph"
    x = Stream(80).normal(SHAPE).astype(np.float32) * np.float32(1.1)
    ex = c.executor({"x": x.shape})
    ex.run({"x": x})
    path = tmp_path / "q.json"
    c.save(path)
    o = OraclePipeline(g, path)
    dev = {n: ex.tensors[n].to_host() for n in fb}
    o.run(x, keep=True, overrides=dev)
    for n in fb:
        want = o.computed[n]
        assert dev[n].size == want.size, n
        d = np.abs(dev[n].astype(np.int64) -
                   want.reshape(dev[n].shape).astype(np.int64))
        assert int(d.max()) <= 1, f"{kind}: {int(d.max())} steps"
        assert float((d == 0).mean()) >= 0.99, \
            f"{kind}: only {float((d == 0).mean()):.4f} exact"
    checked = 0
    for n, t in ex.tensors.items():
        if n in o.env and n not in fb:
            got = t.to_host()
            np.testing.assert_array_equal(got, o.env[n].reshape(got.shape),
                                          err_msg=n)
            checked += 1
    assert checked >= 2
