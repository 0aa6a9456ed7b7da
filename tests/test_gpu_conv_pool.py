"""Convolution fused with the global average pool that consumes it
(qa_d_conv_pool): the pointwise form, whose work-group stages its image's
pixels in LDS, and the general form (a 3x3 kernel). Cases cover channel
counts that are not multiples of 64 (zero bytes past the channels), output
channels that leave part of a work-group's block empty, pixel counts that
are not multiples of 16, and uint8 weights whose zero point needs the row
sums. The pooled int8 / uint8 result equals the oracle's bit for bit (the
reference quantizes the conv output, then pools it:
quant_layers.py:461-468, float_ops.py:588)."""

import numpy as np
import pytest

from oracle.pipeline import OraclePipeline
from quantanything_amd import graph as G
from quantanything_amd.container import QuantContainer
from quantanything_amd.synth import Stream

pytestmark = pytest.mark.gpu


def _head(cin, cout, k, size, act):
    b = G.GraphBuilder(31)
    y = b.op("Relu", [b.conv("x", cin, 2 * cin, 1)])  # an int8 input
    y = b.conv(y, 2 * cin, cout, k)
    if act:
        y = b.silu(y)
    y = b.op("Flatten", [b.op("GlobalAveragePool", [y])], axis=1)
    return b.build("x", [None, cin, size, size], y)


CASES = [
    (24, 80, 1, 7, True),     # 48 channels in (KGp past the channels), 80 out
    (32, 320, 1, 9, True),    # 81 pixels: a partial last tile
    (128, 1280, 1, 7, True),  # the YOLOv8n-cls head
    (8, 24, 1, 5, False),     # 16 channels in, no activation
    (16, 64, 3, 8, True),     # 3x3: the general kernel
]


@pytest.mark.parametrize("quant_type", ["int8", "uint8"])
@pytest.mark.parametrize("cin,cout,k,size,act", CASES)
def test_conv_pool_bit_exact(hip, tmp_path, quant_type, cin, cout, k, size,
                             act):
    g = _head(cin, cout, k, size, act)
    shape = (3, cin, size, size)
    calib = [Stream(90 + i).normal(shape).astype(np.float32)
             for i in range(2)]
    c = QuantContainer(g, quant_type, True)
    c.calibrate(calib)
    x = Stream(99).normal(shape).astype(np.float32) * np.float32(1.2)
    ex = c.executor({"x": x.shape})
    assert any(n.startswith("convpool:") for n, _ in ex.launches), \
        [n for n, _ in ex.launches]
    got = c.integer_outputs(x)[g.outputs[0]]
    path = tmp_path / "q.json"
    c.save(path)
    ints, _ = OraclePipeline(g, path).run(x)
    np.testing.assert_array_equal(got, ints[g.outputs[0]])


def _pw_head(c0, c1, c2, size):
    b = G.GraphBuilder(37)
    y = b.op("Relu", [b.conv("x", 8, c0, 1)])  # an int8 input of c0 channels
    y = b.silu(b.conv(y, c0, c1, 1, w_scale=np.sqrt(1.0 / c0), b_scale=0.05))
    y = b.silu(b.conv(y, c1, c2, 1, w_scale=np.sqrt(1.0 / c1), b_scale=0.05))
    y = b.op("Flatten", [b.op("GlobalAveragePool", [y])], axis=1)
    return b.build("x", [None, 8, size, size], y)


PW_CASES = [
    (384, 256, 1280, 7),  # the YOLOv8n-cls head: Conv_232 -> Conv_240 -> GAP
    (64, 32, 64, 5),      # one K-step each, channel blocks of 16
    (128, 64, 256, 8),    # 64 pixels: four full tiles
    (48, 16, 48, 3),      # K-groups past the channels, one first tile
    (512, 128, 96, 6),    # 8 K-steps in the first convolution
]


@pytest.mark.parametrize("quant_type", ["int8", "uint8"])
@pytest.mark.parametrize("c0,c1,c2,size", PW_CASES)
def test_pointwise_pair_pool_bit_exact(hip, tmp_path, quant_type, c0, c1,
                                       c2, size):
    """A 1x1 convolution feeding a pooled 1x1 convolution: with int8
    weights both run in one launch (qa_d_conv_pw_pool, the intermediate
    never written); with uint8 weights (row sums) the pooled conv alone is
    fused with its pool. The pooled result equals the oracle's bit for
    bit either way."""
    g = _pw_head(c0, c1, c2, size)
    shape = (3, 8, size, size)
    calib = [Stream(190 + i).normal(shape).astype(np.float32)
             for i in range(2)]
    c = QuantContainer(g, quant_type, True)
    c.calibrate(calib)
    x = Stream(199).normal(shape).astype(np.float32) * np.float32(1.2)
    ex = c.executor({"x": x.shape})
    names = [n for n, _ in ex.launches]
    if quant_type == "int8":
        assert any(n.startswith("convpool:") and "+" in n for n in names), \
            names
    else:
        assert any(n.startswith("convpool:") for n in names), names
    got = c.integer_outputs(x)[g.outputs[0]]
    path = tmp_path / "q.json"
    c.save(path)
    ints, _ = OraclePipeline(g, path).run(x)
    np.testing.assert_array_equal(got, ints[g.outputs[0]])
