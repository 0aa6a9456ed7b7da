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
