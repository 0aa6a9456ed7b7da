"""A graph input read only by a convolution whose stride is its kernel (a
transformer's patch embedding) is quantized straight into that
convolution's im2col rows (qa_d_quantize_patches), and the convolution runs
as a 1x1 convolution over one-pixel images of KH*KW*4 channels. The
reference quantizes the input and convolves it through im2col
(quant_container.py:150-155, qa_kernels.cpp:107-175); every tensor the
device pass keeps equals the oracle's bit for bit."""

import numpy as np
import pytest

from oracle.pipeline import OraclePipeline
from quantanything_amd import graph as G
from quantanything_amd.container import QuantContainer
from quantanything_amd.synth import Stream

pytestmark = pytest.mark.gpu


def _patch_graph(cin, cout, k, act):
    b = G.GraphBuilder(7 + k)
    y = b.conv("x", cin, cout, k, k, pad=0,
               w_scale=np.sqrt(2.0 / (cin * k * k)), b_scale=0.05)
    if act:
        y = b.silu(y)
    return b.build("x", [None, cin, None, None], y)


CASES = [
    (3, 64, 16, 32, 32, 2, False),   # ViT-style: 16x16 patches
    (1, 32, 8, 24, 40, 3, True),     # one channel, non-square image
    (4, 16, 4, 12, 12, 2, True),     # four channels, 4x4 patches
    (3, 48, 12, 36, 24, 1, False),   # kernel of 12 columns
]


@pytest.mark.parametrize("quant_type", ["int8", "uint8"])
@pytest.mark.parametrize("cin,cout,k,h,w,batch,act", CASES)
def test_patch_input_bit_exact(hip, tmp_path, quant_type, cin, cout, k, h, w,
                               batch, act):
    g = _patch_graph(cin, cout, k, act)
    shape = (batch, cin, h, w)
    calib = [Stream(30 + i).normal(shape).astype(np.float32)
             for i in range(2)]
    cq = QuantContainer(g, quant_type, True)
    cq.calibrate(calib)
    x = Stream(40).normal(shape).astype(np.float32)
    x[0, 0, 0, :4] = [0.0, 1e9, -1e9, 0.5]  # both clip ends
    path = tmp_path / "q.json"
    cq.save(path)
    oracle = OraclePipeline(g, path)
    oracle.run(x, keep=True)
    ex = cq.executor({"x": x.shape})
    names = [nm for nm, _ in ex.launches]
    assert "patches:x" in names and "quantize:x" not in names, names
    ex.run({"x": x})
    checked = 0
    for name, t in ex.tensors.items():
        if name in oracle.env:
            got = t.to_host()
            np.testing.assert_array_equal(
                got, oracle.env[name].reshape(got.shape), err_msg=name)
            checked += 1
    assert g.outputs[0] in ex.tensors and checked >= 1
