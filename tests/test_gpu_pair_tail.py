"""A C2f block's last 1x1 convolution (cv2) fused into the launch of its
last bottleneck pair (qa_d_conv_pair_tail): cv2 reads the block's Concat,
whose last C channels the pair computes in the same work-group and whose
other channels (the Split halves of cv1 and the earlier bottlenecks) earlier
launches wrote. Cases cover C = 16 and 32, one to six bottlenecks (Concat
widths 48 to 256 channels, K-steps of cv2 partly past the channels), output
widths other than the block's, bottlenecks without the residual Add, and
image sizes whose bands are ragged; C = 64 keeps two launches (the pair's
weights leave too little LDS) and is checked the same way. Every tensor the
device pass keeps equals the oracle's bit for bit (the reference runs the
convolutions one after another: quant_layers.py:320-335)."""

import numpy as np
import pytest

from oracle.pipeline import OraclePipeline
from quantanything_amd import graph as G
from quantanything_amd.container import QuantContainer
from quantanything_amd.synth import Stream

pytestmark = pytest.mark.gpu


def _c2f(c, cout, n, shortcut, seed=61):
    b = G.GraphBuilder(seed)

    def conv(x, cin, co, k):
        return b.silu(b.conv(x, cin, co, k, 1,
                             w_scale=np.sqrt(2.0 / (cin * k * k)),
                             b_scale=0.05))

    y = conv("x", 2 * c, 2 * c, 1)
    first, cur = b.op("Split", [y, b.const(np.array([c, c], np.int64))],
                      n_out=2, axis=1)
    parts = [first, cur]
    for _ in range(n):
        t = conv(conv(cur, c, c, 3), c, c, 3)
        cur = b.op("Add", [cur, t]) if shortcut else t
        parts.append(cur)
    y = conv(b.op("Concat", parts, axis=1), (2 + n) * c, cout, 1)
    return b.build("x", [None, 2 * c, None, None], y)


CASES = [
    (16, 32, 1, True, 20, 2),    # 48 Concat channels (cv2 K-steps past them)
    (32, 64, 2, True, 13, 3),    # 128 channels, two bottlenecks
    (32, 64, 6, True, 9, 2),     # 256 channels: the widest Concat
    (64, 128, 2, True, 9, 2),    # C = 64: not fused
    (16, 48, 3, True, 23, 2),    # five parts, 48 output channels, ragged
    (32, 32, 1, False, 11, 2),   # no residual Add
    (64, 64, 1, True, 7, 1),     # C = 64, one image: not fused
]


@pytest.mark.parametrize("quant_type", ["int8", "uint8"])
@pytest.mark.parametrize("c,cout,n,shortcut,size,batch", CASES)
def test_pair_tail_bit_exact(hip, tmp_path, quant_type, c, cout, n,
                             shortcut, size, batch):
    g = _c2f(c, cout, n, shortcut)
    shape = (batch, 2 * c, size, size)
    calib = [Stream(70 + i).normal(shape).astype(np.float32)
             for i in range(2)]
    cq = QuantContainer(g, quant_type, True)
    cq.calibrate(calib)
    x = Stream(80).normal(shape).astype(np.float32)
    path = tmp_path / "q.json"
    cq.save(path)
    oracle = OraclePipeline(g, path)
    oracle.run(x, keep=True)
    ex = cq.executor({"x": x.shape})
    names = [nm for nm, _ in ex.launches]
    tails = [nm for nm in names if nm.startswith("pairtail:")]
    if quant_type == "int8":
        assert len(tails) == (1 if c <= 32 else 0), names
    if tails:
        # cv2 has no launch of its own
        cv2 = tails[0].rpartition("+")[2]
        assert f"conv:{cv2}" not in names, names
    ex.run({"x": x})
    checked = 0
    for name, t in ex.tensors.items():
        if name in oracle.env:
            got = t.to_host()
            np.testing.assert_array_equal(
                got, oracle.env[name].reshape(got.shape), err_msg=name)
            checked += 1
    assert g.outputs[0] in ex.tensors and checked >= 3
