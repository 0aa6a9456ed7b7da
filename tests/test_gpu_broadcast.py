"""Integer Add / Sub / Mul with NumPy broadcasting on the device (the
reference broadcasts both operands, then runs qa_add / qa_mul element by
element: quantization/native.py:465-500): per-channel and per-column
constants, [N, C, H, W] against [N, C, 1, 1], a constant as the first
operand of Sub, and transposed (strided) operands. Every tensor of the
integer pass equals the oracle's bit for bit, for int8, uint8 and int16."""

import ctypes

import numpy as np
import pytest

from oracle.pipeline import OraclePipeline
from quantanything_amd import graph as G
from quantanything_amd.container import QuantContainer
from quantanything_amd.synth import Stream

pytestmark = pytest.mark.gpu

SHAPE = (2, 6, 9, 11)


def _graph(kind, shape=SHAPE):
    b = G.GraphBuilder(29, opset=13)
    x = "x"
    n, c, h, w = shape
    if kind == "add_channel_const":
        y = b.op("Add", [x, b.weight(c, 1, 1, scale=0.7)])
    elif kind == "sub_const_first":  # per-column constant minus x
        y = b.op("Sub", [b.weight(w, scale=0.7), x])
    elif kind == "mul_gap":  # [N, C, H, W] * [N, C, 1, 1]
        y = b.op("Mul", [x, b.op("Sigmoid", [b.op("GlobalAveragePool",
                                                  [x])])])
    elif kind == "add_gap_first":
        y = b.op("Add", [b.op("GlobalMaxPool", [x]), x])
    elif kind == "mul_row_const":  # a constant over H and W, all channels
        y = b.op("Mul", [x, b.weight(h, w, scale=0.7)])
    elif kind == "add_transposed":  # strided operand, constant per channel
        t = b.op("Transpose", [x], perm=[0, 2, 3, 1])
        y = b.op("Add", [t, b.weight(c, scale=0.7)])
    elif kind == "mul_two_views":  # two differently strided activations
        t = b.op("Transpose", [x], perm=[0, 1, 3, 2])
        u = b.op("Transpose", [b.op("Sigmoid", [x])], perm=[0, 1, 3, 2])
        y = b.op("Mul", [t, u])
    else:
        raise ValueError(kind)
    y = b.op("Relu", [y])
    return b.build(x, [None] + list(shape[1:]), y)


KINDS = ["add_channel_const", "sub_const_first", "mul_gap", "add_gap_first",
         "mul_row_const", "add_transposed", "mul_two_views"]


@pytest.mark.parametrize("quant_type", ["int8", "uint8", "int16"])
@pytest.mark.parametrize("kind", KINDS)
def test_broadcast_binary_bit_exact(hip, tmp_path, quant_type, kind):
    g = _graph(kind)
    calib = [Stream(110 + i).normal(SHAPE).astype(np.float32)
             for i in range(2)]
    c = QuantContainer(g, quant_type, True)
    c.calibrate(calib)
    assert all(r.kind != "float" for r in c.layers), kind
    x = Stream(120).normal(SHAPE).astype(np.float32) * np.float32(1.1)
    got = c.integer_outputs(x)
    path = tmp_path / "q.json"
    c.save(path)
    o = OraclePipeline(g, path)
    ints, _ = o.run(x, keep=True)
    ex = c.executor({"x": x.shape})
    checked = 0
    for name, t in ex.tensors.items():
        if name in o.env:
            v = t.to_host()
            np.testing.assert_array_equal(v, o.env[name].reshape(v.shape),
                                          err_msg=f"{kind}: {name}")
            checked += 1
    assert checked >= 3
    for name in g.outputs:
        np.testing.assert_array_equal(got[name], ints[name])


def test_binary_nd_entry_direct(hip):
    """qa_d_binary_nd on raw device buffers against the reference's
    element-wise formula evaluated in Python integers on the broadcast
    operands: mixed storage codes (int8 with int16), a stride-0 axis on
    each side, a shift of the stored values, Sub (sign -1) and Mul."""
    import torch

    from quantanything_amd.executor import BinaryNd
    lib = hip.require()
    rng = np.random.default_rng(7)
    a = rng.integers(-128, 128, size=(3, 1, 5), dtype=np.int64)
    b = rng.integers(-2000, 2000, size=(4, 1), dtype=np.int64)
    out = (3, 4, 5)
    ad = torch.from_numpy(a.astype(np.int8)).cuda()
    bd = torch.from_numpy(b.astype(np.int16)).cuda()

    def mbqm(v, m, s):
        t = 31 + s
        p = v * m
        return (p + (1 << (t - 1))) >> t if t > 0 else p << -t

    for op, sign in ((0, -1), (0, 1), (1, 1)):
        yd = torch.zeros(out, dtype=torch.int16, device="cuda")
        d = BinaryNd()
        d.a, d.b, d.y = ad.data_ptr(), bd.data_ptr(), yd.data_ptr()
        d.a_code, d.b_code, d.y_code = 1, 2, 2
        d.a_so, d.b_so, d.y_so = 3, -5, 7
        d.ndim, d.op, d.sign = 3, op, sign
        for k, (n_, sa_, sb_, sy_) in enumerate(zip(
                out, (5, 0, 1), (0, 1, 0), (20, 5, 1))):
            d.shape[k], d.as_[k], d.bs[k], d.ys[k] = n_, sa_, sb_, sy_
        d.za, d.ma, d.sa = -4, 1518500250, 1
        d.zb, d.mb, d.sb = 9, 1288490189, 3
        d.zp_out, d.qmin, d.qmax = 11, -30000, 30000
        if op == 1:
            d.ma, d.sa = 1717986918, 2
        assert lib.qa_d_binary_nd(ctypes.byref(d), None) == 0
        torch.cuda.synchronize()
        got = yd.cpu().numpy().astype(np.int64)
        want = np.empty(out, np.int64)
        for i in range(out[0]):
            for j in range(out[1]):
                for k in range(out[2]):
                    va = int(a[i, 0, k]) + 3 - (-4)
                    vb = int(b[j, 0]) - 5 - 9
                    if op == 0:
                        r = mbqm(va, d.ma, d.sa) + sign * mbqm(vb, d.mb,
                                                               d.sb)
                    else:
                        r = mbqm(va * vb, d.ma, d.sa)
                    want[i, j, k] = min(max(r + 11, -30000), 30000) - 7
        np.testing.assert_array_equal(got, want, err_msg=f"op {op}")
