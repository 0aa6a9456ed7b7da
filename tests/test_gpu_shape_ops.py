"""Integer Pad (zero point), MaxPool (qmin padding: explicit pads, dilation,
ceil_mode, auto_pad) and GlobalMaxPool on the device, inside graphs, vs the
oracle pipeline on the same q.json: bit-exact for int8, uint8 and int16
(quant_layers.py:593-650, float_ops.py:499-560, :586-589)."""

import numpy as np
import pytest

from oracle.pipeline import OraclePipeline
from quantanything_amd import graph as G
from quantanything_amd.container import QuantContainer
from quantanything_amd.synth import Stream

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("per_channel", [True, False])
@pytest.mark.parametrize("quant_type", ["int8", "uint8", "int16"])
def test_sppf_pad_maxpool_bit_exact(hip, tmp_path, quant_type, per_channel):
    g = G.mini_sppf(seed=4)
    calib = [Stream(40 + i).normal((3, 3, 33, 31), 1.0).astype(np.float32)
             for i in range(2)]
    c = QuantContainer(g, quant_type, per_channel)
    c.calibrate(calib)
    kinds = {l.node.op_type: l.kind for l in c.layers}
    assert kinds["Pad"] == kinds["MaxPool"] == kinds["GlobalMaxPool"] == \
        "shape"
    path = tmp_path / "q.json"
    c.save(path)
    for x in calib:
        got = c.integer_outputs(x)
        ints, _ = OraclePipeline(g, path).run(x)
        for name in g.outputs:
            assert got[name].shape == ints[name].shape, name
            np.testing.assert_array_equal(got[name], ints[name],
                                          err_msg=name)


def test_maxpool_pads_with_qmin_not_zero_point(hip, tmp_path):
    """All-negative activations (zero point far above every value): a
    window that reaches into the padding must still return the window's
    maximum, so the padding must be qmin, not the zero point."""
    g = G.mini_sppf(seed=5)
    calib = [-np.abs(Stream(50).normal((2, 3, 32, 32), 1.0)).astype(
        np.float32) - 0.5]
    c = QuantContainer(g, "uint8", True)
    c.calibrate(calib)
    path = tmp_path / "q.json"
    c.save(path)
    got = c.integer_outputs(calib[0])
    ints, _ = OraclePipeline(g, path).run(calib[0])
    for name in g.outputs:
        np.testing.assert_array_equal(got[name], ints[name], err_msg=name)


def _brute_maxpool(x, k, s, d, pt, pl, oh, ow, pad):
    n, c, h, w = x.shape
    y = np.full((n, c, oh, ow), pad, np.int64)
    for oy in range(oh):
        for ox in range(ow):
            for ky in range(k[0]):
                for kx in range(k[1]):
                    iy, ix = oy * s[0] - pt + ky * d[0], ox * s[1] - pl + \
                        kx * d[1]
                    v = x[:, :, iy, ix] if 0 <= iy < h and 0 <= ix < w \
                        else pad
                    y[:, :, oy, ox] = np.maximum(y[:, :, oy, ox], v)
    return y


@pytest.mark.parametrize("dtype", [np.int8, np.int16])
def test_maxpool_kernel_direct(hip, dtype):
    """qa_d_maxpool on a channels-last tensor whose values all lie below
    zero: windows that reach into the padding return the largest real value
    (the padding value, qmin, is below every element), windows entirely in
    the padding (ceil mode) return the padding value."""
    import ctypes

    import torch

    from quantanything_amd.executor import MaxPoolDesc

    n, c, h, w = 2, 5, 7, 9
    x = -Stream(60).integers(1, 100, (n, c, h, w)).astype(np.int64)
    lo = -128 if dtype == np.int8 else -32768
    k, s, d, (pt, pl) = (3, 2), (2, 3), (2, 1), (2, 1)
    oh, ow = 6, 4  # the last row of windows lies entirely in the padding
    xd = torch.from_numpy(x.transpose(0, 2, 3, 1).astype(dtype).copy()).cuda()
    yd = torch.full((n, oh, ow, c), 77, dtype=xd.dtype, device="cuda")
    desc = MaxPoolDesc()
    desc.x, desc.code, desc.y = xd.data_ptr(), np.dtype(dtype).itemsize, \
        yd.data_ptr()
    desc.x_sn, desc.x_sc, desc.x_sh, desc.x_sw = h * w * c, 1, w * c, c
    desc.y_sn, desc.y_sc, desc.y_sh, desc.y_sw = oh * ow * c, 1, ow * c, c
    desc.N, desc.C, desc.H, desc.W, desc.OH, desc.OW = n, c, h, w, oh, ow
    desc.KH, desc.KW, desc.SH, desc.SW, desc.DH, desc.DW = *k, *s, *d
    desc.PT, desc.PL, desc.pad = pt, pl, lo
    lib = hip.library()
    assert lib.qa_d_maxpool(ctypes.byref(desc), None) == 0
    torch.cuda.synchronize()
    got = yd.cpu().numpy().astype(np.int64).transpose(0, 3, 1, 2)
    want = _brute_maxpool(x, k, s, d, pt, pl, oh, ow, lo)
    np.testing.assert_array_equal(got, want)
    assert (got == lo).any() and (got < 0).all()
