"""Softmax float fallback on the device: the fused form that also writes
the dequantized graph output equals the separate Softmax + dequantize
launches exactly, and stays within one quantization step of the oracle's
float64 softmax (quant_layers.py:195-205: dequantize -> float op ->
quantize)."""

import numpy as np
import pytest

from oracle import float_ref
from oracle.pipeline import quantize_np

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows,cols", [(64, 1000), (3, 2500), (5, 7)])
def test_softmax_with_float_output(hip, rows, cols):
    import torch

    lib = hip.library()
    rng = np.random.default_rng(rows * 7 + cols)
    xq = rng.integers(-128, 128, (rows, cols)).astype(np.int8)
    in_scale, in_zp = 0.07, -3
    out_scale, out_zp, qmin, qmax = 1.0 / 255.0, -128, -128, 127
    x = torch.from_numpy(xq).cuda()
    y1 = torch.empty((rows, cols), dtype=torch.int8, device="cuda")
    y2 = torch.empty_like(y1)
    f1 = torch.empty((rows, cols), dtype=torch.float32, device="cuda")
    f2 = torch.empty_like(f1)
    s = torch.cuda.current_stream().cuda_stream
    args = (x.data_ptr(), 1, rows, cols, in_scale, in_zp, 0)
    tail = (out_scale, out_zp, qmin, qmax, 0)
    assert lib.qa_d_softmax(*args, y1.data_ptr(), 1, *tail, s) == 0
    assert lib.qa_d_dequantize_f32(y1.data_ptr(), 1, f1.data_ptr(),
                                   rows * cols, out_scale, out_zp, 0, s) == 0
    assert lib.qa_d_softmax_f32(*args, y2.data_ptr(), 1, *tail,
                                f2.data_ptr(), s) == 0
    torch.cuda.synchronize()
    np.testing.assert_array_equal(y1.cpu().numpy(), y2.cpu().numpy())
    np.testing.assert_array_equal(f1.cpu().numpy(), f2.cpu().numpy())
    ref = quantize_np(float_ref.softmax(
        ((xq.astype(np.float64) - in_zp) * in_scale).astype(np.float32), 1),
        out_scale, out_zp, qmin, qmax)
    assert np.abs(y2.cpu().numpy().astype(np.int64) - ref).max() <= 1
