"""The device element-wise entries on their vectorized paths (rows of one
channel for requantize: int32 accumulators to int8 storage; a byte table in
LDS for int8 -> int8 lookups) against the oracle's requantize and lookup
(qa_kernels.cpp:207-228, :348-358), bit for bit, including extreme
multipliers and shifts, biases on either side and clipping at both ends."""

import numpy as np
import pytest

from quantanything_amd.synth import Stream

pytestmark = pytest.mark.gpu


def _dev(a, dtype):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a, dtype=dtype)).cuda()


@pytest.mark.parametrize("outer,C,inner", [(3, 16, 64), (2, 5, 3136),
                                          (1, 70, 100), (5, 3, 4096)])
@pytest.mark.parametrize("qrange,out_so", [((0, 255), 128), ((-128, 127), 0),
                                           ((-100, 20), 0)])
def test_requantize_rows_match_oracle(hip, oracle_lib, outer, C, inner,
                                      qrange, out_so):
    import torch

    st = Stream(8000 + outer * C + inner)
    acc = st.integers(-(2**31), 2**31 - 1, (outer, C, inner)).astype(np.int32)
    acc[0, 0, :8] = [-(2**31), 2**31 - 1, 0, -1, 1, 2**30, -(2**30), 7]
    mult = st.integers(-(2**31) + 1, 2**31 - 1, (C,))
    mult[0] = 1 << 30
    shift = st.integers(-4, 30, (C,))
    shift[0] = 0
    pre = st.integers(-(2**31), 2**31 - 1, (C,))
    post = st.integers(-300, 300, (C,))
    qmin, qmax = qrange
    zp = 3
    want = oracle_lib.requantize(acc, outer, C, inner, mult, shift, zp, qmin,
                                 qmax, pre_bias=pre, post_bias=post)
    lib = hip.library()
    d_acc = _dev(acc, np.int32)
    out = torch.full((outer * C * inner,), 55, dtype=torch.int8,
                     device="cuda")
    params = [_dev(v, np.int64) for v in (mult, shift, pre, post)]
    rc = lib.qa_d_requantize(d_acc.data_ptr(), 4, out.data_ptr(), 1, outer,
                             C, inner, *(p.data_ptr() for p in params), zp,
                             qmin, qmax, 0, out_so, None)
    assert rc == 0
    torch.cuda.synchronize()
    got = out.cpu().numpy().astype(np.int64).reshape(acc.shape) + out_so
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("n", [16, 4096, 6422528])
@pytest.mark.parametrize("in_so,out_so,offset", [(128, 128, 0), (0, 0, -128),
                                                 (0, 128, -100)])
def test_lut_int8_table_path_matches_oracle(hip, oracle_lib, n, in_so,
                                            out_so, offset):
    import torch

    st = Stream(8100 + n)
    stored = st.integers(-128, 127, (n,)).astype(np.int8)
    length = 200  # shorter than the byte range: indices clip at both ends
    lo = out_so - 128  # values whose stored form q - out_so is int8
    table = st.integers(lo, lo + 255, (length,)).astype(np.int32)
    q = stored.astype(np.int32) + in_so
    want = oracle_lib.lut(q, table, offset)
    x = _dev(stored, np.int8)
    y = torch.empty_like(x)
    t = _dev(table, np.int32)
    rc = hip.library().qa_d_lut(x.data_ptr(), 1, n, y.data_ptr(), 1, n, 1, n,
                                offset, t.data_ptr(), length, in_so, out_so,
                                None)
    assert rc == 0
    torch.cuda.synchronize()
    np.testing.assert_array_equal(y.cpu().numpy().astype(np.int64) + out_so,
                                  want)
