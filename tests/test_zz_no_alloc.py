"""The allocation-free GEMM entry (qa_gemm_i16_i32_noalloc) against the
existing ABI entry qa_gemm_i16_i32 on the same operands: bit-exact, over
consecutive calls that share the static scratch array (the later calls
smaller), through both device-side paths (int8 MFMA and exact VALU)."""

import numpy as np
import pytest

from quantanything_amd import synth

pytestmark = pytest.mark.gpu


def _noalloc(lib, a, b):
    import torch

    m, k = a.shape
    n = b.shape[1]
    da = torch.from_numpy(np.ascontiguousarray(a, np.int16)).cuda()
    db = torch.from_numpy(np.ascontiguousarray(b, np.int16)).cuda()
    dc = torch.full((m, n), -7, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.qa_gemm_i16_i32_noalloc(m, n, k, da.data_ptr(), db.data_ptr(),
                                     dc.data_ptr(), stream)
    err = lib.qa_last_error()
    lib.qa_clear_error()
    assert rc == 0, err
    torch.cuda.synchronize()
    return dc.cpu().numpy()


def _operands(seed, m, k, n, a_span, b_kind):
    st = synth.Stream(seed)
    zp = int(st.integers(0, 255, (1,))[0])
    a = (st.integers(0, a_span - 1, (m, k)) - zp).astype(np.int32)
    if b_kind == "int8":
        b = st.integers(-127, 127, (k, n)).astype(np.int32)
    elif b_kind == "uint8":  # asymmetric: per-column offsets on the device
        b = (st.integers(0, 255, (k, n)) - st.integers(0, 255, (1, n)))
        b = b.astype(np.int32)
    else:  # spans more than 256 values
        b = st.integers(-700, 700, (k, n)).astype(np.int32)
    return a, b


def test_noalloc_gemm_matches_abi_entry(hip):
    lib = hip.library()
    lib.qa_clear_error()
    cases = [
        # the standalone GEMM shape, u8 activations, int8 weights: MFMA
        (9100, 4096, 576, 64, 256, "int8"),
        # smaller, asymmetric weights: MFMA with column offsets
        (9101, 300, 200, 70, 256, "uint8"),
        # smaller again, activations spanning 600 values: VALU
        (9102, 33, 100, 17, 600, "int8"),
        # smaller, weights spanning 1401 values: VALU
        (9103, 7, 37, 30, 256, "wide"),
        # MFMA again after the VALU calls (the header is re-initialised)
        (9104, 5, 16, 3, 256, "int8"),
    ]
    for seed, m, k, n, span, kind in cases:
        a, b = _operands(seed, m, k, n, span, kind)
        want = hip.gemm_int(a, b, False)  # qa_gemm_i16_i32
        got = _noalloc(lib, a, b)
        np.testing.assert_array_equal(got, want, err_msg=f"case {seed}")


def test_noalloc_gemm_empty_reduction_and_rejection(hip):
    import torch

    lib = hip.library()
    lib.qa_clear_error()
    a = np.zeros((3, 0), np.int16)
    b = np.zeros((0, 5), np.int16)
    got = _noalloc(lib, a, b)
    np.testing.assert_array_equal(got, np.zeros((3, 5), np.int32))

    cap = lib.qa_noalloc_scratch_bytes()
    assert cap == 32 << 20
    m, k, n = 1 << 20, 64, 64
    assert lib.qa_gemm_i16_i32_noalloc_need(m, n, k) > cap
    tiny = torch.zeros(16, dtype=torch.int32, device="cuda")
    rc = lib.qa_gemm_i16_i32_noalloc(m, n, k, tiny.data_ptr(),
                                     tiny.data_ptr(), tiny.data_ptr(), None)
    err = lib.qa_last_error()
    lib.qa_clear_error()
    assert rc == -1 and b"maximum" in err
    torch.cuda.synchronize()
    assert not tiny.cpu().numpy().any()  # nothing was queued
