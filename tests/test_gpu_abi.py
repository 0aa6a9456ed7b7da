"""HIP library vs the compiled reference (golden vectors) and the CPU oracle,
through the same C ABI the reference loader binds (test_native.py's cases
and more). Integer results must be bit-exact."""

import hashlib

import numpy as np
import pytest

from quantanything_amd import synth
from tests.golden.cases import (
    CONV_CASES,
    GEMM_CASES,
    conv_case_inputs,
    elementwise_cases,
    gemm_case_inputs,
    quantize_cases,
    requantize_cases,
)

pytestmark = pytest.mark.gpu


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def test_backend_is_the_gpu_library(hip):
    assert hip.backend() == "hip-gfx950"
    buf = np.zeros(64, np.uint8)
    import ctypes

    cbuf = ctypes.create_string_buffer(64)
    assert hip.library().qa_device_arch(cbuf, 64) == 0
    assert cbuf.value.decode().startswith("gfx950"), cbuf.value
    assert hip.library().qa_has_openmp() == 0
    assert hip.library().qa_num_threads() > 0
    del buf


# ------------------------------------------------------------ conv (ABI) --
@pytest.mark.parametrize("wide", [False, True])
@pytest.mark.parametrize("i", range(len(CONV_CASES)))
def test_conv_int_matches_reference(hip, golden, i, wide):
    """Reference test ranges (activations span 511 values: VALU path)."""
    x, w, args = conv_case_inputs(i)
    got = hip.conv2d_int(x, w, *args, wide=wide)
    assert got.dtype == (np.int64 if wide else np.int32)
    np.testing.assert_array_equal(got, golden[f"conv{i}_y{int(wide)}"])


@pytest.mark.parametrize("weights", ["int8", "uint8"])
@pytest.mark.parametrize("wide", [False, True])
@pytest.mark.parametrize("i", range(len(CONV_CASES)))
def test_conv_int_mfma_path(hip, oracle_lib, i, wide, weights):
    """Quantized-model ranges: uint8 activations minus a zero point, int8 or
    uint8-asymmetric weights -> the int8 MFMA path with correction terms."""
    n, c, h, w_, co, k, s, p, d, g = CONV_CASES[i]
    st = synth.Stream(7000 + i)
    zp = int(st.integers(0, 255, (1,))[0])
    x = (st.integers(0, 255, (n, c, h, w_)) - zp).astype(np.int32)
    if weights == "int8":
        w = st.integers(-127, 127, (co, c // g, k, k)).astype(np.int32)
    else:
        wzp = st.integers(0, 255, (co, 1, 1, 1))
        w = (st.integers(0, 255, (co, c // g, k, k)) - wzp).astype(np.int32)
    args = ((s, s), (p, p, p, p), (d, d), g)
    got = hip.conv2d_int(x, w, *args, wide=wide)
    np.testing.assert_array_equal(got, oracle_lib.conv2d_int(x, w, *args,
                                                             wide=wide))


def test_conv_asymmetric_padding(hip, oracle_lib):
    st = synth.Stream(7100)
    x = st.integers(-9, 9, (1, 2, 6, 6)).astype(np.int32)
    w = st.integers(-9, 9, (3, 2, 3, 3)).astype(np.int32)
    args = ((1, 2), (0, 2, 1, 0), (1, 1), 1)
    for wide in (False, True):
        np.testing.assert_array_equal(
            hip.conv2d_int(x, w, *args, wide=wide),
            oracle_lib.conv2d_int(x, w, *args, wide=wide))


def test_conv_shape_mismatch_raises(hip):
    with pytest.raises(ValueError, match="conv shape mismatch"):
        hip.conv2d_int(np.zeros((1, 4, 5, 5), np.int32),
                       np.zeros((3, 3, 3, 3), np.int32))


@pytest.mark.parametrize("i", range(len(CONV_CASES)))
def test_conv_f32(hip, golden, i):
    x, w, args = conv_case_inputs(i)
    xf, wf = (x / 64.0).astype(np.float32), (w / 32.0).astype(np.float32)
    ref = golden[f"conv{i}_yf"]
    np.testing.assert_allclose(hip.conv2d_f32(xf, wf, *args), ref, rtol=1e-4,
                               atol=1e-4 * max(1.0, np.abs(ref).max()))


# ------------------------------------------------------------ GEMM (ABI) --
@pytest.mark.parametrize("i", range(len(GEMM_CASES)))
def test_gemm_int_matches_reference(hip, golden, i):
    a, b = gemm_case_inputs(i)
    for wide in (False, True):
        np.testing.assert_array_equal(hip.gemm_int(a, b, wide),
                                      golden[f"gemm{i}_c{int(wide)}"])


@pytest.mark.parametrize("weights", ["int8", "uint8"])
@pytest.mark.parametrize("i", range(len(GEMM_CASES)))
def test_gemm_int_mfma_path(hip, i, weights):
    m, k, n = GEMM_CASES[i]
    st = synth.Stream(7200 + i)
    a = (st.integers(0, 255, (m, k)) - 77).astype(np.int32)
    if weights == "int8":
        b = st.integers(-127, 127, (k, n)).astype(np.int32)
    else:
        b = (st.integers(0, 255, (k, n)) - st.integers(0, 255, (1, n)))
        b = b.astype(np.int32)
    exact = a.astype(np.int64) @ b.astype(np.int64)
    for wide in (False, True):
        np.testing.assert_array_equal(hip.gemm_int(a, b, wide), exact)


@pytest.mark.parametrize("i", range(len(GEMM_CASES)))
def test_gemm_f32(hip, golden, i):
    a, b = gemm_case_inputs(i)
    np.testing.assert_allclose(hip.gemm_f32(a / 16.0, b / 8.0),
                               golden[f"gemm{i}_cf"], rtol=1e-5, atol=1e-3)


# ------------------------------------------------ requantize / elementwise --
@pytest.mark.parametrize("i", range(len(requantize_cases())))
def test_requantize_matches_reference(hip, golden, i):
    rc = requantize_cases()[i]
    got = hip.requantize(rc["acc"], rc["outer"], rc["C"], rc["inner"],
                         rc["mult"], rc["shift"], rc["zp"], rc["qmin"],
                         rc["qmax"], pre_bias=rc["pre"], post_bias=rc["post"])
    assert got.dtype == np.int32
    np.testing.assert_array_equal(got, golden[f"rq{i}_out"])


def test_requantize_scalar_multiplier_kat(hip):
    acc = np.arange(-60, 60, dtype=np.int32).reshape(2, 3, 20)
    out = hip.requantize(acc, 2, 3, 20, 1 << 30, 0, 1, -128, 127)
    np.testing.assert_array_equal(
        out, np.clip(np.floor(acc * 0.5 + 0.5) + 1, -128, 127))


@pytest.mark.parametrize("i", range(len(elementwise_cases())))
def test_elementwise_matches_reference(hip, golden, i):
    ec = elementwise_cases()[i]
    kind = ec["kind"]
    if kind == "rescale":
        got = hip.rescale(ec["x"], *ec["args"])
    elif kind == "add":
        got = hip.add(ec["a"], ec["b"], *ec["args"])
    elif kind == "mul":
        got = hip.mul(ec["a"], ec["b"], *ec["args"])
    else:
        got = hip.lut(ec["x"], ec["table"], ec["offset"])
    np.testing.assert_array_equal(got, golden[f"ew{i}_out"])


def test_add_broadcasts(hip):
    a = np.arange(6, dtype=np.int32).reshape(2, 3)
    b = np.array([10], dtype=np.int32)
    one = (1 << 30, -1)
    np.testing.assert_array_equal(
        hip.add(a, b, 0, *one, 0, *one, 0, -128, 127), a + b)


@pytest.mark.parametrize("i", range(len(quantize_cases())))
def test_quantize_dequantize_match_reference(hip, golden, i):
    qc = quantize_cases()[i]
    q = hip.quantize_f32(qc["x"], *qc["args"])
    np.testing.assert_array_equal(q, golden[f"qz{i}_q"])
    dq = hip.dequantize_f32(q, qc["args"][0], qc["args"][1])
    np.testing.assert_array_equal(dq.view(np.int32),
                                  golden[f"qz{i}_dq"].view(np.int32))


# -------------------------------------------------------- full workloads --
def test_gemm_workload_abi(hip, golden_workloads):
    """M=4096 K=576 N=64 uint8 x int8 GEMM + requantize through the ABI."""
    g = synth.gemm_workload()
    acc = hip.gemm_int(g["a"].astype(np.int32) - g["zp_in"],
                       g["w"].astype(np.int32))
    out = hip.requantize(acc, g["M"], g["N"], 1, g["mult"], g["shift"],
                         g["zp_out"], g["qmin"], g["qmax"], g["bias"])
    exp = golden_workloads["gemm"]
    assert sha(acc) == exp["acc_sha256"]
    assert sha(out) == exp["out_sha256"]


def test_conv_workload_abi(hip, golden_workloads):
    """b32 64->64 3x3 56x56 conv + requantize + SiLU LUT through the ABI."""
    c = synth.conv_workload()
    exp = golden_workloads["conv"]
    acc = hip.conv2d_int(c["x"].astype(np.int32) - c["zp_in"],
                         c["w"].astype(np.int32), (1, 1), (1,) * 4, (1, 1), 1)
    assert sha(acc) == exp["acc_sha256"]
    n, co, oh, ow = acc.shape
    rq = hip.requantize(acc, n, co, oh * ow, c["mult"], c["shift"],
                        c["zp_out"], c["qmin"], c["qmax"], c["bias"])
    assert sha(rq) == exp["rq_sha256"]
    assert sha(hip.lut(rq, c["lut"], 0)) == exp["out_sha256"]


# ------------------------------------------ error path under a raw loader --
def _raw_conv(lib, x, w, y, n, c, h, w_, co, k, s, p, d, g):
    """A conv call made exactly as the reference's loader makes it: ctypes,
    no error check, no qa_clear_error."""
    import ctypes

    oh = (h + 2 * p - d * (k - 1) - 1) // s + 1
    ow = (w_ + 2 * p - d * (k - 1) - 1) // s + 1
    ptr = lambda a: ctypes.c_void_p(a.ctypes.data)  # noqa: E731
    lib.qa_conv_i32_i16_i32(ptr(x), ptr(w), ptr(y), n, c, h, w_, co, k, k, s,
                            s, p, p, d, d, g, oh, ow)
    return oh, ow


def test_failed_call_does_not_poison_later_calls(hip, golden):
    """A host-side validation failure (groups = 0) zero-fills its output and
    records an error; later calls on the same thread, with the error never
    cleared, compute their full outputs (native.py:104-145 never reads the
    error state)."""
    import ctypes

    lib = hip.library()
    lib.qa_clear_error()
    x = np.ones((1, 4, 5, 5), np.int32)
    w = np.ones((3, 4, 3, 3), np.int16)
    y = np.full((1, 3, 5, 5), 7, np.int32)
    _raw_conv(lib, x, w, y, 1, 4, 5, 5, 3, 3, 1, 1, 1, 0)
    first = lib.qa_last_error()
    assert first is not None and b"geometry" in first
    assert not y.any(), "a failed call must not leave its output unwritten"

    for i in (0, 5):  # a small case and a 64-channel case
        xi, wi, _ = conv_case_inputs(i)
        n, c, h, w_, co, k, s, p, d, g = CONV_CASES[i]
        oh = (h + 2 * p - d * (k - 1) - 1) // s + 1
        ow = (w_ + 2 * p - d * (k - 1) - 1) // s + 1
        yi = np.full((n, co, oh, ow), -1, np.int32)
        _raw_conv(lib, np.ascontiguousarray(xi),
                  np.ascontiguousarray(wi.astype(np.int16)), yi, *CONV_CASES[i])
        np.testing.assert_array_equal(yi, golden[f"conv{i}_y0"])

    a, b = gemm_case_inputs(0)
    m, k = a.shape
    n = b.shape[1]
    a16, b16 = a.astype(np.int16), b.astype(np.int16)
    cm = np.full((m, n), -1, np.int32)
    lib.qa_gemm_i16_i32(m, n, k, ctypes.c_void_p(a16.ctypes.data),
                        ctypes.c_void_p(b16.ctypes.data),
                        ctypes.c_void_p(cm.ctypes.data))
    np.testing.assert_array_equal(cm, golden["gemm0_c0"])
    # the error stays readable until the caller clears it
    assert lib.qa_last_error() is not None
    lib.qa_clear_error()
    assert lib.qa_last_error() is None


@pytest.mark.parametrize("spread", [200, 600])  # MFMA path / VALU path
def test_more_than_65535_output_channels(hip, oracle_lib, spread):
    st = synth.Stream(7300 + spread)
    x = st.integers(-spread // 2, spread // 2, (1, 2, 3, 3)).astype(np.int32)
    w = st.integers(-100, 100, (70001, 2, 1, 1)).astype(np.int32)
    args = ((1, 1), (0, 0, 0, 0), (1, 1), 1)
    for wide in (False, True):
        np.testing.assert_array_equal(
            hip.conv2d_int(x, w, *args, wide=wide),
            oracle_lib.conv2d_int(x, w, *args, wide=wide))


@pytest.mark.parametrize("spread", [200, 600])
def test_more_than_65535_images(hip, oracle_lib, spread):
    st = synth.Stream(7400 + spread)
    x = st.integers(-spread // 2, spread // 2, (70003, 1, 2, 2)).astype(
        np.int32)
    w = st.integers(-100, 100, (3, 1, 2, 2)).astype(np.int32)
    args = ((1, 1), (1, 1, 1, 1), (1, 1), 1)
    for wide in (False, True):
        np.testing.assert_array_equal(
            hip.conv2d_int(x, w, *args, wide=wide),
            oracle_lib.conv2d_int(x, w, *args, wide=wide))


@pytest.mark.parametrize("spread", [200, 600])
def test_gemm_more_than_65535_columns(hip, spread):
    st = synth.Stream(7500 + spread)
    a = st.integers(-spread // 2, spread // 2, (3, 5)).astype(np.int32)
    b = st.integers(-100, 100, (5, 70001)).astype(np.int32)
    exact = a.astype(np.int64) @ b.astype(np.int64)
    for wide in (False, True):
        np.testing.assert_array_equal(hip.gemm_int(a, b, wide), exact)
