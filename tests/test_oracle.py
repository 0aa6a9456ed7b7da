"""Pins the CPU oracle: golden vectors from the compiled reference kernels,
closed forms and the reference test-suite's known-answer cases."""

import hashlib

import numpy as np
import pytest

from oracle import abi, twins
from quantanything_amd import synth
from tests.golden.cases import (
    CONV_CASES,
    GEMM_CASES,
    WRAP_CASE,
    conv_case_inputs,
    elementwise_cases,
    gemm_case_inputs,
    quantize_cases,
    requantize_cases,
)


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


# ------------------------------------------------------ generator drift --
def test_seeded_inputs_match_fixture_digests(golden):
    for i in range(len(CONV_CASES)):
        x, w, _ = conv_case_inputs(i)
        assert str(golden[f"conv{i}_in_sha"]) == sha(x) + sha(w)
    for i in range(len(GEMM_CASES)):
        a, b = gemm_case_inputs(i)
        assert str(golden[f"gemm{i}_in_sha"]) == sha(a) + sha(b)
    for i, rc in enumerate(requantize_cases()):
        assert str(golden[f"rq{i}_in_sha"]) == sha(rc["acc"])


# --------------------------------------------------------- golden vectors --
@pytest.mark.parametrize("wide", [False, True])
@pytest.mark.parametrize("i", range(len(CONV_CASES)))
def test_oracle_conv_matches_reference_build(oracle_lib, golden, i, wide):
    x, w, args = conv_case_inputs(i)
    got = oracle_lib.conv2d_int(x, w, *args, wide=wide)
    assert got.dtype == (np.int64 if wide else np.int32)
    np.testing.assert_array_equal(got, golden[f"conv{i}_y{int(wide)}"])


@pytest.mark.parametrize("i", range(len(CONV_CASES)))
def test_oracle_conv_closed_form(oracle_lib, i):
    """Direct sum == sliding-window einsum (the reference test's oracle)."""
    x, w, args = conv_case_inputs(i)
    ref = twins.np_conv(x, w, *args)
    np.testing.assert_array_equal(oracle_lib.conv2d_int(x, w, *args,
                                                        wide=True), ref)
    if i == WRAP_CASE:  # narrow path: activations wrap to int16 first
        ref = twins.np_conv(x.astype(np.int16), w, *args)
    np.testing.assert_array_equal(oracle_lib.conv2d_int(x, w, *args),
                                  ref.astype(np.int32))


@pytest.mark.parametrize("i", range(len(CONV_CASES)))
def test_oracle_conv_f32(oracle_lib, golden, i):
    x, w, args = conv_case_inputs(i)
    xf, wf = (x / 64.0).astype(np.float32), (w / 32.0).astype(np.float32)
    got = oracle_lib.conv2d_f32(xf, wf, *args)
    ref = golden[f"conv{i}_yf"]
    np.testing.assert_allclose(got, ref, rtol=1e-4,
                               atol=1e-4 * max(1.0, np.abs(ref).max()))


@pytest.mark.parametrize("i", range(len(GEMM_CASES)))
def test_oracle_gemm(oracle_lib, golden, i):
    a, b = gemm_case_inputs(i)
    exact = a.astype(np.int64) @ b.astype(np.int64)
    for wide in (False, True):
        got = oracle_lib.gemm_int(a, b, wide)
        np.testing.assert_array_equal(got, golden[f"gemm{i}_c{int(wide)}"])
        np.testing.assert_array_equal(got, exact)
    cf = oracle_lib.gemm_f32(a / 16.0, b / 8.0)
    np.testing.assert_allclose(cf, golden[f"gemm{i}_cf"], rtol=1e-5,
                               atol=1e-3)


def test_conv_shape_mismatch_raises():
    with pytest.raises(ValueError, match="conv shape mismatch"):
        abi.conv_geometry((1, 4, 5, 5), (3, 3, 3, 3), (1, 1), (0,) * 4,
                          (1, 1), 1)


@pytest.mark.parametrize("i", range(len(requantize_cases())))
def test_oracle_requantize(oracle_lib, golden, i):
    rc = requantize_cases()[i]
    args = (rc["acc"], rc["outer"], rc["C"], rc["inner"], rc["mult"],
            rc["shift"], rc["zp"], rc["qmin"], rc["qmax"])
    got = oracle_lib.requantize(*args, rc["pre"], rc["post"])
    assert got.dtype == np.int32
    np.testing.assert_array_equal(got, golden[f"rq{i}_out"])
    exact = twins.requantize_exact(*args, rc["pre"], rc["post"])
    np.testing.assert_array_equal(got, exact)


def test_requantize_half_up_kat(oracle_lib):
    """M0 = 2^30, shift 0 is x0.5 rounded half up (test_native.py:104-110)."""
    acc = np.arange(-60, 60, dtype=np.int32).reshape(2, 3, 20)
    out = oracle_lib.requantize(acc, 2, 3, 20, 1 << 30, 0, 1, -128, 127)
    np.testing.assert_array_equal(
        out, np.clip(np.floor(acc * 0.5 + 0.5) + 1, -128, 127))


@pytest.mark.parametrize("i", range(len(elementwise_cases())))
def test_oracle_elementwise(oracle_lib, golden, i):
    ec = elementwise_cases()[i]
    kind = ec["kind"]
    if kind == "rescale":
        got = oracle_lib.rescale(ec["x"], *ec["args"])
        exact = twins.rescale_exact(ec["x"], *ec["args"])
    elif kind == "add":
        got = oracle_lib.add(ec["a"], ec["b"], *ec["args"])
        exact = twins.add_exact(ec["a"], ec["b"], *ec["args"])
    elif kind == "mul":
        got = oracle_lib.mul(ec["a"], ec["b"], *ec["args"])
        exact = twins.mul_exact(ec["a"], ec["b"], *ec["args"])
    else:
        got = oracle_lib.lut(ec["x"], ec["table"], ec["offset"])
        idx = np.clip(ec["x"].astype(np.int64) - ec["offset"], 0,
                      len(ec["table"]) - 1)
        exact = ec["table"][idx]
    np.testing.assert_array_equal(got, golden[f"ew{i}_out"])
    np.testing.assert_array_equal(got, exact)


def test_add_exact_one_kat(oracle_lib):
    """Multipliers of exactly 1.0 add exactly (test_native.py:134-139)."""
    a = np.arange(6, dtype=np.int32).reshape(2, 3)
    b = np.array([10], dtype=np.int32)
    one = (1 << 30, -1)
    out = oracle_lib.add(a, b, 0, *one, 0, *one, 0, -128, 127)
    np.testing.assert_array_equal(out, a + b)


@pytest.mark.parametrize("i", range(len(quantize_cases())))
def test_oracle_quantize_dequantize(oracle_lib, golden, i):
    qc = quantize_cases()[i]
    q = oracle_lib.quantize_f32(qc["x"], *qc["args"])
    np.testing.assert_array_equal(q, golden[f"qz{i}_q"])
    scale, zp = qc["args"][0], qc["args"][1]
    dq = oracle_lib.dequantize_f32(q, scale, zp)
    np.testing.assert_array_equal(dq.view(np.int32),
                                  golden[f"qz{i}_dq"].view(np.int32))


def test_quantize_kats(oracle_lib):
    q = oracle_lib.quantize_f32(
        np.array([0.5, 1.5, 2.5, -0.5, -1.5], np.float32), 1.0, 0, -128, 127)
    np.testing.assert_array_equal(q, [0, 2, 2, 0, -2])
    q = oracle_lib.quantize_f32(np.array([1e6, -1e6], np.float32), 0.1, 0,
                                -128, 127)
    np.testing.assert_array_equal(q, [127, -128])


# ------------------------------------------------------------- workloads --
def test_oracle_gemm_workload(oracle_lib, golden_workloads):
    g = synth.gemm_workload()
    acc = oracle_lib.gemm_int(g["a"].astype(np.int32) - g["zp_in"],
                              g["w"].astype(np.int32))
    out = oracle_lib.requantize(acc, g["M"], g["N"], 1, g["mult"], g["shift"],
                                g["zp_out"], g["qmin"], g["qmax"], g["bias"])
    exp = golden_workloads["gemm"]
    assert sha(acc) == exp["acc_sha256"]
    assert sha(out) == exp["out_sha256"]


def test_oracle_conv_workload(oracle_lib, golden_workloads):
    c = synth.conv_workload()
    exp = golden_workloads["conv"]
    assert c["lut"].tolist() == exp["lut"]
    acc = oracle_lib.conv2d_int(c["x"].astype(np.int32) - c["zp_in"],
                                c["w"].astype(np.int32), (1, 1), (1,) * 4,
                                (1, 1), 1)
    assert sha(acc) == exp["acc_sha256"]
    n, co, oh, ow = acc.shape
    rq = oracle_lib.requantize(acc, n, co, oh * ow, c["mult"], c["shift"],
                               c["zp_out"], c["qmin"], c["qmax"], c["bias"])
    assert sha(rq) == exp["rq_sha256"]
    assert sha(oracle_lib.lut(rq, c["lut"], 0)) == exp["out_sha256"]
