"""The built library loads on a machine without a GPU and exports every
function the public header declares (no compute calls here)."""

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "qa_hip.h"
LIB = ROOT / "quantanything_amd" / "libqa_hip.so"

REFERENCE_ABI = {
    "qa_num_threads", "qa_set_num_threads", "qa_has_openmp", "qa_gemm_f32",
    "qa_gemm_i16_i32", "qa_gemm_i32_i64", "qa_conv_f32",
    "qa_conv_i32_i16_i32", "qa_conv_i32_i32_i64", "qa_requantize_i32",
    "qa_requantize_i64", "qa_rescale", "qa_add", "qa_mul", "qa_lut",
    "qa_quantize_f32", "qa_dequantize_f32",
}


def declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(qa_\w+)\s*\(", text))


def test_header_declares_the_reference_abi():
    names = declared()
    assert REFERENCE_ABI <= names
    assert len(REFERENCE_ABI) == 17


def test_library_exports_every_declared_symbol():
    if not LIB.exists():
        pytest.skip("libqa_hip.so not built")
    lib = ctypes.CDLL(str(LIB))
    missing = [n for n in sorted(declared()) if not hasattr(lib, n)]
    assert not missing, missing


def test_native_module_binds_without_gpu():
    if not LIB.exists():
        pytest.skip("libqa_hip.so not built")
    from quantanything_amd import native

    assert native.available(), native.load_error()
    assert set(native.SYMBOLS) == declared()
    assert native.backend() == "hip-gfx950"
