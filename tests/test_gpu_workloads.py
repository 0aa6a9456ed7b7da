"""Full-size single-layer workloads through the fused device path, checked
against the digests of the compiled reference's separate conv / GEMM,
requantize and LUT calls (tests/golden/workloads.json)."""

import hashlib

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def test_fused_gemm_workload_matches_reference(hip, golden_workloads):
    from quantanything_amd.workloads import GemmWorkload

    w = GemmWorkload()
    w.launch()
    out = w.output().astype(np.int32)
    exp = golden_workloads["gemm"]
    assert out[:8].tolist() == exp["out_rows_0_8"]
    assert sha(out) == exp["out_sha256"]
    assert len(np.unique(out)) > 50  # not a saturated, degenerate output


def test_fused_conv_workload_matches_reference(hip, golden_workloads):
    from quantanything_amd.workloads import ConvWorkload

    w = ConvWorkload()
    w.launch()
    out = w.output().astype(np.int32)
    exp = golden_workloads["conv"]
    assert out[5, 7, 0].tolist() == exp["out_img5_ch7_row_0"]
    assert sha(out) == exp["out_sha256"]


def test_fused_workloads_repeat_identically(hip):
    """Re-launching on the same buffers gives the same bytes (no state)."""
    from quantanything_amd.workloads import ConvWorkload

    w = ConvWorkload(batch=4)
    w.launch()
    a = w.output()
    for _ in range(3):
        w.launch()
    np.testing.assert_array_equal(a, w.output())


@pytest.mark.parametrize("which", ["gemm", "conv"])
def test_workloads_match_reference_for_every_tile(hip, golden_workloads,
                                                  which):
    """Every tile code the executor may pick gives the reference's output."""
    from quantanything_amd.executor import DeviceExecutor
    from quantanything_amd.workloads import ConvWorkload, GemmWorkload

    w = GemmWorkload() if which == "gemm" else ConvWorkload()
    for code in DeviceExecutor.tile_candidates(w.d):
        w.d.tile = code
        w.y.fill_(0)
        w.launch()
        out = w.output().astype(np.int32)
        assert sha(out) == golden_workloads[which]["out_sha256"], hex(code)
