"""End-to-end integer inference on the GPU (device-resident executor) vs the
oracle pipeline on the same graph, q.json and input. Integer outputs must be
bit-exact; the float Softmax fallback may differ by one quantization step
(float64 exp / summation order)."""

import numpy as np
import pytest

from oracle.pipeline import OraclePipeline
from quantanything_amd import graph as G
from quantanything_amd.container import QuantContainer
from quantanything_amd.synth import Stream

pytestmark = pytest.mark.gpu


def _images(seed, n, size, lo=0.0, hi=1.0):
    return Stream(seed).uniform((n, 3, size, size), lo, hi).astype(np.float32)


def _calibrated(g, quant_type, per_channel, batches):
    c = QuantContainer(g, quant_type, per_channel)
    c.calibrate(batches)
    return c


def _qjson(c, tmp_path):
    path = tmp_path / "q.json"
    c.save(path)
    return path


@pytest.mark.parametrize("per_channel", [True, False])
@pytest.mark.parametrize("quant_type", ["int8", "uint8", "int16"])
def test_mini_yolo_integer_bit_exact(hip, tmp_path, quant_type, per_channel):
    g = G.mini_yolo(seed=0, softmax=False)
    calib = [_images(1 + i, 4, 32) for i in range(3)]
    c = _calibrated(g, quant_type, per_channel, calib)
    x = calib[0]
    got = c.integer_outputs(x)
    ints, _ = OraclePipeline(g, _qjson(c, tmp_path)).run(x)
    for name in g.outputs:
        np.testing.assert_array_equal(got[name], ints[name])


@pytest.mark.parametrize("quant_type", ["int8", "uint8", "int16"])
def test_mini_yolo_with_softmax_within_one_step(hip, tmp_path, quant_type):
    g = G.mini_yolo(seed=0)
    calib = [_images(1 + i, 4, 32) for i in range(3)]
    c = _calibrated(g, quant_type, True, calib)
    got = c.integer_outputs(calib[1])[g.outputs[0]]
    ints, floats = OraclePipeline(g, _qjson(c, tmp_path)).run(calib[1])
    assert np.abs(got.astype(np.int64) - ints[g.outputs[0]]).max() <= 1
    out = c.run_graph(calib[1], "integer")
    step = c.qparams[g.outputs[0]].scale
    assert np.abs(out - floats[0]).max() <= step * 1.0001
    assert out.dtype == np.float32 and out.shape == (4, 10)


def test_yolov8n_cls_int8_bit_exact(hip, tmp_path):
    g = G.yolov8n_cls(seed=3, softmax=False)
    calib = [Stream(40 + i).normal((2, 3, 224, 224)).astype(np.float32)
             for i in range(2)]
    c = _calibrated(g, "int8", True, calib)
    x = Stream(50).normal((2, 3, 224, 224)).astype(np.float32)
    got = c.integer_outputs(x)[g.outputs[0]]
    ints, _ = OraclePipeline(g, _qjson(c, tmp_path)).run(x)
    np.testing.assert_array_equal(got, ints[g.outputs[0]])


@pytest.mark.parametrize("model,quant_type", [("yolov8n_cls", "int8"),
                                              ("mini_yolo", "uint8")])
def test_every_conv_tile_is_bit_exact(hip, tmp_path, model, quant_type):
    """Every int8 MFMA conv forced through each tile code it accepts
    (channel-block width, K-split, weights in LDS): every tensor the device
    pass keeps equals the oracle's."""
    if model == "yolov8n_cls":
        g = G.yolov8n_cls(seed=3, softmax=False)
        x = Stream(51).normal((2, 3, 224, 224)).astype(np.float32)
        calib = [Stream(40).normal((2, 3, 224, 224)).astype(np.float32)]
    else:
        g = G.mini_yolo(seed=0, softmax=False)
        calib = [_images(1 + i, 4, 32) for i in range(3)]
        x = _images(9, 3, 32)
    c = _calibrated(g, quant_type, True, calib)
    oracle = OraclePipeline(g, _qjson(c, tmp_path))
    oracle.run(x, keep=True)
    ex = c.executor({"images": x.shape})
    assert any(n.startswith("qconv:") for n, _ in ex.launches), \
        "input quantization not fused into the stem"
    assert any(n.startswith("convpool:") for n, _ in ex.launches) and \
        not any(n.startswith("gap:") for n, _ in ex.launches), \
        "pool not fused into the last convolution"
    descs = [t[1] for t in ex.tunables]
    # fused convolutions (a pair, a chain, a pair with its block's 1x1
    # tail: names joined by "+") are one tunable launch
    fused = sum(n.count("+") for n, _ in ex.launches
                if n.startswith(("pair:", "chain:", "pairtail:")))
    # two pointwise convolutions with the pool: no tile choice at all
    fused += sum(n.count("+") + 1 for n, _ in ex.launches
                 if n.startswith("convpool:") and "+" in n)
    assert len(descs) == len(ex.mfma_descs) - fused
    cands = [t[2] for t in ex.tunables]
    for r in range(max(len(cc) for cc in cands)):
        for d, cc in zip(descs, cands):
            d.tile = cc[r % len(cc)]
        ex.run({"images": x})
        checked = 0
        for name, t in ex.tensors.items():
            if name in oracle.env:
                got = t.to_host()
                np.testing.assert_array_equal(
                    got, oracle.env[name].reshape(got.shape),
                    err_msg=f"{name}, tiles {[hex(d.tile) for d in descs]}")
                checked += 1
        assert checked > len(descs) // 2


def _stem_graph(cin, cout, k, stride, pad, dil, size):
    b = G.GraphBuilder(7)
    y = b.silu(b.conv("images", cin, cout, k, stride, pad=pad, dilation=dil))
    y = b.op("Flatten", [b.op("GlobalAveragePool", [y])], axis=1)
    return b.build("images", [None, cin, size, size], y)


@pytest.mark.parametrize("quant_type", ["int8", "uint8"])
@pytest.mark.parametrize("cin,cout,k,stride,pad,dil,size", [
    (3, 16, 3, 2, 1, 1, 32),   # the image stem, float4 rows
    (1, 8, 3, 1, 1, 1, 30),    # one channel, rows not a multiple of 4
    (4, 20, 4, 2, 2, 1, 36),   # 4 channels, 4x4 taps, a partial channel block
    (2, 16, 2, 1, 0, 2, 29),   # dilation 2, no padding, odd width
    (3, 32, 1, 1, 0, 1, 16),   # 1x1
])
def test_input_quantization_fused_into_stem(hip, tmp_path, quant_type, cin,
                                            cout, k, stride, pad, dil, size):
    """qa_d_quantize_conv (float input quantized inside the layout-1 conv)
    gives the oracle's conv output for every band height it accepts."""
    g = _stem_graph(cin, cout, k, stride, pad, dil, size)
    calib = [Stream(20 + i).uniform((3, cin, size, size), -1.0, 1.0)
             .astype(np.float32) for i in range(2)]
    c = _calibrated(g, quant_type, True, calib)
    # beyond the calibrated range
    x = Stream(30).uniform((3, cin, size, size), -1.2, 1.2).astype(np.float32)
    oracle = OraclePipeline(g, _qjson(c, tmp_path))
    oracle.run(x, keep=True)
    ex = c.executor({"images": x.shape})
    fused = [t for t in ex.tunables if t[0].startswith("qconv:")]
    assert len(fused) == 1 and "images" not in ex.tensors
    _, d, codes, _ = fused[0]
    for code in codes:
        d.tile = code
        ex.run({"images": x})
        for name, t in ex.tensors.items():
            if name in oracle.env:
                got = t.to_host()
                np.testing.assert_array_equal(
                    got, oracle.env[name].reshape(got.shape),
                    err_msg=f"{name}, band code {code:#x}")


@pytest.mark.parametrize("quant_type", ["int8", "uint8"])
def test_stem_quantization_edge_values(hip, tmp_path, quant_type):
    """The fused stem's float32 quantization (exact unless a value is near a
    rounding tie, where the double form decides) on the values that test
    it: exact ties (k + 1/2) * scale, one float step either side of them,
    the clip bounds and one step past them, magnitudes beyond 2^23 steps,
    +-1e30, +-inf and -0.0; every integer tensor equals the oracle's."""
    g = _stem_graph(3, 16, 3, 2, 1, 1, 32)
    calib = [Stream(20).uniform((3, 3, 32, 32), -1.0, 1.0).astype(np.float32)]
    c = _calibrated(g, quant_type, True, calib)
    qp = c.qparams["images"]
    scale, zp = float(qp.scale), int(qp.zp)
    x = Stream(31).uniform((3, 3, 32, 32), -1.2, 1.2).astype(np.float32)
    flat = x.reshape(-1)
    ks = np.arange(-140, 140)
    ties = ((ks + 0.5) * scale).astype(np.float32)
    special = np.concatenate([
        ties,
        np.nextafter(ties, np.float32(np.inf)),
        np.nextafter(ties, np.float32(-np.inf)),
        np.float32([(qp.qmin - zp) * scale, (qp.qmax - zp) * scale,
                    (qp.qmin - zp - 1) * scale, (qp.qmax - zp + 1) * scale,
                    2.0 ** 23 * scale, -(2.0 ** 23) * scale,
                    2.0 ** 24 * scale, -(2.0 ** 24) * scale,
                    1e30, -1e30, np.inf, -np.inf, -0.0, 0.0,
                    1e-40, -1e-40])])
    idx = Stream(32).integers(0, flat.size - 1, (special.size,))
    flat[idx] = special
    oracle = OraclePipeline(g, _qjson(c, tmp_path))
    oracle.run(x, keep=True)
    ex = c.executor({"images": x.shape})
    fused = [t for t in ex.tunables if t[0].startswith("qconv:")]
    assert len(fused) == 1
    _, d, codes, _ = fused[0]
    for code in codes:  # every band height and bands-a-work-group form
        d.tile = code
        ex.run({"images": x})
        checked = 0
        for name, t in ex.tensors.items():
            if name in oracle.env:
                got = t.to_host()
                np.testing.assert_array_equal(
                    got, oracle.env[name].reshape(got.shape),
                    err_msg=f"{name}, band code {code:#x}")
                checked += 1
        assert checked >= 2


def _conv_graph(cin, cout, k, stride, pad, dil, groups, size):
    b = G.GraphBuilder(11)
    y = b.silu(b.conv("images", cin, cout, k, stride, pad=pad, groups=groups,
                      dilation=dil))
    y = b.op("Flatten", [b.op("GlobalAveragePool", [y])], axis=1)
    return b.build("images", [None, cin, size, size], y)


@pytest.mark.parametrize("wtype", ["int16", "int32"])
@pytest.mark.parametrize("cin,cout,k,stride,pad,dil,groups,size", [
    (3, 16, 3, 2, 1, 1, 1, 32),    # the stem: 3 of 4 stored channels
    (16, 24, 3, 1, 1, 1, 1, 17),   # a partial 16-channel block
    (20, 40, 1, 1, 0, 1, 1, 12),   # 20 channels: one per lane and chunk
    (48, 32, 3, 2, 2, 2, 1, 19),   # dilation 2, stride 2, 4 per lane
    (64, 80, 3, 1, 1, 1, 1, 14),   # 8 channels per lane and chunk
    (32, 64, 3, 1, 1, 1, 2, 10),   # two groups
    (24, 24, 3, 1, 1, 1, 24, 9),   # depthwise
])
def test_int16_conv_on_fp64_matrix_cores(hip, tmp_path, monkeypatch, wtype,
                                         cin, cout, k, stride, pad, dil,
                                         groups, size):
    """16-bit convolutions run on the FP64 MFMA path (w_code 8, weights
    packed as int16 or int32) or, for int16 weights and a multiple of 16
    channels per group (or at most 4 input channels, the stem), by default
    in the byte-split form on the int8 matrix cores (tile codes 0x11000 |
    wm | tm << 4); under every tile code
    every tensor equals the oracle's int64-accumulated one (inputs past the
    calibrated range saturate to the int16 extremes)."""
    from quantanything_amd import executor
    from quantanything_amd.executor import ConvDesc

    monkeypatch.setattr(executor, "F64_WEIGHT_TYPES", (np.dtype(wtype).type,))

    g = _conv_graph(cin, cout, k, stride, pad, dil, groups, size)
    calib = [Stream(60 + i).uniform((3, cin, size, size), -1.0, 1.0)
             .astype(np.float32) for i in range(2)]
    c = _calibrated(g, "int16", True, calib)
    x = Stream(70).uniform((3, cin, size, size), -1.3, 1.3).astype(np.float32)
    oracle = OraclePipeline(g, _qjson(c, tmp_path))
    oracle.run(x, keep=True)
    ex = c.executor({"images": x.shape})
    assert [(d.w_code, d.w_layout) for d in ex.keep
            if isinstance(d, ConvDesc)] == [(8, np.dtype(wtype).itemsize)]
    [(_, d, codes, _)] = ex.tunables
    assert len(codes) >= 4
    split = wtype == "int16" and ((cin // groups) % 16 == 0 or
                                  (cin <= 4 and groups == 1))
    assert bool(d.wsplit) == split
    assert any(c & 0x1000 for c in codes) == split
    for code in codes:
        d.tile = code
        ex.run({"images": x})
        checked = 0
        for name, t in ex.tensors.items():
            if name in oracle.env:
                got = t.to_host()
                np.testing.assert_array_equal(
                    got, oracle.env[name].reshape(got.shape),
                    err_msg=f"{name}, tile {code:#x}")
                checked += 1
        assert checked >= 2


def test_yolov8n_cls_int16_bit_exact(hip, tmp_path):
    """The 16-bit YOLOv8n-cls pass (every conv and the head GEMM on the FP64
    matrix cores) equals the oracle's int64 pass."""
    from quantanything_amd.executor import ConvDesc

    g = G.yolov8n_cls(seed=3, softmax=False)
    calib = [Stream(40 + i).normal((2, 3, 224, 224)).astype(np.float32)
             for i in range(2)]
    c = _calibrated(g, "int16", True, calib)
    x = Stream(52).normal((2, 3, 224, 224)).astype(np.float32)
    ex = c.executor({"images": x.shape})
    codes = [d.w_code for d in ex.keep if isinstance(d, ConvDesc)]
    assert len(codes) > 20 and set(codes) == {8}
    got = c.integer_outputs(x)[g.outputs[0]]
    oracle = OraclePipeline(g, _qjson(c, tmp_path))
    ints, _ = oracle.run(x, keep=True)
    np.testing.assert_array_equal(got, ints[g.outputs[0]])
    # every layer through each of its tiles
    assert len(ex.tunables) == len(codes)
    for r in range(max(len(t[2]) for t in ex.tunables)):
        for _, d, cc, _ in ex.tunables:
            d.tile = cc[r % len(cc)]
        ex.run({"images": x})
        for name, t in ex.tensors.items():
            if name in oracle.env:
                got = t.to_host()
                np.testing.assert_array_equal(
                    got, oracle.env[name].reshape(got.shape),
                    err_msg=f"{name}, pass {r}")


@pytest.mark.parametrize("quant_type", ["int8", "uint8"])
@pytest.mark.parametrize("cin,cout,k,stride,pad,size", [
    (3, 32, 16, 16, 0, 64),   # a ViT patch embedding: 4 groups per row
    (3, 24, 7, 2, 3, 30),     # 7x7 stem: 2 groups per row, 3 columns real
    (4, 16, 5, 1, 2, 19),     # 5x5, padding on both sides
    (1, 16, 8, 4, 0, 36),     # one channel, 8 columns
])
def test_wide_kernel_rows_layout(hip, tmp_path, quant_type, cin, cout, k,
                                 stride, pad, size):
    """Convolutions of <= 4 channels with kernels wider than 4 columns use
    the row layout (ceil(KW/4) 16-byte groups per kernel row) and equal the
    oracle for every tile code. A patch embedding of the graph input
    (stride = kernel, no padding) instead reads the input quantized into
    its im2col rows, as a 1x1 convolution of KH*KW*4 channels."""
    b = G.GraphBuilder(13)
    y = b.conv("images", cin, cout, k, stride, pad=pad,
               w_scale=np.sqrt(1.0 / (cin * k * k)))
    y = b.op("Relu", [y])
    g = b.build("images", [None, cin, size, size], y)
    calib = [Stream(70 + i).normal((2, cin, size, size)).astype(np.float32)
             for i in range(2)]
    c = _calibrated(g, quant_type, True, calib)
    x = Stream(80).normal((2, cin, size, size)).astype(np.float32)
    oracle = OraclePipeline(g, _qjson(c, tmp_path))
    oracle.run(x, keep=True)
    ex = c.executor({"images": x.shape})
    convs = [t for t in ex.tunables if t[0].startswith("conv:")]
    patch = stride == k and pad == 0 and k % 4 == 0 and size % k == 0
    assert len(convs) == 1 and convs[0][1].w_layout == (0 if patch else 1)
    assert ("patches:images" in dict(ex.launches)) == patch
    _, d, codes, _ = convs[0]
    for code in codes:
        d.tile = code
        ex.run({"images": x})
        for name, t in ex.tensors.items():
            if name in oracle.env:
                got = t.to_host()
                np.testing.assert_array_equal(
                    got, oracle.env[name].reshape(got.shape),
                    err_msg=f"{name}, tile {code:#x}")


def test_tuned_tiles_keep_results(hip):
    g = G.mini_yolo(seed=0)
    calib = [_images(1 + i, 4, 32) for i in range(3)]
    c = _calibrated(g, "int8", True, calib)
    ex = c.executor({"images": (4, 3, 32, 32)})
    before = ex.run({"images": calib[0]})
    report = ex.tune(launches=2, reps=1)
    assert set(report) == {t[0] for t in ex.tunables}
    for code, best, lib in report.values():
        assert best <= lib
        assert code == 0 or code & 0x10000
    after = ex.run({"images": calib[0]}, use_graph=True)
    for k in before:
        np.testing.assert_array_equal(after[k], before[k])


def test_saved_qparams_reload_to_identical_results(hip, tmp_path):
    g = G.mini_yolo(seed=0)
    calib = [_images(1 + i, 4, 32) for i in range(3)]
    c = _calibrated(g, "int16", True, calib)
    path = _qjson(c, tmp_path)
    loaded = QuantContainer.load(g, path)
    assert loaded.quant_type == "int16" and loaded.calibrated
    np.testing.assert_array_equal(c.run_graph(calib[2], "integer"),
                                  loaded.run_graph(calib[2], "integer"))


def test_batch_size_can_change_after_calibration(hip):
    g = G.mini_yolo(seed=0)
    calib = [_images(1 + i, 4, 32) for i in range(3)]
    c = _calibrated(g, "int8", True, calib)
    one = c.run_graph(calib[0][:1], "integer")
    many = c.run_graph(np.concatenate(calib), "integer")
    np.testing.assert_array_equal(one, many[:1])


def test_batches_in_flight_match_their_own_passes(hip):
    """Two executors (own inputs and buffers) as parallel branches of one
    graph: every replay gives each executor its own eager result, with eager
    work and synchronisation between the replays, and the second batch
    (the first one's images rolled) the first one's outputs rolled."""
    import torch

    from quantanything_amd.executor import (DeviceExecutor, InFlight,
                                            tune_in_flight)

    g = G.yolov8n_cls(seed=3)
    calib = [Stream(40 + i).normal((2, 3, 224, 224)).astype(np.float32)
             for i in range(2)]
    c = _calibrated(g, "int8", True, calib)
    x = Stream(51).normal((2, 3, 224, 224)).astype(np.float32)
    exs = [DeviceExecutor(c, {"images": x.shape}) for _ in range(2)]
    eager = [exs[0].run({"images": x}),
             exs[1].run({"images": np.roll(x, 1, 0)})]
    for k in eager[0]:
        np.testing.assert_array_equal(eager[1][k], np.roll(eager[0][k], 1, 0))
    fl = InFlight(exs)
    for _ in range(3):
        fl.replay()
        torch.cuda.synchronize()
        for ex, want in zip(exs, eager):
            for k, v in ex.outputs_f32.items():
                np.testing.assert_array_equal(v.cpu().numpy(), want[k])
        torch.zeros(1024, device="cuda").sum().item()
    # tile choice in flight: every launch gets one of its own codes, and the
    # results stay the same
    keep = exs[0].tunables[0][0]
    chosen = tune_in_flight(exs, sweeps=1, reps=2, rounds=1, keep=(keep,))
    for name, d, codes, _ in exs[0].tunables:
        assert chosen[name] in codes and (name != keep or chosen[name] == 0)
    fl = InFlight(exs)
    fl.replay()
    torch.cuda.synchronize()
    for ex, want in zip(exs, eager):
        for k, v in ex.outputs_f32.items():
            np.testing.assert_array_equal(v.cpu().numpy(), want[k])


def test_graph_replay_matches_eager(hip):
    """A captured HIP graph replayed several times (with eager work and
    synchronisation in between) gives the eager result every time."""
    import torch

    g = G.mini_yolo(seed=0)
    calib = [_images(1 + i, 4, 32) for i in range(3)]
    c = _calibrated(g, "int8", True, calib)
    ex = c.executor({"images": (4, 3, 32, 32)})
    eager = ex.run({"images": calib[0]})
    for _ in range(3):
        replay = ex.run({"images": calib[0]}, use_graph=True)
        for k in eager:
            np.testing.assert_array_equal(replay[k], eager[k])
        torch.zeros(1024, device="cuda").sum().item()
    other = ex.run({"images": calib[1]}, use_graph=True)
    eager_other = ex.run({"images": calib[1]})
    for k in other:
        np.testing.assert_array_equal(other[k], eager_other[k])


def test_uncalibrated_container_refuses(hip):
    with pytest.raises(ValueError, match="not calibrated"):
        QuantContainer(G.mini_yolo()).run_graph(_images(0, 1, 32), "integer")


@pytest.mark.parametrize("cin,cout,k,stride,pad,dil,size,residual", [
    (64, 64, 3, 1, 1, 1, 23, False),   # 4 channel tiles, ragged rows
    (32, 40, 3, 2, 1, 1, 31, True),    # partial channel quad, stride 2
    (48, 16, 3, 1, 2, 2, 17, False),   # 3 channel blocks a tap, dilation 2
    (16, 96, 1, 1, 0, 1, 9, True),     # 1x1, two channel blocks of 64
    (128, 24, 3, 1, 0, 1, 12, False),  # no padding, 18 K-steps
])
def test_weights_in_registers_kernel(hip, tmp_path, cin, cout, k, stride, pad,
                                     dil, size, residual):
    """The convolution kernel that holds its weights in VGPRs (tile codes
    0x11000 | wm) equals the oracle on ragged bands, partial channel
    blocks, strides, dilation and a fused residual Add, for every tile code
    of the layer."""
    b = G.GraphBuilder(17)
    r = None
    if residual:  # built first, so that the Add fuses into the k x k conv
        r = b.conv("images", cin, cout, 1, stride, pad=0,
                   w_scale=np.sqrt(1.0 / cin))
    y = b.silu(b.conv("images", cin, cout, k, stride, pad=pad, dilation=dil,
                      w_scale=np.sqrt(1.0 / (cin * k * k))))
    if residual:
        y = b.op("Add", [r, y])
    g = b.build("images", [None, cin, size, size], y)
    calib = [Stream(110 + i).normal((3, cin, size, size)).astype(np.float32)
             for i in range(2)]
    c = _calibrated(g, "int8", True, calib)
    x = Stream(120).normal((3, cin, size, size)).astype(np.float32)
    oracle = OraclePipeline(g, _qjson(c, tmp_path))
    oracle.run(x, keep=True)
    ex = c.executor({"images": x.shape})
    main = [t for t in ex.tunables
            if (t[1].res is not None) == residual and t[1].KH == k]
    assert len(main) == 1
    assert any(code & 0x11000 == 0x11000 for code in main[0][2])
    codes = main[0][2]
    for code in codes:
        for _, d, _, _ in ex.tunables:
            d.tile = code if d is main[0][1] else 0
        ex.run({"images": x})
        for name, t in ex.tensors.items():
            if name in oracle.env:
                got = t.to_host()
                np.testing.assert_array_equal(
                    got, oracle.env[name].reshape(got.shape),
                    err_msg=f"{name}, tile {code:#x}")


@pytest.mark.parametrize("c,size,batch,residual", [
    (16, 23, 3, True),    # ragged bands
    (32, 14, 2, True),
    (64, 9, 3, True),
    (32, 11, 2, False),
    (64, 7, 1, False),
    (128, 7, 2, True),    # channel-split form (weights from L2)
    (128, 10, 1, False),
])
def test_fused_conv_pair(hip, tmp_path, c, size, batch, residual):
    """Two chained 3x3 convolutions (a C2f bottleneck: conv, SiLU, conv,
    SiLU, Add of the input; 16 to 128 channels) run as one launch with the
    intermediate in LDS
    and equal the oracle bit for bit; the intermediate tensor is never
    materialized."""
    b = G.GraphBuilder(23)
    w = np.sqrt(1.0 / (9 * c))
    t = b.silu(b.conv("images", c, c, 3, 1, w_scale=w, b_scale=0.05))
    t = b.silu(b.conv(t, c, c, 3, 1, w_scale=w, b_scale=0.05))
    y = b.op("Add", ["images", t]) if residual else t
    g = b.build("images", [None, c, size, size], y)
    calib = [Stream(130 + i).normal((2, c, size, size)).astype(np.float32)
             for i in range(2)]
    cq = _calibrated(g, "int8", True, calib)
    x = Stream(140).normal((batch, c, size, size)).astype(np.float32)
    oracle = OraclePipeline(g, _qjson(cq, tmp_path))
    oracle.run(x, keep=True)
    ex = cq.executor({"images": x.shape})
    assert [n for n, _ in ex.launches if n.startswith("pair:")], \
        [n for n, _ in ex.launches]
    ex.run({"images": x})
    checked = 0
    for name, tt in ex.tensors.items():
        if name in oracle.env:
            got = tt.to_host()
            np.testing.assert_array_equal(
                got, oracle.env[name].reshape(got.shape), err_msg=name)
            checked += 1
    assert checked >= 2


@pytest.mark.parametrize("cin,c,k,stride,size,batch", [
    (16, 32, 3, 2, 29, 2),   # a stride-2 conv feeding a C2f's 1x1
    (32, 64, 3, 2, 15, 3),
    (16, 16, 3, 1, 20, 2),
    (64, 64, 1, 1, 9, 3),    # 1x1 then 1x1
    (64, 128, 3, 2, 15, 2),  # the narrow chain: im2col rows, 128 channels
    (128, 256, 3, 2, 14, 2),  # 18 K-steps, 256 channels
    (128, 128, 1, 1, 7, 3),  # the narrow chain over GEMM rows
])
def test_fused_conv_chain(hip, tmp_path, cin, c, k, stride, size, batch):
    """A convolution whose output only feeds a 1x1 convolution of the same
    width runs with it as one launch (the intermediate kept in LDS) and the
    result equals the oracle bit for bit for every tile code of the fused
    launch (band heights of the weights-in-registers chain, row tiles of
    the narrow chain); the intermediate tensor is never materialized."""
    b = G.GraphBuilder(29)
    t = b.silu(b.conv("images", cin, c, k, stride,
                      w_scale=np.sqrt(1.0 / (k * k * cin)), b_scale=0.05))
    y = b.silu(b.conv(t, c, c, 1, 1, pad=0, w_scale=np.sqrt(1.0 / c),
                      b_scale=0.05))
    if c >= 32:  # a C2f-style Split / Concat: the 1x1 output gets a copy
        h1, h2 = b.op("Split", [y, b.const(np.array([c // 2, c // 2],
                                                     np.int64))],
                      n_out=2, axis=1)
        y = b.op("Concat", [h1, b.silu(b.conv(h2, c // 2, c // 2, 3, 1,
                                               w_scale=0.1)), h2], axis=1)
    g = b.build("images", [None, cin, size, size], y)
    calib = [Stream(150 + i).normal((2, cin, size, size)).astype(np.float32)
             for i in range(2)]
    cq = _calibrated(g, "int8", True, calib)
    x = Stream(160).normal((batch, cin, size, size)).astype(np.float32)
    oracle = OraclePipeline(g, _qjson(cq, tmp_path))
    oracle.run(x, keep=True)
    ex = cq.executor({"images": x.shape})
    assert [n for n, _ in ex.launches if n.startswith("chain:")], \
        [n for n, _ in ex.launches]
    chain = [t for t in ex.tunables if t[0].startswith("chain:")]
    assert len(chain) == 1
    d2, codes = chain[0][1], chain[0][2]
    if cin % 64 == 0:
        assert 0x12000 in codes
    for code in codes:
        d2.tile = code
        ex.run({"images": x})
        checked = 0
        for name, tt in ex.tensors.items():
            if name in oracle.env:
                got = tt.to_host()
                np.testing.assert_array_equal(
                    got, oracle.env[name].reshape(got.shape),
                    err_msg=f"{name}, tile {code:#x}")
                checked += 1
        assert checked >= 2


@pytest.mark.parametrize("quant_type", ["int8", "uint8"])
@pytest.mark.parametrize("cin,cout,size,batch", [
    (64, 16, 9, 3),     # one channel block: 4 row tiles a work-group
    (128, 32, 7, 2),    # two channel blocks, 98 rows (a partial work-group)
    (576, 64, 5, 3),    # 9 K-steps, 75 rows
    (192, 64, 16, 2),   # 3 K-steps, 512 rows
    (256, 256, 7, 4),   # 4 channel blocks of 64
    (128, 200, 6, 3),   # a partial last channel block (200 = 3 x 64 + 8)
    (1280, 1000, 1, 64),  # a classifier head: 20 K-steps, one pixel an image
    (128, 128, 9, 2),   # with a rescaled copy (a C2f's Split / Concat)
])
def test_narrow_gemm_kernel(hip, tmp_path, quant_type, cin, cout, size,
                            batch):
    """The narrow-GEMM kernel (tile codes 0x12000 / 0x12001: activations
    staged in LDS by coalesced direct loads, swizzled; weights from their
    fragment-order copy, or staged like the activations without one) equals
    the oracle for 16, 32 and 64 output channels, blocks of 64 channels
    (a partial last one), K up to 1280, ragged row counts and weights with
    an offset (uint8: the row sums)."""
    b = G.GraphBuilder(23)
    y = b.silu(b.conv("images", cin, cout, 1, 1, pad=0,
                      w_scale=np.sqrt(1.0 / cin), b_scale=0.05))
    if cin == cout == 128:  # a C2f-style Split / Concat: the copy y2
        h1, h2 = b.op("Split", [y, b.const(np.array([64, 64], np.int64))],
                      n_out=2, axis=1)
        # both halves first, as a C2f concatenates them, and a wider range
        # in the Concat, so that they are copied rescaled by the 1x1 conv
        y = b.op("Concat", [h1, h2, b.conv(h2, 64, 64, 3, 1, w_scale=1.0)],
                 axis=1)
    g = b.build("images", [None, cin, size, size], y)
    calib = [Stream(130 + i).normal((batch, cin, size, size))
             .astype(np.float32) for i in range(2)]
    c = _calibrated(g, quant_type, True, calib)
    x = Stream(140).normal((batch, cin, size, size)).astype(np.float32)
    oracle = OraclePipeline(g, _qjson(c, tmp_path))
    oracle.run(x, keep=True)
    ex = c.executor({"images": x.shape})
    first = [t for t in ex.tunables if t[1].KH == 1]
    assert len(first) == 1
    d, codes = first[0][1], first[0][2]
    assert 0x12000 in codes and d.w_frag
    assert bool(d.y2) == (cin == cout == 128)
    frag = d.w_frag
    # past 9 K-steps only the fragment-order weights are taken
    forms = (frag, None) if cin <= 576 else (frag,)
    for code, wf in [(c_, f) for c_ in codes if c_ & 0x12000 == 0x12000
                     for f in forms]:
        d.tile, d.w_frag = code, wf
        ex.run({"images": x})
        checked = 0
        for name, t in ex.tensors.items():
            if name in oracle.env:
                got = t.to_host()
                np.testing.assert_array_equal(
                    got, oracle.env[name].reshape(got.shape),
                    err_msg=f"{name}, tile {code:#x}")
                checked += 1
        assert checked >= 1


@pytest.mark.parametrize("quant_type", ["int8", "uint8"])
@pytest.mark.parametrize("cin,cout,k,stride,pad,dil,size,batch", [
    (64, 64, 3, 1, 1, 1, 13, 2),     # the 3x3 64 -> 64 layer form
    (128, 256, 3, 2, 1, 1, 14, 2),   # stride 2, 18 K-steps
    (64, 128, 3, 2, 1, 1, 15, 3),    # stride 2, odd size
    (64, 32, 3, 1, 2, 2, 11, 2),     # dilation 2
    (64, 16, 2, 2, 0, 1, 9, 2),      # 2x2, no padding
])
def test_narrow_kernel_on_convolutions(hip, tmp_path, quant_type, cin, cout,
                                       k, stride, pad, dil, size, batch):
    """The narrow-GEMM kernel over a convolution's im2col rows (taps
    outside the image get the pad value in LDS) equals the oracle for every
    row-tile code, strides, dilation and weights with an offset."""
    b = G.GraphBuilder(27)
    y = b.silu(b.conv("images", cin, cout, k, stride, pad=pad, dilation=dil,
                      w_scale=np.sqrt(1.0 / (cin * k * k)), b_scale=0.05))
    g = b.build("images", [None, cin, size, size], y)
    calib = [Stream(150 + i).normal((batch, cin, size, size))
             .astype(np.float32) for i in range(2)]
    c = _calibrated(g, quant_type, True, calib)
    x = Stream(160).normal((batch, cin, size, size)).astype(np.float32)
    oracle = OraclePipeline(g, _qjson(c, tmp_path))
    oracle.run(x, keep=True)
    ex = c.executor({"images": x.shape})
    assert len(ex.tunables) == 1
    d, codes = ex.tunables[0][1], ex.tunables[0][2]
    narrow = [c_ for c_ in codes if c_ & 0x12000 == 0x12000]
    assert narrow and d.w_frag
    for code in narrow:
        d.tile = code
        ex.run({"images": x})
        checked = 0
        for name, t in ex.tensors.items():
            if name in oracle.env:
                got = t.to_host()
                np.testing.assert_array_equal(
                    got, oracle.env[name].reshape(got.shape),
                    err_msg=f"{name}, tile {code:#x}")
                checked += 1
        assert checked >= 1
