"""Model files on the device: a graph written to ONNX and read back
calibrates to the same q.json and the same integer outputs, and its integer
pass equals the oracle pipeline's on the loaded graph; a PyTorch-style ViT
export (decomposed LayerNorms, explicit attention scale, Shape-chain class
token) loads through the reference's passes to the operator multiset of the
post-pass builder and runs bit-exact against the oracle on its integer
layers, within one step on its float fallbacks; the QDQ export
of a calibrated container carries every q.json parameter and, run with the
ONNX float semantics of QuantizeLinear / DequantizeLinear, reproduces the
container's fake quantization (quant_container.py:150-160)."""

import json

import numpy as np
import pytest

from oracle.pipeline import OraclePipeline
from quantanything_amd import float_ops
from quantanything_amd import graph as G
from quantanything_amd import onnx_io
from quantanything_amd.container import QuantContainer
from quantanything_amd.synth import Stream
from tests.test_gpu_vit import _check_against_oracle
from tests.test_onnx_io import CFG, PB

pytestmark = pytest.mark.gpu

MODELS = {
    "mini_yolo": lambda: (G.mini_yolo(seed=0), (4, 3, 32, 32)),
    "mini_sppf": lambda: (G.mini_sppf(seed=4), (3, 3, 33, 31)),
}


def _calib(shape, seed=70):
    return [Stream(seed + i).normal(shape, 1.0).astype(np.float32)
            for i in range(2)]


@pytest.mark.parametrize("quant_type", ["int8", "uint8", "int16"])
@pytest.mark.parametrize("model", sorted(MODELS))
def test_written_model_runs_identically(hip, tmp_path, model, quant_type):
    g, shape = MODELS[model]()
    h = onnx_io.load_onnx(onnx_io.save_onnx(g, tmp_path / "m.onnx"))
    calib = _calib(shape)
    a = QuantContainer(g, quant_type, True)
    b = QuantContainer(h, quant_type, True)
    a.calibrate(calib)
    b.calibrate(calib)
    a.save(tmp_path / "a.json")
    b.save(tmp_path / "b.json")
    assert json.loads((tmp_path / "a.json").read_text()) == \
        json.loads((tmp_path / "b.json").read_text())
    ia, ib = a.integer_outputs(calib[1]), b.integer_outputs(calib[1])
    for name in g.outputs:
        np.testing.assert_array_equal(ia[name], ib[name])


@pytest.mark.parametrize("quant_type", ["int8", "uint8", "int16"])
@pytest.mark.parametrize("model", sorted(MODELS))
def test_loaded_model_matches_oracle(hip, tmp_path, model, quant_type):
    """The loaded graph's integer pass against the oracle pipeline run on
    the same loaded graph and q.json: every tensor bit-exact."""
    print(f"case loaded {model} {quant_type}", flush=True)
    g, shape = MODELS[model]()
    h = onnx_io.load_onnx(onnx_io.save_onnx(g, tmp_path / "m.onnx"))
    calib = _calib(shape)
    c = QuantContainer(h, quant_type, True)
    c.calibrate(calib)
    ex = c.executor({h.input_names[0]: shape})
    ex.run({h.input_names[0]: calib[1]})
    c.save(tmp_path / "q.json")
    o = OraclePipeline(h, tmp_path / "q.json")
    o.run(calib[1], keep=True)
    checked = 0
    for n, t in ex.tensors.items():
        if n in o.env:
            got = t.to_host()
            np.testing.assert_array_equal(got, o.env[n].reshape(got.shape),
                                          err_msg=n)
            checked += 1
    assert checked >= 10


@pytest.mark.parametrize("gelu", ["tanh", "erf"])
@pytest.mark.parametrize("quant_type", ["int8", "uint8"])
def test_loaded_vit_export_matches_oracle(hip, tmp_path, quant_type, gelu):
    """A ViT export loaded through the reference's passes (LayerNorm fusion,
    attention scale and LayerNorm affine folded, class-token Gather hoisted)
    quantizes at the post-pass graph's points: its operators are those of
    graph.vit, its integer layers are bit-exact against the oracle and its
    float fallbacks (LayerNorm, Softmax, activation MatMuls, Gather) within
    one step."""
    from collections import Counter
    print(f"case vit export {quant_type} {gelu}", flush=True)
    raw = G.vit_export(gelu=gelu, **CFG)
    h = onnx_io.load_onnx(onnx_io.save_onnx(raw, tmp_path / "vit.onnx"))
    want = Counter(n.op_type for n in G.vit(seed=7, **CFG).nodes)
    if gelu == "erf":
        want["FusedElementwise"] += want.pop("Gelu")
    assert Counter(n.op_type for n in h.nodes) == want
    shape = (CFG["batch"], 3, CFG["size"], CFG["size"])
    calib = _calib(shape, seed=90)
    c = QuantContainer(h, quant_type, True)
    c.calibrate(calib)
    x = Stream(95).normal(shape, 1.0).astype(np.float32)
    ex = c.executor({"images": x.shape}, fuse_attention=False)
    ex.run({"images": x})
    worst, exact, checked = _check_against_oracle(c, h, tmp_path, x, ex)
    assert worst <= 1 and exact >= 0.99, (worst, exact)
    assert checked >= 20


def _grid_close(got, want, step, exact):
    """Both on the output grid (float32 rounding of the dequantized values
    aside): grid indices within one step, equal on ``exact`` of them."""
    qg = np.rint(np.asarray(got, np.float64) / step)
    qw = np.rint(np.asarray(want, np.float64) / step)
    assert np.abs(np.asarray(got, np.float64) - qg * step).max() <= \
        1e-4 * step + 2 * float(np.spacing(np.float32(np.abs(want).max())))
    d = np.abs(qg - qw)
    assert d.max() <= 1, d.max()
    assert (d == 0).mean() >= exact, (d == 0).mean()


@pytest.mark.parametrize("quant_type", ["int8", "uint8", "int16"])
@pytest.mark.parametrize("model", sorted(MODELS))
def test_qdq_export(hip, tmp_path, model, quant_type):
    g, shape = MODELS[model]()
    c = QuantContainer(g, quant_type, True)
    calib = _calib(shape)
    c.calibrate(calib)
    data = onnx_io.export_qdq(c, tmp_path / "qdq.onnx")

    # structure, read by the protobuf runtime
    m = PB["ModelProto"]()
    m.ParseFromString(data)
    inits = {t.name: t for t in m.graph.initializer}

    def value(name):
        t = inits[name]
        dt = np.dtype(onnx_io.DTYPES[t.data_type])
        return np.frombuffer(t.raw_data, dt).reshape(tuple(t.dims))

    qnodes = {n.output[0][:-2]: n for n in m.graph.node
              if n.op_type == "QuantizeLinear"}
    quantized = [n for n, r in ((o, r) for r in c.layers
                                for o in r.node.outputs)
                 if r.kind != "shape"]
    assert set(quantized) <= set(qnodes)
    for name in quantized + list(g.input_names):
        qp = c.qparams[name]
        n = qnodes[name] if name in qnodes else qnodes[name + "_dq"]
        assert value(n.input[1]).reshape(-1).tolist() == \
            [np.float32(qp.scale)]
        assert value(n.input[2]).reshape(-1).tolist() == [qp.zp]
    for r in c.layers:
        if r.kind in ("conv", "gemm"):
            np.testing.assert_array_equal(
                value(r.node.name + "_w_quant").astype(np.int64), r.w_q)
    want_opset = 13 if quant_type.endswith("8") else 21
    assert [o.version for o in m.opset_import] == [want_opset]

    # numbers: every quantized tensor of the QDQ model's float run against
    # the record's fake-quantized evaluation on the same inputs (the file's
    # scales are float32, the ONNX type, so a value next to a rounding tie
    # may move by one step)
    h = onnx_io.load_onnx(data, optimize=False)
    env = float_ops.run_float(h, calib[1], keep_all=True)
    exact = 0.99 if quant_type.endswith("8") else 0.95

    def read(name):
        if name in g.input_names:
            return env[name + "_dq"]
        if name in c.const_names:
            return env[name + "_deq"]
        return env[name]

    for r in c.layers:
        got = r.fake([read(n) for n in r.inputs])
        for o, v, qp in zip(r.node.outputs, got, r.out_qp):
            _grid_close(env[o], v, qp.scale, exact)
