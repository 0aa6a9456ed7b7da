"""ViT-S/16 at its real configuration (224x224 input, 196 patches + the
class token = 197 tokens, dim 384, 6 heads, MLP 1536, 12 layers) through the
device executor against the oracle: every integer tensor bit-exact given
the same inputs, the float fallbacks (LayerNorm, Softmax, activation x
activation MatMul, Gather) within one step and exact on >= 98% of elements
(the scheme of test_gpu_vit.py), at batch 2, each operator on its own; the
fused attention launches give that pass bit for bit; then the batch-32
pass of the same model and q.json reproduces the batch-2 logits in its
first two rows."""

import time

import numpy as np
import pytest

from oracle import abi
from quantanything_amd import graph as G
from quantanything_amd.container import QuantContainer
from quantanything_amd.synth import Stream
from tests.test_gpu_vit import _check_against_oracle

pytestmark = pytest.mark.gpu


def test_vit_s16_full_size(hip, tmp_path, monkeypatch):
    t0 = time.time()
    g2 = G.vit(seed=5, batch=2)
    assert sum(1 for n in g2.nodes if n.op_type == "Softmax") == 12
    calib = [Stream(80 + i).normal((2, 3, 224, 224)).astype(np.float32)
             for i in range(2)]
    c = QuantContainer(g2, "int8", True)
    c.calibrate(calib)
    x2 = Stream(85).normal((2, 3, 224, 224)).astype(np.float32)
    # each operator on its own for the oracle comparison
    ex = c.executor({"images": x2.shape}, fuse_attention=False)
    out2 = ex.run({"images": x2})
    print(f"calibrated and ran b2 in {time.time() - t0:.1f}s", flush=True)
    # the compiled reference kernels are the faster CPU checker here
    if abi.ref_available():
        import oracle.pipeline as P

        real = P.OraclePipeline.__init__
        monkeypatch.setattr(P.OraclePipeline, "__init__",
                            lambda self, g, q, lib="ref": real(self, g, q,
                                                               lib))
    worst, exact, checked = _check_against_oracle(c, g2, tmp_path, x2, ex)
    print(f"oracle checked {checked} tensors in {time.time() - t0:.1f}s: "
          f"fallbacks within {worst} step, {exact:.4f} exact", flush=True)
    assert worst <= 1 and exact >= 0.99, (worst, exact)
    assert checked >= 12 * 8

    # the fused attention launches give the same integer pass
    exf = c.executor({"images": x2.shape})
    assert sum(n.startswith("attention:") for n, _ in exf.launches) == 12
    exf.run({"images": x2})
    for n, t in exf.tensors.items():
        if n in ex.tensors:
            np.testing.assert_array_equal(t.to_host(), ex.tensors[n].to_host(),
                                          err_msg=n)

    # batch 32 (fused attention) with the same weights and q.json
    path = tmp_path / "q.json"
    c.save(path)
    g32 = G.vit(seed=5, batch=32)
    c32 = QuantContainer.load(g32, path)
    x32 = np.concatenate([x2, Stream(86).normal((30, 3, 224, 224)).astype(
        np.float32)])
    ints32 = c32.integer_outputs(x32)
    ints2 = ex.integer_outputs()
    (name,) = g2.outputs
    assert ints32[g32.outputs[0]].shape[0] == 32
    np.testing.assert_array_equal(ints32[g32.outputs[0]][:2], ints2[name])
    assert out2[name].shape == (2, 1000)
