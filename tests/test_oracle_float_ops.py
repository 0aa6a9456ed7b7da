"""Pins of the oracle's float operator semantics used by the transformer
fallbacks (``oracle/float_ref.py``): closed forms and invariants that a
dropped term, a wrong axis or a transposed operand would break."""

import numpy as np

from oracle.float_ref import eval_node, layer_norm, softmax
from quantanything_amd.graph import Node


def _node(op, **attrs):
    return Node("n", op, ["a", "b", "c"], ["y"], attrs)


def test_softmax_closed_form_and_invariants():
    y = softmax(np.array([[0.0, np.log(2.0)]], np.float32), 1)
    np.testing.assert_allclose(y, [[1 / 3, 2 / 3]], rtol=1e-6)
    x = np.random.default_rng(0).normal(size=(4, 7)).astype(np.float32)
    s = softmax(x, 1)
    np.testing.assert_allclose(s.sum(axis=1), 1.0, rtol=1e-6)
    np.testing.assert_allclose(softmax(x + np.float32(3.0), 1), s, rtol=1e-5)
    assert s.dtype == np.float32 and (np.argmax(s, 1) == np.argmax(x, 1)).all()


def test_layer_norm_closed_form():
    y = layer_norm(np.array([[1.0, 3.0]], np.float32), np.float32(1.0),
                   None, 1, 0.0)
    np.testing.assert_array_equal(y, [[-1.0, 1.0]])
    g = np.array([2.0, 0.5], np.float32)
    b = np.array([1.0, -1.0], np.float32)
    y = layer_norm(np.array([[1.0, 3.0]], np.float32), g, b, 1, 0.0)
    np.testing.assert_array_equal(y, [[-1.0, -0.5]])
    x = np.random.default_rng(1).normal(3.0, 2.0, size=(5, 64)).astype(
        np.float32)
    y = layer_norm(x, np.float32(1.0), None, 1, 1e-6).astype(np.float64)
    np.testing.assert_allclose(y.mean(axis=1), 0.0, atol=1e-6)
    np.testing.assert_allclose(y.var(axis=1), 1.0, rtol=1e-5)
    node = _node("LayerNormalization", axis=-1, epsilon=0.0)
    out = eval_node(node, [np.array([[1.0, 3.0]], np.float32),
                           np.ones(2, np.float32), None])[0]
    np.testing.assert_array_equal(out, [[-1.0, 1.0]])


def test_matmul_brute_force_and_batching():
    rng = np.random.default_rng(2)
    a = rng.integers(-5, 6, size=(2, 3, 4, 5)).astype(np.float32)
    b = rng.integers(-5, 6, size=(2, 3, 5, 6)).astype(np.float32)
    y = eval_node(_node("MatMul"), [a, b])[0]
    want = np.zeros((2, 3, 4, 6))
    for i in range(2):
        for h in range(3):
            for m in range(4):
                for n in range(6):
                    want[i, h, m, n] = sum(a[i, h, m, k] * b[i, h, k, n]
                                           for k in range(5))
    np.testing.assert_array_equal(y, want)  # small integers: exact
    assert y.dtype == np.float32


def test_gather_squeeze_unsqueeze():
    x = np.arange(2 * 3 * 4, dtype=np.float32).reshape(2, 3, 4)
    g = eval_node(_node("Gather", axis=1), [x, np.array(0)])[0]
    np.testing.assert_array_equal(g, x[:, 0, :])
    g = eval_node(_node("Gather", axis=2), [x, np.array([3, 1])])[0]
    np.testing.assert_array_equal(g, x[:, :, [3, 1]])
    s = eval_node(_node("Squeeze"), [x[None], np.array([0])])[0]
    assert s.shape == (2, 3, 4)
    u = eval_node(_node("Unsqueeze"), [x, np.array([0, -1])])[0]
    assert u.shape == (1, 2, 3, 4, 1)


def test_gelu_tanh_closed_form():
    node = Node("n", "Gelu", ["a"], ["y"], {"approximate": "tanh"})
    x = np.array([0.0, 1.0, -1.0, 8.0], np.float32)
    y = eval_node(node, [x])[0].astype(np.float64)
    t = 0.5 * (1 + np.tanh(np.sqrt(2 / np.pi) * (1 + 0.044715)))
    np.testing.assert_allclose(y, [0.0, t, t - 1.0, 8.0], rtol=1e-6,
                               atol=1e-7)
