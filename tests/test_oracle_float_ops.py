"""Pins of the oracle's float operator semantics used by the transformer
fallbacks (``oracle/float_ref.py``): closed forms and invariants that a
dropped term, a wrong axis or a transposed operand would break."""

import numpy as np
import pytest

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


# ------------------------------------------------------------ pooling ----
def _maxpool_brute(x, k, s, d, pads, pad_value):
    """Direct loops: output (oy, ox) covers input rows oy*s - top + ky*d;
    the padded array is sized so that ceil-mode's extra end padding only
    ever adds pad values."""
    n, c, h, w = x.shape
    pt, pl, pb, pr = pads
    oh = (h + pt + pb - (d[0] * (k[0] - 1) + 1)) // s[0] + 1
    ow = (w + pl + pr - (d[1] * (k[1] - 1) + 1)) // s[1] + 1
    y = np.empty((n, c, oh, ow), x.dtype)
    for oy in range(oh):
        for ox in range(ow):
            best = np.full((n, c), pad_value, dtype=np.float64)
            for ky in range(k[0]):
                for kx in range(k[1]):
                    iy = oy * s[0] - pt + ky * d[0]
                    ix = ox * s[1] - pl + kx * d[1]
                    if 0 <= iy < h and 0 <= ix < w:
                        best = np.maximum(best, x[:, :, iy, ix])
            y[:, :, oy, ox] = best
    return y


def _pool_node(**attrs):
    return Node("mp", "MaxPool", ["x"], ["y"], attrs)


@pytest.mark.parametrize("attrs, pads", [
    (dict(kernel_shape=[3, 3], strides=[2, 2], pads=[1, 1, 1, 1]),
     (1, 1, 1, 1)),
    (dict(kernel_shape=[5, 5], strides=[1, 1], pads=[2, 2, 2, 2]),
     (2, 2, 2, 2)),
    (dict(kernel_shape=[2, 3], strides=[1, 2], dilations=[2, 2]),
     (0, 0, 0, 0)),
])
def test_maxpool_matches_brute_force(attrs, pads):
    x = np.random.default_rng(3).integers(-100, 100, (2, 3, 9, 11)).astype(
        np.int32)
    got = eval_node(_pool_node(**attrs), [x], pad_value=-128)[0]
    k = attrs["kernel_shape"]
    want = _maxpool_brute(x, k, attrs["strides"],
                          attrs.get("dilations", [1, 1]), pads, -128)
    np.testing.assert_array_equal(got, want)


def test_maxpool_ceil_mode_output_size_and_values():
    # H = 6, k = 3, s = 2, no pads: floor gives 2 rows, ceil gives 3
    # (ONNX: ceil((6 - 3) / 2) + 1); the extra window holds the last row
    # and padding only.
    x = np.arange(2 * 6 * 7, dtype=np.int32).reshape(1, 2, 6, 7)
    floor = eval_node(_pool_node(kernel_shape=[3, 3], strides=[2, 2]), [x],
                      pad_value=-9)[0]
    ceil = eval_node(_pool_node(kernel_shape=[3, 3], strides=[2, 2],
                                ceil_mode=1), [x], pad_value=-9)[0]
    assert floor.shape == (1, 2, 2, 3) and ceil.shape == (1, 2, 3, 3)
    np.testing.assert_array_equal(ceil[:, :, :2, :], floor)
    # increasing values: a window's max is its bottom-right valid element
    np.testing.assert_array_equal(ceil[0, 0, 2], x[0, 0, 5, [2, 4, 6]])


def test_maxpool_auto_pad_same_lower_puts_extra_padding_first():
    x = np.arange(5, dtype=np.int32).reshape(1, 1, 1, 5)
    y = eval_node(_pool_node(kernel_shape=[1, 2], strides=[1, 2],
                             auto_pad="SAME_LOWER"), [x], pad_value=-9)[0]
    # out = ceil(5 / 2) = 3, one pad column, placed at the start
    np.testing.assert_array_equal(y.reshape(-1), [0, 2, 4])
    y = eval_node(_pool_node(kernel_shape=[1, 2], strides=[1, 2],
                             auto_pad="SAME_UPPER"), [x], pad_value=-9)[0]
    np.testing.assert_array_equal(y.reshape(-1), [1, 3, 4])


def test_chained_5x5_max_pools_equal_one_9x9():
    """The SPPF identity: with stride 1, 'same' padding and a padding value
    below every element, pool5(pool5(x)) = pool9(x)."""
    x = np.random.default_rng(9).integers(-50, 50, (1, 2, 12, 10)).astype(
        np.int32)
    p5 = _pool_node(kernel_shape=[5, 5], strides=[1, 1], pads=[2, 2, 2, 2])
    p9 = _pool_node(kernel_shape=[9, 9], strides=[1, 1], pads=[4, 4, 4, 4])
    twice = eval_node(p5, [eval_node(p5, [x], pad_value=-128)[0]],
                      pad_value=-128)[0]
    np.testing.assert_array_equal(twice, eval_node(p9, [x],
                                                   pad_value=-128)[0])


def test_global_max_pool_and_pad():
    x = np.random.default_rng(4).integers(-9, 9, (2, 3, 4, 5)).astype(
        np.int32)
    gmp = eval_node(Node("g", "GlobalMaxPool", ["x"], ["y"], {}), [x])[0]
    assert gmp.shape == (2, 3, 1, 1)
    for n in range(2):
        for c in range(3):
            assert gmp[n, c, 0, 0] == max(x[n, c].reshape(-1).tolist())
    pads = np.array([0, 1, 2, 0, 1, 0, 0, 3], np.int64)
    y = eval_node(Node("p", "Pad", ["x", "p"], ["y"], {}), [x, pads],
                  pad_value=7)[0]
    assert y.shape == (3, 4, 6, 8)
    assert (y[2] == 7).all() and (y[:, 0] == 7).all()
    assert (y[:, :, :2] == 7).all() and (y[:, :, :, 5:] == 7).all()
    np.testing.assert_array_equal(y[:2, 1:, 2:, :5], x)
