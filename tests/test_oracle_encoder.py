"""The oracle's encoder ops against the reference's known answers and
independent mathematics (CPU only).

* softmaxRows: TestSoftmaxRows / TestSoftmaxRowsBatched
  (runtime/backend/tensor_ops_test.go:500-511, 422-433).
* layerNormRows: TestLayerNormRows(Batched) (tensor_ops_test.go:395-412).
* geluTensor: the reference's test restates the formula, so it is pinned
  here by the tanh approximation's value at 1 (0.8411920) and by the
  identity gelu(x) - gelu(-x) = x of 0.5 x (1 + tanh(odd function of x)).
* The encoder pipeline (examples/encoder_trainable_q8.manta:37-60): against
  a float64 numpy evaluation of the same steps, and by its T = 1 reduction
  (softmax of one score is 1, so attention passes v through).
"""
import numpy as np

from oracle import oracle as orc


def test_softmax_known_answers():
    got = orc.softmax_rows(np.array([[0, 0], [1, 0]], np.float32))
    np.testing.assert_allclose(got, [[0.5, 0.5], [0.7310586, 0.26894143]], rtol=0, atol=1e-7)
    e, e2 = np.float32(np.exp(1)), np.float32(np.exp(2))
    got = orc.softmax_rows(np.array([[[0, 1], [1, 0]], [[2, 0], [0, 2]]], np.float32))
    want = [[[1 / (1 + e), e / (1 + e)], [e / (1 + e), 1 / (1 + e)]],
            [[e2 / (1 + e2), 1 / (1 + e2)], [1 / (1 + e2), e2 / (1 + e2)]]]
    np.testing.assert_allclose(got, want, rtol=1e-6)


def test_softmax_properties():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal((7, 33)) * 5).astype(np.float32)
    p = orc.softmax_rows(x)
    np.testing.assert_allclose(p.sum(1), 1.0, rtol=1e-6)
    np.testing.assert_array_equal(np.argmax(p, 1), np.argmax(x, 1))
    # invariant to a constant shift, exp ratios preserved
    np.testing.assert_allclose(orc.softmax_rows(x + 3.0), p, rtol=2e-5, atol=1e-7)
    np.testing.assert_allclose(p[:, 1] / p[:, 0], np.exp(x[:, 1].astype(np.float64) - x[:, 0]), rtol=1e-5)


def test_layernorm_known_answers_and_moments():
    got = orc.layernorm_rows(np.array([[2, 4], [6, 8], [1, 3], [5, 7]], np.float32).reshape(2, 2, 2))
    np.testing.assert_allclose(got.reshape(4, 2), [[-0.999995, 0.999995]] * 4, rtol=0, atol=1e-6)
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((5, 384)) * 3 + 2).astype(np.float32)
    y = orc.layernorm_rows(x).astype(np.float64)
    np.testing.assert_allclose(y.mean(1), 0.0, atol=1e-5)
    var = x.astype(np.float64).var(1)
    np.testing.assert_allclose(y.var(1), var / (var + 1e-5), rtol=1e-4)


def test_gelu_value_and_odd_identity():
    g = orc.gelu(np.array([0.0, 1.0, -1.0], np.float32))
    assert g[0] == 0.0
    assert abs(g[1] - 0.8411920) < 2e-7
    x = np.linspace(-6, 6, 97).astype(np.float32)
    np.testing.assert_allclose(orc.gelu(x) - orc.gelu(-x), x, atol=2e-6)
    # far tails: x for large x, 0 for very negative x
    np.testing.assert_allclose(orc.gelu(np.array([10.0, -10.0], np.float32)), [10.0, 0.0], atol=1e-6)


def _case(seed, b, t, vocab, d, h):
    rng = np.random.default_rng(seed)
    tokens = rng.integers(0, vocab, size=(b, t), dtype=np.int32)
    lengths = rng.integers(1, t + 1, size=b)
    mask = (np.arange(t)[None, :] < lengths[:, None]).astype(np.int32)
    table = (rng.standard_normal((vocab, d)) * 0.5).astype(np.float32)
    ws = [(rng.standard_normal(s) / np.sqrt(s[0])).astype(np.float32)
          for s in [(d, d), (d, d), (d, d), (d, d), (d, h), (h, d)]]
    return tokens, mask, table, ws


def _numpy_f64(tokens, mask, table, ws, layers=1):
    wq, wk, wv, wo, wup, wproj = [w.astype(np.float64) for w in ws]

    def ln(z):
        m = z.mean(-1, keepdims=True)
        return (z - m) / np.sqrt(((z - m) ** 2).mean(-1, keepdims=True) + 1e-5)

    e = table.astype(np.float64)[tokens]
    for _ in range(layers):  # encoder_trainable_q8x2: the block twice, shared weights
        x = e
        q, k, v = x @ wq, x @ wk, x @ wv
        s = q @ np.swapaxes(k, 1, 2)
        s = np.exp(s - s.max(-1, keepdims=True))
        p = s / s.sum(-1, keepdims=True)
        a = (p @ v) @ wo + x
        ah = ln(a)
        f = ah @ wup
        f = 0.5 * f * (1 + np.tanh(0.7978845608 * (f + 0.044715 * f ** 3)))
        e = ln(f @ wproj + ah)
    e = e / np.linalg.norm(e, axis=-1, keepdims=True)
    m = mask.astype(np.float64)[..., None]
    cnt = m.sum(1)
    return np.where(cnt > 0, (e * m).sum(1) / np.maximum(cnt, 1), 0.0)


def test_encoder_pipeline_against_float64():
    tokens, mask, table, ws = _case(3, 4, 12, 40, 48, 96)
    got = orc.encoder_pooled(tokens, mask, table, *ws)
    want = _numpy_f64(tokens, mask, table, ws)
    np.testing.assert_allclose(got, want, rtol=0, atol=5e-5)


def test_encoder_single_token_passes_v_through():
    # T = 1: softmax of one score is 1, so mixed = v = x @ wv
    tokens, mask, table, ws = _case(4, 3, 1, 20, 32, 64)
    got = orc.encoder_pooled(tokens, mask, table, *ws)
    want = _numpy_f64(tokens, mask, table, ws)
    np.testing.assert_allclose(got, want, rtol=0, atol=5e-5)


def test_two_layer_encoder_against_float64():
    """encoder_trainable_q8x2.manta:9-50: the second block reads the first
    block's encoded output; the same float64 evaluation applied twice."""
    tokens, mask, table, ws = _case(5, 3, 10, 30, 40, 80)
    got = orc.encoder_pooled(tokens, mask, table, *ws, layers=2)
    np.testing.assert_allclose(got, _numpy_f64(tokens, mask, table, ws, layers=2), rtol=0, atol=5e-5)
    # the second block matters: one block is far from two
    assert np.max(np.abs(got - _numpy_f64(tokens, mask, table, ws, layers=1))) > 1e-2
