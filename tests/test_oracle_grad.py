"""Pins of the gradient hand-off oracle (objc/bridge.m:902-948): the token
scatter-add against an independent sequential implementation (numpy's
unbuffered ufunc.at), a known answer that only the loop's summation order
gives, the out-of-range token rule, and the elementwise accumulation."""
import numpy as np

import oracle


def test_scatter_matches_ufunc_at():
    rng = np.random.default_rng(1)
    vocab, d, n = 50, 17, 600
    tokens = rng.zipf(1.3, n).astype(np.uint32) % 70  # repeats and some >= vocab
    dx0 = rng.standard_normal((n, d)).astype(np.float32) * 1e3
    g = rng.standard_normal((vocab, d)).astype(np.float32)
    want = g.copy()
    np.add.at(want, np.where(tokens < vocab, tokens, 0), dx0)  # sequential, float32
    oracle.embed_scatter(g, tokens, dx0)
    np.testing.assert_array_equal(g.view(np.uint32), want.view(np.uint32))


def test_scatter_order_known_answer():
    """Rows of one token added in increasing i: ((1e8 + 1) - 1e8) + 1 = 1 in
    fp32 (the first 1 is below half an ulp of 1e8); the same rows summed in
    reverse order give 0, so the answer pins the order."""
    g = np.zeros((4, 1), np.float32)
    oracle.embed_scatter(g, np.array([3, 3, 3, 3], np.uint32),
                         np.array([[1e8], [1.0], [-1e8], [1.0]], np.float32))
    assert g[3, 0] == 1.0 and not g[:3].any()
    r = np.zeros((4, 1), np.float32)
    oracle.embed_scatter(r, np.array([3, 3, 3, 3], np.uint32),
                         np.array([[1.0], [-1e8], [1.0], [1e8]], np.float32))
    assert r[3, 0] == 0.0


def test_scatter_out_of_range_goes_to_row_zero():
    """bridge.m:923: a token >= vocab is added into row 0."""
    g = np.zeros((3, 2), np.float32)
    oracle.embed_scatter(g, np.array([2, 3, 7, 0], np.uint32),
                         np.array([[1, 1], [2, 2], [4, 4], [8, 8]], np.float32))
    assert g.tolist() == [[14, 14], [0, 0], [1, 1]]


def test_accumulate():
    rng = np.random.default_rng(2)
    a = rng.standard_normal(1000).astype(np.float32)
    b = rng.standard_normal(1000).astype(np.float32)
    want = a + b
    oracle.grad_accumulate(a, b)
    np.testing.assert_array_equal(a, want)
