"""Bound of the LayerNorm folded into the next matrix's rows (the persistent
decode kernel's LN2/LN3), in float32, against LayerNorm then matmul in float64.

For a row W of the next matrix, W . LN(x) = rsd * (W . (g*x) - mean * (W . g))
+ (W . b + bias), with mean and rsd from the two-pass statistics of
internal/ml/ops.go:166-193. The subtraction cancels the mean's share of the
dot, so the relative error grows linearly with |mean| / spread: measured here
4e-7 at mean 0, 2e-5 at mean 50, 2.3e-4 at mean 500 and 2.8e-3 at mean 5000
(spread 1, d = 1280), so inside the 1e-3 logits bar up to |mean| ~ 2000 x
spread. A one-pass variance E[x^2] - mean^2 is already off by more than 1e-3 at
mean 500.
"""
import numpy as np
import pytest


def _fold_f32(W, g, b, bias, x):
    f = np.float32
    W, g, b, bias, x = (np.asarray(a, f) for a in (W, g, b, bias, x))
    n = x.size
    mean = f(np.sum(x, dtype=f) / f(n))
    var = f(np.sum((x - mean) * (x - mean), dtype=f) / f(n))
    rsd = f(1.0 / np.sqrt(np.float64(var + f(1e-5))))
    dot = (W @ (g * x)).astype(f)
    c = (W @ g).astype(f)
    e = (W @ b + bias).astype(f)
    return rsd * (dot - mean * c) + e


def _exact(W, g, b, bias, x):
    x = x.astype(np.float64)
    ln = (x - x.mean()) / np.sqrt(x.var() + 1e-5) * g + b
    return W.astype(np.float64) @ ln + bias


@pytest.mark.parametrize("mean,bound", [(0.0, 1e-5), (50.0, 1e-4), (500.0, 1e-3)])
def test_folded_layernorm_error(mean, bound):
    rng = np.random.default_rng(int(mean) + 1)
    d, rows = 1280, 256
    W = (rng.standard_normal((rows, d)) * 0.02).astype(np.float32)
    g = (1 + rng.standard_normal(d) * 0.02).astype(np.float32)
    b = (rng.standard_normal(d) * 0.02).astype(np.float32)
    bias = (rng.standard_normal(rows) * 0.02).astype(np.float32)
    worst = 0.0
    for _ in range(8):
        x = (mean + rng.standard_normal(d)).astype(np.float32)
        got = _fold_f32(W, g, b, bias, x)
        want = _exact(W, g, b, bias, x)
        worst = max(worst, float(np.max(np.abs(got - want)) / np.max(np.abs(want))))
    assert worst < bound, worst


def test_one_pass_variance_fails_at_large_mean():
    """Why the statistics are two-pass: E[x^2] - mean^2 in float32 at mean 500."""
    rng = np.random.default_rng(3)
    f = np.float32
    x = (500 + rng.standard_normal(1280)).astype(f)
    n = f(x.size)
    m = f(np.sum(x, dtype=f) / n)
    one = f(np.sum(x * x, dtype=f) / n) - m * m
    two = f(np.sum((x - m) * (x - m), dtype=f) / n)
    exact = np.var(x.astype(np.float64))
    assert abs(two - exact) / exact < 1e-5
    assert abs(one - exact) / exact > 1e-3
