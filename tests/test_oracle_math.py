"""Oracle LN / GELU / fast-exp softmax / attention / dot / sampling pinned to
the reference's own tests (internal/ml/ops_test.go, attention_test.go,
matmul_q8_test.go, internal/model/decoder_bench_test.go) and closed forms."""
import math

import numpy as np
import pytest

QTYPES = [2, 3, 6, 7, 8]


def approx(a, b, tol):
    return abs(float(a) - float(b)) <= tol


def test_gelu_known_values(orc):
    """ops_test.go:223-240 (tolerance 1e-3) and the tanh closed form."""
    for x, want in [(0, 0), (1, 0.8413), (-1, -0.1587), (2, 1.9545)]:
        assert approx(orc.gelu([x])[0], want, 1e-3)
    x = np.linspace(-8, 8, 1001).astype(np.float32)
    closed = 0.5 * x.astype(np.float64) * (1 + np.tanh(math.sqrt(2 / math.pi) * (x + 0.044715 * x.astype(np.float64) ** 3)))
    assert np.max(np.abs(orc.gelu(x) - closed)) < 1e-5


def test_layernorm_known_values(orc):
    """ops_test.go:243-286."""
    x = np.array([[1, 2, 3, 4]], np.float32)
    y = orc.layernorm(x, np.ones(4), np.zeros(4))
    assert approx(y.mean(), 0, 1e-5) and approx(((y - y.mean()) ** 2).mean(), 1, 1e-4)
    y = orc.layernorm(x, np.full(4, 2.0), np.ones(4))
    for got, want in zip(y[0], [-1.68328, 0.10557, 1.89442, 3.68328]):
        assert approx(got, want, 1e-3)
    rng = np.random.default_rng(0)
    x = rng.standard_normal((3, 1280)).astype(np.float32)
    w, b = rng.standard_normal(1280).astype(np.float32), rng.standard_normal(1280).astype(np.float32)
    x64 = x.astype(np.float64)
    ref = (x64 - x64.mean(1, keepdims=True)) / np.sqrt(x64.var(1, keepdims=True) + 1e-5) * w + b
    assert np.max(np.abs(orc.layernorm(x, w, b) - ref)) < 1e-4


def test_fast_exp(orc):
    """attention.go:34-61: 4th-order polynomial * 2^k; 0 at and below -20."""
    xs = np.linspace(-19.99, 0, 4001)
    rel = [abs(orc.fast_exp(x) / math.exp(np.float32(x)) - 1) for x in xs]
    # truncation bound of the degree-4 Taylor polynomial on [0, ln 2)
    r = math.log(2)
    bound = 1 - (1 + r + r ** 2 / 2 + r ** 3 / 6 + r ** 4 / 24) / 2
    assert 0.9 * bound < max(rel) < bound + 2e-6  # the approximation is really in use
    assert orc.fast_exp(0.0) == 1.0
    assert orc.fast_exp(-20.0) == 0.0 and orc.fast_exp(-1e9) == 0.0


def test_softmax(orc):
    """ops_test.go:289-314 and attention.go:93-171 (fast and exact)."""
    for fast in (True, False):
        y = orc.softmax(np.array([1, 0, 0], np.float32), fast)
        for got, want in zip(y, [0.5762, 0.2119, 0.2119]):
            assert approx(got, want, 2e-3)
        assert approx(orc.softmax(np.array([3, 1, 0.2], np.float32), fast).sum(), 1, 1e-5)
    row = np.array([0, -np.inf, -np.inf], np.float32)
    assert list(orc.softmax(row)) == [1.0, 0.0, 0.0]


def test_attention_known_values(orc):
    """ops_test.go:349-437: causal mask and exact weights (Tq=Tk=2)."""
    q = np.array([[[1, 0, 0, 0], [0, 1, 0, 0]]], np.float32)
    out, w = orc.sdpa(q, q, q, causal=True, fast=False, weights=True)
    assert approx(w[0, 0, 1], 0, 1e-5) and approx(w[0, 0, 0], 1, 1e-5)
    e = math.exp(0.5)
    assert approx(out[0, 0, 0], 1, 1e-5)
    assert approx(out[0, 1, 0], 1 / (1 + e), 1e-4) and approx(out[0, 1, 1], e / (1 + e), 1e-4)
    _, w = orc.sdpa(q, q, q, causal=False, fast=False, weights=True)
    assert np.allclose(w.sum(-1), 1, atol=1e-5)


def test_attention_fast_vs_exact(orc):
    """attention_test.go:9-60: max abs deviation <= 0.02 on uniform(-1,1) data."""
    rng = np.random.default_rng(7)
    q, k, v = (rng.uniform(-1, 1, (4, 32, 64)).astype(np.float32) for _ in range(3))
    d = np.max(np.abs(orc.sdpa(q, k, v, False, True) - orc.sdpa(q, k, v, False, False)))
    assert d <= 0.02


def test_attention_single_query_causal_is_row0(orc):
    """P1 (attention.go:250-256): with Tq = 1 the causal mask leaves key 0 only,
    so the output equals V row 0 exactly."""
    rng = np.random.default_rng(1)
    q = rng.standard_normal((3, 1, 64)).astype(np.float32)
    k = rng.standard_normal((3, 9, 64)).astype(np.float32)
    v = rng.standard_normal((3, 9, 64)).astype(np.float32)
    out = orc.sdpa(q, k, v, causal=True)
    assert np.array_equal(out[:, 0], v[:, 0])


def test_attention_textbook(orc):
    rng = np.random.default_rng(2)
    q = rng.standard_normal((2, 3, 16)).astype(np.float32)
    k = rng.standard_normal((2, 40, 16)).astype(np.float32)
    v = rng.standard_normal((2, 40, 16)).astype(np.float32)
    s = np.einsum("hqd,hkd->hqk", q.astype(np.float64), k) / 4.0
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    ref = np.einsum("hqk,hkd->hqd", p, v)
    assert np.max(np.abs(orc.sdpa(q, k, v, False, fast=False) - ref)) < 1e-5
    assert np.max(np.abs(orc.sdpa(q, k, v, False, fast=True) - ref)) < 2e-3


def _quant_row(orc, qtype, x):
    return orc.quantize(x, qtype)


def test_dot_q8_reference_case(orc):
    """matmul_q8_test.go:95-115: dot of a Q8_0 row with small integers, tol 0.5."""
    i = np.arange(64)
    f = (i % 7 - 3).astype(np.float32)
    g = ((i * 3) % 11 - 5).astype(np.float32)
    q = orc.quantize(g, 8)
    for variant in (0, 1):
        assert approx(orc.dot(8, q, f, variant), float(f @ g), 0.5)


def test_gemv_reference_cases(orc):
    """matmul_q8_test.go:117-207: m=2, k=64, n=3 against the float product,
    tolerances 1.0 (Q8_0) and 4/4/3/3/1 for all types."""
    m, k, n = 2, 64, 3
    a = ((np.arange(m * k) % 17 - 8) * 0.07).astype(np.float32).reshape(m, k)
    b = ((np.arange(n * k) % 11 - 5) * 0.11).astype(np.float32).reshape(n, k)
    ref = a.astype(np.float64) @ b.T.astype(np.float64)
    for qtype, tol in [(2, 4.0), (3, 4.0), (6, 3.0), (7, 3.0), (8, 1.0)]:
        raw = np.concatenate([orc.quantize(r, qtype) for r in b])
        for variant in (0, 1):
            got = orc.gemv(qtype, raw, n, k, a, variant)
            assert np.max(np.abs(got - ref)) <= tol
    a2 = ((np.arange(m * k) % 13 - 6) * 0.1).astype(np.float32).reshape(m, k)
    b2 = ((np.arange(n * k) % 9 - 4) * 0.2).astype(np.float32).reshape(n, k)
    raw = np.concatenate([orc.quantize(r, 8) for r in b2])
    assert np.max(np.abs(orc.gemv(8, raw, n, k, a2) - a2.astype(np.float64) @ b2.T)) <= 1.0


@pytest.mark.parametrize("qtype", QTYPES)
@pytest.mark.parametrize("cols", [32, 100, 1280, 5120 + 17])
def test_dot_vs_float64_bruteforce(orc, qtype, cols):
    """Both dot variants equal sum(x * dequant(w)) computed in float64 to fp32
    accumulation accuracy (tail blocks included)."""
    rng = np.random.default_rng(cols + qtype)
    w = (rng.standard_normal(cols) * 0.02).astype(np.float32)
    x = rng.standard_normal(cols).astype(np.float32)
    raw = orc.quantize(w, qtype)
    deq = orc.dequantize(raw, qtype, cols).astype(np.float64)
    exact = float(deq @ x.astype(np.float64))
    scale = float(np.abs(deq) @ np.abs(x.astype(np.float64))) + 1e-30
    for variant in (0, 1):
        assert abs(orc.dot(qtype, raw, x, variant) - exact) / scale < 3e-6


def test_repetition_penalty(orc):
    """decoder.go:1140-1167: subtract 2*count over the last 128 ids, prompt included."""
    logits = np.zeros(100, np.float32)
    hist = [5] * 3 + [7] + list(range(10, 10 + 200)) + [9, 9]
    hist = [h % 100 for h in hist]
    got = orc.repetition_penalty(logits, hist)
    window = hist[-128:]
    want = np.zeros(100, np.float32)
    for t in set(window):
        want[t] -= 2.0 * window.count(t)
    assert np.array_equal(got, want)
    assert np.array_equal(orc.repetition_penalty(logits, []), logits)


def _bench_logits(n=51865):
    lg = (-8.0 + 0.00003 * (np.arange(n) % 1000)).astype(np.float32)
    lg[17], lg[3], lg[9] = 7.5, 6.25, 5.75
    return lg


def test_greedy_and_topk_on_reference_pattern(orc):
    """decoder_bench_test.go:62-73 logits pattern: argmax 17, top-3 {17, 3, 9};
    log-probabilities normalised by logZ."""
    lg = _bench_logits()
    assert orc.sample_greedy(lg, 1.0) == 17
    tok, lp = orc.topk(lg, 3)
    assert list(tok) == [17, 3, 9]
    l64 = lg.astype(np.float64)
    # the reference accumulates float32(exp(float64(.))) sequentially in float32
    terms = np.exp(l64 - l64.max()).astype(np.float32)
    es = np.cumsum(terms, dtype=np.float32)[-1]
    logz = np.float32(np.log(np.float64(es))) + np.float32(l64.max())
    assert np.allclose(lp, lg[[17, 3, 9]] - logz, atol=1e-6)
    exact = np.log(np.exp(l64 - l64.max()).sum()) + l64.max()
    assert abs(float(logz) - exact) < 3e-3  # float32 accumulation drift of the reference


def test_greedy_ties_and_suppression(orc):
    """Strict '>' keeps the lowest index on ties; SuppressNST re-selects
    excluding EOT when logit[eot] < -NoSpeechThold (decoder.go:1006-1034)."""
    lg = np.zeros(60000, np.float32)
    lg[[50, 20, 80]] = 3.0
    assert orc.sample_greedy(lg, 1.0) == 20
    lg = np.full(60000, -5.0, np.float32)
    lg[50256] = -1.0
    lg[123] = -2.0
    assert orc.sample_greedy(lg, 1.0, suppress_nst=True, no_speech_thold=0.5) == 123
    assert orc.sample_greedy(lg, 1.0, suppress_nst=True, no_speech_thold=2.0) == 50256
    assert orc.sample_greedy(lg, 0.5) == 50256


def test_topk_replace_min_ties(orc):
    """The replace-min scan keeps a history-dependent member among equal values
    (decoder.go:1089-1121): for k=2 over [2a, 2b, 5, 2c] it keeps {5, 2b}."""
    tok, _ = orc.topk(np.array([2, 2, 5, 2], np.float32), 2)
    assert sorted(tok) == [1, 2]
