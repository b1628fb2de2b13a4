"""Pin the CPU oracle before trusting it: golden vectors from independent implementations,
textbook float64 forms, and the reference's own known-answer tests."""
from pathlib import Path

import numpy as np
import pytest

import oracle.encoder as E
from laya_cuda import synthetic

GOLDEN = Path(__file__).resolve().parent / "golden"


def _cfg(spec):
    return {"width": spec.width, "heads": spec.heads, "eps": spec.eps, "layers": spec.layers}


def _small():
    spec = synthetic.adapter(None, layers=2, width=128, heads=2, intermediate=512, vocab=1000, positions=64,
                             max_len=64)
    g = np.load(GOLDEN / "bert_small.npz")
    w = E.structured(synthetic.weights(spec, seed=int(g["seed"]), random_norms=True, std=float(g["std"])), _cfg(spec))
    return spec, g, w


def test_encoder_matches_transformers_bert():
    spec, g, w = _small()
    for s in range(int(g["n_seq"])):
        hidden = E.encoder_sequence(g[f"ids{s}"], w, _cfg(spec))
        np.testing.assert_allclose(hidden, g[f"hidden{s}"], atol=2e-5, rtol=1e-5)


def test_head_matches_torch_head():
    spec, g, w = _small()
    hidden = [E.encoder_sequence(g[f"ids{s}"], w, _cfg(spec)) for s in range(int(g["n_seq"]))]
    for q in range(int(g["n_q"])):
        logits, acts, feats = E.head(hidden[int(g[f"q{q}_seq"])], g[f"q{q}_markers"], int(g[f"q{q}_kind"]), w)
        np.testing.assert_allclose(logits, g[f"q{q}_logits"], atol=2e-5, rtol=1e-5)
        np.testing.assert_allclose(feats, g[f"q{q}_feats"], atol=2e-5, rtol=1e-5)
        np.testing.assert_allclose(acts, g[f"q{q}_acts"], atol=2e-5, rtol=1e-5)


def test_full_size_l83_matches_transformers():
    spec = synthetic.adapter("l83")
    g = np.load(GOLDEN / "l83.npz")
    w = E.structured(synthetic.weights(spec, seed=int(g["seed"])), _cfg(spec))
    logits, acts, hidden = E.forward([g["ids0"]], [(0, g["q0_markers"], 0)], w, _cfg(spec))
    rows = hidden[0][np.concatenate([[0], g["q0_markers"]])]
    np.testing.assert_allclose(rows, g["q0_rows"], atol=2e-4, rtol=1e-4)
    np.testing.assert_allclose(logits[0], g["q0_logits"], atol=2e-5)
    np.testing.assert_allclose(acts[0], g["q0_acts"], atol=2e-5)


def test_layer_norm_matches_float64_textbook():
    rng = np.random.default_rng(11)
    x = rng.normal(2, .3, (5, 768)).astype(np.float32)
    gamma, beta = rng.normal(1, .1, 768).astype(np.float32), rng.normal(0, .1, 768).astype(np.float32)
    x64 = x.astype(np.float64)
    expected = (x64 - x64.mean(-1, keepdims=True)) / np.sqrt(x64.var(-1, keepdims=True) + 1e-12) * gamma + beta
    np.testing.assert_allclose(E.layer_norm(x, gamma, beta, 1e-12), expected, atol=2e-5, rtol=1e-5)


def test_gelu_matches_math_erf():
    import math
    xs = np.linspace(-6, 6, 97).astype(np.float32)
    expected = np.array([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in xs.astype(np.float64)])
    np.testing.assert_allclose(E.gelu(xs), expected, atol=1e-6, rtol=1e-6)
    assert E.gelu(np.float32(0)) == 0


@pytest.mark.parametrize("window", [-1, 8])
def test_attention_matches_float64_softmax(window):
    """The float64 method of the reference's tests/test_attention.py:45-53."""
    rng = np.random.default_rng(3)
    L, h = 40, 2
    q, k, v = (rng.normal(0, 1, (L, h, 64)).astype(np.float32) for _ in range(3))
    qh, kh, vh = (a.astype(np.float64).transpose(1, 0, 2) for a in (q, k, v))
    s = qh @ kh.transpose(0, 2, 1) / 8
    if window >= 0:
        s[:, np.abs(np.arange(L)[:, None] - np.arange(L)) > window] = -np.inf
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    expected = (p @ vh).transpose(1, 0, 2).reshape(L, h * 64)
    np.testing.assert_allclose(E.attention(q, k, v, window), expected, atol=1e-5, rtol=1e-5)


def test_attention_key_order_invariance_and_uniform_case():
    """Bidirectional attention is invariant to the order of (key, value) pairs, and a zero query
    attends uniformly (output = mean of V)."""
    rng = np.random.default_rng(4)
    L, h = 24, 1
    q, k, v = (rng.normal(0, 1, (L, h, 64)).astype(np.float32) for _ in range(3))
    out = E.attention(q, k, v)
    perm = rng.permutation(L)
    np.testing.assert_allclose(E.attention(q, k[perm], v[perm]), out, atol=1e-5)
    assert np.allclose(E.attention(q * 0, k, v), np.broadcast_to(v.mean(0).reshape(1, -1), (L, 64)), atol=1e-6)


def test_features_known_cases():
    cls = np.arange(4, dtype=np.float32)
    single = E.features(cls, np.array([7.0], np.float32), 1)
    np.testing.assert_array_equal(single[:4], cls)
    np.testing.assert_allclose(single[4:], [1.0, 1.0, 0.0, 2 / 255])
    even = E.features(cls, np.zeros(4, np.float32), 4)
    np.testing.assert_allclose(even[4:], [0.25, 0.0, 1.0, 4 / 255], rtol=1e-6)


def test_softmax_known_answer():
    """tests/test_contract.py:42-43 of the reference."""
    np.testing.assert_allclose(E.softmax([10000, 10000]), [.5, .5])


def test_planted_mistakes_fail_the_golden_check():
    """A plausible mistake in the oracle (pre-LN order, tanh GELU, no positions) must fail."""
    spec, g, w = _small()
    cfg = _cfg(spec)
    good = E.encoder_sequence(g["ids0"], w, cfg)
    original = E.gelu
    try:
        E.gelu = lambda x: (0.5 * x * (1 + np.tanh(0.7978845608 * (x + 0.044715 * x ** 3)))).astype(np.float32)
        tanh = E.encoder_sequence(g["ids0"], w, cfg)
    finally:
        E.gelu = original
    assert np.abs(tanh - g["hidden0"]).max() > 1e-4
    w2 = dict(w)
    w2["encoder.embeddings"] = dict(w["encoder.embeddings"], pos=np.zeros_like(w["encoder.embeddings"]["pos"]))
    assert np.abs(E.encoder_sequence(g["ids0"], w2, cfg) - g["hidden0"]).max() > 1e-2
    assert np.abs(good - g["hidden0"]).max() < 2e-5


# ---------------- ModernBERT variant (the reference's executor) ----------------

def _modernbert():
    import oracle.modernbert as M
    spec = synthetic.modernbert_adapter(layers=4, width=128, heads=2, intermediate=256, vocab=1000, positions=512,
                                        max_len=512, head_layers=2)
    g = np.load(GOLDEN / "modernbert_small.npz")
    weights = synthetic.weights(spec, seed=int(g["seed"]), random_norms=True, std=float(g["std"]))
    items = [(g[f"q{q}_ids"], list(g[f"q{q}_markers"]), int(g[f"q{q}_kind"])) for q in range(int(g["n_q"]))]
    return M, spec, g, M.structured(weights, M.config(spec)), items


def test_modernbert_encoder_matches_transformers():
    """Pre-LN, RoPE (global and local theta), +-64 window on local layers, GeGLU, final norm."""
    M, spec, g, w, items = _modernbert()
    for q, (ids, _, _) in enumerate(items):
        hidden = M.encoder_sequence(ids, w, M.config(spec))
        np.testing.assert_allclose(hidden, g[f"q{q}_hidden"], atol=3e-5, rtol=1e-5)


def test_modernbert_head_layers_match_torch_transformer_layers():
    M, spec, g, w, items = _modernbert()
    logits, acts, _ = M.forward(items, w, M.config(spec))
    for q in range(len(items)):
        np.testing.assert_allclose(logits[q], g[f"q{q}_logits"], atol=3e-5, rtol=1e-5)
        np.testing.assert_allclose(acts[q], g[f"q{q}_acts"], atol=3e-5, rtol=1e-5)


def test_modernbert_window_and_rope_are_load_bearing():
    """A planted mistake in the oracle (no window on local layers, or RoPE off) fails the fixture."""
    M, spec, g, w, items = _modernbert()
    ids = items[0][0]
    no_window = dict(M.config(spec), window=10 ** 6)
    assert np.abs(M.encoder_sequence(ids, w, no_window) - g["q0_hidden"]).max() > 1e-3
    same_theta = dict(M.config(spec), theta=[spec.theta[0], spec.theta[0]])
    assert np.abs(M.encoder_sequence(ids, w, same_theta) - g["q0_hidden"]).max() > 1e-3


def test_rope_tables_match_closed_form():
    import oracle.modernbert as M
    cos, sin = M.rope_tables(10000.0, 300)
    i = np.arange(32)
    angle = np.arange(300)[:, None] / 10000.0 ** (2 * i / 64)
    np.testing.assert_allclose(cos, np.cos(angle), atol=2e-5)
    np.testing.assert_allclose(sin, np.sin(angle), atol=2e-5)
    x = np.random.default_rng(0).normal(0, 1, (300, 2, 64)).astype(np.float32)
    r = M.rope(x, cos, sin)  # a rotation: norms per (position, pair) are preserved
    np.testing.assert_allclose(np.hypot(r[..., :32], r[..., 32:]), np.hypot(x[..., :32], x[..., 32:]), rtol=1e-5)


def test_rope_scores_depend_only_on_relative_position():
    """q.k after RoPE at positions (i, j) equals the same vectors' score at (i + s, j + s)."""
    import oracle.modernbert as M
    cos, sin = M.rope_tables(160000.0, 400)
    rng = np.random.default_rng(1)
    q, k = rng.normal(0, 1, (2, 1, 1, 64)).astype(np.float32)
    def score(i, j):
        return float((M.rope(q, cos[i:i + 1], sin[i:i + 1]) * M.rope(k, cos[j:j + 1], sin[j:j + 1])).sum())
    for i, j, s in [(0, 5, 7), (10, 3, 200), (64, 64, 300), (1, 129, 100)]:
        assert abs(score(i, j) - score(i + s, j + s)) < 2e-4 * max(1.0, abs(score(i, j)))
    assert abs(score(0, 5) - score(0, 6)) > 1e-4  # and it does depend on the offset
