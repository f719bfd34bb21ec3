"""Pins of the router restatement (oracle/moe.py: scoring, route_topk with
bias / hash routing, dedupe_topk) on the CPU: closed forms of the score
functions, brute-force selection, and a direct loop transcription of
dedupe_topk's update rule checked on inputs with many repeats."""
import numpy as np
import pytest

from oracle import moe


def test_score_functions_closed_forms():
    x = np.array([0.0, 1.0, -1.0, 30.0, -30.0, 100.0, -100.0], np.float32)
    sg = moe.scoring(x, "sigmoid")
    np.testing.assert_allclose(sg, 1 / (1 + np.exp(-x.astype(np.float64))), rtol=1e-6, atol=1e-30)
    assert sg[0] == np.float32(0.5)
    sp = moe.scoring(x, "sqrtsoftplus").astype(np.float64)
    want = np.sqrt(np.logaddexp(0.0, x.astype(np.float64)))  # log(1 + e^x) without overflow
    np.testing.assert_allclose(sp[:6], want[:6], rtol=2e-7)
    np.testing.assert_allclose(sp[6], want[6], rtol=2e-2)   # softplus(-100) ~ 3.7e-44 is an f32 subnormal
    assert abs(sp[0] - np.sqrt(np.log(2.0))) < 1e-7
    assert np.isfinite(sp).all() and sp[6] > 0                 # no overflow / underflow to 0 at +-100
    sm = moe.scoring(np.zeros((3, 8), np.float32), "softmax")
    np.testing.assert_array_equal(sm, np.full((3, 8), 0.125, np.float32))


def test_bias_routing_selects_on_biased_keys_and_weighs_unbiased():
    rng = np.random.default_rng(0)
    logits = rng.standard_normal((64, 16)).astype(np.float32)
    bias = rng.standard_normal(16).astype(np.float32)
    w, ids = moe.route_topk(logits, 4, scoring_fn="sigmoid", bias=bias)
    s = moe.scoring(logits, "sigmoid")
    for t in range(64):
        key = s[t] + bias
        order = sorted(range(16), key=lambda e: (-key[e], e))[:4]
        assert list(ids[t]) == order
        np.testing.assert_array_equal(w[t], s[t, order])


def test_hash_routing_gathers_scores_and_renormalize_sums_to_one():
    rng = np.random.default_rng(1)
    logits = rng.standard_normal((32, 24)).astype(np.float32)
    hid = rng.integers(0, 24, (32, 6)).astype(np.int32)
    w, ids = moe.route_topk(logits, 6, scoring_fn="sqrtsoftplus", hash_ids=hid, renormalize=True)
    np.testing.assert_array_equal(ids, hid)
    s = moe.scoring(logits, "sqrtsoftplus")
    g = np.take_along_axis(s, hid, axis=1)
    np.testing.assert_allclose(w, g / g.sum(axis=1, keepdims=True), rtol=1e-6)
    np.testing.assert_allclose(w.sum(axis=1), 1.0, rtol=1e-6)


def _dedupe_loop(w, ids, E):
    """Scalar transcription of dedupe_topk's update, token by token."""
    w = w.astype(np.float32).copy()
    ids = ids.astype(np.int32).copy()
    T, k = ids.shape
    C = min(2 * k, E)
    for t in range(T):
        for j in range(1, k):
            prev = [q for q in range(j) if ids[t, q] == ids[t, j]]
            first = prev[0] if prev else 0
            w[t, first] = np.float32(w[t, first] + (w[t, j] if prev else np.float32(0)))
            held = set(int(v) for v in ids[t])
            free = next((c for c in range(C) if c not in held), 0)
            if prev:
                ids[t, j] = free
                w[t, j] = 0
    return w, ids


@pytest.mark.parametrize("k,E", [(4, 64), (8, 12), (6, 6), (3, 2)])
def test_dedupe_topk_matches_loop_and_keeps_mass(k, E):
    rng = np.random.default_rng(k * 100 + E)
    ids = rng.integers(0, min(E, 5), (200, k)).astype(np.int32)   # many repeats
    w = rng.random((200, k)).astype(np.float32)
    got_w, got_ids = moe.dedupe_topk(w, ids, E)
    want_w, want_ids = _dedupe_loop(w, ids, E)
    np.testing.assert_array_equal(got_ids, want_ids)
    np.testing.assert_array_equal(got_w, want_w)
    if 2 * k <= E:
        assert all(len(set(r)) == k for r in got_ids)              # distinct when candidates suffice
    np.testing.assert_allclose(got_w.sum(1), w.sum(1), rtol=1e-6)  # weight only moves
