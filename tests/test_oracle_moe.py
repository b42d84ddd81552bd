"""Pins the MoE router / combine oracle (oracle/moe.py) without a GPU: closed forms, invariants
and a brute-force selection written independently of the oracle's sort."""
import itertools

import numpy as np
import pytest

from oracle import moe


def brute_topk(row, k):
    """descending probability, ties to the lower expert, by comparing every pair"""
    n = len(row)
    chosen = []
    for _ in range(k):
        best = None
        for i in range(n):
            if i in chosen:
                continue
            if best is None or row[i] > row[best]:      # strict: an equal later expert never wins
                best = i
        chosen.append(best)
    return chosen


@pytest.mark.parametrize("n,k", [(8, 2), (16, 5), (60, 8), (130, 10)])
def test_topk_matches_brute_force(n, k):
    g = np.random.default_rng(n * 31 + k)
    logits = np.round(g.standard_normal((7, n)) * 2, 1)      # rounded: many exact ties
    ids, w = moe.topk(logits, k, 0.0, np.inf)
    p = np.exp(logits - logits.max(axis=1, keepdims=True))
    for t in range(7):
        assert list(ids[t]) == brute_topk(p[t], k)
        sel = p[t][brute_topk(p[t], k)]
        np.testing.assert_allclose(w[t], sel / sel.sum(), rtol=1e-12)


def test_float32_exp_ties_go_to_the_lower_expert():
    """Distinct logits whose float32 exp(x - max) is equal tie, and the lower expert wins (the
    reference ranks the float32 exp values, and ggml's SOFT_MAX -> ARGSORT the float32
    probabilities).  exp(-1e-8) and exp(-2e-8) are within half an ulp of 1 (ulp 2^-24 below 1),
    so every correctly rounded exp returns 1.0f for them, as for the maximum itself."""
    assert np.exp(np.float32(-1e-8)) == np.float32(1.0) and np.exp(np.float32(-2e-8)) == np.float32(1.0)
    logits = np.full((1, 400), -3.0, np.float32)
    logits[0, 300] = 0.0                                  # the maximum, at a high index
    logits[0, 7] = -2e-8
    logits[0, 5] = -1e-8
    logits[0, 9] = -0.5
    ids, w = moe.topk(logits, 4, 0.0, np.inf)
    assert list(ids[0]) == [5, 7, 300, 9]                  # logit order would be 300, 5, 7, 9
    np.testing.assert_allclose(w[0, :3], w[0, 0], rtol=1e-7)


def test_uniform_logits_pick_the_lowest_experts_with_equal_weights():
    ids, w = moe.topk(np.full((3, 40), 1.25), 6, 6.103515625e-5, np.inf)
    assert (ids == np.arange(6)).all()
    np.testing.assert_allclose(w, 1.0 / 6.0, rtol=1e-15)


def test_shift_invariance_and_softmax_sum():
    g = np.random.default_rng(5)
    x = g.standard_normal((4, 33)) * 4
    np.testing.assert_allclose(moe.softmax(x).sum(axis=1), 1.0, rtol=1e-14)
    a = moe.topk(x, 7, 0.0, np.inf)
    b = moe.topk(x + 123.0, 7, 0.0, np.inf)
    assert (a[0] == b[0]).all()
    np.testing.assert_allclose(a[1], b[1], rtol=1e-12)


def test_clamp_bounds_the_weight_sum():
    # one dominant expert: the top-1 probability is ~1, the others tiny
    x = np.zeros((1, 10))
    x[0, 3] = 30.0
    ids, w = moe.topk(x, 1, 0.0, 0.5)                         # sum ~1 clamped down to 0.5: weight ~2
    assert ids[0, 0] == 3 and abs(w[0, 0] - 2.0) < 1e-9
    ids, w = moe.topk(x, 2, 0.0, np.inf)                      # unclamped: weights sum to 1
    assert abs(w.sum() - 1.0) < 1e-12
    ids, w = moe.topk(x[:, [0, 1, 2]], 1, 0.5, np.inf)        # uniform 1/3 clamped up to 0.5
    assert ids[0, 0] == 0 and abs(w[0, 0] - (1 / 3) / 0.5) < 1e-12


def test_combine_closed_forms():
    g = np.random.default_rng(9)
    e = g.standard_normal((3, 1, 17)).astype(np.float32)
    w = g.standard_normal((3, 1)).astype(np.float32)
    np.testing.assert_array_equal(moe.combine(e, w), e[:, 0, :] * w)          # k = 1: one product
    e2 = np.concatenate([e, np.zeros_like(e)], axis=1)
    w2 = np.concatenate([w, g.standard_normal((3, 1)).astype(np.float32)], axis=1)
    np.testing.assert_array_equal(moe.combine(e2, w2), e[:, 0, :] * w)       # a zero expert adds nothing
    s = g.standard_normal((3, 17)).astype(np.float32)
    y = moe.combine(e, w, s, np.zeros(3, np.float32))                         # sigmoid(0) = 0.5 exactly
    np.testing.assert_array_equal(y, e[:, 0, :] * w + s * np.float32(0.5))


def test_combine_sums_slots_in_order():
    # float32 addition is not associative: the oracle must add slot 0, then 1, then 2
    e = np.array([[[1e8], [1.0], [-1e8]]], np.float32)
    w = np.ones((1, 3), np.float32)
    assert moe.combine(e, w)[0, 0] == np.float32(np.float32(np.float32(1e8) + 1.0) - np.float32(1e8))
    for perm in itertools.permutations(range(3)):
        if perm == (0, 1, 2):
            continue
        other = np.float32(0)
        for j in perm:
            other = np.float32(other + e[0, j, 0])
        if other != moe.combine(e, w)[0, 0]:
            return
    pytest.fail("the case does not tell the orders apart")
