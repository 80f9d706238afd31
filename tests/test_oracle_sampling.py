"""Pins of the sampler oracle (oracle/sampling.py) against what fixes it independently:

* samp_exp within one weight unit of floor(2^40 e^d) from the C library's exp, over its whole range;
* dist against the literal float-probability formula of phase0/specsample.py:53-67 in fp64 (softmax,
  descending sort, keep while cumsum - p <= top_p, renormalise), ties ordered by id;
* hand-computed known answers for top-k / top-p boundaries and inverse-CDF draws;
* greedy = first argmax; the accept protocol is lossless (every slot's output distributed as p)."""
import math

import numpy as np
import pytest

from oracle import sampling as S


def test_samp_exp_within_one_unit_of_exp():
    d = np.concatenate([np.linspace(-27.75, 0.0, 200001), -np.log(2.0) * np.arange(0, 40),
                        [-1e-300, -5e-324, -27.7, -27.74999]])
    got = S.samp_exp(d).astype(np.float64)
    want = np.array([math.floor(math.ldexp(math.exp(v), 40)) for v in d], dtype=np.float64)
    assert np.max(np.abs(got - want)) <= 1.0
    assert int(S.samp_exp(np.array([0.0]))[0]) == 1 << 40
    assert (S.samp_exp(np.array([-27.76, -100.0, -np.inf])) == 0).all()


def _ref_dist(x, temp, top_k, top_p):
    """phase0/specsample.py:53-67 read literally, in fp64 (sort ties broken by id)."""
    z = np.asarray(x, dtype=np.float32) / np.float32(max(temp, 1e-6))
    z = z.astype(np.float64)
    if top_k and 0 < top_k < z.size:
        kth = np.sort(z)[::-1][top_k - 1]
        z = np.where(z < kth, -np.inf, z)
    p = np.exp(z - z.max())
    p /= p.sum()
    if 0.0 < top_p < 1.0:
        idx = np.lexsort((np.arange(p.size), -p))
        sp = p[idx]
        cum = np.cumsum(sp)
        keep = cum - sp <= top_p
        sp = np.where(keep, sp, 0.0)
        p = np.zeros_like(p)
        p[idx] = sp
        p /= p.sum()
    return p


@pytest.mark.parametrize("temp,top_k,top_p,ties", [
    (1.0, 0, 1.0, False), (0.7, 0, 0.9, False), (1.3, 40, 1.0, False), (0.5, 200, 0.95, False),
    (2.0, 0, 0.3, True), (1.0, 7, 0.8, True), (1e-3, 0, 0.9, False)])
def test_dist_matches_reference_formula(temp, top_k, top_p, ties):
    rng = np.random.default_rng(int(temp * 100) + top_k)
    x = rng.standard_normal(5000).astype(np.float32) * 3
    if ties:
        x = np.round(x * 2) / 2                       # a few dozen distinct values: boundary ties
    x = x.astype(np.float32)
    w = S.weights(x, temp, top_k, top_p)
    got = S.probs(w).astype(np.float64)
    want = _ref_dist(x, temp, top_k, top_p)
    assert np.array_equal(got > 0, want > 0), "kept sets differ"
    assert np.max(np.abs(got - want)) <= 1e-6


def test_top_p_known_answers():
    w = S.weights(np.zeros(4, np.float32), 1.0, 0, 0.5)            # four equal tokens, T = 2 units
    assert list(S.probs(w)) == [np.float32(1 / 3)] * 3 + [0.0]     # preceding weight 0, 1, 2 <= 2 kept
    x = np.array([2.0, 1.0, 0.0], np.float32)                      # p0 = e^2 / (e^2 + e + 1) = 0.665
    assert list(S.weights(x, 1.0, 0, 0.5) > 0) == [True, False, False]
    assert list(S.weights(x, 1.0, 0, 0.7) > 0) == [True, True, False]
    assert list(S.weights(x, 1.0, 2, 1.0) > 0) == [True, True, False]
    assert int(S.weights(x, 1.0, 0, 1e-9)[0]) == 1 << 40 and S.weights(x, 1.0, 0, 1e-9)[1:].sum() == 0
    y = np.array([1.0, 3.0, 3.0, 3.0, 0.0], np.float32)            # top-k counts ties: k=2 keeps all three
    assert list(S.weights(y, 1.0, 2, 1.0) > 0) == [False, True, True, True, False]
    z = np.array([-0.0, 0.0, -1.0], np.float32)                    # -0 and +0 are one value: id order
    assert list(S.weights(z, 1.0, 0, 0.4) > 0) == [True, False, False]


def test_draw_known_answers():
    w = np.array([1, 2, 3], np.uint64)
    assert [S.draw(w, u) for u in (0.0, 1 / 6, 0.34, 0.5, 0.999999)] == [0, 1, 1, 2, 2]
    assert [S.draw(w, u, exclude=2) for u in (0.0, 0.34, 0.5, 0.99)] == [0, 1, 1, 1]
    assert S.draw(np.array([0, 5, 0], np.uint64), 0.7, exclude=1) == 1          # nothing left: argmax
    assert S.draw(np.array([4, 5, 5], np.uint64), 0.7, exclude=-1) == 2
    assert S.draw_probs(np.array([0.25, 0.0, 0.75], np.float32), 0.3) == 2
    assert S.draw_probs(np.zeros(3, np.float32), 0.3) == 0


def test_greedy_first_argmax():
    x = np.array([1.0, 5.0, 5.0, -3.0], np.float32)
    assert S.greedy(x) == 1
    assert S.accept([x, x[::-1].copy()], [1], 0.0, 0, 1.0, iter([])) == [1, 1]


def test_accept_is_lossless():
    """Every slot's output is distributed as p: P(r0 = d) = p(d), P(r0 = y) = p(y) for y != d."""
    rng = np.random.default_rng(7)
    logits = [rng.standard_normal(6).astype(np.float32) for _ in range(3)]
    temp, top_k, top_p = 0.8, 5, 0.95
    p0 = S.probs(S.weights(logits[0], temp, top_k, top_p)).astype(np.float64)
    p2 = S.probs(S.weights(logits[2], temp, top_k, top_p)).astype(np.float64)
    draft = [int(np.argsort(p0)[-2]), 0]                           # a plausible but not top token
    uni = np.random.default_rng(11)
    n = 40000
    first = np.zeros(6)
    bonus = np.zeros(6)
    for _ in range(n):
        r = S.accept(logits, draft, temp, top_k, top_p, iter(uni.random(4)))
        first[r[0]] += 1
        if r[0] == draft[0] and r[1] == draft[1]:
            bonus[r[2]] += 1
    assert 0.5 * np.abs(first / n - p0).sum() < 0.015
    assert bonus.sum() > 0 and 0.5 * np.abs(bonus / bonus.sum() - p2).sum() < 0.05
    # a draft the filters removed is never emitted
    dead = int(np.argmin(p0)) if p0.min() == 0 else None
    if dead is not None:
        for _ in range(200):
            assert S.accept(logits, [dead, 0], temp, top_k, top_p, iter(uni.random(4)))[0] != dead
