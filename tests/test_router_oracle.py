"""CPU pins of the MoE router restatement (oracle hro_moe_router, a literal
restatement of kernels.cu:536-684 with glibc expf):

* closed forms: softmax weights of small rows, the normalised pair, sigmoid
  gating whose bias changes the order but not the weights, equal scores,
  the non-finite fallbacks, weights_scale, ties to the lowest expert id, and
  the NaN-key sequence of the sigmoid scan (worked out from the loop);
* an independent formulation (sort by (weight desc, id asc), vectorised) on
  random rows without NaN, bit for bit.
"""
import math

import numpy as np

from oracle import oracle as O

F32 = np.float32


def test_softmax_closed_forms():
    O.build()
    x = np.array([[1, 2, 3, 0.5]], F32)
    ids, w = O.moe_router(x, 2)
    assert ids.tolist() == [[2, 1]]
    d = 1 + math.exp(-1) + math.exp(-2) + math.exp(-2.5)
    np.testing.assert_allclose(w[0], [1 / d, math.exp(-1) / d], rtol=1e-6)
    ids, w = O.moe_router(x, 2, norm_topk=True)
    np.testing.assert_allclose(w[0], [1 / (1 + math.exp(-1)), math.exp(-1) / (1 + math.exp(-1))], rtol=1e-6)
    ids, w2 = O.moe_router(x, 2, norm_topk=True, weights_scale=2.5)
    assert np.array_equal(w2, (w * F32(2.5)).astype(F32))
    # k = 1 never normalises
    ids, w = O.moe_router(x, 1, norm_topk=True)
    np.testing.assert_allclose(w[0], [1 / d], rtol=1e-6)


def test_equal_scores_and_ties():
    ids, w = O.moe_router(np.full((1, 8), 0.25, F32), 3)
    assert ids.tolist() == [[0, 1, 2]] and np.allclose(w, 1 / 8, rtol=1e-6)
    ids, w = O.moe_router(np.full((1, 8), 0.25, F32), 3, norm_topk=True)
    assert np.allclose(w, 1 / 3, rtol=1e-6)
    x = np.array([[0.0, 5.0, 1.0, 5.0, 5.0, 1.0]], F32)
    ids, _ = O.moe_router(x, 5)
    assert ids.tolist() == [[1, 3, 4, 2, 5]]


def test_non_finite_fallbacks():
    # a +inf or all -inf row: non-finite max
    for row in ([0.0, np.inf, 1.0, 2.0], [-np.inf] * 4):
        ids, w = O.moe_router(np.array([row], F32), 3)
        assert ids.tolist() == [[0, 1, 2]] and np.allclose(w, 1 / 4)
        ids, w = O.moe_router(np.array([row], F32), 3, norm_topk=True)
        assert np.allclose(w, 1 / 3)
    # NaN: ignored by the max, but the sum becomes NaN
    ids, w = O.moe_router(np.array([[1.0, np.nan, 3.0, 2.0]], F32), 2)
    assert ids.tolist() == [[0, 1]] and np.allclose(w, 1 / 4)


def test_sigmoid_gating():
    x = np.array([[1, 2, 3, 0.5]], F32)
    sig = lambda v: 1 / (1 + math.exp(-v))
    ids, w = O.moe_router(x, 2, gating_sigmoid=True, bias=np.array([5, 0, 0, 0], F32))
    assert ids.tolist() == [[0, 2]]
    np.testing.assert_allclose(w[0], [sig(1), sig(3)], rtol=1e-6)
    ids, w = O.moe_router(x, 3, gating_sigmoid=True, norm_topk=True)
    assert ids.tolist() == [[2, 1, 0]]
    s = sig(3) + sig(2) + sig(1)
    np.testing.assert_allclose(w[0], [sig(3) / s, sig(2) / s, sig(1) / s], rtol=1e-6)
    # NaN score -> score 0 (key 0 + bias); -inf score -> 0
    ids, w = O.moe_router(np.array([[np.nan, -np.inf, 0.0]], F32), 3, gating_sigmoid=True)
    assert ids.tolist() == [[2, 0, 1]] and w[0].tolist() == [0.5, 0.0, 0.0]
    # NaN key at the first expert: rank 0 keeps it (nothing compares larger),
    # then no expert is eligible below a NaN key: rank 1 falls back to id 1
    # with key -inf, and rank 2 finds no key below -inf: id 2
    ids, w = O.moe_router(np.array([[0.0, 1.0, 2.0]], F32), 3, gating_sigmoid=True,
                          bias=np.array([np.nan, 0, 0], F32))
    assert ids.tolist() == [[0, 1, 2]] and w[0].tolist() == [0.5, 0.0, 0.0]
    # a NaN key later in the row never wins
    ids, _ = O.moe_router(np.array([[0.0, 1.0, 2.0]], F32), 2, gating_sigmoid=True,
                          bias=np.array([0, np.nan, 0], F32))
    assert ids.tolist() == [[2, 0]]


def _independent(x, k, norm, sigmoid, bias, scale):
    """Vectorised restatement: weights once, order by (key desc, id asc)."""
    rows, E = x.shape
    ids = np.zeros((rows, k), np.uint32)
    out = np.zeros((rows, k), F32)
    for r in range(rows):
        if sigmoid:
            e = O.expf(-x[r])
            score = (F32(1) / (F32(1) + e)).astype(F32)
            score[~np.isfinite(score)] = 0
            key = (score + bias).astype(F32) if bias is not None else score
            wt = score
        else:
            mx = np.max(x[r])
            t = O.expf((x[r] - mx).astype(F32))
            d = F32(0)
            for v in t:
                d = F32(d + v)
            wt = (t / d).astype(F32)
            key = wt
        order = np.lexsort((np.arange(E), -key.astype(np.float64)))[:k]
        ids[r] = order
        sel = wt[order]
        s = F32(0)
        for v in sel:
            s = F32(s + v)
        if norm and k > 1 and s > F32(1e-7) and np.isfinite(s):
            sel = (sel / s).astype(F32)
        if scale != 1.0:
            sel = (sel * F32(scale)).astype(F32)
        out[r] = sel
    return ids, out


def test_router_matches_independent_formulation():
    rng = np.random.default_rng(11)
    for E, k in ((8, 2), (64, 6), (160, 8), (256, 8), (300, 300)):
        x = (rng.standard_normal((6, E)) * 2).astype(F32)
        x[1, 5] = x[1, 3]  # a tie
        bias = (rng.standard_normal(E) * 0.1).astype(F32)
        for sigmoid in (False, True):
            for norm in (False, True):
                b = bias if sigmoid else None
                got = O.moe_router(x, k, bias=b, norm_topk=norm, gating_sigmoid=sigmoid, weights_scale=1.5)
                want = _independent(x, k, norm, sigmoid, b, 1.5)
                assert np.array_equal(got[0], want[0]), (E, k, sigmoid, norm)
                assert np.array_equal(got[1].view(np.uint32), want[1].view(np.uint32)), (E, k, sigmoid, norm)
