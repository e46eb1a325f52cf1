"""Pins the router oracle: brute force on tiny inputs, torch closed forms, invariants."""
import itertools

import numpy as np
import pytest
import torch

from oracle import router as R
from oracle.mathfn import sigmoid_f32


def _brute_topk(row, k):
    return [i for _, i in sorted(((-float(v), i) for i, v in enumerate(row)))[:k]]


def test_topk_desc_matches_full_sort_with_ties():
    rng = np.random.default_rng(0)
    x = rng.integers(0, 5, (200, 12)).astype(np.float32)        # many ties
    ids = R.topk_desc(x, 4)
    for t in range(200):
        assert list(ids[t]) == _brute_topk(x[t], 4)


def test_topk_act_softmax_matches_reference_semantics():
    """router.py:384-441: topk on logits, softmax over the k values, scatter."""
    rng = np.random.default_rng(1)
    lg = rng.normal(0, 2, (64, 8)).astype(np.float32)
    ids, w = R.route_topk_act(lg, 2, R.SOFTMAX)
    tl = torch.from_numpy(lg)
    tv, ti = torch.topk(tl, 2, dim=-1)
    assert np.array_equal(ids, ti.numpy().astype(np.int32))
    ref = torch.softmax(tv.double(), dim=-1).numpy()
    assert np.allclose(w, ref, rtol=1e-6, atol=0)
    aff = R.scatter_dense(ids, w, 8)
    assert np.allclose(aff.sum(1), 1.0, atol=1e-6)
    assert np.all((aff != 0).sum(1) == 2)


def test_act_topk_renorm_sigmoid():
    """router.py:444-504: activation over all E, topk, L1 renorm (no epsilon)."""
    rng = np.random.default_rng(2)
    lg = rng.normal(0, 1, (50, 16)).astype(np.float32)
    ids, w = R.route_act_topk_renorm(lg, 3, R.SIGMOID, renorm=True, eps=0.0)
    p = 1 / (1 + np.exp(-lg.astype(np.float64)))
    for t in range(50):
        assert list(ids[t]) == _brute_topk(p[t], 3)
        sel = p[t, ids[t]]
        assert np.allclose(w[t], sel / sel.sum(), rtol=1e-6)


def _brute_grouped(c, s, k, n_group, topk_group, scale, renorm):
    E = len(c)
    gs = E // n_group
    gsc = []
    for j in range(n_group):
        vals = sorted((float(v) for v in c[j * gs:(j + 1) * gs]), reverse=True)
        gsc.append(np.float32(vals[0]) if gs == 1 else np.float32(np.float32(vals[0]) + np.float32(vals[1])))
    # exhaustive over group subsets: the chosen subset maximises the sorted score vector
    best = None
    for sub in itertools.combinations(range(n_group), topk_group):
        key = sorted(((-float(gsc[j]), j) for j in sub))
        if best is None or key < best[0]:
            best = (key, sub)
    kept = set(best[1])
    cand = [e for e in range(E) if e // gs in kept]
    ids = [i for _, i in sorted((-float(c[e]), e) for e in cand)[:k]]
    w = np.array([s[i] for i in ids], np.float64)
    if renorm:
        w = w / (w.sum() + 1e-20)
    return ids, w * scale


@pytest.mark.parametrize("E,n_group,topk_group,k", [(16, 4, 2, 4), (12, 3, 1, 2), (8, 8, 3, 3)])
def test_grouped_matches_exhaustive_search(E, n_group, topk_group, k):
    rng = np.random.default_rng(E * 100 + n_group)
    lg = rng.normal(0, 1.5, (40, E)).astype(np.float32)
    bias = rng.normal(0, 0.3, E).astype(np.float32)
    ids, w = R.route_grouped(lg, bias, k, n_group, topk_group, R.SIGMOID, renorm=True, scale=2.5)
    s = sigmoid_f32(lg)
    c = (s + bias).astype(np.float32)
    for t in range(40):
        bi, bw = _brute_grouped(c[t], s[t], k, n_group, topk_group, 2.5, True)
        assert list(ids[t]) == bi
        assert np.allclose(w[t], bw, rtol=1e-6)


def test_grouped_bias_selects_but_does_not_weight():
    lg = np.array([[2.0, 1.0, 0.0, -1.0]], np.float32)
    bias = np.array([0.0, 5.0, 0.0, 0.0], np.float32)
    ids, w = R.route_grouped(lg, bias, 1, 1, 1, R.SIGMOID, renorm=False, scale=1.0)
    assert ids[0, 0] == 1                                        # bias flips the selection
    assert np.isclose(w[0, 0], 1 / (1 + np.exp(-1.0)), rtol=1e-6)  # weight is the unbiased score


def test_grouped_with_one_group_is_plain_topk():
    rng = np.random.default_rng(5)
    lg = rng.normal(0, 1, (30, 32)).astype(np.float32)
    ids, w = R.route_grouped(lg, None, 6, 1, 1, R.SIGMOID, renorm=True, scale=1.0)
    for t in range(30):
        assert list(ids[t]) == _brute_topk(lg[t], 6)              # sigmoid is increasing
        assert np.isclose(w[t].sum(), 1.0, atol=1e-6)


def test_renorm_scale_sums_to_routed_scaling():
    rng = np.random.default_rng(6)
    lg = rng.normal(0, 1, (100, 256)).astype(np.float32)
    bias = rng.normal(0, 0.01, 256).astype(np.float32)
    ids, w = R.route_grouped(lg, bias, 8, 8, 4, R.SIGMOID, renorm=True, scale=2.5)
    assert np.allclose(w.sum(1), 2.5, rtol=1e-5)
    assert np.all(np.diff(np.sort(ids, axis=1), axis=1) > 0)          # distinct experts
    # every id lies in one of at most 4 groups
    assert np.all(np.array([len(set(r // 32)) for r in ids]) <= 4)


def test_rms_norm_closed_form():
    rng = np.random.default_rng(7)
    x = rng.normal(0, 3, (5, 64)).astype(np.float32)
    gamma = rng.normal(1, 0.1, 64).astype(np.float32)
    y = R.rms_norm(x, gamma, 1e-6)
    ref = x / np.sqrt((x.astype(np.float64) ** 2).mean(-1, keepdims=True) + 1e-6) * gamma
    assert np.allclose(y, ref, rtol=1e-5)


def test_rms_norm_padded_closed_forms():
    rng = np.random.default_rng(11)
    H, ha = 96, 80
    gamma = rng.normal(1, 0.2, H).astype(np.float32)
    # a constant row c: rsqrt(c^2 + eps) * c * gamma on the real columns, 0 on the padding
    c = np.float32(1.75)
    x = np.full((1, H), c, np.float32)
    x[0, ha:] = 100.0                                  # padding must not enter the variance
    y = R.rms_norm_padded(x, gamma, 1e-6, ha)
    ref = c / np.sqrt(float(c) ** 2 + 1e-6) * gamma[:ha].astype(np.float64)
    assert np.allclose(y[0, :ha], ref, rtol=2e-7)
    assert np.all(y[0, ha:] == 0)
    # scale invariance at eps = 0 (a power of two scales every step exactly)
    x = rng.normal(0, 2, (4, H)).astype(np.float32)
    assert np.array_equal(R.rms_norm_padded(4 * x, gamma, 0.0, ha), R.rms_norm_padded(x, gamma, 0.0, ha))
    # hidden_actual = H is the plain _torch_rms_norm
    assert np.array_equal(R.rms_norm_padded(x, gamma, 1e-6), R.rms_norm(x, gamma, 1e-6))


def test_topk_scatter_act_matches_closed_forms():
    rng = np.random.default_rng(12)
    lg = rng.normal(0, 2, (9, 12)).astype(np.float32)
    k = 3
    sm = R.route_topk_scatter_act(lg, k, R.SOFTMAX)
    sg = R.route_topk_scatter_act(lg, k, R.SIGMOID)
    for t in range(lg.shape[0]):
        top = _brute_topk(lg[t], k)
        assert sorted(np.nonzero(sm[t])[0].tolist()) == sorted(top)
        assert sorted(np.nonzero(sg[t])[0].tolist()) == sorted(top)
        v = lg[t, top].astype(np.float64)
        e = np.exp(v - v.max())
        assert np.allclose(sm[t, top], e / e.sum(), rtol=1e-6)
        assert np.allclose(sg[t, top], 1 / (1 + np.exp(-v)), rtol=1e-6)
    # same ids and (to rounding) weights as the topk -> act order
    ids, w = R.route_topk_act(lg, k, R.SOFTMAX)
    assert np.allclose(np.take_along_axis(sm, ids.astype(np.int64), 1), w, rtol=1e-6)
