"""The routing audit's own logic, on the CPU: margins against brute force, no
unexplained mismatch when two logit sets differ within the stated tolerance, and a
planted selection error (logits moved far beyond it) reported as unexplained."""
import itertools

import numpy as np

from _routing_audit import audit, key_bounds, selection_margins
from oracle import router as R


def test_margins_match_brute_force():
    rng = np.random.default_rng(0)
    lg = rng.standard_normal((40, 8)).astype(np.float32)
    eg, gg = selection_margins(lg, 3, R.SOFTMAX, False)
    for t in range(40):
        v = sorted(lg[t].astype(np.float64), reverse=True)
        assert eg[t] == min(v[j] - v[j + 1] for j in range(3))
    assert np.all(np.isinf(gg))
    # grouped: 8 experts in 4 groups of 2, 2 kept: group scores are pair sums
    bias = rng.standard_normal(8).astype(np.float32) * 0.1
    eg, gg = selection_margins(lg, 2, R.SIGMOID, True, bias, 4, 2)
    c = (R._activate(lg, R.SIGMOID) + bias).astype(np.float32)
    for t in range(40):
        g = sorted([float(np.float32(c[t, 2 * j] + c[t, 2 * j + 1])) if c[t, 2 * j] >= c[t, 2 * j + 1]
                    else float(np.float32(c[t, 2 * j + 1] + c[t, 2 * j])) for j in range(4)], reverse=True)
        assert np.isclose(gg[t], g[1] - g[2], rtol=0, atol=1e-7)
        best = max(itertools.combinations(range(4), 2),
                   key=lambda s: (sum(np.float32(c[t, 2 * j]) + np.float32(c[t, 2 * j + 1]) for j in s)))
        kept = sorted([float(c[t, e]) for j in best for e in (2 * j, 2 * j + 1)], reverse=True)
        assert np.isclose(eg[t], min(kept[0] - kept[1], kept[1] - kept[2]), rtol=0, atol=1e-7)


def _route(lg, bias, grouped):
    if grouped:
        return R.route_grouped(lg, bias, 8, 8, 4, R.SIGMOID, True, 1e-20, 2.5)[0]
    return R.route_topk_act(lg, 8, R.SOFTMAX)[0]


def test_perturbation_within_tolerance_is_always_explained():
    rng = np.random.default_rng(1)
    for grouped in (False, True):
        lg = (rng.standard_normal((4000, 64)) * 2).astype(np.float32)
        lg[::7, 5] = lg[::7, 9]                                    # exact ties
        bias = (rng.standard_normal(64) * 0.05).astype(np.float32) if grouped else None
        u = rng.uniform(-0.9, 0.9, lg.shape)
        v = rng.uniform(-0.9, 0.9, lg.shape)
        lg2 = (lg + u * 1e-5 * np.abs(lg) + v * 2e-5).astype(np.float32)
        rep = audit(lg, lg2, _route(lg2, bias, grouped), _route(lg, bias, grouped), 8,
                    R.SIGMOID if grouped else R.SOFTMAX, grouped, bias, 8 if grouped else 1,
                    4 if grouped else 1)
        assert rep["mismatched"] > 0, rep              # the ties do flip
        assert rep["unexplained"] == [], rep


def test_planted_selection_error_is_unexplained():
    rng = np.random.default_rng(2)
    lg = (rng.standard_normal((200, 64)) * 2).astype(np.float32)
    ids = _route(lg, None, False)
    wrong = ids.copy()
    t = int(np.argmax(selection_margins(lg, 8, R.SOFTMAX, False)[0]))   # the clearest token
    outside = next(e for e in range(64) if e not in ids[t])
    wrong[t, 7] = outside
    rep = audit(lg, lg, wrong, ids, 8, R.SOFTMAX, False)
    assert rep["unexplained"] == [t], rep
    de, _ = key_bounds(lg, R.SOFTMAX, False)
    assert np.all(de > 2e-5)
