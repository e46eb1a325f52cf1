"""End-to-end routing audit (test infrastructure).

The GPU's selection is compared bit for bit with the oracle's selector fed the
GPU's own logits (the layer tests assert that). This audit starts the oracle
from its own logits instead: numpy's fp32 product of the same bf16 operands, in
another summation order, as the reference's torch fallback computes them
(F.linear in fp32, router.py:420-424). The two logit sets differ in the last
bits, and the reference itself notes that this flips near-tie selections
(rmsnorm_router_topk_tkg.py:248-252). Every token whose ids differ must
therefore be a near-tie in the oracle's own keys:

* the selection keys of a token move by at most delta when its logits move by at
  most d = rtol * |logit| + atol (the tolerance the layer tests assert on the
  logits): delta = d for raw-logit keys (route_topk_act sorts the logits);
  delta = d / 4 + r for sigmoid keys (the sigmoid's slope is at most 1/4; r
  covers the rounding of the fp32 sigmoid and of the bias add), and twice that
  for a group score (the sum of a group's two largest keys);
* two keys can trade places only when their gap is at most 2 * delta. A token is
  explained when, in the oracle's keys, some adjacent pair among its first k + 1
  experts (in the kept groups), or the pair at the group cut, is that close.

The counts (mismatched tokens, the largest measured logit difference, the
smallest margin of a mismatch against its bound) are printed with the case.
"""
import numpy as np

from oracle import router as R

F = np.float32


def _sorted_gaps(keys, n):
    """Per row: the gaps key[j] - key[j + 1], j < n, of the keys sorted descending
    (-inf keys of masked experts included)."""
    srt = -np.sort(-np.asarray(keys, np.float64), axis=-1)
    n = min(n, srt.shape[-1] - 1)
    if n <= 0:
        return np.full(srt.shape[:-1] + (1,), np.inf)
    with np.errstate(invalid="ignore"):
        g = srt[..., :n] - srt[..., 1:n + 1]
    return np.where(np.isnan(g), np.inf, g)


def selection_margins(lg, k, scoring, grouped, bias=None, n_group=1, topk_group=1):
    """(expert_gap [T], group_gap [T]) of the oracle's selection from logits lg [T, E]:
    the smallest gap between adjacent keys among the first k + 1 candidates (order
    and cut of the top-k), and the gap at the kept-group cut (inf when every group
    is kept or there are no groups)."""
    lg = np.asarray(lg, F)
    T, E = lg.shape
    if not grouped:
        return _sorted_gaps(lg, k).min(axis=-1), np.full(T, np.inf)
    s = R._activate(lg, scoring)
    c = s if bias is None else (s + np.asarray(bias, F)[None, :]).astype(F)
    gs = E // n_group
    cg = c.reshape(T, n_group, gs)
    srt = -np.sort(-cg, axis=-1)
    gscore = srt[..., 0] if gs == 1 else (srt[..., 0] + srt[..., 1]).astype(F)
    if topk_group < n_group:
        gsrt = -np.sort(-gscore.astype(np.float64), axis=-1)
        ggap = gsrt[:, topk_group - 1] - gsrt[:, topk_group]
    else:
        ggap = np.full(T, np.inf)
    gsel = R.topk_desc(gscore, topk_group)
    keep = np.zeros((T, n_group), bool)
    np.put_along_axis(keep, gsel.astype(np.int64), True, axis=1)
    masked = np.where(np.repeat(keep, gs, axis=1), c, -np.inf)
    return _sorted_gaps(masked, k).min(axis=-1), ggap


def key_bounds(lg, scoring, grouped, bias=None, rtol=1e-5, atol=2e-5):
    """(delta_expert [T], delta_group [T]): how far one key (one group score) of each
    token can move when its logits move within rtol * |logit| + atol."""
    d = (rtol * np.abs(np.asarray(lg, np.float64)) + atol).max(axis=-1)
    if not grouped:
        return d, d
    if scoring != R.SIGMOID:
        raise NotImplementedError("grouped softmax keys have no Lipschitz bound here")
    bmax = 0.0 if bias is None else float(np.abs(np.asarray(bias, np.float64)).max())
    r = 4 * 2.0 ** -24 * (1.0 + bmax)          # rounding of sigmoid_f32 and the bias add
    de = d / 4 + r
    return de, 2 * de + 2 * r


def audit(lg_oracle, lg_gpu, ids_gpu, ids_oracle, k, scoring, grouped, bias=None, n_group=1,
          topk_group=1, rtol=1e-5, atol=2e-5):
    """Count the tokens whose GPU ids differ from the oracle's end-to-end ids and check
    that each is a near-tie. Returns a dict of counts; 'unexplained' lists the tokens
    that are not (an empty list is the pass condition)."""
    ids_gpu = np.asarray(ids_gpu)
    ids_oracle = np.asarray(ids_oracle)
    mis = np.nonzero((ids_gpu != ids_oracle).any(axis=1))[0]
    set_mis = [t for t in mis if set(ids_gpu[t].tolist()) != set(ids_oracle[t].tolist())]
    eg, gg = selection_margins(lg_oracle, k, scoring, grouped, bias, n_group, topk_group)
    de, dg = key_bounds(lg_oracle, scoring, grouped, bias, rtol, atol)
    ok = (eg <= 2 * de) | (gg <= 2 * dg)
    unexplained = [int(t) for t in mis if not ok[t]]
    ratio = [float(min(eg[t] / (2 * de[t]), gg[t] / (2 * dg[t]))) for t in mis]
    return {"tokens": int(ids_gpu.shape[0]), "mismatched": int(mis.size),
            "set_mismatched": len(set_mis), "order_only": int(mis.size) - len(set_mis),
            "near_ties_in_oracle": int(ok.sum()),
            "max_dlogit": float(np.abs(np.asarray(lg_oracle, np.float64)
                                       - np.asarray(lg_gpu, np.float64)).max()),
            "worst_margin_over_bound": max(ratio) if ratio else None,
            "unexplained": unexplained}
