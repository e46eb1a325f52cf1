"""Router oracle (test infrastructure).

Follows the torch fallbacks of vllm_neuron/functional/moe/router.py:
  * route_topk_act            <- _torch_router_impl_prenorm_linear_topk_act_scatter, router.py:384-441
  * route_act_topk_renorm     <- _torch_router_impl_prenorm_linear_act_topk_renorm_scatter, router.py:444-504
                                 and the router_pre_norm branch of moe_block_tkg.py:165-185
  * route_grouped             <- not in the reference: DeepSeek-V3 "noaux_tc" grouped top-k
                                 (sigmoid + selection-only correction bias + group top-2 sum)
  * route_topk_scatter_act    <- _torch_router_impl_prenorm_linear_topk_scatter_act, router.py:507-566
  * rms_norm                  <- _torch_rms_norm, router.py:681-688
  * rms_norm_padded           <- the RMSNorm step of _torch_moe_block_tkg_impl, moe_block_tkg.py:135-151

Tie rule everywhere: equal keys select the lower expert (or group) index,
and the K outputs are ordered by descending key.
Softmax/sigmoid use the deterministic fp32 exp of oracle.mathfn so that the
GPU selector can be compared bit for bit.
"""
import numpy as np

from .mathfn import exp_f32, sigmoid_f32

F = np.float32
SOFTMAX, SIGMOID = 0, 1


def rms_norm(x, gamma, eps):
    """router.py:681-688: fp32 variance/rsqrt, times gamma, cast back by the caller."""
    x = np.asarray(x, dtype=F)
    var = np.mean(x.astype(F) ** 2, axis=-1, keepdims=True, dtype=F)
    return (x * (F(1.0) / np.sqrt(var + F(eps))).astype(F) * np.asarray(gamma, F)).astype(F)


def rms_norm_padded(x, gamma, eps, hidden_actual=None):
    """moe_block_tkg.py:135-151: mean of squares over the first hidden_actual columns; those
    columns become (x * rsqrt(var + eps)) * gamma, the rest 0 (the caller casts back)."""
    x = np.asarray(x, F)
    H = x.shape[-1]
    ha = H if hidden_actual is None else int(hidden_actual)
    var = np.mean(x[..., :ha] ** 2, axis=-1, keepdims=True, dtype=F)
    r = (F(1.0) / np.sqrt((var + F(eps)).astype(F))).astype(F)
    y = np.zeros_like(x)
    y[..., :ha] = ((x[..., :ha] * r).astype(F) * np.asarray(gamma, F).reshape(-1)[:ha]).astype(F)
    return y


def router_logits(x, w_eh, bias=None):
    """logits[t,e] = sum_h x[t,h] * W[e,h] (+bias[e]); operands are bf16 values held in fp32,
    products exact in fp32, fp32 accumulation (F.linear in fp32, router.py:420-424)."""
    out = np.asarray(x, F) @ np.asarray(w_eh, F).T
    if bias is not None:
        out = out + np.asarray(bias, F)[None, :]
    return out.astype(F)


def topk_desc(keys, k):
    """Indices of the k largest entries per row, descending, ties -> lower index."""
    keys = np.asarray(keys)
    order = np.argsort(-keys, axis=-1, kind="stable")
    return order[:, :k].astype(np.int32)


def softmax_rows_f32(v):
    """Softmax over the last axis: exp_f32(v - v_max) / sum, the sum taken left to right."""
    v = np.asarray(v, F)
    m = np.max(v, axis=-1, keepdims=True)
    e = exp_f32((v - m).astype(F))
    s = np.zeros(v.shape[:-1], F)
    for j in range(v.shape[-1]):
        s = (s + e[..., j]).astype(F)
    return (e / s[..., None]).astype(F)


def _activate(v, scoring):
    return softmax_rows_f32(v) if scoring == SOFTMAX else sigmoid_f32(v)


def _renorm(w, eps):
    s = np.zeros(w.shape[0], F)
    for j in range(w.shape[1]):
        s = (s + w[:, j]).astype(F)
    return (w / (s + F(eps)).astype(F)[:, None]).astype(F)


def scatter_dense(ids, w, E):
    T = ids.shape[0]
    aff = np.zeros((T, E), F)
    np.put_along_axis(aff, ids.astype(np.int64), w, axis=1)
    return aff


def route_topk_act(logits, k, scoring=SOFTMAX, renorm=False, eps=0.0, scale=1.0):
    """router.py:384-441 (and moe_block_tkg.py:187-205 with router_pre_norm=False):
    topk on raw logits -> activation on the k selected values -> (optional renorm) -> scatter."""
    logits = np.asarray(logits, F)
    ids = topk_desc(logits, k)
    vals = np.take_along_axis(logits, ids.astype(np.int64), axis=1)
    w = _activate(vals, scoring)
    if renorm:
        w = _renorm(w, eps)
    w = (w * F(scale)).astype(F)
    return ids, w


def route_act_topk_renorm(logits, k, scoring=SOFTMAX, renorm=True, eps=0.0, scale=1.0):
    """router.py:444-504 (always renorm, eps 0) and moe_block_tkg.py:165-185 (router_pre_norm,
    renorm with +1e-20 when norm_topk_prob): activation over all E, topk, optional renorm.
    For softmax the selection key is the raw logit (softmax is strictly increasing in it)."""
    logits = np.asarray(logits, F)
    probs = _activate(logits, scoring)
    key = logits if scoring == SOFTMAX else probs
    ids = topk_desc(key, k)
    w = np.take_along_axis(probs, ids.astype(np.int64), axis=1)
    if renorm:
        w = _renorm(w, eps)
    w = (w * F(scale)).astype(F)
    return ids, w


def route_topk_scatter_act(logits, k, scoring=SOFTMAX):
    """router.py:507-566: top-k of the raw logits scattered into a row of -inf, then the
    activation over the full row (softmax: sum left to right over E; sigmoid(-inf) = 0).
    Returns the dense affinities [T, E]."""
    logits = np.asarray(logits, F)
    ids = topk_desc(logits, k).astype(np.int64)
    full = np.full(logits.shape, -np.inf, F)
    np.put_along_axis(full, ids, np.take_along_axis(logits, ids, axis=1), axis=1)
    if scoring == SOFTMAX:
        m = np.max(full, axis=-1, keepdims=True)
        e = np.where(np.isinf(full), F(0), exp_f32(np.where(np.isinf(full), F(0), full - m)))
        e = e.astype(F)
        s = np.zeros(full.shape[0], F)
        for j in range(full.shape[1]):
            s = (s + e[:, j]).astype(F)
        return (e / s[:, None]).astype(F)
    return np.where(np.isinf(full), F(0), sigmoid_f32(np.where(np.isinf(full), F(0), full)))


def route_grouped(logits, bias, k, n_group, topk_group, scoring=SIGMOID, renorm=True,
                  eps=1e-20, scale=1.0):
    """DeepSeek-V3 grouped routing, restated from the public model definition:
        s = act(logits); c = s + bias (selection only)
        group score g_j = sum of the two largest c in group j (the largest alone if a group has 1 expert)
        keep the topk_group best groups; ids = topk of c over the kept experts
        w = s[ids]; optional renorm w / (sum w + eps); w *= scale
    """
    logits = np.asarray(logits, F)
    T, E = logits.shape
    if E % n_group:
        raise ValueError("E must be divisible by n_group")
    gs = E // n_group
    if topk_group * gs < k:
        raise ValueError("topk_group * group size must be >= top_k")
    s = _activate(logits, scoring)
    c = s if bias is None else (s + np.asarray(bias, F)[None, :]).astype(F)
    cg = c.reshape(T, n_group, gs)
    srt = -np.sort(-cg, axis=-1)
    gscore = srt[..., 0] if gs == 1 else (srt[..., 0] + srt[..., 1]).astype(F)
    gsel = topk_desc(gscore, topk_group)
    keep = np.zeros((T, n_group), bool)
    np.put_along_axis(keep, gsel.astype(np.int64), True, axis=1)
    keep_e = np.repeat(keep, gs, axis=1)
    masked = np.where(keep_e, c, -np.inf).astype(F)
    ids = topk_desc(masked, k)
    w = np.take_along_axis(s, ids.astype(np.int64), axis=1)
    if renorm:
        w = _renorm(w, eps)
    w = (w * F(scale)).astype(F)
    return ids, w
