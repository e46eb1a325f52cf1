"""Expert-MLP / layer oracle (test infrastructure).

* moe_dense_reference  <- _torch_moe_impl, vllm_neuron/functional/moe/moe_cte.py:465-612
                          (all experts over all tokens, einsum, POST_SCALE accumulate in
                          expert order e = 0..E-1, SiLU activation, :558-559, :574-575,
                          :586-588, :603-606). Used on small shapes only.
* moe_sparse_fp8       <- the same math computed per expert on the gathered tokens
                          (non-selected affinities are 0, so the sums are equal), with the
                          fp8 operands the kernels consume: x quantized 1x128, weights
                          dequantized from 128x128 blocks (times optional per-channel
                          scales), SiLU(g)*u requantized 1x128 before the down projection;
                          fp32 accumulation; the shared expert
                          (moe_block_tkg.py:314-316, kernel-only in the reference) added
                          with weight 1.
* topk_reduce          <- _cpu_topk_reduce, vllm_neuron/functional/moe/topk_reduce.py:144-159.
* moe_block_tkg_fp8    <- _torch_moe_block_tkg_impl, vllm_neuron/functional/moe/moe_block_tkg.py:57-303
                          (RMSNorm -> fp32 router -> pre/post-norm selection -> experts on
                          the normalized input, NO_SCALE or POST_SCALE), composed from the
                          functions above and the router oracle.
"""
import numpy as np

from .fp8 import dequant_act_1x128, dequant_weight_128x128, quant_act_1x128

F = np.float32


def bf16_round(x):
    """float32 -> nearest-even bfloat16 value, returned as float32."""
    u = np.asarray(x, F).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(F)


def silu(g):
    g = np.asarray(g, F)
    return (g / (F(1.0) + np.exp(-g).astype(F))).astype(F)


def expert_mlp(xhat, w13hat, w2hat, requant_h=True):
    """One expert on dequantized operands: h = SiLU(x W_g^T) * (x W_u^T); y = h W_d^T.
    w13hat [2I, H] (gate rows first), w2hat [H, I]."""
    I = w13hat.shape[0] // 2
    gu = (np.asarray(xhat, F) @ np.asarray(w13hat, F).T).astype(F)
    h = (silu(gu[:, :I]) * gu[:, I:]).astype(F)
    if requant_h:
        hq, hs = quant_act_1x128(h)
        h = dequant_act_1x128(hq, hs)
    return (h @ np.asarray(w2hat, F).T).astype(F)


def moe_sparse_fp8(x, ids, w, w13_q, w13_s, w2_q, w2_s, shared=None, requant_h=True,
                   experts=None, chan=None):
    """Layer output in fp32 before the final bf16 cast.

    x [T,H] float32 holding bf16 values; ids/w [T,K]; w13_q [E,2I,H] uint8, w13_s [E,2I/128,H/128];
    w2_q [E,H,I] uint8, w2_s [E,H/128,I/128]; shared = (w13_q, w13_s, w2_q, w2_s) of one
    expert, a list of such tuples (their outputs added in list order), or None. ``experts`` optionally restricts the routed experts evaluated (the others
    contribute nothing) so full-size layers can be checked on a subset. ``chan`` = (c13
    [E, 2I], c2 [E, H]) multiplies each routed expert's dequantized weight rows (the
    reference's FP8 per-channel weight scales, moe_cte.py:178-188, moe_tkg.py:87-91).
    """
    x = np.asarray(x, F)
    T, H = x.shape
    E = w13_q.shape[0]
    xq, xs = quant_act_1x128(x)
    xhat = dequant_act_1x128(xq, xs)
    out = np.zeros((T, H), F)
    ids = np.asarray(ids)
    for e in (range(E) if experts is None else sorted(experts)):
        sel = ids == e
        rows = np.nonzero(sel.any(axis=1))[0]
        if rows.size == 0:
            continue
        wt = (np.asarray(w, F) * sel).sum(axis=1)[rows].astype(F)
        w13 = dequant_weight_128x128(w13_q[e], w13_s[e])
        w2 = dequant_weight_128x128(w2_q[e], w2_s[e])
        if chan is not None:
            w13 = (w13 * np.asarray(chan[0][e], F)[:, None]).astype(F)
            w2 = (w2 * np.asarray(chan[1][e], F)[:, None]).astype(F)
        y = expert_mlp(xhat[rows], w13, w2, requant_h)
        out[rows] = (out[rows] + y * wt[:, None]).astype(F)
    for sh in ([] if shared is None else shared if isinstance(shared, list) else [shared]):
        sq13, ss13, sq2, ss2 = sh
        y = expert_mlp(xhat, dequant_weight_128x128(sq13, ss13),
                       dequant_weight_128x128(sq2, ss2), requant_h)
        out = (out + y).astype(F)
    return out


def moe_dense_reference(hidden, affinities_flat, gate_up, down):
    """_torch_moe_impl (moe_cte.py:465-612), POST_SCALE, SiLU, no bias/clamp.
    hidden [T,H]; affinities_flat [T*E,1]; gate_up [E,H,2,I] (NF layout); down [E,I,H]."""
    hidden = np.asarray(hidden, F)
    E = gate_up.shape[0]
    T = affinities_flat.shape[0] // E
    aff = np.asarray(affinities_flat, F).reshape(T, E)
    hidden = hidden[:T]
    gate = np.einsum("th,ehi->eti", hidden, np.asarray(gate_up[:, :, 0, :], F)).astype(F)
    up = np.einsum("th,ehi->eti", hidden, np.asarray(gate_up[:, :, 1, :], F)).astype(F)
    inter = (up * silu(gate)).astype(F)
    nxt = np.einsum("eti,eih->eth", inter, np.asarray(down, F)).astype(F)
    out = np.zeros((T, hidden.shape[1]), F)
    for e in range(E):
        out = (out + nxt[e] * aff[:, e:e + 1]).astype(F)
    return out


def topk_reduce(inp_rows, token_ids_1based, T):
    """_cpu_topk_reduce (topk_reduce.py:144-159): out[t] = sum of rows whose 1-based token id
    is t+1; ids <= 0 go to a discarded bin."""
    H = inp_rows.shape[1]
    out = np.zeros((T + 1, H), F)
    b = np.clip(np.asarray(token_ids_1based, np.int64), 0, None)
    np.add.at(out, b, np.asarray(inp_rows, F))
    return out[1:]


def moe_block_tkg_fp8(x, gamma, eps, w_router_eh, router_bias, k, scoring, pre_norm,
                      norm_topk_prob, post_scale, w13_q, w13_s, w2_q, w2_s, shared=None,
                      hidden_actual=None, logits=None, chan=None):
    """_torch_moe_block_tkg_impl (moe_block_tkg.py:57-303) with fp8 128x128 experts and a
    shared expert of weight 1: RMSNorm (padded columns 0) cast to bf16 -> fp32 router
    matmul (+ bias) -> pre_norm: activation then top-k, else top-k then activation
    (norm_topk_prob: / (sum + 1e-20)) -> experts on the normalized input, NO_SCALE weight
    1 or POST_SCALE affinity. ``logits`` (optional) replaces the router matmul so that a
    selection made from GPU logits can be compared exactly; ``chan`` as moe_sparse_fp8. Returns
    (out fp32 before the final cast, logits, ids, weights)."""
    from .router import (SOFTMAX, rms_norm_padded, route_act_topk_renorm, route_topk_act,
                         router_logits)
    xn = bf16_round(rms_norm_padded(x, gamma, eps, hidden_actual))
    if logits is None:
        logits = router_logits(xn, w_router_eh, router_bias)
    route = route_act_topk_renorm if pre_norm else route_topk_act
    ids, w = route(logits, k, scoring, norm_topk_prob, 1e-20, 1.0)
    if not post_scale:
        w = np.ones_like(w)
    out = moe_sparse_fp8(xn, ids, w, w13_q, w13_s, w2_q, w2_s, shared=shared, chan=chan)
    return out, logits, ids, w

