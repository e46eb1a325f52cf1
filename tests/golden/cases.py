"""Golden-fixture cases for the fused-MoE layer: seeded inputs and the oracle's outputs.

The reference ships no test vectors for this path (its test tree is absent), so the
fixtures are the oracle's outputs on three small layers, frozen in
``tests/golden/*.npz`` by ``make_fixtures.py``:

* ``c0_small``  the reference's CPU-runnable shape: T 64, H 1024, I 512, 8 experts,
                softmax top-2 in the default order (topk, then activation; router.py:384-441)
* ``dsv3_tiny`` DeepSeek-V3 routing on a tiny layer: 16 experts in 4 groups, 2 groups
                kept, sigmoid + correction bias, top-4, renorm (+1e-20), x2.5, 1 shared expert
* ``zipf_tiny`` skewed routing: softmax top-4 over logits biased by c*log(p_e) with p a
                Zipf(1.2) law over a seeded permutation and 2 experts forced empty (-1e4)

Inputs come from numpy's PCG64 generator (``np.random.default_rng``), whose
float32 normal stream is the same on every x86 host, and are quantized by the oracle
(128x128 weight blocks, 1x128 activation groups). The activations and router weights
are stored in the fixture; the expert weights are regenerated from the seed and
checked against a stored SHA-256 digest of their codes and scales.
"""
import hashlib
import os

import numpy as np

from oracle import blockwise as BW
from oracle import fp8 as Q
from oracle import router as R
from oracle.moe import moe_sparse_fp8

HERE = os.path.dirname(os.path.abspath(__file__))
BLOCK = 256  # mapping block size (the reference default, model_bf16.py:1101)

CASES = {
    "c0_small": dict(T=64, H=1024, I=512, E=8, K=2, scoring="softmax", grouped=False,
                     n_group=1, topk_group=1, renorm=False, scale=1.0, n_shared=0, zipf=False,
                     seed=20261),
    "dsv3_tiny": dict(T=40, H=256, I=128, E=16, K=4, scoring="sigmoid", grouped=True,
                      n_group=4, topk_group=2, renorm=True, scale=2.5, n_shared=1, zipf=False,
                      seed=20262),
    "zipf_tiny": dict(T=48, H=256, I=128, E=16, K=4, scoring="softmax", grouped=False,
                      n_group=1, topk_group=1, renorm=True, scale=1.0, n_shared=0, zipf=True,
                      seed=20263),
}


def path(name):
    return os.path.join(HERE, name + ".npz")


def bf16_bits(x):
    """float32 -> bfloat16 bit patterns, round to nearest even (inputs here are finite)."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def bf16_value(bits):
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def gen_inputs(case):
    """Seeded inputs of one case (numpy only)."""
    c = CASES[case]
    T, H, I, E = c["T"], c["H"], c["I"], c["E"]
    rng = np.random.default_rng(c["seed"])
    x_bits = bf16_bits(rng.standard_normal((T, H), dtype=np.float32))
    rw_bits = bf16_bits(rng.standard_normal((E, H), dtype=np.float32) * np.float32(0.02))
    corr = (rng.standard_normal(E, dtype=np.float32) * np.float32(0.01)) if c["grouped"] else None
    bias = None
    if c["zipf"]:
        perm = rng.permutation(E)
        p = np.arange(1, E + 1, dtype=np.float64) ** -1.2
        p /= p.sum()
        b = np.empty(E, np.float64)
        b[perm] = np.log(p)
        b[perm[E - 2:]] = -1e4
        bias = b.astype(np.float32)

    def expert():
        w13 = rng.standard_normal((2 * I, H), dtype=np.float32) * np.float32(0.02)
        w2 = rng.standard_normal((H, I), dtype=np.float32) * np.float32(0.02)
        return Q.quant_weight_128x128(w13) + Q.quant_weight_128x128(w2)

    routed = [expert() for _ in range(E)]
    q13 = np.stack([r[0] for r in routed])
    s13 = np.stack([r[1] for r in routed])
    q2 = np.stack([r[2] for r in routed])
    s2 = np.stack([r[3] for r in routed])
    shared = expert() if c["n_shared"] else None
    return dict(x_bits=x_bits, router_w_bits=rw_bits, corr_bias=corr, router_bias=bias,
                w13=q13, w13_scale=s13, w2=q2, w2_scale=s2, shared=shared)


def weights_digest(inp):
    h = hashlib.sha256()
    arrs = [inp["w13"], inp["w13_scale"], inp["w2"], inp["w2_scale"]]
    if inp["shared"] is not None:
        arrs += list(inp["shared"])
    for a in arrs:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def route(case, logits, corr_bias):
    c = CASES[case]
    sc = R.SOFTMAX if c["scoring"] == "softmax" else R.SIGMOID
    if c["grouped"]:
        return R.route_grouped(logits, corr_bias, c["K"], c["n_group"], c["topk_group"], sc,
                               c["renorm"], 1e-20, c["scale"])
    return R.route_topk_act(logits, c["K"], sc, c["renorm"], 1e-20, c["scale"])


def oracle_outputs(case, inp, logits=None, ids=None, wts=None):
    """Oracle outputs of a case. Given logits (or ids and weights), the later stages start
    from them, so a check can pin each stage on the previous stage's frozen result."""
    x = bf16_value(inp["x_bits"])
    rw = bf16_value(inp["router_w_bits"])
    lg = R.router_logits(x, rw, inp["router_bias"]) if logits is None else logits
    if ids is None:
        ids, wts = route(case, lg, inp["corr_bias"])
    tpid, b2e, cond, counts, inv = BW.mapping_from_ids(ids, CASES[case]["E"], BLOCK)
    xq, xs = Q.quant_act_1x128(x)
    out = moe_sparse_fp8(x, ids, wts, inp["w13"], inp["w13_scale"], inp["w2"], inp["w2_scale"],
                         shared=inp["shared"])
    return dict(logits=lg, ids=ids.astype(np.int32), weights=wts.astype(np.float32),
                token_position_to_id=tpid, block_to_expert=b2e, conditions=cond,
                expert_counts=counts, inv_pos=inv, xq=xq, xs=xs, out=out)


def load(case):
    with np.load(path(case), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}
