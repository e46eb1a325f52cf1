"""Seeded synthetic layer inputs (no checkpoints or datasets are available offline).

Seed of every tensor = 1_000_003 * cfg_index + tag, with tags x=1, router=2,
correction bias=3, shared expert=4 (+j), routed expert e=1000+e, so any expert
can be regenerated alone. Distributions: x ~ N(0,1) bf16; router weight
N(0, 0.02) bf16; expert weights N(0, 0.02) fp32 quantized to e4m3fn with
128x128 block scales (amax/448); correction bias N(0, 0.01) fp32.
"""
import math

import torch

from .weights import Fp8MoEWeights, quant_weight_blocks

SEED_STRIDE = 1_000_003


def _gen(device, seed):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def hidden_states(T, H, cfg_index, device="cpu"):
    g = _gen(device, SEED_STRIDE * cfg_index + 1)
    return torch.randn(T, H, generator=g, device=device, dtype=torch.float32).to(torch.bfloat16)


def expert_fp32(cfg_index, e, H, I, device="cpu", tag_base=1000):
    g = _gen(device, SEED_STRIDE * cfg_index + tag_base + e)
    w13 = torch.randn(2 * I, H, generator=g, device=device, dtype=torch.float32) * 0.02
    w2 = torch.randn(H, I, generator=g, device=device, dtype=torch.float32) * 0.02
    return w13, w2


def zipf_router_bias(E, cfg_index, s=1.2, empty_frac=0.10, c=1.0, device="cpu"):
    """Logit bias c*log(p_e) with p ~ Zipf(s) over a seeded expert permutation; the
    last floor(empty_frac*E) experts of the permutation get -1e4 (never selected)."""
    g = _gen("cpu", SEED_STRIDE * cfg_index + 5)
    perm = torch.randperm(E, generator=g)
    n_empty = int(math.floor(empty_frac * E))
    ranks = torch.arange(1, E + 1, dtype=torch.float64)
    p = ranks ** (-s)
    p = p / p.sum()
    bias = torch.empty(E, dtype=torch.float64)
    bias[perm] = c * torch.log(p)
    if n_empty:
        bias[perm[E - n_empty:]] = -1e4
    return bias.float().to(device)


def make_weights(cfg, cfg_index, device="cpu", zipf=False, experts_device=None):
    """Fp8MoEWeights for `cfg`; expert weights are generated and quantized on
    `experts_device` (default `device`) one expert at a time."""
    H, I, E = cfg.hidden, cfg.intermediate, cfg.n_experts
    edev = experts_device or device
    g = _gen("cpu", SEED_STRIDE * cfg_index + 2)
    router_w = (torch.randn(E, H, generator=g) * 0.02).to(torch.bfloat16).to(device)
    corr = None
    if cfg.grouped:
        g3 = _gen("cpu", SEED_STRIDE * cfg_index + 3)
        corr = (torch.randn(E, generator=g3) * 0.01).float().to(device)
    rbias = zipf_router_bias(E, cfg_index, device=device) if zipf else None
    w13 = torch.empty(E, 2 * I, H, dtype=torch.float8_e4m3fn, device=device)
    s13 = torch.empty(E, 2 * I // 128, H // 128, dtype=torch.float32, device=device)
    w2 = torch.empty(E, H, I, dtype=torch.float8_e4m3fn, device=device)
    s2 = torch.empty(E, H // 128, I // 128, dtype=torch.float32, device=device)
    for e in range(E):
        a, b = expert_fp32(cfg_index, e, H, I, edev)
        qa, sa = quant_weight_blocks(a)
        qb, sb = quant_weight_blocks(b)
        w13[e].copy_(qa)
        s13[e].copy_(sa)
        w2[e].copy_(qb)
        s2[e].copy_(sb)
    kw = {}
    if cfg.n_shared:
        sw13, ss13, sw2, ss2 = [], [], [], []
        for j in range(cfg.n_shared):
            a, b = expert_fp32(cfg_index, 100 * j, H, I, edev, tag_base=4)
            qa, sa = quant_weight_blocks(a)
            qb, sb = quant_weight_blocks(b)
            sw13.append(qa)
            ss13.append(sa)
            sw2.append(qb)
            ss2.append(sb)
        kw = dict(shared_w13=torch.stack(sw13).to(device), shared_w13_scale=torch.stack(ss13).to(device),
                  shared_w2=torch.stack(sw2).to(device), shared_w2_scale=torch.stack(ss2).to(device))
    return Fp8MoEWeights(router_w=router_w, w13=w13, w13_scale=s13, w2=w2, w2_scale=s2,
                         router_bias=rbias, corr_bias=corr, **kw).validate()


def make_mx_weights(E, H, I, cfg_index, device="cpu", h_real=None, i_real=None, fmt="fp4",
                    bias=True):
    """MxMoEWeights of E experts at padded sizes H, I whose real sizes are h_real,
    i_real (GPT-OSS: 2880 padded to 3072): N(0, 0.02) fp32 weights on the real block,
    zero in the padding, OCP-quantized per 32 values along K; biases N(0, 0.1) with
    the +1 of the reference's loaders on the up half (zero in the padding); router
    weight N(0, 0.02) bf16 and bias N(0, 0.1). Generated one expert at a time."""
    from .weights_mx import MxMoEWeights, quant_mx_weight
    hr, ir = h_real or H, i_real or I
    per = 2 if fmt == "fp4" else 1
    cdt = torch.uint8 if fmt == "fp4" else torch.float8_e4m3fn
    w13 = torch.empty(E, 2 * I, H // per, dtype=cdt, device=device)
    s13 = torch.empty(E, 2 * I, H // 32, dtype=torch.uint8, device=device)
    w2 = torch.empty(E, H, I // per, dtype=cdt, device=device)
    s2 = torch.empty(E, H, I // 32, dtype=torch.uint8, device=device)
    for e in range(E):
        a, b = expert_fp32(cfg_index, e, hr, ir, device, tag_base=2000)
        full13 = torch.zeros(2 * I, H, device=device)
        full13[:ir, :hr] = a[:ir]
        full13[I:I + ir, :hr] = a[ir:]
        full2 = torch.zeros(H, I, device=device)
        full2[:hr, :ir] = b
        q, s = quant_mx_weight(full13, fmt)
        w13[e].copy_(q)
        s13[e].copy_(s)
        q, s = quant_mx_weight(full2, fmt)
        w2[e].copy_(q)
        s2[e].copy_(s)
    g = _gen("cpu", SEED_STRIDE * cfg_index + 2)
    router_w = torch.zeros(E, H, dtype=torch.bfloat16)
    router_w[:, :hr] = (torch.randn(E, hr, generator=g) * 0.02).to(torch.bfloat16)
    router_b = (torch.randn(E, generator=g) * 0.1).float()
    b13 = b2 = None
    if bias:
        b13 = torch.zeros(E, 2 * I)
        b13[:, :ir] = torch.randn(E, ir, generator=g) * 0.1
        b13[:, I:I + ir] = torch.randn(E, ir, generator=g) * 0.1 + 1.0
        b2 = torch.zeros(E, H)
        b2[:, :hr] = torch.randn(E, hr, generator=g) * 0.1
        b13, b2 = b13.to(device), b2.to(device)
    return MxMoEWeights(router_w=router_w.to(device), w13=w13, w13_scale=s13, w2=w2, w2_scale=s2,
                        b13=b13, b2=b2, router_bias=router_b.to(device), fmt=fmt).validate()
