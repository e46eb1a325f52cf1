"""Typed torch wrappers over the C ABI (one per entry point of include/moe_fp8.h).

Each wrapper checks device, dtype and shape, allocates its outputs with torch
(device memory only; the kernels never allocate), and enqueues the HIP kernel
on the current torch stream. CPU tensors are rejected: there is no CPU path.
"""
import ctypes

import numpy as np
import torch

from . import _lib
from ._lib import ptr

ORDER_TOPK_ACT, ORDER_ACT_TOPK, ORDER_GROUPED = 0, 1, 2
SCORING = {"softmax": 0, "sigmoid": 1}
FP8 = torch.float8_e4m3fn
BLOCK_TILES_HEADER = 16  # int32 header of a block-tile list (MOE_BLOCK_TILES_HEADER)


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _need_cuda(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError("vllm_neuron_amd kernels need GPU tensors (no CPU fallback)")


def _need(t, dtype, shape=None, name="tensor"):
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _u8(t):
    return t.view(torch.uint8) if t.dtype == FP8 else t


def num_blocks(T, K, E, B):
    return _lib.load().moe_num_blocks(T, K, E, B)


def use_block_kernels(T, K, E):
    """The layer switches to the 256x256 block kernels above 32 rows per expert on
    average (the measured crossover against every row-tile height)."""
    return -(-T * min(K, E) // E) > 32


def choose_mt(T, K, E):
    avg = -(-T * min(K, E) // E)
    for limit, mt in ((4, 16), (24, 32), (48, 64)):
        if avg <= limit:
            return mt
    return 128


# ---------------------------------------------------------------- router

def router_logits(x, router_w, bias=None):
    """x [T,H] bf16, router_w [E,H] bf16, bias [E] fp32 -> logits [T,E] fp32."""
    _need_cuda(x, router_w, bias)
    T, H = x.shape
    E = router_w.shape[0]
    _need(x, torch.bfloat16, (T, H), "hidden_states")
    _need(router_w, torch.bfloat16, (E, H), "router weight [E, H]")
    if bias is not None:
        _need(bias, torch.float32, (E,), "router_bias")
    out = torch.empty(T, E, device=x.device, dtype=torch.float32)
    lib = _lib.load()
    wsb = lib.moe_router_logits_workspace_bytes(T, H, E)
    ws = torch.empty(max(wsb, 1), device=x.device, dtype=torch.uint8)
    _lib.call("moe_router_logits", ptr(x), ptr(router_w), ptr(bias), T, H, E, ptr(out), ptr(ws),
              wsb, _stream())
    return out


def router_logits_f32(x, router_w, bias=None):
    """x [T,H] fp32, router_w [E,H] fp32 or bf16, bias [E] fp32 -> logits [T,E] fp32
    (fp32 operands, fp32 MFMA)."""
    _need_cuda(x, router_w, bias)
    T, H = x.shape
    E = router_w.shape[0]
    _need(x, torch.float32, (T, H), "hidden_states")
    if router_w.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"router weight must be float32 or bfloat16, got {router_w.dtype}")
    _need(router_w, router_w.dtype, (E, H), "router weight [E, H]")
    if bias is not None:
        _need(bias, torch.float32, (E,), "router_bias")
    out = torch.empty(T, E, device=x.device, dtype=torch.float32)
    lib = _lib.load()
    wsb = lib.moe_router_logits_workspace_bytes(T, H, E)
    ws = torch.empty(max(wsb, 1), device=x.device, dtype=torch.uint8)
    _lib.call("moe_router_logits_f32", ptr(x), ptr(router_w),
              int(router_w.dtype == torch.float32), ptr(bias), T, H, E, ptr(out), ptr(ws), wsb,
              _stream())
    return out


def rms_norm(x, gamma, eps, hidden_actual=None, out_dtype=None):
    """RMSNorm of x [T,H] (bf16 or fp32) with gamma [H]; fp32 math; columns at or
    beyond hidden_actual are 0. Output dtype defaults to x's."""
    _need_cuda(x, gamma)
    T, H = x.shape
    if x.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"hidden_states must be float32 or bfloat16, got {x.dtype}")
    _need(x, x.dtype, (T, H), "hidden_states")
    g = gamma.reshape(-1)
    if g.numel() != H:
        raise ValueError(f"gamma must hold H={H} values, got shape {tuple(gamma.shape)}")
    g = g.to(torch.float32).contiguous()
    od = x.dtype if out_dtype is None else out_dtype
    if od not in (torch.float32, torch.bfloat16):
        raise ValueError(f"out_dtype must be float32 or bfloat16, got {od}")
    ha = H if hidden_actual is None else int(hidden_actual)
    out = torch.empty(T, H, device=x.device, dtype=od)
    _lib.call("moe_rms_norm", ptr(x), int(x.dtype == torch.float32), ptr(g), T, H, ha,
              float(eps), ptr(out), int(od == torch.float32), _stream())
    return out


def rms_norm_quant(x, gamma, eps, hidden_actual=None, residual=None):
    """Fused decode prologue on bf16 x [T,H]: v = x, or bf16(x + residual) when a
    residual is given; xn = RMSNorm(v) (bf16, as rms_norm); q, s = act_quant(xn).
    Returns (xn, q, s, v or None)."""
    _need_cuda(x, gamma, residual)
    T, H = x.shape
    _need(x, torch.bfloat16, (T, H), "hidden_states")
    if residual is not None:
        _need(residual, torch.bfloat16, (T, H), "residual")
    g = gamma.reshape(-1)
    if g.numel() != H:
        raise ValueError(f"gamma must hold H={H} values, got shape {tuple(gamma.shape)}")
    g = g.to(torch.float32).contiguous()
    ha = H if hidden_actual is None else int(hidden_actual)
    xn = torch.empty(T, H, device=x.device, dtype=torch.bfloat16)
    q = torch.empty(T, H, device=x.device, dtype=FP8)
    sc = torch.empty(T, H // 128, device=x.device, dtype=torch.float32)
    v = None if residual is None else torch.empty(T, H, device=x.device, dtype=torch.bfloat16)
    _lib.call("moe_rms_norm_quant", ptr(x), ptr(residual), ptr(g), T, H, ha, float(eps), ptr(xn),
              ptr(v), ptr(_u8(q)), ptr(sc), _stream())
    return xn, q, sc, v


def router_topk(logits, top_k, order, scoring, n_group=1, topk_group=1, corr_bias=None,
                renorm=False, eps=0.0, scale=1.0, dense=False):
    """logits [T,E] fp32 -> ids [T,K] int32, weights [T,K] fp32 (+ affinities [T,E] if dense)."""
    _need_cuda(logits, corr_bias)
    T, E = logits.shape
    _need(logits, torch.float32, (T, E), "logits")
    if corr_bias is not None:
        _need(corr_bias, torch.float32, (E,), "correction bias")
    ids = torch.empty(T, top_k, device=logits.device, dtype=torch.int32)
    w = torch.empty(T, top_k, device=logits.device, dtype=torch.float32)
    aff = torch.empty(T, E, device=logits.device, dtype=torch.float32) if dense else None
    _lib.call("moe_router_topk", ptr(logits), ptr(corr_bias), T, E, top_k, order,
              SCORING[scoring] if isinstance(scoring, str) else int(scoring), n_group, topk_group,
              int(bool(renorm)), float(eps), float(scale), ptr(ids), ptr(w), ptr(aff), _stream())
    return (ids, w, aff) if dense else (ids, w)


# ---------------------------------------------------------------- mapping

def blockwise_mapping(ids=None, affinities=None, n_experts=None, top_k=None, block_size=256,
                      padding_mask=None, check=False):
    """Reference blockwise mapping from ids [T,K] or affinities [T,E]; returns a dict with
    token_position_to_id [N*B], block_to_expert [N], conditions [N], expert_counts [E] and
    inv_pos [T,K] (ids) or affinities_masked [T*E, 1] (affinities)."""
    src = ids if ids is not None else affinities
    if (ids is None) == (affinities is None):
        raise ValueError("give exactly one of ids / affinities")
    _need_cuda(src, padding_mask)
    dev = src.device
    if ids is not None:
        T, K = ids.shape
        E = int(n_experts)
        _need(ids, torch.int32, (T, K), "ids")
    else:
        T, E = affinities.shape
        K = int(top_k)
        _need(affinities, torch.float32, (T, E), "expert_affinities")
    B = int(block_size)
    N = num_blocks(T, K, E, B)
    lib = _lib.load()
    out = {
        "token_position_to_id": torch.empty(N * B, device=dev, dtype=torch.int32),
        "block_to_expert": torch.empty(N, device=dev, dtype=torch.int32),
        "conditions": torch.empty(N, device=dev, dtype=torch.int32),
        "expert_counts": torch.empty(E, device=dev, dtype=torch.int32),
        "num_blocks": N,
    }
    inv = torch.empty(T, K, device=dev, dtype=torch.int32) if ids is not None else None
    aff_m = torch.empty(T * E, 1, device=dev, dtype=torch.float32) if affinities is not None else None
    pm = None
    if padding_mask is not None:
        if tuple(padding_mask.shape) != (T,):
            raise ValueError(f"padding_mask must be [T], got {tuple(padding_mask.shape)}")
        pm = padding_mask.to(torch.uint8).contiguous()
    wsb = lib.moe_mapping_workspace_bytes(T, E)
    ws = torch.empty(wsb, device=dev, dtype=torch.uint8)
    _lib.call("moe_blockwise_mapping", ptr(ids), ptr(affinities), ptr(pm), T, K, E, B, N,
              ptr(out["token_position_to_id"]), ptr(out["block_to_expert"]),
              ptr(out["conditions"]), ptr(out["expert_counts"]), ptr(inv), ptr(aff_m), ptr(ws),
              wsb, _stream())
    if check:
        dropped = ctypes.c_int(0)
        _lib.call("moe_mapping_status", ptr(ws), _stream(), ctypes.byref(dropped))
        if dropped.value:
            raise IndexError(f"{dropped.value} routed (token, expert) pairs do not fit the "
                             f"N*B = {N * B} mapping (or expert ids out of range)")
    if inv is not None:
        out["inv_pos"] = inv
    if aff_m is not None:
        out["affinities_masked"] = aff_m
    return out


def invert_mapping(tpid, b2e, B, T, E):
    _need_cuda(tpid, b2e)
    N = b2e.numel()
    inv = torch.empty(T, E, device=tpid.device, dtype=torch.int32)
    _lib.call("moe_invert_mapping", ptr(tpid), ptr(b2e), N, B, T, E, ptr(inv), _stream())
    return inv


# ---------------------------------------------------------------- quant / GEMM / combine

def act_quant(x):
    """x [R,C] bf16 -> (codes [R,C] e4m3fn, scales [R, C/128] fp32)."""
    _need_cuda(x)
    R, C = x.shape
    _need(x, torch.bfloat16, (R, C), "activations")
    q = torch.empty(R, C, device=x.device, dtype=FP8)
    s = torch.empty(R, C // 128, device=x.device, dtype=torch.float32)
    _lib.call("moe_act_quant_1x128", ptr(x), R, C, ptr(q), ptr(s), _stream())
    return q, s


def build_tiles(tpid, b2e, B, T, K, E, n_shared, mt):
    N = b2e.numel()
    lib = _lib.load()
    max_tiles = lib.moe_max_tiles(T, K, E, N, B, n_shared, mt)
    tiles = torch.empty(max_tiles, 4, device=tpid.device, dtype=torch.int32)
    num = torch.empty(1, device=tpid.device, dtype=torch.int32)
    _lib.call("moe_build_tiles", ptr(tpid), ptr(b2e), N, B, T, E, n_shared, mt, ptr(tiles),
              max_tiles, ptr(num), _stream())
    return tiles, num, max_tiles


def expert_gate_up(xq, xs, w, tpid, NB, tiles, num_tiles, max_tiles, mt):
    T, H = xq.shape
    E, I2, _ = w.w13.shape
    I = I2 // 2
    S = w.n_shared
    P = NB + S * T
    hq = torch.empty(P, I, device=xq.device, dtype=FP8)
    hs = torch.empty(P, I // 128, device=xq.device, dtype=torch.float32)
    _lib.call("moe_expert_gate_up", ptr(_u8(xq)), ptr(xs), T, H, I, E, ptr(_u8(w.w13)),
              ptr(w.w13_scale), ptr(w.w13_chan), ptr(_u8(w.shared_w13)) if S else None,
              ptr(w.shared_w13_scale) if S else None, ptr(w.shared_w13_chan) if S else None, S,
              ptr(tpid), NB, ptr(tiles),
              ptr(num_tiles), max_tiles, mt, ptr(_u8(hq)), ptr(hs), _stream())
    return hq, hs


def expert_down(hq, hs, w, T, NB, tiles, num_tiles, max_tiles, mt):
    E, H, I = w.w2.shape
    S = w.n_shared
    y = torch.empty(hq.shape[0], H, device=hq.device, dtype=torch.bfloat16)
    _lib.call("moe_expert_down", ptr(_u8(hq)), ptr(hs), T, H, I, E, ptr(_u8(w.w2)),
              ptr(w.w2_scale), ptr(w.w2_chan), ptr(_u8(w.shared_w2)) if S else None,
              ptr(w.shared_w2_scale) if S else None, ptr(w.shared_w2_chan) if S else None, S, NB,
              ptr(tiles), ptr(num_tiles),
              max_tiles, mt, ptr(y), _stream())
    return y


def combine(y, inv, wts, T, H, NB, n_shared):
    """out[t] = sum_s wts[t,s] * y[inv[t,s]] + shared rows; inv/wts [T,S] (wts None -> 1)."""
    S = 0 if inv is None else inv.shape[1]
    out = torch.empty(T, H, device=y.device, dtype=torch.bfloat16)
    _lib.call("moe_combine", ptr(y), ptr(inv), ptr(wts), S, T, H, NB, n_shared, ptr(out),
              _stream())
    return out


def build_block_tiles(tpid, b2e, B, T, K, E, n_shared):
    """Tile list of the prefill-sized kernels (up to 256 slots of one expert per tile)."""
    N = b2e.numel()
    lib = _lib.load()
    max_tiles = lib.moe_max_block_tiles(T, K, E, N, B, n_shared)
    tiles = torch.empty(max_tiles * 6, device=tpid.device, dtype=torch.int32)
    # the list's header: the tile count, then the XCD ranges the block kernels read
    num = torch.empty(BLOCK_TILES_HEADER, device=tpid.device, dtype=torch.int32)
    wsb = lib.moe_block_tiles_workspace_bytes(N, max_tiles)
    ws = torch.empty(wsb, device=tpid.device, dtype=torch.uint8)
    _lib.call("moe_build_block_tiles", ptr(tpid), ptr(b2e), N, B, T, E, n_shared, ptr(tiles),
              max_tiles, ptr(num), ptr(ws), wsb, _stream())
    return tiles, num, max_tiles


def expert_gate_up_block(xq, xs, w, tpid, NB, tiles, num_tiles, max_tiles):
    T, H = xq.shape
    E, I2, _ = w.w13.shape
    I = I2 // 2
    S = w.n_shared
    hq = torch.empty(NB + S * T, I, device=xq.device, dtype=FP8)
    hs = torch.empty(NB + S * T, I // 128, device=xq.device, dtype=torch.float32)
    _lib.call("moe_expert_gate_up_block", ptr(_u8(xq)), ptr(xs), T, H, I, E, ptr(_u8(w.w13)),
              ptr(w.w13_scale), ptr(w.w13_chan), ptr(_u8(w.shared_w13)) if S else None,
              ptr(w.shared_w13_scale) if S else None, ptr(w.shared_w13_chan) if S else None, S,
              ptr(tpid), NB, ptr(tiles),
              ptr(num_tiles), max_tiles, ptr(_u8(hq)), ptr(hs), _stream())
    return hq, hs


def expert_down_block(hq, hs, w, T, NB, tiles, num_tiles, max_tiles):
    E, H, I = w.w2.shape
    S = w.n_shared
    y = torch.empty(hq.shape[0], H, device=hq.device, dtype=torch.bfloat16)
    _lib.call("moe_expert_down_block", ptr(_u8(hq)), ptr(hs), T, H, I, E, ptr(_u8(w.w2)),
              ptr(w.w2_scale), ptr(w.w2_chan), ptr(_u8(w.shared_w2)) if S else None,
              ptr(w.shared_w2_scale) if S else None, ptr(w.shared_w2_chan) if S else None, S, NB,
              ptr(tiles), ptr(num_tiles),
              max_tiles, ptr(y), _stream())
    return y


def selftest_fp8_encode(first=0, count=0x43E00001, blocks=4096, device="cuda"):
    """(mismatches, smallest mismatching fp32 pattern or None) of the hardware e4m3fn
    encoder against the integer encoder over fp32 patterns [first, first + count),
    both signs, values up to 448 (the default range is all of them)."""
    out = torch.empty(2 * blocks, device=device, dtype=torch.int32)
    _lib.call("moe_selftest_fp8_encode", first, count, ptr(out), blocks, _stream())
    r = out.cpu().numpy().view(np.uint32)
    n = int(r[:blocks].astype(np.int64).sum())
    mn = int(r[blocks:].min())
    return n, (None if mn == 0xFFFFFFFF else mn)


def selftest_bf16_encode(first=0, count=1 << 31, blocks=4096, device="cuda"):
    """(mismatches, smallest mismatching pattern or None) of the hardware bf16 encoder
    against the integer encoder over fp32 patterns [first, first + count)."""
    out = torch.empty(2 * blocks, device=device, dtype=torch.int32)
    _lib.call("moe_selftest_bf16_encode", first, count, ptr(out), blocks, _stream())
    r = out.cpu().numpy().view(np.uint32)
    n = int(r[:blocks].astype(np.int64).sum())
    mn = int(r[blocks:].min())
    return n, (None if mn == 0xFFFFFFFF else mn)


def selftest_quant_div(mode, first=0, count=1 << 31, blocks=4096, device="cuda"):
    """(mismatches, smallest mismatching index or None) of the quantizers' shared-divisor
    division against the IEEE division: mode 0 over (bf16 amax, bf16 value) pairs,
    mode 1 over random fp32 pairs (indices [first, first + count) of 2^31)."""
    out = torch.empty(2 * blocks, device=device, dtype=torch.int32)
    _lib.call("moe_selftest_quant_div", mode, first, count, ptr(out), blocks, _stream())
    r = out.cpu().numpy().view(np.uint32)
    n = int(r[:blocks].astype(np.int64).sum())
    mn = int(r[blocks:].min())
    return n, (None if mn == 0xFFFFFFFF else mn)


def selftest_mfma(a, b, shape=0):
    """shape 0: a, b [16,128] -> c [16,16] (one 16x16x128 fp8 MFMA);
    shape 1: a, b [32,128] -> c [32,32] (two 32x32x64 fp8 MFMAs)."""
    _need_cuda(a, b)
    n = 16 if shape == 0 else 32
    c = torch.empty(n, n, device=a.device, dtype=torch.float32)
    _lib.call("moe_selftest_mfma_fp8", ptr(_u8(a.contiguous())), ptr(_u8(b.contiguous())), ptr(c),
              shape, _stream())
    return c


# ---------------------------------------------------------------- whole layer

def _no_channel_scales(w):
    if getattr(w, "has_channel_scales", False):
        raise NotImplementedError(
            "the whole-layer entry takes 128x128 block-scaled experts; experts with per-channel "
            "scales run through the operator path (functional.moe.moe_cte / moe_tkg)")


def layer_forward(x, w, cfg, return_routing=False, gamma=None, eps=1e-6, hidden_actual=None,
                  residual=None):
    """Whole layer on the HIP path.

    x [T,H] bf16. gamma [H] (optional): the layer's pre-MoE RMSNorm weight, applied
    to x (after adding residual [T,H] bf16, if given) over its first hidden_actual
    columns; the router and the experts then read the normalized rows.
    Returns out [T,H] bf16; (out, residual_sum) when a residual is given; the
    routing (ids, weights, logits) is appended when return_routing."""
    _need_cuda(x, w.w13, gamma, residual)
    _no_channel_scales(w)
    T, H = x.shape
    _need(x, torch.bfloat16, (T, H), "hidden_states")
    if residual is not None:
        if gamma is None:
            raise ValueError("the residual add is fused into the norm: residual needs gamma")
        _need(residual, torch.bfloat16, (T, H), "residual")
    g = None
    if gamma is not None:
        g = gamma.reshape(-1)
        if g.numel() != H:
            raise ValueError(f"gamma must hold H={H} values, got shape {tuple(gamma.shape)}")
        g = g.to(torch.float32).contiguous()
    E, I = w.n_experts, w.intermediate
    K, S, B = cfg.top_k, w.n_shared, cfg.block_size
    lib = _lib.load()
    wsb = lib.moe_layer_workspace_bytes(T, H, I, E, K, S, B, int(g is not None))
    ws = torch.empty(wsb, device=x.device, dtype=torch.uint8)
    out = torch.empty(T, H, device=x.device, dtype=torch.bfloat16)
    rsum = torch.empty_like(x) if residual is not None else None
    ids = torch.empty(T, K, device=x.device, dtype=torch.int32) if return_routing else None
    wts = torch.empty(T, K, device=x.device, dtype=torch.float32) if return_routing else None
    lg = torch.empty(T, E, device=x.device, dtype=torch.float32) if return_routing else None
    order = ORDER_GROUPED if cfg.grouped else ORDER_TOPK_ACT
    ha = 0 if hidden_actual is None else int(hidden_actual)
    _lib.call("moe_layer_forward", ptr(x), ptr(residual), ptr(g), float(eps), ha, T, H, I, E, K,
              S, ptr(w.router_w), ptr(w.router_bias), ptr(w.corr_bias), order,
              SCORING[cfg.scoring], cfg.n_group, cfg.topk_group, int(cfg.renorm), 1e-20,
              float(cfg.routed_scaling), ptr(_u8(w.w13)), ptr(w.w13_scale), ptr(_u8(w.w2)),
              ptr(w.w2_scale), ptr(_u8(w.shared_w13)) if S else None,
              ptr(w.shared_w13_scale) if S else None, ptr(_u8(w.shared_w2)) if S else None,
              ptr(w.shared_w2_scale) if S else None, B, ptr(out), ptr(rsum), ptr(ids), ptr(wts),
              ptr(lg), ptr(ws), wsb, _stream())
    res = (out,) if residual is None else (out, rsum)
    if return_routing:
        res = res + (ids, wts, lg)
    return res[0] if len(res) == 1 else res


def layer_forward_noalloc(x, w, cfg, return_routing=False, gamma=None, eps=1e-6,
                          hidden_actual=None, residual=None):
    """layer_forward through moe_layer_forward_noalloc: the library's static per-GPU
    scratch replaces the workspace, so only the outputs are allocated here (by the
    caller, in code that must not allocate). Same arguments and results."""
    _need_cuda(x, w.w13, gamma, residual)
    _no_channel_scales(w)
    T, H = x.shape
    _need(x, torch.bfloat16, (T, H), "hidden_states")
    if residual is not None:
        _need(residual, torch.bfloat16, (T, H), "residual")
    g = None
    if gamma is not None:
        g = gamma.reshape(-1).to(torch.float32).contiguous()
        if g.numel() != H:
            raise ValueError(f"gamma must hold H={H} values, got shape {tuple(gamma.shape)}")
    E, I = w.n_experts, w.intermediate
    K, S, B = cfg.top_k, w.n_shared, cfg.block_size
    out = torch.empty(T, H, device=x.device, dtype=torch.bfloat16)
    rsum = torch.empty_like(x) if residual is not None else None
    ids = torch.empty(T, K, device=x.device, dtype=torch.int32) if return_routing else None
    wts = torch.empty(T, K, device=x.device, dtype=torch.float32) if return_routing else None
    lg = torch.empty(T, E, device=x.device, dtype=torch.float32) if return_routing else None
    order = ORDER_GROUPED if cfg.grouped else ORDER_TOPK_ACT
    ha = 0 if hidden_actual is None else int(hidden_actual)
    _lib.call("moe_layer_forward_noalloc", ptr(x), ptr(residual), ptr(g), float(eps), ha, T, H, I,
              E, K, S, ptr(w.router_w), ptr(w.router_bias), ptr(w.corr_bias), order,
              SCORING[cfg.scoring], cfg.n_group, cfg.topk_group, int(cfg.renorm), 1e-20,
              float(cfg.routed_scaling), ptr(_u8(w.w13)), ptr(w.w13_scale), ptr(_u8(w.w2)),
              ptr(w.w2_scale), ptr(_u8(w.shared_w13)) if S else None,
              ptr(w.shared_w13_scale) if S else None, ptr(_u8(w.shared_w2)) if S else None,
              ptr(w.shared_w2_scale) if S else None, B, ptr(out), ptr(rsum), ptr(ids), ptr(wts),
              ptr(lg), _stream())
    res = (out,) if residual is None else (out, rsum)
    if return_routing:
        res = res + (ids, wts, lg)
    return res[0] if len(res) == 1 else res


# ---------------------------------------------------------------- MX experts

MX_FMT = {"fp8": 0, "fp4": 1}
ACT = {"silu": 0, "swish": 1}
NAN = float("nan")


def _lim(v):
    return NAN if v is None else float(v)


def act_quant_mx(x):
    """x [R, C] bf16 -> (MXFP8 codes [R, C] e4m3fn, E8M0 scale bytes [R, C/32] uint8)."""
    _need_cuda(x)
    R, C = x.shape
    _need(x, torch.bfloat16, (R, C), "activations")
    q = torch.empty(R, C, device=x.device, dtype=FP8)
    s = torch.empty(R, C // 32, device=x.device, dtype=torch.uint8)
    _lib.call("moe_act_quant_mx", ptr(x), R, C, ptr(_u8(q)), ptr(s), _stream())
    return q, s


def expert_gate_up_mx(xq, xs, w, tpid, NB, tiles, num_tiles, max_tiles, mt, rows, act="swish",
                      gate_limits=(None, None), up_limits=(None, None)):
    """MX gate_up over row tiles; returns (hq [rows, I] e4m3fn, hs [rows, I/32] uint8)."""
    T, H = xq.shape
    E, I = w.n_experts, w.intermediate
    hq = torch.empty(rows, I, device=xq.device, dtype=FP8)
    hs = torch.empty(rows, I // 32, device=xq.device, dtype=torch.uint8)
    _lib.call("moe_expert_gate_up_mx", ptr(_u8(xq)), ptr(xs), T, H, I, E, MX_FMT[w.fmt],
              ptr(_u8(w.w13)), ptr(w.w13_scale), ptr(w.b13), None, None, None, 0, ptr(tpid), NB,
              ptr(tiles), ptr(num_tiles), max_tiles, mt, ACT[act], _lim(gate_limits[0]),
              _lim(gate_limits[1]), _lim(up_limits[0]), _lim(up_limits[1]), ptr(_u8(hq)), ptr(hs),
              _stream())
    return hq, hs


def expert_down_mx(hq, hs, w, T, NB, tiles, num_tiles, max_tiles, mt):
    E, H, I = w.n_experts, w.hidden, w.intermediate
    y = torch.empty(hq.shape[0], H, device=hq.device, dtype=torch.bfloat16)
    _lib.call("moe_expert_down_mx", ptr(_u8(hq)), ptr(hs), T, H, I, E, MX_FMT[w.fmt],
              ptr(_u8(w.w2)), ptr(w.w2_scale), ptr(w.b2), None, None, None, 0, NB, ptr(tiles),
              ptr(num_tiles), max_tiles, mt, ptr(y), _stream())
    return y


def selftest_mfma_mx(a, sa, b, sb, fmt="fp4"):
    """c[16,16] = (a[16,128] fp8 with scale bytes sa[16,4]) . (b with sb[16,4])^T through
    one scaled MFMA; b is packed fp4 [16,64] uint8 or fp8 [16,128]."""
    _need_cuda(a, sa, b, sb)
    c = torch.empty(16, 16, device=a.device, dtype=torch.float32)
    _lib.call("moe_selftest_mfma_mx", ptr(_u8(a.contiguous())), ptr(sa.contiguous()),
              ptr(_u8(b.contiguous())), ptr(sb.contiguous()), MX_FMT[fmt], ptr(c), _stream())
    return c


def mx_experts(x, ids, wts, w, act="swish", gate_limits=(None, None), up_limits=(None, None),
               block_size=256, xq=None, xs=None):
    """Experts of ids [T, K] weighted by wts [T, K] with MX weights: [T, H] bf16.
    Routed rows are compacted per expert (the mapping's inv holds rows, not slots)."""
    T, K = ids.shape
    E, H = w.n_experts, w.hidden
    m = blockwise_mapping(ids=ids.contiguous(), n_experts=E, top_k=K, block_size=block_size)
    tpid, b2e = m["token_position_to_id"], m["block_to_expert"]
    NB = tpid.numel()
    if xq is None:
        xq, xs = act_quant_mx(x)
    mt = min(choose_mt(T, K, E), 64)  # the MX kernels stop at 64-row tiles (as the layer)
    tiles, num, max_tiles = build_tiles(tpid, b2e, block_size, T, K, E, 0, mt)
    hq, hs = expert_gate_up_mx(xq, xs, w, tpid, NB, tiles, num, max_tiles, mt, NB, act,
                               gate_limits, up_limits)
    y = expert_down_mx(hq, hs, w, T, NB, tiles, num, max_tiles, mt)
    return combine(y, m["inv_pos"], wts.contiguous(), T, H, NB, 0)


def layer_forward_mx(x, w, top_k, act="swish", gate_limits=(None, None), up_limits=(None, None),
                     scoring="softmax", order=ORDER_TOPK_ACT, renorm=False, return_routing=False,
                     gamma=None, eps=1e-6, hidden_actual=None, residual=None, block_size=256):
    """The layer with MX experts (moe_layer_forward_mx): x [T, H] bf16, w MxMoEWeights.
    Returns out [T, H] bf16; (out, residual_sum) with a residual; the routing (ids,
    weights, logits) appended when return_routing."""
    _need_cuda(x, w.w13, gamma, residual)
    T, H = x.shape
    _need(x, torch.bfloat16, (T, H), "hidden_states")
    if residual is not None:
        if gamma is None:
            raise ValueError("the residual add is fused into the norm: residual needs gamma")
        _need(residual, torch.bfloat16, (T, H), "residual")
    g = None
    if gamma is not None:
        g = gamma.reshape(-1).to(torch.float32).contiguous()
        if g.numel() != H:
            raise ValueError(f"gamma must hold H={H} values, got shape {tuple(gamma.shape)}")
    E, I, K = w.n_experts, w.intermediate, int(top_k)
    lib = _lib.load()
    wsb = lib.moe_layer_workspace_bytes(T, H, I, E, K, 0, block_size, int(g is not None))
    ws = torch.empty(wsb, device=x.device, dtype=torch.uint8)
    out = torch.empty(T, H, device=x.device, dtype=torch.bfloat16)
    rsum = torch.empty_like(x) if residual is not None else None
    ids = torch.empty(T, K, device=x.device, dtype=torch.int32) if return_routing else None
    wts = torch.empty(T, K, device=x.device, dtype=torch.float32) if return_routing else None
    lg = torch.empty(T, E, device=x.device, dtype=torch.float32) if return_routing else None
    ha = 0 if hidden_actual is None else int(hidden_actual)
    _lib.call("moe_layer_forward_mx", ptr(x), ptr(residual), ptr(g), float(eps), ha, T, H, I, E, K,
              ptr(w.router_w), ptr(w.router_bias), int(order),
              SCORING[scoring] if isinstance(scoring, str) else int(scoring), int(bool(renorm)),
              1e-20, 1.0, MX_FMT[w.fmt], ptr(_u8(w.w13)), ptr(w.w13_scale), ptr(w.b13),
              ptr(_u8(w.w2)), ptr(w.w2_scale), ptr(w.b2), ACT[act], _lim(gate_limits[0]),
              _lim(gate_limits[1]), _lim(up_limits[0]), _lim(up_limits[1]), block_size, ptr(out),
              ptr(rsum), ptr(ids), ptr(wts), ptr(lg), ptr(ws), wsb, _stream())
    res = (out,) if residual is None else (out, rsum)
    if return_routing:
        res = res + (ids, wts, lg)
    return res[0] if len(res) == 1 else res
