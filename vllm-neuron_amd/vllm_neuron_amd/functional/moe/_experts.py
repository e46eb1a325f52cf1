"""Expert weights at the operator boundary and the expert pipeline over a mapping.

The operator API of the reference passes expert weights per call in its own
layout (gate_up [E, H, 2, I], down [E, I, H]; moe_cte.py:122-131). The HIP
kernels read the DeepSeek-V3 checkpoint stacking (w13 [E, 2I, H], w2 [E, H, I],
128x128 fp32 block scales, or per-output-channel scales), which is K-contiguous.
Both are accepted here; the
reference layout is converted once per weight tensor and the result cached
(a second copy of the experts while the caller keeps the originals: pass the
stacked layout to avoid it).

The key is what the bytes are, not which Python object holds them: the storage
address, the view's offset, shape, strides and dtype, and the version counter
(which views share with their base, so an in-place write through any of them
invalidates the entry). A fresh view of the same parameter on every call (the
reference's decode passes `self.gate_up_proj_weight.reshape(...)`,
model_bf16.py:1278) therefore hits. An entry lives as long as the tensors that
own the storage (a view's base, else the tensor itself): a finalizer on each
owner drops it, so a later tensor allocated at a freed address never hits a
stale entry.
"""
import weakref

import torch

from ... import ops
from ...weights import FP8, Fp8MoEWeights, quant_weight_blocks

_CACHE = {}
_CACHE_MAX = 8
BUILDS = [0]  # conversions run so far (read by the tests)


def _key(*ts):
    return tuple((t.untyped_storage().data_ptr(), t.storage_offset(), tuple(t.shape),
                  tuple(t.stride()), t.dtype, t.device, t._version) if t is not None else None
                 for t in ts)


def _owner(t):
    """The tensor whose lifetime is the storage's: a view's base, else t."""
    return t if t._base is None else t._base


def _drop(key):
    _CACHE.pop(key, None)


def _cached(key, build, sources):
    """build() once per key; the entry is dropped when the owner of any tensor of
    ``sources`` is garbage-collected (before its memory can be handed to another
    tensor)."""
    hit = _CACHE.get(key)
    if hit is None:
        if len(_CACHE) >= _CACHE_MAX:
            _CACHE.pop(next(iter(_CACHE)))
        hit = build()
        BUILDS[0] += 1
        _CACHE[key] = hit
        for t in sources:
            if t is not None:
                weakref.finalize(_owner(t), _drop, key)
    return hit


def _need_fp8(t, name):
    if t.dtype != FP8:
        raise NotImplementedError(
            f"{name} is {t.dtype}: this build runs float8_e4m3fn experts with 128x128 block "
            "scales (quantize with vllm_neuron_amd.weights.quant_weight_blocks)")


def _ones_scale(E, O, I, device):
    return torch.ones(E, O // 128, I // 128, device=device, dtype=torch.float32)


def weight_dims(gate_up, down):
    """(E, H, I) of routed expert weights in either layout, from shapes alone: stacked
    gate_up [E, 2I, H] / down [E, H, I], or reference gate_up [E, H, 2, I] / down
    [E, I, H]."""
    if gate_up.dim() == 3:
        E, I2, H = gate_up.shape
        return E, H, I2 // 2
    if gate_up.dim() != 4 or gate_up.shape[2] != 2:
        raise ValueError(f"gate_up_proj_weight must be [E, H, 2, I] or [E, 2I, H], got "
                         f"{tuple(gate_up.shape)}")
    E, H, _, I = gate_up.shape
    return E, H, I


def _channel_scales(gate_up_scale, down_scale, E, H, I, block13, block2):
    """The reference's FP8 per-channel weight-scale formats as fp32 (c13 [E, 2I],
    c2 [E, H]), or (None, None) when both scales are 128x128 blocks (shapes block13 /
    block2) or absent. Accepted: gate_up [E, 1, 2I] (moe_cte shard_on_block,
    moe_cte.py:178-181: gate channels, then up), [E, 2, I] (moe_tkg row
    quantization, moe_tkg.py:87-88), [E, 2, 1] (moe_tkg static, :88-89), [E, 2I];
    down [E, 1, H] (moe_cte.py:186-188), [E, H] (moe_tkg row, :90), [E, 1] (moe_tkg
    static, :90-91). Both scales must use the same family (block or channel)."""
    def is_block(t, shape):
        return t is None or tuple(t.shape) == shape

    if is_block(gate_up_scale, block13) and is_block(down_scale, block2):
        return None, None

    def chan13(t):
        if t is None:
            return torch.ones(E, 2 * I, device=dev)
        sh = tuple(t.shape)
        if sh in ((E, 1, 2 * I), (E, 2 * I)):
            return t.reshape(E, 2 * I).float()
        if sh in ((E, 2, I), (E, 2, 1)):
            return t.float().expand(E, 2, I).reshape(E, 2 * I)
        raise NotImplementedError(
            f"gate_up_proj_scale {sh}: supported are 128x128 blocks {block13} and the per-channel "
            f"[E, 1, 2I] / [E, 2, I] / [E, 2, 1] (E={E}, I={I})")

    def chan2(t):
        if t is None:
            return torch.ones(E, H, device=dev)
        sh = tuple(t.shape)
        if sh in ((E, 1, H), (E, H)):
            return t.reshape(E, H).float()
        if sh == (E, 1):
            return t.float().expand(E, H)
        raise NotImplementedError(
            f"down_proj_scale {sh}: supported are 128x128 blocks {block2} and the per-channel "
            f"[E, 1, H] / [E, H] / [E, 1] (E={E}, H={H})")

    dev = (gate_up_scale if gate_up_scale is not None else down_scale).device
    if (gate_up_scale is not None and tuple(gate_up_scale.shape) == block13) or \
            (down_scale is not None and tuple(down_scale.shape) == block2):
        raise NotImplementedError("gate_up and down scales mix 128x128 blocks and per-channel scales")
    return chan13(gate_up_scale).contiguous(), chan2(down_scale).contiguous()


def routed_weights(gate_up, down, gate_up_scale=None, down_scale=None):
    """(w13, w13_scale, w2, w2_scale, w13_chan, w2_chan) in the kernels' layout from either
    layout.

    Stacked: gate_up [E, 2I, H], down [E, H, I]; reference: gate_up [E, H, 2, I], down
    [E, I, H] (moe_cte.py:122-131). Scales are 128x128 blocks (stacked [E, 2I/128, H/128]
    / [E, H/128, I/128]; reference [E, H/128, 2, I/128] / [E, I/128, H/128]), in which
    case the channel scales are None, or the reference's FP8 per-channel formats (see
    _channel_scales), in which case the block scales are ones and the channel scales
    carry them. Missing scales mean 1.0 (codes used as values)."""
    _need_fp8(gate_up, "gate_up_proj_weight")
    _need_fp8(down, "down_proj_weight")
    dev = gate_up.device
    if gate_up.dim() == 3:
        E, I2, H = gate_up.shape
        I = I2 // 2
        if tuple(down.shape) != (E, H, I):
            raise ValueError(f"down_proj_weight must be [E, H, I] = {(E, H, I)} for a stacked "
                             f"gate_up [E, 2I, H], got {tuple(down.shape)}")
        c13, c2 = _channel_scales(gate_up_scale, down_scale, E, H, I, (E, I2 // 128, H // 128),
                                  (E, H // 128, I // 128))
        if c13 is not None:
            return (gate_up.contiguous(), _ones_scale(E, I2, H, dev), down.contiguous(),
                    _ones_scale(E, H, I, dev), c13, c2)
        s13 = gate_up_scale if gate_up_scale is not None else _ones_scale(E, I2, H, dev)
        s2 = down_scale if down_scale is not None else _ones_scale(E, H, I, dev)
        return (gate_up.contiguous(), s13.float().contiguous(), down.contiguous(),
                s2.float().contiguous(), None, None)
    if gate_up.dim() != 4 or gate_up.shape[2] != 2:
        raise ValueError(f"gate_up_proj_weight must be [E, H, 2, I] or [E, 2I, H], got "
                         f"{tuple(gate_up.shape)}")
    E, H, _, I = gate_up.shape
    if tuple(down.shape) != (E, I, H):
        raise ValueError(f"down_proj_weight must be [E, I, H] = {(E, I, H)}, got "
                         f"{tuple(down.shape)}")
    c13, c2 = _channel_scales(gate_up_scale, down_scale, E, H, I, (E, H // 128, 2, I // 128),
                              (E, I // 128, H // 128))
    if c13 is None:
        gate_up_block, down_block = gate_up_scale, down_scale
    else:
        gate_up_block = down_block = None

    def build():
        w13 = gate_up.permute(0, 2, 3, 1).reshape(E, 2 * I, H).contiguous()
        if gate_up_block is None:
            s13 = _ones_scale(E, 2 * I, H, dev)
        else:
            s13 = gate_up_block.permute(0, 2, 3, 1).reshape(E, 2 * I // 128, H // 128)
        w2 = down.transpose(1, 2).contiguous()
        s2 = _ones_scale(E, H, I, dev) if down_block is None else down_block.transpose(1, 2)
        return w13, s13.float().contiguous(), w2, s2.float().contiguous(), c13, c2

    srcs = (gate_up, down, gate_up_scale, down_scale)
    return _cached(("nf",) + _key(*srcs), build, srcs)


def shared_weights(gate_w, up_w, down_w, I):
    """A shared expert given as gate [H, I_sh], up [H, I_sh], down [I_sh, H]
    (moe_block_tkg.py:314-316) as n = I_sh / I stacked experts of intermediate I.

    Floating-point weights are quantized once to e4m3fn with 128x128 block
    scales (amax / 448, round-to-nearest-even), and cached; fp8 weights are
    taken with unit scales."""
    H, I_sh = gate_w.shape
    if tuple(up_w.shape) != (H, I_sh) or tuple(down_w.shape) != (I_sh, H):
        raise ValueError("shared expert weights must be gate [H, I], up [H, I], down [I, H]")
    if I_sh % I:
        raise ValueError(f"shared intermediate {I_sh} must be a multiple of the expert "
                         f"intermediate {I}")

    def build():
        w13 = torch.cat([gate_w.t(), up_w.t()], dim=0)  # [2 I_sh, H]
        w2 = down_w.t()                                  # [H, I_sh]
        if w13.dtype == FP8:
            q13, s13 = w13.contiguous(), torch.ones(2 * I_sh // 128, H // 128,
                                                    device=w13.device)
            q2, s2 = w2.contiguous(), torch.ones(H // 128, I_sh // 128, device=w2.device)
        else:
            q13, s13 = quant_weight_blocks(w13.float())
            q2, s2 = quant_weight_blocks(w2.float())
        n = I_sh // I
        g, u = q13[:I_sh], q13[I_sh:]
        gs, us = s13[:I_sh // 128], s13[I_sh // 128:]
        w13s = torch.stack([torch.cat([g[j * I:(j + 1) * I], u[j * I:(j + 1) * I]])
                            for j in range(n)])
        s13s = torch.stack([torch.cat([gs[j * I // 128:(j + 1) * I // 128],
                                       us[j * I // 128:(j + 1) * I // 128]]) for j in range(n)])
        w2s = torch.stack([q2[:, j * I:(j + 1) * I] for j in range(n)])
        s2s = torch.stack([s2[:, j * I // 128:(j + 1) * I // 128] for j in range(n)])
        return (w13s.contiguous(), s13s.float().contiguous(), w2s.contiguous(),
                s2s.float().contiguous())

    srcs = (gate_w, up_w, down_w)
    return _cached(("shared", I) + _key(*srcs), build, srcs)


def make_weights(w13, s13, w2, s2, c13=None, c2=None, shared=None):
    """Fp8MoEWeights of routed experts (with optional channel scales c13 / c2) and
    optional shared experts (w13, s13, w2, s2); shared experts without channel scales
    get unit ones when the routed experts have them."""
    kw = {}
    if shared is not None:
        kw = dict(shared_w13=shared[0], shared_w13_scale=shared[1], shared_w2=shared[2],
                  shared_w2_scale=shared[3])
    return Fp8MoEWeights(router_w=None, w13=w13, w13_scale=s13, w2=w2, w2_scale=s2,
                         w13_chan=c13, w2_chan=c2, **kw)


def as_bf16(x):
    """Activations enter the fp8 quantizer as bf16."""
    return x if x.dtype == torch.bfloat16 else x.to(torch.bfloat16)


def run_experts(x_bf16, tpid, b2e, B, k_rows, k_bound, w, xq=None, xs=None):
    """gate_up -> SiLU * up -> down for every slot of a blockwise mapping.

    x_bf16 [T, H]; tpid [N*B] int32 (slot -> token, -1 or >= T for padding);
    b2e [N] int32. k_rows is the expected routed rows per token (picks the tile
    height), k_bound an upper bound on them (sizes the tile list). Returns
    (y [N*B + n_shared*T, H] bf16, N*B). xq/xs: x's 1x128 codes and scales when
    already computed (the fused norm prologue)."""
    T = x_bf16.shape[0]
    E, S = w.n_experts, w.n_shared
    N = b2e.numel()
    NB = N * B
    if xq is None:
        xq, xs = ops.act_quant(x_bf16)
    if ops.use_block_kernels(T, k_rows, E):
        tiles, num, mbt = ops.build_block_tiles(tpid, b2e, B, T, k_bound, E, S)
        hq, hs = ops.expert_gate_up_block(xq, xs, w, tpid, NB, tiles, num, mbt)
        y = ops.expert_down_block(hq, hs, w, T, NB, tiles, num, mbt)
    else:
        mt = ops.choose_mt(T, k_rows, E)
        tiles, num, max_tiles = ops.build_tiles(tpid, b2e, B, T, k_bound, E, S, mt)
        hq, hs = ops.expert_gate_up(xq, xs, w, tpid, NB, tiles, num, max_tiles, mt)
        y = ops.expert_down(hq, hs, w, T, NB, tiles, num, max_tiles, mt)
    return y, NB


def routed_forward(x_bf16, ids, wts, w, block_size=256, xq=None, xs=None):
    """Experts of ids [T, K] int32 weighted by wts [T, K] fp32 (+ the shared
    experts of w, weight 1), combined per token in k order: [T, H] bf16."""
    T, K = ids.shape
    E, H = w.n_experts, w.hidden
    m = ops.blockwise_mapping(ids=ids.contiguous(), n_experts=E, top_k=K, block_size=block_size)
    y, NB = run_experts(x_bf16, m["token_position_to_id"], m["block_to_expert"], block_size, K, K,
                        w, xq, xs)
    return ops.combine(y, m["inv_pos"], wts.contiguous(), T, H, NB, w.n_shared)


# ---------------------------------------------------------------- MX experts

def is_mx_weights(gate_up, gate_up_scale):
    """MX experts are uint8 (packed fp4) or float8_e4m3fn codes with uint8 E8M0 scales."""
    return gate_up_scale is not None and gate_up_scale.dtype == torch.uint8


def mx_weights(gate_up, down, gate_up_scale, down_scale, gate_up_bias=None, down_bias=None):
    """MxMoEWeights from the stacked MX layout: gate_up [E, 2I, H/2] uint8 (fp4) or
    [E, 2I, H] float8_e4m3fn (fp8) with scales [E, 2I, H/32] uint8; down [E, H, I/2] or
    [E, H, I] with [E, H, I/32]; biases [E, 2, I] (the reference's shape) or [E, 2I],
    and [E, 1, H] or [E, H]. The reference's Trainium-tiled uint16 layout is refused
    (load the HF checkpoint with weights_mx.from_hf_gpt_oss instead)."""
    from ...weights_mx import MxMoEWeights
    if gate_up.dtype == torch.uint16 or down.dtype == torch.uint16:
        raise NotImplementedError(
            "MX weights in the Trainium-tiled uint16 layout: pass the stacked layout "
            "(vllm_neuron_amd.weights_mx.from_hf_gpt_oss converts the HF checkpoint)")
    if gate_up.dim() != 3 or down.dim() != 3:
        raise ValueError(f"MX gate_up must be [E, 2I, H/2] (fp4) or [E, 2I, H] (fp8), got "
                         f"{tuple(gate_up.shape)}")
    fmt = "fp4" if gate_up.dtype == torch.uint8 else "fp8"
    if fmt == "fp8" and gate_up.dtype != FP8:
        raise ValueError(f"MX expert codes must be uint8 (fp4) or float8_e4m3fn, got {gate_up.dtype}")
    if down_scale is None or down_scale.dtype != torch.uint8:
        raise ValueError("MX down_proj_scale must be uint8 E8M0 bytes")
    E, I2 = gate_up.shape[:2]
    H = down.shape[1]
    b13 = None if gate_up_bias is None else gate_up_bias.reshape(E, I2).float().contiguous()
    b2 = None if down_bias is None else down_bias.reshape(E, H).float().contiguous()
    w = MxMoEWeights(router_w=gate_up.new_empty(E, H, dtype=torch.bfloat16), w13=gate_up.contiguous(),
                     w13_scale=gate_up_scale.contiguous(), w2=down.contiguous(),
                     w2_scale=down_scale.contiguous(), b13=b13, b2=b2, fmt=fmt)
    w.validate()
    return w


def mx_dims(gate_up, down):
    """(E, H, I) of stacked MX weights from shapes alone."""
    E, I2 = gate_up.shape[:2]
    return E, down.shape[1], I2 // 2
