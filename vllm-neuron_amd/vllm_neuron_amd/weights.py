"""Expert weight container in the DeepSeek-V3 fp8 checkpoint layout.

Per expert the checkpoint holds gate_proj / up_proj [I, H] and down_proj
[H, I] as float8_e4m3fn with fp32 ``weight_scale_inv`` blocks of 128x128
([ceil(out/128), ceil(in/128)]); dequantization is W = q * S[o//128, i//128].
The device layout stacks them without re-quantizing:

    w13 [E, 2I, H]  (gate rows, then up rows)   w13_scale [E, 2I/128, H/128]
    w2  [E, H, I]                               w2_scale  [E, H/128, I/128]

The checkpoint enumerates fp8 expert tensors per expert as
[gate_w, gate_s, up_w, up_s] (vllm_neuron/utils/weight_loader.py:719-744);
``from_checkpoint_tensors`` takes them in that order. The reference operator
layout gate_up [E, H, 2, I] / down [E, I, H] (moe_cte.py:122-131) is accepted
by ``from_nf_layout`` with a one-time transpose.
"""
from dataclasses import dataclass
from typing import Optional

import torch

FP8 = torch.float8_e4m3fn
FP8_MAX = 448.0
AMAX_FLOOR = 1e-10


def quant_weight_blocks(w):
    """fp32 [..., O, I] -> (e4m3fn codes [..., O, I], fp32 scales [..., O/128, I/128]).

    scale = max(amax, 1e-10) / 448 per 128x128 block; codes = RNE(clamp(w / scale)).
    Used to build synthetic checkpoints; runs wherever ``w`` lives."""
    *lead, O, I = w.shape
    if O % 128 or I % 128:
        raise ValueError("weight dims must be multiples of 128")
    b = w.float().reshape(*lead, O // 128, 128, I // 128, 128)
    amax = b.abs().amax(dim=(-3, -1))
    # A tensor divisor keeps this an IEEE division on the GPU (a Python-scalar
    # divisor becomes a multiply by the rounded reciprocal there).
    s = torch.clamp(amax, min=AMAX_FLOOR) / torch.full_like(amax, FP8_MAX)
    y = (b / s[..., :, None, :, None]).clamp(-FP8_MAX, FP8_MAX)
    return y.to(FP8).reshape(*lead, O, I), s.float()


def dequant_weight_blocks(q, s):
    *lead, O, I = q.shape
    v = q.float().reshape(*lead, O // 128, 128, I // 128, 128)
    return (v * s[..., :, None, :, None]).reshape(*lead, O, I)


@dataclass
class Fp8MoEWeights:
    router_w: torch.Tensor                      # [E, H] bf16 (the reference passes .T = [H, E])
    w13: torch.Tensor                           # [E, 2I, H] e4m3fn
    w13_scale: torch.Tensor                     # [E, 2I/128, H/128] fp32
    w2: torch.Tensor                            # [E, H, I] e4m3fn
    w2_scale: torch.Tensor                      # [E, H/128, I/128] fp32
    router_bias: Optional[torch.Tensor] = None  # [E] fp32, added to the logits (router.py:419-424)
    corr_bias: Optional[torch.Tensor] = None    # [E] fp32, selection-only correction bias
    shared_w13: Optional[torch.Tensor] = None   # [S, 2I, H] e4m3fn
    shared_w13_scale: Optional[torch.Tensor] = None
    shared_w2: Optional[torch.Tensor] = None    # [S, H, I] e4m3fn
    shared_w2_scale: Optional[torch.Tensor] = None
    # Optional per-output-channel weight scales (the reference's FP8 row / static
    # formats, moe_cte.py:178-188, moe_tkg.py:87-91): W = q * block_scale * chan[row],
    # with all-ones block scales. fp32 [E, 2I] / [E, H] (and [S, 2I] / [S, H]).
    w13_chan: Optional[torch.Tensor] = None
    w2_chan: Optional[torch.Tensor] = None
    shared_w13_chan: Optional[torch.Tensor] = None
    shared_w2_chan: Optional[torch.Tensor] = None

    @property
    def n_experts(self):
        return self.w13.shape[0]

    @property
    def hidden(self):
        return self.w13.shape[2]

    @property
    def intermediate(self):
        return self.w13.shape[1] // 2

    @property
    def n_shared(self):
        return 0 if self.shared_w13 is None else self.shared_w13.shape[0]

    def to(self, device):
        kw = {k: (None if v is None else v.to(device)) for k, v in self.__dict__.items()}
        return Fp8MoEWeights(**kw)

    def validate(self):
        E, I2, H = self.w13.shape
        I = I2 // 2
        if self.w13.dtype != FP8 or self.w2.dtype != FP8:
            raise ValueError("expert weights must be float8_e4m3fn")
        if tuple(self.w2.shape) != (E, H, I):
            raise ValueError(f"w2 must be [E, H, I] = {(E, H, I)}, got {tuple(self.w2.shape)}")
        if tuple(self.w13_scale.shape) != (E, I2 // 128, H // 128):
            raise ValueError("w13_scale must be [E, 2I/128, H/128]")
        if tuple(self.w2_scale.shape) != (E, H // 128, I // 128):
            raise ValueError("w2_scale must be [E, H/128, I/128]")
        if tuple(self.router_w.shape) != (E, H) or self.router_w.dtype != torch.bfloat16:
            raise ValueError("router_w must be bf16 [E, H]")
        if self.shared_w13 is not None:
            S = self.shared_w13.shape[0]
            if tuple(self.shared_w13.shape) != (S, I2, H) or tuple(self.shared_w2.shape) != (S, H, I):
                raise ValueError("shared expert weights must be [S, 2I, H] / [S, H, I]")
        for name, t, shape in (("w13_chan", self.w13_chan, (E, I2)), ("w2_chan", self.w2_chan, (E, H)),
                               ("shared_w13_chan", self.shared_w13_chan, (self.n_shared, I2)),
                               ("shared_w2_chan", self.shared_w2_chan, (self.n_shared, H))):
            if t is not None and (tuple(t.shape) != shape or t.dtype != torch.float32):
                raise ValueError(f"{name} must be fp32 {shape}, got {t.dtype} {tuple(t.shape)}")
        return self

    @property
    def has_channel_scales(self):
        return any(t is not None for t in (self.w13_chan, self.w2_chan, self.shared_w13_chan,
                                           self.shared_w2_chan))


def from_checkpoint_tensors(items, n_experts):
    """Stack per-expert checkpoint tensors enumerated [gate_w, gate_s, up_w, up_s] per expert
    (the fp8 DeepSeek enumeration of weight_loader.py:719-744) into (w13, w13_scale)."""
    if len(items) != 4 * n_experts:
        raise ValueError(f"expected 4 tensors per expert, got {len(items)} for {n_experts}")
    w13, s13 = [], []
    for e in range(n_experts):
        gw, gs, uw, us = items[4 * e: 4 * e + 4]
        w13.append(torch.cat([gw, uw], dim=0))
        s13.append(torch.cat([gs, us], dim=0))
    return torch.stack(w13).contiguous(), torch.stack(s13).float().contiguous()


def split_shared_expert(w13, s13, w2, s2, I):
    """A shared expert of intermediate n*I as n experts of intermediate I.

    The MLP is a sum over its intermediate columns, so gate/up rows and down
    columns can be split into n independent experts whose outputs add up."""
    I_sh = w13.shape[0] // 2
    if I_sh % I:
        raise ValueError("shared intermediate must be a multiple of the expert intermediate")
    n = I_sh // I
    g, u = w13[:I_sh], w13[I_sh:]
    gs, us = s13[:I_sh // 128], s13[I_sh // 128:]
    w13s = torch.stack([torch.cat([g[j * I:(j + 1) * I], u[j * I:(j + 1) * I]]) for j in range(n)])
    s13s = torch.stack([torch.cat([gs[j * I // 128:(j + 1) * I // 128],
                                   us[j * I // 128:(j + 1) * I // 128]]) for j in range(n)])
    w2s = torch.stack([w2[:, j * I:(j + 1) * I] for j in range(n)])
    s2s = torch.stack([s2[:, j * I // 128:(j + 1) * I // 128] for j in range(n)])
    return w13s.contiguous(), s13s.contiguous(), w2s.contiguous(), s2s.contiguous()


def from_nf_layout(gate_up, down, gate_up_scale, down_scale):
    """Reference operator layout -> device layout (one-time copy).

    gate_up [E, H, 2, I], gate_up_scale [E, H/128, 2, I/128]; down [E, I, H],
    down_scale [E, I/128, H/128]."""
    E, H, two, I = gate_up.shape
    if two != 2:
        raise ValueError("gate_up must be [E, H, 2, I]")
    w13 = gate_up.permute(0, 2, 3, 1).reshape(E, 2 * I, H).contiguous()
    s13 = gate_up_scale.permute(0, 2, 3, 1).reshape(E, 2 * I // 128, H // 128).contiguous()
    w2 = down.transpose(1, 2).contiguous()
    s2 = down_scale.transpose(1, 2).contiguous()
    return w13, s13.float(), w2, s2.float()
