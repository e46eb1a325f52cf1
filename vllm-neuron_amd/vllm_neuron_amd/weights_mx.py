"""MX (microscaling) expert weights: the GPT-OSS MXFP4 checkpoint format.

Per expert the HF GPT-OSS checkpoint holds gate_up_proj_blocks [2I, H/32, 16]
uint8 (two E2M1 codes per byte, the low nibble first; rows interleaved gate 0,
up 0, gate 1, ...), gate_up_proj_scales [2I, H/32] (E8M0 bytes, 2^(b - 127)),
gate_up_proj_bias [2I], and down_proj_blocks [H, I/32, 16], down_proj_scales
[H, I/32], down_proj_bias [H]. The reference converts the same tensors into its
Trainium tiling (model/gpt_oss/weight_loaders_mxfp4.py:301-560), de-interleaving
gate and up and adding +1 to the up bias (:418-464; the bf16 path
weight_loaders_bf16.py:386-419 does the same). The device layout here stacks them
K-contiguous, gate rows first, without changing a code or scale:

    w13 [E, 2I, H/2] uint8   w13_scale [E, 2I, H/32] uint8   b13 [E, 2I] fp32
    w2  [E, H, I/2]  uint8   w2_scale  [E, H, I/32]  uint8   b2  [E, H]  fp32

MXFP8 weights (E4M3 codes, [E, 2I, H] / [E, H, I]) use the same scale layout.
Hidden and intermediate sizes that are not multiples of 256 / 128 are zero-padded
(GPT-OSS pads 2880 to 3072, model_bf16.py:103-138), padded rows and columns
contributing nothing.
"""
from dataclasses import dataclass
from typing import Optional

import torch

FP4_LEVELS = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0)


def quant_fp4_codes(v):
    """float tensor (already scaled into [-6, 6]) -> E2M1 codes (uint8 0..15), round to
    nearest, ties to the code with a zero mantissa bit (the even code)."""
    a = v.abs().clamp(max=6.0)
    mids = torch.tensor([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0], device=v.device, dtype=a.dtype)
    k = (a.unsqueeze(-1) > mids).sum(-1)
    tie = (a.unsqueeze(-1) == mids).any(-1) & (k % 2 == 1)
    k = k + tie.to(k.dtype)
    sign = (torch.signbit(v) & (k > 0)).to(torch.uint8) << 3
    return k.to(torch.uint8) | sign


def quant_mx_weight(w, fmt="fp4"):
    """fp32 [..., O, K] -> (codes, scale bytes [..., O, K/32]) with OCP MX quantization
    along K: e = max(floor(log2(amax)) - emax, -127) (emax 2 for E2M1, 8 for E4M3),
    elements w / 2^e clamped to the format's maximum and rounded to nearest even.
    fp4 codes come packed two per byte (low nibble first): [..., O, K/2]."""
    *lead, O, K = w.shape
    if K % 32:
        raise ValueError("K must be a multiple of 32")
    b = w.float().reshape(*lead, O, K // 32, 32)
    amax = b.abs().amax(-1)
    ef = (amax.view(torch.int32) >> 23) & 0xFF
    emax = 2 if fmt == "fp4" else 8
    e = torch.clamp(ef - 127 - emax, min=-127)
    scaled = b * torch.exp2(-e.float()).unsqueeze(-1)
    if fmt == "fp4":
        codes = quant_fp4_codes(scaled).reshape(*lead, O, K)
        packed = codes[..., 0::2] | (codes[..., 1::2] << 4)
        return packed.contiguous(), (e + 127).to(torch.uint8).contiguous()
    q = scaled.clamp(-448.0, 448.0).to(torch.float8_e4m3fn).reshape(*lead, O, K)
    return q.contiguous(), (e + 127).to(torch.uint8).contiguous()


@dataclass
class MxMoEWeights:
    router_w: torch.Tensor                    # [E, H] bf16
    w13: torch.Tensor                         # [E, 2I, H/2] uint8 (fp4) or [E, 2I, H] e4m3fn
    w13_scale: torch.Tensor                   # [E, 2I, H/32] uint8 (E8M0)
    w2: torch.Tensor                          # [E, H, I/2] uint8 or [E, H, I] e4m3fn
    w2_scale: torch.Tensor                    # [E, H, I/32] uint8
    b13: Optional[torch.Tensor] = None        # [E, 2I] fp32 (up half with +1 for Swish)
    b2: Optional[torch.Tensor] = None         # [E, H] fp32
    router_bias: Optional[torch.Tensor] = None  # [E] fp32
    fmt: str = "fp4"

    @property
    def n_experts(self):
        return self.w13.shape[0]

    @property
    def hidden(self):
        return self.w2.shape[1]

    @property
    def intermediate(self):
        return self.w13.shape[1] // 2

    @property
    def n_shared(self):
        return 0

    def validate(self):
        E, I2 = self.w13.shape[:2]
        H, I = self.hidden, I2 // 2
        per = 2 if self.fmt == "fp4" else 1
        want_dtype = torch.uint8 if self.fmt == "fp4" else torch.float8_e4m3fn
        if self.fmt not in ("fp4", "fp8"):
            raise ValueError(f"fmt must be 'fp4' or 'fp8', got {self.fmt}")
        if self.w13.dtype != want_dtype or self.w2.dtype != want_dtype:
            raise ValueError(f"{self.fmt} expert codes must be {want_dtype}")
        if tuple(self.w13.shape) != (E, I2, H // per) or tuple(self.w2.shape) != (E, H, I // per):
            raise ValueError("w13 must be [E, 2I, H/p], w2 [E, H, I/p] (p = 2 for fp4)")
        if tuple(self.w13_scale.shape) != (E, I2, H // 32) or tuple(self.w2_scale.shape) != (E, H, I // 32):
            raise ValueError("scales must be [E, 2I, H/32] and [E, H, I/32] uint8")
        if self.w13_scale.dtype != torch.uint8 or self.w2_scale.dtype != torch.uint8:
            raise ValueError("MX scales are uint8 E8M0 bytes")
        if self.b13 is not None and tuple(self.b13.shape) != (E, I2):
            raise ValueError("b13 must be [E, 2I]")
        if self.b2 is not None and tuple(self.b2.shape) != (E, H):
            raise ValueError("b2 must be [E, H]")
        if tuple(self.router_w.shape) != (E, H):
            raise ValueError("router_w must be [E, H]")
        return self


def from_hf_gpt_oss(gate_up_blocks, gate_up_scales, gate_up_bias, down_blocks, down_scales,
                    down_bias, router_w, router_bias=None, hidden=None, intermediate=None,
                    up_bias_offset=1.0):
    """HF GPT-OSS expert tensors -> MxMoEWeights (no re-quantization).

    De-interleaves gate and up rows, adds up_bias_offset to the up bias (the
    reference's loaders add 1 for its Swish convention), and zero-pads H / I to
    `hidden` / `intermediate` when given (padded codes and scale bytes 0, padded
    bias 0, so padded rows contribute nothing)."""
    E, I2, HB, _ = gate_up_blocks.shape
    I, H = I2 // 2, HB * 32
    Hp = hidden or H
    Ip = intermediate or I
    dev = gate_up_blocks.device
    w13 = torch.zeros(E, 2 * Ip, Hp // 2, dtype=torch.uint8, device=dev)
    s13 = torch.zeros(E, 2 * Ip, Hp // 32, dtype=torch.uint8, device=dev)
    b13 = torch.zeros(E, 2 * Ip, dtype=torch.float32, device=dev)
    gb = gate_up_blocks.reshape(E, I2, H // 2)
    w13[:, :I, :H // 2] = gb[:, 0::2]
    w13[:, Ip:Ip + I, :H // 2] = gb[:, 1::2]
    s13[:, :I, :H // 32] = gate_up_scales[:, 0::2]
    s13[:, Ip:Ip + I, :H // 32] = gate_up_scales[:, 1::2]
    b13[:, :I] = gate_up_bias[:, 0::2].float()
    b13[:, Ip:Ip + I] = gate_up_bias[:, 1::2].float() + up_bias_offset
    w2 = torch.zeros(E, Hp, Ip // 2, dtype=torch.uint8, device=dev)
    s2 = torch.zeros(E, Hp, Ip // 32, dtype=torch.uint8, device=dev)
    b2 = torch.zeros(E, Hp, dtype=torch.float32, device=dev)
    w2[:, :H, :I // 2] = down_blocks.reshape(E, H, I // 2)
    s2[:, :H, :I // 32] = down_scales
    b2[:, :H] = down_bias.float()
    rw = torch.zeros(E, Hp, dtype=torch.bfloat16, device=router_w.device)
    rw[:, :H] = router_w.to(torch.bfloat16)
    rb = None if router_bias is None else router_bias.float().contiguous()
    return MxMoEWeights(router_w=rw, w13=w13, w13_scale=s13, w2=w2, w2_scale=s2, b13=b13, b2=b2,
                        router_bias=rb, fmt="fp4").validate()
