"""The GPT-OSS MoE expert layer with MXFP4 (or MXFP8) experts, as a torch module.

Reference: GptOssExperts of the MXFP4 model (model/gpt_oss/model_mxfp4.py:1019-1770):
MXFP4 expert weights with biases (loaded with +1 on the up bias,
weight_loaders_mxfp4.py:418-464), softmax top-k routing with a router bias
(model_bf16.py:1362-1370), the pre-MoE RMSNorm over the unpadded hidden size
(GptOssRMSNorm, model_bf16.py:103-138), and the Swish activation with
gate <= limit and 1 - limit <= up <= 1 + limit (model_bf16.py:1296-1302,
:1460-1466; swiglu_limit 7.0, config.py:62). forward(hidden_states, positions,
is_decode, rank, rsag_dispatch=False, residual=None) follows model_mxfp4.py:1362-1377:
prefill with a residual returns (out, hidden + residual), decode one tensor.

The whole layer is one C-ABI call (moe_layer_forward_mx) registered as the
torch.library operator moe_fp8::layer_mx.
"""
from typing import Optional, Tuple

import torch
from torch import Tensor

from . import ops
from .weights_mx import MxMoEWeights


@torch.library.custom_op("moe_fp8::layer_mx", mutates_args=())
def moe_layer_mx(x: Tensor, residual: Optional[Tensor], gamma: Optional[Tensor], eps: float,
                 hidden_actual: int, router_w: Tensor, router_bias: Optional[Tensor], w13: Tensor,
                 w13_scale: Tensor, b13: Optional[Tensor], w2: Tensor, w2_scale: Tensor,
                 b2: Optional[Tensor], fmt: str, top_k: int, act: str, gate_lo: float,
                 gate_hi: float, up_lo: float, up_hi: float, scoring: str,
                 block_size: int) -> Tuple[Tensor, Tensor]:
    """Opaque graph node of the MX layer. NaN limits mean no clamp. Returns (out,
    residual_sum or an empty [0, H])."""
    w = MxMoEWeights(router_w=router_w, w13=w13, w13_scale=w13_scale, w2=w2, w2_scale=w2_scale,
                     b13=b13, b2=b2, router_bias=router_bias, fmt=fmt)
    nan_none = lambda v: None if v != v else v
    r = ops.layer_forward_mx(x, w, top_k, act, (nan_none(gate_lo), nan_none(gate_hi)),
                             (nan_none(up_lo), nan_none(up_hi)), scoring=scoring, gamma=gamma,
                             eps=eps, hidden_actual=None if hidden_actual <= 0 else hidden_actual,
                             residual=residual, block_size=block_size)
    if residual is None:
        return r, x.new_empty(0, x.shape[1])
    return r


@moe_layer_mx.register_fake
def _moe_layer_mx_fake(x, residual, gamma, eps, hidden_actual, router_w, router_bias, w13,
                       w13_scale, b13, w2, w2_scale, b2, fmt, top_k, act, gate_lo, gate_hi,
                       up_lo, up_hi, scoring, block_size):
    T, H = x.shape
    return x.new_empty(T, H), x.new_empty(0 if residual is None else T, H)


class MXFP4MoE(torch.nn.Module):
    """weights: MxMoEWeights (vllm_neuron_amd.weights_mx.from_hf_gpt_oss loads the HF
    GPT-OSS tensors); norm_weight [H]: post_attention_layernorm.weight; hidden_actual:
    the unpadded hidden size (GPT-OSS: 2880 of 3072)."""

    def __init__(self, weights: MxMoEWeights, top_k: int, norm_weight=None, eps=1e-5,
                 hidden_actual=None, act="swish", limit: Optional[float] = 7.0,
                 scoring="softmax", block_size=256):
        super().__init__()
        weights.validate()
        if not 1 <= top_k <= weights.n_experts:
            raise ValueError(f"top_k must be in [1, {weights.n_experts}], got {top_k}")
        if act not in ops.ACT:
            raise NotImplementedError(f"activation {act!r}: 'swish' and 'silu' are supported")
        H = weights.hidden
        if norm_weight is not None and norm_weight.numel() != H:
            raise ValueError(f"norm_weight must hold hidden={H} values")
        self.w = weights
        self.top_k = int(top_k)
        self.act = act
        nan = float("nan")
        # GPT-OSS clamps: gate <= limit, 1 - limit <= up (bias holds the +1) <= 1 + limit
        self.limits = (nan, nan, nan, nan) if limit is None else (nan, float(limit),
                                                                  1.0 - limit, 1.0 + limit)
        self.scoring = scoring
        self.block_size = block_size
        self.rms_norm_eps = float(eps)
        self.hidden_actual = None if hidden_actual is None else int(hidden_actual)
        self.register_buffer(
            "norm_weight", None if norm_weight is None else
            norm_weight.detach().reshape(-1).to(torch.float32).contiguous())

    def forward(self, hidden_states, positions=None, is_decode=False, rank=None,
                rsag_dispatch=False, residual=None):
        if rsag_dispatch:
            raise NotImplementedError("rsag_dispatch needs expert parallelism (one GPU here)")
        x = hidden_states
        lead = x.shape[:-1]
        x2 = x.reshape(-1, x.shape[-1])
        if x2.dtype != torch.bfloat16:
            raise ValueError(f"hidden_states must be bf16, got {x2.dtype}")
        res = None if (is_decode or residual is None) else residual.reshape(x2.shape)
        if res is not None and self.norm_weight is None:
            raise ValueError("residual is added inside the layer's norm: give norm_weight")
        w = self.w
        gl, gh, ul, uh = self.limits
        xc, rc = x2.contiguous(), None if res is None else res.contiguous()
        if torch.compiler.is_compiling():
            # one opaque node of the compiled graph
            out, rsum = moe_layer_mx(
                xc, rc, self.norm_weight, self.rms_norm_eps,
                0 if self.hidden_actual is None else self.hidden_actual,
                w.router_w, w.router_bias, w.w13, w.w13_scale, w.b13, w.w2, w.w2_scale, w.b2,
                w.fmt, self.top_k, self.act, gl, gh, ul, uh, self.scoring, self.block_size)
        else:
            # eager: the operator's body without the dispatcher
            nan_none = lambda v: None if v != v else v
            r = ops.layer_forward_mx(xc, w, self.top_k, self.act, (nan_none(gl), nan_none(gh)),
                                     (nan_none(ul), nan_none(uh)), scoring=self.scoring,
                                     gamma=self.norm_weight, eps=self.rms_norm_eps,
                                     hidden_actual=self.hidden_actual, residual=rc,
                                     block_size=self.block_size)
            out, rsum = (r, None) if rc is None else r
        if positions is not None and not is_decode:
            # model_bf16.py:1380-1384: tokens after the last real position are padding
            pos = positions.reshape(-1)
            keep = torch.arange(pos.numel(), device=pos.device) <= torch.argmax(pos)
            out = out * keep.to(out.dtype).unsqueeze(1)
        out = out.reshape(*lead, out.shape[-1])
        if res is not None:
            return out, rsum.reshape(*lead, rsum.shape[-1])
        return out
