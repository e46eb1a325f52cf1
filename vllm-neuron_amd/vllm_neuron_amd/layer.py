"""The MoE expert layer as a torch module with the reference layer's forward signature.

Reference: GptOssExperts (vllm_neuron/model/gpt_oss/model_bf16.py:1002-1484,
model_mxfp4.py:1019-1770). forward(hidden_states, positions, is_decode, rank,
rsag_dispatch=False[, residual]) (model_bf16.py:1221-1232, model_mxfp4.py:1362-1377)
dispatches to forward_prefill, which applies the layer's own pre-MoE RMSNorm
(post_attention_layernorm, :1359) before the router, build_blockwise_mapping and
moe_cte (:1347-1484), or to forward_decode, which hands the same norm weight to the
fused moe_block_tkg as gamma (:1274-1307). The MXFP4 layer's prefill also takes the
pre-norm residual, adds it inside the norm, and returns (out, hidden + residual)
(model_mxfp4.py:1584-1609, :1765-1769); its decode returns one tensor.

Here both phases run one HIP pipeline through one C-ABI call (residual add +
RMSNorm + 1x128 quantization fused -> router logits -> top-k -> align -> fp8
gate_up/SiLU -> fp8 down -> combine); the phase only changes the row-tile height,
which the library picks from the average routed rows per expert (T*K/E). The call
is the torch.library operator moe_fp8::layer, an opaque node under torch.compile.
"""
from typing import Optional, Tuple

import torch
from torch import Tensor

from . import ops
from .config import MoEConfig
from .weights import Fp8MoEWeights


@torch.library.custom_op("moe_fp8::layer", mutates_args=())
def moe_layer(x: Tensor, residual: Optional[Tensor], gamma: Optional[Tensor], eps: float,
              hidden_actual: int, router_w: Tensor, router_bias: Optional[Tensor],
              corr_bias: Optional[Tensor], w13: Tensor, w13_scale: Tensor, w2: Tensor,
              w2_scale: Tensor, shared_w13: Optional[Tensor], shared_w13_scale: Optional[Tensor],
              shared_w2: Optional[Tensor], shared_w2_scale: Optional[Tensor], top_k: int,
              grouped: bool, scoring: str, n_group: int, topk_group: int, renorm: bool,
              routed_scaling: float, block_size: int) -> Tuple[Tensor, Tensor]:
    """The whole layer (moe_layer_forward) as one opaque torch.library node.
    Returns (out [T, H] bf16, residual_sum [T, H], or [0, H] without a residual)."""
    w = Fp8MoEWeights(router_w=router_w, w13=w13, w13_scale=w13_scale, w2=w2, w2_scale=w2_scale,
                      router_bias=router_bias, corr_bias=corr_bias, shared_w13=shared_w13,
                      shared_w13_scale=shared_w13_scale, shared_w2=shared_w2,
                      shared_w2_scale=shared_w2_scale)
    cfg = MoEConfig(w.hidden, w.intermediate, w.n_experts, top_k, n_shared=w.n_shared,
                    scoring=scoring, grouped=grouped, n_group=n_group, topk_group=topk_group,
                    renorm=renorm, routed_scaling=routed_scaling, block_size=block_size)
    r = ops.layer_forward(x, w, cfg, gamma=gamma, eps=eps,
                          hidden_actual=None if hidden_actual <= 0 else hidden_actual,
                          residual=residual)
    if residual is None:
        return r, x.new_empty(0, x.shape[1])
    return r


@moe_layer.register_fake
def _moe_layer_fake(x, residual, gamma, eps, hidden_actual, router_w, router_bias, corr_bias,
                    w13, w13_scale, w2, w2_scale, shared_w13, shared_w13_scale, shared_w2,
                    shared_w2_scale, top_k, grouped, scoring, n_group, topk_group, renorm,
                    routed_scaling, block_size):
    T, H = x.shape
    return x.new_empty(T, H), x.new_empty(0 if residual is None else T, H)


class FP8BlockMoE(torch.nn.Module):
    """norm_weight [H] is post_attention_layernorm.weight (GptOssRMSNorm,
    model_bf16.py:103-138: fp32 math over the first hidden_actual columns, the rest
    zeroed, cast back to bf16); eps is rms_norm_eps. Without a norm weight the layer
    takes already-normalized hidden states."""

    def __init__(self, cfg: MoEConfig, weights: Fp8MoEWeights, norm_weight=None, eps=1e-6,
                 hidden_actual=None):
        super().__init__()
        weights.validate()
        if (weights.n_experts, weights.hidden, weights.intermediate) != (
                cfg.n_experts, cfg.hidden, cfg.intermediate):
            raise ValueError("weights do not match the config shape")
        if weights.n_shared != cfg.n_shared:
            raise ValueError(f"config has {cfg.n_shared} shared experts, weights {weights.n_shared}")
        if norm_weight is not None and norm_weight.numel() != cfg.hidden:
            raise ValueError(f"norm_weight must hold hidden={cfg.hidden} values, got "
                             f"{tuple(norm_weight.shape)}")
        if hidden_actual is not None and not 1 <= int(hidden_actual) <= cfg.hidden:
            raise ValueError(f"hidden_actual must be in [1, {cfg.hidden}], got {hidden_actual}")
        self.cfg = cfg
        self.w = weights
        self.rms_norm_eps = float(eps)
        self.hidden_actual = None if hidden_actual is None else int(hidden_actual)
        # a buffer, so module.to(device) moves it with the module
        self.register_buffer(
            "norm_weight", None if norm_weight is None else
            norm_weight.detach().reshape(-1).to(torch.float32).contiguous())

    def forward(self, hidden_states, positions=None, is_decode=False, rank=None,
                rsag_dispatch=False, residual=None):
        # rank is the tensor-parallel rank; with every expert on this GPU (expert-parallel
        # degree 1) the reference's forward does not use it (model_bf16.py:1234-1255).
        if rsag_dispatch:
            raise NotImplementedError("rsag_dispatch needs expert parallelism (one GPU here)")
        x = hidden_states
        lead = x.shape[:-1]
        x2 = x.reshape(-1, x.shape[-1])
        if x2.dtype != torch.bfloat16:
            raise ValueError(f"hidden_states must be bf16, got {x2.dtype}")
        # decode returns one tensor and takes no residual (model_mxfp4.py:1371-1377)
        res = None if (is_decode or residual is None) else residual.reshape(x2.shape)
        if res is not None and self.norm_weight is None:
            raise ValueError("residual is added inside the layer's norm: give norm_weight")
        w, cfg = self.w, self.cfg
        xc, rc = x2.contiguous(), None if res is None else res.contiguous()
        if torch.compiler.is_compiling():
            # one opaque node of the compiled graph
            out, rsum = moe_layer(
                xc, rc, self.norm_weight, self.rms_norm_eps,
                0 if self.hidden_actual is None else self.hidden_actual,
                w.router_w, w.router_bias, w.corr_bias, w.w13, w.w13_scale, w.w2, w.w2_scale,
                w.shared_w13, w.shared_w13_scale, w.shared_w2, w.shared_w2_scale, cfg.top_k,
                cfg.grouped, cfg.scoring, cfg.n_group, cfg.topk_group, cfg.renorm,
                float(cfg.routed_scaling), cfg.block_size)
        else:
            # eager: the operator's body without the dispatcher (about 20 us of host
            # time per call, which a one-token decode step would otherwise wait on)
            r = ops.layer_forward(xc, w, cfg, gamma=self.norm_weight, eps=self.rms_norm_eps,
                                  hidden_actual=self.hidden_actual, residual=rc)
            out, rsum = (r, None) if rc is None else r
        if res is None:
            rsum = None
        if positions is not None and not is_decode:
            # model_bf16.py:1380-1384: tokens after the last real position are padding
            pos = positions.reshape(-1)
            keep = torch.arange(pos.numel(), device=pos.device) <= torch.argmax(pos)
            out = out * keep.to(out.dtype).unsqueeze(1)
        out = out.reshape(*lead, out.shape[-1])
        if rsum is not None:
            return out, rsum.reshape(*lead, rsum.shape[-1])
        return out
