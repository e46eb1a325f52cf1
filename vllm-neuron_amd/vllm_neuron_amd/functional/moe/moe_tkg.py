"""moe_tkg(): decode expert MLP for given routing, with the reference's signature.

Reference: vllm_neuron/functional/moe/moe_tkg.py:17-196. Token t runs the
experts expert_index[t, :] (selective) or every expert (is_all_expert); each
contributes with weight 1 (NO_SCALE, the default) or expert_affinities[t, e]
(POST_SCALE; in all-expert mode zeroed outside expert_index[t, :] when
mask_unselected_experts). Compute path (all HIP): align-by-expert mapping of
the ids, fp8 1x128 activation quant, fp8 gate_up + SiLU * up, fp8 down,
combine in k order with fp32 accumulation.

Experts are float8_e4m3fn in the reference layout ([E, H, 2, I] / [E, I, H]) or
the checkpoint stacking, with 128x128 fp32 block scales or the reference's FP8
per-channel scales: row quantization [E, 2, I] / [E, H] and static [E, 2, 1] /
[E, 1] (moe_tkg.py:87-91), applied per output column by the GEMM epilogues.
Static activation input scales, MX weights, biases, clamps, non-SiLU
activations, A2A-v layouts and expert-parallel slicing raise
NotImplementedError (activations are quantized dynamically per 1x128 group).
"""
from typing import Optional

import torch
from torch import Tensor

from . import _experts
from .types import ActFnType, ExpertAffinityScaleMode, MoEAllToAllVStrategy


def moe_tkg(
    hidden_input: Tensor,
    expert_gate_up_weights: Tensor,
    expert_down_weights: Tensor,
    expert_affinities: Tensor,
    expert_index: Tensor,
    is_all_expert: bool,
    rank_id: Optional[Tensor] = None,
    expert_gate_up_bias: Optional[Tensor] = None,
    expert_down_bias: Optional[Tensor] = None,
    expert_gate_up_weights_scale: Optional[Tensor] = None,
    expert_down_weights_scale: Optional[Tensor] = None,
    hidden_input_scale: Optional[Tensor] = None,
    expert_gate_up_input_scale: Optional[Tensor] = None,
    expert_down_input_scale: Optional[Tensor] = None,
    mask_unselected_experts: bool = False,
    expert_affinities_eager: Optional[Tensor] = None,
    expert_affinities_scaling_mode: ExpertAffinityScaleMode = ExpertAffinityScaleMode.NO_SCALE,
    activation_fn: ActFnType = ActFnType.SiLU,
    output_dtype: Optional[torch.dtype] = None,
    gate_clamp_upper_limit: Optional[float] = None,
    gate_clamp_lower_limit: Optional[float] = None,
    up_clamp_upper_limit: Optional[float] = None,
    up_clamp_lower_limit: Optional[float] = None,
    output_in_sbuf: bool = False,
    is_all_expert_dynamic: bool = False,
    block_size: Optional[int] = None,
    input_dequant_scale: Optional[Tensor] = None,
    all_to_all_v_strategy: MoEAllToAllVStrategy = MoEAllToAllVStrategy.DISABLED,
) -> Tensor:
    """Output [T, H] in output_dtype (default: hidden_input's dtype)."""
    bad = {
        "expert biases": expert_gate_up_bias is not None or expert_down_bias is not None,
        "static / MX input scales": any(v is not None for v in (
            hidden_input_scale, expert_gate_up_input_scale, expert_down_input_scale,
            input_dequant_scale)),
        "gate/up clamps": any(v is not None for v in (gate_clamp_upper_limit, gate_clamp_lower_limit,
                                                      up_clamp_upper_limit, up_clamp_lower_limit)),
        f"activation {getattr(activation_fn, 'name', activation_fn)}": activation_fn != ActFnType.SiLU,
        f"scaling mode {expert_affinities_scaling_mode.name}": expert_affinities_scaling_mode not in (
            ExpertAffinityScaleMode.NO_SCALE, ExpertAffinityScaleMode.POST_SCALE),
        "all_to_all_v layouts": all_to_all_v_strategy != MoEAllToAllVStrategy.DISABLED,
        "output_in_sbuf": bool(output_in_sbuf),
    }
    bad = [k for k, v in bad.items() if v]
    if bad:
        raise NotImplementedError(f"moe_tkg: {', '.join(bad)} not supported by this build")
    if hidden_input.dim() != 2:
        raise ValueError(f"hidden_input must be [T, H], got {tuple(hidden_input.shape)}")
    E_L, H_w, _ = _experts.weight_dims(expert_gate_up_weights, expert_down_weights)
    T, H = hidden_input.shape
    if H != H_w:
        raise ValueError(f"hidden_input has H={H}, weights H={H_w}")
    if expert_affinities.dim() != 2 or expert_affinities.shape[0] != T:
        raise ValueError(f"expert_affinities must be [T, E], got {tuple(expert_affinities.shape)}")
    if expert_affinities.shape[1] != E_L:
        raise NotImplementedError(
            f"expert_affinities has {expert_affinities.shape[1]} experts, the weights {E_L}: "
            "expert-parallel slicing needs several GPUs; this build keeps every expert on one")
    if rank_id is not None and not torch.compiler.is_compiling() and \
            int(torch.as_tensor(rank_id).reshape(-1)[0]) != 0:
        raise NotImplementedError("rank_id != 0: one GPU holds every expert")
    aff = expert_affinities.float()
    post = expert_affinities_scaling_mode == ExpertAffinityScaleMode.POST_SCALE
    if is_all_expert:
        ids = torch.arange(E_L, device=aff.device, dtype=torch.int32).expand(T, E_L)
        if post:
            wts = aff
            if mask_unselected_experts:
                sel = torch.zeros_like(aff).scatter_(1, expert_index.long(), 1.0)
                wts = aff * sel
        else:
            wts = torch.ones(T, E_L, device=aff.device)
    else:
        if expert_index.dim() != 2 or expert_index.shape[0] != T:
            raise ValueError(f"expert_index must be [T, K], got {tuple(expert_index.shape)}")
        ids = expert_index.to(torch.int32)
        wts = aff.gather(1, ids.long()) if post else torch.ones(ids.shape, device=aff.device)
    od = output_dtype if output_dtype is not None else hidden_input.dtype
    return _moe_tkg_op(hidden_input, expert_gate_up_weights, expert_down_weights,
                       expert_gate_up_weights_scale, expert_down_weights_scale,
                       ids.contiguous(), wts.float().contiguous(), od)


@torch.library.custom_op("moe_fp8::moe_tkg", mutates_args=())
def _moe_tkg_op(hidden_input: Tensor, gate_up: Tensor, down: Tensor,
                gate_up_scale: Optional[Tensor], down_scale: Optional[Tensor], ids: Tensor,
                wts: Tensor, output_dtype: torch.dtype) -> Tensor:
    """Opaque graph node of moe_tkg (arguments checked by moe_tkg): experts ids [T, K]
    weighted by wts [T, K], combined per token in k order."""
    w13, s13, w2, s2, c13, c2 = _experts.routed_weights(gate_up, down, gate_up_scale, down_scale)
    x = _experts.as_bf16(hidden_input).contiguous()
    w = _experts.make_weights(w13, s13, w2, s2, c13, c2)
    out = _experts.routed_forward(x, ids, wts, w)
    return out if output_dtype == torch.bfloat16 else out.to(output_dtype)


@_moe_tkg_op.register_fake
def _moe_tkg_fake(hidden_input, gate_up, down, gate_up_scale, down_scale, ids, wts,
                  output_dtype):
    return hidden_input.new_empty(hidden_input.shape, dtype=output_dtype)
