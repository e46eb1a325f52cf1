"""moe_block_tkg(): fused decode MoE block, with the reference's signature.

Reference: vllm_neuron/functional/moe/moe_block_tkg.py:306-591 (API),
:57-303 (_torch_moe_block_tkg_impl, the math):
  1. RMSNorm over the first hidden_actual columns (fp32), times gamma, cast to
     the input dtype, padded columns 0                        (:135-151)
  2. router logits = norm(x) . W_r in fp32 (+ bias)           (:153-163)
  3. router_pre_norm: activation on all experts, then top-k;
     else top-k, then activation on the k values; norm_topk_prob divides by
     (sum + 1e-20)                                            (:165-205)
  4. experts on norm(x); NO_SCALE adds each selected expert with weight 1,
     POST_SCALE with its affinity, fp32 accumulation          (:225-296)
  5. the shared expert (gate [H, I_sh], up [H, I_sh], down [I_sh, H]) is added
     with weight 1 (kernel-only in the reference, :314-316, :389-391)
Returns (output [T, H], router_logits [T, E] fp32), or output alone when
skip_router_logits; with a residual [T, H] (bf16), the pre-norm sum inp + residual
is normalized and returned last as residual_out (moe_block_tkg.py:421-428).

Compute path (all HIP): moe_rms_norm_quant (bf16 input: residual add, RMSNorm and
the experts' 1x128 quantization in one pass; fp32 input: moe_rms_norm) -> moe_router_logits (bf16 operands, as
the reference's fp32 matmul of bf16 values) -> moe_router_topk -> blockwise
mapping -> fp8 experts -> combine. Routed experts are float8_e4m3fn with
128x128 block scales (expert_gate_up_weights_scale / expert_down_weights_scale
in the block-scale shapes) or the reference's FP8 per-channel scales (row
[E, 2, I] / [E, H], static [E, 2, 1] / [E, 1], moe_tkg.py:87-91, applied per
output column by the GEMM epilogues); floating-point shared-expert weights are quantized
once to the same format. router_mm_dtype is accepted for signature
compatibility; the logits are always accumulated in fp32. The GPU work is one
torch.library operator (moe_fp8::moe_block_tkg), an opaque node under torch.compile.
MX experts (uint8 E8M0 scales: stacked MXFP4 / MXFP8 weights, the GPT-OSS decode
call of model_bf16.py:1274-1307) take expert biases ([E, 2, I], [E, H]), SiLU or
Swish and the gate / up clamps (moe_fp8::moe_block_tkg_mx).
"""
from typing import Optional, Tuple

import torch
from torch import Tensor

from ... import ops
from . import _experts
from .types import ActFnType, ExpertAffinityScaleMode, RouterActFnType


def moe_block_tkg(
    inp: Tensor,
    gamma: Tensor,
    router_weights: Tensor,
    expert_gate_up_weights: Tensor,
    expert_down_weights: Tensor,
    rank_id: Optional[Tensor] = None,
    top_k: int = 1,
    shared_expert_gate_w: Optional[Tensor] = None,
    shared_expert_up_w: Optional[Tensor] = None,
    shared_expert_down_w: Optional[Tensor] = None,
    expert_gate_up_weights_scale: Optional[Tensor] = None,
    expert_down_weights_scale: Optional[Tensor] = None,
    router_bias: Optional[Tensor] = None,
    expert_gate_up_bias: Optional[Tensor] = None,
    expert_down_bias: Optional[Tensor] = None,
    shared_expert_gate_bias: Optional[Tensor] = None,
    shared_expert_up_bias: Optional[Tensor] = None,
    shared_expert_down_bias: Optional[Tensor] = None,
    eps: float = 1e-6,
    router_act_fn: RouterActFnType = RouterActFnType.SIGMOID,
    router_pre_norm: bool = True,
    norm_topk_prob: bool = False,
    expert_affinities_scaling_mode: ExpertAffinityScaleMode = ExpertAffinityScaleMode.NO_SCALE,
    hidden_act_fn: ActFnType = ActFnType.SiLU,
    hidden_act_scale_factor: Optional[float] = None,
    hidden_act_bias: Optional[float] = None,
    gate_clamp_upper_limit: Optional[float] = None,
    gate_clamp_lower_limit: Optional[float] = None,
    up_clamp_upper_limit: Optional[float] = None,
    up_clamp_lower_limit: Optional[float] = None,
    router_mm_dtype=None,
    hidden_actual: Optional[int] = None,
    skip_router_logits: bool = False,
    is_all_expert: bool = False,
    residual: Optional[Tensor] = None,
    expert_gate_up_input_scale: Optional[Tensor] = None,
    expert_down_input_scale: Optional[Tensor] = None,
) -> Tuple[Tensor, ...]:
    """See the module docstring. is_all_expert selects the reference's all-expert
    kernel schedule; the result equals the selective one (unselected experts
    carry zero weight), which is what runs here."""
    if hidden_act_scale_factor is not None or hidden_act_bias is not None:
        raise NotImplementedError(
            "hidden_act_scale_factor and hidden_act_bias are placeholders and must be None.")
    mx = _experts.is_mx_weights(expert_gate_up_weights, expert_gate_up_weights_scale)
    acts = (ActFnType.SiLU, ActFnType.Swish) if mx else (ActFnType.SiLU,)
    bad = {
        "expert biases with fp8 128x128 experts": not mx and (
            expert_gate_up_bias is not None or expert_down_bias is not None),
        "shared-expert biases": any(v is not None for v in (
            shared_expert_gate_bias, shared_expert_up_bias, shared_expert_down_bias)),
        "a shared expert with MX experts": mx and shared_expert_gate_w is not None,
        "STATIC_MX input scales": expert_gate_up_input_scale is not None
            or expert_down_input_scale is not None,
        "fused residual add on float32 input": residual is not None and inp.dtype != torch.bfloat16,
        "gate/up clamps with fp8 128x128 experts": not mx and any(v is not None for v in (
            gate_clamp_upper_limit, gate_clamp_lower_limit, up_clamp_upper_limit,
            up_clamp_lower_limit)),
        f"activation {getattr(hidden_act_fn, 'name', hidden_act_fn)}": hidden_act_fn not in acts,
        f"scaling mode {expert_affinities_scaling_mode.name}": expert_affinities_scaling_mode not in (
            ExpertAffinityScaleMode.NO_SCALE, ExpertAffinityScaleMode.POST_SCALE),
    }
    bad = [k for k, v in bad.items() if v]
    if bad:
        raise NotImplementedError(f"moe_block_tkg: {', '.join(bad)} not supported by this build")
    if router_act_fn not in (RouterActFnType.SOFTMAX, RouterActFnType.SIGMOID):
        raise NotImplementedError(f"Router activation {router_act_fn} is not supported.")
    if (shared_expert_gate_w is None) != (shared_expert_down_w is None) or \
            (shared_expert_gate_w is None) != (shared_expert_up_w is None):
        raise ValueError("shared expert gate, up and down weights must be given together")

    x = inp.reshape(-1, inp.shape[-1]) if inp.dim() == 3 else inp
    if x.dim() != 2:
        raise ValueError(f"inp must be [B, S, H] or [T, H], got {tuple(inp.shape)}")
    T, H = x.shape
    if router_weights.dim() != 2 or router_weights.shape[0] != H:
        raise ValueError(f"router_weights must be [H, E] with H={H}, got "
                         f"{tuple(router_weights.shape)}")
    E_global = router_weights.shape[1]
    if mx:
        E_L, H_w, _ = _experts.mx_dims(expert_gate_up_weights, expert_down_weights)
    else:
        E_L, H_w, _ = _experts.weight_dims(expert_gate_up_weights, expert_down_weights)
    if H_w != H:
        raise ValueError(f"expert weights have H={H_w}, inp H={H}")
    if E_L != E_global:
        raise NotImplementedError(
            f"{E_L} local of {E_global} experts: expert-parallel slicing needs several GPUs; "
            "this build keeps every expert on one")
    if rank_id is not None and not torch.compiler.is_compiling() and \
            int(torch.as_tensor(rank_id).reshape(-1)[0]) != 0:
        raise NotImplementedError("rank_id != 0: one GPU holds every expert")
    if not 1 <= top_k <= E_global:
        raise ValueError(f"top_k must be between 1 and {E_global}, got {top_k}")
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"inp must be bfloat16 or float32, got {x.dtype}")
    r = None
    if residual is not None:
        r = residual.reshape(-1, residual.shape[-1]) if residual.dim() == 3 else residual
        if tuple(r.shape) != (T, H) or r.dtype != torch.bfloat16:
            raise ValueError(f"residual must be bfloat16 [T, H] = [{T}, {H}], got "
                             f"{r.dtype} {tuple(residual.shape)}")
    if mx:
        nan = float("nan")
        lim = lambda v: nan if v is None else float(v)
        out, logits, res_out = _block_tkg_mx_op(
            x, gamma, router_weights, expert_gate_up_weights, expert_down_weights,
            expert_gate_up_weights_scale, expert_down_weights_scale, expert_gate_up_bias,
            expert_down_bias, router_bias, r, int(top_k), float(eps),
            0 if router_act_fn == RouterActFnType.SOFTMAX else 1, bool(router_pre_norm),
            bool(norm_topk_prob),
            expert_affinities_scaling_mode == ExpertAffinityScaleMode.POST_SCALE,
            0 if hidden_actual is None else int(hidden_actual),
            "swish" if hidden_act_fn == ActFnType.Swish else "silu", lim(gate_clamp_lower_limit),
            lim(gate_clamp_upper_limit), lim(up_clamp_lower_limit), lim(up_clamp_upper_limit))
        res = (out,) if skip_router_logits else (out, logits)
        if residual is not None:
            res = res + (res_out.reshape(inp.shape),)
        return res[0] if len(res) == 1 else res
    out, logits, res_out = _block_tkg_op(
        x, gamma, router_weights, expert_gate_up_weights, expert_down_weights,
        expert_gate_up_weights_scale, expert_down_weights_scale, shared_expert_gate_w,
        shared_expert_up_w, shared_expert_down_w, router_bias, r, int(top_k), float(eps),
        0 if router_act_fn == RouterActFnType.SOFTMAX else 1, bool(router_pre_norm),
        bool(norm_topk_prob), expert_affinities_scaling_mode == ExpertAffinityScaleMode.POST_SCALE,
        0 if hidden_actual is None else int(hidden_actual))
    # (output, router_logits[, residual_out]) as the reference's kernel path (:480)
    res = (out,) if skip_router_logits else (out, logits)
    if residual is not None:
        res = res + (res_out.reshape(inp.shape),)
    return res[0] if len(res) == 1 else res


@torch.library.custom_op("moe_fp8::moe_block_tkg", mutates_args=())
def _block_tkg_op(x: Tensor, gamma: Tensor, router_weights: Tensor, gate_up: Tensor,
                  down: Tensor, gate_up_scale: Optional[Tensor], down_scale: Optional[Tensor],
                  shared_gate: Optional[Tensor], shared_up: Optional[Tensor],
                  shared_down: Optional[Tensor], router_bias: Optional[Tensor],
                  residual: Optional[Tensor], top_k: int, eps: float, scoring: int,
                  pre_norm: bool, norm_topk_prob: bool, post_scale: bool,
                  hidden_actual: int) -> Tuple[Tensor, Tensor, Tensor]:
    """Opaque graph node of moe_block_tkg (arguments checked by moe_block_tkg).
    Returns (out [T, H], logits [T, E] fp32, residual_out [T, H] or [0, H])."""
    T, H = x.shape
    ha = None if hidden_actual <= 0 else hidden_actual
    w13, s13, w2, s2, c13, c2 = _experts.routed_weights(gate_up, down, gate_up_scale, down_scale)
    I = w13.shape[1] // 2
    # 1. (residual add, :341, :421-428) RMSNorm, cast back to the input dtype (:135-151).
    # bf16 input: one fused pass that also quantizes the normalized rows for the experts.
    xq = xs = res_out = None
    if x.dtype == torch.bfloat16:
        r = None if residual is None else residual.contiguous()
        xn, xq, xs, res_out = ops.rms_norm_quant(x.contiguous(), gamma, eps, ha, r)
    else:
        xn = ops.rms_norm(x.contiguous(), gamma, eps, ha, out_dtype=x.dtype)
    # 2. fp32 router matmul on the normalized values (:153-163)
    wt = router_weights.t()
    wt = wt if wt.is_contiguous() else wt.contiguous()
    bias = None if router_bias is None else router_bias.reshape(-1).float().contiguous()
    if xn.dtype == torch.bfloat16 and wt.dtype == torch.bfloat16:
        logits = ops.router_logits(xn, wt, bias)
    else:
        if wt.dtype not in (torch.float32, torch.bfloat16):
            wt = wt.float().contiguous()
        logits = ops.router_logits_f32(xn.float().contiguous(), wt, bias)
    # 3. selection (:165-205)
    order = ops.ORDER_ACT_TOPK if pre_norm else ops.ORDER_TOPK_ACT
    ids, wts = ops.router_topk(logits, top_k, order, scoring, renorm=norm_topk_prob, eps=1e-20,
                               scale=1.0)
    if not post_scale:
        wts = torch.ones_like(wts)
    # 4./5. routed experts (+ shared expert) on the normalized values
    shared = None
    if shared_gate is not None:
        shared = _experts.shared_weights(shared_gate, shared_up, shared_down, I)
    w = _experts.make_weights(w13, s13, w2, s2, c13, c2, shared)
    out = _experts.routed_forward(_experts.as_bf16(xn), ids, wts, w, xq=xq, xs=xs)
    if x.dtype != torch.bfloat16:
        out = out.to(x.dtype)
    if res_out is None:
        res_out = x.new_empty(0, H, dtype=torch.bfloat16)
    return out, logits, res_out


@_block_tkg_op.register_fake
def _block_tkg_fake(x, gamma, router_weights, gate_up, down, gate_up_scale, down_scale,
                    shared_gate, shared_up, shared_down, router_bias, residual, top_k, eps,
                    scoring, pre_norm, norm_topk_prob, post_scale, hidden_actual):
    T, H = x.shape
    E = router_weights.shape[1]
    nres = 0 if residual is None or x.dtype != torch.bfloat16 else T
    return (x.new_empty(T, H), x.new_empty(T, E, dtype=torch.float32),
            x.new_empty(nres, H, dtype=torch.bfloat16))


def _norm_route(x, gamma, router_weights, router_bias, residual, top_k, eps, scoring, pre_norm,
                norm_topk_prob, post_scale, ha):
    """Steps 1-3 of the decode block on the GPU (RMSNorm with the residual add, fp32
    router logits, selection): (xn, logits, ids, weights, residual_out)."""
    res_out = None
    if x.dtype == torch.bfloat16 and residual is not None:
        xn, _, _, res_out = ops.rms_norm_quant(x.contiguous(), gamma, eps, ha, residual.contiguous())
    else:
        xn = ops.rms_norm(x.contiguous(), gamma, eps, ha, out_dtype=x.dtype)
    wt = router_weights.t()
    wt = wt if wt.is_contiguous() else wt.contiguous()
    bias = None if router_bias is None else router_bias.reshape(-1).float().contiguous()
    if xn.dtype == torch.bfloat16 and wt.dtype == torch.bfloat16:
        logits = ops.router_logits(xn, wt, bias)
    else:
        if wt.dtype not in (torch.float32, torch.bfloat16):
            wt = wt.float().contiguous()
        logits = ops.router_logits_f32(xn.float().contiguous(), wt, bias)
    order = ops.ORDER_ACT_TOPK if pre_norm else ops.ORDER_TOPK_ACT
    ids, wts = ops.router_topk(logits, top_k, order, scoring, renorm=norm_topk_prob, eps=1e-20,
                               scale=1.0)
    if not post_scale:
        wts = torch.ones_like(wts)
    return xn, logits, ids, wts, res_out


@torch.library.custom_op("moe_fp8::moe_block_tkg_mx", mutates_args=())
def _block_tkg_mx_op(x: Tensor, gamma: Tensor, router_weights: Tensor, gate_up: Tensor,
                     down: Tensor, gate_up_scale: Tensor, down_scale: Tensor,
                     gate_up_bias: Optional[Tensor], down_bias: Optional[Tensor],
                     router_bias: Optional[Tensor], residual: Optional[Tensor], top_k: int,
                     eps: float, scoring: int, pre_norm: bool, norm_topk_prob: bool,
                     post_scale: bool, hidden_actual: int, act: str, gate_lo: float,
                     gate_hi: float, up_lo: float, up_hi: float) -> Tuple[Tensor, Tensor, Tensor]:
    """Opaque graph node of moe_block_tkg with MX experts (GPT-OSS decode,
    model_bf16.py:1274-1307: Swish, clamps, biases). Returns (out, logits,
    residual_out or an empty [0, H])."""
    T, H = x.shape
    ha = None if hidden_actual <= 0 else hidden_actual
    xn, logits, ids, wts, res_out = _norm_route(x, gamma, router_weights, router_bias, residual,
                                                top_k, eps, scoring, pre_norm, norm_topk_prob,
                                                post_scale, ha)
    w = _experts.mx_weights(gate_up, down, gate_up_scale, down_scale, gate_up_bias, down_bias)
    none = lambda v: None if v != v else v
    out = ops.mx_experts(_experts.as_bf16(xn).contiguous(), ids, wts, w, act,
                         (none(gate_lo), none(gate_hi)), (none(up_lo), none(up_hi)))
    if x.dtype != torch.bfloat16:
        out = out.to(x.dtype)
    if res_out is None:
        res_out = x.new_empty(0, H, dtype=torch.bfloat16)
    return out, logits, res_out


@_block_tkg_mx_op.register_fake
def _block_tkg_mx_fake(x, gamma, router_weights, gate_up, down, gate_up_scale, down_scale,
                       gate_up_bias, down_bias, router_bias, residual, top_k, eps, scoring,
                       pre_norm, norm_topk_prob, post_scale, hidden_actual, act, gate_lo, gate_hi,
                       up_lo, up_hi):
    T, H = x.shape
    E = router_weights.shape[1]
    nres = 0 if residual is None or x.dtype != torch.bfloat16 else T
    return (x.new_empty(T, H), x.new_empty(T, E, dtype=torch.float32),
            x.new_empty(nres, H, dtype=torch.bfloat16))
