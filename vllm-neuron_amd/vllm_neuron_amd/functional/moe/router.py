"""router(): MoE expert selection with the reference's signature and validation.

Reference: vllm_neuron/functional/moe/router.py:72-298 (dispatcher),
:19-69 (RouterComputationOrder), :384-566 (the three computation orders),
:569-599 (_apply_activation), :602-678 (_validate_router_inputs),
:681-688 (_torch_rms_norm).

Compute path (all HIP): optional RMSNorm (moe_rms_norm), logits
(moe_router_logits on bf16 operands when they are bf16-exact, else
moe_router_logits_f32 on fp32 operands), then top-k + activation + dense
scatter (moe_router_topk). The reference casts hidden_states to
computation_dtype first (router.py:236), so with computation_dtype float32 a
bf16 input keeps bf16-exact operands unless gamma normalizes it in fp32.
With computation_dtype bfloat16 / float16 the logits are rounded to that type
before selection and the affinities are returned in it (F.linear and the
activation produce that dtype in the reference).

Kernel-only layout hints of the reference (shard_on_tokens, x_sb_layout,
use_column_tiling, use_indirect_dma_scatter, use_PE_broadcast_w_bias) are
accepted and have no effect.
"""
from enum import Enum
from typing import Callable, Optional, Tuple, Union

import torch
from torch import Tensor

from ... import ops


class RouterComputationOrder(Enum):
    """Order of the routing steps (router.py:19-69).

    PRENORM_LINEAR_TOPK_ACT_SCATTER: RMSNorm? -> linear -> top-k -> activation on the
        k values -> scatter.
    PRENORM_LINEAR_ACT_TOPK_RENORM_SCATTER: RMSNorm? -> linear -> activation on all
        experts -> top-k -> L1 renorm (no epsilon) -> scatter.
    PRENORM_LINEAR_TOPK_SCATTER_ACT: RMSNorm? -> linear -> top-k -> scatter the raw
        values into -inf -> activation on the full row.
    """

    PRENORM_LINEAR_TOPK_ACT_SCATTER = "prenorm_linear_topk_act_scatter"
    PRENORM_LINEAR_ACT_TOPK_RENORM_SCATTER = "prenorm_linear_act_topk_renorm_scatter"
    PRENORM_LINEAR_TOPK_SCATTER_ACT = "prenorm_linear_topk_scatter_act"


_SUPPORTED_DTYPES = (torch.float32, torch.float16, torch.bfloat16)


def _validate_router_inputs(hidden_states, router_weights, top_k, router_bias, gamma,
                            computation_dtype, router_computation_order,
                            transposed_hidden_states):
    """Same checks and ValueError messages as router.py:602-678."""
    if hidden_states.dim() != 2:
        raise ValueError(
            f"Expected hidden_states to be 2D [T, H], got shape {hidden_states.shape}")
    if router_weights.dim() != 2:
        raise ValueError(
            f"Expected router_weights to be 2D [H, E], got shape {router_weights.shape}")
    if transposed_hidden_states:
        H, T = hidden_states.shape
    else:
        T, H = hidden_states.shape
    H_w, E = router_weights.shape
    if H != H_w:
        raise ValueError(
            f"Hidden dimension mismatch: hidden_states has {H}, router_weights has {H_w}")
    if router_bias is not None and router_bias.shape != (E,):
        raise ValueError(f"Expected router_bias shape [E], got {router_bias.shape}")
    if gamma is not None and gamma.shape != (H,):
        raise ValueError(f"Expected gamma shape [H], got {gamma.shape}")
    if top_k < 1 or top_k > E:
        raise ValueError(f"top_k must be between 1 and {E}, got {top_k}")
    if computation_dtype not in _SUPPORTED_DTYPES:
        raise ValueError(
            f"computation_dtype must be one of {set(_SUPPORTED_DTYPES)}, got {computation_dtype}")
    if not isinstance(router_computation_order, RouterComputationOrder):
        raise ValueError(
            "router_computation_order must be a RouterComputationOrder enum, got "
            f"{type(router_computation_order)}")


def _scoring(activation):
    """'softmax' / 'sigmoid' -> kernel scoring code (router.py:569-599 semantics)."""
    if isinstance(activation, str):
        if activation in ops.SCORING:
            return ops.SCORING[activation]
        raise ValueError(
            f"Unsupported activation function: {activation}. Use 'softmax' or 'sigmoid'.")
    if callable(activation):
        raise NotImplementedError(
            "callable router activations run arbitrary host code; this build's router "
            "kernels implement 'softmax' and 'sigmoid'")
    raise ValueError(
        "Activation must be either a string ('softmax' or 'sigmoid') or a callable function. "
        f"Got: {type(activation)}")


def router_logits(hidden_states, router_weights, router_bias=None, gamma=None, eps=1e-6,
                  computation_dtype=torch.float32):
    """Logits [T, E] fp32 of router() (its RMSNorm and linear steps), on the GPU.

    hidden_states [T, H]; router_weights [H, E] as the reference passes them
    (used without a copy when they are the transpose view of a contiguous
    [E, H] parameter)."""
    x = hidden_states.to(computation_dtype)
    if gamma is not None:
        if x.dtype == torch.float16:
            # fp32 norm, then the fp16 rounding _torch_rms_norm's cast back applies
            x = ops.rms_norm(x.float().contiguous(), gamma, eps).half()
        else:
            x = ops.rms_norm(x.contiguous(), gamma, eps)  # output in x's dtype (router.py:681-688)
    wt = router_weights.t()
    if not wt.is_contiguous():
        wt = wt.contiguous()
    bias = None if router_bias is None else router_bias.to(computation_dtype).float().contiguous()
    if x.dtype == torch.bfloat16 and wt.dtype == torch.bfloat16:
        logits = ops.router_logits(x.contiguous(), wt, bias)
    else:
        if computation_dtype != torch.float32 and wt.dtype != computation_dtype:
            # F.linear's operands are router_weights.to(computation_dtype) (router.py:419-424)
            wt = wt.to(computation_dtype)
        if wt.dtype not in (torch.float32, torch.bfloat16):
            wt = wt.to(torch.float32)  # exact: fp16 values are fp32 values
        logits = ops.router_logits_f32(x.float().contiguous(), wt.contiguous(), bias)
    if computation_dtype != torch.float32:
        logits = logits.to(computation_dtype).float()  # F.linear's output rounding
    return logits


@torch.library.custom_op("moe_fp8::router", mutates_args=())
def _router_op(hidden_states: Tensor, router_weights: Tensor, top_k: int,
               router_bias: Optional[Tensor], scoring: int, gamma: Optional[Tensor], eps: float,
               computation_dtype: torch.dtype, order: int, renorm: bool) -> Tuple[Tensor, Tensor]:
    """Opaque graph node of router(): logits -> top-k -> dense affinities on the GPU.
    hidden_states [T, H] (already un-transposed), router_weights [H, E]."""
    logits = router_logits(hidden_states, router_weights, router_bias, gamma, eps,
                           computation_dtype)
    _, _, aff = ops.router_topk(logits, top_k, order, scoring, renorm=renorm, eps=0.0, scale=1.0,
                                dense=True)
    if computation_dtype != torch.float32:
        aff = aff.to(computation_dtype)
        logits = logits.to(computation_dtype)
    return aff, logits


@_router_op.register_fake
def _router_fake(hidden_states, router_weights, top_k, router_bias, scoring, gamma, eps,
                 computation_dtype, order, renorm):
    T, E = hidden_states.shape[0], router_weights.shape[1]
    return (hidden_states.new_empty(T, E, dtype=computation_dtype),
            hidden_states.new_empty(T, E, dtype=computation_dtype))


def router(
    hidden_states: Tensor,
    router_weights: Tensor,
    top_k: int,
    router_bias: Optional[Tensor] = None,
    activation: Union[str, Callable[[Tensor], Tensor]] = "softmax",
    return_logits: bool = False,
    gamma: Optional[Tensor] = None,
    eps: float = 1e-6,
    computation_dtype: torch.dtype = torch.float32,
    router_computation_order: RouterComputationOrder = RouterComputationOrder.PRENORM_LINEAR_TOPK_ACT_SCATTER,
    shard_on_tokens: Optional[bool] = None,
    transposed_hidden_states: bool = False,
    x_sb_layout: Optional[int] = None,
    use_column_tiling: Optional[bool] = None,
    use_indirect_dma_scatter: Optional[bool] = None,
    use_PE_broadcast_w_bias: Optional[bool] = None,
) -> Union[Tensor, Tuple[Tensor, Tensor]]:
    """Expert affinities [T, E] (zeros for unselected experts), and the raw logits
    [T, E] when return_logits. Same arguments as router.py:72-89; see the module
    docstring for the compute path. The GPU work is one torch.library operator
    (moe_fp8::router), an opaque node under torch.compile."""
    _validate_router_inputs(hidden_states, router_weights, top_k, router_bias, gamma,
                            computation_dtype, router_computation_order,
                            transposed_hidden_states)
    scoring = _scoring(activation)
    x = hidden_states.t() if transposed_hidden_states else hidden_states
    O = RouterComputationOrder
    if router_computation_order == O.PRENORM_LINEAR_ACT_TOPK_RENORM_SCATTER:
        order, renorm = ops.ORDER_ACT_TOPK, True
    else:
        # TOPK_SCATTER_ACT: softmax over a row holding -inf outside the top-k is the
        # softmax of the k values, and sigmoid(-inf) = 0, so it selects and weighs
        # as TOPK_ACT does (router.py:507-566 vs :384-441).
        order, renorm = ops.ORDER_TOPK_ACT, False
    aff, logits = _router_op(x.contiguous(), router_weights, int(top_k), router_bias, scoring,
                             gamma, float(eps), computation_dtype, order, renorm)
    if return_logits:
        return aff, logits
    return aff
