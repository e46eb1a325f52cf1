"""moe_cte(): blockwise expert MLP over a given mapping, with the reference's signature.

Reference: vllm_neuron/functional/moe/moe_cte.py:35-437 (API and dispatch),
:465-612 (_torch_moe_impl, the math):
    out[t] = sum_e affinity[t, e] * ( act(x_t W_g,e) * (x_t W_u,e) ) W_d,e
summed in expert order, accumulated in fp32 (POST_SCALE), cast to the input
dtype; T = expert_affinities_masked.shape[0] // E (:533-536). The GPU work is one
torch.library operator (moe_fp8::moe_cte), an opaque node under torch.compile.

Compute path (all HIP): 1x128 fp8 activation quant -> row tiles of the given
token_position_to_id / block_to_expert -> fp8 gate_up with SiLU * up and the
1x128 requant of h -> fp8 down -> inverse mapping -> combine weighted by the
dense affinities in expert order. Experts are float8_e4m3fn with 128x128 fp32
block scales, in the reference layout (gate_up [E, H, 2, I], scales
[E, H/128, 2, I/128]; down [E, I, H], scales [E, I/128, H/128]) or the
checkpoint stacking (gate_up [E, 2I, H], down [E, H, I]), or with the
reference's FP8 per-channel scales gate_up_proj_scale [E, 1, 2I] and
down_proj_scale [E, 1, H] (moe_cte.py:178-188), which the GEMM epilogues apply
per output column.

Supported: SiLU, POST_SCALE and NO_SCALE, implementation shard_on_block /
shard_on_i / shard_on_i_hybrid / shard_on_i_dropping (one kernel family serves
them all; the choice is a Trainium sharding hint). MX experts (implementation
shard_on_block_mx / shard_on_i_mx*, quantization_type MX, or uint8 E8M0 scales):
stacked MXFP4 / MXFP8 weights with biases, SiLU or Swish and gate / up clamps, on
the E8M0-scaled MFMA kernels (moe_fp8::moe_cte_mx). Raises NotImplementedError for
STATIC_MX, the Trainium-tiled uint16 MX layout, biases / clamps / Swish with the
fp8 128x128 experts, GELU, PRE_SCALE / PRE_SCALE_DELAYED and activation
checkpoint buffers.
"""
from typing import Any, Optional

import torch
from torch import Tensor

from ... import ops
from . import _experts
from .types import (MX_IMPLEMENTATIONS, ActFnType, BlockShardStrategy, ExpertAffinityScaleMode,
                    MoECTEImplementation, QuantizationType)


def _unsupported(**kw):
    bad = [k for k, v in kw.items() if v]
    if bad:
        raise NotImplementedError(f"moe_cte: {', '.join(bad)} not supported by this build "
                                  "(fp8 128x128 blockwise experts, SiLU, POST_SCALE / NO_SCALE)")


def moe_cte(
    hidden_states: Tensor,
    expert_affinities_masked: Optional[Tensor],
    gate_up_proj_weight: Tensor,
    down_proj_weight: Tensor,
    token_position_to_id: Tensor,
    block_to_expert: Tensor,
    block_size: int,
    implementation: MoECTEImplementation,
    n_block_per_iter: int = 1,
    block_sharding_strategy: BlockShardStrategy = BlockShardStrategy.PING_PONG,
    n_static_blocks: int = -1,
    n_dynamic_blocks: int = -1,
    top_k: int = 1,
    ep_degree: int = 1,
    ep_rank: Optional[Tensor] = None,
    checkpoint_activation: bool = False,
    expert_affinity_multiply_on_I: bool = False,
    num_static_block: Optional[int] = None,
    conditions: Optional[Tensor] = None,
    gate_and_up_proj_bias: Optional[Tensor] = None,
    down_proj_bias: Optional[Tensor] = None,
    gate_up_proj_scale: Optional[Tensor] = None,
    down_proj_scale: Optional[Tensor] = None,
    gate_up_activations_T: Optional[Tensor] = None,
    down_activations: Optional[Tensor] = None,
    activation_function: ActFnType = ActFnType.SiLU,
    skip_token: bool = False,
    skip_weight: bool = False,
    compute_dtype: Any = None,
    is_tensor_update_accumulating: bool = True,
    expert_affinities_scaling_mode: ExpertAffinityScaleMode = ExpertAffinityScaleMode.POST_SCALE,
    gate_clamp_upper_limit: Optional[float] = None,
    gate_clamp_lower_limit: Optional[float] = None,
    up_clamp_upper_limit: Optional[float] = None,
    up_clamp_lower_limit: Optional[float] = None,
    quantization_type: QuantizationType = QuantizationType.NONE,
    gate_w_scale: Optional[Tensor] = None,
    up_w_scale: Optional[Tensor] = None,
    down_w_scale: Optional[Tensor] = None,
    gate_up_in_scale: Optional[Tensor] = None,
    down_in_scale: Optional[Tensor] = None,
    use_packed_scales: bool = False,
) -> Tensor:
    """Output [T, H] in hidden_states' dtype; see the module docstring."""
    if not isinstance(implementation, MoECTEImplementation):
        raise ValueError(f"implementation must be a MoECTEImplementation, got {implementation!r}")
    if implementation in MX_IMPLEMENTATIONS or quantization_type == QuantizationType.MX or \
            _experts.is_mx_weights(gate_up_proj_weight, gate_up_proj_scale):
        return _moe_cte_mx(hidden_states, expert_affinities_masked, gate_up_proj_weight,
                           down_proj_weight, token_position_to_id, block_to_expert, block_size,
                           quantization_type, ep_degree, ep_rank, checkpoint_activation,
                           gate_and_up_proj_bias, down_proj_bias, gate_up_proj_scale,
                           down_proj_scale, gate_up_activations_T, down_activations,
                           activation_function, expert_affinities_scaling_mode,
                           gate_clamp_upper_limit, gate_clamp_lower_limit, up_clamp_upper_limit,
                           up_clamp_lower_limit)
    _unsupported(**{
        f"implementation {implementation.name}": implementation in MX_IMPLEMENTATIONS,
        f"quantization_type {quantization_type.name}": quantization_type != QuantizationType.NONE,
        "expert biases": gate_and_up_proj_bias is not None or down_proj_bias is not None,
        "gate/up clamps": any(v is not None for v in (gate_clamp_upper_limit, gate_clamp_lower_limit,
                                                      up_clamp_upper_limit, up_clamp_lower_limit)),
        f"activation {getattr(activation_function, 'name', activation_function)}":
            activation_function != ActFnType.SiLU,
        f"scaling mode {expert_affinities_scaling_mode.name}": expert_affinities_scaling_mode not in (
            ExpertAffinityScaleMode.POST_SCALE, ExpertAffinityScaleMode.NO_SCALE),
        "activation checkpoint buffers": gate_up_activations_T is not None
            or down_activations is not None or checkpoint_activation,
        "packed affinities (expert_affinities_masked=None)": expert_affinities_masked is None,
        "ep_rank / ep_degree": ep_rank is not None or int(ep_degree) != 1,
    })
    if (gate_up_proj_scale is None) != (down_proj_scale is None):
        raise ValueError("gate_up_proj_scale and down_proj_scale must be provided together")
    if hidden_states.dim() != 2:
        raise ValueError(f"hidden_states must be [T, H] or [T+1, H], got {tuple(hidden_states.shape)}")

    E, H, _ = _experts.weight_dims(gate_up_proj_weight, down_proj_weight)
    if hidden_states.shape[1] != H:
        raise ValueError(f"hidden_states has H={hidden_states.shape[1]}, weights H={H}")
    if expert_affinities_masked.numel() % E:
        raise ValueError(f"expert_affinities_masked holds {expert_affinities_masked.numel()} "
                         f"values, not a multiple of E={E}")
    T = expert_affinities_masked.numel() // E
    if hidden_states.shape[0] not in (T, T + 1):
        raise ValueError(f"hidden_states must have T={T} or T+1 rows, got {hidden_states.shape[0]}")
    B = int(block_size)
    tpid = token_position_to_id.reshape(-1)
    b2e = block_to_expert.reshape(-1)
    N = b2e.numel()
    if tpid.numel() != N * B:
        raise ValueError(f"token_position_to_id has {tpid.numel()} slots, block_to_expert "
                         f"{N} blocks of {B}")
    if tpid.dtype != torch.int32 or b2e.dtype != torch.int32:
        raise ValueError("token_position_to_id and block_to_expert must be int32")
    no_scale = expert_affinities_scaling_mode == ExpertAffinityScaleMode.NO_SCALE
    return _moe_cte_op(hidden_states, expert_affinities_masked, gate_up_proj_weight,
                       down_proj_weight, gate_up_proj_scale, down_proj_scale, tpid, b2e, B,
                       no_scale)


@torch.library.custom_op("moe_fp8::moe_cte", mutates_args=())
def _moe_cte_op(hidden_states: Tensor, expert_affinities_masked: Tensor, gate_up: Tensor,
                down: Tensor, gate_up_scale: Optional[Tensor], down_scale: Optional[Tensor],
                token_position_to_id: Tensor, block_to_expert: Tensor, block_size: int,
                no_scale: bool) -> Tensor:
    """Opaque graph node of moe_cte (arguments checked by moe_cte): the experts of a
    mapping, combined per token with the dense affinities in expert order."""
    w13, s13, w2, s2, c13, c2 = _experts.routed_weights(gate_up, down, gate_up_scale, down_scale)
    E, H = w13.shape[0], w13.shape[2]
    T = expert_affinities_masked.numel() // E
    B = block_size
    tpid = token_position_to_id.contiguous()
    b2e = block_to_expert.contiguous()
    N = b2e.numel()
    x = _experts.as_bf16(hidden_states[:T]).contiguous()
    w = _experts.make_weights(w13, s13, w2, s2, c13, c2)
    # Expected routed rows per token from the mapping size (N ~ T*K/B + E - 1);
    # it only picks the tile height. Tile lists are sized for any mapping (K = E).
    k_rows = max(1, min(E, ((N - E + 1) * B + E - 1) // max(T, 1)))
    y, NB = _experts.run_experts(x, tpid, b2e, B, k_rows, E, w)
    inv = ops.invert_mapping(tpid, b2e, B, T, E)  # [T, E] slot of (t, e) or -1
    aff = expert_affinities_masked.reshape(T, E).float()
    if no_scale:
        aff = (aff != 0).float()  # moe_block_tkg.py:280-289 binary weights
    out = ops.combine(y, inv, aff.contiguous(), T, H, NB, 0)
    return out if hidden_states.dtype == torch.bfloat16 else out.to(hidden_states.dtype)


@_moe_cte_op.register_fake
def _moe_cte_fake(hidden_states, expert_affinities_masked, gate_up, down, gate_up_scale,
                  down_scale, token_position_to_id, block_to_expert, block_size, no_scale):
    E, H, _ = _experts.weight_dims(gate_up, down)
    T = expert_affinities_masked.numel() // E
    return hidden_states.new_empty(T, H)


def _check_mapping(hidden_states, expert_affinities_masked, E, H, token_position_to_id,
                   block_to_expert, block_size):
    if hidden_states.dim() != 2:
        raise ValueError(f"hidden_states must be [T, H] or [T+1, H], got {tuple(hidden_states.shape)}")
    if hidden_states.shape[1] != H:
        raise ValueError(f"hidden_states has H={hidden_states.shape[1]}, weights H={H}")
    if expert_affinities_masked.numel() % E:
        raise ValueError(f"expert_affinities_masked holds {expert_affinities_masked.numel()} "
                         f"values, not a multiple of E={E}")
    T = expert_affinities_masked.numel() // E
    if hidden_states.shape[0] not in (T, T + 1):
        raise ValueError(f"hidden_states must have T={T} or T+1 rows, got {hidden_states.shape[0]}")
    B = int(block_size)
    tpid = token_position_to_id.reshape(-1)
    b2e = block_to_expert.reshape(-1)
    if tpid.numel() != b2e.numel() * B:
        raise ValueError(f"token_position_to_id has {tpid.numel()} slots, block_to_expert "
                         f"{b2e.numel()} blocks of {B}")
    if tpid.dtype != torch.int32 or b2e.dtype != torch.int32:
        raise ValueError("token_position_to_id and block_to_expert must be int32")
    return T, B, tpid, b2e


def _moe_cte_mx(hidden_states, expert_affinities_masked, gate_up, down, token_position_to_id,
                block_to_expert, block_size, quantization_type, ep_degree, ep_rank,
                checkpoint_activation, gate_and_up_proj_bias, down_proj_bias, gate_up_scale,
                down_scale, gate_up_activations_T, down_activations, activation_function,
                scaling_mode, gate_hi, gate_lo, up_hi, up_lo):
    """moe_cte with MX experts (the shard_on_block_mx path, moe_cte.py:122-130, :178-191):
    stacked MXFP4 / MXFP8 weights with E8M0 scales, optional biases (the reference's
    [E, 2, I] and [E, 1, H] shapes), SiLU or Swish, gate / up clamps."""
    _unsupported(**{
        f"quantization_type {quantization_type.name}": quantization_type == QuantizationType.STATIC_MX,
        f"activation {getattr(activation_function, 'name', activation_function)}":
            activation_function not in (ActFnType.SiLU, ActFnType.Swish),
        f"scaling mode {scaling_mode.name}": scaling_mode not in (
            ExpertAffinityScaleMode.POST_SCALE, ExpertAffinityScaleMode.NO_SCALE),
        "activation checkpoint buffers": gate_up_activations_T is not None
            or down_activations is not None or checkpoint_activation,
        "packed affinities (expert_affinities_masked=None)": expert_affinities_masked is None,
        "ep_rank / ep_degree": ep_rank is not None or int(ep_degree) != 1,
    })
    if gate_up.dtype == torch.uint16 or down.dtype == torch.uint16:
        raise NotImplementedError(
            "MX weights in the Trainium-tiled uint16 layout: pass the stacked layout "
            "(vllm_neuron_amd.weights_mx.from_hf_gpt_oss converts the HF checkpoint)")
    if gate_up_scale is None or down_scale is None:
        raise ValueError("MX experts need gate_up_proj_scale and down_proj_scale")
    if (gate_and_up_proj_bias is None) != (down_proj_bias is None):
        raise ValueError("gate_and_up_proj_bias and down_proj_bias must be provided together")
    E, H, _ = _experts.mx_dims(gate_up, down)
    T, B, tpid, b2e = _check_mapping(hidden_states, expert_affinities_masked, E, H,
                                     token_position_to_id, block_to_expert, block_size)
    act = "swish" if activation_function == ActFnType.Swish else "silu"
    nan = float("nan")
    lim = lambda v: nan if v is None else float(v)
    return _moe_cte_mx_op(hidden_states, expert_affinities_masked, gate_up, down, gate_up_scale,
                          down_scale, gate_and_up_proj_bias, down_proj_bias, tpid, b2e, B,
                          scaling_mode == ExpertAffinityScaleMode.NO_SCALE, act, lim(gate_lo),
                          lim(gate_hi), lim(up_lo), lim(up_hi))


@torch.library.custom_op("moe_fp8::moe_cte_mx", mutates_args=())
def _moe_cte_mx_op(hidden_states: Tensor, expert_affinities_masked: Tensor, gate_up: Tensor,
                   down: Tensor, gate_up_scale: Tensor, down_scale: Tensor,
                   gate_up_bias: Optional[Tensor], down_bias: Optional[Tensor],
                   token_position_to_id: Tensor, block_to_expert: Tensor, block_size: int,
                   no_scale: bool, act: str, gate_lo: float, gate_hi: float, up_lo: float,
                   up_hi: float) -> Tensor:
    """Opaque graph node of moe_cte with MX experts (arguments checked by moe_cte)."""
    w = _experts.mx_weights(gate_up, down, gate_up_scale, down_scale, gate_up_bias, down_bias)
    E, H = w.n_experts, w.hidden
    T = expert_affinities_masked.numel() // E
    B = block_size
    tpid = token_position_to_id.contiguous()
    b2e = block_to_expert.contiguous()
    N = b2e.numel()
    NB = N * B
    x = _experts.as_bf16(hidden_states[:T]).contiguous()
    xq, xs = ops.act_quant_mx(x)
    k_rows = max(1, min(E, ((N - E + 1) * B + E - 1) // max(T, 1)))
    mt = min(ops.choose_mt(T, k_rows, E), 64)  # the MX kernels stop at 64-row tiles
    tiles, num, max_tiles = ops.build_tiles(tpid, b2e, B, T, E, E, 0, mt)
    none = lambda v: None if v != v else v
    hq, hs = ops.expert_gate_up_mx(xq, xs, w, tpid, NB, tiles, num, max_tiles, mt, NB, act,
                                   (none(gate_lo), none(gate_hi)), (none(up_lo), none(up_hi)))
    y = ops.expert_down_mx(hq, hs, w, T, NB, tiles, num, max_tiles, mt)
    inv = ops.invert_mapping(tpid, b2e, B, T, E)
    aff = expert_affinities_masked.reshape(T, E).float()
    if no_scale:
        aff = (aff != 0).float()
    out = ops.combine(y, inv, aff.contiguous(), T, H, NB, 0)
    return out if hidden_states.dtype == torch.bfloat16 else out.to(hidden_states.dtype)


@_moe_cte_mx_op.register_fake
def _moe_cte_mx_fake(hidden_states, expert_affinities_masked, gate_up, down, gate_up_scale,
                     down_scale, gate_up_bias, down_bias, token_position_to_id, block_to_expert,
                     block_size, no_scale, act, gate_lo, gate_hi, up_lo, up_hi):
    E, H, _ = _experts.mx_dims(gate_up, down)
    return hidden_states.new_empty(expert_affinities_masked.numel() // E, H)
