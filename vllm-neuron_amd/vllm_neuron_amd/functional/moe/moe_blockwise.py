"""build_blockwise_mapping(): align-by-expert mapping with the reference's signature.

Reference: vllm_neuron/functional/moe/moe_blockwise.py:25-157 (API and
outputs), :325-437 (_build_blockwise_mapping_torch, the slot order),
:480-498 (_apply_padding_mask). Computed by the moe_blockwise_mapping HIP
kernels (deterministic, no atomics); outputs are bit-identical to the
reference's torch flow.
"""
from typing import Optional

import torch
from torch import Tensor

from ... import ops


def _single_rank(moe_group):
    if moe_group is None:
        return True
    ws = getattr(moe_group, "world_size", None)
    return ws is None or int(ws) == 1


def build_blockwise_mapping(
    expert_affinities: Tensor,
    num_local_experts: int,
    num_experts_per_token: int,
    block_size: int,
    moe_group=None,
    tp_degree: int = 1,
    padding_mask: Optional[Tensor] = None,
) -> tuple:
    """Returns (expert_affinities_masked [T*E, 1] fp32, token_position_to_id [N*B]
    int32, block_to_expert [N] int32, conditions [N] int32).

    expert_affinities [T, E] (zeros for unselected experts); padding_mask [T]
    bool, True = real token. N = min(ceil((T*min(K,E) - (E-1)) / B) + E - 1,
    T*min(K,E)). moe_group is the reference's process group; one GPU holds
    every expert here, so it must be None or a single-rank group, and
    tp_degree must be 1 (intermediate sharding needs collectives).
    Raises IndexError when more (token, expert) pairs are routed than the
    N*B slots hold (a token with more than num_experts_per_token nonzero
    affinities)."""
    if expert_affinities.dim() != 2:
        raise ValueError(f"expert_affinities must be [T, E], got {tuple(expert_affinities.shape)}")
    T, E = expert_affinities.shape
    if E != num_local_experts:
        raise ValueError(f"expert_affinities has {E} experts, num_local_experts is "
                         f"{num_local_experts}")
    if block_size < 1:
        raise ValueError(f"block_size must be >= 1, got {block_size}")
    if int(tp_degree) != 1:
        raise NotImplementedError("tp_degree > 1 shards experts over ranks; this build keeps "
                                  "all experts on one GPU")
    if not _single_rank(moe_group):
        raise NotImplementedError("multi-rank moe_group: this build keeps all experts on one GPU")
    aff = expert_affinities
    if aff.dtype != torch.float32:
        aff = aff.float()
    out = ops.blockwise_mapping(affinities=aff.contiguous(), top_k=int(num_experts_per_token),
                                block_size=int(block_size), padding_mask=padding_mask,
                                check=True)
    return (out["affinities_masked"], out["token_position_to_id"], out["block_to_expert"],
            out["conditions"])
