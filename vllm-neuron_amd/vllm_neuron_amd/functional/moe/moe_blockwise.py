"""build_blockwise_mapping(): align-by-expert mapping with the reference's signature.

Reference: vllm_neuron/functional/moe/moe_blockwise.py:25-157 (API and
outputs), :325-437 (_build_blockwise_mapping_torch, the slot order),
:480-498 (_apply_padding_mask). Computed by the moe_blockwise_mapping HIP
kernels (deterministic, no atomics); outputs are bit-identical to the
reference's torch flow.
"""
import os
from typing import Optional, Tuple

import torch
from torch import Tensor

from ... import ops


def _single_rank(moe_group):
    if moe_group is None:
        return True
    ws = getattr(moe_group, "world_size", None)
    return ws is None or int(ws) == 1


def num_blocks(T, K, E, B):
    """N = min(ceil((T*min(K,E) - (E-1)) / B) + E - 1, T*min(K,E)) (moe_blockwise.py:376-382),
    in Python integers (shape functions run without the library)."""
    total = T * min(K, E)
    q = -((-(total - (E - 1))) // B)  # ceil division, also for a negative numerator
    return min(q + E - 1, total)


# Debug check, off by default: synchronize after each mapping and raise when routed
# (token, expert) pairs did not fit the N*B slots (a token with more than
# num_experts_per_token nonzero affinities). The kernels drop such pairs and count
# them in the workspace status word either way; the check costs a host sync.
CHECK_OVERFLOW = os.environ.get("VLLM_NEURON_AMD_CHECK_MAPPING", "0") == "1"


@torch.library.custom_op("moe_fp8::blockwise_mapping", mutates_args=())
def _mapping_op(affinities: Tensor, top_k: int, block_size: int,
                padding_mask: Optional[Tensor]) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    """Opaque graph node of build_blockwise_mapping (no host synchronization unless
    CHECK_OVERFLOW)."""
    out = ops.blockwise_mapping(affinities=affinities, top_k=top_k, block_size=block_size,
                                padding_mask=padding_mask, check=CHECK_OVERFLOW)
    return (out["affinities_masked"], out["token_position_to_id"], out["block_to_expert"],
            out["conditions"])


@_mapping_op.register_fake
def _mapping_fake(affinities, top_k, block_size, padding_mask):
    T, E = affinities.shape
    N = num_blocks(T, top_k, E, block_size)
    i32 = torch.int32
    return (affinities.new_empty(T * E, 1), affinities.new_empty(N * block_size, dtype=i32),
            affinities.new_empty(N, dtype=i32), affinities.new_empty(N, dtype=i32))


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
    Routed (token, expert) pairs beyond the N*B slots (a token with more than
    num_experts_per_token nonzero affinities) are dropped; with
    VLLM_NEURON_AMD_CHECK_MAPPING=1 the call synchronizes and raises IndexError
    for them instead. The GPU work is one torch.library operator
    (moe_fp8::blockwise_mapping)."""
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
    if padding_mask is not None and tuple(padding_mask.shape) != (T,):
        raise ValueError(f"padding_mask must be [T], got {tuple(padding_mask.shape)}")
    aff = expert_affinities
    if aff.dtype != torch.float32:
        aff = aff.float()
    return _mapping_op(aff.contiguous(), int(num_experts_per_token), int(block_size),
                       padding_mask)
