"""Blockwise (align-by-expert) mapping oracle (test infrastructure).

Restates _build_blockwise_mapping_torch, vllm_neuron/functional/moe/moe_blockwise.py:325-437,
and the surrounding build_blockwise_mapping, moe_blockwise.py:91-157, in integer form:

  mask[t,e]          = affinities[t,e] != 0                          (:91, from the unpadded affinities)
  counts[e]          = sum_t mask[t,e]                               (:370)
  blocks[e]          = ceil(counts[e] / B)                           (:373-375)
  N                  = min(ceil((T*min(K,E) - (E-1)) / B) + E - 1, T*min(K,E))   (:376-382)
  cum                = inclusive cumsum of blocks                    (:385-387)
  block_to_expert[b] = #{ e < E-1 : b >= cum[e] }                     (:388-390)
  slot(t,e)          = cum_excl[e]*B + #{ t' < t : mask[t',e] }       (:393-398 with the 1-based
                                                                     cumsum and the [1:] shift, :426-431)
  token_position_to_id[slot(t,e)] = t, -1 elsewhere                   (:422-431)
  conditions[b]      = any(token_position_to_id[b*B:(b+1)*B] != -1)   (:148-150)
  expert_affinities_masked = (affinities * padding_mask).view(T*E, 1) (:92-94, :480-498)
"""
import math

import numpy as np


def num_blocks(T, K, E, B):
    total = T * min(K, E)
    n = math.ceil((total - (E - 1)) / B) + E - 1
    return int(min(n, total))


def build_blockwise_mapping(affinities, num_local_experts, num_experts_per_token, block_size,
                            padding_mask=None):
    aff = np.asarray(affinities, np.float32)
    T, E = aff.shape
    if E != num_local_experts:
        raise ValueError("affinities must be [T, num_local_experts]")
    B = int(block_size)
    mask = aff != 0
    masked = aff if padding_mask is None else aff * np.asarray(padding_mask, np.float32)[:, None]
    counts = mask.sum(axis=0).astype(np.int64)
    blocks = (counts + B - 1) // B
    N = num_blocks(T, num_experts_per_token, E, B)
    cum = np.cumsum(blocks)
    b = np.arange(N)
    block_to_expert = (b[:, None] >= cum[None, :-1]).sum(axis=1).astype(np.int32)
    cum_excl = np.concatenate([[0], cum[:-1]])
    rank = np.cumsum(mask, axis=0) - 1                         # 0-based rank of t among expert e's tokens
    slot = cum_excl[None, :] * B + rank
    tpid = np.full(N * B, -1, np.int64)
    tt, ee = np.nonzero(mask)
    s = slot[tt, ee]
    if s.size and s.max() >= N * B:
        raise ValueError("more routed (token, expert) pairs than the N*B mapping can hold")
    tpid[s] = tt
    conditions = (tpid.reshape(N, B) != -1).any(axis=1).astype(np.int32)
    return (masked.reshape(T * E, 1).astype(np.float32), tpid.astype(np.int32),
            block_to_expert, conditions)


def mapping_from_ids(ids, E, B):
    """Same mapping from top-k ids [T,K] (each row distinct experts; -1 = unused slot).

    Also returns expert_counts [E] and inv_pos [T,K] (slot of (t, ids[t,k]) or -1)."""
    ids = np.asarray(ids, np.int64)
    T, K = ids.shape
    aff = np.zeros((T, E), np.float32)
    for k in range(K):
        v = ids[:, k] >= 0
        aff[np.nonzero(v)[0], ids[v, k]] = 1.0
    _, tpid, b2e, cond = build_blockwise_mapping(aff, E, K, B)
    counts = (aff != 0).sum(axis=0).astype(np.int32)
    inv = np.full((T, K), -1, np.int32)
    lookup = {}
    for p, t in enumerate(tpid):
        if t >= 0:
            lookup[(int(t), int(b2e[p // B]))] = p
    for t in range(T):
        for k in range(K):
            if ids[t, k] >= 0:
                inv[t, k] = lookup[(t, int(ids[t, k]))]
    return tpid, b2e, cond, counts, inv
