"""Pins the blockwise mapping oracle (moe_blockwise.py:325-437) against a loop
brute force, the block-count formula and the mapping invariants."""
import math

import numpy as np
import pytest

from oracle.blockwise import build_blockwise_mapping, mapping_from_ids, num_blocks


def _brute(aff, B, K):
    T, E = aff.shape
    lists = [[t for t in range(T) if aff[t, e] != 0] for e in range(E)]
    blocks = [math.ceil(len(l) / B) for l in lists]
    total = T * min(K, E)
    N = min(math.ceil((total - (E - 1)) / B) + E - 1, total)
    tpid = [-1] * (N * B)
    b2e = []
    off = 0
    for e in range(E):
        for r, t in enumerate(lists[e]):
            tpid[off * B + r] = t
        off += blocks[e]
    cum, acc = [], 0
    for b in blocks:
        acc += b
        cum.append(acc)
    for b in range(N):
        b2e.append(sum(1 for e in range(E - 1) if b >= cum[e]))
    cond = [int(any(v != -1 for v in tpid[b * B:(b + 1) * B])) for b in range(N)]
    return tpid, b2e, cond


@pytest.mark.parametrize("T,E,K,B,seed", [(16, 4, 2, 4, 0), (33, 8, 3, 8, 1), (7, 16, 4, 2, 2),
                                          (64, 8, 2, 256, 3), (5, 6, 1, 1, 4)])
def test_mapping_matches_brute_force(T, E, K, B, seed):
    rng = np.random.default_rng(seed)
    aff = np.zeros((T, E), np.float32)
    for t in range(T):
        aff[t, rng.choice(E, K, replace=False)] = rng.uniform(0.1, 1, K)
    am, tpid, b2e, cond = build_blockwise_mapping(aff, E, K, B)
    bt, bb, bc = _brute(aff, B, K)
    assert list(tpid) == bt and list(b2e) == bb and list(cond) == bc
    assert am.shape == (T * E, 1) and np.array_equal(am[:, 0], aff.reshape(-1))


def test_block_count_formula_at_named_shapes():
    assert num_blocks(64, 2, 8, 256) == 8
    assert num_blocks(64, 8, 256, 256) == 257
    assert num_blocks(8192, 8, 256, 256) == 511
    assert num_blocks(4096, 8, 160, 256) == 287
    assert num_blocks(16384, 8, 384, 256) == 894
    assert num_blocks(1, 8, 256, 256) == 8


def test_invariants_with_empty_and_overfull_experts():
    rng = np.random.default_rng(9)
    T, E, K, B = 300, 10, 3, 16
    aff = np.zeros((T, E), np.float32)
    p = np.array([0.5, 0.2, 0.1, 0.1, 0.05, 0.05, 0, 0, 0, 0])  # 4 empty experts, one overfull
    for t in range(T):
        aff[t, rng.choice(E, K, replace=False, p=None if t % 2 else None)] = 1.0
    aff[:, 6:] = 0
    aff[:, 0] = 1.0
    _, tpid, b2e, cond = build_blockwise_mapping(aff, E, K + 1, B)
    counts = (aff != 0).sum(0)
    assert (tpid >= 0).sum() == counts.sum()
    assert np.all(np.diff(b2e) >= 0)
    for e in range(E):
        slots = np.nonzero(np.isin(np.arange(len(tpid)) // B, np.nonzero(b2e == e)[0]))[0]
        toks = tpid[slots]
        toks = toks[toks >= 0]
        assert np.array_equal(toks, np.nonzero(aff[:, e])[0])     # ascending token order
    assert np.array_equal(cond, (tpid.reshape(-1, B) >= 0).any(1).astype(np.int32))
    del p


def test_padding_mask_only_masks_affinities():
    rng = np.random.default_rng(10)
    T, E, K, B = 12, 4, 2, 4
    aff = np.zeros((T, E), np.float32)
    for t in range(T):
        aff[t, rng.choice(E, K, replace=False)] = 0.5
    pm = np.arange(T) < 9
    am, tpid, _, _ = build_blockwise_mapping(aff, E, K, B, padding_mask=pm)
    _, tpid0, _, _ = build_blockwise_mapping(aff, E, K, B)
    assert np.array_equal(tpid, tpid0)                           # positions ignore padding
    assert np.all(am.reshape(T, E)[9:] == 0) and np.array_equal(am.reshape(T, E)[:9], aff[:9])


def test_mapping_from_ids_inverse():
    rng = np.random.default_rng(11)
    T, E, K, B = 40, 8, 3, 8
    ids = np.stack([rng.choice(E, K, replace=False) for _ in range(T)]).astype(np.int32)
    tpid, b2e, cond, counts, inv = mapping_from_ids(ids, E, B)
    assert counts.sum() == T * K
    for t in range(T):
        for k in range(K):
            p = inv[t, k]
            assert tpid[p] == t and b2e[p // B] == ids[t, k]
