"""Property-based pins of the oracle (hypothesis, CPU): the blockwise mapping equals the
loop brute force on arbitrary small shapes (including experts nobody picks and tokens
routed to fewer than K experts), and grouped routing equals an exhaustive search over
group subsets, ties included."""
import numpy as np
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

from oracle import router as R
from oracle.blockwise import build_blockwise_mapping, mapping_from_ids
from oracle.mathfn import sigmoid_f32
from test_oracle_blockwise import _brute

SETTINGS = dict(max_examples=60, deadline=None, suppress_health_check=[HealthCheck.too_slow])


@st.composite
def affinities(draw):
    T = draw(st.integers(1, 24))
    E = draw(st.integers(1, 12))
    K = draw(st.integers(1, E))
    B = draw(st.sampled_from([1, 2, 3, 4, 8, 16]))
    seed = draw(st.integers(0, 2 ** 31 - 1))
    rng = np.random.default_rng(seed)
    aff = np.zeros((T, E), np.float32)
    for t in range(T):
        k = int(rng.integers(0, K + 1))            # some tokens pick fewer than K experts
        aff[t, rng.choice(E, k, replace=False)] = rng.uniform(0.05, 1, k).astype(np.float32)
    return aff, K, B


@settings(**SETTINGS)
@given(affinities())
def test_mapping_equals_brute_force(case):
    aff, K, B = case
    T, E = aff.shape
    am, tpid, b2e, cond = build_blockwise_mapping(aff, E, K, B)
    bt, bb, bc = _brute(aff, B, K)
    assert list(tpid) == bt and list(b2e) == bb and list(cond) == bc
    # the slots hold every (token, expert) pair exactly once, tokens ascending per expert
    pairs = sorted((t, b2e[i // B]) for i, t in enumerate(tpid) if t >= 0)
    assert pairs == sorted(zip(*np.nonzero(aff)))


@settings(**SETTINGS)
@given(st.integers(1, 20), st.integers(2, 10), st.integers(1, 4), st.sampled_from([1, 2, 4, 16]),
       st.integers(0, 2 ** 31 - 1))
def test_mapping_from_ids_round_trip(T, E, K, B, seed):
    K = min(K, E)
    rng = np.random.default_rng(seed)
    ids = np.stack([rng.choice(E, K, replace=False) for _ in range(T)]).astype(np.int32)
    tpid, b2e, cond, counts, inv = mapping_from_ids(ids, E, B)
    assert np.array_equal(counts, np.bincount(ids.ravel(), minlength=E))
    for t in range(T):
        for k in range(K):
            s = inv[t, k]
            assert tpid[s] == t and b2e[s // B] == ids[t, k]


def _exhaustive_grouped(c, k, n_group, topk_group):
    """Best group subset by the group score (sum of the two largest), lower index first
    on ties; then the k best experts inside it, lower index first on ties."""
    E = c.shape[0]
    gs = E // n_group
    score = [np.sort(c[j * gs:(j + 1) * gs])[::-1][:min(2, gs)].sum(dtype=np.float32)
             for j in range(n_group)]
    groups = sorted(range(n_group), key=lambda j: (-score[j], j))[:topk_group]
    cand = [e for j in groups for e in range(j * gs, (j + 1) * gs)]
    return sorted(cand, key=lambda e: (-c[e], e))[:k]


@settings(**SETTINGS)
@given(st.sampled_from([(8, 4), (12, 3), (16, 4), (16, 8), (6, 6)]), st.integers(0, 2 ** 31 - 1),
       st.booleans())
def test_grouped_routing_equals_exhaustive_search(shape, seed, ties):
    E, n_group = shape
    rng = np.random.default_rng(seed)
    gs = E // n_group
    topk_group = int(rng.integers(1, n_group + 1))
    k = int(rng.integers(1, topk_group * gs + 1))
    logits = rng.normal(0, 1.5, (3, E)).astype(np.float32)
    if ties:
        logits = np.round(logits * 2) / 2                   # exact ties between experts
    bias = rng.normal(0, 0.01, E).astype(np.float32)
    ids, w = R.route_grouped(logits, bias, k, n_group, topk_group, R.SIGMOID, renorm=False)
    s = sigmoid_f32(logits)
    for t in range(logits.shape[0]):
        c = (s[t] + bias).astype(np.float32)
        assert list(ids[t]) == _exhaustive_grouped(c, k, n_group, topk_group)
        assert np.array_equal(w[t], s[t][ids[t]])
