"""Pins the expert-MLP oracle: float64 loops on tiny shapes, the reference's dense
all-expert form (moe_cte.py:465-612), linearity, permutation invariance, and the
topk_reduce docstring example (topk_reduce.py:70-82)."""
import numpy as np

from oracle.fp8 import dequant_weight_128x128, quant_weight_128x128
from oracle.moe import expert_mlp, moe_dense_reference, moe_sparse_fp8, topk_reduce
from oracle.router import route_topk_act, scatter_dense


def _expert_loop64(x, w13, w2):
    I = w13.shape[0] // 2
    out = np.zeros((x.shape[0], w2.shape[0]))
    for t in range(x.shape[0]):
        g = np.array([sum(float(x[t, h]) * float(w13[i, h]) for h in range(x.shape[1])) for i in range(I)])
        u = np.array([sum(float(x[t, h]) * float(w13[I + i, h]) for h in range(x.shape[1])) for i in range(I)])
        hh = g / (1 + np.exp(-g)) * u
        out[t] = [sum(hh[i] * float(w2[o, i]) for i in range(I)) for o in range(w2.shape[0])]
    return out


def test_expert_mlp_matches_float64_loops():
    rng = np.random.default_rng(0)
    x = rng.normal(0, 1, (3, 128)).astype(np.float32)
    w13 = rng.normal(0, 0.05, (256, 128)).astype(np.float32)
    w2 = rng.normal(0, 0.05, (128, 128)).astype(np.float32)
    got = expert_mlp(x, w13, w2, requant_h=False)
    ref = _expert_loop64(x, w13, w2)
    assert np.allclose(got, ref, rtol=1e-4, atol=1e-5)


def _small_layer(seed, T=24, H=256, I=128, E=4, K=2):
    rng = np.random.default_rng(seed)
    x = rng.normal(0, 1, (T, H)).astype(np.float32)
    q13, s13, q2, s2 = [], [], [], []
    for _ in range(E):
        a, sa = quant_weight_128x128(rng.normal(0, 0.02, (2 * I, H)).astype(np.float32))
        b, sb = quant_weight_128x128(rng.normal(0, 0.02, (H, I)).astype(np.float32))
        q13.append(a), s13.append(sa), q2.append(b), s2.append(sb)
    lg = rng.normal(0, 1, (T, E)).astype(np.float32)
    ids, w = route_topk_act(lg, K)
    return x, ids, w, np.stack(q13), np.stack(s13), np.stack(q2), np.stack(s2)


def test_sparse_equals_reference_dense_form():
    """Per-expert gathered computation == _torch_moe_impl's dense einsum over all experts
    when fed the same (dequantized, unrequantized) operands."""
    from oracle.fp8 import dequant_act_1x128, quant_act_1x128
    x, ids, w, q13, s13, q2, s2 = _small_layer(1)
    E, I2, H = q13.shape
    I = I2 // 2
    T = x.shape[0]
    sparse = moe_sparse_fp8(x, ids, w, q13, s13, q2, s2, requant_h=False)
    xh = dequant_act_1x128(*quant_act_1x128(x))
    w13 = np.stack([dequant_weight_128x128(q13[e], s13[e]) for e in range(E)])
    w2 = np.stack([dequant_weight_128x128(q2[e], s2[e]) for e in range(E)])
    gate_up = np.stack([w13[:, :I, :], w13[:, I:, :]], axis=2).transpose(0, 3, 2, 1)  # [E,H,2,I]
    down = w2.transpose(0, 2, 1)                                                       # [E,I,H]
    aff = scatter_dense(ids, w, E).reshape(T * E, 1)
    dense = moe_dense_reference(xh, aff, gate_up, down)
    assert np.allclose(sparse, dense, rtol=1e-4, atol=1e-5)


def test_linear_in_routing_weights_and_permutation_invariant():
    x, ids, w, q13, s13, q2, s2 = _small_layer(2)
    base = moe_sparse_fp8(x, ids, w, q13, s13, q2, s2)
    double = moe_sparse_fp8(x, ids, 2 * w, q13, s13, q2, s2)
    assert np.allclose(double, 2 * base, rtol=1e-6, atol=1e-7)
    perm = np.random.default_rng(3).permutation(x.shape[0])
    permuted = moe_sparse_fp8(x[perm], ids[perm], w[perm], q13, s13, q2, s2)
    assert np.allclose(permuted, base[perm], rtol=0, atol=0)


def test_shared_expert_adds_with_unit_weight():
    x, ids, w, q13, s13, q2, s2 = _small_layer(4)
    shared = (q13[0:1], s13[0:1], q2[0:1], s2[0:1])
    with_sh = moe_sparse_fp8(x, ids, w, q13, s13, q2, s2, shared=tuple(a[0] for a in shared))
    routed = moe_sparse_fp8(x, ids, w, q13, s13, q2, s2)
    only = moe_sparse_fp8(x, np.zeros_like(ids), np.ones_like(w) * 0.5, q13[:1], s13[:1], q2[:1], s2[:1])
    assert np.allclose(with_sh - routed, only, rtol=1e-5, atol=1e-6)
    # two shared experts (a list): each adds its own unit-weight output
    two = moe_sparse_fp8(x, ids, w, q13, s13, q2, s2,
                         shared=[tuple(a[0] for a in shared), (q13[1], s13[1], q2[1], s2[1])])
    only1 = moe_sparse_fp8(x, np.zeros_like(ids), np.ones_like(w) * 0.5, q13[1:2], s13[1:2], q2[1:2],
                           s2[1:2])
    assert np.allclose(two - routed, only + only1, rtol=1e-5, atol=1e-6)


def test_topk_reduce_docstring_examples():
    rows = np.arange(16, dtype=np.float32).reshape(4, 4)
    out = topk_reduce(rows, [1, 1, 2, 2], 2)
    assert np.array_equal(out, np.stack([rows[0] + rows[1], rows[2] + rows[3]]))
    rows8 = np.arange(32, dtype=np.float32).reshape(8, 4)
    out = topk_reduce(rows8, [1, -1, 1, 2, -1, -1, 2, -1], 2)
    assert np.array_equal(out, np.stack([rows8[0] + rows8[2], rows8[3] + rows8[6]]))


def _block_case(seed, T=10, H=256, I=128, E=4):
    rng = np.random.default_rng(seed)
    x = rng.normal(0, 1, (T, H)).astype(np.float32)
    gamma = rng.normal(1, 0.1, H).astype(np.float32)
    wr = (rng.normal(0, 0.05, (E, H))).astype(np.float32)
    q13, s13, q2, s2 = [], [], [], []
    for _ in range(E):
        a, sa = quant_weight_128x128(rng.normal(0, 0.02, (2 * I, H)).astype(np.float32))
        b, sb = quant_weight_128x128(rng.normal(0, 0.02, (H, I)).astype(np.float32))
        q13.append(a), s13.append(sa), q2.append(b), s2.append(sb)
    return x, gamma, wr, (np.stack(q13), np.stack(s13), np.stack(q2), np.stack(s2))


def test_block_tkg_no_scale_all_experts_is_the_dense_form():
    from oracle.moe import bf16_round, moe_block_tkg_fp8
    from oracle.router import SOFTMAX, rms_norm_padded
    x, gamma, wr, (q13, s13, q2, s2) = _block_case(21)
    E, H, I = q13.shape[0], x.shape[1], q13.shape[1] // 2
    out, _, ids, w = moe_block_tkg_fp8(x, gamma, 1e-6, wr, None, E, SOFTMAX, True, False, False,
                                       q13, s13, q2, s2)
    assert np.all(w == 1)
    xn = bf16_round(rms_norm_padded(x, gamma, 1e-6))
    gu = np.stack([dequant_weight_128x128(q13[e], s13[e]).T.reshape(H, 2, I) for e in range(E)])
    dn = np.stack([dequant_weight_128x128(q2[e], s2[e]).T for e in range(E)])
    dense = moe_dense_reference(xn, np.ones((x.shape[0] * E, 1), np.float32), gu, dn)
    # the dense form has unquantized activations: fp8 activation error only
    err = np.linalg.norm(out - dense) / np.linalg.norm(dense)
    assert err < 5e-2, err


def test_block_tkg_scaling_modes_and_selection_order():
    from oracle.moe import moe_block_tkg_fp8
    from oracle.router import SOFTMAX
    x, gamma, wr, ws = _block_case(22)
    T = x.shape[0]
    # K = 1: POST_SCALE is NO_SCALE times the affinity, exactly
    no, lg, ids1, _ = moe_block_tkg_fp8(x, gamma, 1e-6, wr, None, 1, SOFTMAX, True, False, False, *ws)
    post, _, ids2, w = moe_block_tkg_fp8(x, gamma, 1e-6, wr, None, 1, SOFTMAX, True, False, True, *ws)
    assert np.array_equal(ids1, ids2)
    assert np.array_equal(post, (no * w[:, :1]).astype(np.float32))
    # softmax before top-k: global probabilities (sum < 1); after: softmax of the k (sum 1)
    _, _, ia, wa = moe_block_tkg_fp8(x, gamma, 1e-6, wr, None, 2, SOFTMAX, True, False, True, *ws)
    _, _, ib, wb = moe_block_tkg_fp8(x, gamma, 1e-6, wr, None, 2, SOFTMAX, False, False, True, *ws)
    assert np.array_equal(ia, ib)
    assert np.all(wa.sum(1) < 1 - 1e-3) and np.allclose(wb.sum(1), 1, atol=1e-6)
    # padding columns do not reach the output
    xp = x.copy()
    xp[:, 200:] = 50.0
    a, *_ = moe_block_tkg_fp8(x, gamma, 1e-6, wr, None, 2, SOFTMAX, True, True, True, *ws,
                              hidden_actual=200)
    b, *_ = moe_block_tkg_fp8(xp, gamma, 1e-6, wr, None, 2, SOFTMAX, True, True, True, *ws,
                              hidden_actual=200)
    assert np.array_equal(a, b)
    # token permutation commutes with the layer
    p = np.random.default_rng(0).permutation(T)
    c, *_ = moe_block_tkg_fp8(x[p], gamma, 1e-6, wr, None, 2, SOFTMAX, True, True, True, *ws)
    d, *_ = moe_block_tkg_fp8(x, gamma, 1e-6, wr, None, 2, SOFTMAX, True, True, True, *ws)
    assert np.array_equal(c, d[p])


def test_channel_scales_equal_the_dense_form_and_scale_exactly():
    """Per-channel weight scales (the reference's FP8 row / static formats): the sparse
    form with chan = (c13, c2) equals _torch_moe_impl's dense form on weights whose rows
    were multiplied by the scales beforehand; doubling the up-half scales or the down
    scales doubles the output exactly (powers of two commute with every rounding)."""
    from oracle.fp8 import dequant_act_1x128, quant_act_1x128
    x, ids, w, q13, s13, q2, s2 = _small_layer(5)
    E, I2, H = q13.shape
    I = I2 // 2
    T = x.shape[0]
    rng = np.random.default_rng(6)
    c13 = rng.uniform(0.5, 2.0, (E, I2)).astype(np.float32)
    c2 = rng.uniform(0.5, 2.0, (E, H)).astype(np.float32)
    got = moe_sparse_fp8(x, ids, w, q13, s13, q2, s2, requant_h=False, chan=(c13, c2))
    xh = dequant_act_1x128(*quant_act_1x128(x))
    w13 = np.stack([dequant_weight_128x128(q13[e], s13[e]) * c13[e][:, None] for e in range(E)])
    w2 = np.stack([dequant_weight_128x128(q2[e], s2[e]) * c2[e][:, None] for e in range(E)])
    gate_up = np.stack([w13[:, :I, :], w13[:, I:, :]], axis=2).transpose(0, 3, 2, 1)
    aff = scatter_dense(ids, w, E).reshape(T * E, 1)
    dense = moe_dense_reference(xh, aff, gate_up, w2.transpose(0, 2, 1))
    assert np.allclose(got, dense, rtol=1e-4, atol=1e-5)
    assert not np.allclose(got, moe_sparse_fp8(x, ids, w, q13, s13, q2, s2, requant_h=False),
                           rtol=1e-2, atol=1e-3)
    base = moe_sparse_fp8(x, ids, w, q13, s13, q2, s2, chan=(c13, c2))
    up2 = c13.copy()
    up2[:, I:] *= 2
    assert np.array_equal(moe_sparse_fp8(x, ids, w, q13, s13, q2, s2, chan=(up2, c2)), 2 * base)
    assert np.array_equal(moe_sparse_fp8(x, ids, w, q13, s13, q2, s2, chan=(c13, 2 * c2)), 2 * base)
