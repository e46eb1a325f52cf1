"""GPU parity of the individual kernels against the oracle (bit-exact for integer,
index and fp8-code work; tolerances stated where the result is floating point)."""
import numpy as np
import pytest
import torch

from _util import np_f32, np_u8, say
from oracle import router as R
from oracle.blockwise import build_blockwise_mapping, mapping_from_ids
from oracle.fp8 import e4m3fn_decode, quant_act_1x128
from vllm_neuron_amd import ops

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("shape,n", [(0, 16), (1, 32)])
def test_mfma_fp8_fragment_layout(cuda, shape, n):
    """Integer-valued operands: every partial sum is exact, so any lane-layout error
    (row/column/K mapping, output placement) shows as an exact mismatch."""
    say("mfma fragment layout", shape)
    from oracle.fp8 import e4m3fn_encode
    rng = np.random.default_rng(shape)
    ai = rng.integers(-8, 9, (n, 128)).astype(np.float32)
    bi = rng.integers(-8, 9, (n, 128)).astype(np.float32)
    ta = torch.from_numpy(e4m3fn_encode(ai)).view(torch.float8_e4m3fn).to(cuda)
    tb = torch.from_numpy(e4m3fn_encode(bi)).view(torch.float8_e4m3fn).to(cuda)
    c = ops.selftest_mfma(ta, tb, shape).cpu().numpy()
    assert np.array_equal(c, ai @ bi.T)


def test_fp8_conversion_instruction_matches_encoder(cuda):
    """The quantizers encode with the gfx950 conversion instruction; it equals the
    integer round-to-nearest-even encoder (the one the oracle's encoder pins through
    the quantizer tests) on every fp32 value in [-448, 448], both signs."""
    say("fp8 encode exhaustive")
    n, first_bad = ops.selftest_fp8_encode()
    assert n == 0, (n, None if first_bad is None else hex(first_bad))


@pytest.mark.parametrize("half", [0, 1])
def test_bf16_conversion_instruction_matches_encoder(cuda, half):
    """The output stages round to bf16 with the gfx950 conversion instruction; it
    equals the integer round-to-nearest-even encoder on every fp32 pattern (NaNs
    stay NaNs), checked in two halves of 2^31 patterns."""
    say("bf16 encode exhaustive", half)
    n, first_bad = ops.selftest_bf16_encode(first=half << 31)
    assert n == 0, (n, None if first_bad is None else hex(first_bad))


@pytest.mark.parametrize("mode", [0, 1])
def test_shared_divisor_division_is_correctly_rounded(cuda, mode):
    """The quantizers' reciprocal-and-correction quotient gives the IEEE division's
    e4m3 code everywhere and its exact fp32 value wherever the code can be nonzero
    (|quotient| >= 2^-10): mode 0 on every (bf16 group amax, bf16 value) pair, mode 1
    on 2^31 random fp32 pairs spanning 80 binades."""
    say("shared-divisor division", mode)
    n, first_bad = ops.selftest_quant_div(mode)
    assert n == 0, (n, None if first_bad is None else hex(first_bad))


def test_mfma_fp8_wide_range_accumulation(cuda):
    """Full-range random codes: products are exact, but the MFMA's inner sum is not an
    exact fp32 sum; it stays within 1e-3 of the largest |product| sum (measured ~1e-4)."""
    say("mfma wide range")
    rng = np.random.default_rng(1)
    finite = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], np.uint8)
    a = rng.choice(finite, (16, 128)).astype(np.uint8)
    b = rng.choice(finite, (16, 128)).astype(np.uint8)
    ta = torch.from_numpy(a).view(torch.float8_e4m3fn).to(cuda)
    tb = torch.from_numpy(b).view(torch.float8_e4m3fn).to(cuda)
    c = ops.selftest_mfma(ta, tb).cpu().numpy()
    da, db = e4m3fn_decode(a).astype(np.float64), e4m3fn_decode(b).astype(np.float64)
    ref = da @ db.T
    scale = np.abs(da) @ np.abs(db).T
    err = np.abs(c - ref) / scale
    say("mfma wide-range max error / sum|products|", float(err.max()))
    assert err.max() < 1e-3


@pytest.mark.parametrize("R_,C,offset", [(64, 1024, 0), (3, 7168, 0), (1, 128, 0), (257, 5120, 0),
                                         (8192, 7168, 0), (5, 384, 2), (33, 1024, 6)])
def test_act_quant_bit_exact(cuda, R_, C, offset):
    """offset > 0 starts x that many bf16 elements into its buffer (4-byte but not
    16-byte aligned), which takes the scalar kernel instead of the vector one."""
    say("act_quant", R_, C, offset)
    g = torch.Generator().manual_seed(R_ * 7 + C)
    x = torch.randn(R_, C, generator=g)
    if R_ > 2:
        x[0, :128] = 0.0
        x[1, :256] *= 1e-30          # bf16 subnormal / tiny range
        x[2, 128:256] *= 1e4
    xb = x.to(torch.bfloat16)
    xd = xb.to(cuda)
    if offset:
        buf = torch.empty(R_ * C + offset, dtype=torch.bfloat16, device=cuda)
        xd = buf[offset:].view(R_, C)
        xd.copy_(xb.to(cuda))
        assert xd.data_ptr() % 16 != 0
    q, s = ops.act_quant(xd)
    torch.cuda.synchronize()
    oq, os_ = quant_act_1x128(xb.float().numpy())
    assert np.array_equal(np_u8(q), oq)
    assert np.array_equal(np_f32(s), os_)


@pytest.mark.parametrize("T,H,E", [(64, 1024, 8), (64, 7168, 256), (300, 5120, 160), (1, 7168, 384),
                                   # wide tiles (T >= 2048, 128 <= E <= 256), ragged last tile
                                   (2100, 1024, 128), (4096, 7168, 256), (2048, 5120, 160)])
def test_router_logits_close(cuda, T, H, E):
    say("router_logits", T, H, E)
    g = torch.Generator().manual_seed(T + H + E)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    w = (torch.randn(E, H, generator=g) * 0.02).to(torch.bfloat16)
    bias = torch.randn(E, generator=g) * 0.1
    lg = ops.router_logits(x.to(cuda), w.to(cuda), bias.to(cuda)).cpu().numpy()
    ref = R.router_logits(x.float().numpy(), w.float().numpy(), bias.numpy())
    # bf16 products are exact in fp32; only the fp32 summation order differs
    assert np.allclose(lg, ref, rtol=1e-5, atol=2e-5)


ROUTER_CASES = [
    # name, E, K, order, scoring, n_group, topk_group, renorm, eps, scale, bias
    ("softmax_topk_act_c0", 8, 2, 0, 0, 1, 1, False, 0.0, 1.0, False),
    ("sigmoid_topk_act", 64, 4, 0, 1, 1, 1, False, 0.0, 1.0, False),
    ("softmax_act_topk_renorm", 128, 6, 1, 0, 1, 1, True, 0.0, 1.0, False),
    ("sigmoid_act_topk_norm_eps", 256, 8, 1, 1, 1, 1, True, 1e-20, 1.0, False),
    ("dsv3_grouped", 256, 8, 2, 1, 8, 4, True, 1e-20, 2.5, True),
    ("kimi_grouped_1group", 384, 8, 2, 1, 1, 1, True, 1e-20, 2.827, True),
    ("glm_160", 160, 8, 2, 1, 1, 1, True, 1e-20, 2.5, True),
    ("grouped_softmax", 64, 6, 2, 0, 8, 3, False, 0.0, 1.0, True),
    ("grouped_1expert_groups", 16, 3, 2, 1, 16, 5, True, 1e-20, 1.0, False),
    # more selections than an 8-long merge list: K rounds of a wave maximum
    ("sigmoid_act_topk_k16_rounds", 128, 16, 1, 1, 1, 1, True, 1e-20, 1.0, False),
    # 1024 experts (16 per lane): merge lists of 16
    ("softmax_topk_act_k12_e1024", 1024, 12, 0, 0, 1, 1, False, 0.0, 1.0, False),
]


@pytest.mark.parametrize("case", ROUTER_CASES, ids=[c[0] for c in ROUTER_CASES])
@pytest.mark.parametrize("T", [1, 77, 2048])
def test_router_topk_bit_exact(cuda, case, T):
    name, E, K, order, scoring, ng, tg, renorm, eps, scale, use_bias = case
    say("router_topk", name, T)
    rng = np.random.default_rng(E * 1000 + T)
    lg = rng.normal(0, 1.5, (T, E)).astype(np.float32)
    lg[: T // 4] = np.round(lg[: T // 4] * 2) / 2         # exact ties in a quarter of the rows
    bias = rng.normal(0, 0.01, E).astype(np.float32) if use_bias else None
    ids, w, aff = ops.router_topk(torch.from_numpy(lg).to(cuda), K, order, scoring, ng, tg,
                                  None if bias is None else torch.from_numpy(bias).to(cuda),
                                  renorm, eps, scale, dense=True)
    sc = R.SOFTMAX if scoring == 0 else R.SIGMOID
    if order == 0:
        oi, ow = R.route_topk_act(lg, K, sc, renorm, eps, scale)
    elif order == 1:
        oi, ow = R.route_act_topk_renorm(lg, K, sc, renorm, eps, scale)
    else:
        oi, ow = R.route_grouped(lg, bias, K, ng, tg, sc, renorm, eps, scale)
    assert np.array_equal(ids.cpu().numpy(), oi)
    assert np.array_equal(w.cpu().numpy(), ow)
    assert np.array_equal(aff.cpu().numpy(), R.scatter_dense(oi, ow, E))


@pytest.mark.parametrize("gs", [32, 8])
def test_router_grouped_nonfinite_group_scores(cuda, gs):
    """Correction biases of +-inf give group scores of +inf, -inf and NaN (+inf + -inf):
    a NaN group ranks below a -inf group, which ranks below every finite group."""
    E, K, ng = 8 * gs, 8, 8
    say("router_topk_nonfinite", gs)
    rng = np.random.default_rng(gs)
    lg = rng.normal(0, 1.5, (64, E)).astype(np.float32)
    bias = rng.normal(0, 0.01, E).astype(np.float32)
    bias[0] = np.inf                  # group 0: +inf and the rest -inf -> NaN
    bias[1:gs] = -np.inf
    bias[gs:2 * gs] = -np.inf         # group 1: all -inf -> -inf
    bias[2 * gs + 3] = np.inf         # group 2: one +inf among finite -> +inf
    for tg in (2, 6, 7):
        ids, w = ops.router_topk(torch.from_numpy(lg).to(cuda), K, 2, 1, ng, tg,
                                 torch.from_numpy(bias).to(cuda), True, 1e-20, 2.5)
        with np.errstate(invalid="ignore"):
            oi, ow = R.route_grouped(lg, bias, K, ng, tg, R.SIGMOID, True, 1e-20, 2.5)
        assert not (oi == 0).any()    # the NaN group is never kept while finite or -inf groups are left
        assert np.array_equal(ids.cpu().numpy(), oi), tg
        assert np.array_equal(w.cpu().numpy(), ow), tg


NAN_ZERO_CASES = [c for c in ROUTER_CASES if c[4] == 1 and (c[3] != 2 or c[5] == 1)]


@pytest.mark.parametrize("case", NAN_ZERO_CASES, ids=[c[0] for c in NAN_ZERO_CASES])
@pytest.mark.parametrize("T", [1, 64])
def test_router_topk_nan_and_signed_zero_keys(cuda, case, T):
    """NaN keys are never selected and -0 ties +0 (then the lower index wins), as in
    the oracle's stable descending sort; rows of mostly tied keys exercise the
    index order. Sigmoid scoring, so a NaN logit leaves the other keys finite."""
    name, E, K, order, scoring, ng, tg, renorm, eps, scale, use_bias = case
    say("router_topk_nan_zero", name, T)
    rng = np.random.default_rng(E + 7 * T)
    lg = rng.normal(0, 1.5, (T, E)).astype(np.float32)
    for t in range(T):
        kind = t % 4 if T > 1 else 0
        if kind == 0:   # NaN keys among finite ones, fewer than E - K of them
            lg[t, rng.choice(E, max(1, (E - K) // 3), replace=False)] = np.nan
            lg[t, rng.choice(E, E // 4, replace=False)] = rng.choice(np.float32([0.0, -0.0]), E // 4)
        elif kind == 1:  # only signed zeros and a few +-1: ties everywhere
            lg[t] = rng.choice(np.float32([0.0, -0.0, 0.0, -0.0, 1.0, -1.0]), E)
        elif kind == 2:  # all keys -0 or +0
            lg[t] = rng.choice(np.float32([0.0, -0.0]), E)
    bias = rng.normal(0, 0.01, E).astype(np.float32) if use_bias else None
    ids, w, aff = ops.router_topk(torch.from_numpy(lg).to(cuda), K, order, scoring, ng, tg,
                                  None if bias is None else torch.from_numpy(bias).to(cuda),
                                  renorm, eps, scale, dense=True)
    with np.errstate(invalid="ignore"):
        if order == 0:
            oi, ow = R.route_topk_act(lg, K, R.SIGMOID, renorm, eps, scale)
        elif order == 1:
            oi, ow = R.route_act_topk_renorm(lg, K, R.SIGMOID, renorm, eps, scale)
        else:
            oi, ow = R.route_grouped(lg, bias, K, ng, tg, R.SIGMOID, renorm, eps, scale)
    assert not np.isnan(lg[np.arange(T)[:, None], oi]).any()
    assert np.array_equal(ids.cpu().numpy(), oi)
    assert np.array_equal(w.cpu().numpy(), ow)
    assert np.array_equal(aff.cpu().numpy(), R.scatter_dense(oi, ow, E))


MAP_CASES = [(1, 8, 256, 256), (7, 2, 8, 4), (64, 2, 8, 256), (64, 8, 256, 256), (300, 8, 160, 16),
             (4096, 8, 160, 256), (8192, 8, 256, 256), (1000, 6, 384, 64), (513, 1, 5, 1),
             (256, 16, 64, 32), (200, 12, 96, 8),  # one chunk, more than 2 ids per thread
             (256, 256, 512, 1), (256, 300, 300, 2)]  # one chunk with >= 2^16 ids: unpacked scans


@pytest.mark.parametrize("T,K,E,B", MAP_CASES)
def test_mapping_from_ids_bit_exact(cuda, T, K, E, B):
    say("mapping ids", T, K, E, B)
    rng = np.random.default_rng(T + K + E + B)
    p = rng.zipf(1.5, E).astype(np.float64)
    p[rng.permutation(E)[: E // 10]] = 0                   # ~10% empty experts, skewed rest
    p = p / p.sum()
    ids = np.stack([rng.choice(E, K, replace=False, p=p) if (p > 0).sum() >= K else
                    rng.choice(E, K, replace=False) for _ in range(T)]).astype(np.int32)
    m = ops.blockwise_mapping(ids=torch.from_numpy(ids).to(cuda), n_experts=E, block_size=B, check=True)
    tpid, b2e, cond, counts, inv = mapping_from_ids(ids, E, B)
    assert np.array_equal(m["token_position_to_id"].cpu().numpy(), tpid)
    assert np.array_equal(m["block_to_expert"].cpu().numpy(), b2e)
    assert np.array_equal(m["conditions"].cpu().numpy(), cond)
    assert np.array_equal(m["expert_counts"].cpu().numpy(), counts)
    assert np.array_equal(m["inv_pos"].cpu().numpy(), inv)


@pytest.mark.parametrize("T,K,E,B", [(64, 2, 8, 256), (300, 8, 160, 16), (2048, 8, 256, 256)])
def test_mapping_from_affinities_bit_exact(cuda, T, K, E, B):
    say("mapping affinities", T, K, E, B)
    rng = np.random.default_rng(T * 3 + E)
    lg = rng.normal(0, 1, (T, E)).astype(np.float32)
    ids, w = R.route_topk_act(lg, K, R.SOFTMAX)
    aff = R.scatter_dense(ids, w, E)
    pm = np.arange(T) < (T - T // 5)
    m = ops.blockwise_mapping(affinities=torch.from_numpy(aff).to(cuda), top_k=K, block_size=B,
                              padding_mask=torch.from_numpy(pm).to(cuda), check=True)
    am, tpid, b2e, cond = build_blockwise_mapping(aff, E, K, B, padding_mask=pm)
    assert np.array_equal(m["affinities_masked"].cpu().numpy(), am)
    assert np.array_equal(m["token_position_to_id"].cpu().numpy(), tpid)
    assert np.array_equal(m["block_to_expert"].cpu().numpy(), b2e)
    assert np.array_equal(m["conditions"].cpu().numpy(), cond)


def test_mapping_overflow_is_reported(cuda):
    say("mapping overflow")
    T, K, E, B = 16, 1, 4, 4
    aff = np.ones((T, E), np.float32)                     # 4 nonzeros per row but top_k = 1
    with pytest.raises(IndexError):
        ops.blockwise_mapping(affinities=torch.from_numpy(aff).to(cuda), top_k=K, block_size=B, check=True)


@pytest.mark.parametrize("mt", [16, 32, 64, 128])
def test_tiles_cover_every_slot_once(cuda, mt):
    say("tiles", mt)
    rng = np.random.default_rng(mt)
    T, K, E, B = 700, 4, 24, 64
    ids = np.stack([rng.choice(E, K, replace=False) for _ in range(T)]).astype(np.int32)
    m = ops.blockwise_mapping(ids=torch.from_numpy(ids).to(cuda), n_experts=E, block_size=B)
    tiles, num, max_tiles = ops.build_tiles(m["token_position_to_id"], m["block_to_expert"], B, T, K, E, 1, mt)
    n = int(num.item())
    tl = tiles[:n].cpu().numpy()
    tpid = m["token_position_to_id"].cpu().numpy()
    b2e = m["block_to_expert"].cpu().numpy()
    NB = tpid.size
    seen = np.zeros(NB + T, np.int32)
    for e, s0, rows, _ in tl:
        assert 1 <= rows <= mt
        for s in range(s0, s0 + rows):
            seen[s] += 1
            if e < E:
                assert b2e[s // B] == e and s // B == s0 // B
            else:
                assert s >= NB
    assert np.all(seen[:NB][tpid >= 0] == 1) and np.all(seen[NB:] == 1)
    assert n <= max_tiles


@pytest.mark.parametrize("T,K,E,B,S", [(700, 4, 24, 64, 1), (4096, 8, 40, 256, 1), (300, 2, 3, 16, 0),
                                       (9000, 8, 256, 256, 1)])
def test_block_tiles_cover_every_slot_once(cuda, T, K, E, B, S):
    """Block tiles: <= 256 consecutive slots of one expert; every routed slot in exactly one
    tile; the segment records let every (tile, column tile) item be recovered."""
    say("block tiles", T, K, E, B)
    rng = np.random.default_rng(T + E)
    p = rng.zipf(1.3, E).astype(np.float64)
    p[: max(1, E // 10)] = 0
    p /= p.sum()
    ids = np.stack([rng.choice(E, K, replace=False, p=p) for _ in range(T)]).astype(np.int32)
    m = ops.blockwise_mapping(ids=torch.from_numpy(ids).to(cuda), n_experts=E, block_size=B)
    tiles, num, mx = ops.build_block_tiles(m["token_position_to_id"], m["block_to_expert"], B, T, K, E, S)
    hdr = num.cpu().numpy()
    n = int(hdr[0])
    raw = tiles.cpu().numpy()
    tl = raw[: 4 * mx].reshape(mx, 4)[:n]
    sg = raw[4 * mx:].reshape(mx, 2)[:n]
    tpid = m["token_position_to_id"].cpu().numpy()
    b2e = m["block_to_expert"].cpu().numpy()
    NB = tpid.size
    seen = np.zeros(NB + S * T, np.int32)
    for t, (e, s0, rows, _) in enumerate(tl):
        assert 1 <= rows <= 256
        first, cnt = sg[t]
        assert first <= t < first + cnt and np.all(tl[first:first + cnt, 0] == e)
        seen[s0:s0 + rows] += 1
        if e < E:
            assert np.all(b2e[np.arange(s0, s0 + rows) // B] == e)
    assert np.all(seen[:NB][tpid >= 0] == 1) and np.all(seen[NB:] == 1)
    assert np.all(seen[:NB][tpid < 0] <= 1)
    # XCD ranges: a partition of the tiles into 8 runs of at most cap tiles (the grid's
    # share per XCD); a cut leaves an expert boundary only where the cap forces it, and
    # with every cut on a boundary each range is within one expert's cost of an equal
    # share (tile cost 3 + ceil(rows / 64))
    cut = hdr[1:10]
    cap = max(3 * mx // 16, (mx + 7) // 8)
    assert cut[0] == 0 and cut[8] == n and np.all(np.diff(cut) >= 0), cut
    assert np.all(np.diff(cut) <= cap), (cut, cap)
    on_boundary = [c in (0, n) or tl[c, 0] != tl[c - 1, 0] for c in cut[1:8]]
    for x, ok in zip(range(1, 8), on_boundary):
        assert ok or cut[x] in (cut[x - 1] + cap, n - (8 - x) * cap), (x, cut, cap)
    if all(on_boundary):
        cost = 3 + (tl[:, 2] + 63) // 64
        pref = np.concatenate([[0], np.cumsum(cost)])
        share = pref[-1] / 8
        seg_cost = max(pref[f + c] - pref[f] for f, c in sg)
        for x in range(8):
            assert pref[cut[x + 1]] - pref[cut[x]] <= share + seg_cost, (x, cut, share, seg_cost)
    say("block tiles", n, "tiles, XCD cuts", cut.tolist(), "cap", cap)


@pytest.mark.parametrize("T,K,S,with_w", [(64, 8, 1, True), (300, 6, 0, True), (5, 2, 2, False),
                                         (1000, 8, 1, True)])
def test_combine_matches_sequential_sum(cuda, T, K, S, with_w):
    """out[t] = sum over t's live slots in slot order of w * y[slot] (+ shared rows, weight 1),
    fp32 accumulation, bf16 result: within one bf16 rounding of the float64 sum. Dead slots
    (-1) are skipped."""
    say("combine", T, K, S, with_w)
    H, NB = 1024, 4096
    rng = np.random.default_rng(T + K + S)
    y = rng.normal(0, 1, (NB + S * T, H)).astype(np.float32)
    inv = rng.choice(NB, (T, K), replace=True).astype(np.int32)
    inv[rng.random((T, K)) < 0.15] = -1
    w = rng.uniform(0.1, 1, (T, K)).astype(np.float32) if with_w else None
    yb = torch.from_numpy(y).to(torch.bfloat16)
    out = ops.combine(yb.to(cuda), torch.from_numpy(inv).to(cuda),
                      None if w is None else torch.from_numpy(w).to(cuda), T, H, NB, S)
    y64 = yb.double().numpy()
    ref = np.zeros((T, H))
    for t in range(T):
        for k in range(K):
            if inv[t, k] >= 0:
                ref[t] += (1.0 if w is None else float(w[t, k])) * y64[inv[t, k]]
        for j in range(S):
            ref[t] += y64[NB + j * T + t]
    got = out.float().cpu().numpy()
    assert np.allclose(got, ref, rtol=2 ** -7, atol=1e-5)
