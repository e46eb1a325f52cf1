"""Whole-layer GPU parity: the HIP pipeline (router -> top-k -> align -> act quant ->
fp8 gate_up/SiLU -> fp8 down -> combine) against the oracle.

Gates: routing ids and weights bit-exact when the oracle selector is fed the GPU's
logits; logits within fp32 summation-order tolerance; output rel-L2 <= 1e-2 against
the fp32-accumulate dequant oracle that consumes the same fp8 operands."""
import numpy as np
import pytest
import torch

from _routing_audit import audit
from _util import np_f32, np_u8, oracle_shared, oracle_weights, rel_l2, say
from oracle import router as R
from oracle.moe import bf16_round, moe_sparse_fp8
from vllm_neuron_amd import FP8BlockMoE, MoEConfig, PRESETS, ops, synthetic

pytestmark = pytest.mark.gpu
TOL_REL_L2 = 1e-2


def _route_oracle(cfg, lg, w):
    sc = R.SOFTMAX if cfg.scoring == "softmax" else R.SIGMOID
    if cfg.grouped:
        return R.route_grouped(lg, None if w.corr_bias is None else np_f32(w.corr_bias), cfg.top_k,
                               cfg.n_group, cfg.topk_group, sc, cfg.renorm, 1e-20, cfg.routed_scaling)
    return R.route_topk_act(lg, cfg.top_k, sc, cfg.renorm, 1e-20, cfg.routed_scaling)


def _routing_audit(cfg, w, ref_lg, lg, ids, tag):
    """The oracle end to end (its own logits -> its own ids) against the GPU's ids:
    every token that differs must be a near-tie within the logits tolerance."""
    oi, _ = _route_oracle(cfg, ref_lg, w)
    sc = R.SOFTMAX if cfg.scoring == "softmax" else R.SIGMOID
    rep = audit(ref_lg, lg, ids, oi, cfg.top_k, sc, cfg.grouped,
                None if (not cfg.grouped or w.corr_bias is None) else np_f32(w.corr_bias),
                cfg.n_group if cfg.grouped else 1, cfg.topk_group if cfg.grouped else 1)
    say(tag, "routing audit", {k: v for k, v in rep.items() if k != "unexplained"},
        "unexplained", rep["unexplained"][:10])
    assert not rep["unexplained"], (tag, rep["unexplained"][:10])


def _check_layer(cfg, w, x, tokens=None, tag=""):
    out, ids, wts, lg = ops.layer_forward(x, w, cfg, return_routing=True)
    torch.cuda.synchronize()
    lg = lg.cpu().numpy()
    ids = ids.cpu().numpy()
    wts = wts.cpu().numpy()
    xs = np_f32(x)
    ref_lg = R.router_logits(xs, np_f32(w.router_w), None if w.router_bias is None else np_f32(w.router_bias))
    assert np.allclose(lg, ref_lg, rtol=1e-5, atol=2e-5), tag
    oi, ow = _route_oracle(cfg, lg, w)
    assert np.array_equal(ids, oi), tag
    assert np.array_equal(wts, ow), tag
    _routing_audit(cfg, w, ref_lg, lg, ids, tag)
    sel = np.arange(x.shape[0]) if tokens is None else np.asarray(tokens)
    experts = set(np.unique(ids[sel]).tolist())
    q13, s13, q2, s2 = oracle_weights(w, experts if tokens is not None else None)
    ref = moe_sparse_fp8(xs[sel], ids[sel], wts[sel], q13, s13, q2, s2, shared=oracle_shared(w),
                         experts=experts)
    got = np_f32(out)[sel]
    err = rel_l2(got, ref)
    err_bf16 = rel_l2(got, bf16_round(ref))
    say(tag, "rel_l2", err, "vs bf16-rounded oracle", err_bf16)
    assert err <= TOL_REL_L2, (tag, err)
    return out


def _op_path(cfg, w, x):
    """The layer of a grouped-routing config run op by op through the C-ABI entry points
    (router logits with their own reduce, top-k, the chunked or one-launch mapping, the
    1x128 quantizer, the expert kernels the layer picks, combine). The layer fuses the
    quantization into its router launch and, at decode sizes, the mapping into its top-k
    launch; every output must be the same bits."""
    T = x.shape[0]
    E, K, B = cfg.n_experts, cfg.top_k, cfg.block_size
    lg = ops.router_logits(x, w.router_w, w.router_bias)
    ids, wts = ops.router_topk(lg, K, ops.ORDER_GROUPED, cfg.scoring, cfg.n_group, cfg.topk_group,
                               w.corr_bias, cfg.renorm, 1e-20, cfg.routed_scaling)
    m = ops.blockwise_mapping(ids=ids, n_experts=E, block_size=B)
    tpid, b2e = m["token_position_to_id"], m["block_to_expert"]
    NB = tpid.numel()
    xq, xs = ops.act_quant(x)
    if ops.use_block_kernels(T, K, E):
        tiles, num, mbt = ops.build_block_tiles(tpid, b2e, B, T, K, E, cfg.n_shared)
        hq, hs = ops.expert_gate_up_block(xq, xs, w, tpid, NB, tiles, num, mbt)
        y = ops.expert_down_block(hq, hs, w, T, NB, tiles, num, mbt)
    else:
        mt = ops.choose_mt(T, K, E)
        tiles, num, mx = ops.build_tiles(tpid, b2e, B, T, K, E, cfg.n_shared, mt)
        hq, hs = ops.expert_gate_up(xq, xs, w, tpid, NB, tiles, num, mx, mt)
        y = ops.expert_down(hq, hs, w, T, NB, tiles, num, mx, mt)
    return ops.combine(y, m["inv_pos"], wts, T, cfg.hidden, NB, cfg.n_shared)


def test_layer_small_config(cuda):
    """64 tokens, H 1024, I 512, 8 experts, softmax top-2, no shared expert."""
    cfg = PRESETS["small"]
    say("layer small")
    w = synthetic.make_weights(cfg, 0, device=cuda)
    x = synthetic.hidden_states(64, cfg.hidden, 0).to(cuda)
    _check_layer(cfg, w, x, tag="small")


def test_layer_tiny_grouped_with_shared(cuda):
    cfg = MoEConfig(512, 256, 16, 4, n_shared=1, scoring="sigmoid", grouped=True, n_group=4,
                    topk_group=2, renorm=True, routed_scaling=2.5)
    say("layer tiny grouped")
    w = synthetic.make_weights(cfg, 11, device=cuda)
    for T in (1, 5, 64, 333):
        x = synthetic.hidden_states(T, cfg.hidden, 11).to(cuda)
        _check_layer(cfg, w, x, tag=f"tiny T={T}")


def test_layer_full_k_dims(cuda):
    """DeepSeek-V3 hidden/intermediate sizes (K = 7168 and 2048) on 16 experts."""
    cfg = PRESETS["dsv3"].with_(n_experts=16, n_group=8, topk_group=4, top_k=4)
    say("layer full dims")
    w = synthetic.make_weights(cfg, 12, device=cuda)
    x = synthetic.hidden_states(64, cfg.hidden, 12).to(cuda)
    _check_layer(cfg, w, x, tag="dsv3 dims E=16")


def test_layer_zipf_skew_with_empty_experts(cuda):
    """Skewed routing (Zipf 1.2 logit bias, 10% of experts never chosen) with a shared expert."""
    cfg = PRESETS["glm45"].with_(hidden=1024, intermediate=512, n_experts=40)
    say("layer zipf")
    w = synthetic.make_weights(cfg, 4, device=cuda, zipf=True)
    x = synthetic.hidden_states(512, cfg.hidden, 4).to(cuda)
    _check_layer(cfg, w, x, tag="zipf")
    ids = ops.layer_forward(x, w, cfg, return_routing=True)[1].cpu().numpy()
    counts = np.bincount(ids.reshape(-1), minlength=40)
    assert (counts == 0).sum() >= 4 and counts.max() > 4 * counts[counts > 0].mean() / 2


def test_layer_row_tile_heights_agree(cuda):
    """The op-by-op pipeline gives bit-identical outputs for every row-tile height, and
    agrees with the layer entry point (which picks the block kernels at this size)."""
    cfg = MoEConfig(1024, 256, 12, 3, n_shared=1, scoring="sigmoid", grouped=True, n_group=4,
                    topk_group=2, renorm=True, routed_scaling=1.5, block_size=64)
    say("layer mt variants")
    w = synthetic.make_weights(cfg, 13, device=cuda)
    T = 200
    x = synthetic.hidden_states(T, cfg.hidden, 13).to(cuda)
    ref = ops.layer_forward(x, w, cfg)
    lg = ops.router_logits(x, w.router_w, w.router_bias)
    ids, wts = ops.router_topk(lg, cfg.top_k, ops.ORDER_GROUPED, cfg.scoring, cfg.n_group,
                               cfg.topk_group, w.corr_bias, cfg.renorm, 1e-20, cfg.routed_scaling)
    m = ops.blockwise_mapping(ids=ids, n_experts=cfg.n_experts, block_size=cfg.block_size)
    xq, xs = ops.act_quant(x)
    NB = m["token_position_to_id"].numel()
    outs = []
    for mt in (16, 32, 64, 128):
        tiles, num, mx = ops.build_tiles(m["token_position_to_id"], m["block_to_expert"], cfg.block_size,
                                         T, cfg.top_k, cfg.n_experts, 1, mt)
        hq, hs = ops.expert_gate_up(xq, xs, w, m["token_position_to_id"], NB, tiles, num, mx, mt)
        y = ops.expert_down(hq, hs, w, T, NB, tiles, num, mx, mt)
        outs.append(ops.combine(y, m["inv_pos"], wts, T, cfg.hidden, NB, 1))
    # the row-tile kernels agree bit for bit across tile heights; the layer itself runs
    # the block kernels here (50 rows per expert), whose MFMA shape differs
    assert ops.use_block_kernels(T, cfg.top_k, cfg.n_experts)
    for o in outs:
        assert torch.equal(o, outs[0])
    assert rel_l2(np_f32(ref), np_f32(outs[0])) < 5e-3


@pytest.mark.parametrize("T,E", [(64, 64), (4096, 128), (1, 384), (7, 1024), (100, 256),
                                 (255, 384), (300, 256)])
def test_layer_router_matches_op_path(cuda, T, E):
    """Inside the layer the top-k kernel sums the router's split-K partials itself (28
    partials at 64 tokens and below; 8 from the 128-token wide tiles at 4096). Up to 256
    tokens and 512 experts the top-k launch also builds the mapping (its last workgroup),
    with one token per workgroup up to 64 tokens and ceil(T / 64) above (two at T = 100,
    four at T = 255, three in the last workgroup); otherwise four tokens per workgroup
    (T = 7 with 1024 experts: three in the last; T = 300). Logits, ids and weights equal,
    bit for bit, those of ops.router_logits (reduce kernel) followed by ops.router_topk."""
    cfg = PRESETS["dsv3"].with_(n_experts=E, intermediate=128, n_group=8, topk_group=4)
    say("layer router vs op path", T, E)
    w = synthetic.make_weights(cfg, 30 + E, device=cuda)
    x = synthetic.hidden_states(T, cfg.hidden, 30 + E).to(cuda)
    _, ids, wts, lg = ops.layer_forward(x, w, cfg, return_routing=True)
    lg2 = ops.router_logits(x, w.router_w, w.router_bias)
    ids2, wts2 = ops.router_topk(lg2, cfg.top_k, ops.ORDER_GROUPED, cfg.scoring, cfg.n_group,
                                 cfg.topk_group, w.corr_bias, cfg.renorm, 1e-20, cfg.routed_scaling)
    assert torch.equal(lg, lg2) and torch.equal(ids, ids2) and torch.equal(wts, wts2)
    if T in (100, 255):  # the mapping built by the top-k launch's last workgroup
        _check_layer(cfg, w, x, tag=f"router op path T={T} E={E}")


def test_layer_deterministic_and_module_api(cuda):
    cfg = PRESETS["small"]
    say("layer determinism")
    w = synthetic.make_weights(cfg, 0, device=cuda)
    x = synthetic.hidden_states(64, cfg.hidden, 0).to(cuda)
    layer = FP8BlockMoE(cfg, w)
    a = layer(x, positions=None, is_decode=True)
    b = layer(x.reshape(1, 64, -1), positions=None, is_decode=False).reshape(64, -1)
    assert torch.equal(a, b)
    pos = torch.arange(64, device=cuda)
    pos[50:] = 0                                    # padding after the last real position
    c = layer(x, positions=pos, is_decode=False)
    assert torch.equal(c[:50], a[:50]) and torch.all(c[50:] == 0)
    # rank (the tensor-parallel rank) does not change the result with every expert local
    assert torch.equal(layer(x, None, True, torch.tensor([1])), a)
    with pytest.raises(NotImplementedError):
        layer(x, None, False, None, rsag_dispatch=True)


def _big_weights(cfg, idx, cuda):
    return synthetic.make_weights(cfg, idx, device=cuda, experts_device=cuda)


@pytest.mark.parametrize("T,idx,tokens", [(64, 1, [0, 17, 40, 63]), (8192, 2, [0, 4097, 8191])])
def test_layer_dsv3_full_size(cuda, T, idx, tokens):
    """DeepSeek-V3 layer (256 experts + 1 shared): decode 64 and prefill 8192 tokens.
    Outputs are per token, so the oracle checks a token subset (only their experts are
    dequantized on the host), plus the tokens in the last slot of experts whose last
    256-row tiles cover every 64-row band; routing is checked bit-exact for every token."""
    cfg = PRESETS["dsv3"]
    say("layer dsv3 full", T)
    w = _big_weights(cfg, idx, cuda)
    x = synthetic.hidden_states(T, cfg.hidden, idx).to(cuda)
    ids = ops.layer_forward(x, w, cfg, return_routing=True)[1].cpu().numpy()
    tokens, experts = _tile_tokens(ids, cfg.n_experts, extra=tokens)
    say("dsv3 tokens", tokens, "experts", experts)
    out = _check_layer(cfg, w, x, tokens=tokens, tag=f"dsv3 T={T}")
    if T <= 256:  # every token: the op-by-op path gives the same bits
        assert torch.equal(out, _op_path(cfg, w, x))
    del w
    torch.cuda.empty_cache()


def _block_op_path(cfg, w, x):
    """The grouped-routing layer op by op through the block kernels: the routing, the
    mapping, the operands and y (unweighted expert outputs per slot row) besides the
    combined output."""
    T, E, K, B = x.shape[0], cfg.n_experts, cfg.top_k, cfg.block_size
    lg = ops.router_logits(x, w.router_w, w.router_bias)
    ids, wts = ops.router_topk(lg, K, ops.ORDER_GROUPED, cfg.scoring, cfg.n_group, cfg.topk_group,
                               w.corr_bias, cfg.renorm, 1e-20, cfg.routed_scaling)
    m = ops.blockwise_mapping(ids=ids, n_experts=E, block_size=B)
    tpid, b2e = m["token_position_to_id"], m["block_to_expert"]
    NB = tpid.numel()
    xq, xs = ops.act_quant(x)
    tiles, num, mbt = ops.build_block_tiles(tpid, b2e, B, T, K, E, cfg.n_shared)
    hq, hs = ops.expert_gate_up_block(xq, xs, w, tpid, NB, tiles, num, mbt)
    y = ops.expert_down_block(hq, hs, w, T, NB, tiles, num, mbt)
    out = ops.combine(y, m["inv_pos"], wts, T, cfg.hidden, NB, cfg.n_shared)
    return dict(ids=ids, wts=wts, m=m, tpid=tpid, b2e=b2e, NB=NB, xq=xq, xs=xs, y=y, out=out,
                tiles=(tiles, num, mbt))


def _check_expert_rows(cfg, w, x, p, experts, tag):
    """Every slot row of y of each expert in `experts` against the oracle's expert MLP
    on the same fp8 operands (slots hold an expert's tokens in ascending order)."""
    from oracle.fp8 import dequant_act_1x128, dequant_weight_128x128, quant_act_1x128
    from oracle.moe import expert_mlp
    counts = p["m"]["expert_counts"].cpu().numpy()
    tp, b2 = p["tpid"].cpu().numpy(), p["b2e"].cpu().numpy()
    xhat = dequant_act_1x128(*quant_act_1x128(np_f32(x)))
    for e in experts:
        first = int(np.nonzero(b2 == e)[0][0]) * cfg.block_size
        slots = np.arange(first, first + counts[e])
        toks = tp[slots]
        assert np.all(toks >= 0) and np.all(np.diff(toks) > 0)
        w13 = dequant_weight_128x128(np_u8(w.w13[e]), np_f32(w.w13_scale[e]))
        w2 = dequant_weight_128x128(np_u8(w.w2[e]), np_f32(w.w2_scale[e]))
        ref = expert_mlp(xhat[toks], w13, w2)
        got = np_f32(p["y"][torch.from_numpy(slots).to(x.device)])
        err = rel_l2(got, ref)
        say(tag, "expert", e, "rows", counts[e], "rel_l2", err)
        assert err <= TOL_REL_L2, (tag, e, err)
    return xhat


def test_dsv3_prefill_every_row_of_chosen_experts(cuda):
    """DeepSeek-V3 prefill (8192 tokens) through the block kernels: every slot row of y
    (the unweighted expert outputs) of several whole experts against the oracle's expert
    MLP on the same fp8 operands: experts whose second 256-row tile is partial (1-64 and
    65-128 rows), the most loaded one, one below 256 rows, and the shared expert's last
    two tiles. The same routing through the row-tile kernels (128-row tiles) agrees
    with the block kernels on the whole layer output."""
    from oracle.fp8 import dequant_weight_128x128
    from oracle.moe import expert_mlp
    cfg = PRESETS["dsv3"]
    T, E, K, B = 8192, cfg.n_experts, cfg.top_k, cfg.block_size
    say("dsv3 prefill every row", T)
    w = _big_weights(cfg, 2, cuda)
    x = synthetic.hidden_states(T, cfg.hidden, 2).to(cuda)
    p = _block_op_path(cfg, w, x)
    counts = p["m"]["expert_counts"].cpu().numpy()
    picks = []
    for lo, hi in ((256, 320), (320, 384)):
        band = np.nonzero((counts > lo) & (counts <= hi))[0]
        if band.size:
            picks.append(int(band[0]))
    picks.append(int(np.argmax(counts)))
    small = np.nonzero((counts > 0) & (counts < 256))[0]
    if small.size:
        picks.append(int(small[0]))
    picks = list(dict.fromkeys(picks))
    assert len(picks) >= 3, counts
    say("experts", picks, "counts", counts[picks].tolist())
    xhat = _check_expert_rows(cfg, w, x, p, picks, "dsv3 8192")
    NB, y = p["NB"], p["y"]
    # shared expert: slots NB + t; its last two 256-row tiles
    sh = np.arange(T - 512, T)
    w13 = dequant_weight_128x128(np_u8(w.shared_w13[0]), np_f32(w.shared_w13_scale[0]))
    w2 = dequant_weight_128x128(np_u8(w.shared_w2[0]), np_f32(w.shared_w2_scale[0]))
    ref = expert_mlp(xhat[sh], w13, w2)
    got = np_f32(y[NB + T - 512:NB + T])
    err = rel_l2(got, ref)
    say("shared expert last tiles rel_l2", err)
    assert err <= TOL_REL_L2, err
    # row-tile kernels on the same routing and operands
    tpid, b2e, xq, xs = p["tpid"], p["b2e"], p["xq"], p["xs"]
    tiles, num, mx = ops.build_tiles(tpid, b2e, B, T, K, E, 1, 128)
    hq2, hs2 = ops.expert_gate_up(xq, xs, w, tpid, NB, tiles, num, mx, 128)
    y2 = ops.expert_down(hq2, hs2, w, T, NB, tiles, num, mx, 128)
    out_row = ops.combine(y2, p["m"]["inv_pos"], p["wts"], T, cfg.hidden, NB, 1)
    err = rel_l2(np_f32(out_row), np_f32(p["out"]))
    say("row tiles vs block kernels rel_l2", err)
    assert err < 5e-3, err
    assert torch.equal(p["out"], ops.layer_forward(x, w, cfg))
    del w, y, y2, hq2, p
    torch.cuda.empty_cache()


@pytest.fixture(scope="module")
def kimi_weights(cuda):
    w = _big_weights(PRESETS["kimi_k2"], 3, cuda)
    yield w
    del w
    torch.cuda.empty_cache()


def _tile_tokens(ids, E, extra=(), n_experts=6):
    """Tokens that put the oracle on the last (partial) 256-row tile of several experts.

    Slots hold an expert's tokens in ascending order, so the expert's largest token id
    sits in its last slot, on its last tile. The experts are picked by count mod 256
    (one per 64-row band of the last tile's height, then the most and least loaded)."""
    ids = np.asarray(ids)
    counts = np.bincount(ids.reshape(-1), minlength=E)
    live = np.nonzero(counts)[0]
    rem = (counts[live] - 1) % 256 + 1                    # rows of each expert's last tile
    picks = []
    for lo in (0, 64, 128, 192):
        band = live[(rem > lo) & (rem <= lo + 64)]
        if band.size:
            picks.append(int(band[np.argmax(counts[band])]))
    picks += [int(live[np.argmax(counts[live])]), int(live[np.argmin(counts[live])])]
    picks = list(dict.fromkeys(picks))[:n_experts]
    toks = {int(np.nonzero((ids == e).any(axis=1))[0].max()) for e in picks}
    return sorted(toks | set(extra)), picks


@pytest.mark.parametrize("T", [1, 16, 256, 2048, 16384])
def test_layer_kimi_k2_full_size(cuda, kimi_weights, T):
    """Kimi-K2 layer (384 experts + 1 shared, sigmoid top-8 over one group, x2.827) over
    its whole token sweep: 1 and 16 tokens (16-row tiles), 256 (32-row tiles), 2048
    (block kernels on mostly one partial tile per expert, ~43 rows) and 16384 (block
    kernels, ~341 rows per expert). The oracle checks the first and last token and the
    tokens in the last slot of experts whose last tiles cover every 64-row band; up to
    2048 tokens every token also equals the op-by-op path bit for bit."""
    cfg = PRESETS["kimi_k2"]
    say("layer kimi-k2 full", T)
    x = synthetic.hidden_states(T, cfg.hidden, 3).to(cuda)
    ids = ops.layer_forward(x, kimi_weights, cfg, return_routing=True)[1].cpu().numpy()
    tokens, experts = _tile_tokens(ids, cfg.n_experts, extra=(0, T - 1))
    say("kimi tokens", tokens, "experts", experts)
    out = _check_layer(cfg, kimi_weights, x, tokens=tokens, tag=f"kimi T={T}")
    if T <= 2048:  # every token: the op-by-op path gives the same bits
        assert torch.equal(out, _op_path(cfg, kimi_weights, x))


@pytest.mark.parametrize("T,B", [(100, 256), (128, 16), (160, 256), (256, 64), (256, 16)])
def test_layer_fused_mapping_tile_heights(cuda, T, B):
    """Up to 256 tokens the layer's top-k launch ends in the mapping and writes the tile
    list from each expert's own thread. A small grouped layer (32 experts, top-8, four
    groups with two kept, one shared expert) reaches the tile heights the full-size
    configs do not at these token counts: 25-32 rows per expert (64-row tiles) and
    40-64 (block tiles with their XCD cuts), with 256- and 16-slot blocks. Every token
    against the oracle, and the op-by-op path (separate mapping and tile-list kernels)
    bit for bit."""
    cfg = MoEConfig(1024, 512, 32, 8, n_shared=1, scoring="sigmoid", grouped=True, n_group=4,
                    topk_group=2, renorm=True, routed_scaling=2.5, block_size=B)
    block = ops.use_block_kernels(T, cfg.top_k, cfg.n_experts)
    say("layer fused mapping", T, B, "block" if block else f"mt {ops.choose_mt(T, cfg.top_k, cfg.n_experts)}")
    w = synthetic.make_weights(cfg, 7, device=cuda, experts_device=cuda)
    x = synthetic.hidden_states(T, cfg.hidden, 7).to(cuda)
    out = _check_layer(cfg, w, x, tag=f"fused mapping T={T} B={B}")
    assert torch.equal(out, _op_path(cfg, w, x))


@pytest.mark.parametrize("B,S,K", [(256, 1, 8), (16, 2, 4), (1, 0, 1), (64, 1, 2), (3, 2, 8)])
def test_layer_one_token_mapping(cuda, B, S, K):
    """At one token the top-k launch's mapping is written by one wave: each selected
    expert e gets block, slot, compact row and tile rank(e) (its place among the
    selected experts), and the shared experts' tiles follow. Over block sizes (1, 3,
    16, 64, 256 slots), 0-2 shared experts and top-1/2/4/8 the layer equals the
    oracle and the op-by-op path (the general mapping kernel and tile builder) bit for
    bit."""
    cfg = MoEConfig(1024, 512, 32, K, n_shared=S, scoring="sigmoid", grouped=True, n_group=4,
                    topk_group=2, renorm=True, routed_scaling=2.5, block_size=B)
    say("layer one-token mapping", B, S, K)
    w = synthetic.make_weights(cfg, 11, device=cuda, experts_device=cuda)
    for seed in (11, 12):
        x = synthetic.hidden_states(1, cfg.hidden, seed).to(cuda)
        out = _check_layer(cfg, w, x, tag=f"one-token mapping B={B} S={S} K={K} seed={seed}")
        assert torch.equal(out, _op_path(cfg, w, x))


@pytest.mark.parametrize("B", [256, 3])
def test_layer_one_token_fewer_candidates_than_top_k(cuda, B):
    """A NaN correction bias makes every expert but three a NaN key, which is never
    selected: at one token the top-8 holds three experts and five -1 ids, so the
    one-token mapping has three blocks, three tiles and the shared expert's, and five
    pairs with no row. The layer equals the op-by-op path (the general mapping kernel
    and tile builder) bit for bit, and its routing equals ops.router_topk's."""
    cfg = MoEConfig(1024, 512, 32, 8, n_shared=1, scoring="sigmoid", grouped=True, n_group=1,
                    topk_group=1, renorm=True, routed_scaling=2.5, block_size=B)
    say("layer one token, fewer candidates", B)
    w = synthetic.make_weights(cfg, 13, device=cuda, experts_device=cuda)
    cb = torch.full((cfg.n_experts,), float("nan"), device=cuda)
    cb[[3, 17, 29]] = torch.tensor([0.01, -0.02, 0.0], device=cuda)
    w.corr_bias = cb
    x = synthetic.hidden_states(1, cfg.hidden, 13).to(cuda)
    out, ids, wts, lg = ops.layer_forward(x, w, cfg, return_routing=True)
    ids2, wts2 = ops.router_topk(lg, cfg.top_k, ops.ORDER_GROUPED, cfg.scoring, cfg.n_group,
                                 cfg.topk_group, w.corr_bias, cfg.renorm, 1e-20, cfg.routed_scaling)
    assert torch.equal(ids, ids2) and torch.equal(wts, wts2)
    got = ids.cpu().numpy()[0]
    assert sorted(got[got >= 0].tolist()) == [3, 17, 29] and int((got == -1).sum()) == 5
    assert torch.equal(out.view(torch.int16), _op_path(cfg, w, x).view(torch.int16))


def test_layer_glm45_full_size_zipf(cuda):
    """GLM-4.5 layer (hidden 5120, intermediate 1536, 160 experts + 1 shared) at 4096
    tokens with Zipf(1.2) expert popularity and 10% of the experts empty: overfull
    experts span many 256-row tiles, empty ones none. The oracle checks the tokens in
    the last slot of experts whose last tiles cover every 64-row band (and the most and
    least loaded), every token equals the op-by-op path bit for bit, and every slot
    row of the two heaviest experts is checked against the oracle's expert MLP."""
    cfg = PRESETS["glm45"]
    say("layer glm-4.5 full zipf")
    w = synthetic.make_weights(cfg, 4, device=cuda, zipf=True, experts_device=cuda)
    x = synthetic.hidden_states(4096, cfg.hidden, 4).to(cuda)
    ids = ops.layer_forward(x, w, cfg, return_routing=True)[1].cpu().numpy()
    counts = np.bincount(ids.reshape(-1), minlength=cfg.n_experts)
    assert (counts == 0).sum() >= 16 and counts.max() > 3 * counts[counts > 0].mean()
    tokens, experts = _tile_tokens(ids, cfg.n_experts, extra=(0, 1234, 4095))
    say("glm tokens", tokens, "experts", experts, "counts", counts[experts].tolist())
    out = _check_layer(cfg, w, x, tokens=tokens, tag="glm45 T=4096")
    p = _block_op_path(cfg, w, x)
    assert torch.equal(out, p["out"])
    heavy = [int(e) for e in np.argsort(-counts, kind="stable")[:2]]
    _check_expert_rows(cfg, w, x, p, heavy, "glm45 heaviest")
    del w, out, p
    torch.cuda.empty_cache()


@pytest.mark.parametrize("T,E,K,S", [(2048, 8, 2, 0), (3000, 16, 4, 1), (700, 4, 2, 1)])
def test_layer_block_kernels(cuda, T, E, K, S):
    """Block-kernel path (> 32 rows per expert): block kernels against the oracle,
    including partial 256-row tiles, and agreement with the row-tile kernels."""
    cfg = MoEConfig(1024, 512, E, K, n_shared=S, scoring="sigmoid", grouped=True, n_group=1,
                    topk_group=1, renorm=True, routed_scaling=1.0)
    say("layer block kernels", T, E, K, S)
    assert ops.use_block_kernels(T, K, E)
    w = synthetic.make_weights(cfg, 21 + E, device=cuda)
    x = synthetic.hidden_states(T, cfg.hidden, 21 + E).to(cuda)
    out = _check_layer(cfg, w, x, tag=f"block T={T} E={E}")
    # the same routing through the row-tile kernels (different MFMA shape and order)
    lg = ops.router_logits(x, w.router_w, w.router_bias)
    ids, wts = ops.router_topk(lg, K, ops.ORDER_GROUPED, "sigmoid", 1, 1, w.corr_bias, True, 1e-20, 1.0)
    m = ops.blockwise_mapping(ids=ids, n_experts=E, block_size=256)
    xq, xs = ops.act_quant(x)
    NB = m["token_position_to_id"].numel()
    tiles, num, mx = ops.build_tiles(m["token_position_to_id"], m["block_to_expert"], 256, T, K, E, S, 128)
    hq, hs = ops.expert_gate_up(xq, xs, w, m["token_position_to_id"], NB, tiles, num, mx, 128)
    y = ops.expert_down(hq, hs, w, T, NB, tiles, num, mx, 128)
    alt = ops.combine(y, m["inv_pos"], wts, T, cfg.hidden, NB, S)
    assert rel_l2(np_f32(out), np_f32(alt)) < 5e-3


def test_block_kernels_k_blocks_not_multiple_of_four(cuda):
    """Block kernels with H = 768 (6 K blocks for gate_up: the activation scales load
    one block per step, not four) and I = 384 (3 K blocks for down), against the
    oracle."""
    cfg = MoEConfig(768, 384, 4, 2, n_shared=1, scoring="sigmoid", routed_scaling=1.0)
    T = 1024
    say("block kernels K blocks", cfg.hidden, cfg.intermediate)
    assert ops.use_block_kernels(T, cfg.top_k, cfg.n_experts)
    w = synthetic.make_weights(cfg, 77, device=cuda)
    x = synthetic.hidden_states(T, cfg.hidden, 77).to(cuda)
    _check_layer(cfg, w, x, tag="block K blocks")


def test_block_kernels_every_tile_height(cuda):
    """Block kernels on fixed expert counts whose tiles cover every row-group size
    (1-64, 65-128, 129-192 and 193-256 rows, full 256-row tiles before each
    remainder, and a 141-row shared-expert tail), against the oracle."""
    cfg = MoEConfig(1024, 512, 8, 1, n_shared=1, scoring="sigmoid", routed_scaling=1.0)
    counts = [256 + 30, 256 + 100, 256 + 170, 256 + 250, 50, 120, 190, 255]
    T = sum(counts)
    say("block kernels tile heights", T, counts)
    rng = np.random.default_rng(7)
    ids_np = rng.permutation(np.repeat(np.arange(8), counts)).astype(np.int32).reshape(T, 1)
    wts_np = rng.uniform(0.5, 1.5, size=(T, 1)).astype(np.float32)
    w = synthetic.make_weights(cfg, 40, device=cuda)
    x = synthetic.hidden_states(T, cfg.hidden, 40).to(cuda)
    ids, wts = torch.from_numpy(ids_np).to(cuda), torch.from_numpy(wts_np).to(cuda)
    m = ops.blockwise_mapping(ids=ids, n_experts=8, block_size=256)
    tpid, b2e = m["token_position_to_id"], m["block_to_expert"]
    NB = tpid.numel()
    xq, xs = ops.act_quant(x)
    tiles, num, mx = ops.build_block_tiles(tpid, b2e, 256, T, 1, 8, 1)
    rows = sorted(tiles[:4 * int(num[0].item())].cpu().numpy().reshape(-1, 4)[:, 2].tolist())
    assert {(r - 1) // 64 for r in rows} == {0, 1, 2, 3}, rows
    hq, hs = ops.expert_gate_up_block(xq, xs, w, tpid, NB, tiles, num, mx)
    y = ops.expert_down_block(hq, hs, w, T, NB, tiles, num, mx)
    out = ops.combine(y, m["inv_pos"], wts, T, cfg.hidden, NB, 1)
    # the same tile list runs again with identical results (rows of padding slots
    # are never written, so only live rows are compared)
    live = torch.cat([tpid >= 0, torch.ones(T, dtype=torch.bool, device=cuda)])
    hq2, hs2 = ops.expert_gate_up_block(xq, xs, w, tpid, NB, tiles, num, mx)
    assert torch.equal(hq2.view(torch.uint8)[live], hq.view(torch.uint8)[live])
    assert torch.equal(hs2[live], hs[live])
    assert torch.equal(ops.expert_down_block(hq2, hs2, w, T, NB, tiles, num, mx)[live], y[live])
    q13, s13, q2, s2 = oracle_weights(w, None)
    ref = moe_sparse_fp8(np_f32(x), ids_np, wts_np, q13, s13, q2, s2, shared=oracle_shared(w))
    err = rel_l2(np_f32(out), ref)
    say("tile heights rel_l2", err)
    assert err <= TOL_REL_L2, err


# ---------------------------------------------------------------- the layer's own norm

def _check_layer_norm(cfg, w, x, gamma, residual=None, hidden_actual=None, tokens=None, tag=""):
    """Layer with its pre-MoE RMSNorm (and the fused residual add) against the oracle
    composition: v = bf16(x + residual) -> xn = bf16(RMSNorm(v)) -> router on xn ->
    selection -> experts on xn. The normalized rows come from the same fused kernel
    (ops.rms_norm_quant); the kernel itself is pinned against the oracle's norm in
    test_rms_norm_quant_fused."""
    r = ops.layer_forward(x, w, cfg, return_routing=True, gamma=gamma, eps=1e-6,
                          hidden_actual=hidden_actual, residual=residual)
    if residual is not None:
        out, rsum, ids, wts, lg = r
        assert np.array_equal(np_f32(rsum), bf16_round(np_f32(x) + np_f32(residual))), tag
    else:
        out, ids, wts, lg = r
    xn, _, _, _ = ops.rms_norm_quant(x, gamma, 1e-6, hidden_actual, residual)
    v = np_f32(x) if residual is None else np_f32(rsum)
    ref_xn = R.rms_norm_padded(v, np_f32(gamma), 1e-6, hidden_actual)
    assert np.allclose(np_f32(xn), bf16_round(ref_xn), rtol=2 ** -7, atol=0), tag
    xs = np_f32(xn)
    lg, ids, wts = lg.cpu().numpy(), ids.cpu().numpy(), wts.cpu().numpy()
    ref_lg = R.router_logits(xs, np_f32(w.router_w), None if w.router_bias is None else np_f32(w.router_bias))
    assert np.allclose(lg, ref_lg, rtol=1e-5, atol=2e-5), tag
    oi, ow = _route_oracle(cfg, lg, w)
    assert np.array_equal(ids, oi) and np.array_equal(wts, ow), tag
    _routing_audit(cfg, w, ref_lg, lg, ids, tag)
    sel = np.arange(x.shape[0]) if tokens is None else np.asarray(tokens)
    experts = set(np.unique(ids[sel]).tolist())
    q13, s13, q2, s2 = oracle_weights(w, experts if tokens is not None else None)
    ref = moe_sparse_fp8(xs[sel], ids[sel], wts[sel], q13, s13, q2, s2, shared=oracle_shared(w),
                         experts=experts)
    err = rel_l2(np_f32(out)[sel], ref)
    say(tag, "rel_l2", err)
    assert err <= TOL_REL_L2, (tag, err)
    # without the norm the same layer differs (the norm is applied, not skipped)
    return out


def _gamma(H, seed, device):
    g = torch.Generator().manual_seed(seed)
    return (1 + 0.2 * torch.randn(H, generator=g)).to(torch.bfloat16).float().to(device)


@pytest.mark.parametrize("residual, hidden_actual", [(False, None), (True, None), (True, 1000)])
def test_layer_norm_small(cuda, residual, hidden_actual):
    """Small layer (64 tokens, H 1024) with the layer's own RMSNorm, the residual add
    and a padded hidden size."""
    cfg = PRESETS["small"]
    say("layer norm small", residual, hidden_actual)
    w = synthetic.make_weights(cfg, 0, device=cuda)
    x = (3 * synthetic.hidden_states(64, cfg.hidden, 0)).to(torch.bfloat16).to(cuda)
    r = synthetic.hidden_states(64, cfg.hidden, 7).to(cuda) if residual else None
    gamma = _gamma(cfg.hidden, 1, cuda)
    out = _check_layer_norm(cfg, w, x, gamma, r, hidden_actual, tag=f"norm small {residual}")
    assert not torch.equal(out, ops.layer_forward(x, w, cfg))


@pytest.mark.parametrize("T,idx,tokens", [(64, 1, None), (8192, 2, [0, 3001, 8191])])
def test_layer_norm_dsv3_full_size(cuda, T, idx, tokens):
    """DeepSeek-V3 decode 64 and prefill 8192 with the layer's RMSNorm and residual add."""
    cfg = PRESETS["dsv3"]
    say("layer norm dsv3", T)
    w = _big_weights(cfg, idx, cuda)
    x = synthetic.hidden_states(T, cfg.hidden, idx).to(cuda)
    r = synthetic.hidden_states(T, cfg.hidden, idx + 50).to(cuda)
    gamma = _gamma(cfg.hidden, idx, cuda)
    if tokens is None:
        tokens = [0, 17, 40, 63]
    _check_layer_norm(cfg, w, x, gamma, r, tokens=tokens, tag=f"norm dsv3 T={T}")
    del w
    torch.cuda.empty_cache()


def test_layer_module_norm_and_residual(cuda):
    """FP8BlockMoE with a norm weight: prefill with a residual returns (out, x +
    residual) and equals the functional layer; decode applies the same norm and returns
    one tensor; padding rows after the last real position are zero."""
    cfg = PRESETS["small"]
    say("layer module norm")
    w = synthetic.make_weights(cfg, 0, device=cuda)
    x = synthetic.hidden_states(64, cfg.hidden, 0).to(cuda)
    r = synthetic.hidden_states(64, cfg.hidden, 9).to(cuda)
    gamma = _gamma(cfg.hidden, 2, cuda)
    layer = FP8BlockMoE(cfg, w, norm_weight=gamma.to(torch.bfloat16), eps=1e-6)
    out, rsum = layer(x, positions=None, is_decode=False, rank=None, residual=r)
    ref_out, ref_sum = ops.layer_forward(x, w, cfg, gamma=gamma, eps=1e-6, residual=r)
    assert torch.equal(out, ref_out) and torch.equal(rsum, ref_sum)
    dec = layer(rsum, None, True, None)
    assert torch.equal(dec, ops.layer_forward(rsum, w, cfg, gamma=gamma, eps=1e-6))
    assert torch.equal(dec, out)  # norm(x + r) either way
    pos = torch.arange(64, device=cuda)
    pos[40:] = 0
    pad, _ = layer(x, positions=pos, is_decode=False, residual=r)
    assert torch.equal(pad[:40], out[:40]) and torch.all(pad[40:] == 0)
    with pytest.raises(ValueError):
        FP8BlockMoE(cfg, w)(x, None, False, None, residual=r)


NORM_RIDE_SHAPES = {
    # Kimi-K2's router (7168 columns: 3-4 chunks per thread; 384 experts: 6 x 28 logits
    # workgroups), small experts, with the residual add
    "kimi_router": (MoEConfig(7168, 128, 384, 8, n_shared=1, scoring="sigmoid", grouped=True,
                              n_group=1, topk_group=1, renorm=True, routed_scaling=2.827), None, True),
    # padded hidden size (1000 real columns of 1024), no residual
    "padded": (MoEConfig(1024, 512, 16, 4, n_shared=1, scoring="sigmoid", grouped=True, n_group=4,
                         topk_group=2, renorm=True, routed_scaling=2.5), 1000, False),
    "padded_residual": (MoEConfig(1024, 512, 16, 4, n_shared=1, scoring="sigmoid", grouped=True,
                                  n_group=4, topk_group=2, renorm=True, routed_scaling=2.5), 1000, True),
}


@pytest.mark.parametrize("T", [1, 3, 4, 5])
@pytest.mark.parametrize("shape", sorted(NORM_RIDE_SHAPES))
def test_layer_norm_rides_in_router_launch(cuda, shape, T):
    """Up to four tokens the layer's RMSNorm (with the residual add) runs inside the
    router logits launch: every logits and quantization workgroup reads the token rows
    and computes their norm factors itself, and the quantization workgroups write the
    residual stream. From five tokens the norm is a launch of its own. Either way every
    output is the same bits as the layer without its norm, run on the rows
    ops.rms_norm_quant normalizes (pinned against the oracle's norm in
    test_rms_norm_quant_fused)."""
    cfg, ha, with_res = NORM_RIDE_SHAPES[shape]
    say("norm in the router launch", shape, T)
    w = synthetic.make_weights(cfg, 3, device=cuda)
    x = (2 * synthetic.hidden_states(T, cfg.hidden, 10 + T)).to(torch.bfloat16).to(cuda)
    r = synthetic.hidden_states(T, cfg.hidden, 20 + T).to(cuda) if with_res else None
    gamma = _gamma(cfg.hidden, 4, cuda)
    got = ops.layer_forward(x, w, cfg, return_routing=True, gamma=gamma, eps=1e-6,
                            hidden_actual=ha, residual=r)
    if with_res:
        out, rsum, *routing = got
        assert np.array_equal(np_f32(rsum), bf16_round(np_f32(x) + np_f32(r)))
    else:
        out, *routing = got
    xn = ops.rms_norm_quant(x, gamma, 1e-6, ha, r)[0]
    ref_out, *ref_routing = ops.layer_forward(xn, w, cfg, return_routing=True)
    assert torch.equal(out, ref_out)
    for a, b in zip(routing, ref_routing):  # ids, weights, logits
        assert torch.equal(a, b)
    assert not torch.equal(out, ops.layer_forward(x, w, cfg))  # the norm is applied
