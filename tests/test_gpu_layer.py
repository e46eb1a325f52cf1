"""Whole-layer GPU parity: the HIP pipeline (router -> top-k -> align -> act quant ->
fp8 gate_up/SiLU -> fp8 down -> combine) against the oracle.

Gates: routing ids and weights bit-exact when the oracle selector is fed the GPU's
logits; logits within fp32 summation-order tolerance; output rel-L2 <= 1e-2 against
the fp32-accumulate dequant oracle that consumes the same fp8 operands."""
import numpy as np
import pytest
import torch

from _util import np_f32, oracle_shared, oracle_weights, rel_l2, say
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


@pytest.mark.parametrize("T,E", [(64, 64), (4096, 128)])
def test_layer_router_matches_op_path(cuda, T, E):
    """Inside the layer the top-k kernel sums the router's split-K partials itself (28
    partials at 64 tokens; 8 from the 128-token wide tiles at 4096). Logits, ids and
    weights equal, bit for bit, those of ops.router_logits (reduce kernel) followed by
    ops.router_topk."""
    cfg = PRESETS["dsv3"].with_(n_experts=E, intermediate=128, n_group=8, topk_group=4)
    say("layer router vs op path", T, E)
    w = synthetic.make_weights(cfg, 30 + E, device=cuda)
    x = synthetic.hidden_states(T, cfg.hidden, 30 + E).to(cuda)
    _, ids, wts, lg = ops.layer_forward(x, w, cfg, return_routing=True)
    lg2 = ops.router_logits(x, w.router_w, w.router_bias)
    ids2, wts2 = ops.router_topk(lg2, cfg.top_k, ops.ORDER_GROUPED, cfg.scoring, cfg.n_group,
                                 cfg.topk_group, w.corr_bias, cfg.renorm, 1e-20, cfg.routed_scaling)
    assert torch.equal(lg, lg2) and torch.equal(ids, ids2) and torch.equal(wts, wts2)


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
    with pytest.raises(NotImplementedError):
        layer(x, None, False, torch.tensor([1]))


def _big_weights(cfg, idx, cuda):
    return synthetic.make_weights(cfg, idx, device=cuda, experts_device=cuda)


@pytest.mark.parametrize("T,idx,tokens", [(64, 1, [0, 17, 40, 63]), (8192, 2, [0, 4097, 8191])])
def test_layer_dsv3_full_size(cuda, T, idx, tokens):
    """DeepSeek-V3 layer (256 experts + 1 shared): decode 64 and prefill 8192 tokens.
    Outputs are per token, so the oracle checks a token subset (only their experts are
    dequantized on the host); routing is checked bit-exact for every token."""
    cfg = PRESETS["dsv3"]
    say("layer dsv3 full", T)
    w = _big_weights(cfg, idx, cuda)
    x = synthetic.hidden_states(T, cfg.hidden, idx).to(cuda)
    _check_layer(cfg, w, x, tokens=tokens, tag=f"dsv3 T={T}")
    del w
    torch.cuda.empty_cache()


@pytest.fixture(scope="module")
def kimi_weights(cuda):
    w = _big_weights(PRESETS["kimi_k2"], 3, cuda)
    yield w
    del w
    torch.cuda.empty_cache()


@pytest.mark.parametrize("T,tokens", [(1, [0]), (256, [0, 131, 255]), (16384, [0, 9001, 16383])])
def test_layer_kimi_k2_full_size(cuda, kimi_weights, T, tokens):
    """Kimi-K2 layer (384 experts + 1 shared, sigmoid top-8 over one group, x2.827) at the
    ends and middle of its token sweep: 1 token (row tiles), 256, and 16384 (block
    kernels, ~341 rows per expert)."""
    cfg = PRESETS["kimi_k2"]
    say("layer kimi-k2 full", T)
    x = synthetic.hidden_states(T, cfg.hidden, 3).to(cuda)
    _check_layer(cfg, kimi_weights, x, tokens=tokens, tag=f"kimi T={T}")


def test_layer_glm45_full_size_zipf(cuda):
    """GLM-4.5 layer (hidden 5120, intermediate 1536, 160 experts + 1 shared) at 4096
    tokens with Zipf(1.2) expert popularity and 10% of the experts empty: overfull
    experts span many 256-row tiles, empty ones none."""
    cfg = PRESETS["glm45"]
    say("layer glm-4.5 full zipf")
    w = synthetic.make_weights(cfg, 4, device=cuda, zipf=True, experts_device=cuda)
    x = synthetic.hidden_states(4096, cfg.hidden, 4).to(cuda)
    out = _check_layer(cfg, w, x, tokens=[0, 1234, 4095], tag="glm45 T=4096")
    ids = ops.layer_forward(x, w, cfg, return_routing=True)[1].cpu().numpy()
    counts = np.bincount(ids.reshape(-1), minlength=cfg.n_experts)
    assert (counts == 0).sum() >= 16 and counts.max() > 3 * counts[counts > 0].mean()
    del w, out
    torch.cuda.empty_cache()


@pytest.mark.parametrize("T,E,K,S", [(2048, 8, 2, 0), (3000, 16, 4, 1), (700, 4, 2, 1)])
def test_layer_block_kernels(cuda, T, E, K, S):
    """Block-kernel path (> 20 rows per expert): block kernels against the oracle,
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
    rows = sorted(tiles[:4 * int(num.item())].cpu().numpy().reshape(-1, 4)[:, 2].tolist())
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
