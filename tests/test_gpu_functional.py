"""GPU parity of the operator mirrors (vllm_neuron_amd.functional.moe) against the oracle.

Gates: routing, mappings and selections bit-exact when the oracle is fed the GPU's
logits; fp32 logits and RMSNorm within fp32 rounding of a float64 evaluation; layer
outputs rel-L2 <= 1e-2 against the fp32-accumulate dequant oracle on the same fp8
operands."""
import numpy as np
import pytest
import torch

from _util import np_f32, np_u8, oracle_weights, rel_l2, say
from oracle import blockwise as BW
from oracle import router as R
from oracle.fp8 import quant_weight_128x128
from oracle.moe import bf16_round, moe_block_tkg_fp8, moe_sparse_fp8
from vllm_neuron_amd import PRESETS, ops, synthetic
from vllm_neuron_amd.functional import moe as M
from vllm_neuron_amd.functional.moe import _experts

pytestmark = pytest.mark.gpu
TOL_REL_L2 = 1e-2


def _small(cuda, seed=0):
    cfg = PRESETS["small"]
    return cfg, synthetic.make_weights(cfg, seed, device=cuda)


def _nf(w):
    """Stacked device layout -> the reference operator layout (and block scales)."""
    E, I2, H = w.w13.shape
    I = I2 // 2
    gu = w.w13.view(torch.uint8).reshape(E, 2, I, H).permute(0, 3, 1, 2).contiguous()
    gs = w.w13_scale.reshape(E, 2, I // 128, H // 128).permute(0, 3, 1, 2).contiguous()
    dn = w.w2.view(torch.uint8).transpose(1, 2).contiguous()
    ds = w.w2_scale.transpose(1, 2).contiguous()
    return gu.view(torch.float8_e4m3fn), gs, dn.view(torch.float8_e4m3fn), ds


def _ids_weights_from_dense(aff):
    """Selected experts of each row (ascending) and their affinities."""
    a = np_f32(aff)
    K = int((a != 0).sum(1).max())
    ids = np.zeros((a.shape[0], K), np.int32)
    wts = np.zeros((a.shape[0], K), np.float32)
    for t in range(a.shape[0]):
        nz = np.nonzero(a[t])[0]
        ids[t, :len(nz)] = nz
        wts[t, :len(nz)] = a[t, nz]
    return ids, wts


# ---------------------------------------------------------------- kernels

@pytest.mark.parametrize("x_dtype, out_dtype, ha, H", [
    (torch.bfloat16, torch.bfloat16, None, 1024), (torch.bfloat16, torch.bfloat16, 1000, 1024),
    (torch.float32, torch.float32, None, 1024), (torch.float32, torch.bfloat16, 777, 1024),
    (torch.bfloat16, torch.float32, None, 7168), (torch.bfloat16, torch.bfloat16, 1000, 1004)])
def test_rms_norm_kernel(cuda, x_dtype, out_dtype, ha, H):
    """H % 8 == 0 runs the vector kernel (row held in registers), H = 1004 the scalar one."""
    say("rms_norm", x_dtype, out_dtype, ha, H)
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(37, H, generator=g) * 3).to(x_dtype).to(cuda)
    gamma = (1 + 0.1 * torch.randn(H, generator=g)).to(cuda)
    y = ops.rms_norm(x, gamma, 1e-6, ha, out_dtype=out_dtype)
    ref = R.rms_norm_padded(np_f32(x), np_f32(gamma), 1e-6, ha)
    got = np_f32(y)
    if out_dtype == torch.float32:
        assert np.allclose(got, ref, rtol=2e-6, atol=1e-30)
    else:  # within one bf16 rounding of the fp32 result
        assert np.allclose(got, bf16_round(ref), rtol=2 ** -7, atol=0)
    if ha is not None:
        assert np.all(got[:, ha:] == 0)


@pytest.mark.parametrize("T, H, ha, with_res", [(1, 7168, None, False), (64, 7168, None, True),
                                                (37, 1024, 1000, True), (300, 1024, None, False)])
def test_rms_norm_quant_fused(cuda, T, H, ha, with_res):
    """The fused prologue equals residual add -> rms_norm -> act_quant bit for bit; the
    sum is the bf16 rounding of the fp32 sum, the codes the oracle's 1x128 quantization
    of the normalized rows, and those rows within one bf16 rounding of the fp32 norm."""
    from oracle.fp8 import quant_act_1x128
    say("rms_norm_quant", T, H, ha, with_res)
    g = torch.Generator().manual_seed(T + H)
    x = (torch.randn(T, H, generator=g) * 3).to(torch.bfloat16).to(cuda)
    r = torch.randn(T, H, generator=g).to(torch.bfloat16).to(cuda) if with_res else None
    gamma = (1 + 0.1 * torch.randn(H, generator=g)).to(cuda)
    xn, q, s, v = ops.rms_norm_quant(x, gamma, 1e-6, ha, r)
    v_ref = x + r if with_res else x
    if with_res:
        assert torch.equal(v, v_ref)
        assert np.array_equal(np_f32(v), bf16_round(np_f32(x) + np_f32(r)))
    else:
        assert v is None
    xn_ref = ops.rms_norm(v_ref, gamma, 1e-6, ha)
    q_ref, s_ref = ops.act_quant(xn_ref)
    assert torch.equal(xn, xn_ref)
    assert torch.equal(q.view(torch.uint8), q_ref.view(torch.uint8)) and torch.equal(s, s_ref)
    ref = R.rms_norm_padded(np_f32(v_ref), np_f32(gamma), 1e-6, ha)
    assert np.allclose(np_f32(xn), bf16_round(ref), rtol=2 ** -7, atol=0)
    oq, os_ = quant_act_1x128(np_f32(xn))
    assert np.array_equal(np_u8(q), oq) and np.array_equal(np_f32(s), os_)


def test_rms_norm_quant_rejects_bad_arguments(cuda):
    x = torch.zeros(4, 1000, dtype=torch.bfloat16, device=cuda)
    with pytest.raises(ValueError):                         # H not a multiple of 128
        ops.rms_norm_quant(x, torch.ones(1000, device=cuda), 1e-6)
    x = torch.zeros(4, 1024, dtype=torch.bfloat16, device=cuda)
    with pytest.raises(ValueError):                         # hidden_actual beyond H
        ops.rms_norm_quant(x, torch.ones(1024, device=cuda), 1e-6, hidden_actual=2000)


@pytest.mark.parametrize("T, H, E, w_dtype", [(100, 512, 40, torch.float32),
                                             (3000, 512, 40, torch.bfloat16),
                                             (7, 128, 96, torch.float32), (1, 1024, 8, torch.bfloat16)])
def test_router_logits_f32(cuda, T, H, E, w_dtype):
    say("router_logits_f32", T, H, E, w_dtype)
    g = torch.Generator().manual_seed(T + H)
    x = torch.randn(T, H, generator=g).to(cuda)
    w = (0.05 * torch.randn(E, H, generator=g)).to(w_dtype).to(cuda)
    b = torch.randn(E, generator=g).to(cuda)
    got = np_f32(ops.router_logits_f32(x, w, b))
    ref = np_f32(x).astype(np.float64) @ np_f32(w).astype(np.float64).T + np_f32(b)
    scale = np.abs(np_f32(x)).astype(np.float64) @ np.abs(np_f32(w)).astype(np.float64).T
    assert np.all(np.abs(got - ref) <= 1e-6 * scale + 1e-6), np.max(np.abs(got - ref) / (scale + 1))


# ---------------------------------------------------------------- router()

ORDERS = [M.RouterComputationOrder.PRENORM_LINEAR_TOPK_ACT_SCATTER,
          M.RouterComputationOrder.PRENORM_LINEAR_ACT_TOPK_RENORM_SCATTER,
          M.RouterComputationOrder.PRENORM_LINEAR_TOPK_SCATTER_ACT]


@pytest.mark.parametrize("order", ORDERS, ids=lambda o: o.name)
@pytest.mark.parametrize("activation", ["softmax", "sigmoid"])
@pytest.mark.parametrize("with_gamma", [False, True])
def test_router_api(cuda, order, activation, with_gamma):
    say("router", order.name, activation, with_gamma)
    g = torch.Generator().manual_seed(3)
    T, H, E, K = 77, 512, 24, 4
    x = torch.randn(T, H, generator=g).to(torch.bfloat16).to(cuda)
    w_param = (0.05 * torch.randn(E, H, generator=g)).to(torch.bfloat16).to(cuda)
    bias = (0.1 * torch.randn(E, generator=g)).to(cuda)
    gamma = (1 + 0.1 * torch.randn(H, generator=g)).to(cuda) if with_gamma else None
    aff, lg = M.router(x, w_param.t(), K, router_bias=bias, activation=activation,
                       return_logits=True, gamma=gamma, router_computation_order=order)
    assert aff.shape == (T, E) and lg.shape == (T, E) and aff.dtype == torch.float32
    xs = np_f32(x)
    if with_gamma:
        xs = R.rms_norm(xs, np_f32(gamma), 1e-6)   # fp32 normalization, fp32 operands
    ref_lg = R.router_logits(xs, np_f32(w_param), np_f32(bias))
    lg = np_f32(lg)
    assert np.allclose(lg, ref_lg, rtol=1e-5, atol=1e-5)
    sc = R.SOFTMAX if activation == "softmax" else R.SIGMOID
    a = np_f32(aff)
    if order == ORDERS[0]:
        ids, wts = R.route_topk_act(lg, K, sc)
        assert np.array_equal(a, R.scatter_dense(ids, wts, E))
    elif order == ORDERS[1]:
        ids, wts = R.route_act_topk_renorm(lg, K, sc, True, 0.0)
        assert np.array_equal(a, R.scatter_dense(ids, wts, E))
    else:
        ref = R.route_topk_scatter_act(lg, K, sc)
        assert np.array_equal(a != 0, ref != 0)
        assert np.allclose(a, ref, rtol=1e-6, atol=0)


def test_router_bf16_computation(cuda):
    say("router bf16 computation dtype")
    g = torch.Generator().manual_seed(4)
    T, H, E, K = 50, 256, 16, 2
    x = torch.randn(T, H, generator=g).to(torch.bfloat16).to(cuda)
    w_param = (0.05 * torch.randn(E, H, generator=g)).to(torch.bfloat16).to(cuda)
    aff, lg = M.router(x, w_param.t(), K, return_logits=True, computation_dtype=torch.bfloat16)
    assert aff.dtype == torch.bfloat16 and lg.dtype == torch.bfloat16
    lgf = np_f32(lg)   # logits rounded to bf16 before selection
    ids, wts = R.route_topk_act(lgf, K, R.SOFTMAX)
    assert np.array_equal(np_f32(aff), bf16_round(R.scatter_dense(ids, wts, E)))


@pytest.mark.parametrize("with_gamma", [False, True])
def test_router_fp16_computation(cuda, with_gamma):
    """computation_dtype float16: hidden states, the RMSNorm output and the bf16 router
    weights are rounded to fp16 before the fp32-accumulated product (router.py:236,
    :419-424, :681-688); logits and affinities come back in fp16, and the selection
    made from the returned logits is the oracle's."""
    say("router fp16 computation dtype", with_gamma)
    g = torch.Generator().manual_seed(6)
    T, H, E, K = 64, 512, 32, 4
    x = torch.randn(T, H, generator=g).to(torch.bfloat16).to(cuda)
    w_param = (0.05 * torch.randn(E, H, generator=g)).to(torch.bfloat16).to(cuda)
    bias = (0.1 * torch.randn(E, generator=g)).to(cuda)
    gamma = (1 + 0.1 * torch.randn(H, generator=g)).to(cuda) if with_gamma else None
    aff, lg = M.router(x, w_param.t(), K, router_bias=bias, return_logits=True, gamma=gamma,
                       computation_dtype=torch.float16)
    assert aff.dtype == torch.float16 and lg.dtype == torch.float16
    xs = np_f32(x.half())
    if with_gamma:
        xs = np_f32(torch.from_numpy(R.rms_norm(xs, np_f32(gamma), 1e-6)).half())
    w16 = np_f32(w_param.half())
    ref_lg = np_f32(torch.from_numpy(R.router_logits(xs, w16, np_f32(bias.half()))).half())
    lgf = np_f32(lg)
    # fp16 output rounding dominates the fp32 summation-order differences
    assert np.allclose(lgf, ref_lg, rtol=2 ** -10, atol=2 ** -14)
    ids, wts = R.route_topk_act(lgf, K, R.SOFTMAX)
    ref_aff = np_f32(torch.from_numpy(R.scatter_dense(ids, wts, E)).half())
    assert np.array_equal(np_f32(aff), ref_aff)


# ---------------------------------------------------------------- mapping / experts

def test_build_blockwise_mapping_api(cuda):
    say("build_blockwise_mapping api")
    cfg, w = _small(cuda)
    x = synthetic.hidden_states(64, cfg.hidden, 0).to(cuda)
    aff = M.router(x, w.router_w.t(), cfg.top_k)
    pm = torch.ones(64, dtype=torch.bool)
    pm[60:] = False
    for mask in (None, pm.to(cuda)):
        am, tpid, b2e, cond = M.build_blockwise_mapping(aff, cfg.n_experts, cfg.top_k, 256,
                                                        padding_mask=mask)
        ref = BW.build_blockwise_mapping(np_f32(aff), cfg.n_experts, cfg.top_k, 256,
                                         None if mask is None else mask.cpu().numpy())
        for got, exp in zip((am, tpid, b2e, cond), ref):
            assert np.array_equal(got.cpu().numpy().reshape(-1), np.asarray(exp).reshape(-1))


@pytest.mark.parametrize("T", [64, 2048])
def test_moe_cte_api(cuda, T):
    say("moe_cte api T", T)
    cfg, w = _small(cuda, 1)
    E, K = cfg.n_experts, cfg.top_k
    x = synthetic.hidden_states(T, cfg.hidden, 1).to(cuda)
    aff = M.router(x, w.router_w.t(), K)
    am, tpid, b2e, cond = M.build_blockwise_mapping(aff, E, K, 256)
    gu, gs, dn, ds = _nf(w)
    impl = M.MoECTEImplementation.shard_on_block
    out = M.moe_cte(x, am, gu, dn, tpid, b2e, 256, impl, gate_up_proj_scale=gs,
                    down_proj_scale=ds)
    out_stacked = M.moe_cte(x, am, w.w13, w.w2, tpid, b2e, 256, impl,
                            gate_up_proj_scale=w.w13_scale, down_proj_scale=w.w2_scale)
    assert torch.equal(out, out_stacked)
    # [T+1, H] hidden states: the last row is a padding sink and is not returned
    xp = torch.cat([x, torch.zeros_like(x[:1])])
    assert torch.equal(M.moe_cte(xp, am, gu, dn, tpid, b2e, 256, impl, gate_up_proj_scale=gs,
                                 down_proj_scale=ds), out)
    ids, wts = _ids_weights_from_dense(aff)
    q13, s13, q2, s2 = oracle_weights(w)
    ref = moe_sparse_fp8(np_f32(x), ids, wts, q13, s13, q2, s2)
    err = rel_l2(np_f32(out), ref)
    say("moe_cte rel_l2", err)
    assert err <= TOL_REL_L2
    no = M.moe_cte(x, am, gu, dn, tpid, b2e, 256, impl, gate_up_proj_scale=gs,
                   down_proj_scale=ds,
                   expert_affinities_scaling_mode=M.ExpertAffinityScaleMode.NO_SCALE)
    ref_no = moe_sparse_fp8(np_f32(x), ids, np.ones_like(wts), q13, s13, q2, s2)
    assert rel_l2(np_f32(no), ref_no) <= TOL_REL_L2


def test_moe_tkg_api(cuda):
    say("moe_tkg api")
    cfg, w = _small(cuda, 2)
    E, K = cfg.n_experts, cfg.top_k
    x = synthetic.hidden_states(32, cfg.hidden, 2).to(cuda)
    aff = M.router(x, w.router_w.t(), K)
    ids, _ = ops.router_topk(ops.router_logits(x, w.router_w), K, ops.ORDER_TOPK_ACT, "softmax")
    gu, gs, dn, ds = _nf(w)
    kw = dict(expert_gate_up_weights_scale=gs, expert_down_weights_scale=ds)
    post = M.moe_tkg(x, gu, dn, aff, ids, False,
                     expert_affinities_scaling_mode=M.ExpertAffinityScaleMode.POST_SCALE, **kw)
    no = M.moe_tkg(x, gu, dn, aff, ids, False, **kw)
    q13, s13, q2, s2 = oracle_weights(w)
    idn = ids.cpu().numpy()
    wts = np.take_along_axis(np_f32(aff), idn.astype(np.int64), 1)
    assert rel_l2(np_f32(post), moe_sparse_fp8(np_f32(x), idn, wts, q13, s13, q2, s2)) <= TOL_REL_L2
    assert rel_l2(np_f32(no), moe_sparse_fp8(np_f32(x), idn, np.ones_like(wts), q13, s13, q2,
                                             s2)) <= TOL_REL_L2
    # all-expert schedule with unselected experts masked: K = E rows per token (another
    # tile height), the same layer
    allx = M.moe_tkg(x, gu, dn, aff, ids, True, mask_unselected_experts=True,
                     expert_affinities_scaling_mode=M.ExpertAffinityScaleMode.POST_SCALE, **kw)
    assert rel_l2(np_f32(allx), moe_sparse_fp8(np_f32(x), idn, wts, q13, s13, q2, s2)) <= TOL_REL_L2
    assert rel_l2(np_f32(allx), np_f32(post)) <= 1e-3


@pytest.mark.parametrize("act, pre_norm, norm_topk, post, ha", [
    (M.RouterActFnType.SIGMOID, True, True, True, None),
    (M.RouterActFnType.SOFTMAX, False, False, False, 1000),
    (M.RouterActFnType.SOFTMAX, True, False, True, None)])
def test_moe_block_tkg_api(cuda, act, pre_norm, norm_topk, post, ha):
    say("moe_block_tkg", act.name, pre_norm, norm_topk, post, ha)
    cfg, w = _small(cuda, 3)
    E, K, H, I = cfg.n_experts, cfg.top_k, cfg.hidden, cfg.intermediate
    g = torch.Generator().manual_seed(9)
    x = synthetic.hidden_states(24, H, 3).to(cuda).reshape(2, 12, H)   # [B, S, H]
    gamma = (1 + 0.1 * torch.randn(1, H, generator=g)).to(cuda)
    bias = (0.1 * torch.randn(1, E, generator=g)).to(cuda)
    sh = [(0.02 * torch.randn(*s, generator=g)).to(torch.bfloat16).to(cuda)
          for s in ((H, I), (H, I), (I, H))]
    gu, gs, dn, ds = _nf(w)
    mode = M.ExpertAffinityScaleMode.POST_SCALE if post else M.ExpertAffinityScaleMode.NO_SCALE
    out, lg = M.moe_block_tkg(x, gamma, w.router_w.t(), gu, dn, top_k=K, shared_expert_gate_w=sh[0],
                              shared_expert_up_w=sh[1], shared_expert_down_w=sh[2],
                              expert_gate_up_weights_scale=gs, expert_down_weights_scale=ds,
                              router_bias=bias, router_act_fn=act, router_pre_norm=pre_norm,
                              norm_topk_prob=norm_topk, expert_affinities_scaling_mode=mode,
                              hidden_actual=ha)
    assert out.shape == (24, H) and out.dtype == torch.bfloat16
    # shared expert quantization (weight preparation) equals the oracle's 128x128 quantizer
    sq = _experts.shared_weights(sh[0], sh[1], sh[2], I)
    q13_ref, s13_ref = quant_weight_128x128(np.concatenate([np_f32(sh[0]).T, np_f32(sh[1]).T]))
    assert np.array_equal(np_u8(sq[0][0]), q13_ref) and np.array_equal(np_f32(sq[1][0]), s13_ref)
    shared = (np_u8(sq[0][0]), np_f32(sq[1][0]), np_u8(sq[2][0]), np_f32(sq[3][0]))
    xs = np_f32(x.reshape(24, H))
    sc = R.SOFTMAX if act == M.RouterActFnType.SOFTMAX else R.SIGMOID
    lg = np_f32(lg)
    ref_out, ref_lg, _, _ = moe_block_tkg_fp8(xs, np_f32(gamma), 1e-6, np_f32(w.router_w),
                                              np_f32(bias).reshape(-1), K, sc, pre_norm,
                                              norm_topk, post, *oracle_weights(w), shared=shared,
                                              hidden_actual=ha)
    assert np.allclose(lg, ref_lg, rtol=1e-4, atol=1e-4)
    ref_sel, _, _, _ = moe_block_tkg_fp8(xs, np_f32(gamma), 1e-6, np_f32(w.router_w), None, K, sc,
                                         pre_norm, norm_topk, post, *oracle_weights(w),
                                         shared=shared, hidden_actual=ha, logits=lg)
    err = rel_l2(np_f32(out), ref_sel)
    say("moe_block_tkg rel_l2", err)
    assert err <= TOL_REL_L2


def test_moe_block_tkg_fused_residual(cuda):
    """residual: the block normalizes inp + residual and returns that sum last; the
    output and logits equal those of the block run on the sum (same kernels)."""
    say("moe_block_tkg residual")
    cfg, w = _small(cuda, 4)
    K, H = cfg.top_k, cfg.hidden
    g = torch.Generator().manual_seed(11)
    x = synthetic.hidden_states(24, H, 4).to(cuda).reshape(2, 12, H)
    res = torch.randn(2, 12, H, generator=g).to(torch.bfloat16).to(cuda)
    gamma = (1 + 0.1 * torch.randn(1, H, generator=g)).to(cuda)
    gu, gs, dn, ds = _nf(w)
    kw = dict(top_k=K, expert_gate_up_weights_scale=gs, expert_down_weights_scale=ds,
              router_act_fn=M.RouterActFnType.SIGMOID, norm_topk_prob=True,
              expert_affinities_scaling_mode=M.ExpertAffinityScaleMode.POST_SCALE)
    out, lg, ro = M.moe_block_tkg(x, gamma, w.router_w.t(), gu, dn, residual=res, **kw)
    s = x + res
    out2, lg2 = M.moe_block_tkg(s, gamma, w.router_w.t(), gu, dn, **kw)
    assert torch.equal(ro, s) and ro.shape == x.shape
    assert torch.equal(out, out2) and torch.equal(lg, lg2)
    only = M.moe_block_tkg(x, gamma, w.router_w.t(), gu, dn, residual=res, skip_router_logits=True,
                           **kw)
    assert len(only) == 2 and torch.equal(only[0], out) and torch.equal(only[1], s)


def test_moe_block_tkg_fresh_weight_views_convert_once(cuda):
    """The reference's decode hands moe_block_tkg a fresh `.reshape` view of the
    gate_up parameter on every step (model_bf16.py:1278). Three calls with fresh views
    of one stored parameter re-layout the experts once and give equal outputs."""
    say("moe_block_tkg fresh views")
    cfg, w = _small(cuda, 5)
    E, K, H, I = cfg.n_experts, cfg.top_k, cfg.hidden, cfg.intermediate
    gu, gs, dn, ds = _nf(w)
    gate_up_param = gu.reshape(E, H, 2 * I).clone()      # stored flat, as the model's parameter
    x = synthetic.hidden_states(8, H, 5).to(cuda).reshape(1, 8, H)
    gamma = torch.ones(1, H, device=cuda)
    kw = dict(top_k=K, expert_gate_up_weights_scale=gs, expert_down_weights_scale=ds,
              router_act_fn=M.RouterActFnType.SOFTMAX, router_pre_norm=False,
              expert_affinities_scaling_mode=M.ExpertAffinityScaleMode.POST_SCALE)
    before = _experts.BUILDS[0]
    outs = [M.moe_block_tkg(x, gamma, w.router_w.t(), gate_up_param.reshape(E, H, 2, I), dn, **kw)[0]
            for _ in range(3)]
    torch.cuda.synchronize()
    assert _experts.BUILDS[0] == before + 1
    assert torch.equal(outs[1], outs[0]) and torch.equal(outs[2], outs[0])
    ref = M.moe_block_tkg(x, gamma, w.router_w.t(), gu, dn, **kw)[0]
    assert torch.equal(ref, outs[0])


# ---------------------------------------------------------------- per-channel fp8 scales

FP8 = torch.float8_e4m3fn


def _chan_experts(E, H, I, seed, device):
    """fp8 expert codes with per-output-channel scales (the reference's FP8 row
    formats): the stacked codes q13 [E, 2I, H] / q2 [E, H, I], the channel scales
    c13 [E, 2I] (gate, then up) / c2 [E, H] (dequantized weights ~ N(0, 0.02)), and the
    same codes in the reference operator layout gate_up [E, H, 2, I] / down [E, I, H]."""
    g = torch.Generator().manual_seed(seed)
    q13 = (torch.randn(E, 2 * I, H, generator=g) * 64).clamp(-448, 448).to(FP8)
    q2 = (torch.randn(E, H, I, generator=g) * 64).clamp(-448, 448).to(FP8)
    c13 = (torch.rand(E, 2 * I, generator=g) + 0.5) * (0.02 / 64)
    c2 = (torch.rand(E, H, generator=g) + 0.5) * (0.02 / 64)
    gu = q13.view(torch.uint8).reshape(E, 2, I, H).permute(0, 3, 1, 2).contiguous().view(FP8)
    dn = q2.view(torch.uint8).transpose(1, 2).contiguous().view(FP8)
    return q13, q2, c13, c2, gu.to(device), dn.to(device)


def _chan_oracle(x, ids, wts, q13, q2, c13, c2):
    E, I2, H = q13.shape
    ones13 = np.ones((E, I2 // 128, H // 128), np.float32)
    ones2 = np.ones((E, H // 128, I2 // 2 // 128), np.float32)
    return moe_sparse_fp8(np_f32(x), ids, wts, q13.view(torch.uint8).numpy(), ones13,
                          q2.view(torch.uint8).numpy(), ones2, chan=(c13.numpy(), c2.numpy()))


@pytest.mark.parametrize("T", [64, 2048])
def test_moe_cte_per_channel_scales(cuda, T):
    """moe_cte with the reference's FP8 per-channel scales gate_up_proj_scale [E, 1, 2I]
    and down_proj_scale [E, 1, H] (moe_cte.py:178-188), against the oracle's per-channel
    dequantization: row tiles at 64 tokens, block kernels at 2048 (512 rows per
    expert)."""
    say("moe_cte per-channel T", T)
    E, K, H, I = 8, 2, 1024, 512
    q13, q2, c13, c2, gu, dn = _chan_experts(E, H, I, 50 + T, cuda)
    x = synthetic.hidden_states(T, H, 5).to(cuda)
    g = torch.Generator().manual_seed(51)
    rw = (torch.randn(H, E, generator=g) * 0.02).to(torch.bfloat16).to(cuda)
    aff = M.router(x, rw, K)
    am, tpid, b2e, cond = M.build_blockwise_mapping(aff, E, K, 256)
    out = M.moe_cte(x, am, gu, dn, tpid, b2e, 256, M.MoECTEImplementation.shard_on_block,
                    gate_up_proj_scale=c13.reshape(E, 1, 2 * I).to(cuda),
                    down_proj_scale=c2.reshape(E, 1, H).to(cuda))
    ids, wts = _ids_weights_from_dense(aff)
    ref = _chan_oracle(x, ids, wts, q13, q2, c13, c2)
    err = rel_l2(np_f32(out), ref)
    say("moe_cte per-channel rel_l2", err)
    assert err <= TOL_REL_L2, err


def test_moe_tkg_row_and_static_scales(cuda):
    """moe_tkg with FP8 row quantization scales [E, 2, I] / [E, H] and static scales
    [E, 2, 1] / [E, 1] (moe_tkg.py:87-91) against the oracle."""
    say("moe_tkg row / static scales")
    E, K, H, I = 8, 2, 1024, 512
    q13, q2, c13, c2, gu, dn = _chan_experts(E, H, I, 60, cuda)
    x = synthetic.hidden_states(32, H, 6).to(cuda)
    g = torch.Generator().manual_seed(61)
    rw = (torch.randn(E, H, generator=g) * 0.02).to(torch.bfloat16).to(cuda)
    ids, _ = ops.router_topk(ops.router_logits(x, rw), K, ops.ORDER_TOPK_ACT, "softmax")
    aff = torch.softmax(ops.router_logits(x, rw), dim=1)
    idn = ids.cpu().numpy()
    wts = np.take_along_axis(np_f32(aff), idn.astype(np.int64), 1)
    post = M.ExpertAffinityScaleMode.POST_SCALE
    row = M.moe_tkg(x, gu, dn, aff, ids, False, expert_gate_up_weights_scale=c13.reshape(E, 2, I).to(cuda),
                    expert_down_weights_scale=c2.to(cuda), expert_affinities_scaling_mode=post)
    err = rel_l2(np_f32(row), _chan_oracle(x, idn, wts, q13, q2, c13, c2))
    say("moe_tkg row rel_l2", err)
    assert err <= TOL_REL_L2, err
    st13 = (torch.rand(E, 2, 1, generator=g) + 0.5) * (0.02 / 64)
    st2 = (torch.rand(E, 1, generator=g) + 0.5) * (0.02 / 64)
    static = M.moe_tkg(x, gu, dn, aff, ids, False, expert_gate_up_weights_scale=st13.to(cuda),
                       expert_down_weights_scale=st2.to(cuda), expert_affinities_scaling_mode=post)
    ref = _chan_oracle(x, idn, wts, q13, q2, st13.expand(E, 2, I).reshape(E, 2 * I),
                       st2.expand(E, H))
    err = rel_l2(np_f32(static), ref)
    say("moe_tkg static rel_l2", err)
    assert err <= TOL_REL_L2, err


def test_moe_block_tkg_row_scales_with_shared_expert(cuda):
    """moe_block_tkg with per-channel routed scales and a bf16 shared expert (quantized
    to 128x128 blocks): the routed experts take the channel scales, the shared expert
    none, in the same launch."""
    say("moe_block_tkg row scales + shared")
    E, K, H, I = 8, 2, 1024, 512
    q13, q2, c13, c2, gu, dn = _chan_experts(E, H, I, 70, cuda)
    g = torch.Generator().manual_seed(71)
    x = synthetic.hidden_states(16, H, 7).to(cuda).reshape(1, 16, H)
    gamma = (1 + 0.1 * torch.randn(1, H, generator=g)).to(cuda)
    rw = (torch.randn(E, H, generator=g) * 0.02).to(torch.bfloat16).to(cuda)
    sh = [(0.02 * torch.randn(*s, generator=g)).to(torch.bfloat16).to(cuda)
          for s in ((H, I), (H, I), (I, H))]
    out, lg = M.moe_block_tkg(x, gamma, rw.t(), gu, dn, top_k=K, shared_expert_gate_w=sh[0],
                              shared_expert_up_w=sh[1], shared_expert_down_w=sh[2],
                              expert_gate_up_weights_scale=c13.reshape(E, 2, I).to(cuda),
                              expert_down_weights_scale=c2.to(cuda),
                              router_act_fn=M.RouterActFnType.SOFTMAX,
                              expert_affinities_scaling_mode=M.ExpertAffinityScaleMode.POST_SCALE)
    sq = _experts.shared_weights(sh[0], sh[1], sh[2], I)
    shared = (np_u8(sq[0][0]), np_f32(sq[1][0]), np_u8(sq[2][0]), np_f32(sq[3][0]))
    E_, I2 = E, 2 * I
    ones13 = np.ones((E_, I2 // 128, H // 128), np.float32)
    ones2 = np.ones((E_, H // 128, I // 128), np.float32)
    xs = np_f32(x.reshape(16, H))
    ref, _, _, _ = moe_block_tkg_fp8(xs, np_f32(gamma), 1e-6, np_f32(rw), None, K, R.SOFTMAX, True,
                                     False, True, q13.view(torch.uint8).numpy(), ones13,
                                     q2.view(torch.uint8).numpy(), ones2, shared=shared,
                                     logits=np_f32(lg), chan=(c13.numpy(), c2.numpy()))
    err = rel_l2(np_f32(out), ref)
    say("moe_block_tkg row scales rel_l2", err)
    assert err <= TOL_REL_L2, err
