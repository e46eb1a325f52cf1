"""GPU parity of the MX (microscaling) expert path: MXFP4 / MXFP8 weights, MXFP8
activations and E8M0 scales applied by gfx950's scaled MFMA, with GPT-OSS's Swish,
clamps and biases (moe_cte.py:440-612), against the oracle (oracle/mx.py).

Gates: MXFP8 activation codes and scale bytes bit-exact; one scaled MFMA within fp32
summation rounding of the float64 product; expert and layer outputs rel-L2 <= 1e-2
against the oracle on the same MX operands."""
import numpy as np
import pytest
import torch

from _util import np_f32, rel_l2, say
from oracle import mx as OX
from oracle.fp8 import e4m3fn_decode
from vllm_neuron_amd import ops
from vllm_neuron_amd.weights_mx import MxMoEWeights, quant_mx_weight

pytestmark = pytest.mark.gpu
TOL_REL_L2 = 1e-2
LIMIT = 7.0  # GPT-OSS swiglu_limit (model/gpt_oss/config.py:62)


def _np_u8(t):
    return t.view(torch.uint8).cpu().numpy() if t.dtype == torch.float8_e4m3fn else t.cpu().numpy()


def _rand_fp8_codes(g, shape):
    c = torch.randint(0, 256, shape, generator=g, dtype=torch.int32)
    c[(c & 0x7F) == 0x7F] = 0x3F  # no NaN codes
    return c.to(torch.uint8)


def _scaled_mfma_case(cuda, fmt, g, a, sa, sb, small):
    if fmt == "fp4":
        bc = torch.randint(0, 16, (16, 128), generator=g, dtype=torch.int32).to(torch.uint8)
        b = (bc[:, 0::2] | (bc[:, 1::2] << 4)).contiguous()
        bval = OX.fp4_decode(bc.numpy())
    elif small:
        bv = torch.randint(-8, 9, (16, 128), generator=g).float()
        b = bv.to(torch.float8_e4m3fn).view(torch.uint8)
        bval = bv.numpy()
    else:
        b = _rand_fp8_codes(g, (16, 128))
        bval = e4m3fn_decode(b.numpy())
    c = ops.selftest_mfma_mx(a.to(cuda), sa.to(cuda), b.to(cuda), sb.to(cuda), fmt).cpu().numpy()
    A = OX.dequant_mx(e4m3fn_decode(a.numpy()), sa.numpy())
    B = OX.dequant_mx(bval, sb.numpy())
    return c, A @ B.T, np.abs(A) @ np.abs(B).T


@pytest.mark.parametrize("fmt", ["fp4", "fp8"])
def test_scaled_mfma_layout(cuda, fmt):
    """One v_mfma_scale_f32_16x16x128_f8f6f4 with the GEMMs' lane mapping against the
    float64 product of the dequantized operands: pins the fp8 and fp4 operand layouts,
    the fp4 nibble order, the scale lanes and E8M0. Small integers and scales 2^-1..2^1
    keep every partial sum exact, so that case is bit for bit; over the full fp8 range
    the MFMA's internal accumulation is compared as in the unscaled fp8 test."""
    say("scaled mfma", fmt)
    g = torch.Generator().manual_seed(1 if fmt == "fp4" else 2)
    av = torch.randint(-8, 9, (16, 128), generator=g).float()
    a = av.to(torch.float8_e4m3fn).view(torch.uint8)
    sa = torch.randint(126, 129, (16, 4), generator=g, dtype=torch.int32).to(torch.uint8)
    sb = torch.randint(126, 129, (16, 4), generator=g, dtype=torch.int32).to(torch.uint8)
    c, ref, _ = _scaled_mfma_case(cuda, fmt, g, a, sa, sb, small=True)
    assert np.array_equal(c, ref)
    a = _rand_fp8_codes(g, (16, 128))
    sa = torch.randint(110, 145, (16, 4), generator=g, dtype=torch.int32).to(torch.uint8)
    sb = torch.randint(110, 145, (16, 4), generator=g, dtype=torch.int32).to(torch.uint8)
    c, ref, bound = _scaled_mfma_case(cuda, fmt, g, a, sa, sb, small=False)
    err = np.abs(c - ref) / (bound + 1e-30)
    say("scaled mfma wide-range max error / sum|products|", float(err.max()))
    assert err.max() < 1e-3


@pytest.mark.parametrize("R,C", [(1, 32), (37, 512), (300, 3072)])
def test_act_quant_mx_bit_exact(cuda, R, C):
    """MXFP8 codes and E8M0 bytes equal the oracle's OCP quantizer, including all-zero
    blocks and blocks spanning many binades."""
    say("act quant mx", R, C)
    g = torch.Generator().manual_seed(R + C)
    x = torch.randn(R, C, generator=g) * torch.exp2(torch.randint(-20, 20, (R, 1), generator=g).float())
    x[0, :32] = 0.0
    if C >= 64:
        x[-1, 32:64] = torch.exp2(torch.arange(32).float() - 16)  # 32 binades in one block
    xb = x.to(torch.bfloat16)
    q, s = ops.act_quant_mx(xb.to(cuda))
    oq, os_ = OX.quant_mxfp8(np_f32(xb))
    assert np.array_equal(_np_u8(q), oq)
    assert np.array_equal(s.cpu().numpy(), os_)


def make_mx_weights(E, H, I, seed, device, fmt="fp4", bias=True):
    g = torch.Generator(device="cpu").manual_seed(seed)
    w13 = (torch.randn(E, 2 * I, H, generator=g) * 0.02).to(device)
    w2 = (torch.randn(E, H, I, generator=g) * 0.02).to(device)
    q13, s13 = quant_mx_weight(w13, fmt)
    q2, s2 = quant_mx_weight(w2, fmt)
    b13 = b2 = None
    if bias:
        b13 = (torch.randn(E, 2 * I, generator=g) * 0.1).to(device)
        b13[:, I:] += 1.0  # the +1 the reference's loaders fold into the up bias
        b2 = (torch.randn(E, H, generator=g) * 0.1).to(device)
    rw = (torch.randn(E, H, generator=g) * 0.02).to(torch.bfloat16).to(device)
    rb = (torch.randn(E, generator=g) * 0.1).to(device)
    return MxMoEWeights(router_w=rw, w13=q13, w13_scale=s13, w2=q2, w2_scale=s2, b13=b13, b2=b2,
                        router_bias=rb, fmt=fmt).validate()


def oracle_mx_weights(w):
    """numpy operands of the oracle: packed fp4 (or fp8 codes), scales, biases."""
    cv = _np_u8
    return (cv(w.w13), cv(w.w13_scale), None if w.b13 is None else np_f32(w.b13), cv(w.w2),
            cv(w.w2_scale), None if w.b2 is None else np_f32(w.b2))


def oracle_layer(x, ids, wts, w, act, gl, ul, experts=None):
    x = x if isinstance(x, np.ndarray) else np_f32(x)
    q13, s13, b13, q2, s2, b2 = oracle_mx_weights(w)
    if w.fmt == "fp4":
        return OX.moe_sparse_mx(x, ids, wts, q13, s13, b13, q2, s2, b2, act, gl, ul, experts)
    # fp8 weights: dequantize the codes with the same helper path
    xhat = OX.dequant_mxfp8(*OX.quant_mxfp8(x))
    out = np.zeros(x.shape, np.float32)
    for e in (range(w.n_experts) if experts is None else sorted(experts)):
        sel = ids == e
        rows = np.nonzero(sel.any(axis=1))[0]
        if rows.size == 0:
            continue
        wt = (wts * sel).sum(axis=1)[rows].astype(np.float32)
        y = OX.expert_mlp_mx(xhat[rows], OX.dequant_mxfp8(q13[e], s13[e]), b13[e],
                             OX.dequant_mxfp8(q2[e], s2[e]), b2[e], act, gl, ul)
        out[rows] += y * wt[:, None]
    return out


@pytest.mark.parametrize("fmt,act,T,E,K", [("fp4", "swish", 64, 8, 2), ("fp4", "silu", 200, 16, 4),
                                           ("fp8", "swish", 64, 8, 2), ("fp4", "swish", 1, 8, 4)])
def test_mx_experts_match_oracle(cuda, fmt, act, T, E, K):
    """The op pipeline (mapping -> MXFP8 quant -> MX gate_up with bias, clamps and
    activation -> MX down with bias -> combine) against the oracle."""
    H, I = 512, 256
    say("mx experts", fmt, act, T, E, K)
    w = make_mx_weights(E, H, I, 5 + T, cuda, fmt)
    g = torch.Generator().manual_seed(T)
    x = (torch.randn(T, H, generator=g) * 2).to(torch.bfloat16).to(cuda)
    ids = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)]).to(torch.int32)
    wts = torch.rand(T, K, generator=g)
    gl, ul = ((None, LIMIT), (1 - LIMIT, 1 + LIMIT)) if act == "swish" else ((None, None), (None, None))
    out = ops.mx_experts(x, ids.to(cuda), wts.to(cuda), w, act, gl, ul)
    ref = oracle_layer(x, ids.numpy(), wts.numpy(), w, act, gl, ul)
    err = rel_l2(np_f32(out), ref)
    say("rel_l2", err)
    assert err <= TOL_REL_L2, err


@pytest.mark.parametrize("fmt,T,E,K,H,I", [
    ("fp4", 64, 64, 2, 1024, 2048),    # 16-row tiles, 3-stage ring, scale table, ~1000 items
    ("fp4", 128, 16, 2, 1024, 2048),   # 32-row tiles, 2-stage ring, scale table
    ("fp4", 2048, 8, 2, 1024, 2048),   # 64-row tiles, 2-stage ring, scale table
    ("fp4", 4096, 8, 2, 4608, 512),    # gate_up K > 4096: per-stage scale loads
    ("fp4", 2048, 8, 2, 4096, 256),    # down K = 256: fewer stages than the ring (drain)
    ("fp8", 64, 64, 2, 1024, 1024),    # MXFP8 weights: one K block per stage
    ("fp4", 1, 64, 2, 1024, 2048),     # one token: 2-wave half-width items, scale table
    ("fp8", 1, 64, 2, 1024, 1024),     # ... MXFP8 weights
    ("fp4", 1, 8, 2, 4608, 512)])      # ... gate_up without the scale table (K > 4096)
def test_mx_experts_persistent_grid(cuda, fmt, T, E, K, H, I):
    """Shapes with more work items than CUs, so each persistent workgroup runs several
    items and its load ring crosses from item to item (or drains between them when K
    has fewer stages than the ring), with and without the per-item scale table; and
    one-token shapes, whose items run on 2-wave workgroups of half the width (one
    item per CU)."""
    say("mx persistent", fmt, T, E, K, H, I)
    w = make_mx_weights(E, H, I, 11 + T, cuda, fmt)
    g = torch.Generator().manual_seed(3 * T + E)
    x = (torch.randn(T, H, generator=g) * 2).to(torch.bfloat16).to(cuda)
    ids = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)]).to(torch.int32)
    wts = torch.rand(T, K, generator=g)
    gl, ul = (None, LIMIT), (1 - LIMIT, 1 + LIMIT)
    out = ops.mx_experts(x, ids.to(cuda), wts.to(cuda), w, "swish", gl, ul)
    ref = oracle_layer(x, ids.numpy(), wts.numpy(), w, "swish", gl, ul)
    err = rel_l2(np_f32(out), ref)
    say("rel_l2", err)
    assert err <= TOL_REL_L2, err
    # run to run the same bits
    assert torch.equal(out, ops.mx_experts(x, ids.to(cuda), wts.to(cuda), w, "swish", gl, ul))
    del w
    torch.cuda.empty_cache()


# ---------------------------------------------------------------- GPT-OSS-120B layer

GPT_OSS = dict(E=128, H=3072, I=3072, h_real=2880, i_real=2880, K=4)   # hidden 2880 padded to 3072


@pytest.fixture(scope="module")
def gpt_oss_weights(cuda):
    from vllm_neuron_amd import synthetic
    c = GPT_OSS
    w = synthetic.make_mx_weights(c["E"], c["H"], c["I"], 7, device=cuda, h_real=c["h_real"],
                                  i_real=c["i_real"])
    yield w
    del w
    torch.cuda.empty_cache()


def _padded_hidden(T, seed, cuda):
    g = torch.Generator().manual_seed(seed)
    x = torch.zeros(T, GPT_OSS["H"])
    x[:, :GPT_OSS["h_real"]] = torch.randn(T, GPT_OSS["h_real"], generator=g)
    return x.to(torch.bfloat16).to(cuda)


@pytest.mark.parametrize("T,tokens", [(1, [0]), (64, [0, 9, 31, 63]), (2048, [0, 700, 2047])])
def test_gpt_oss_120b_layer(cuda, gpt_oss_weights, T, tokens):
    """GPT-OSS-120B expert shapes (128 MXFP4 experts, hidden and intermediate 2880
    padded to 3072, top-4 softmax with a router bias, Swish with gate <= 7 and
    -6 <= up <= 8, biases) through MXFP4MoE with the layer's RMSNorm and residual add:
    routing bit-exact from the GPU's logits, output rel-L2 <= 1e-2 on a token subset."""
    from oracle import router as R
    from oracle.moe import bf16_round
    from vllm_neuron_amd import MXFP4MoE
    c = GPT_OSS
    w = gpt_oss_weights
    say("gpt-oss-120b layer", T)
    x = _padded_hidden(T, 100 + T, cuda)
    r = _padded_hidden(T, 200 + T, cuda)
    g = torch.Generator().manual_seed(T)
    gamma = torch.zeros(c["H"])
    gamma[:c["h_real"]] = 1 + 0.1 * torch.randn(c["h_real"], generator=g)
    gamma = gamma.to(torch.bfloat16).float().to(cuda)
    layer = MXFP4MoE(w, c["K"], norm_weight=gamma, eps=1e-5, hidden_actual=c["h_real"])
    out, rsum = layer(x, None, False, None, residual=r)
    out2, rsum2, ids, wts, lg = ops.layer_forward_mx(
        x, w, c["K"], "swish", (None, LIMIT), (1 - LIMIT, 1 + LIMIT), return_routing=True,
        gamma=gamma, eps=1e-5, hidden_actual=c["h_real"], residual=r)
    assert torch.equal(out, out2) and torch.equal(rsum, rsum2)
    assert np.array_equal(np_f32(rsum), bf16_round(np_f32(x) + np_f32(r)))
    dec = layer(rsum, None, True, None)   # decode: the same norm, one tensor
    assert torch.equal(dec, out)
    xn = ops.rms_norm_quant(x, gamma, 1e-5, c["h_real"], r)[0]
    ref_xn = R.rms_norm_padded(np_f32(rsum), np_f32(gamma), 1e-5, c["h_real"])
    assert np.allclose(np_f32(xn), bf16_round(ref_xn), rtol=2 ** -7, atol=0)
    xs = np_f32(xn)
    lg, ids, wts = lg.cpu().numpy(), ids.cpu().numpy(), wts.cpu().numpy()
    ref_lg = R.router_logits(xs, np_f32(w.router_w), np_f32(w.router_bias))
    assert np.allclose(lg, ref_lg, rtol=1e-5, atol=2e-5)
    oi, ow = R.route_topk_act(lg, c["K"], R.SOFTMAX)
    assert np.array_equal(ids, oi) and np.array_equal(wts, ow)
    sel = np.asarray(tokens)
    ref = oracle_layer(xn[sel], ids[sel], wts[sel], w, "swish", (None, LIMIT),
                       (1 - LIMIT, 1 + LIMIT), experts=set(np.unique(ids[sel]).tolist()))
    got = np_f32(out)[sel]
    err = rel_l2(got, ref)
    say("gpt-oss rel_l2", err)
    assert err <= TOL_REL_L2, err
    assert np.all(got[:, c["h_real"]:] == 0)  # padded hidden columns stay zero


@pytest.mark.parametrize("seed,act,limited", [(1, "swish", True), (2, "swish", True), (3, "silu", False)])
def test_gpt_oss_one_token_layer_equals_op_path(cuda, gpt_oss_weights, seed, act, limited):
    """At one token the layer's MX GEMMs (K = 3072) keep each wave's weight fragments for
    the whole K in registers, loaded in one memory round trip, and down and the combine
    run as one launch; the op-by-op path runs the ring kernels and moe_combine through
    the public entry points. Same scaled MFMAs in the same K order, the same epilogues
    and the same pair sum, so the layer's output is the same bits, with and without the
    clamps."""
    c = GPT_OSS
    w = gpt_oss_weights
    say("gpt-oss one token vs op path", seed, act, limited)
    gl, ul = ((None, LIMIT), (1 - LIMIT, 1 + LIMIT)) if limited else ((None, None), (None, None))
    x = _padded_hidden(1, 500 + seed, cuda)
    out, ids, wts, lg = ops.layer_forward_mx(x, w, c["K"], act, gl, ul, return_routing=True)
    ref = ops.mx_experts(x, ids, wts, w, act, gl, ul)
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))


def test_gpt_oss_one_token_pairs_without_rows(cuda, gpt_oss_weights):
    """A token with fewer finite router logits than top-k (a NaN router bias on all but
    three experts) has pairs with no row (-1 ids): in the one-token down-and-combine
    launch they add nothing, as in moe_combine, so the output equals the op path bit
    for bit and stays finite."""
    import dataclasses
    c = GPT_OSS
    w = gpt_oss_weights
    say("gpt-oss one token, three candidates")
    keep = [5, 77, 120]
    bias = torch.full((c["E"],), float("nan"), device=cuda)
    bias[keep] = w.router_bias[keep] if w.router_bias is not None else 0.0
    w3 = dataclasses.replace(w, router_bias=bias)
    gl, ul = (None, LIMIT), (1 - LIMIT, 1 + LIMIT)
    x = _padded_hidden(1, 900, cuda)
    out, ids, wts, lg = ops.layer_forward_mx(x, w3, c["K"], "swish", gl, ul, return_routing=True)
    assert sorted(i for i in ids[0].tolist() if i >= 0) == keep
    assert int((ids[0] < 0).sum()) == c["K"] - 3
    ref = ops.mx_experts(x, ids, wts, w3, "swish", gl, ul)
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    assert bool(torch.isfinite(out.float()).all())


@pytest.mark.parametrize("T,with_res", [(1, True), (1, False), (4, True), (5, True)])
def test_gpt_oss_norm_rides_in_router_launch(cuda, gpt_oss_weights, T, with_res):
    """Up to four tokens the GPT-OSS layer's RMSNorm (and residual add) runs inside the
    router logits launch, whose MXFP8 quantization workgroups normalize the rows
    again and write the residual stream; from five tokens the norm is a launch of its
    own. Either way every output is the same bits as the layer without its norm, run
    on the rows ops.rms_norm_quant normalizes."""
    from oracle.moe import bf16_round
    c = GPT_OSS
    w = gpt_oss_weights
    say("gpt-oss norm in the router launch", T, with_res)
    x = _padded_hidden(T, 300 + T, cuda)
    r = _padded_hidden(T, 400 + T, cuda) if with_res else None
    gamma = torch.zeros(c["H"])
    gamma[:c["h_real"]] = 1 + 0.1 * torch.randn(c["h_real"], generator=torch.Generator().manual_seed(9))
    gamma = gamma.to(torch.bfloat16).float().to(cuda)
    args = (w, c["K"], "swish", (None, LIMIT), (1 - LIMIT, 1 + LIMIT))
    got = ops.layer_forward_mx(x, *args, return_routing=True, gamma=gamma, eps=1e-5,
                               hidden_actual=c["h_real"], residual=r)
    if with_res:
        out, rsum, *routing = got
        assert np.array_equal(np_f32(rsum), bf16_round(np_f32(x) + np_f32(r)))
    else:
        out, *routing = got
    xn = ops.rms_norm_quant(x, gamma, 1e-5, c["h_real"], r)[0]
    ref_out, *ref_routing = ops.layer_forward_mx(xn, *args, return_routing=True)
    assert torch.equal(out, ref_out)
    for a, b in zip(routing, ref_routing):  # ids, weights, logits
        assert torch.equal(a, b)


def _ids_from_dense(a):
    K = int((a != 0).sum(1).max())
    ids = np.zeros((a.shape[0], K), np.int32)
    wts = np.zeros((a.shape[0], K), np.float32)
    for t in range(a.shape[0]):
        nz = np.nonzero(a[t])[0]
        ids[t, :len(nz)] = nz
        wts[t, :len(nz)] = a[t, nz]
    return ids, wts


@pytest.mark.parametrize("T", [512, 2048])
def test_gpt_oss_moe_cte_mx_api(cuda, gpt_oss_weights, T):
    """The reference's GPT-OSS prefill call chain on MX experts: router (softmax, router
    bias) -> build_blockwise_mapping -> moe_cte(shard_on_block_mx, Swish, gate <= 7,
    -6 <= up <= 8, biases in the reference's [E, 2, I] / [E, 1, H] shapes, POST_SCALE)
    (model_bf16.py:1362-1470) against the oracle. At 2048 tokens (64 routed rows per
    expert) the tile height is capped at the 64 rows the MX kernels are built for."""
    from vllm_neuron_amd.functional import moe as M
    c, w = GPT_OSS, gpt_oss_weights
    say("gpt-oss moe_cte mx", T)
    x = _padded_hidden(T, 300, cuda)
    aff = M.router(x, w.router_w.t(), c["K"], router_bias=w.router_bias, activation="softmax")
    am, tpid, b2e, cond = M.build_blockwise_mapping(aff, c["E"], c["K"], 256)
    E, I2 = w.w13.shape[:2]
    out = M.moe_cte(x, am, w.w13, w.w2, tpid, b2e, 256, M.MoECTEImplementation.shard_on_block_mx,
                    conditions=cond, gate_and_up_proj_bias=w.b13.reshape(E, 2, I2 // 2),
                    down_proj_bias=w.b2.unsqueeze(1), gate_up_proj_scale=w.w13_scale,
                    down_proj_scale=w.w2_scale, activation_function=M.ActFnType.Swish,
                    quantization_type=M.QuantizationType.MX, gate_clamp_upper_limit=LIMIT,
                    up_clamp_upper_limit=LIMIT + 1, up_clamp_lower_limit=-LIMIT + 1,
                    expert_affinities_scaling_mode=M.ExpertAffinityScaleMode.POST_SCALE)
    ids, wts = _ids_from_dense(np_f32(aff))
    sel = np.array([0, 111, T - 1])
    ref = oracle_layer(x[sel], ids[sel], wts[sel], w, "swish", (None, LIMIT), (1 - LIMIT, 1 + LIMIT),
                       experts=set(np.unique(ids[sel]).tolist()))
    err = rel_l2(np_f32(out)[sel], ref)
    say("moe_cte mx rel_l2", err)
    assert err <= TOL_REL_L2, err


def test_gpt_oss_moe_block_tkg_mx_api(cuda, gpt_oss_weights):
    """The reference's GPT-OSS decode call (model_bf16.py:1274-1307): moe_block_tkg with
    gamma, router bias, softmax top-4 after the linear (router_pre_norm False), Swish,
    clamps, expert biases and hidden_actual 2880, on MX experts."""
    from oracle import router as R
    from oracle.moe import bf16_round
    from vllm_neuron_amd.functional import moe as M
    c, w = GPT_OSS, gpt_oss_weights
    T = 32
    say("gpt-oss moe_block_tkg mx", T)
    x = _padded_hidden(T, 400, cuda)
    gamma = torch.zeros(c["H"], device=cuda)
    gamma[:c["h_real"]] = 1.0
    E, I2 = w.w13.shape[:2]
    out, lg = M.moe_block_tkg(
        x.unsqueeze(0), gamma.unsqueeze(0), w.router_w.t(), w.w13, w.w2, top_k=c["K"],
        expert_gate_up_weights_scale=w.w13_scale, expert_down_weights_scale=w.w2_scale,
        router_bias=w.router_bias.unsqueeze(0), expert_gate_up_bias=w.b13.reshape(E, 2, I2 // 2),
        expert_down_bias=w.b2, eps=1e-5, router_act_fn=M.RouterActFnType.SOFTMAX,
        router_pre_norm=False, expert_affinities_scaling_mode=M.ExpertAffinityScaleMode.POST_SCALE,
        hidden_act_fn=M.ActFnType.Swish, gate_clamp_upper_limit=LIMIT,
        up_clamp_upper_limit=LIMIT + 1, up_clamp_lower_limit=-LIMIT + 1,
        hidden_actual=c["h_real"])
    xn = bf16_round(R.rms_norm_padded(np_f32(x), np_f32(gamma), 1e-5, c["h_real"]))
    lg = np_f32(lg)
    assert np.allclose(lg, R.router_logits(xn, np_f32(w.router_w), np_f32(w.router_bias)),
                       rtol=1e-5, atol=2e-5)
    ids, wts = R.route_topk_act(lg, c["K"], R.SOFTMAX)
    sel = np.array([0, 13, 31])
    ref = oracle_layer(xn[sel], ids[sel], wts[sel], w, "swish", (None, LIMIT), (1 - LIMIT, 1 + LIMIT),
                       experts=set(np.unique(ids[sel]).tolist()))
    err = rel_l2(np_f32(out.reshape(T, -1))[sel], ref)
    say("moe_block_tkg mx rel_l2", err)
    assert err <= TOL_REL_L2, err


@pytest.mark.parametrize("T", [1, 64])
def test_gpt_oss_layer_captures_in_hip_graph(cuda, gpt_oss_weights, T):
    """The GPT-OSS layer forward (norm with the residual add, router with the MXFP8
    quantization in its launch, top-k ending in the mapping, MX experts, combine)
    recorded into a HIP graph: three replays on new inputs, with eager work and
    synchronizations between them, each equal to an eager run bit for bit."""
    from vllm_neuron_amd import MXFP4MoE
    c = GPT_OSS
    say("gpt-oss hip graph", T)
    g = torch.Generator().manual_seed(40 + T)
    gamma = torch.zeros(c["H"])
    gamma[:c["h_real"]] = 1 + 0.1 * torch.randn(c["h_real"], generator=g)
    layer = MXFP4MoE(gpt_oss_weights, c["K"], norm_weight=gamma.to(cuda), eps=1e-5,
                     hidden_actual=c["h_real"])
    sx = _padded_hidden(T, 300 + T, cuda)
    sr = _padded_hidden(T, 400 + T, cuda)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):  # warm up the allocator and the library outside the capture
            layer(sx, None, False, None, residual=sr)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gout, gsum = layer(sx, None, False, None, residual=sr)
    for i in range(3):
        x = _padded_hidden(T, 500 + 10 * T + i, cuda)
        r = _padded_hidden(T, 600 + 10 * T + i, cuda)
        ref_out, ref_sum = layer(x, None, False, None, residual=r)
        torch.cuda.synchronize()
        sx.copy_(x)
        sr.copy_(r)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(gout, ref_out) and torch.equal(gsum, ref_sum), i
