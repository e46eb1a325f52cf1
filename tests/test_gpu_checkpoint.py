"""Checkpoint path on the GPU: a layer written to local safetensors under the HF keys,
loaded by the product's loaders and run, against the same layer built in memory (bit
for bit) and against the oracle.

* DeepSeek-V3 format (fp8 experts with 128x128 weight_scale_inv, per-expert keys in
  the [gate_w, gate_s, up_w, up_s] enumeration of utils/weight_loader.py:719-744):
  load_moe_layer -> FP8BlockMoE.
* GPT-OSS MXFP4 format (the keys of model_mxfp4.py:2660-2695, interleaved gate / up,
  E8M0 scales, biases): load_gpt_oss_moe_layer -> MXFP4MoE, hidden 2880 padded to 3072."""
import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from _util import np_f32, oracle_shared, oracle_weights, rel_l2, say
from oracle import router as R
from oracle.moe import moe_sparse_fp8
from test_checkpoint import LAYER, _hf_tensors, gpt_oss_hf_tensors
from vllm_neuron_amd import FP8BlockMoE, MXFP4MoE, PRESETS, ops, synthetic
from vllm_neuron_amd.checkpoint import load_gpt_oss_moe_layer, load_moe_layer

pytestmark = pytest.mark.gpu


def test_dsv3_checkpoint_layer(cuda, tmp_path):
    cfg = PRESETS["dsv3"].with_(n_experts=16, n_group=8, topk_group=4, top_k=4)
    say("dsv3 checkpoint", cfg.n_experts)
    w = synthetic.make_weights(cfg, 50, device="cpu", experts_device=cuda)
    save_file(_hf_tensors(w), str(tmp_path / "model.safetensors"))
    v = load_moe_layer(str(tmp_path), LAYER, cfg, device=cuda)
    wd = w.to(cuda)
    g = torch.Generator().manual_seed(50)
    gamma = (1 + 0.1 * torch.randn(cfg.hidden, generator=g)).to(torch.bfloat16).float().to(cuda)
    x = synthetic.hidden_states(64, cfg.hidden, 50).to(cuda)
    out = FP8BlockMoE(cfg, v, norm_weight=gamma)(x, None, True, None)
    assert torch.equal(out, FP8BlockMoE(cfg, wd, norm_weight=gamma)(x, None, True, None))
    _, ids, wts, lg = ops.layer_forward(x, v, cfg, return_routing=True, gamma=gamma)
    xn = ops.rms_norm_quant(x, gamma, 1e-6)[0]
    lg, ids, wts = lg.cpu().numpy(), ids.cpu().numpy(), wts.cpu().numpy()
    oi, ow = R.route_grouped(lg, np_f32(v.corr_bias), cfg.top_k, cfg.n_group, cfg.topk_group,
                             R.SIGMOID, cfg.renorm, 1e-20, cfg.routed_scaling)
    assert np.array_equal(ids, oi) and np.array_equal(wts, ow)
    q13, s13, q2, s2 = oracle_weights(v)
    ref = moe_sparse_fp8(np_f32(xn), ids, wts, q13, s13, q2, s2, shared=oracle_shared(v))
    err = rel_l2(np_f32(out), ref)
    say("dsv3 checkpoint rel_l2", err)
    assert err <= 1e-2, err


def test_gpt_oss_checkpoint_layer(cuda, tmp_path):
    from test_gpu_mx import LIMIT, oracle_layer
    E, Hp, Ip, H, I = 8, 3072, 3072, 2880, 2880
    say("gpt-oss checkpoint", E)
    w = synthetic.make_mx_weights(E, Hp, Ip, 60, device=cuda, h_real=H, i_real=I)
    # the HF tensors of these weights: interleaved rows, real sizes, up bias without the +1
    cpu = lambda t: t.cpu()
    gub = torch.empty(E, 2 * I, H // 32, 16, dtype=torch.uint8)
    gub[:, 0::2] = cpu(w.w13[:, :I, :H // 2]).reshape(E, I, H // 32, 16)
    gub[:, 1::2] = cpu(w.w13[:, Ip:Ip + I, :H // 2]).reshape(E, I, H // 32, 16)
    gus = torch.empty(E, 2 * I, H // 32, dtype=torch.uint8)
    gus[:, 0::2] = cpu(w.w13_scale[:, :I, :H // 32])
    gus[:, 1::2] = cpu(w.w13_scale[:, Ip:Ip + I, :H // 32])
    gb = torch.empty(E, 2 * I)
    gb[:, 0::2] = cpu(w.b13[:, :I])
    gb[:, 1::2] = cpu(w.b13[:, Ip:Ip + I]) - 1.0
    db = cpu(w.w2[:, :H, :I // 2]).reshape(E, H, I // 32, 16).contiguous()
    ds = cpu(w.w2_scale[:, :H, :I // 32]).contiguous()
    dbias = cpu(w.b2[:, :H]).contiguous()
    norm = (1 + 0.1 * torch.randn(H, generator=torch.Generator().manual_seed(60))).to(torch.bfloat16)
    save_file(gpt_oss_hf_tensors(gub, gus, gb, db, ds, dbias, cpu(w.router_w[:, :H]).contiguous(),
                                 cpu(w.router_bias), norm), str(tmp_path / "model.safetensors"))
    v, nw = load_gpt_oss_moe_layer(str(tmp_path), LAYER, hidden=Hp, intermediate=Ip, device=cuda)
    for k in ("w13", "w13_scale", "w2", "w2_scale", "b13", "b2", "router_w", "router_bias"):
        assert torch.equal(getattr(v, k), getattr(w, k)), k
    x = torch.zeros(48, Hp)
    x[:, :H] = torch.randn(48, H, generator=torch.Generator().manual_seed(61))
    x = x.to(torch.bfloat16).to(cuda)
    layer = MXFP4MoE(v, 4, norm_weight=nw, eps=1e-5, hidden_actual=H)
    out = layer(x, None, True, None)
    assert torch.equal(out, MXFP4MoE(w, 4, norm_weight=nw, eps=1e-5, hidden_actual=H)(x, None, True, None))
    _, ids, wts, lg = ops.layer_forward_mx(x, v, 4, "swish", (None, LIMIT), (1 - LIMIT, 1 + LIMIT),
                                           return_routing=True, gamma=nw, eps=1e-5, hidden_actual=H)
    xn = ops.rms_norm(x, nw, 1e-5, H)
    ids, wts = ids.cpu().numpy(), wts.cpu().numpy()
    oi, ow = R.route_topk_act(lg.cpu().numpy(), 4, R.SOFTMAX)
    assert np.array_equal(ids, oi) and np.array_equal(wts, ow)
    sel = np.array([0, 20, 47])
    ref = oracle_layer(np_f32(xn)[sel], ids[sel], wts[sel], v, "swish", (None, LIMIT),
                       (1 - LIMIT, 1 + LIMIT), experts=set(np.unique(ids[sel]).tolist()))
    err = rel_l2(np_f32(out)[sel], ref)
    say("gpt-oss checkpoint rel_l2", err)
    assert err <= 1e-2, err
