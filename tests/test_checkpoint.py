"""Checkpoint loader (CPU): a DeepSeek-V3-format fp8 MoE layer written to local
safetensors files (per-expert keys, 128x128 weight_scale_inv blocks) loads back into
exactly the stacked tensors it was written from, through a sharded index or a plain
directory scan; missing or mis-shaped tensors raise."""
import json
import os

import pytest
import torch
from safetensors.torch import save_file

from vllm_neuron_amd import PRESETS, synthetic
from vllm_neuron_amd.checkpoint import CheckpointIndex, load_moe_layer

LAYER = 3


def _hf_tensors(w, layer=LAYER):
    """The checkpoint keys of one MoE layer from a stacked Fp8MoEWeights."""
    E, I2, H = w.w13.shape
    I = I2 // 2
    base = f"model.layers.{layer}.mlp"
    out = {f"{base}.gate.weight": w.router_w.clone()}
    if w.corr_bias is not None:
        out[f"{base}.gate.e_score_correction_bias"] = w.corr_bias.clone()
    for e in range(E):
        own = f"{base}.experts.{e}"
        out[f"{own}.gate_proj.weight"] = w.w13[e, :I].clone()
        out[f"{own}.up_proj.weight"] = w.w13[e, I:].clone()
        out[f"{own}.gate_proj.weight_scale_inv"] = w.w13_scale[e, :I // 128].clone()
        out[f"{own}.up_proj.weight_scale_inv"] = w.w13_scale[e, I // 128:].clone()
        out[f"{own}.down_proj.weight"] = w.w2[e].clone()
        out[f"{own}.down_proj.weight_scale_inv"] = w.w2_scale[e].clone()
    if w.shared_w13 is not None:
        sh = f"{base}.shared_experts"
        S = w.shared_w13.shape[0]
        out[f"{sh}.gate_proj.weight"] = torch.cat([w.shared_w13[j, :I] for j in range(S)])
        out[f"{sh}.up_proj.weight"] = torch.cat([w.shared_w13[j, I:] for j in range(S)])
        out[f"{sh}.gate_proj.weight_scale_inv"] = torch.cat([w.shared_w13_scale[j, :I // 128] for j in range(S)])
        out[f"{sh}.up_proj.weight_scale_inv"] = torch.cat([w.shared_w13_scale[j, I // 128:] for j in range(S)])
        out[f"{sh}.down_proj.weight"] = torch.cat([w.shared_w2[j] for j in range(S)], dim=1)
        out[f"{sh}.down_proj.weight_scale_inv"] = torch.cat([w.shared_w2_scale[j] for j in range(S)], dim=1)
    return {k: v.contiguous() for k, v in out.items()}


def _same(a, b):
    if a is None or b is None:
        return a is None and b is None
    if a.dtype == torch.float8_e4m3fn:
        a, b = a.view(torch.uint8), b.view(torch.uint8)
    return a.dtype == b.dtype and torch.equal(a, b)


def _assert_equal_weights(w, v):
    for k in ("router_w", "w13", "w13_scale", "w2", "w2_scale", "corr_bias", "shared_w13",
              "shared_w13_scale", "shared_w2", "shared_w2_scale"):
        assert _same(getattr(w, k), getattr(v, k)), k


@pytest.fixture(scope="module")
def small():
    cfg = PRESETS["small"].with_(scoring="sigmoid", grouped=True, n_shared=1)
    return cfg, synthetic.make_weights(cfg, 5)


def test_sharded_index_round_trip(tmp_path, small):
    cfg, w = small
    t = _hf_tensors(w)
    keys = sorted(t)
    half = len(keys) // 2
    shards = {"model-00001-of-00002.safetensors": keys[:half],
              "model-00002-of-00002.safetensors": keys[half:]}
    wm = {}
    for fn, ks in shards.items():
        save_file({k: t[k] for k in ks}, str(tmp_path / fn))
        wm.update({k: fn for k in ks})
    with open(tmp_path / "model.safetensors.index.json", "w") as f:
        json.dump({"metadata": {}, "weight_map": wm}, f)
    v = load_moe_layer(str(tmp_path), LAYER, cfg, device=None)
    _assert_equal_weights(w, v)


def test_directory_scan_round_trip(tmp_path, small):
    cfg, w = small
    t = _hf_tensors(w)
    t["model.layers.0.self_attn.q_proj.weight"] = torch.zeros(4, 4)   # other layers are ignored
    save_file(t, str(tmp_path / "model.safetensors"))
    v = load_moe_layer(str(tmp_path), LAYER, cfg, device=None)
    _assert_equal_weights(w, v)
    ix = CheckpointIndex(str(tmp_path / "model.safetensors"))   # a single file works too
    _assert_equal_weights(w, load_moe_layer(None, LAYER, cfg, device=None, index=ix))


def test_wide_shared_expert_is_split(tmp_path):
    """A shared expert of intermediate 2I loads as two experts of intermediate I."""
    cfg = PRESETS["small"].with_(n_shared=2)
    w = synthetic.make_weights(cfg, 6)
    save_file(_hf_tensors(w), str(tmp_path / "m.safetensors"))
    v = load_moe_layer(str(tmp_path), LAYER, cfg, device=None)
    _assert_equal_weights(w, v)


def test_missing_and_misshaped_tensors_raise(tmp_path, small):
    cfg, w = small
    t = _hf_tensors(w)
    base = f"model.layers.{LAYER}.mlp"
    bad = dict(t)
    del bad[f"{base}.experts.1.down_proj.weight_scale_inv"]
    save_file(bad, str(tmp_path / "a.safetensors"))
    with pytest.raises(KeyError):
        load_moe_layer(str(tmp_path / "a.safetensors"), LAYER, cfg, device=None)
    bad = dict(t)
    bad[f"{base}.experts.0.gate_proj.weight"] = bad[f"{base}.experts.0.gate_proj.weight"][:-1].contiguous()
    save_file(bad, str(tmp_path / "b.safetensors"))
    with pytest.raises(ValueError):
        load_moe_layer(str(tmp_path / "b.safetensors"), LAYER, cfg, device=None)
    bad = dict(t)
    del bad[f"{base}.gate.e_score_correction_bias"]
    save_file(bad, str(tmp_path / "c.safetensors"))
    with pytest.raises(ValueError, match="grouped"):
        load_moe_layer(str(tmp_path / "c.safetensors"), LAYER, cfg, device=None)
    with pytest.raises(FileNotFoundError):
        load_moe_layer(str(tmp_path / "nothing_here"), LAYER, cfg, device=None)
    os.makedirs(tmp_path / "empty")
    with pytest.raises(FileNotFoundError):
        load_moe_layer(str(tmp_path / "empty"), LAYER, cfg, device=None)


def gpt_oss_hf_tensors(gub, gus, gb, db, ds, dbias, rw, rb, norm, layer=LAYER):
    base = f"model.layers.{layer}"
    ex = f"{base}.mlp.experts"
    return {f"{ex}.gate_up_proj_blocks": gub, f"{ex}.gate_up_proj_scales": gus,
            f"{ex}.gate_up_proj_bias": gb, f"{ex}.down_proj_blocks": db,
            f"{ex}.down_proj_scales": ds, f"{ex}.down_proj_bias": dbias,
            f"{base}.mlp.router.weight": rw, f"{base}.mlp.router.bias": rb,
            f"{base}.post_attention_layernorm.weight": norm}


def test_gpt_oss_mxfp4_checkpoint_round_trip(tmp_path):
    """A GPT-OSS MXFP4 layer under the HF keys the reference maps (model_mxfp4.py:
    2660-2695) loads into the oracle's stacked layout: gate / up de-interleaved, +1 on
    the up bias, H and I zero-padded, codes and scales unchanged."""
    import numpy as np

    from oracle import mx as OX
    from vllm_neuron_amd.checkpoint import load_gpt_oss_moe_layer
    g = torch.Generator().manual_seed(9)
    E, I, H = 4, 96, 160
    gub = torch.randint(0, 256, (E, 2 * I, H // 32, 16), generator=g, dtype=torch.int32).to(torch.uint8)
    gus = torch.randint(118, 134, (E, 2 * I, H // 32), generator=g, dtype=torch.int32).to(torch.uint8)
    gb = torch.randn(E, 2 * I, generator=g).to(torch.bfloat16)
    db = torch.randint(0, 256, (E, H, I // 32, 16), generator=g, dtype=torch.int32).to(torch.uint8)
    ds = torch.randint(118, 134, (E, H, I // 32), generator=g, dtype=torch.int32).to(torch.uint8)
    dbias = torch.randn(E, H, generator=g).to(torch.bfloat16)
    rw = torch.randn(E, H, generator=g).to(torch.bfloat16)
    rb = torch.randn(E, generator=g).to(torch.bfloat16)
    norm = torch.randn(H, generator=g).to(torch.bfloat16)
    save_file(gpt_oss_hf_tensors(gub, gus, gb, db, ds, dbias, rw, rb, norm),
              str(tmp_path / "model.safetensors"))
    w, nw = load_gpt_oss_moe_layer(str(tmp_path), LAYER, hidden=256, intermediate=128, device=None)
    ow13, os13, ob13, ow2, os2, ob2 = OX.from_hf_gpt_oss(
        gub.numpy(), gus.numpy(), gb.float().numpy(), db.numpy(), ds.numpy(), dbias.float().numpy())
    assert np.array_equal(w.w13[:, :I, :H // 2].numpy(), ow13[:, :I])
    assert np.array_equal(w.w13[:, 128:128 + I, :H // 2].numpy(), ow13[:, I:])
    assert np.array_equal(w.w13_scale[:, 128:128 + I, :H // 32].numpy(), os13[:, I:])
    assert np.array_equal(w.b13[:, 128:128 + I].numpy(), ob13[:, I:])
    assert np.array_equal(w.w2[:, :H, :I // 2].numpy(), ow2)
    assert np.array_equal(w.w2_scale[:, :H, :I // 32].numpy(), os2)
    assert np.array_equal(w.b2[:, :H].numpy(), ob2)
    assert torch.equal(w.router_w[:, :H], rw) and torch.all(w.router_w[:, H:] == 0)
    assert torch.equal(nw[:H], norm.float()) and torch.all(nw[H:] == 0)
    with pytest.raises(KeyError):
        load_gpt_oss_moe_layer(str(tmp_path), LAYER + 1, device=None)
