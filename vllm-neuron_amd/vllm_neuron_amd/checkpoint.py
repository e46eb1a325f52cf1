"""Load one MoE layer of a local safetensors checkpoint: DeepSeek-V3-format fp8
experts (load_moe_layer) or GPT-OSS MXFP4 experts (load_gpt_oss_moe_layer).

DeepSeek-V3, Kimi-K2 and GLM-4.5 publish their MoE layers under the same keys:

    {prefix}.{L}.mlp.gate.weight                          [E, H]  bf16 router
    {prefix}.{L}.mlp.gate.e_score_correction_bias         [E]     fp32 (grouped routing)
    {prefix}.{L}.mlp.experts.{e}.{gate,up}_proj.weight    [I, H]  float8_e4m3fn
    {prefix}.{L}.mlp.experts.{e}.down_proj.weight         [H, I]  float8_e4m3fn
    {prefix}.{L}.mlp.experts.{e}.*.weight_scale_inv       128x128 block scales, fp32
    {prefix}.{L}.mlp.shared_experts.{gate,up,down}_proj.*  one shared expert (optional)

The experts are read per expert in the [gate_w, gate_s, up_w, up_s] order of the
reference's fp8 enumeration (vllm_neuron/utils/weight_loader.py:719-744) and
stacked by ``weights.from_checkpoint_tensors``; nothing is re-quantized. A
directory is read as its sorted ``*.safetensors`` files, as the reference's local
checkpoint source does (utils/checkpoints.py:66-91), or through the shard map
``model.safetensors.index.json`` when one is present. Only local paths are read:
there is no download.
"""
import glob
import json
import os
from typing import Dict, Optional

import torch

from .weights import FP8, Fp8MoEWeights, from_checkpoint_tensors, split_shared_expert

try:
    from safetensors import safe_open
except ImportError:  # pragma: no cover - safetensors ships with the image
    safe_open = None


class CheckpointIndex:
    """key -> file of a local safetensors checkpoint (a file, or a directory)."""

    def __init__(self, path: str):
        if safe_open is None:
            raise RuntimeError("the safetensors package is required to read checkpoints")
        if os.path.isfile(path):
            files = [path]
            root = os.path.dirname(path)
        elif os.path.isdir(path):
            root = path
            idx = os.path.join(path, "model.safetensors.index.json")
            if os.path.exists(idx):
                with open(idx) as f:
                    wm = json.load(f)["weight_map"]
                self.key_file = {k: os.path.join(root, v) for k, v in wm.items()}
                self._handles = {}
                return
            files = sorted(glob.glob(os.path.join(path, "*.safetensors")))
        else:
            raise FileNotFoundError(f"no checkpoint at {path!r} (local files only)")
        if not files:
            raise FileNotFoundError(f"no .safetensors files under {path!r}")
        self.key_file = {}
        for fn in files:
            with safe_open(fn, framework="pt", device="cpu") as f:
                for k in f.keys():
                    self.key_file[k] = fn
        self._handles = {}

    def __contains__(self, key):
        return key in self.key_file

    def get(self, key: str) -> torch.Tensor:
        if key not in self.key_file:
            raise KeyError(f"checkpoint has no tensor {key!r}")
        fn = self.key_file[key]
        h = self._handles.get(fn)
        if h is None:
            h = safe_open(fn, framework="pt", device="cpu")
            self._handles[fn] = h
        return h.get_tensor(key)


def _check(t: torch.Tensor, shape, dtype, key: str) -> torch.Tensor:
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{key}: expected shape {tuple(shape)}, got {tuple(t.shape)}")
    if dtype is not None and t.dtype != dtype:
        raise ValueError(f"{key}: expected {dtype}, got {t.dtype}")
    return t


def load_moe_layer(path: str, layer: int, cfg, device="cuda", prefix: str = "model.layers",
                   index: Optional[CheckpointIndex] = None) -> Fp8MoEWeights:
    """Fp8MoEWeights of MoE layer ``layer`` of the checkpoint at ``path``.

    cfg gives E, H, I (and whether a correction bias is expected: cfg.grouped).
    A shared expert whose intermediate is a multiple of I is split into that many
    experts of intermediate I (the MLP sums over its intermediate columns)."""
    ix = index or CheckpointIndex(path)
    E, H, I = cfg.n_experts, cfg.hidden, cfg.intermediate
    base = f"{prefix}.{layer}.mlp"
    sI, sH = (I + 127) // 128, (H + 127) // 128

    def proj(owner: str, name: str, out_dim: int, in_dim: int):
        kw, ks = f"{owner}.{name}.weight", f"{owner}.{name}.weight_scale_inv"
        w = _check(ix.get(kw), (out_dim, in_dim), FP8, kw)
        s = _check(ix.get(ks), ((out_dim + 127) // 128, (in_dim + 127) // 128), None, ks).float()
        return w, s

    items, w2, s2 = [], [], []
    for e in range(E):
        own = f"{base}.experts.{e}"
        gw, gs = proj(own, "gate_proj", I, H)
        uw, us = proj(own, "up_proj", I, H)
        dw, ds = proj(own, "down_proj", H, I)
        items += [gw, gs, uw, us]
        w2.append(dw)
        s2.append(ds)
    w13, s13 = from_checkpoint_tensors(items, E)
    w2 = torch.stack(w2).contiguous()
    s2 = torch.stack(s2).float().contiguous()
    _check(s13, (E, 2 * sI, sH), torch.float32, "gate/up scales")

    kr = f"{base}.gate.weight"
    router_w = _check(ix.get(kr), (E, H), None, kr).to(torch.bfloat16).contiguous()
    kb = f"{base}.gate.e_score_correction_bias"
    corr = None
    if kb in ix:
        corr = _check(ix.get(kb), (E,), None, kb).float().contiguous()
    elif getattr(cfg, "grouped", False):
        raise ValueError(f"{kb} is missing but the configuration uses grouped routing")

    kw: Dict[str, torch.Tensor] = {}
    sh = f"{base}.shared_experts"
    if f"{sh}.gate_proj.weight" in ix:
        I_sh = ix.get(f"{sh}.gate_proj.weight").shape[0]
        gw, gs = proj(sh, "gate_proj", I_sh, H)
        uw, us = proj(sh, "up_proj", I_sh, H)
        dw, ds = proj(sh, "down_proj", H, I_sh)
        sw13, ss13 = torch.cat([gw, uw]), torch.cat([gs, us])
        a, b, c, d = split_shared_expert(sw13, ss13, dw, ds, I)
        if a.shape[0] != cfg.n_shared:
            raise ValueError(f"shared expert of intermediate {I_sh} is {a.shape[0]} experts of "
                             f"intermediate {I}; the configuration expects {cfg.n_shared}")
        kw = dict(shared_w13=a, shared_w13_scale=b, shared_w2=c, shared_w2_scale=d)
    elif cfg.n_shared:
        raise ValueError(f"{sh}.* is missing but the configuration has {cfg.n_shared} shared experts")

    w = Fp8MoEWeights(router_w=router_w, w13=w13, w13_scale=s13, w2=w2, w2_scale=s2,
                      corr_bias=corr, **kw).validate()
    return w.to(device) if device is not None else w


def load_gpt_oss_moe_layer(path: str, layer: int, hidden: Optional[int] = None,
                           intermediate: Optional[int] = None, device="cuda",
                           prefix: str = "model.layers",
                           index: Optional[CheckpointIndex] = None):
    """(MxMoEWeights, norm_weight) of MoE layer ``layer`` of a local HF GPT-OSS MXFP4
    checkpoint, under the keys the reference maps (model_mxfp4.py:2660-2695):

        {prefix}.{L}.mlp.router.weight / .bias                     [E, H] / [E]
        {prefix}.{L}.mlp.experts.gate_up_proj_blocks / _scales / _bias
                                      [E, 2I, H/32, 16] uint8 / [E, 2I, H/32] / [E, 2I]
        {prefix}.{L}.mlp.experts.down_proj_blocks / _scales / _bias
                                      [E, H, I/32, 16] uint8 / [E, H, I/32] / [E, H]
        {prefix}.{L}.post_attention_layernorm.weight                [H]

    Gate and up are de-interleaved and the up bias gets +1 as the reference's loaders
    do (weight_loaders_mxfp4.py:301-464); hidden / intermediate pad H and I with zeros
    (GPT-OSS: 2880 -> 3072). Codes and scales are not changed."""
    from .weights_mx import from_hf_gpt_oss
    ix = index or CheckpointIndex(path)
    base = f"{prefix}.{layer}"
    ex = f"{base}.mlp.experts"
    gub = ix.get(f"{ex}.gate_up_proj_blocks")
    if gub.dtype != torch.uint8 or gub.dim() != 4 or gub.shape[-1] != 16:
        raise ValueError(f"{ex}.gate_up_proj_blocks: expected uint8 [E, 2I, H/32, 16], got "
                         f"{gub.dtype} {tuple(gub.shape)}")
    E, I2, HB, _ = gub.shape
    H, I = HB * 32, I2 // 2
    gus = _check(ix.get(f"{ex}.gate_up_proj_scales"), (E, I2, HB), torch.uint8,
                 f"{ex}.gate_up_proj_scales")
    gb = _check(ix.get(f"{ex}.gate_up_proj_bias"), (E, I2), None, f"{ex}.gate_up_proj_bias")
    db = _check(ix.get(f"{ex}.down_proj_blocks"), (E, H, I // 32, 16), torch.uint8,
                f"{ex}.down_proj_blocks")
    ds = _check(ix.get(f"{ex}.down_proj_scales"), (E, H, I // 32), torch.uint8,
                f"{ex}.down_proj_scales")
    dbias = _check(ix.get(f"{ex}.down_proj_bias"), (E, H), None, f"{ex}.down_proj_bias")
    rw = _check(ix.get(f"{base}.mlp.router.weight"), (E, H), None, f"{base}.mlp.router.weight")
    rb = _check(ix.get(f"{base}.mlp.router.bias"), (E,), None, f"{base}.mlp.router.bias")
    kn = f"{base}.post_attention_layernorm.weight"
    norm = _check(ix.get(kn), (H,), None, kn).float() if kn in ix else None
    w = from_hf_gpt_oss(gub, gus, gb, db, ds, dbias, rw, rb, hidden=hidden,
                        intermediate=intermediate)
    if norm is not None and hidden is not None and hidden > H:
        norm = torch.cat([norm, torch.zeros(hidden - H)])
    if device is not None:
        w = type(w)(**{k: (v.to(device) if isinstance(v, torch.Tensor) else v)
                       for k, v in w.__dict__.items()})
        norm = None if norm is None else norm.to(device)
    return w, norm
