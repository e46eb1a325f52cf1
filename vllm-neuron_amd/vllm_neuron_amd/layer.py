"""The MoE expert layer as a torch module with the reference layer's forward signature.

Reference: GptOssExperts.forward(hidden_states, positions, is_decode, rank,
rsag_dispatch=False) (vllm_neuron/model/gpt_oss/model_bf16.py:1221-1232), which
dispatches to forward_prefill (router -> build_blockwise_mapping -> moe_cte,
:1347-1484) or forward_decode (fused moe_block_tkg, :1309-1345). Here both
phases run the same HIP pipeline (router logits -> top-k -> align -> 1x128
act quant -> fp8 gate_up/SiLU -> fp8 down -> combine) through one C-ABI call;
the phase only changes the row-tile height, which the library picks from the
average routed rows per expert (T*K/E).
"""
import torch

from . import ops
from .config import MoEConfig
from .weights import Fp8MoEWeights


class FP8BlockMoE(torch.nn.Module):
    def __init__(self, cfg: MoEConfig, weights: Fp8MoEWeights):
        super().__init__()
        weights.validate()
        if (weights.n_experts, weights.hidden, weights.intermediate) != (
                cfg.n_experts, cfg.hidden, cfg.intermediate):
            raise ValueError("weights do not match the config shape")
        if weights.n_shared != cfg.n_shared:
            raise ValueError(f"config has {cfg.n_shared} shared experts, weights {weights.n_shared}")
        self.cfg = cfg
        self.w = weights

    def forward(self, hidden_states, positions=None, is_decode=False, rank=None,
                rsag_dispatch=False):
        if rsag_dispatch:
            raise NotImplementedError("rsag_dispatch needs expert parallelism (one GPU here)")
        if rank is not None and int(torch.as_tensor(rank).reshape(-1)[0]) != 0:
            raise NotImplementedError("expert parallelism is not supported: rank must be 0")
        x = hidden_states
        lead = x.shape[:-1]
        x2 = x.reshape(-1, x.shape[-1])
        if x2.dtype != torch.bfloat16:
            raise ValueError(f"hidden_states must be bf16, got {x2.dtype}")
        out = ops.layer_forward(x2.contiguous(), self.w, self.cfg)
        if positions is not None and not is_decode:
            # model_bf16.py:1380-1384: tokens after the last real position are padding
            pos = positions.reshape(-1)
            keep = torch.arange(pos.numel(), device=pos.device) <= torch.argmax(pos)
            out = out * keep.to(out.dtype).unsqueeze(1)
        return out.reshape(*lead, out.shape[-1])
