"""MI355X-native FP8-blockwise fused-MoE layer (gfx950 HIP kernels behind a C ABI).

Host-side mirror of the MoE operator API of the vllm-neuron plugin
(vllm_neuron/functional/moe/: router, build_blockwise_mapping, moe_cte,
moe_block_tkg) and of its MoE layer forward, with DeepSeek-V3 style fp8
128x128 block-scaled experts or GPT-OSS MXFP4 experts. All compute runs in the HIP library
``lib/libmoe_fp8.so``; there is no CPU fallback.
"""
from .config import MoEConfig, PRESETS  # noqa: F401
from .layer import FP8BlockMoE  # noqa: F401
from .layer_mx import MXFP4MoE  # noqa: F401
from .weights import Fp8MoEWeights  # noqa: F401
from .weights_mx import MxMoEWeights  # noqa: F401

__all__ = ["MoEConfig", "PRESETS", "FP8BlockMoE", "Fp8MoEWeights", "MXFP4MoE", "MxMoEWeights"]
