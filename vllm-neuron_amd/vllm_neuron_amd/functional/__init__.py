"""Operator API mirroring vllm_neuron.functional (functional/__init__.py:30-51)
for the MoE path."""
from .moe import (ActFnType, ExpertAffinityScaleMode, MoECTEImplementation,  # noqa: F401
                  QuantizationType, RouterActFnType, RouterComputationOrder,
                  build_blockwise_mapping, moe_block_tkg, moe_cte, moe_tkg, router)
