"""MoE operators with the signatures of vllm_neuron.functional.moe (router,
build_blockwise_mapping, moe_cte, moe_tkg, moe_block_tkg) over the HIP kernels."""
from .moe_blockwise import build_blockwise_mapping  # noqa: F401
from .moe_block_tkg import moe_block_tkg  # noqa: F401
from .moe_cte import moe_cte  # noqa: F401
from .moe_tkg import moe_tkg  # noqa: F401
from .router import RouterComputationOrder, router  # noqa: F401
from .types import (ActFnType, BlockShardStrategy, ExpertAffinityScaleMode,  # noqa: F401
                    MoEAllToAllVStrategy, MoECTEImplementation, QuantizationType,
                    RouterActFnType)
