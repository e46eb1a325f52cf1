"""Enums of the MoE operator API.

The reference imports these from nkilib's common_types (moe_cte.py:9-20,
moe_block_tkg.py:9-13, router.py:11); nkilib is not part of the reference tree,
so the member names are taken from their uses there. This build implements
SiLU with POST_SCALE or NO_SCALE affinities and SOFTMAX / SIGMOID routers;
other members are accepted as values and rejected with NotImplementedError by
the functions that receive them.
"""
from enum import Enum


class ActFnType(Enum):
    SiLU = "silu"
    GELU = "gelu"
    Swish = "swish"


class ExpertAffinityScaleMode(Enum):
    NO_SCALE = "no_scale"
    POST_SCALE = "post_scale"
    PRE_SCALE = "pre_scale"
    PRE_SCALE_DELAYED = "pre_scale_delayed"


class RouterActFnType(Enum):
    SOFTMAX = "softmax"
    SIGMOID = "sigmoid"


class MoECTEImplementation(Enum):
    shard_on_block = "shard_on_block"
    shard_on_i = "shard_on_i"
    shard_on_i_hybrid = "shard_on_i_hybrid"
    shard_on_i_dropping = "shard_on_i_dropping"
    shard_on_block_mx = "shard_on_block_mx"
    shard_on_i_mx = "shard_on_i_mx"
    shard_on_i_mx_hybrid = "shard_on_i_mx_hybrid"


class BlockShardStrategy(Enum):
    PING_PONG = "ping_pong"
    HI_LO = "hi_lo"


class QuantizationType(Enum):
    NONE = "none"
    MX = "mx"
    STATIC_MX = "static_mx"


class MoEAllToAllVStrategy(Enum):
    DISABLED = "disabled"
    ENABLED = "enabled"


MX_IMPLEMENTATIONS = (MoECTEImplementation.shard_on_block_mx, MoECTEImplementation.shard_on_i_mx,
                      MoECTEImplementation.shard_on_i_mx_hybrid)
