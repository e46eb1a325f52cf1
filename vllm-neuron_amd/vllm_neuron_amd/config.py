"""Layer configuration and the named workload shapes."""
from dataclasses import dataclass, replace


@dataclass(frozen=True)
class MoEConfig:
    """Shape and routing of one fp8-blockwise MoE layer.

    scoring: "softmax" or "sigmoid"; grouped: DeepSeek-V3 grouped top-k with a
    selection-only correction bias (n_group / topk_group); otherwise the
    reference's default order (topk on logits, then activation,
    router.py:384-441). renorm divides the top-k weights by their sum + 1e-20
    (moe_block_tkg.py:182-185); routed_scaling multiplies them afterwards.
    """
    hidden: int
    intermediate: int
    n_experts: int
    top_k: int
    n_shared: int = 0
    scoring: str = "softmax"
    grouped: bool = False
    n_group: int = 1
    topk_group: int = 1
    renorm: bool = False
    routed_scaling: float = 1.0
    block_size: int = 256

    def with_(self, **kw):
        return replace(self, **kw)


# Named workloads (hidden, moe intermediate, routed experts, top-k, shared experts, routing).
PRESETS = {
    # small CPU-runnable layer: softmax top-2, no shared expert
    "small": MoEConfig(1024, 512, 8, 2),
    # DeepSeek-V3: sigmoid + correction bias, 8 groups / 4 kept, top-8, x2.5, 1 shared expert
    "dsv3": MoEConfig(7168, 2048, 256, 8, n_shared=1, scoring="sigmoid", grouped=True,
                      n_group=8, topk_group=4, renorm=True, routed_scaling=2.5),
    # Kimi-K2: 384 experts, sigmoid grouped top-8 with one group, x2.827
    "kimi_k2": MoEConfig(7168, 2048, 384, 8, n_shared=1, scoring="sigmoid", grouped=True,
                         n_group=1, topk_group=1, renorm=True, routed_scaling=2.827),
    # GLM-4.5: 160 experts, sigmoid top-8 with correction bias, x2.5
    "glm45": MoEConfig(5120, 1536, 160, 8, n_shared=1, scoring="sigmoid", grouped=True,
                       n_group=1, topk_group=1, renorm=True, routed_scaling=2.5),
}
