"""moe_layer_forward_noalloc (the layer forward on the library's static per-GPU
scratch) against moe_layer_forward with a caller workspace, through the C ABI:
two calls in a row, the second with a smaller input, every output bit for bit."""
import pytest
import torch

from _util import say
from vllm_neuron_amd import MoEConfig, PRESETS, _lib, ops, synthetic

pytestmark = pytest.mark.gpu


def _same(a, b):
    a = a if isinstance(a, tuple) else (a,)
    b = b if isinstance(b, tuple) else (b,)
    assert len(a) == len(b)
    for u, v in zip(a, b):
        assert torch.equal(u, v)


def test_noalloc_matches_workspace_entry(cuda):
    cfg = MoEConfig(1024, 512, 16, 4, n_shared=1, scoring="sigmoid", grouped=True, n_group=4,
                    topk_group=2, renorm=True, routed_scaling=2.5)
    w = synthetic.make_weights(cfg, 11, device=cuda)
    g = torch.Generator().manual_seed(11)
    gamma = (1 + 0.1 * torch.randn(cfg.hidden, generator=g)).to(cuda)
    for T in (300, 37):  # the second call is smaller: stale rows of the first stay behind
        say("noalloc", T)
        x = synthetic.hidden_states(T, cfg.hidden, 11 + T).to(cuda)
        r = synthetic.hidden_states(T, cfg.hidden, 12 + T).to(cuda)
        kw = dict(return_routing=True, gamma=gamma, eps=1e-6, residual=r)
        _same(ops.layer_forward_noalloc(x, w, cfg, **kw), ops.layer_forward(x, w, cfg, **kw))
        _same(ops.layer_forward_noalloc(x, w, cfg), ops.layer_forward(x, w, cfg))


def test_noalloc_dsv3_decode_and_limit(cuda):
    """DeepSeek-V3 decode (64 tokens, then 8, then 1) on the static scratch; a call whose
    workspace exceeds the scratch is refused before any work is queued."""
    cfg = PRESETS["dsv3"]
    w = synthetic.make_weights(cfg, 1, device=cuda, experts_device=cuda)
    for T in (64, 8, 1):
        say("noalloc dsv3", T)
        x = synthetic.hidden_states(T, cfg.hidden, 1).to(cuda)
        _same(ops.layer_forward_noalloc(x, w, cfg, return_routing=True),
              ops.layer_forward(x, w, cfg, return_routing=True))
    lib = _lib.load()
    big = 4096
    assert lib.moe_layer_workspace_bytes(big, cfg.hidden, cfg.intermediate, cfg.n_experts,
                                         cfg.top_k, 1, 256, 0) > _lib.NOALLOC_SCRATCH_BYTES
    x = torch.zeros(big, cfg.hidden, dtype=torch.bfloat16, device=cuda)
    with pytest.raises(NotImplementedError, match="static scratch"):
        ops.layer_forward_noalloc(x, w, cfg)
    del w
    torch.cuda.empty_cache()
