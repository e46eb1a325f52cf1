"""torch.library registration (no GPU): every operator of the MoE path is a custom op
with a shape function, so graphs that call it trace with fake tensors and keep it as
one opaque node (the role of the reference's NKI higher-order op inside its compiled
graph, moe_cte.py:363-401; the model is compiled at neuron_model_runner.py:1773-1787).
The GPU tests check that compiled and eager runs give the same bits."""
import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

from vllm_neuron_amd import FP8BlockMoE, MoEConfig, PRESETS, synthetic
from vllm_neuron_amd.functional import moe as M
from vllm_neuron_amd.functional.moe.moe_blockwise import num_blocks

FP8 = torch.float8_e4m3fn
OPS = ("layer", "router", "blockwise_mapping", "moe_cte", "moe_block_tkg", "moe_tkg")


def test_operators_are_registered():
    for name in OPS:
        op = getattr(torch.ops.moe_fp8, name)
        assert op.default._schema.name == f"moe_fp8::{name}"


def test_num_blocks_matches_library():
    from vllm_neuron_amd import _lib
    lib = _lib.load()
    for T in (1, 3, 64, 333, 8192):
        for K, E, B in ((2, 8, 256), (8, 256, 256), (4, 16, 64), (1, 6, 1), (8, 384, 256)):
            assert num_blocks(T, K, E, B) == lib.moe_num_blocks(T, K, E, B)


def _small_layer(device="cpu", norm=True, S=0):
    cfg = PRESETS["small"].with_(n_experts=4, hidden=256, intermediate=128, n_shared=S)
    w = synthetic.make_weights(cfg, 0, device=device)
    gamma = torch.ones(cfg.hidden) if norm else None
    return cfg, FP8BlockMoE(cfg, w, norm_weight=gamma)


@pytest.mark.parametrize("with_residual", [False, True])
def test_layer_exports_as_one_node(with_residual):
    """torch.export traces the module with fake tensors (the shape function runs, the
    kernels do not) into a graph holding one moe_fp8.layer node."""
    cfg, layer = _small_layer(S=1)
    x = torch.zeros(10, cfg.hidden, dtype=torch.bfloat16)
    kw = {"residual": torch.zeros_like(x)} if with_residual else {}

    class Wrap(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.layer = layer

        def forward(self, x, residual=None):
            return self.layer(x, None, False, None, residual=residual)

    ep = torch.export.export(Wrap(), (x,), kwargs=kw)
    targets = [str(n.target) for n in ep.graph.nodes if n.op == "call_function"]
    assert targets.count("moe_fp8.layer.default") == 1, targets
    outs = [n for n in ep.graph.nodes if n.op == "output"][0].args[0]
    assert len(outs) == (2 if with_residual else 1)
    val = outs[0].meta["val"]
    assert tuple(val.shape) == (10, cfg.hidden) and val.dtype == torch.bfloat16


def test_shape_functions():
    """Each operator's fake implementation gives the output shapes and dtypes of the
    reference operator."""
    T, H, E, I, K, B = 37, 256, 8, 128, 2, 64
    with FakeTensorMode():
        x = torch.empty(T, H, dtype=torch.bfloat16)
        wr = torch.empty(H, E, dtype=torch.bfloat16)
        aff, lg = torch.ops.moe_fp8.router(x, wr, K, None, 0, None, 1e-6, torch.float32, 0, False)
        assert aff.shape == (T, E) and lg.shape == (T, E) and aff.dtype == torch.float32
        aff16, _ = torch.ops.moe_fp8.router(x, wr, K, None, 1, None, 1e-6, torch.float16, 1, True)
        assert aff16.dtype == torch.float16
        am, tpid, b2e, cond = torch.ops.moe_fp8.blockwise_mapping(aff, K, B, None)
        N = num_blocks(T, K, E, B)
        assert am.shape == (T * E, 1) and tpid.shape == (N * B,) and b2e.shape == (N,)
        assert cond.shape == (N,) and tpid.dtype == torch.int32
        gu = torch.empty(E, H, 2, I, dtype=FP8)
        dn = torch.empty(E, I, H, dtype=FP8)
        out = torch.ops.moe_fp8.moe_cte(x, am, gu, dn, None, None, tpid, b2e, B, False)
        assert out.shape == (T, H) and out.dtype == torch.bfloat16
        out32 = torch.ops.moe_fp8.moe_cte(torch.empty(T + 1, H), am, gu, dn, None, None, tpid,
                                          b2e, B, False)
        assert out32.shape == (T, H) and out32.dtype == torch.float32
        g = torch.empty(H)
        o, l, r = torch.ops.moe_fp8.moe_block_tkg(x, g, wr, gu, dn, None, None, None, None, None,
                                                  None, x, K, 1e-6, 1, True, False, False, 0)
        assert o.shape == (T, H) and l.shape == (T, E) and l.dtype == torch.float32
        assert r.shape == (T, H)
        ids = torch.empty(T, K, dtype=torch.int32)
        wts = torch.empty(T, K)
        o = torch.ops.moe_fp8.moe_tkg(x, gu, dn, None, None, ids, wts, torch.float32)
        assert o.shape == (T, H) and o.dtype == torch.float32


def test_functional_router_exports_as_one_node():
    class R(torch.nn.Module):
        def forward(self, x, w):
            return M.router(x, w, 2, return_logits=True)

    x = torch.zeros(5, 128, dtype=torch.bfloat16)
    w = torch.zeros(128, 8, dtype=torch.bfloat16)
    ep = torch.export.export(R(), (x, w))
    targets = [str(n.target) for n in ep.graph.nodes if n.op == "call_function"]
    assert "moe_fp8.router.default" in targets, targets
