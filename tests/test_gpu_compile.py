"""The MoE path inside compiled graphs and HIP graphs, on the GPU.

The reference embeds each kernel as an opaque node of its compiled graph
(moe_cte.py:363-401) and compiles the model (neuron_model_runner.py:1773-1787).
Here the operators are torch.library custom ops: a fullgraph torch.compile of the
layer module gives the eager result bit for bit, and the layer forward captures
into a HIP graph (no host synchronization, no allocation outside torch's graph
pool) whose replays match eager runs on new inputs."""
import pytest
import torch

from _util import say
from vllm_neuron_amd import FP8BlockMoE, MoEConfig, PRESETS, synthetic
from vllm_neuron_amd.functional import moe as M

pytestmark = pytest.mark.gpu


def _layer(cuda, cfg, seed, norm=True):
    w = synthetic.make_weights(cfg, seed, device=cuda)
    g = torch.Generator().manual_seed(seed)
    gamma = (1 + 0.1 * torch.randn(cfg.hidden, generator=g)).to(cuda) if norm else None
    return FP8BlockMoE(cfg, w, norm_weight=gamma, eps=1e-6)


CFGS = {
    "small": PRESETS["small"],
    "grouped_shared": MoEConfig(1024, 512, 16, 4, n_shared=1, scoring="sigmoid", grouped=True,
                                n_group=4, topk_group=2, renorm=True, routed_scaling=2.5),
}


@pytest.mark.parametrize("backend", ["aot_eager", "inductor"])
@pytest.mark.parametrize("name, T", [("small", 64), ("grouped_shared", 64),
                                     ("grouped_shared", 2048)])
def test_compiled_layer_equals_eager(cuda, name, T, backend):
    """torch.compile(fullgraph=True) of the module (decode, and prefill with a residual
    and padding positions) against eager, bit for bit; with the default backend
    (Inductor, which a vLLM-ROCm deployment compiles with) the custom ops stay opaque
    nodes and Inductor generates only the glue around them."""
    cfg = CFGS[name]
    say("compile layer", name, T, backend)
    torch._dynamo.reset()
    layer = _layer(cuda, cfg, 3)
    x = synthetic.hidden_states(T, cfg.hidden, 3).to(cuda)
    r = synthetic.hidden_states(T, cfg.hidden, 4).to(cuda)
    pos = torch.arange(T, device=cuda)
    pos[T - 5:] = 0

    def fwd(x, r, pos):
        dec = layer(x, None, True, None)
        out, rsum = layer(x, pos, False, None, residual=r)
        return dec, out, rsum

    ref = fwd(x, r, pos)
    comp = torch.compile(fwd, fullgraph=True, backend=backend)
    got = comp(x, r, pos)
    for a, b in zip(got, ref):
        assert torch.equal(a, b)
    # a second call with new values reuses the compiled graph
    x2 = synthetic.hidden_states(T, cfg.hidden, 5).to(cuda)
    for a, b in zip(comp(x2, r, pos), fwd(x2, r, pos)):
        assert torch.equal(a, b)


@pytest.mark.parametrize("backend", ["aot_eager", "inductor"])
def test_compiled_functional_ops_equal_eager(cuda, backend):
    """router -> build_blockwise_mapping -> moe_cte, and moe_block_tkg, compiled with
    fullgraph against eager."""
    say("compile functional", backend)
    torch._dynamo.reset()
    cfg = PRESETS["small"]
    w = synthetic.make_weights(cfg, 0, device=cuda)
    x = synthetic.hidden_states(64, cfg.hidden, 0).to(cuda)
    gamma = torch.ones(cfg.hidden, device=cuda)

    def prefill(x):
        aff = M.router(x, w.router_w.t(), cfg.top_k)
        am, tpid, b2e, cond = M.build_blockwise_mapping(aff, cfg.n_experts, cfg.top_k, 256)
        return M.moe_cte(x, am, w.w13, w.w2, tpid, b2e, 256, M.MoECTEImplementation.shard_on_block,
                         gate_up_proj_scale=w.w13_scale, down_proj_scale=w.w2_scale,
                         conditions=cond)

    def decode(x):
        return M.moe_block_tkg(x, gamma, w.router_w.t(), w.w13, w.w2, top_k=cfg.top_k,
                               expert_gate_up_weights_scale=w.w13_scale,
                               expert_down_weights_scale=w.w2_scale,
                               router_act_fn=M.RouterActFnType.SOFTMAX,
                               expert_affinities_scaling_mode=M.ExpertAffinityScaleMode.POST_SCALE)

    for fn in (prefill, decode):
        ref = fn(x)
        got = torch.compile(fn, fullgraph=True, backend=backend)(x)
        ref = ref if isinstance(ref, tuple) else (ref,)
        got = got if isinstance(got, tuple) else (got,)
        for a, b in zip(got, ref):
            assert torch.equal(a, b)


def test_opcheck_layer_and_operators(cuda):
    """torch.library.opcheck: schema (declared mutations and aliasing), fake-tensor
    shapes against the real outputs, and the autograd registration (no gradients:
    inference operators). The schema check cannot run on float8 inputs (it compares
    them arithmetically), so for the layer the inputs are compared bytewise instead."""
    say("opcheck")
    cfg = CFGS["grouped_shared"]
    layer = _layer(cuda, cfg, 6)
    w, c = layer.w, layer.cfg
    x = synthetic.hidden_states(40, cfg.hidden, 6).to(cuda)
    utils = ("test_schema", "test_faketensor", "test_autograd_registration")
    for res in (None, torch.zeros_like(x)):
        args = (x, res, layer.norm_weight, 1e-6, 0, w.router_w, w.router_bias, w.corr_bias,
                w.w13, w.w13_scale, w.w2, w.w2_scale, w.shared_w13, w.shared_w13_scale,
                w.shared_w2, w.shared_w2_scale, c.top_k, c.grouped, c.scoring, c.n_group,
                c.topk_group, c.renorm, float(c.routed_scaling), c.block_size)
        before = [a.view(torch.uint8).clone() if a.dtype == torch.float8_e4m3fn else a.clone()
                  for a in args if isinstance(a, torch.Tensor)]
        torch.library.opcheck(torch.ops.moe_fp8.layer.default, args, test_utils=utils[1:])
        after = [a.view(torch.uint8) if a.dtype == torch.float8_e4m3fn else a
                 for a in args if isinstance(a, torch.Tensor)]
        assert all(torch.equal(b, a) for b, a in zip(before, after))
    wt = w.router_w.t()
    torch.library.opcheck(torch.ops.moe_fp8.router.default,
                          (x, wt, 4, None, 1, None, 1e-6, torch.float32, 0, False),
                          test_utils=utils)
    aff = M.router(x, wt, 4)
    torch.library.opcheck(torch.ops.moe_fp8.blockwise_mapping.default, (aff, 4, 64, None),
                          test_utils=utils)


@pytest.mark.parametrize("T", [1, 64, 2048])  # 1: the one-workgroup top-k and mapping
def test_layer_captures_in_hip_graph(cuda, T):
    """The layer forward (norm, residual add, router, mapping, experts, combine)
    recorded into a HIP graph: three replays on new inputs, with eager work and
    synchronizations between them, each equal to an eager run bit for bit."""
    cfg = CFGS["grouped_shared"]
    say("hip graph", T)
    layer = _layer(cuda, cfg, 7)
    sx = synthetic.hidden_states(T, cfg.hidden, 7).to(cuda)
    sr = synthetic.hidden_states(T, cfg.hidden, 8).to(cuda)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):  # warm up the allocator and the library outside the capture
            layer(sx, None, False, None, residual=sr)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        gout, gsum = layer(sx, None, False, None, residual=sr)
    for i in range(3):
        x = synthetic.hidden_states(T, cfg.hidden, 20 + i).to(cuda)
        r = synthetic.hidden_states(T, cfg.hidden, 30 + i).to(cuda)
        ref_out, ref_sum = layer(x, None, False, None, residual=r)
        torch.cuda.synchronize()
        sx.copy_(x)
        sr.copy_(r)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(gout, ref_out) and torch.equal(gsum, ref_sum), i
