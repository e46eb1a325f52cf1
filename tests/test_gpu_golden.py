"""The HIP path against the committed golden fixtures (tests/golden/*.npz).

Bit-exact gates: top-k ids, the blockwise mapping (token_position_to_id,
block_to_expert, conditions, expert counts, inverse positions) and the 1x128 fp8
activation codes and scales. Float gates: router logits within fp32 summation-order
tolerance, top-k weights within 1e-5 relative (they are computed from the GPU's own
logits), layer output rel-L2 <= 1e-2 against the frozen fp32 oracle output."""
import numpy as np
import pytest
import torch

from _util import rel_l2, say
from golden.cases import BLOCK, CASES, gen_inputs, load
from vllm_neuron_amd import MoEConfig, ops
from vllm_neuron_amd.weights import Fp8MoEWeights

pytestmark = pytest.mark.gpu
TOL_REL_L2 = 1e-2


def _device_case(case, dev):
    c = CASES[case]
    f = load(case)
    inp = gen_inputs(case)
    fp8 = lambda a: torch.from_numpy(np.ascontiguousarray(a)).view(torch.float8_e4m3fn).to(dev)
    f32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)
    bf16 = lambda bits: torch.from_numpy(bits.astype(np.int16)).view(torch.bfloat16).to(dev)
    kw = {}
    if inp["shared"] is not None:
        q13, s13, q2, s2 = inp["shared"]
        kw = dict(shared_w13=fp8(q13[None]), shared_w13_scale=f32(s13[None]),
                  shared_w2=fp8(q2[None]), shared_w2_scale=f32(s2[None]))
    w = Fp8MoEWeights(router_w=bf16(inp["router_w_bits"]), w13=fp8(inp["w13"]),
                      w13_scale=f32(inp["w13_scale"]), w2=fp8(inp["w2"]), w2_scale=f32(inp["w2_scale"]),
                      router_bias=None if inp["router_bias"] is None else f32(inp["router_bias"]),
                      corr_bias=None if inp["corr_bias"] is None else f32(inp["corr_bias"]),
                      **kw).validate()
    cfg = MoEConfig(c["H"], c["I"], c["E"], c["K"], n_shared=c["n_shared"], scoring=c["scoring"],
                    grouped=c["grouped"], n_group=c["n_group"], topk_group=c["topk_group"],
                    renorm=c["renorm"], routed_scaling=c["scale"], block_size=BLOCK)
    x = bf16(f["x_bits"])
    return cfg, w, x, f


@pytest.mark.parametrize("case", sorted(CASES))
def test_layer_against_fixture(cuda, case):
    say("golden layer", case)
    cfg, w, x, f = _device_case(case, cuda)
    out, ids, wts, lg = ops.layer_forward(x, w, cfg, return_routing=True)
    torch.cuda.synchronize()
    assert np.allclose(lg.cpu().numpy(), f["logits"], rtol=1e-5, atol=2e-5), case
    assert np.array_equal(ids.cpu().numpy(), f["ids"]), case
    assert np.allclose(wts.cpu().numpy(), f["weights"], rtol=1e-5, atol=1e-7), case
    err = rel_l2(out.float().cpu().numpy(), f["out"])
    say(case, "rel_l2", err)
    assert err <= TOL_REL_L2, (case, err)


@pytest.mark.parametrize("case", sorted(CASES))
def test_mapping_and_act_quant_against_fixture(cuda, case):
    say("golden mapping / act quant", case)
    cfg, w, x, f = _device_case(case, cuda)
    ids = torch.from_numpy(f["ids"]).to(cuda)
    m = ops.blockwise_mapping(ids=ids, n_experts=cfg.n_experts, block_size=BLOCK, check=True)
    for k in ("token_position_to_id", "block_to_expert", "conditions", "expert_counts", "inv_pos"):
        assert np.array_equal(m[k].cpu().numpy(), f[k]), (case, k)
    q, s = ops.act_quant(x)
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), f["xq"]), case
    assert np.array_equal(s.cpu().numpy(), f["xs"]), case
