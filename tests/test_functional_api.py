"""Host-side behaviour of the operator mirrors (no GPU): argument validation raises
the reference's exception types before any kernel runs (router.py:602-678 ValueError;
moe_block_tkg.py:534-565 / moe_cte.py:300-313 NotImplementedError), and CPU tensors
are refused (no CPU path)."""
import pytest
import torch

from vllm_neuron_amd.functional import moe as M

FP8 = torch.float8_e4m3fn


def _router_args(T=4, H=128, E=8):
    return torch.zeros(T, H, dtype=torch.bfloat16), torch.zeros(H, E, dtype=torch.bfloat16)


@pytest.mark.parametrize("mutate, exc", [
    (lambda a: dict(a, hidden_states=torch.zeros(2, 4, 128)), ValueError),
    (lambda a: dict(a, router_weights=torch.zeros(64, 8)), ValueError),
    (lambda a: dict(a, top_k=0), ValueError),
    (lambda a: dict(a, top_k=9), ValueError),
    (lambda a: dict(a, router_bias=torch.zeros(7)), ValueError),
    (lambda a: dict(a, gamma=torch.zeros(64)), ValueError),
    (lambda a: dict(a, computation_dtype=torch.int32), ValueError),
    (lambda a: dict(a, router_computation_order="prenorm_linear_topk_act_scatter"), ValueError),
    (lambda a: dict(a, activation="relu"), ValueError),
    (lambda a: dict(a, activation=3), ValueError),
    (lambda a: dict(a, activation=torch.sigmoid), NotImplementedError),
])
def test_router_validation(mutate, exc):
    x, w = _router_args()
    args = dict(hidden_states=x, router_weights=w, top_k=2)
    with pytest.raises(exc):
        M.router(**mutate(args))


def test_router_refuses_cpu_tensors():
    x, w = _router_args()
    with pytest.raises(RuntimeError, match="GPU"):
        M.router(x, w, 2)


def test_transposed_hidden_states_shape_check():
    x, w = _router_args()
    with pytest.raises(ValueError):
        M.router(x, w, 2, transposed_hidden_states=True)   # [T,H] read as [H,T]


def _experts(E=2, H=256, I=128):
    return torch.zeros(E, H, 2, I, dtype=FP8), torch.zeros(E, I, H, dtype=FP8)


@pytest.mark.parametrize("kw", [
    dict(quantization_type=M.QuantizationType.STATIC_MX),
    dict(activation_function=M.ActFnType.GELU),
    dict(expert_affinities_scaling_mode=M.ExpertAffinityScaleMode.PRE_SCALE),
    dict(gate_clamp_upper_limit=8.0),
    dict(gate_and_up_proj_bias=torch.zeros(2, 2, 128), down_proj_bias=torch.zeros(2, 256)),
    dict(ep_degree=2),
])
def test_moe_cte_unsupported_options(kw):
    gu, dn = _experts()
    base = dict(hidden_states=torch.zeros(4, 256, dtype=torch.bfloat16),
                expert_affinities_masked=torch.zeros(8, 1), gate_up_proj_weight=gu,
                down_proj_weight=dn, token_position_to_id=torch.zeros(512, dtype=torch.int32),
                block_to_expert=torch.zeros(2, dtype=torch.int32), block_size=256,
                implementation=M.MoECTEImplementation.shard_on_block)
    base.update(kw)
    with pytest.raises(NotImplementedError):
        M.moe_cte(**base)


def test_moe_cte_mx_arguments():
    """MX requested with weights that are not in an MX layout is an argument error; the
    reference's Trainium-tiled uint16 MX layout is refused as unsupported."""
    gu, dn = _experts()
    base = dict(hidden_states=torch.zeros(4, 256, dtype=torch.bfloat16),
                expert_affinities_masked=torch.zeros(8, 1), gate_up_proj_weight=gu,
                down_proj_weight=dn, token_position_to_id=torch.zeros(512, dtype=torch.int32),
                block_to_expert=torch.zeros(2, dtype=torch.int32), block_size=256,
                implementation=M.MoECTEImplementation.shard_on_block_mx)
    with pytest.raises(ValueError):
        M.moe_cte(**base)
    tiled = dict(base, gate_up_proj_weight=torch.zeros(2, 128, 2, 1, 128, dtype=torch.uint16),
                 down_proj_weight=torch.zeros(2, 8, 1, 256, dtype=torch.uint16),
                 gate_up_proj_scale=torch.zeros(2, 16, 2, 1, 128, dtype=torch.uint8),
                 down_proj_scale=torch.zeros(2, 1, 1, 256, dtype=torch.uint8))
    with pytest.raises(NotImplementedError, match="uint16"):
        M.moe_cte(**tiled)


def test_moe_cte_rejects_unquantized_experts():
    with pytest.raises(NotImplementedError, match="float8_e4m3fn"):
        M.moe_cte(torch.zeros(4, 256), torch.zeros(8, 1), torch.zeros(2, 256, 2, 128),
                  torch.zeros(2, 128, 256), torch.zeros(512, dtype=torch.int32),
                  torch.zeros(2, dtype=torch.int32), 256, M.MoECTEImplementation.shard_on_block)


def test_blockwise_mapping_arguments():
    aff = torch.zeros(4, 8)
    with pytest.raises(NotImplementedError):
        M.build_blockwise_mapping(aff, 8, 2, 256, tp_degree=2)
    with pytest.raises(ValueError):
        M.build_blockwise_mapping(aff, 6, 2, 256)


def test_moe_block_tkg_unsupported_options():
    gu, dn = _experts()
    x = torch.zeros(4, 256, dtype=torch.bfloat16)
    g = torch.ones(256)
    wr = torch.zeros(256, 2, dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError, match="placeholders"):
        M.moe_block_tkg(x, g, wr, gu, dn, hidden_act_scale_factor=1.0)
    with pytest.raises(NotImplementedError):   # fused residual add on float32 input
        M.moe_block_tkg(x.float(), g, wr, gu, dn, residual=x.float())
    with pytest.raises(NotImplementedError):
        M.moe_block_tkg(x, g, wr, gu, dn, hidden_act_fn=M.ActFnType.Swish)
    with pytest.raises(NotImplementedError):   # 2 local experts of 4 routed
        M.moe_block_tkg(x, g, torch.zeros(256, 4, dtype=torch.bfloat16), gu, dn)


def test_converted_weight_cache_follows_its_sources():
    """The reference-layout conversion is cached per source tensor; when the source is
    freed the entry goes with it, so new weights of the same shape (possibly at the same
    address) are converted afresh instead of hitting another tensor's entry."""
    import gc

    from vllm_neuron_amd.functional.moe import _experts
    _experts._CACHE.clear()
    E, H, I = 2, 256, 128

    def make(seed):
        gg = torch.Generator().manual_seed(seed)
        gu = (torch.randn(E, H, 2, I, generator=gg) * 20).to(FP8)
        dn = (torch.randn(E, I, H, generator=gg) * 20).to(FP8)
        return gu, dn

    for seed in range(4):
        gu, dn = make(seed)
        w13, _, w2, _, c13, c2 = _experts.routed_weights(gu, dn)
        assert c13 is None and c2 is None
        ref13 = gu.view(torch.uint8).permute(0, 2, 3, 1).reshape(E, 2 * I, H)
        assert torch.equal(w13.view(torch.uint8), ref13)
        assert torch.equal(w2.view(torch.uint8), dn.view(torch.uint8).transpose(1, 2))
        assert len(_experts._CACHE) == 1
        # a second call with the same live tensors is a cache hit
        assert _experts.routed_weights(gu, dn)[0] is w13
        del gu, dn, w13, w2
        gc.collect()
        assert len(_experts._CACHE) == 0


def _nf_weights(E=2, H=256, I=128, seed=0):
    g = torch.Generator().manual_seed(seed)
    gu = torch.randn(E, H, 2 * I, generator=g).to(FP8)   # a parameter stored [E, H, 2I]
    dn = torch.randn(E, I, H, generator=g).to(FP8)
    return gu, dn


def test_operator_layout_cache_hits_fresh_views_of_one_parameter():
    """The reference's decode passes a fresh `.reshape` view of each expert parameter
    on every call (model_bf16.py:1278). The re-layout to the kernels' stacking runs
    once for all of them: the cache follows the storage, not the view object."""
    from vllm_neuron_amd.functional.moe import _experts
    gu, dn = _nf_weights()
    E, H, I2 = gu.shape
    before = _experts.BUILDS[0]
    outs = [_experts.routed_weights(gu.reshape(E, H, 2, I2 // 2), dn.reshape(E, I2 // 2, H))
            for _ in range(3)]
    assert _experts.BUILDS[0] == before + 1
    assert all(o[0] is outs[0][0] and o[2] is outs[0][2] for o in outs)
    ref = gu.reshape(E, H, 2, I2 // 2).permute(0, 2, 3, 1).reshape(E, I2, H)
    assert torch.equal(outs[0][0].view(torch.uint8), ref.contiguous().view(torch.uint8))
    # an in-place write through the parameter (a weight reload) bumps the shared
    # version counter: the next call rebuilds
    gu.view(torch.uint8)[0, 0, 0] ^= 1
    _experts.routed_weights(gu.reshape(E, H, 2, I2 // 2), dn.reshape(E, I2 // 2, H))
    assert _experts.BUILDS[0] == before + 2


def test_operator_layout_cache_drops_freed_weights():
    """A freed weight's entry goes with its storage owner, so a tensor allocated later
    (possibly at the same address) is converted afresh, never served stale bytes."""
    import gc
    from vllm_neuron_amd.functional.moe import _experts
    gu, dn = _nf_weights(seed=1)
    E, H, I2 = gu.shape
    a = _experts.routed_weights(gu.reshape(E, H, 2, I2 // 2), dn.reshape(E, I2 // 2, H))[0].clone()
    n = len(_experts._CACHE)
    del gu, dn
    gc.collect()
    assert len(_experts._CACHE) == n - 1
    before = _experts.BUILDS[0]
    gu2, dn2 = _nf_weights(seed=2)
    b = _experts.routed_weights(gu2.reshape(E, H, 2, I2 // 2), dn2.reshape(E, I2 // 2, H))[0]
    assert _experts.BUILDS[0] == before + 1
    assert not torch.equal(a.view(torch.uint8), b.view(torch.uint8))


def test_reference_fp8_channel_scale_formats():
    """The reference's FP8 per-channel weight scales (moe_cte [E, 1, 2I] / [E, 1, H],
    moe_cte.py:178-188; moe_tkg row [E, 2, I] / [E, H] and static [E, 2, 1] / [E, 1],
    moe_tkg.py:87-91) become unit 128x128 block scales plus fp32 channel scales [E, 2I]
    (gate channels, then up) and [E, H]; mixing block and channel scales is refused."""
    from vllm_neuron_amd.functional.moe import _experts
    E, H, I = 3, 256, 128
    g = torch.Generator().manual_seed(5)
    gu = torch.randn(E, H, 2, I, generator=g).to(FP8)
    dn = torch.randn(E, I, H, generator=g).to(FP8)
    s_gu = torch.rand(E, 2, I, generator=g) + 0.5
    s_dn = torch.rand(E, H, generator=g) + 0.5
    for gs, ds in ((s_gu.reshape(E, 1, 2 * I), s_dn.reshape(E, 1, H)), (s_gu, s_dn)):
        w13, s13, w2, s2, c13, c2 = _experts.routed_weights(gu, dn, gs, ds)
        assert torch.all(s13 == 1) and tuple(s13.shape) == (E, 2 * I // 128, H // 128)
        assert torch.all(s2 == 1) and tuple(s2.shape) == (E, H // 128, I // 128)
        assert torch.equal(c13, s_gu.reshape(E, 2 * I)) and torch.equal(c2, s_dn)
        assert torch.equal(c13[:, :I], s_gu[:, 0]) and torch.equal(c13[:, I:], s_gu[:, 1])
    st_gu, st_dn = torch.tensor([[[2.0], [3.0]]]).repeat(E, 1, 1), torch.full((E, 1), 0.25)
    *_, c13, c2 = _experts.routed_weights(gu, dn, st_gu, st_dn)
    assert torch.all(c13[:, :I] == 2) and torch.all(c13[:, I:] == 3) and torch.all(c2 == 0.25)
    # stacked layout with channel scales, and a missing down scale meaning 1
    w13s = gu.permute(0, 2, 3, 1).reshape(E, 2 * I, H).contiguous()
    *_, c13, c2 = _experts.routed_weights(w13s, dn.transpose(1, 2).contiguous(), s_gu, None)
    assert torch.equal(c13, s_gu.reshape(E, 2 * I)) and torch.all(c2 == 1)
    with pytest.raises(NotImplementedError, match="mix"):
        _experts.routed_weights(gu, dn, torch.ones(E, H // 128, 2, I // 128), s_dn)
    with pytest.raises(NotImplementedError):
        _experts.routed_weights(gu, dn, torch.ones(E, 3, I), s_dn)
