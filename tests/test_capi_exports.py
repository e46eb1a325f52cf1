"""The C-ABI library loads and exports every function include/moe_fp8.h declares;
host-side validation errors map onto the reference's exception types. No GPU needed:
argument checks run before any HIP call."""
import ctypes
import os
import re

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "moe_fp8.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w]+\s*\*?\s*(moe_\w+)\s*\(", text, flags=re.M)))


def test_header_and_binding_agree():
    from vllm_neuron_amd import _lib
    names = header_functions()
    assert len(names) >= 15
    assert sorted(_lib.PROTOTYPES) == names


def test_library_exports_every_declared_symbol():
    from vllm_neuron_amd import _lib
    lib = _lib.load()
    for name in header_functions():
        assert hasattr(lib, name), name
    assert lib.moe_abi_version() == _lib.ABI_VERSION == 3


def test_block_formula_and_sizes_match_oracle():
    from oracle.blockwise import num_blocks
    from vllm_neuron_amd import _lib
    lib = _lib.load()
    for T, K, E, B in [(64, 2, 8, 256), (64, 8, 256, 256), (8192, 8, 256, 256), (1, 8, 384, 256),
                       (16384, 8, 384, 256), (4096, 8, 160, 256), (5, 1, 6, 1), (3, 4, 2, 7)]:
        assert lib.moe_num_blocks(T, K, E, B) == num_blocks(T, K, E, B)
    assert lib.moe_mapping_workspace_bytes(64, 256) > 0
    # hq / y hold only the routed and shared rows: DeepSeek-V3 decode 64 needs
    # 64 * 8 + 64 rows, about 12 MB in all (the padded slot space would need ~1 GB)
    ws = lib.moe_layer_workspace_bytes(64, 7168, 2048, 256, 8, 1, 256, 0)
    assert 0 < ws < 16 << 20, ws
    assert lib.moe_layer_workspace_bytes(64, 7168, 2048, 256, 8, 1, 256, 1) >= ws + 64 * 7168 * 2
    assert lib.moe_max_tiles(64, 8, 256, 257, 256, 1, 16) >= 64 * 8 // 16


def _splits_small(T, H, E):
    """Split count of the 64 x 64-tile products (bf16 below the wide-tile sizes, and
    always the fp32 product): about 1024 workgroups, at least 256 columns per chunk."""
    base = -(-T // 64) * -(-E // 64)
    ks = max(1, min(-(-1024 // base), max(1, H // 256)))
    kchunk = -(-(H // 64) // ks) * 64
    return -(-H // kchunk)


def _splits_wide(T, H):
    """Split count of the 128-token wide tiles: about 256 workgroups, K chunks of at
    least 512 columns in steps of 128."""
    nrt = -(-T // 128)
    ks = max(1, min(-(-256 // nrt), H // 512))
    kchunk = -(-(H // 128) // ks) * 128
    return -(-H // kchunk)


@pytest.mark.parametrize("T,H,E", [(64, 7168, 256), (8192, 7168, 256), (2048, 7168, 128),
                                   (4096, 5120, 160), (16384, 7168, 384), (2100, 1024, 128)])
def test_router_workspace_covers_both_products(T, H, E):
    """moe_router_logits_workspace_bytes sizes the split-K partials of whichever
    product runs: the bf16 one (wide tiles from 2048 tokens for 128 <= E <= 256) and
    the fp32 one (always 64 x 64 tiles), which share the query."""
    from vllm_neuron_amd import _lib
    lib = _lib.load()
    wide = T >= 2048 and H % 128 == 0 and E % 16 == 0 and 128 <= E <= 256
    ks_bf16 = _splits_wide(T, H) if wide else _splits_small(T, H, E)
    ks_f32 = _splits_small(T, H, E)
    need = max(k for k in (ks_bf16, ks_f32, 0) if k != 1) * T * E * 4
    assert lib.moe_router_logits_workspace_bytes(T, H, E) == need


def test_argument_errors_raise_reference_exception_types():
    from vllm_neuron_amd import _lib
    lib = _lib.load()
    p = ctypes.c_void_p(16)
    # E above the selector's capacity -> ValueError (router.py:632-678 raises ValueError)
    rc = lib.moe_router_topk(p, None, 4, 2048, 2, 0, 0, 1, 1, 0, 0.0, 1.0, p, p, None, None)
    assert rc == _lib.MOE_ERR_ARG
    with pytest.raises(ValueError, match="E must be"):
        _lib.check(rc)
    # unsupported expert count in the mapping -> NotImplementedError
    rc = lib.moe_blockwise_mapping(p, None, None, 4, 2, 4096, 256, lib.moe_num_blocks(4, 2, 4096, 256),
                                   p, p, p, p, None, None, p, 1 << 20, None)
    assert rc == _lib.MOE_ERR_UNSUPPORTED
    with pytest.raises(NotImplementedError):
        _lib.check(rc)
    # wrong N -> ValueError with the formula value in the message
    rc = lib.moe_blockwise_mapping(p, None, None, 64, 8, 256, 256, 7, p, p, p, p, None, None, p,
                                   1 << 20, None)
    assert rc == _lib.MOE_ERR_ARG and b"257" in lib.moe_last_error()
    rc = lib.moe_expert_gate_up(p, p, 4, 100, 256, 4, p, p, None, None, None, None, 0, p, 0, p, p, 1,
                                 16, p, p, None)
    assert rc == _lib.MOE_ERR_ARG and b"multiples of 128" in lib.moe_last_error()
    rc = lib.moe_layer_forward(p, None, None, 1e-6, 0, 4, 7168, 2048, 256, 8, 1, p, None, None, 2,
                               1, 8, 4, 1, 1e-20, 2.5, p, p, p, p, p, p, p, p, 256, p, None, None,
                               None, None, p, 1, None)
    assert rc == _lib.MOE_ERR_ARG and b"workspace too small" in lib.moe_last_error()
    # the residual add lives in the norm: a residual without gamma is refused
    rc = lib.moe_layer_forward(p, p, None, 1e-6, 0, 4, 7168, 2048, 256, 8, 1, p, None, None, 2,
                               1, 8, 4, 1, 1e-20, 2.5, p, p, p, p, p, p, p, p, 256, p, p, None,
                               None, None, p, 1 << 30, None)
    assert rc == _lib.MOE_ERR_ARG and b"residual needs gamma" in lib.moe_last_error()
    # activation operands beyond 32-bit byte offsets are refused by the block kernels
    rc = lib.moe_expert_down_block(p, p, 4, 7168, 2048, 256, p, p, None, None, None, None, 0, 1 << 21,
                                   p, p, 1, p, None)
    assert rc == _lib.MOE_ERR_UNSUPPORTED and b"exceeds 4 GiB" in lib.moe_last_error()
    # MX expert tiles stop at 64 rows: mt = 128 is refused before any launch
    rc = lib.moe_expert_gate_up_mx(p, p, 4, 3072, 3072, 128, 1, p, p, None, None, None, None, 0, p,
                                   0, p, p, 1, 128, 1, ctypes.c_float(float("nan")),
                                   ctypes.c_float(7.0), ctypes.c_float(-6.0), ctypes.c_float(8.0),
                                   p, p, None)
    assert rc == _lib.MOE_ERR_UNSUPPORTED and b"64 rows" in lib.moe_last_error()
    rc = lib.moe_expert_down_mx(p, p, 4, 3072, 3072, 128, 1, p, p, None, None, None, None, 0, 0,
                                p, p, 1, 128, p, None)
    assert rc == _lib.MOE_ERR_UNSUPPORTED and b"64 rows" in lib.moe_last_error()


def test_ops_reject_cpu_tensors():
    import torch
    from vllm_neuron_amd import ops
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        ops.act_quant(torch.zeros(4, 128, dtype=torch.bfloat16))
