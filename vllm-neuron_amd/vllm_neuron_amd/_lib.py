"""ctypes binding of ``lib/libmoe_fp8.so`` (the C ABI of include/moe_fp8.h).

The library is loaded on first use. There is no fallback: if the shared object
is missing or the GPU is unavailable, the product entry points raise.
Status codes map onto the exception types the reference raises for the same
conditions (router.py:632-678 ValueError, moe_block_tkg.py:534-565
NotImplementedError, moe_cte.py:300-313 RuntimeError).
"""
import ctypes
import os
import threading

_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libmoe_fp8.so")
ABI_VERSION = 3
NOALLOC_SCRATCH_BYTES = 64 << 20  # MOE_NOALLOC_SCRATCH_BYTES

MOE_OK, MOE_ERR_ARG, MOE_ERR_UNSUPPORTED, MOE_ERR_HIP = 0, -1, -2, -3

_p = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float
_sz = ctypes.c_size_t

# name -> (restype, argtypes); must match include/moe_fp8.h
PROTOTYPES = {
    "moe_abi_version": (_i, []),
    "moe_last_error": (ctypes.c_char_p, []),
    "moe_router_logits_workspace_bytes": (_sz, [_i, _i, _i]),
    "moe_router_logits": (_i, [_p, _p, _p, _i, _i, _i, _p, _p, _sz, _p]),
    "moe_router_logits_f32": (_i, [_p, _p, _i, _p, _i, _i, _i, _p, _p, _sz, _p]),
    "moe_rms_norm": (_i, [_p, _i, _p, _i, _i, _i, _f, _p, _i, _p]),
    "moe_rms_norm_quant": (_i, [_p, _p, _p, _i, _i, _i, _f, _p, _p, _p, _p, _p]),
    "moe_router_topk": (_i, [_p, _p, _i, _i, _i, _i, _i, _i, _i, _i, _f, _f, _p, _p, _p, _p]),
    "moe_num_blocks": (_i, [_i, _i, _i, _i]),
    "moe_mapping_workspace_bytes": (_sz, [_i, _i]),
    "moe_blockwise_mapping": (_i, [_p, _p, _p, _i, _i, _i, _i, _i, _p, _p, _p, _p, _p, _p, _p,
                                   _sz, _p]),
    "moe_mapping_status": (_i, [_p, _p, ctypes.POINTER(ctypes.c_int)]),
    "moe_invert_mapping": (_i, [_p, _p, _i, _i, _i, _i, _p, _p]),
    "moe_act_quant_1x128": (_i, [_p, _i, _i, _p, _p, _p]),
    "moe_max_tiles": (_i, [_i, _i, _i, _i, _i, _i, _i]),
    "moe_build_tiles": (_i, [_p, _p, _i, _i, _i, _i, _i, _i, _p, _i, _p, _p]),
    "moe_expert_gate_up": (_i, [_p, _p, _i, _i, _i, _i, _p, _p, _p, _p, _p, _p, _i, _p, _i, _p, _p,
                                _i, _i, _p, _p, _p]),
    "moe_expert_down": (_i, [_p, _p, _i, _i, _i, _i, _p, _p, _p, _p, _p, _p, _i, _i, _p, _p, _i, _i,
                             _p, _p]),
    "moe_combine": (_i, [_p, _p, _p, _i, _i, _i, _i, _i, _p, _p]),
    "moe_layer_workspace_bytes": (_sz, [_i, _i, _i, _i, _i, _i, _i, _i]),
    "moe_layer_forward": (_i, [_p, _p, _p, _f, _i, _i, _i, _i, _i, _i, _i, _p, _p, _p, _i, _i, _i,
                               _i, _i, _f, _f, _p, _p, _p, _p, _p, _p, _p, _p, _i, _p, _p, _p, _p,
                               _p, _p, _sz, _p]),
    "moe_layer_forward_noalloc": (_i, [_p, _p, _p, _f, _i, _i, _i, _i, _i, _i, _i, _p, _p, _p, _i,
                                       _i, _i, _i, _i, _f, _f, _p, _p, _p, _p, _p, _p, _p, _p, _i,
                                       _p, _p, _p, _p, _p, _p]),
    "moe_max_block_tiles": (_i, [_i, _i, _i, _i, _i, _i]),
    "moe_block_tiles_workspace_bytes": (_sz, [_i, _i]),
    "moe_build_block_tiles": (_i, [_p, _p, _i, _i, _i, _i, _i, _p, _i, _p, _p, _sz, _p]),
    "moe_expert_gate_up_block": (_i, [_p, _p, _i, _i, _i, _i, _p, _p, _p, _p, _p, _p, _i, _p, _i,
                                      _p, _p, _i, _p, _p, _p]),
    "moe_expert_down_block": (_i, [_p, _p, _i, _i, _i, _i, _p, _p, _p, _p, _p, _p, _i, _i, _p, _p,
                                   _i, _p, _p]),
    "moe_act_quant_mx": (_i, [_p, _i, _i, _p, _p, _p]),
    "moe_expert_gate_up_mx": (_i, [_p, _p, _i, _i, _i, _i, _i, _p, _p, _p, _p, _p, _p, _i, _p, _i,
                                   _p, _p, _i, _i, _i, _f, _f, _f, _f, _p, _p, _p]),
    "moe_expert_down_mx": (_i, [_p, _p, _i, _i, _i, _i, _i, _p, _p, _p, _p, _p, _p, _i, _i, _p, _p,
                                _i, _i, _p, _p]),
    "moe_selftest_mfma_mx": (_i, [_p, _p, _p, _p, _i, _p, _p]),
    "moe_layer_forward_mx": (_i, [_p, _p, _p, _f, _i, _i, _i, _i, _i, _i, _p, _p, _i, _i, _i, _f,
                                  _f, _i, _p, _p, _p, _p, _p, _p, _i, _f, _f, _f, _f, _i, _p, _p,
                                  _p, _p, _p, _p, _sz, _p]),
    "moe_selftest_mfma_fp8": (_i, [_p, _p, _p, _i, _p]),
    "moe_selftest_fp8_encode": (_i, [ctypes.c_uint32, ctypes.c_uint32, _p, _i, _p]),
    "moe_selftest_bf16_encode": (_i, [ctypes.c_uint32, ctypes.c_uint32, _p, _i, _p]),
    "moe_selftest_quant_div": (_i, [_i, ctypes.c_uint32, ctypes.c_uint32, _p, _i, _p]),
}

_lock = threading.Lock()
_lib = None


def lib_path():
    return _LIB_PATH


def load():
    """Load the shared library (once) and attach the prototypes."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(_LIB_PATH):
                raise RuntimeError(
                    f"HIP extension not built: {_LIB_PATH} is missing "
                    "(run `python -m vllm_neuron_amd._build`)")
            lib = ctypes.CDLL(_LIB_PATH)
            for name, (res, args) in PROTOTYPES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            if lib.moe_abi_version() != ABI_VERSION:
                raise RuntimeError("libmoe_fp8.so ABI version mismatch")
            _lib = lib
    return _lib


def check(rc):
    if rc == MOE_OK:
        return
    msg = load().moe_last_error().decode(errors="replace")
    if rc == MOE_ERR_ARG:
        raise ValueError(msg)
    if rc == MOE_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    raise RuntimeError(msg)


def call(name, *args):
    check(getattr(load(), name)(*args))


def ptr(t):
    """Device pointer of a tensor (or None for an absent optional argument), as the
    plain integer that the prototypes' c_void_p parameters take."""
    return None if t is None else t.data_ptr()
