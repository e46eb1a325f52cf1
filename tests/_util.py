"""Helpers shared by the GPU parity tests (conversion to the oracle's numpy inputs)."""
import sys

import numpy as np
import torch


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def np_u8(t):
    return t.detach().view(torch.uint8).cpu().numpy() if t.dtype == torch.float8_e4m3fn else t.detach().cpu().numpy()


def np_f32(t):
    return t.detach().float().cpu().numpy()


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def oracle_weights(w, experts=None):
    """numpy views of an Fp8MoEWeights (optionally only some experts, others zero-filled lazily)."""
    if experts is None:
        return (np_u8(w.w13), np_f32(w.w13_scale), np_u8(w.w2), np_f32(w.w2_scale))
    E = w.n_experts
    idx = sorted(experts)
    q13 = {e: np_u8(w.w13[e]) for e in idx}
    s13 = {e: np_f32(w.w13_scale[e]) for e in idx}
    q2 = {e: np_u8(w.w2[e]) for e in idx}
    s2 = {e: np_f32(w.w2_scale[e]) for e in idx}

    class _Sparse:
        def __init__(self, d):
            self.d = d
            self.shape = (E,) + next(iter(d.values())).shape

        def __getitem__(self, e):
            return self.d[e]

    return _Sparse(q13), _Sparse(s13), _Sparse(q2), _Sparse(s2)


def oracle_shared(w):
    """The shared experts' operands for oracle.moe.moe_sparse_fp8: None, one tuple, or a
    list of tuples from two shared experts on."""
    if w.n_shared == 0:
        return None
    sh = [(np_u8(w.shared_w13[j]), np_f32(w.shared_w13_scale[j]), np_u8(w.shared_w2[j]),
           np_f32(w.shared_w2_scale[j])) for j in range(w.n_shared)]
    return sh[0] if w.n_shared == 1 else sh
