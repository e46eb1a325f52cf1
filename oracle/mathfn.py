"""Deterministic fp32 exp / sigmoid (oracle; test infrastructure).

Routing ids must be bit-exact between the GPU selector and this oracle, and
sigmoid-scored routing selects on ``sigmoid(logit) + bias``; a one-ulp
difference between two exp implementations can flip a near tie. Both sides
therefore evaluate exp with the same sequence of individually rounded IEEE
fp32 operations (no fused multiply-add):

  Cody-Waite range reduction  n = rint(x * log2(e)),
                              r = (x - n*C1) - n*C2  with C1 = 355/512 exact,
  degree-7 Taylor polynomial  p(r) = 1 + r(1 + r(1/2 + ... + r/5040)) (Horner),
  scaling                     exp(x) = p(r) * 2**n.

The argument is clamped to [-80, 80] so no intermediate is subnormal or
infinite. sigmoid(x) = 1 / (1 + exp(-x)) with an IEEE division.
The reference uses torch.sigmoid / torch.softmax (router.py:569-599);
tests bound this implementation against float64 numpy in ulps.
"""
import numpy as np

F = np.float32
LOG2E = F(1.4426950408889634)
C1 = F(0.693359375)
C2 = F(-2.12194440e-4)
CLAMP = F(80.0)
_COEF = [F(1.0 / 5040.0), F(1.0 / 720.0), F(1.0 / 120.0), F(1.0 / 24.0),
         F(1.0 / 6.0), F(0.5), F(1.0), F(1.0)]


def exp_f32(x):
    x = np.clip(np.asarray(x, dtype=F), -CLAMP, CLAMP).astype(F)
    n = np.rint(x * LOG2E).astype(F)
    r = ((x - n * C1).astype(F) - (n * C2).astype(F)).astype(F)
    p = _COEF[0] * np.ones_like(r)
    for c in _COEF[1:]:
        p = (p * r).astype(F)
        p = (p + c).astype(F)
    return np.ldexp(p, n.astype(np.int32)).astype(F)


def sigmoid_f32(x):
    x = np.asarray(x, dtype=F)
    e = exp_f32(-x)
    return (F(1.0) / (F(1.0) + e).astype(F)).astype(F)
