"""Bounds the oracle's deterministic exp/sigmoid against float64 numpy (closed form)."""
import numpy as np

from oracle.mathfn import exp_f32, sigmoid_f32


def _ulps(got, want):
    want32 = want.astype(np.float32)
    return np.abs(got.astype(np.float64) - want) / np.spacing(np.abs(want32)).astype(np.float64)


def test_exp_within_2_ulp():
    x = np.linspace(-80, 80, 400001).astype(np.float32)
    assert _ulps(exp_f32(x), np.exp(x.astype(np.float64))).max() <= 2.0


def test_exp_special_points():
    assert exp_f32(np.float32(0.0)) == 1.0
    assert exp_f32(np.float32(1000.0)) == exp_f32(np.float32(80.0))   # clamped, finite
    assert np.isfinite(exp_f32(np.float32(80.0)))


def test_sigmoid_within_3_ulp_and_symmetry():
    x = np.linspace(-60, 60, 200001).astype(np.float32)
    want = 1.0 / (1.0 + np.exp(-x.astype(np.float64)))
    s = sigmoid_f32(x)
    assert _ulps(s, want).max() <= 3.0
    assert sigmoid_f32(np.float32(0.0)) == 0.5
    # sigmoid(x) + sigmoid(-x) == 1 to within rounding
    assert np.max(np.abs(s.astype(np.float64) + sigmoid_f32(-x).astype(np.float64) - 1.0)) < 2e-7
