"""Pins the oracle's e4m3fn codec and block quantizers against torch.float8_e4m3fn
(the library routine) and the closed-form properties of the format."""
import numpy as np
import pytest
import torch

from oracle.fp8 import (dequant_act_1x128, dequant_weight_128x128, e4m3fn_decode, e4m3fn_encode,
                        quant_act_1x128, quant_weight_128x128)


def torch_encode(x):
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_decode_all_codes_match_torch():
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = e4m3fn_decode(codes)
    nan = np.isnan(ref)
    assert np.array_equal(nan, np.isnan(got))
    assert np.array_equal(got[~nan], ref[~nan])
    assert got[0x7E] == 448.0 and got[0x01] == 2.0 ** -9 and got[0x08] == 2.0 ** -6


def test_encode_roundtrip_all_finite_codes():
    codes = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], dtype=np.uint8)
    vals = e4m3fn_decode(codes)
    back = e4m3fn_encode(vals)
    # +0 and -0 are distinct codes and both round-trip
    assert np.array_equal(back, codes)


def test_encode_midpoints_round_to_even():
    codes = np.arange(0, 0x7E, dtype=np.uint8)
    v = e4m3fn_decode(codes).astype(np.float64)
    mids = ((v[:-1] + v[1:]) / 2).astype(np.float32)
    got = e4m3fn_encode(mids)
    want = torch_encode(mids)
    assert np.array_equal(got, want)
    # ties go to the even code
    assert np.all(got % 2 == 0)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_encode_random_matches_torch(seed):
    rng = np.random.default_rng(seed)
    x = np.concatenate([rng.normal(0, 100, 20000), rng.normal(0, 1e-2, 20000),
                        rng.uniform(-448, 448, 20000), rng.normal(0, 1e-3, 5000)]).astype(np.float32)
    x = np.clip(x, -448, 448)
    assert np.array_equal(e4m3fn_encode(x), torch_encode(x))


def test_encode_rejects_unclamped():
    with pytest.raises(ValueError):
        e4m3fn_encode(np.array([449.0], np.float32))


def test_act_quant_closed_form():
    rng = np.random.default_rng(3)
    x = rng.normal(0, 1, (7, 384)).astype(np.float32)
    x[0, :128] = 0.0                                  # all-zero group -> floor scale, zero codes
    x[1, 128:256] *= 1e-6
    q, s = quant_act_1x128(x)
    g = x.reshape(7, 3, 128)
    amax = np.abs(g).max(axis=2)
    assert np.array_equal(s, (np.maximum(amax, np.float32(1e-10)) / np.float32(448)).astype(np.float32))
    assert np.all(q[0, :128] == 0)
    # the amax element of every non-zero group maps to +-448 (code 0x7E / 0xFE)
    for r in range(1, 7):
        for j in range(3):
            k = int(np.argmax(np.abs(g[r, j])))
            assert q[r, j * 128 + k] & 0x7F == 0x7E
    # dequantization error: at most half an e4m3 ulp (2^-4 relative for normals,
    # 2^-10 * scale absolute in the subnormal range)
    xh = dequant_act_1x128(q, s)
    err = np.abs(xh - x)
    bound = np.maximum(np.abs(x) * 2.0 ** -4, np.repeat(s, 128, axis=1) * 2.0 ** -10) * 1.0001
    assert np.all(err <= bound)


def test_weight_quant_blocks():
    rng = np.random.default_rng(4)
    w = rng.normal(0, 0.02, (256, 384)).astype(np.float32)
    w[:128, :128] *= 50
    q, s = quant_weight_128x128(w)
    assert s.shape == (2, 3)
    b = w.reshape(2, 128, 3, 128)
    assert np.array_equal(s, (np.abs(b).max(axis=(1, 3)) / np.float32(448)).astype(np.float32))
    wh = dequant_weight_128x128(q, s)
    bound = np.maximum(np.abs(w) * 2.0 ** -4, np.repeat(np.repeat(s, 128, 0), 128, 1) * 2.0 ** -10) * 1.0001
    assert np.all(np.abs(wh - w) <= bound)
    # agrees with the torch quantizer used to build synthetic checkpoints
    from vllm_neuron_amd.weights import quant_weight_blocks
    tq, ts = quant_weight_blocks(torch.from_numpy(w))
    assert np.array_equal(tq.view(torch.uint8).numpy(), q)
    assert np.array_equal(ts.numpy(), s)


def test_bf16_round_matches_torch_bfloat16_cast():
    """oracle.moe.bf16_round equals torch's float32 -> bfloat16 cast (round to nearest
    even) on every exponent, on halfway cases of both parities, and on signed zeros and
    subnormals."""
    import torch

    from oracle.moe import bf16_round
    rng = np.random.default_rng(5)
    u = rng.integers(0, 2 ** 32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    exp_all = ((np.arange(256, dtype=np.uint32) << 23)[:, None] | np.arange(0, 1 << 16, 97, dtype=np.uint32)[None, :]).reshape(-1)
    halfway = (rng.integers(0, 2 ** 16, size=4096, dtype=np.uint64).astype(np.uint32) << 16) | 0x8000
    special = np.array([0, 0x80000000, 1, 0x8000, 0x7F7FFFFF, 0x00800000, 0x3F808000, 0x3F818000],
                       dtype=np.uint32)
    bits = np.concatenate([u, exp_all, exp_all | 0x80000000, halfway, special])
    x = bits.view(np.float32)
    x = x[np.isfinite(x) & (np.abs(x.astype(np.float64)) < 3.3e38)]  # stay below bf16 overflow
    got = bf16_round(x)
    ref = torch.from_numpy(x.copy()).to(torch.bfloat16).float().numpy()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
