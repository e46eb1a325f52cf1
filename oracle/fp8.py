"""OCP float8 e4m3fn codec and the block quantizers (oracle; test infrastructure).

No reference counterpart holds 128x128 block scales on a CPU path; the closest
are the per-channel fp8 / MX scales handed to nkilib (moe_cte.py:178-191,
moe_tkg.py:87-98) and the MX activation quantizer of
rmsnorm_router_topk_tkg.py:288-343. The format restated here is the public
DeepSeek-V3 checkpoint format: e4m3fn codes, fp32 scale per 128x128 weight
block and per 1x128 activation group, scale = amax / 448.
"""
import numpy as np

FP8_MAX = np.float32(448.0)
AMAX_FLOOR = np.float32(1e-10)
GROUP = 128


def e4m3fn_decode(codes):
    """uint8 codes -> float32 values (0x7F/0xFF are NaN; no infinities)."""
    c = np.asarray(codes, dtype=np.uint8).astype(np.int32)
    sign = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = (c & 0x7).astype(np.float64)
    mag = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    out = (sign * mag).astype(np.float32)
    out[(c & 0x7F) == 0x7F] = np.nan
    return out


def e4m3fn_encode(x):
    """float32 -> uint8 e4m3fn codes, round-to-nearest-even.

    Inputs must already be clamped to [-448, 448] (the quantizers below do
    that); the result then equals torch's ``.to(torch.float8_e4m3fn)``.
    """
    x = np.asarray(x, dtype=np.float32)
    if np.any(np.isnan(x)) or np.any(np.abs(x) > FP8_MAX):
        raise ValueError("e4m3fn_encode expects finite inputs clamped to +-448")
    sign = np.signbit(x).astype(np.uint8) << 7
    a = np.abs(x).astype(np.float64)
    code = np.zeros(a.shape, dtype=np.int64)
    sub = a < 2.0 ** -6
    code[sub] = np.rint(a[sub] * 512.0).astype(np.int64)          # 0..8 (8 == min normal)
    nrm = ~sub
    mant, exp = np.frexp(a[nrm])                                  # a = mant * 2**exp, mant in [0.5,1)
    e = exp.astype(np.int64) - 1                                  # a = (2*mant) * 2**e
    q = np.rint((2.0 * mant - 1.0) * 8.0).astype(np.int64)         # 0..8, RNE
    code[nrm] = ((e + 7) << 3) + q                                 # q == 8 carries into exponent
    return (code.astype(np.uint8) | sign).astype(np.uint8)


def quant_act_1x128(x):
    """Per-row, per-128-column activation quantizer.

    x: [R, C] float32 (C % 128 == 0). Returns (codes uint8 [R, C], scales float32 [R, C/128]).
    scale = max(amax, 1e-10) / 448 (fp32); code = RNE_e4m3fn(clamp(x / scale, +-448)).
    """
    x = np.asarray(x, dtype=np.float32)
    R, C = x.shape
    if C % GROUP:
        raise ValueError("columns must be a multiple of 128")
    g = x.reshape(R, C // GROUP, GROUP)
    amax = np.max(np.abs(g), axis=2)
    s = (np.maximum(amax, AMAX_FLOOR) / FP8_MAX).astype(np.float32)
    y = np.clip(g / s[:, :, None], -FP8_MAX, FP8_MAX).astype(np.float32)
    return e4m3fn_encode(y).reshape(R, C), s


def dequant_act_1x128(codes, scales):
    R, C = codes.shape
    v = e4m3fn_decode(codes).reshape(R, C // GROUP, GROUP)
    return (v * scales[:, :, None]).reshape(R, C).astype(np.float32)


def quant_weight_128x128(w):
    """Block quantizer for a weight in HF [out, in] layout (dims multiples of 128).

    Returns (codes uint8 [out, in], scale_inv float32 [out/128, in/128]).
    """
    w = np.asarray(w, dtype=np.float32)
    O, I = w.shape
    if O % GROUP or I % GROUP:
        raise ValueError("weight dims must be multiples of 128")
    b = w.reshape(O // GROUP, GROUP, I // GROUP, GROUP)
    amax = np.max(np.abs(b), axis=(1, 3))
    s = (np.maximum(amax, AMAX_FLOOR) / FP8_MAX).astype(np.float32)
    y = np.clip(b / s[:, None, :, None], -FP8_MAX, FP8_MAX).astype(np.float32)
    return e4m3fn_encode(y).reshape(O, I), s


def dequant_weight_128x128(codes, scale_inv):
    O, I = codes.shape
    v = e4m3fn_decode(codes).reshape(O // GROUP, GROUP, I // GROUP, GROUP)
    return (v * scale_inv[:, None, :, None]).reshape(O, I).astype(np.float32)
