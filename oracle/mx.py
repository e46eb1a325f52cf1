"""MX (OCP Microscaling) formats and the GPT-OSS expert MLP (oracle; test infrastructure).

The reference runs GPT-OSS experts with MXFP4 weights on its Trainium-3 kernels
(shard_on_block_mx, moe_cte.py:122-130, :178-191; loaders
model/gpt_oss/weight_loaders_mxfp4.py:301-560); those kernels are in the
un-vendored nkilib, and its CPU fallback refuses MX inputs (moe_cte.py:226-228).
The formats are therefore restated from the OCP Microscaling Formats (MX) v1.0
specification, and the layer math from the reference's CPU fallback
_torch_moe_impl (moe_cte.py:440-612):

* FP4 E2M1 element: sign, 2 exponent bits (bias 1), 1 mantissa bit; subnormal at
  exponent 0; values 0, 0.5, 1, 1.5, 2, 3, 4, 6 (OCP MX v1.0, section 5.3.3).
* E8M0 scale: 2^(b - 127), b = 255 is NaN (section 5.4).
* MX block: 32 consecutive elements along the reduction dimension share one scale.
* HF GPT-OSS checkpoint packing (the input of weight_loaders_mxfp4.py:301-365):
  blocks [E, 2I, H/32, 16] uint8, two FP4 codes per byte, the low nibble first;
  gate and up rows interleaved (row 2i gate i, row 2i+1 up i, :336-340).
* MXFP8 (E4M3) activation quantization, OCP section 6.3: shared exponent
  X = 2^(floor(log2(amax)) - 8) (8 = emax of E4M3), elements
  RNE_e4m3(clamp(v / X, +-448)).
* Expert MLP (moe_cte.py:557-606): gate/up projections, + bias (:562-564), gate
  clamped to gate limits, up to up limits (:567-571), act(gate) * up (:574-575) with
  Swish g * sigmoid(1.702 g) (:459-461) or SiLU, down projection + down bias
  (:586-591), POST_SCALE weighted sum in expert order (:603-606).
"""
import numpy as np

from .fp8 import e4m3fn_decode, e4m3fn_encode

F = np.float32
FP4_VALUES = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                       -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0], F)
MX_BLOCK = 32
SWISH_ALPHA = F(1.702)   # moe_cte.py:460


def fp4_decode(codes):
    """uint8 codes in [0, 16) -> float32 (closed form of the E2M1 encoding)."""
    c = np.asarray(codes, np.uint8).astype(np.int32)
    s = np.where(c & 8, -1.0, 1.0)
    e = (c >> 1) & 3
    m = c & 1
    mag = np.where(e == 0, 0.5 * m, (1.0 + 0.5 * m) * np.exp2(e - 1.0))
    return (s * mag).astype(F)


def e8m0_decode(b):
    """uint8 scale bytes -> float32 2^(b - 127) (2^-127 is an fp32 subnormal); 255 is NaN."""
    b = np.asarray(b, np.uint8).astype(np.float64)
    out = np.exp2(b - 127.0)
    out[b == 255] = np.nan
    return out.astype(F)


def unpack_fp4(packed):
    """[..., n] uint8 holding two codes each (low nibble first) -> [..., 2n] codes."""
    p = np.asarray(packed, np.uint8)
    out = np.empty(p.shape[:-1] + (2 * p.shape[-1],), np.uint8)
    out[..., 0::2] = p & 0xF
    out[..., 1::2] = p >> 4
    return out


def pack_fp4(codes):
    c = np.asarray(codes, np.uint8)
    return (c[..., 0::2] | (c[..., 1::2] << 4)).astype(np.uint8)


def dequant_mx(elements, scales):
    """elements [R, K] float32 (already decoded), scales [R, K/32] uint8 -> [R, K] float64."""
    el = np.asarray(elements, np.float64)
    R, K = el.shape
    s = np.exp2(np.asarray(scales, np.float64) - 127.0)
    return (el.reshape(R, K // MX_BLOCK, MX_BLOCK) * s[:, :, None]).reshape(R, K)


def dequant_mxfp4(packed, scales):
    """packed [R, K/2] uint8, scales [R, K/32] uint8 -> [R, K] float32 (exact)."""
    return dequant_mx(fp4_decode(unpack_fp4(packed)), scales).astype(F)


def quant_mxfp8(x):
    """OCP MXFP8 (E4M3) quantization of x [R, K] float32 along K in blocks of 32.

    Returns (codes uint8 [R, K], scale bytes uint8 [R, K/32]). The scale exponent is
    floor(log2(amax)) - 8, clamped to the E8M0 range (amax 0 gives byte 0); the
    elements are x / 2^e, clamped to +-448, rounded to nearest even."""
    x = np.asarray(x, F)
    R, K = x.shape
    if K % MX_BLOCK:
        raise ValueError("K must be a multiple of 32")
    blk = x.reshape(R, K // MX_BLOCK, MX_BLOCK)
    amax = np.abs(blk).max(axis=2)
    efield = (amax.view(np.uint32) >> 23).astype(np.int64)      # 0 for zero / subnormal
    e = np.maximum(efield - 127 - 8, -127)
    scaled = (blk.astype(np.float64) * np.exp2(-e.astype(np.float64))[:, :, None])
    q = e4m3fn_encode(np.clip(scaled, -448.0, 448.0).astype(F))
    return q.reshape(R, K), (e + 127).astype(np.uint8)


def dequant_mxfp8(codes, scales):
    return dequant_mx(e4m3fn_decode(codes), scales).astype(F)


def swish(g):
    g = np.asarray(g, F)
    return (g / (F(1.0) + np.exp(-SWISH_ALPHA * g).astype(F))).astype(F)


def silu(g):
    g = np.asarray(g, F)
    return (g / (F(1.0) + np.exp(-g).astype(F))).astype(F)


def clamp(v, lo, hi):
    if lo is None and hi is None:
        return v
    return np.clip(v, -np.inf if lo is None else lo, np.inf if hi is None else hi).astype(F)


def expert_mlp_mx(xhat, w13hat, b13, w2hat, b2, act="swish", gate_limits=(None, None),
                  up_limits=(None, None), requant_h=True):
    """One expert on dequantized operands (moe_cte.py:557-591): gate/up = x W^T + bias,
    clamps, h = act(gate) * up, h requantized to MXFP8 along I (the operand the down
    kernel consumes), y = h W_d^T + b_d. w13hat [2I, H] gate rows first; b13 [2I]."""
    I = w13hat.shape[0] // 2
    gu = (np.asarray(xhat, F) @ np.asarray(w13hat, F).T).astype(F)
    if b13 is not None:
        gu = (gu + np.asarray(b13, F)[None, :]).astype(F)
    g = clamp(gu[:, :I], *gate_limits)
    u = clamp(gu[:, I:], *up_limits)
    a = swish(g) if act == "swish" else silu(g)
    h = (a * u).astype(F)
    if requant_h:
        h = dequant_mxfp8(*quant_mxfp8(h))
    y = (h @ np.asarray(w2hat, F).T).astype(F)
    if b2 is not None:
        y = (y + np.asarray(b2, F)[None, :]).astype(F)
    return y


def moe_sparse_mx(x, ids, w, w13_packed, w13_scale, b13, w2_packed, w2_scale, b2,
                  act="swish", gate_limits=(None, None), up_limits=(None, None), experts=None,
                  requant_h=True):
    """Layer output (fp32, before the final cast) with MXFP4 experts and MXFP8
    activations: x [T, H] float32 holding bf16 values; ids / w [T, K]; w13_packed
    [E, 2I, H/2] (gate rows, then up rows), w13_scale [E, 2I, H/32]; w2_packed
    [E, H, I/2], w2_scale [E, H, I/32]; biases [E, 2I] / [E, H] or None. POST_SCALE
    sum per token in expert order (moe_cte.py:603-606): the down bias is part of each
    expert's output and so is weighted by its affinity (:590-591)."""
    x = np.asarray(x, F)
    T, H = x.shape
    xhat = dequant_mxfp8(*quant_mxfp8(x))
    out = np.zeros((T, H), F)
    ids = np.asarray(ids)
    E = w13_packed.shape[0]
    for e in (range(E) if experts is None else sorted(experts)):
        sel = ids == e
        rows = np.nonzero(sel.any(axis=1))[0]
        if rows.size == 0:
            continue
        wt = (np.asarray(w, F) * sel).sum(axis=1)[rows].astype(F)
        y = expert_mlp_mx(xhat[rows], dequant_mxfp4(w13_packed[e], w13_scale[e]),
                          None if b13 is None else b13[e],
                          dequant_mxfp4(w2_packed[e], w2_scale[e]),
                          None if b2 is None else b2[e], act, gate_limits, up_limits, requant_h)
        out[rows] = (out[rows] + y * wt[:, None]).astype(F)
    return out


def from_hf_gpt_oss(gate_up_blocks, gate_up_scales, gate_up_bias, down_blocks, down_scales,
                    down_bias, up_bias_offset=1.0):
    """HF GPT-OSS expert tensors -> the stacked MX layout used here.

    gate_up_blocks [E, 2I, H/32, 16] (rows interleaved gate, up), gate_up_scales
    [E, 2I, H/32], gate_up_bias [E, 2I]; down_blocks [E, H, I/32, 16], down_scales
    [E, H, I/32], down_bias [E, H]. Returns (w13 [E, 2I, H/2], s13 [E, 2I, H/32], b13
    [E, 2I], w2 [E, H, I/2], s2 [E, H, I/32], b2 [E, H]) with gate rows first; the
    up bias gets up_bias_offset added, as the reference's loaders do
    (weight_loaders_bf16.py:386-419, weight_loaders_mxfp4.py:418-464)."""
    gub = np.asarray(gate_up_blocks)
    E, I2, HB, _ = gub.shape
    w13 = np.concatenate([gub[:, 0::2], gub[:, 1::2]], axis=1).reshape(E, I2, HB * 16)
    gus = np.asarray(gate_up_scales)
    s13 = np.concatenate([gus[:, 0::2], gus[:, 1::2]], axis=1)
    gb = np.asarray(gate_up_bias, F)
    b13 = np.concatenate([gb[:, 0::2], gb[:, 1::2] + F(up_bias_offset)], axis=1)
    db = np.asarray(down_blocks)
    w2 = db.reshape(db.shape[0], db.shape[1], -1)
    return w13, s13, b13, w2, np.asarray(down_scales), np.asarray(down_bias, F)
