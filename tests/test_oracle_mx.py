"""Pins of the MX oracle (oracle/mx.py) without a GPU: every E2M1 code and E8M0 byte
against the torch dtypes and HF transformers' MXFP4 table, the packed dequantizer
against transformers' own GPT-OSS dequantizer, the OCP MXFP8 quantizer by its
defining properties, and the expert MLP's Swish / clamp / bias / +1 conventions
against GPT-OSS's published formula."""
import numpy as np
import pytest
import torch

from oracle import mx as OX
from oracle.fp8 import e4m3fn_decode


def test_fp4_codes_match_hf_table_and_closed_form():
    from transformers.integrations.mxfp4 import FP4_VALUES
    codes = np.arange(16, dtype=np.uint8)
    got = OX.fp4_decode(codes)
    assert np.array_equal(got, np.asarray(FP4_VALUES, np.float32))
    assert np.array_equal(np.signbit(got), codes >= 8)  # -0.0 keeps its sign
    assert np.array_equal(got, OX.FP4_VALUES)


def test_e8m0_bytes_match_torch():
    b = np.arange(256, dtype=np.uint8)
    got = OX.e8m0_decode(b)
    ref = torch.from_numpy(b.copy()).view(torch.float8_e8m0fnu).to(torch.float32).numpy()
    assert np.array_equal(got[:255], ref[:255]) and np.isnan(got[255]) and np.isnan(ref[255])
    assert got[127] == 1.0 and got[128] == 2.0 and got[0] == np.float32(2.0 ** -127)


def test_mxfp4_dequant_matches_transformers():
    """oracle.mx.dequant_mxfp4 on HF-packed blocks equals transformers'
    convert_moe_packed_tensors (the HF GPT-OSS dequantizer), element for element."""
    from transformers.integrations.mxfp4 import convert_moe_packed_tensors
    rng = np.random.default_rng(3)
    E, R, G = 2, 6, 4
    blocks = rng.integers(0, 256, (E, R, G, 16), dtype=np.uint8)
    scales = rng.integers(100, 150, (E, R, G), dtype=np.uint8)
    ref = convert_moe_packed_tensors(torch.from_numpy(blocks), torch.from_numpy(scales),
                                     dtype=torch.float32).numpy()       # [E, G*32, R]
    for e in range(E):
        got = OX.dequant_mxfp4(blocks[e].reshape(R, G * 16), scales[e])  # [R, G*32]
        assert np.array_equal(got, ref[e].T)


def test_from_hf_gpt_oss_deinterleaves_and_offsets_up_bias():
    rng = np.random.default_rng(4)
    E, I, H = 2, 64, 64
    gub = rng.integers(0, 256, (E, 2 * I, H // 32, 16), dtype=np.uint8)
    gus = rng.integers(120, 135, (E, 2 * I, H // 32), dtype=np.uint8)
    gb = rng.standard_normal((E, 2 * I)).astype(np.float32)
    db = rng.integers(0, 256, (E, H, I // 32, 16), dtype=np.uint8)
    ds = rng.integers(120, 135, (E, H, I // 32), dtype=np.uint8)
    dbias = rng.standard_normal((E, H)).astype(np.float32)
    w13, s13, b13, w2, s2, b2 = OX.from_hf_gpt_oss(gub, gus, gb, db, ds, dbias)
    full = OX.dequant_mxfp4(gub[0].reshape(2 * I, -1), gus[0])
    mine = OX.dequant_mxfp4(w13[0], s13[0])
    assert np.array_equal(mine[:I], full[0::2]) and np.array_equal(mine[I:], full[1::2])
    assert np.array_equal(b13[:, :I], gb[:, 0::2]) and np.array_equal(b13[:, I:], gb[:, 1::2] + 1)
    assert np.array_equal(OX.dequant_mxfp4(w2[1], s2[1]),
                          OX.dequant_mxfp4(db[1].reshape(H, -1), ds[1]))


def test_product_weight_loader_matches_oracle_layout():
    """vllm_neuron_amd.weights_mx.from_hf_gpt_oss (the product's loader, torch) gives the
    oracle's stacked layout, padded with zeros."""
    from vllm_neuron_amd.weights_mx import from_hf_gpt_oss
    rng = np.random.default_rng(5)
    E, I, H = 2, 64, 96
    t = lambda a: torch.from_numpy(a)
    gub = rng.integers(0, 256, (E, 2 * I, H // 32, 16), dtype=np.uint8)
    gus = rng.integers(120, 135, (E, 2 * I, H // 32), dtype=np.uint8)
    gb = rng.standard_normal((E, 2 * I)).astype(np.float32)
    db = rng.integers(0, 256, (E, H, I // 32, 16), dtype=np.uint8)
    ds = rng.integers(120, 135, (E, H, I // 32), dtype=np.uint8)
    dbias = rng.standard_normal((E, H)).astype(np.float32)
    rw = torch.randn(E, H).to(torch.bfloat16)
    w = from_hf_gpt_oss(t(gub), t(gus), t(gb), t(db), t(ds), t(dbias), rw, hidden=256,
                        intermediate=128)
    ow13, os13, ob13, ow2, os2, ob2 = OX.from_hf_gpt_oss(gub, gus, gb, db, ds, dbias)
    assert np.array_equal(w.w13[:, :I, :H // 2].numpy(), ow13[:, :I])
    assert np.array_equal(w.w13[:, 128:128 + I, :H // 2].numpy(), ow13[:, I:])
    assert np.array_equal(w.w13_scale[:, :I, :H // 32].numpy(), os13[:, :I])
    assert np.array_equal(w.b13[:, 128:128 + I].numpy(), ob13[:, I:])
    assert np.all(w.w13[:, I:128].numpy() == 0) and np.all(w.b13[:, I:128].numpy() == 0)
    assert np.array_equal(w.w2[:, :H, :I // 2].numpy(), ow2)
    assert np.all(w.w2[:, H:].numpy() == 0) and np.all(w.b2[:, H:].numpy() == 0)


def test_product_mx_weight_quantizer_is_ocp():
    """weights_mx.quant_mx_weight: scale byte = floor(log2 amax) - emax + 127, the
    block maximum lands in [emax range) and every element is the nearest code (ties
    to the even code)."""
    from vllm_neuron_amd.weights_mx import quant_fp4_codes, quant_mx_weight
    levels = torch.tensor([0.0, 0.25, 0.5, 0.75, 1.0, 1.25, 1.75, 2.5, 3.5, 5.0, 6.0, 7.0, -0.25, -5.0])
    codes = quant_fp4_codes(levels).numpy()
    assert OX.fp4_decode(codes).tolist() == [0.0, 0.0, 0.5, 1.0, 1.0, 1.0, 2.0, 2.0, 4.0, 4.0, 6.0,
                                              6.0, -0.0, -4.0]
    g = torch.Generator().manual_seed(0)
    w = torch.randn(8, 256, generator=g) * torch.exp2(torch.randint(-10, 10, (8, 1), generator=g).float())
    q, s = quant_mx_weight(w, "fp4")
    deq = OX.dequant_mxfp4(q.numpy(), s.numpy())
    blk = w.numpy().reshape(8, 8, 32)
    e = np.floor(np.log2(np.abs(blk).max(-1))) - 2
    assert np.array_equal(s.numpy().astype(np.int64), (e + 127).astype(np.int64))
    # nearest representable value per element (brute force over the 16 codes)
    cand = OX.FP4_VALUES[None, None, None, :] * np.exp2(e)[:, :, None, None]
    best = np.abs(blk[..., None] - cand).min(-1)
    assert np.allclose(np.abs(deq.reshape(8, 8, 32) - blk), best, rtol=0, atol=1e-12)


def test_mxfp8_quantizer_properties():
    rng = np.random.default_rng(6)
    x = (rng.standard_normal((5, 96)) * np.exp2(rng.integers(-30, 30, (5, 1)))).astype(np.float32)
    x[2, :32] = 0.0
    q, s = OX.quant_mxfp8(x)
    blk = x.reshape(5, 3, 32)
    amax = np.abs(blk).max(-1)
    with np.errstate(divide="ignore"):
        e = np.where(amax > 0, np.frexp(amax)[1] - 1 - 8, -127)   # floor(log2 amax) - 8
    assert np.array_equal(s.astype(np.int64), np.maximum(e, -127) + 127)
    assert s[2, 0] == 0 and np.all(q.reshape(5, 3, 32)[2, 0] == 0)
    # element codes: torch's e4m3fn cast of the clamped, power-of-two scaled values
    scaled = np.clip(blk / np.exp2(np.maximum(e, -127))[..., None], -448, 448).astype(np.float32)
    ref = torch.from_numpy(scaled.reshape(5, 96)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(q, ref)
    # representable inputs round-trip exactly when the block maximum's mantissa is at
    # most 1.75 (it scales to at most 448) ...
    vals = e4m3fn_decode(np.arange(32, dtype=np.uint8)).reshape(1, 32) * np.float32(2.0 ** -5)
    vals[0, -1] = np.float32(1.5 * 2.0 ** -3)
    qq, ss = OX.quant_mxfp8(vals.astype(np.float32))
    assert np.array_equal(OX.dequant_mxfp8(qq, ss), vals)
    # ... and a maximum with mantissa 1.875 saturates to 448 * 2^e (OCP MX v1.0, 6.3)
    sat = np.full((1, 32), np.float32(1.875), np.float32)
    qs, sb = OX.quant_mxfp8(sat)
    assert sb[0, 0] == 127 - 8 and np.all(OX.dequant_mxfp8(qs, sb) == np.float32(448 * 2.0 ** -8))


def test_expert_mlp_mx_conventions():
    """Swish with alpha 1.702 on the clamped gate, times the clamped up projection whose
    bias carries the +1 (limits 1 -+ 7), equals GPT-OSS's published
    (clamp(up, -7, 7) + 1) * gate * sigmoid(1.702 * min(gate, 7)); without clamps and
    with SiLU it is the plain SwiGLU of moe_cte.py:574-575."""
    rng = np.random.default_rng(7)
    T, H, I = 5, 64, 32
    x = rng.standard_normal((T, H)).astype(np.float32) * 3
    w13 = rng.standard_normal((2 * I, H)).astype(np.float32) * 0.5
    w2 = rng.standard_normal((H, I)).astype(np.float32) * 0.1
    bg = rng.standard_normal(I).astype(np.float32)
    bu = rng.standard_normal(I).astype(np.float32)
    b2 = rng.standard_normal(H).astype(np.float32)
    got = OX.expert_mlp_mx(x, w13, np.concatenate([bg, bu + 1]), w2, b2, "swish", (None, 7.0),
                           (-6.0, 8.0), requant_h=False)
    xd = x.astype(np.float64)
    gate = xd @ w13[:I].T + bg
    up = xd @ w13[I:].T + bu
    gate = np.minimum(gate, 7.0)
    up = np.clip(up, -7.0, 7.0)
    glu = gate / (1 + np.exp(-1.702 * gate))
    ref = ((up + 1) * glu) @ w2.T.astype(np.float64) + b2
    assert np.allclose(got, ref, rtol=1e-4, atol=1e-4)
    silu = OX.expert_mlp_mx(x, w13, None, w2, None, "silu", requant_h=False)
    g2 = xd @ w13[:I].T
    ref2 = (g2 / (1 + np.exp(-g2)) * (xd @ w13[I:].T)) @ w2.T.astype(np.float64)
    assert np.allclose(silu, ref2, rtol=1e-4, atol=1e-4)


# ---------------------------------------------------------------- the MX layer composition

def _mx_layer(seed, T=7, H=64, I=64, E=4, K=2):
    """A tiny MX layer: random fp4 codes and E8M0 bytes near 2^0, biases, softmax
    top-K routing weights."""
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((T, H)) * 2).astype(np.float32)
    w13 = rng.integers(0, 256, (E, 2 * I, H // 2), dtype=np.uint8)
    s13 = rng.integers(119, 124, (E, 2 * I, H // 32), dtype=np.uint8)
    w2 = rng.integers(0, 256, (E, H, I // 2), dtype=np.uint8)
    s2 = rng.integers(119, 124, (E, H, I // 32), dtype=np.uint8)
    b13 = rng.standard_normal((E, 2 * I)).astype(np.float32)
    b2 = rng.standard_normal((E, H)).astype(np.float32)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    ids = np.argsort(-lg, axis=1, kind="stable")[:, :K].astype(np.int32)
    w = rng.uniform(0.1, 1.0, (T, K)).astype(np.float32)
    return x, ids, w, w13, s13, b13, w2, s2, b2


def _torch_moe_impl_dense_mx(x, ids, w, w13, s13, b13, w2, s2, b2, act, gl, ul, requant_h):
    """_torch_moe_impl (moe_cte.py:465-612) in float64 over every expert and every
    token, on the dequantized MX operands: gate / up einsums over all E, biases
    (:562-564), clamps (:567-571), act(gate) * up (:574-575), down einsum + down bias
    for every expert (:585-591), then the POST_SCALE sum over e = 0..E-1 with the
    dense affinities (zero for unselected experts, :603-606). requant_h applies the
    MXFP8 quantizer to each intermediate row, the operand the MX down kernel reads."""
    T, H = x.shape
    E, I = w13.shape[0], w13.shape[1] // 2
    xh = OX.dequant_mxfp8(*OX.quant_mxfp8(x)).astype(np.float64)
    W13 = np.stack([OX.dequant_mxfp4(w13[e], s13[e]) for e in range(E)]).astype(np.float64)
    W2 = np.stack([OX.dequant_mxfp4(w2[e], s2[e]) for e in range(E)]).astype(np.float64)
    aff = np.zeros((T, E))
    for t in range(T):
        for j in range(ids.shape[1]):
            aff[t, ids[t, j]] += w[t, j]
    gate = np.einsum("th,eih->eti", xh, W13[:, :I]) + b13[:, None, :I]
    up = np.einsum("th,eih->eti", xh, W13[:, I:]) + b13[:, None, I:]
    lo, hi = gl
    gate = np.clip(gate, -np.inf if lo is None else lo, np.inf if hi is None else hi)
    lo, hi = ul
    up = np.clip(up, -np.inf if lo is None else lo, np.inf if hi is None else hi)
    a = gate / (1 + np.exp(-1.702 * gate)) if act == "swish" else gate / (1 + np.exp(-gate))
    inter = a * up
    if requant_h:
        inter = np.stack([OX.dequant_mxfp8(*OX.quant_mxfp8(inter[e].astype(np.float32)))
                          for e in range(E)]).astype(np.float64)
    nxt = np.einsum("eti,ehi->eth", inter, W2) + b2[:, None, :]
    out = np.zeros((T, H))
    for e in range(E):
        out = out + nxt[e] * aff[:, e:e + 1]
    return out


@pytest.mark.parametrize("act, gl, ul", [("swish", (None, 7.0), (-6.0, 8.0)),
                                         ("silu", (None, None), (None, None))])
@pytest.mark.parametrize("requant_h", [False, True])
def test_moe_sparse_mx_equals_the_dense_reference_form(act, gl, ul, requant_h):
    """The oracle's per-expert gathered MX layer equals the reference fallback's dense
    all-expert form (moe_cte.py:465-612) on the same dequantized operands: the gather,
    the weight of each selected expert, the down bias weighted by the affinity and
    the scatter-add are what this pins."""
    x, ids, w, w13, s13, b13, w2, s2, b2 = _mx_layer(11)
    got = OX.moe_sparse_mx(x, ids, w, w13, s13, b13, w2, s2, b2, act, gl, ul, requant_h=requant_h)
    ref = _torch_moe_impl_dense_mx(x, ids, w, w13, s13, b13, w2, s2, b2, act, gl, ul, requant_h)
    err = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    # fp32 products against float64 (measured 1e-7); a dropped or unweighted bias
    # term moves the output by more than 1e-3
    assert err < 1e-5, err


def test_moe_sparse_mx_float64_loops():
    """Element-by-element loops of the POST_SCALE layer on a 3-token layer (no vector
    routine involved): sum_k w_k * (act(clamp(x.Wg_e + bg_e)) * clamp(x.Wu_e + bu_e)) . Wd_e
    + bd_e)."""
    x, ids, w, w13, s13, b13, w2, s2, b2 = _mx_layer(12, T=3, H=64, I=32, E=3)
    got = OX.moe_sparse_mx(x, ids, w, w13, s13, b13, w2, s2, b2, "swish", (None, 7.0),
                           (-6.0, 8.0), requant_h=False)
    xh = OX.dequant_mxfp8(*OX.quant_mxfp8(x))
    T, H = x.shape
    I = w13.shape[1] // 2
    out = np.zeros((T, H))
    for t in range(T):
        for j in range(ids.shape[1]):
            e = int(ids[t, j])
            W13 = OX.dequant_mxfp4(w13[e], s13[e])
            W2 = OX.dequant_mxfp4(w2[e], s2[e])
            hh = []
            for i in range(I):
                g = sum(float(xh[t, k]) * float(W13[i, k]) for k in range(H)) + float(b13[e, i])
                u = sum(float(xh[t, k]) * float(W13[I + i, k]) for k in range(H)) + float(b13[e, I + i])
                g = min(g, 7.0)
                u = min(max(u, -6.0), 8.0)
                hh.append(g / (1.0 + np.exp(-1.702 * g)) * u)
            for o in range(H):
                yv = sum(hh[i] * float(W2[o, i]) for i in range(I)) + float(b2[e, o])
                out[t, o] += float(w[t, j]) * yv
    assert np.allclose(got, out, rtol=1e-4, atol=1e-4)


def test_moe_sparse_mx_linear_in_routing_weights_and_bias_weighted():
    """Doubling the routing weights doubles the output (the down bias included); with
    all-zero weight codes each token's output is sum_k w_k * b_down[e_k] exactly."""
    x, ids, w, w13, s13, b13, w2, s2, b2 = _mx_layer(13)
    base = OX.moe_sparse_mx(x, ids, w, w13, s13, b13, w2, s2, b2)
    twice = OX.moe_sparse_mx(x, ids, 2 * w, w13, s13, b13, w2, s2, b2)
    assert np.allclose(twice, 2 * base, rtol=1e-6, atol=1e-6)
    zero = OX.moe_sparse_mx(x, ids, w, np.zeros_like(w13), s13, b13, np.zeros_like(w2), s2, b2)
    ref = np.zeros_like(zero)
    for t in range(x.shape[0]):
        for j in range(ids.shape[1]):
            ref[t] = (ref[t] + w[t, j] * b2[ids[t, j]]).astype(np.float32)
    assert np.array_equal(zero, ref)
