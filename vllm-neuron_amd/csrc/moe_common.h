// Device helpers shared by the FP8-blockwise MoE kernels (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

#define MOE_WAVE 64
#define MOE_GROUP 128  // quantization group along K (weights 128x128, activations 1x128)

// ---------------------------------------------------------------------------
// bf16 <-> fp32
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float(((uint32_t)b) << 16);
}

// Round-to-nearest-even fp32 -> bf16 bits (NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// Two bf16 from the gfx950 conversion instruction (v_cvt_pk_bf16_f32, round to
// nearest even): bf16(a) in bits 0-15, bf16(b) in bits 16-31. Equal to
// f32_to_bf16_bits on every non-NaN fp32 value (and NaN stays NaN), which
// moe_selftest_bf16_encode checks over all 2^32 patterns.
typedef __bf16 moe_bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t bf16x2(float a, float b) {
  const moe_bf16x2_t v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}

// ---------------------------------------------------------------------------
// OCP float8 e4m3fn encode, round-to-nearest-even. The caller clamps the input
// to [-448, 448] first (max finite e4m3fn), so no NaN/overflow path is needed.
// Normal range: keep the fp32 exponent, round the 23-bit mantissa to 3 bits;
// a mantissa carry propagates into the exponent field by the integer add.
// Subnormal range (|x| < 2^-6): code = rint(|x| * 2^9), 0..8 (8 == min normal).
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t f32_to_e4m3fn(float x) {
  uint32_t u = __float_as_uint(x);
  uint32_t sign = (u >> 24) & 0x80u;
  uint32_t a = u & 0x7fffffffu;
  uint32_t code;
  if (a < 0x3c800000u) {                       // |x| < 2^-6
    code = (uint32_t)__builtin_rintf(__uint_as_float(a) * 512.0f);
  } else {
    uint32_t exp = (a >> 23) - 120u;           // (e - 127) + 7
    uint32_t mant = a & 0x7fffffu;
    uint32_t lsb = (mant >> 20) & 1u;
    uint32_t m3 = (mant + 0x7ffffu + lsb) >> 20;  // 0..8
    code = (exp << 3) + m3;
  }
  return code | sign;
}

// Two codes from the gfx950 conversion instruction (v_cvt_pk_fp8_f32: OCP e4m3,
// round to nearest even): code(a) in bits 0-7, code(b) in bits 8-15. For inputs
// in [-448, 448] it equals f32_to_e4m3fn bit for bit, which
// moe_selftest_fp8_encode checks over every fp32 value of that range.
__device__ __forceinline__ uint32_t e4m3x2(float a, float b) {
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false) & 0xffffu;
}

// x / d from rd = 1 / d (itself a correctly rounded IEEE division): q = x * rd
// is within one ulp of x / d, the residual q * d - x is exact under a fused
// multiply-add while it does not underflow, and one correction step then gives
// the correctly rounded quotient (Markstein's theorem); zeros keep the sign of x.
// Three instructions instead of a full division per element when many elements
// share one divisor. For the quantizers' divisors (at least 1e-10 / 448) every
// quotient of magnitude 2^-10 or more, the only ones with a nonzero e4m3 code, is
// correctly rounded; moe_selftest_quant_div checks this, and equal codes, on every
// (bf16 value, bf16 group amax) pair of the 1x128 quantizer and on random fp32
// pairs.
__device__ __forceinline__ float div_by(float x, float d, float rd) {
  const float q = x * rd;
  const float r = __builtin_fmaf(q, d, -x);
  return __builtin_fmaf(-r, rd, q);
}

// ---------------------------------------------------------------------------
// Deterministic fp32 exp / sigmoid built from individually rounded IEEE ops
// (no contraction), so the host oracle reproduces them bit for bit:
// Cody-Waite reduction with C1 = 355/512 (exact), degree-7 Taylor (Horner),
// scale by 2^n. Argument clamped to [-80, 80] (no subnormal intermediates); a NaN
// argument returns NaN, as the oracle's clip does (fmaxf would turn it into -80,
// and a NaN logit into a sigmoid key of 1).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float det_exp_f32(float x) {
#pragma clang fp contract(off)
  if (x != x) return x;
  x = fminf(fmaxf(x, -80.0f), 80.0f);
  float n = __builtin_rintf(x * 0x1.715476p+0f);          // log2(e)
  float r = (x - n * 0x1.63p-1f) - n * -0x1.bd0106p-13f;  // ln2 = C1 + C2, C1 = 355/512
  float p = 0x1.a01a02p-13f;                               // 1/5040
  p = p * r + 0x1.6c16c2p-10f;                             // 1/720
  p = p * r + 0x1.111112p-7f;                              // 1/120
  p = p * r + 0x1.555556p-5f;                              // 1/24
  p = p * r + 0x1.555556p-3f;                              // 1/6
  p = p * r + 0.5f;
  p = p * r + 1.0f;
  p = p * r + 1.0f;
  return __builtin_ldexpf(p, (int)n);
}

__device__ __forceinline__ float det_sigmoid_f32(float x) {
#pragma clang fp contract(off)
  float e = det_exp_f32(-x);
  return 1.0f / (1.0f + e);
}

// s_waitcnt vmcnt(N), other counters untouched (gfx9 encoding: vmcnt[3:0] | [15:14]).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

// Direct-to-LDS loads (global_load_lds_dwordx4 / _dword): lane l's 16 (4) bytes
// from g land at lds_wave_base + 16 l (4 l); completion is counted by vmcnt.
typedef __attribute__((address_space(3))) void* lds_ptr_t;

__device__ __forceinline__ void load_lds16(const void* g, uint8_t* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(g, (lds_ptr_t)lds_wave_base, 16, 0, 0);
}

// The same with the non-temporal hint (nt): for data read once per call, such as
// expert weights streamed at decode. It keeps the stream from displacing reused
// lines (activation rows, scales) in L2 and the MALL, and raised the decode GEMMs'
// weight stream from 6.2 to 6.7 TB/s (a plain read probe: 6.1-6.4 TB/s without the
// hint, 6.6 with it).
__device__ __forceinline__ void load_lds16_nt(const void* g, uint8_t* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(g, (lds_ptr_t)lds_wave_base, 16, 0, 2);
}

__device__ __forceinline__ void load_lds4(const void* g, uint8_t* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(g, (lds_ptr_t)lds_wave_base, 4, 0, 0);
}

// LDS byte address of a pointer into a __shared__ object.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  typedef __attribute__((address_space(3))) const uint8_t* lds_cptr;
  return (uint32_t)(uintptr_t)(lds_cptr)p;
}

// Logical 16-byte chunk c of row r lives at chunk c ^ ((r >> 1) & 7): any 16
// consecutive rows read at one logical chunk touch 16 distinct 16-byte bank
// groups of the 64-bank LDS (two 128-byte rows span the banks once).
__device__ __forceinline__ int swz(int row, int chunk) { return chunk ^ ((row >> 1) & 7); }

// Workgroup barrier that waits only for this wave's LDS operations (lgkmcnt).
// __syncthreads() also drains vmcnt: it waits for every global load in flight,
// prefetches included. Direct-to-LDS data needs its own explicit vmcnt wait.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt/expcnt untouched
  __builtin_amdgcn_s_barrier();
}

// ---------------------------------------------------------------------------
// Wave reductions (wave64).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_max_f32(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, MOE_WAVE));
  return v;
}

// Reduction across the 16 lanes that share lane/16 (one MFMA output row group).
__device__ __forceinline__ float group16_max_f32(float v) {
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, MOE_WAVE));
  return v;
}

// One 1x128 activation quantization group by one wave: lane l holds columns 2l,
// 2l + 1 (`pair`, two bf16 bit patterns) and writes their codes to q + 2l; lane 0
// writes the scale. s = max(amax, 1e-10) / 448 and q = RNE_e4m3fn(clamp(x / s,
// +-448)), both correctly rounded fp32 divisions, so codes and scales match the oracle bit
// for bit.
__device__ __forceinline__ void quant_pair_1x128(uint32_t pair, uint8_t* q, float* s, int lane) {
  const float v0 = bf16_bits_to_f32((uint16_t)(pair & 0xffffu));
  const float v1 = bf16_bits_to_f32((uint16_t)(pair >> 16));
  const float amax = wave_max_f32(fmaxf(fabsf(v0), fabsf(v1)));
  const float sc = fmaxf(amax, 0x1.b7cdfep-34f) / 448.0f;
  const float rs = 1.0f / sc;
  const float y0 = fminf(fmaxf(div_by(v0, sc, rs), -448.0f), 448.0f);
  const float y1 = fminf(fmaxf(div_by(v1, sc, rs), -448.0f), 448.0f);
  *(uint16_t*)(q + 2 * lane) = (uint16_t)e4m3x2(y0, y1);
  if (lane == 0) *s = sc;
}

// One 1x128 group held by 16 consecutive lanes (a 16-aligned lane segment): each
// lane holds 8 consecutive values v (bf16 values widened to fp32) and writes their
// codes as 8 bytes at q; the segment's first lane writes the scale. Same arithmetic
// as quant_pair_1x128 (exact amax, correctly rounded divisions), so the codes are identical.
__device__ __forceinline__ void quant8_1x128(const float (&v)[8], uint8_t* q, float* s, bool first) {
  float a = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) a = fmaxf(a, fabsf(v[e]));
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) a = fmaxf(a, __shfl_xor(a, o, MOE_WAVE));
  const float sc = fmaxf(a, 0x1.b7cdfep-34f) / 448.0f;
  float y[8];
  const float rs = 1.0f / sc;
#pragma unroll
  for (int e = 0; e < 8; ++e) y[e] = fminf(fmaxf(div_by(v[e], sc, rs), -448.0f), 448.0f);
  const uint32_t lo = e4m3x2(y[0], y[1]) | (e4m3x2(y[2], y[3]) << 16);
  const uint32_t hi = e4m3x2(y[4], y[5]) | (e4m3x2(y[6], y[7]) << 16);
  *(uint2*)q = make_uint2(lo, hi);
  if (first) *s = sc;
}

// Widen 8 bf16 values (one 16-byte chunk) to fp32.
__device__ __forceinline__ void bf16x8_to_f32(const int4 c, float (&v)[8]) {
  const uint32_t w[4] = {(uint32_t)c.x, (uint32_t)c.y, (uint32_t)c.z, (uint32_t)c.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __uint_as_float(w[i] << 16);
    v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

// ---------------------------------------------------------------------------
// RMSNorm steps shared by every kernel that normalizes rows, so all of them give
// the same bits. A row v (x, or bf16(x + residual)) of H values, ha of them real:
//   rn = 1 / sqrt(sum_{c < ha} v_c^2 / ha + eps),  y_c = (v_c * rn) * gamma_c for
//   c < ha, else 0,
// with the sum of squares taken by a 256-thread workgroup: each thread over its
// 8-value chunks (chunk c = thread + 256 j) in order, a butterfly over the wave,
// then the four wave sums in order.
// ---------------------------------------------------------------------------
// v = bf16(v + r) for one chunk: the next residual stream, rounded to nearest even.
__device__ __forceinline__ void norm_residual8(float (&v)[8], const int4 rc) {
  float r[8];
  bf16x8_to_f32(rc, r);
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = bf16_bits_to_f32(f32_to_bf16_bits(v[e] + r[e]));
}

// The squares of one chunk (columns [col, col + 8)) added to ss, columns from ha on left out.
__device__ __forceinline__ float norm_sumsq8(float ss, const float (&v)[8], int col, int ha) {
#pragma unroll
  for (int e = 0; e < 8; ++e)
    if (col + e < ha) ss += v[e] * v[e];
  return ss;
}

__device__ __forceinline__ float norm_wave_sum(float ss) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
  return ss;
}

// rn from the four wave sums of the row.
__device__ __forceinline__ float norm_factor(const float* wave_sums, int ha, float eps) {
  const float tot = ((wave_sums[0] + wave_sums[1]) + wave_sums[2]) + wave_sums[3];
  return 1.0f / sqrtf(tot / (float)ha + eps);
}

// The normalized values of one chunk in fp32 (before the bf16 rounding); gamma of
// the chunk in g0, g1.
__device__ __forceinline__ void norm_apply8(const float (&v)[8], float rn, const float4 g0,
                                            const float4 g1, int col, int ha, float (&y)[8]) {
  const float gm[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
#pragma unroll
  for (int e = 0; e < 8; ++e) y[e] = (col + e < ha) ? (v[e] * rn) * gm[e] : 0.f;
}

// E8M0 exponent e of an MX block with magnitude maximum amax (OCP MX v1.0 6.3):
// floor(log2(amax)) - 8 (8 = emax of e4m3), at least -127; the scale byte is
// e + 127 and the elements are v * 2^-e (a power of two: exact), clamped to +-448
// and rounded to nearest even. amax = 0 or subnormal gives e = -127.
__device__ __forceinline__ int mx_exponent(float amax) {
  const int ef = (int)((__float_as_uint(amax) >> 23) & 0xffu);
  return max(ef - 135, -127);
}

// 2^-e for e in [-127, 119] (the range mx_exponent returns for finite input).
__device__ __forceinline__ float mx_inv_scale(int e) { return __uint_as_float((uint32_t)(127 - e) << 23); }

__device__ __forceinline__ uint32_t mx_e4m3x2(float a, float b, float f) {
  return e4m3x2(fminf(fmaxf(a * f, -448.0f), 448.0f), fminf(fmaxf(b * f, -448.0f), 448.0f));
}

// MXFP8 codes of chunk c (8 consecutive values v of a 32-value block; lanes 4k ..
// 4k + 3 hold the block's four chunks): the block amax is combined over the 4-lane
// group, which writes 32 codes and one scale byte. Every lane calls it (live: the
// chunk exists; whole 4-lane groups share it).
__device__ __forceinline__ void mx_quant_chunk(const float (&v)[8], bool live, long c,
                                               uint8_t* __restrict__ q, uint8_t* __restrict__ s) {
  float a = 0.f;
  if (live) {
#pragma unroll
    for (int i = 0; i < 8; ++i) a = fmaxf(a, fabsf(v[i]));
  }
  a = fmaxf(a, __shfl_xor(a, 1, MOE_WAVE));
  a = fmaxf(a, __shfl_xor(a, 2, MOE_WAVE));
  if (live) {
    const int ex = mx_exponent(a);
    const float f = mx_inv_scale(ex);
    const uint32_t lo = mx_e4m3x2(v[0], v[1], f) | (mx_e4m3x2(v[2], v[3], f) << 16);
    const uint32_t hi = mx_e4m3x2(v[4], v[5], f) | (mx_e4m3x2(v[6], v[7], f) << 16);
    *(uint2*)(q + c * 8) = make_uint2(lo, hi);
    if ((c & 3) == 0) s[c >> 2] = (uint8_t)(ex + 127);
  }
}

// MXFP8 quantization of `chunks` 8-value chunks of bf16 rows (chunks % 4 == 0) by
// workgroup `blk` of `nblk` equal workgroups: lane q of a 4-lane group holds 8
// consecutive values of one 32-value block (one 16-byte load).
__device__ __forceinline__ void mx_act_quant_body(const uint16_t* __restrict__ x, long chunks,
                                                  uint8_t* __restrict__ q, uint8_t* __restrict__ s,
                                                  int blk, int nblk) {
  const long stride = (long)nblk * blockDim.x;
  for (long c0 = (long)blk * blockDim.x; c0 < chunks; c0 += stride) {
    const long c = c0 + threadIdx.x;  // whole 4-lane groups share the bound (chunks % 4 == 0)
    float v[8];
    if (c < chunks) bf16x8_to_f32(*(const int4*)(x + c * 8), v);
    mx_quant_chunk(v, c < chunks, c, q, s);
  }
}

// 1x128 quantization of `groups` consecutive bf16 groups (x 16-byte aligned, q
// 8-byte aligned) by workgroup `blk` of `nblk` equal workgroups: lane l of a wave
// takes the 16-byte chunk (l & 15) of group 4 * quad + l / 16, so a wave covers
// four groups per load instruction; each wave keeps U quads of loads in flight.
__device__ __forceinline__ void act_quant_vec_body(const uint16_t* __restrict__ x, long groups,
                                                   uint8_t* __restrict__ q, float* __restrict__ s,
                                                   int blk, int nblk) {
  constexpr int U = 4;
  const int lane = threadIdx.x & 63, wpb = blockDim.x >> 6;
  const long quads = (groups + 3) / 4;
  const long nwaves = (long)nblk * wpb;
  for (long q0 = (long)blk * wpb + (threadIdx.x >> 6); q0 < quads; q0 += U * nwaves) {
    int4 c[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const long gi = 4 * (q0 + u * nwaves) + (lane >> 4);
      c[u] = (gi < groups) ? *(const int4*)(x + gi * MOE_GROUP + 8 * (lane & 15)) : make_int4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const long gi = 4 * (q0 + u * nwaves) + (lane >> 4);  // whole 16-lane segments share gi
      if (gi < groups) {
        float v[8];
        bf16x8_to_f32(c[u], v);
        quant8_1x128(v, q + gi * MOE_GROUP + 8 * (lane & 15), s + gi, (lane & 15) == 0);
      }
    }
  }
}

// The same, loading the group from x (bf16, 128 columns).
__device__ __forceinline__ void quant_group_1x128(const uint16_t* x, uint8_t* q, float* s, int lane) {
  quant_pair_1x128(*(const uint32_t*)(x + 2 * lane), q, s, lane);
}
