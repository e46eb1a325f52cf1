// Router kernels for gfx950: logits GEMM (bf16 MFMA, fp32 accumulate) and the
// per-token top-k selector (one wave per token, wave shuffles for the argmax).
//
// Reference behaviour: vllm_neuron/functional/moe/router.py:384-566 (torch
// fallback orders), moe_block_tkg.py:153-205 (router_pre_norm / norm_topk_prob),
// plus DeepSeek-V3 grouped sigmoid routing with a selection-only correction bias.
#include <type_traits>

#include "mapping.h"

namespace moe {

// Side jobs of the logits launch, for the layer: `zero` (when set) is cleared by
// workgroup 0 before the top-k launch counts workgroups on it, and x is quantized
// (1x128 groups into qq / qs, or MXFP8 32-value blocks with E8M0 scale bytes when
// qmx is set) since the quantization does not depend on the routing and needs no
// launch of its own: by the extra workgroups [qblk0, qblk0 + qnblk)
// (act_quant_vec_body / mx_act_quant_body) in the 64 x 64 form, by the wide form
// as it loads x (1x128 only: qq set, qnblk 0).
// With norm.gamma set (64 x 64 form, T <= kNormRideT) x holds the raw rows: every
// workgroup computes the rows' norm factors and normalizes what it reads, and the
// quantization workgroups also write the residual stream.
struct LogitsSide {
  int* zero;
  const uint16_t* qx;
  long qgroups;  // 1x128 groups, or 8-value chunks (qmx)
  uint8_t* qq;
  void* qs;
  int qblk0, qnblk, qmx;
  NormRide norm;
};

// ---------------------------------------------------------------------------
// The RMSNorm riding in the logits launch, for up to kNormRideT token rows. Each
// workgroup (256 threads) sums the squares of every row itself with
// rms_norm_vec_kernel's steps (the same chunks per thread, butterfly and wave-sum
// order), so the normalized rows are bit-identical to moe_rms_norm_quant's.
// ---------------------------------------------------------------------------
constexpr int kNormRideChunks = kNormRideMaxH / (8 * 256);  // 16-byte chunks per thread and row

// Norm factors of rows [0, T) of x into s_rn (T <= kNormRideT), for the whole
// workgroup (two barriers).
__device__ __forceinline__ void norm_ride_factors(const uint16_t* __restrict__ x, const NormRide& nr,
                                                  int T, int H, float (*s_ws)[4], float* s_rn) {
  const int tid = threadIdx.x, nch = H >> 3;
#pragma unroll
  for (int t = 0; t < kNormRideT; ++t) {
    if (t < T) {  // workgroup-uniform
      int4 xc[kNormRideChunks], rc[kNormRideChunks];
#pragma unroll
      for (int j = 0; j < kNormRideChunks; ++j) {
        const int c = tid + 256 * j;
        if (c < nch) {
          xc[j] = *(const int4*)(x + (size_t)t * H + 8 * c);
          if (nr.res != nullptr) rc[j] = *(const int4*)(nr.res + (size_t)t * H + 8 * c);
        }
      }
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < kNormRideChunks; ++j) {
        const int c = tid + 256 * j;
        if (c < nch) {
          float v[8];
          bf16x8_to_f32(xc[j], v);
          if (nr.res != nullptr) norm_residual8(v, rc[j]);
          ss = norm_sumsq8(ss, v, 8 * c, nr.ha);
        }
      }
      ss = norm_wave_sum(ss);
      if ((tid & 63) == 0) s_ws[t][tid >> 6] = ss;
    }
  }
  __syncthreads();
  if (tid < T) s_rn[tid] = norm_factor(s_ws[tid], nr.ha, nr.eps);
  __syncthreads();
}

// The normalized chunk at element offset off (column col of its row, factor rn) as
// four bf16x2 words; v receives the chunk's row values (bf16(x + residual), or x).
__device__ __forceinline__ int4 norm_ride_chunk(const uint16_t* __restrict__ x, const NormRide& nr,
                                                size_t off, int col, float rn, float (&v)[8]) {
  bf16x8_to_f32(*(const int4*)(x + off), v);
  if (nr.res != nullptr) norm_residual8(v, *(const int4*)(nr.res + off));
  const float4 g0 = *(const float4*)(nr.gamma + col), g1 = *(const float4*)(nr.gamma + col + 4);
  float y[8];
  norm_apply8(v, rn, g0, g1, col, nr.ha, y);
  return make_int4((int)bf16x2(y[0], y[1]), (int)bf16x2(y[2], y[3]), (int)bf16x2(y[4], y[5]),
                   (int)bf16x2(y[6], y[7]));
}

__device__ __forceinline__ void norm_ride_res_out(const NormRide& nr, size_t off, const float (&v)[8]) {
  if (nr.res_out != nullptr)
    *(int4*)(nr.res_out + off) = make_int4((int)bf16x2(v[0], v[1]), (int)bf16x2(v[2], v[3]),
                                           (int)bf16x2(v[4], v[5]), (int)bf16x2(v[6], v[7]));
}

// act_quant_vec_body on the normalized rows (groups = T * H / 128, the same lane
// mapping, one quad per wave at a time), writing the residual stream as it goes.
__device__ __forceinline__ void act_quant_norm_body(const uint16_t* __restrict__ x, const NormRide& nr,
                                                    const float* s_rn, int H, long groups,
                                                    uint8_t* __restrict__ q, float* __restrict__ s,
                                                    int blk, int nblk) {
  const int lane = threadIdx.x & 63, wpb = blockDim.x >> 6, G = H / MOE_GROUP;
  const long quads = (groups + 3) / 4;
  const long nwaves = (long)nblk * wpb;
  for (long q0 = (long)blk * wpb + (threadIdx.x >> 6); q0 < quads; q0 += nwaves) {
    const long gi = 4 * q0 + (lane >> 4);
    if (gi < groups) {  // whole 16-lane segments share gi
      const long row = gi / G;
      const int col = (int)(gi - row * G) * MOE_GROUP + 8 * (lane & 15);
      const size_t off = (size_t)row * H + col;
      float v[8], yb[8];
      const int4 yw = norm_ride_chunk(x, nr, off, col, s_rn[row], v);
      norm_ride_res_out(nr, off, v);
      bf16x8_to_f32(yw, yb);
      quant8_1x128(yb, q + off, s + gi, (lane & 15) == 0);
    }
  }
}

// mx_act_quant_body on the normalized rows (chunks = T * H / 8), writing the
// residual stream as it goes.
__device__ __forceinline__ void mx_act_quant_norm_body(const uint16_t* __restrict__ x, const NormRide& nr,
                                                       const float* s_rn, int H, long chunks,
                                                       uint8_t* __restrict__ q, uint8_t* __restrict__ s,
                                                       int blk, int nblk) {
  const long stride = (long)nblk * blockDim.x;
  const int nch = H >> 3;
  for (long c0 = (long)blk * blockDim.x; c0 < chunks; c0 += stride) {
    const long c = c0 + threadIdx.x;  // whole 4-lane groups share the bound (chunks % 4 == 0)
    float yb[8];
    if (c < chunks) {
      const long row = c / nch;
      const int col = (int)(c - row * nch) * 8;
      float v[8];
      const int4 yw = norm_ride_chunk(x, nr, (size_t)c * 8, col, s_rn[row], v);
      norm_ride_res_out(nr, (size_t)c * 8, v);
      bf16x8_to_f32(yw, yb);
    }
    mx_quant_chunk(yb, c < chunks, c, q, s);
  }
}

// ---------------------------------------------------------------------------
// logits[t, e] = sum_h x[t, h] * w[e, h]   (bf16 operands, fp32 accumulation)
//
// Workgroup tile: 64 tokens x 64 experts, 4 waves; wave w owns experts
// [16w, 16w + 16) for all 64 tokens (4 MFMA row tiles). K advances 256 per
// iteration (four steps of two v_mfma_f32_16x16x32_bf16), in ascending K for
// every accumulator. The x tile goes through LDS (shared by the four waves);
// each wave streams its 16 router rows straight into registers.
// Operand lane layout: lane l holds row l%16 and the 8 K-values
// [s*32 + (l/16)*8, +8) of sub-step s; A and B use the same mapping, so the
// MFMA forms the full 32-long dot product per sub-step.
// K is split into ks chunks; with more than one chunk the kernel writes fp32
// partials [ks, T, E] that router_logits_reduce sums in chunk order.
// ---------------------------------------------------------------------------
// NORM: x holds the raw rows and the norm rides along (side.norm; T <= kNormRideT).
template <bool NORM>
__global__ __launch_bounds__(256) void router_logits_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
    const float* __restrict__ bias, int T, int H, int E, int kchunk, int ks,
    float* __restrict__ out, LogitsSide side) {
  // x tile: 64 rows x 256 columns (four 64-column K steps), rows padded by 8.
  constexpr int KW = 256, LDX = KW + 8;
  __shared__ __attribute__((aligned(16))) uint16_t sx[64][LDX];
  __shared__ float s_ws[kNormRideT][4], s_rn[kNormRideT];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // Tiles (64 tokens x 64 experts x one K chunk) are numbered expert tile fastest,
  // then K chunk, then token tile, and workgroup b takes tile (b % 8) * per + b / 8:
  // each XCD (b % 8) runs a contiguous tile range, so the expert tiles that share
  // an x tile run together on one L2 and x is read from HBM once.
  const int nct = (E + 63) / 64;
  const long total = (long)nct * ((T + 63) / 64) * ks;
  const long per = (total + 7) / 8;
  if (side.qnblk > 0 && (int)blockIdx.x >= side.qblk0) {  // whole workgroup
    if constexpr (NORM) {
      norm_ride_factors(side.qx, side.norm, T, H, s_ws, s_rn);
      if (side.qmx)
        mx_act_quant_norm_body(side.qx, side.norm, s_rn, H, side.qgroups, side.qq, (uint8_t*)side.qs,
                               blockIdx.x - side.qblk0, side.qnblk);
      else
        act_quant_norm_body(side.qx, side.norm, s_rn, H, side.qgroups, side.qq, (float*)side.qs,
                            blockIdx.x - side.qblk0, side.qnblk);
    } else if (side.qmx) {
      mx_act_quant_body(side.qx, side.qgroups, side.qq, (uint8_t*)side.qs, blockIdx.x - side.qblk0,
                        side.qnblk);
    } else {
      act_quant_vec_body(side.qx, side.qgroups, side.qq, (float*)side.qs, blockIdx.x - side.qblk0,
                         side.qnblk);
    }
    return;
  }
  if (side.zero != nullptr && blockIdx.x == 0 && threadIdx.x == 0) *side.zero = 0;
  const long L = (long)(blockIdx.x & 7) * per + (blockIdx.x >> 3);
  if (L >= total) return;  // whole workgroup
  const int ct = (int)(L % nct);
  const long rk = L / nct;
  const int kz = (int)(rk % ks), rt = (int)(rk / ks);
  const int t0 = rt * 64, e0 = ct * 64;
  const int k_begin = kz * kchunk;
  const int k_end = min(H, k_begin + kchunk);
  const int g = lane >> 4, r16 = lane & 15;

  int erow = e0 + wave * 16 + r16;
  const bool erow_ok = erow < E;
  if (!erow_ok) erow = E - 1;
  const uint16_t* wrow = w + (size_t)erow * H;
  // NORM (T <= kNormRideT, so t0 = 0): the rows' norm factors first; then every x-tile
  // chunk below row T is normalized as it is loaded (only chunk 0 of threads tid < 32 T,
  // or 8 T in the 64-column steps; the rest of the tile stays zero).
  if constexpr (NORM) norm_ride_factors(x, side.norm, T, H, s_ws, s_rn);
  // chunk (row, col) of the x tile, row < T: the raw or the normalized bf16 values
  auto x_chunk = [&](int row, int col) -> int4 {
    if constexpr (NORM) {
      float v[8];
      return norm_ride_chunk(x, side.norm, (size_t)row * H + col, col, s_rn[row], v);
    } else {
      return *(const int4*)(x + (size_t)row * H + col);
    }
  };

  v4f acc[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) acc[m] = (v4f){0.f, 0.f, 0.f, 0.f};

  // Main loop: 256 columns per iteration. All of an iteration's global loads
  // (8 x-tile chunks and 8 router fragments per thread) are issued together,
  // so each iteration waits for one memory latency instead of four.
  int k0 = k_begin;
  for (; k0 + KW <= k_end; k0 += KW) {
    int4 xv[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int idx = tid + c * 256, row = idx >> 5, col = (idx & 31) * 8;
      if (NORM) {
        xv[c] = (t0 + row < T) ? x_chunk(t0 + row, k0 + col) : make_int4(0, 0, 0, 0);
      } else {
        const int tr = min(t0 + row, T - 1);  // rows past T load row T-1 and are zeroed
        xv[c] = x_chunk(tr, k0 + col);
        if (t0 + row >= T) xv[c] = make_int4(0, 0, 0, 0);
      }
    }
    v8bf b[4][2];
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int s = 0; s < 2; ++s) b[q][s] = *(const v8bf*)(wrow + k0 + q * 64 + s * 32 + g * 8);
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int idx = tid + c * 256, row = idx >> 5, col = (idx & 31) * 8;
      *(int4*)&sx[row][col] = xv[c];
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          v8bf a = *(const v8bf*)&sx[m * 16 + r16][q * 64 + s * 32 + g * 8];
          acc[m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[q][s], acc[m], 0, 0, 0);
        }
    __syncthreads();
  }
  // Remaining columns, 64 at a time (H is a multiple of 64).
  for (; k0 < k_end; k0 += 64) {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      int idx = tid + c * 256;
      int row = idx >> 3, col = (idx & 7) * 8;
      int4 v = {0, 0, 0, 0};
      if (t0 + row < T) v = x_chunk(t0 + row, k0 + col);
      *(int4*)&sx[row][col] = v;
    }
    v8bf b[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) b[s] = *(const v8bf*)(wrow + k0 + s * 32 + g * 8);
    __syncthreads();
#pragma unroll
    for (int m = 0; m < 4; ++m) {
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        v8bf a = *(const v8bf*)&sx[m * 16 + r16][s * 32 + g * 8];
        acc[m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[s], acc[m], 0, 0, 0);
      }
    }
    __syncthreads();
  }
  // C layout: lane l, register i -> row 4*(l/16)+i of the 16-row tile, column l%16.
  if (!erow_ok) return;
  const int e = e0 + wave * 16 + r16;
  float bv = (bias != nullptr && ks == 1) ? bias[e] : 0.f;
  float* o = out + (size_t)kz * T * E;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      int t = t0 + m * 16 + g * 4 + i;
      if (t < T) o[(size_t)t * E + e] = acc[m][i] + bv;
    }
  }
}

// ---------------------------------------------------------------------------
// Large-T form: one workgroup holds 128 tokens x all E experts, so x is read
// once per (token tile, K chunk) instead of once per 64-expert tile, and the
// router rows once per 128 tokens. E / (16 EF) waves; wave w owns experts
// [16 EF w, +16 EF) for the 128 tokens (8 x EF MFMA tiles). K advances 128 per
// iteration (four 32-long sub-steps) in ascending order for every accumulator;
// same lane layout as router_logits_kernel. Partials [ks, T, E] as there.
// ---------------------------------------------------------------------------
template <int EF>
__global__ __launch_bounds__(1024) void router_logits_wide_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
    const float* __restrict__ bias, int T, int H, int E, int kchunk, int ks,
    float* __restrict__ out, LogitsSide side) {
  constexpr int KW = 128, LDX = KW + 8;
  __shared__ __attribute__((aligned(16))) uint16_t sx[128][LDX];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nthreads = blockDim.x;
  // Tiles numbered token tile fastest within a K chunk; XCD x runs the contiguous
  // range [x per, (x + 1) per), so its workgroups share the K chunk's router rows.
  const int nrt = (T + 127) / 128;
  const long total = (long)nrt * ks;
  const long per = (total + 7) / 8;
  if (side.zero != nullptr && blockIdx.x == 0 && threadIdx.x == 0) *side.zero = 0;
  const long L = (long)(blockIdx.x & 7) * per + (blockIdx.x >> 3);
  if (L >= total) return;  // whole workgroup
  const int kz = (int)(L / nrt), rt = (int)(L % nrt);
  const int t0 = rt * 128;
  const int k_begin = kz * kchunk, k_end = min(H, k_begin + kchunk);
  const int g = lane >> 4, r16 = lane & 15;

  const uint16_t* wrow[EF];
#pragma unroll
  for (int n = 0; n < EF; ++n) wrow[n] = w + (size_t)(wave * 16 * EF + n * 16 + r16) * H;

  v4f acc[8][EF];
#pragma unroll
  for (int m = 0; m < 8; ++m)
#pragma unroll
    for (int n = 0; n < EF; ++n) acc[m][n] = (v4f){0.f, 0.f, 0.f, 0.f};

  for (int k0 = k_begin; k0 < k_end; k0 += KW) {
    // x tile: 128 rows x 128 columns = 2048 16-byte chunks (at least 512 threads).
    int4 xv[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int idx = tid + c * nthreads;
      const int row = idx >> 4, col = (idx & 15) * 8;
      const int tr = min(t0 + row, T - 1);  // rows past T load row T-1 and are zeroed
      xv[c] = (idx < 2048) ? *(const int4*)(x + (size_t)tr * H + k0 + col) : make_int4(0, 0, 0, 0);
      if (t0 + row >= T) xv[c] = make_int4(0, 0, 0, 0);
    }
    if (side.qq != nullptr) {
      // Every x element is loaded once (one token tile per K chunk); the 16 lanes of a
      // row chunk (idx >> 4) hold one 1x128 group, so they quantize it here.
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int idx = tid + c * nthreads, row = idx >> 4, col = (idx & 15) * 8;
        if (idx < 2048 && t0 + row < T) {  // whole 16-lane segments
          float v[8];
          bf16x8_to_f32(xv[c], v);
          const size_t t = (size_t)(t0 + row);
          quant8_1x128(v, side.qq + t * H + k0 + col,
                       (float*)side.qs + t * (H / MOE_GROUP) + k0 / MOE_GROUP, (lane & 15) == 0);
        }
      }
    }
    v8bf b[EF][4];
#pragma unroll
    for (int n = 0; n < EF; ++n)
#pragma unroll
      for (int q = 0; q < 4; ++q) b[n][q] = *(const v8bf*)(wrow[n] + k0 + q * 32 + g * 8);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int idx = tid + c * nthreads;
      if (idx < 2048) *(int4*)&sx[idx >> 4][(idx & 15) * 8] = xv[c];
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        const v8bf a = *(const v8bf*)&sx[m * 16 + r16][q * 32 + g * 8];
#pragma unroll
        for (int n = 0; n < EF; ++n)
          acc[m][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[n][q], acc[m][n], 0, 0, 0);
      }
    __syncthreads();
  }
  float* o = out + (size_t)kz * T * E;
#pragma unroll
  for (int n = 0; n < EF; ++n) {
    const int e = wave * 16 * EF + n * 16 + r16;
    const float bv = (bias != nullptr && ks == 1) ? bias[e] : 0.f;
#pragma unroll
    for (int m = 0; m < 8; ++m)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = t0 + m * 16 + g * 4 + i;
        if (t < T) o[(size_t)t * E + e] = acc[m][n][i] + bv;
      }
  }
}

// Launch plan of the logits product: the wide form for many tokens (E a multiple
// of 16 in [128, 256], one wave per 16 experts; H a multiple of 128), else 64 x 64
// tiles. ks K chunks give at least about 256 wide (or 1024 small) workgroups.
struct RouterPlan {
  bool wide;
  int ef;  // experts per wave / 16 (wide form)
  int ks;
  int kchunk;
};

static RouterPlan router_plan(int T, int H, int E) {
  RouterPlan pl{};
  const int ef = 1;  // waves of 16 experts: 8 to 16 waves (128 registers per lane at 16)
  pl.wide = T >= 2048 && H % 128 == 0 && E % 16 == 0 && E >= 128 && E <= 256;
  if (pl.wide) {
    pl.ef = ef;
    const int nrt = (T + 127) / 128;
    const int ks = std::max(1, std::min((256 + nrt - 1) / nrt, H / 512));
    pl.kchunk = ((H / 128 + ks - 1) / ks) * 128;
  } else {
    const int ks = router_logits_splits(T, H, E);
    pl.kchunk = ((H / 64 + ks - 1) / ks) * 64;
  }
  pl.ks = (H + pl.kchunk - 1) / pl.kchunk;
  return pl;
}

// The logits product into out (ks == 1: the logits with bias) or into the
// partials [ks, T, E].
// Workgroups of the 64 x 64 form (a multiple of 8, for the XCD mapping).
static long logits_blocks(const RouterPlan& pl, int T, int E) {
  const long tiles = (long)((T + 63) / 64) * ((E + 63) / 64) * pl.ks;
  return ((tiles + 7) / 8) * 8;
}

// side.qnblk > 0 only with the 64 x 64 form (qblk0 = logits_blocks); the wide form
// quantizes inline (side.qq set).
static void launch_router_logits(const RouterPlan& pl, const void* x_bf16, const void* w_bf16,
                                 const float* bias, int T, int H, int E, float* out,
                                 hipStream_t st, const LogitsSide& side = LogitsSide{}) {
  if (pl.wide) {
    const long tiles = (long)((T + 127) / 128) * pl.ks;
    const dim3 grid((unsigned)(((tiles + 7) / 8) * 8));
    const dim3 block((unsigned)(64 * (E / (16 * pl.ef))));
#define MOE_WIDE(EFV)                                                                              \
  hipLaunchKernelGGL(router_logits_wide_kernel<EFV>, grid, block, 0, st, (const uint16_t*)x_bf16, \
                     (const uint16_t*)w_bf16, bias, T, H, E, pl.kchunk, pl.ks, out, side)
    MOE_WIDE(1);
#undef MOE_WIDE
  } else {
    const long blocks = logits_blocks(pl, T, E) + std::max(side.qnblk, 0);
    if (side.norm.gamma != nullptr)
      hipLaunchKernelGGL(router_logits_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, st,
                         (const uint16_t*)x_bf16, (const uint16_t*)w_bf16, bias, T, H, E, pl.kchunk,
                         pl.ks, out, side);
    else
      hipLaunchKernelGGL(router_logits_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, st,
                         (const uint16_t*)x_bf16, (const uint16_t*)w_bf16, bias, T, H, E, pl.kchunk,
                         pl.ks, out, side);
  }
}

__global__ void router_logits_reduce(const float* __restrict__ part, const float* __restrict__ bias,
                                     int T, int E, int ksplit, float* __restrict__ out) {
  size_t n = (size_t)T * E;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x) {
    // Sum in split order, eight partial loads in flight at a time.
    float s = 0.f;
    for (int k0 = 0; k0 < ksplit; k0 += 8) {
      float v[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) v[q] = part[(size_t)min(k0 + q, ksplit - 1) * n + i];
#pragma unroll
      for (int q = 0; q < 8; ++q)
        if (k0 + q < ksplit) s += v[q];
    }
    if (bias != nullptr) s += bias[i % E];
    out[i] = s;
  }
}

// ---------------------------------------------------------------------------
// Top-k selector: one wave per token.
//
// Key used for selection:
//   ORDER_TOPK_ACT : the raw logit                                (router.py:411-427)
//   ORDER_ACT_TOPK : softmax -> the raw logit (softmax is strictly increasing),
//                    sigmoid -> sigmoid(logit)                    (router.py:473-494)
//   ORDER_GROUPED  : act(logit) + correction_bias, restricted to the topk_group
//                    groups with the largest sum-of-top-2 keys    (DeepSeek-V3)
// Ties select the lower expert (group) index; ids come out in descending key.
// Weights: ORDER_TOPK_ACT applies the activation to the K selected logits
// (softmax over the K values, or sigmoid); the other orders gather act(logit).
// Optional renorm w / (sum_k w + eps), sums taken k = 0..K-1; then * scale.
// Softmax over all experts sums e = 0..E-1 sequentially (matches the oracle).
// ---------------------------------------------------------------------------
constexpr int kTopkMaxE = 1024;
constexpr int kTopkMaxP = kTopkMaxE / 64;

__device__ __forceinline__ bool better(float v, int i, float v2, int i2) {
  return v > v2 || (v == v2 && i < i2);
}

// DPP lane moves (gfx9 encodings): quad_perm [1,0,3,2], quad_perm [2,3,0,1],
// row_half_mirror, row_mirror, row_bcast:15, row_bcast:31. Lanes a move does
// not write keep `old`, their own value.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(v, v, CTRL, ROW_MASK, 0xF, false);
}
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(dpp_i<CTRL, ROW_MASK>(__float_as_int(v)));
}

// Selection candidates as doubles: u * 1024 + (1023 - e), with u an order-preserving
// u32 image of the key (negative keys inverted, the sign bit set on the rest; -0 taken
// as +0, which better() treats as equal) and the expert e < 1024, is an integer below
// 2^42, so exact, and a larger value is exactly better() (larger key, then lower
// index): a reduction step is one v_max_f64 (a packed u64 took a 64-bit compare and
// two selects). 0 is "no candidate": NaN keys (never packed), masked experts and lanes
// past E (u >= 1 for every key that is not NaN).
__device__ __forceinline__ double pack_key_d(float v, int e) {
  uint32_t u = (uint32_t)__float_as_int(v == 0.f ? 0.f : v);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return (double)u * 1024.0 + (double)(1023 - e);
}
__device__ __forceinline__ uint32_t packed_key_u(double p) { return (uint32_t)floor(p * (1.0 / 1024.0)); }
__device__ __forceinline__ int unpack_id_d(double p) {
  return 1023 - (int)(p - (double)packed_key_u(p) * 1024.0);
}
__device__ __forceinline__ float unpack_key_d(double p) {
  const uint32_t o = packed_key_u(p);
  return __int_as_float((int)((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o));
}

// Per-lane bitonic sort of N (a power of two) packed candidates, descending.
template <int N>
__device__ __forceinline__ void sort_desc_d(double (&a)[N]) {
#pragma unroll
  for (int k = 2; k <= N; k <<= 1)
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1)
#pragma unroll
      for (int i = 0; i < N; ++i) {
        const int l = i ^ j;
        if (l > i) {
          const double hi = fmax(a[i], a[l]), lo = fmin(a[i], a[l]);
          a[i] = ((i & k) == 0) ? hi : lo;
          a[l] = ((i & k) == 0) ? lo : hi;
        }
      }
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ void max_step_d(double& v) {
  const uint64_t b = (uint64_t)__double_as_longlong(v);
  const uint32_t lo = (uint32_t)dpp_i<CTRL, ROW_MASK>((int)(uint32_t)b);
  const uint32_t hi = (uint32_t)dpp_i<CTRL, ROW_MASK>((int)(uint32_t)(b >> 32));
  v = fmax(v, __longlong_as_double((long long)(((uint64_t)hi << 32) | lo)));
}

// Wave maximum of packed candidates (the same reduction tree), read from lane 63.
__device__ __forceinline__ double wave_max_d(double v) {
  max_step_d<0xB1, 0xF>(v);
  max_step_d<0x4E, 0xF>(v);
  max_step_d<0x141, 0xF>(v);
  max_step_d<0x140, 0xF>(v);
  max_step_d<0x142, 0xA>(v);
  max_step_d<0x143, 0xC>(v);
  const uint64_t b = (uint64_t)__double_as_longlong(v);
  const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)b, 63);
  const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), 63);
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// Value of lane k (k wave-uniform): a scalar read, no LDS round trip.
__device__ __forceinline__ float lane_f32(float v, int k) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), k));
}

// Top-2 values of (t1, t2) pairs under fmaxf/fminf (inputs never NaN).
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ void top2_step(float& t1, float& t2) {
  const float b1 = dpp_f<CTRL, ROW_MASK>(t1), b2 = dpp_f<CTRL, ROW_MASK>(t2);
  const float lo = fminf(t1, b1);
  t1 = fmaxf(t1, b1);
  t2 = fmaxf(lo, fmaxf(t2, b2));
}

// The mapping that the top-k launch ends in (MAP): blockwise_mapping's outputs
// and workspace for the ids the launch selects.
struct MapJob {
  int B, N;
  int32_t *tpid, *b2e, *cond, *counts, *inv;
  MapWs ws;
  TileOut to;
};

template <int PM, bool MAP>
__global__ __launch_bounds__(MAP ? 1024 : 256) void router_topk_kernel(
    const float* __restrict__ logits, const float* __restrict__ corr_bias, int T, int E, int K,
    int order, int scoring, int n_group, int topk_group, int renorm, float eps, float scale,
    int32_t* __restrict__ ids, float* __restrict__ weights, float* __restrict__ aff,
    const float* __restrict__ part, int ksplit, const float* __restrict__ lbias,
    float* __restrict__ logits_out, int tpb, MapJob mj) {
  __shared__ float s_act[4][PM * 64];
  __shared__ float s_key[4][PM * 64];
  // one workgroup (one token) ending in the mapping: its ids also go to LDS
  __shared__ __attribute__((aligned(16))) int s_ids[MAP ? 64 : 4];
  const bool lds_ids = MAP && gridDim.x == 1 && T * K <= 64;  // workgroup-uniform
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t0 = blockIdx.x * tpb, t = t0 + wave;
  const int P = (E + 63) / 64;
  const float NEG_INF = -__builtin_inff();
  const bool need_act = order != MOE_ORDER_TOPK_ACT;
  // With split-K partials the whole workgroup visits every (token, expert) pair
  // to sum them, and a sigmoid activation (selection keys and weights read only
  // the activation, never the raw logit again) is applied right there rather
  // than by the token's single wave.
  const bool pre_act = part != nullptr && need_act && scoring == MOE_SCORING_SIGMOID;

  // The correction bias is loaded first so its latency overlaps the logits' loads.
  float cb[PM];
#pragma unroll
  for (int j = 0; j < PM; ++j) {
    const int e = lane + 64 * j;
    cb[j] = (order == MOE_ORDER_GROUPED && corr_bias != nullptr && j < P && e < E) ? corr_bias[e] : 0.f;
  }

  if (part != nullptr) {
    // Split-K partials [ksplit, T, E] summed by the whole workgroup for its tpb
    // (at most four) tokens, in split order and then + bias, exactly as router_logits_reduce
    // does; the sums are also written to logits_out. A thread owns (token, expert)
    // pairs and keeps up to 32 partial loads in flight, so a single token (decode)
    // costs one memory round trip per pair for up to 32 splits (H / 256 splits up
    // to H = 8192) instead of one per pair of splits. The sums are staged in
    // s_act[token], which each wave reads back for its own token below before it
    // writes activations there.
    const size_t TE = (size_t)T * E;
    const int npairs = min(tpb, T - t0) * E;
    auto finish = [&](int q, float sum) {
      const int tl = q / E, e = q - tl * E;
      const float lgv = (lbias != nullptr) ? sum + lbias[e] : sum;
      if (logits_out != nullptr) logits_out[(size_t)(t0 + tl) * E + e] = lgv;
      s_act[tl][e] = pre_act ? det_sigmoid_f32(lgv) : lgv;
    };
    // Up to 16 splits: Q >= ksplit loads per pair and 32 / Q pairs per thread at a
    // time (32 loads in flight). Pairs past the end reload the last pair.
    auto sum_few = [&](auto qc) {
      constexpr int Q = decltype(qc)::value, PB = 32 / Q;
      for (int q0 = threadIdx.x; q0 < npairs; q0 += PB * (int)blockDim.x) {
        float v[PB][Q];
#pragma unroll
        for (int p = 0; p < PB; ++p) {
          const int q = min(q0 + p * (int)blockDim.x, npairs - 1);
          const int tl = q / E;
          const float* src = part + (size_t)(t0 + tl) * E + (q - tl * E);
#pragma unroll
          for (int u = 0; u < Q; ++u) v[p][u] = src[(size_t)min(u, ksplit - 1) * TE];
        }
#pragma unroll
        for (int p = 0; p < PB; ++p) {
          const int q = q0 + p * (int)blockDim.x;
          if (q < npairs) {
            float sum = 0.f;
#pragma unroll
            for (int u = 0; u < Q; ++u)
              if (u < ksplit) sum += v[p][u];
            finish(q, sum);
          }
        }
      }
    };
    if (ksplit <= 4) {
      sum_few(std::integral_constant<int, 4>{});
    } else if (ksplit <= 8) {
      sum_few(std::integral_constant<int, 8>{});
    } else if (ksplit <= 16) {
      sum_few(std::integral_constant<int, 16>{});
    } else {
      constexpr int Q = 32;  // 32 splits at a time, one pair per thread
      for (int q = threadIdx.x; q < npairs; q += blockDim.x) {
        const int tl = q / E;
        const float* src = part + (size_t)(t0 + tl) * E + (q - tl * E);
        float sum = 0.f;
        for (int k0 = 0; k0 < ksplit; k0 += Q) {
          float v[Q];
#pragma unroll
          for (int u = 0; u < Q; ++u) v[u] = src[(size_t)min(k0 + u, ksplit - 1) * TE];
#pragma unroll
          for (int u = 0; u < Q; ++u)
            if (k0 + u < ksplit) sum += v[u];
        }
        finish(q, sum);
      }
    }
    __syncthreads();
  }
  if (wave < tpb && t < T) {  // wave-uniform: one wave per token
    float lg[PM];
    if (part == nullptr) {
      const float* row = logits + (size_t)t * E;
#pragma unroll
      for (int j = 0; j < PM; ++j) {
        int e = lane + 64 * j;
        lg[j] = (j < P && e < E) ? row[e] : NEG_INF;
      }
    } else if (!pre_act) {
#pragma unroll
      for (int j = 0; j < PM; ++j) {
        int e = lane + 64 * j;
        lg[j] = (j < P && e < E) ? s_act[wave][e] : NEG_INF;
      }
    } else {
#pragma unroll
      for (int j = 0; j < PM; ++j) lg[j] = NEG_INF;  // not read: s_act holds the activations
    }

    if (need_act && !pre_act) {
      if (scoring == MOE_SCORING_SIGMOID) {
#pragma unroll
        for (int j = 0; j < PM; ++j) {
          int e = lane + 64 * j;
          if (j < P && e < E) s_act[wave][e] = det_sigmoid_f32(lg[j]);
        }
      } else {
        float m = NEG_INF;
#pragma unroll
        for (int j = 0; j < PM; ++j) m = fmaxf(m, lg[j]);
        m = wave_max_f32(m);
#pragma unroll
        for (int j = 0; j < PM; ++j) {
          int e = lane + 64 * j;
          if (j < P && e < E) s_act[wave][e] = det_exp_f32(lg[j] - m);
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        float sum = 0.f;
        for (int e = 0; e < E; ++e) sum += s_act[wave][e];
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int j = 0; j < PM; ++j) {
          int e = lane + 64 * j;
          if (j < P && e < E) s_act[wave][e] = s_act[wave][e] / sum;
        }
      }
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");

    // Selection keys (kept in registers, mirrored in LDS for the group scan).
    float key[PM];
    bool valid[PM];
#pragma unroll
    for (int j = 0; j < PM; ++j) {
      int e = lane + 64 * j;
      valid[j] = (j < P && e < E);
      float kv = NEG_INF;
      if (valid[j]) {
        if (order == MOE_ORDER_TOPK_ACT || (order == MOE_ORDER_ACT_TOPK && scoring == MOE_SCORING_SOFTMAX)) {
          kv = lg[j];
        } else if (order == MOE_ORDER_ACT_TOPK) {
          kv = s_act[wave][e];
        } else {
          kv = s_act[wave][e] + cb[j];
        }
        s_key[wave][e] = kv;
      }
      key[j] = kv;
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");

    if (order == MOE_ORDER_GROUPED && n_group > 1 && topk_group < n_group) {
      const int gs = E / n_group;
      float gscore = NEG_INF;
      int gidx = 0x7fffffff;
      if (gs == 32 && P * 64 == E) {
        // Groups of 32: group 2j + lane / 32 is register j of one 32-lane half,
        // so its top 2 is a DPP reduction within the half (lane 31 / 63 gets it).
        // NaN keys count as -inf, as in the sequential scan, which skips them.
#pragma unroll
        for (int j = 0; j < PM; ++j) {
          if (j < P) {
            float t1 = (key[j] == key[j]) ? key[j] : NEG_INF, t2 = NEG_INF;
            top2_step<0xB1, 0xF>(t1, t2);
            top2_step<0x4E, 0xF>(t1, t2);
            top2_step<0x141, 0xF>(t1, t2);
            top2_step<0x140, 0xF>(t1, t2);
            top2_step<0x142, 0xA>(t1, t2);
            const float g_lo = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t1 + t2), 31));
            const float g_hi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t1 + t2), 63));
            if (lane == 2 * j) {
              gscore = g_lo;
              gidx = lane;
            }
            if (lane == 2 * j + 1) {
              gscore = g_hi;
              gidx = lane;
            }
          }
        }
      } else if (lane < n_group) {
        float t1 = NEG_INF, t2 = NEG_INF;
        for (int q = 0; q < gs; ++q) {
          float v = s_key[wave][lane * gs + q];
          if (v > t1) {
            t2 = t1;
            t1 = v;
          } else if (v > t2) {
            t2 = v;
          }
        }
        gscore = (gs == 1) ? t1 : t1 + t2;
        gidx = lane;
      }
      // A NaN group score (+inf + -inf) ranks below every number, -inf included,
      // lower group first: it competes as -inf with its index moved past 63.
      if (gidx < n_group && gscore != gscore) {
        gscore = NEG_INF;
        gidx += 64;
      }
      // Group g (lane g < n_group) is kept when fewer than topk_group groups rank above
      // it under better(): one scan of the n_group scores instead of topk_group rounds
      // of a wave arg-max (the same set: better() is a total order on the groups).
      int above = 0;
      for (int q = 0; q < n_group; ++q) {
        const float sq = lane_f32(gscore, q);
        const int iq = __builtin_amdgcn_readlane(gidx, q);
        above += better(sq, iq, gscore, gidx) ? 1 : 0;
      }
      const uint64_t keep = __ballot(lane < n_group && above < topk_group);
#pragma unroll
      for (int j = 0; j < PM; ++j) {
        int e = lane + 64 * j;
        if (valid[j] && !((keep >> (e / gs)) & 1ull)) valid[j] = false;
      }
    }

    // K rounds; lane k keeps the k-th winner. Each lane sorts its own packed
    // candidates once, so a round is the wave maximum of the lane heads (one u64
    // compare per step), after which the winning lane (the one whose head it is:
    // indices are distinct) drops its head. A NaN key is never a candidate; with
    // no candidate left the round's maximum is 0 and its id is -1.
    double pk[PM];
#pragma unroll
    for (int j = 0; j < PM; ++j)
      pk[j] = (valid[j] && key[j] == key[j]) ? pack_key_d(key[j], lane + 64 * j) : 0.0;
    sort_desc_d<PM>(pk);
    int my_id = -1;
    float my_key = 0.f;
    for (int k = 0; k < K; ++k) {
      const double best = wave_max_d(pk[0]);
      if (pk[0] == best) {  // the winner; lanes with nothing left shift zeros
#pragma unroll
        for (int j = 0; j + 1 < PM; ++j) pk[j] = pk[j + 1];
        pk[PM - 1] = 0.0;
      }
      if (lane == k) {
        my_id = best != 0.0 ? unpack_id_d(best) : -1;
        my_key = best != 0.0 ? unpack_key_d(best) : NEG_INF;
      }
    }

    // Weights for the K selections (lane k holds selection k).
    float wv = 0.f;
    if (order == MOE_ORDER_TOPK_ACT) {
      if (scoring == MOE_SCORING_SOFTMAX) {
        float m0 = lane_f32(my_key, 0);
        float ex = (lane < K) ? det_exp_f32(my_key - m0) : 0.f;
        float sum = 0.f;
        for (int k = 0; k < K; ++k) sum += lane_f32(ex, k);
        wv = ex / sum;
      } else {
        wv = (lane < K) ? det_sigmoid_f32(my_key) : 0.f;
      }
    } else {
      wv = (lane < K && my_id >= 0) ? s_act[wave][my_id] : 0.f;
    }
    if (renorm) {
      float sum = 0.f;
      for (int k = 0; k < K; ++k) sum += lane_f32(wv, k);
      float den = sum + eps;
      wv = wv / den;
    }
    wv = wv * scale;

    if (lane < K) {
      ids[(size_t)t * K + lane] = my_id;
      weights[(size_t)t * K + lane] = wv;
      if (lds_ids) s_ids[t * K + lane] = my_id;
    }
    if (aff != nullptr) {
      // round of each expert's selection (-1: not selected), from the winners
      int taken[PM];
#pragma unroll
      for (int j = 0; j < PM; ++j) taken[j] = -1;
      for (int k = 0; k < K; ++k) {
        const int id = __builtin_amdgcn_readlane(my_id, k);
#pragma unroll
        for (int j = 0; j < PM; ++j)
          if (id >= 0 && lane + 64 * j == id) taken[j] = k;
      }
#pragma unroll
      for (int j = 0; j < PM; ++j) {
        int e = lane + 64 * j;
        int k = taken[j];
        float v = __shfl(wv, k < 0 ? 0 : k, 64);  // all lanes take part in the shuffle
        if (j < P && e < E) aff[(size_t)t * E + e] = (k >= 0) ? v : 0.f;
      }
    }
  }
  if constexpr (MAP) {
    // The last workgroup to finish builds the mapping from every token's ids
    // (the decode form of blockwise_mapping, map_small_body). After the barrier
    // (every wave's stores done) one thread per workgroup releases them at device
    // scope and takes a ticket; the last one acquires every workgroup's ids. One
    // fence per workgroup: a device-scope fence writes back (release) or
    // invalidates (acquire) the whole L2 of its XCD. mj.ws.status[1] was cleared
    // by the logits launch. One token with row tiles: the same outputs from the ids
    // in LDS (map_one_token), with no barrier or scan.
    __shared__ uint32_t s_bm[PM * 64][8];
    __shared__ int s_blk[PM * 64], s_cnt[PM * 64], s_cex[PM * 64], s_tile[PM * 64];
    __shared__ int s_wave[16];
    __shared__ int s_last;
    __syncthreads();
    if (gridDim.x > 1) {  // workgroup-uniform
      if (threadIdx.x == 0) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        const bool last = atomicAdd(mj.ws.status + 1, 1) == (int)gridDim.x - 1;
        if (last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        s_last = last;
      }
      __syncthreads();
      if (!s_last) return;  // whole workgroup
    }
    if (T == 1 && lds_ids && !mj.to.span) {  // workgroup-uniform: one token, row tiles
      map_one_token(s_ids, K, E, mj.B, mj.N, mj.tpid, mj.b2e, mj.cond, mj.counts, mj.inv, mj.ws,
                    mj.to);
      return;
    }
    map_small_body(ids, lds_ids ? s_ids : nullptr, T, K, E, mj.B, mj.N, mj.tpid, mj.b2e, mj.cond,
                   mj.counts, mj.inv, mj.ws, mj.to, s_bm, s_blk, s_cnt, s_cex, s_tile, s_wave);
  }
}

}  // namespace moe

using namespace moe;

extern "C" int moe_router_logits(const void* x_bf16, const void* w_bf16, const float* bias, int T,
                                 int H, int E, float* logits, void* workspace,
                                 size_t workspace_bytes, void* stream) {
  MOE_API_BEGIN("moe_router_logits");
  MOE_CHECK_ARG(x_bf16 && w_bf16 && logits, "null pointer argument");
  MOE_CHECK_ARG(T >= 0 && H > 0 && E > 0, "bad sizes T=%d H=%d E=%d", T, H, E);
  MOE_CHECK_ARG(H % 64 == 0, "H must be a multiple of 64, got %d", H);
  MOE_CHECK_ARG(((uintptr_t)x_bf16 & 15) == 0 && ((uintptr_t)w_bf16 & 15) == 0,
                "x and w must be 16-byte aligned");
  if (T == 0) return MOE_OK;
  hipStream_t st = (hipStream_t)stream;
  const RouterPlan pl = router_plan(T, H, E);
  if (pl.ks == 1) {
    launch_router_logits(pl, x_bf16, w_bf16, bias, T, H, E, logits, st);
  } else {
    size_t need = (size_t)pl.ks * T * E * sizeof(float);
    MOE_CHECK_ARG(workspace != nullptr && workspace_bytes >= need,
                  "workspace too small: need %zu bytes", need);
    float* part = (float*)workspace;
    launch_router_logits(pl, x_bf16, w_bf16, bias, T, H, E, part, st);
    size_t n = (size_t)T * E;
    int blocks = (int)std::min<size_t>((n + 255) / 256, 4096);
    hipLaunchKernelGGL(router_logits_reduce, dim3(blocks), dim3(256), 0, st, part, bias, T, E, pl.ks,
                       logits);
  }
  MOE_API_END();
}

extern "C" size_t moe_router_logits_workspace_bytes(int T, int H, int E) {
  if (T <= 0 || H <= 0 || E <= 0 || H % 64) return 0;
  // Covers both products: the bf16 one (this plan) and the fp32 one (64 x 64 tiles).
  const RouterPlan pl = router_plan(T, H, E);
  int ks32 = router_logits_splits(T, H, E);
  const int kc32 = ((H / 64 + ks32 - 1) / ks32) * 64;
  ks32 = (H + kc32 - 1) / kc32;
  const int ks = std::max(pl.ks > 1 ? pl.ks : 0, ks32 > 1 ? ks32 : 0);
  return (size_t)ks * T * E * sizeof(float);
}

extern "C" int moe_router_topk(const float* logits, const float* corr_bias, int T, int E, int K,
                               int order, int scoring, int n_group, int topk_group, int renorm,
                               float renorm_eps, float routed_scale, int32_t* ids, float* weights,
                               float* affinities, void* stream) {
  MOE_API_BEGIN("moe_router_topk");
  MOE_CHECK_ARG(logits && ids && weights, "null pointer argument");
  MOE_CHECK_ARG(T >= 0 && E > 0 && E <= kTopkMaxE, "E must be in [1, %d], got %d", kTopkMaxE, E);
  MOE_CHECK_ARG(K >= 1 && K <= E && K <= 64, "top_k must be in [1, min(E, 64)], got %d", K);
  MOE_CHECK_ARG(order >= MOE_ORDER_TOPK_ACT && order <= MOE_ORDER_GROUPED, "bad order %d", order);
  MOE_CHECK_ARG(scoring == MOE_SCORING_SOFTMAX || scoring == MOE_SCORING_SIGMOID,
                "bad scoring %d", scoring);
  if (order == MOE_ORDER_GROUPED) {
    MOE_CHECK_ARG(n_group >= 1 && n_group <= 64 && E % n_group == 0,
                  "n_group must divide E and be <= 64 (E=%d, n_group=%d)", E, n_group);
    MOE_CHECK_ARG(topk_group >= 1 && topk_group <= n_group, "bad topk_group %d", topk_group);
    MOE_CHECK_ARG((long)topk_group * (E / n_group) >= K,
                  "topk_group * group size must be >= top_k");
  }
  if (T == 0) return MOE_OK;
  // Registers and LDS sized for the smallest power-of-two count of 64-expert chunks
  // that covers E, so the per-chunk loops unroll without dead iterations.
  const int P = (E + 63) / 64;
#define MOE_TOPK_LAUNCH(PMV)                                                                   \
  hipLaunchKernelGGL((router_topk_kernel<PMV, false>), dim3((T + 3) / 4), dim3(256), 0,            \
                     (hipStream_t)stream, logits, corr_bias, T, E, K, order, scoring, n_group,     \
                     topk_group, renorm, renorm_eps, routed_scale, ids, weights, affinities,       \
                     nullptr, 0, nullptr, nullptr, 4, MapJob{})
  if (P <= 1)
    MOE_TOPK_LAUNCH(1);
  else if (P <= 2)
    MOE_TOPK_LAUNCH(2);
  else if (P <= 4)
    MOE_TOPK_LAUNCH(4);
  else if (P <= 8)
    MOE_TOPK_LAUNCH(8);
  else
    MOE_TOPK_LAUNCH(kTopkMaxP);
#undef MOE_TOPK_LAUNCH
  MOE_API_END();
}

// Router logits and top-k for the layer: with a split-K logits product the top-k
// kernel sums the partials itself (same order and values as router_logits_reduce,
// written to logits), one launch fewer than moe_router_logits + moe_router_topk.
// With `fuse` the logits launch also quantizes x and, for up to 256 tokens and
// 512 experts, the top-k launch ends in the mapping (see RouterFuse).
// Arguments are those of the two entry points, already checked by the caller.
int moe::router_logits_topk(const void* x_bf16, const void* w_bf16, const float* bias, int T, int H,
                            int E, float* logits, void* workspace, size_t workspace_bytes,
                            const float* corr_bias, int K, int order, int scoring, int n_group,
                            int topk_group, int renorm, float renorm_eps, float routed_scale,
                            int32_t* ids, float* weights, void* stream, RouterFuse* fuse) {
  if (fuse != nullptr) fuse->quant_done = fuse->map_done = false;
  const RouterPlan pl = router_plan(T, H, E);
  const int ks = pl.ks;
  const bool separate =
      T == 0 || E > kTopkMaxE ||
      (ks > 1 && (workspace == nullptr || workspace_bytes < (size_t)ks * T * E * sizeof(float)));
  // The norm rides in the logits launch (with the quantization) where that launch can
  // carry it: the 64 x 64 form, at most kNormRideT tokens and kNormRideMaxH columns, the
  // arguments moe_rms_norm_quant accepts. Otherwise moe_rms_norm_quant runs first (and
  // reports bad arguments) and the router reads its rows.
  bool ride = false, quant_by_norm = false;
  if (fuse != nullptr && fuse->norm.gamma != nullptr) {
    const NormRide& nr = fuse->norm;
    auto a16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
    ride = !separate && T <= kNormRideT && !pl.wide && H % MOE_GROUP == 0 && H <= kNormRideMaxH &&
           nr.ha >= 1 && nr.ha <= H && nr.eps >= 0.f && (nr.res == nullptr) == (nr.res_out == nullptr) &&
           a16(x_bf16) && a16(nr.res) && a16(nr.res_out) && a16(nr.gamma) && fuse->xq != nullptr &&
           fuse->xs != nullptr && ((uintptr_t)fuse->xq & 7) == 0;
    if (!ride) {
      const int rc = moe_rms_norm_quant(x_bf16, nr.res, nr.gamma, T, H, nr.ha, nr.eps, fuse->xn,
                                        nr.res_out, fuse->xq, (float*)fuse->xs, stream);
      if (rc != MOE_OK) return rc;
      x_bf16 = fuse->xn;
      quant_by_norm = !fuse->quant_mx;  // its 1x128 codes are the layer's
    }
  }
  if (separate) {
    int rc = moe_router_logits(x_bf16, w_bf16, bias, T, H, E, logits, workspace, workspace_bytes,
                               stream);
    if (rc != MOE_OK) return rc;
    rc = moe_router_topk(logits, corr_bias, T, E, K, order, scoring, n_group, topk_group, renorm,
                         renorm_eps, routed_scale, ids, weights, nullptr, stream);
    if (rc == MOE_OK && fuse != nullptr) fuse->quant_done = quant_by_norm;
    return rc;
  }
  MOE_API_BEGIN("moe_layer_forward (router)");
  // The checks of moe_router_logits and moe_router_topk.
  MOE_CHECK_ARG(x_bf16 && w_bf16 && logits && ids && weights, "null pointer argument");
  MOE_CHECK_ARG(T > 0 && H > 0 && H % 64 == 0 && E > 0, "bad sizes T=%d H=%d E=%d", T, H, E);
  MOE_CHECK_ARG(((uintptr_t)x_bf16 & 15) == 0 && ((uintptr_t)w_bf16 & 15) == 0,
                "x and w must be 16-byte aligned");
  MOE_CHECK_ARG(K >= 1 && K <= E && K <= 64, "top_k must be in [1, min(E, 64)], got %d", K);
  MOE_CHECK_ARG(order >= MOE_ORDER_TOPK_ACT && order <= MOE_ORDER_GROUPED, "bad order %d", order);
  MOE_CHECK_ARG(scoring == MOE_SCORING_SOFTMAX || scoring == MOE_SCORING_SIGMOID,
                "bad scoring %d", scoring);
  if (order == MOE_ORDER_GROUPED) {
    MOE_CHECK_ARG(n_group >= 1 && n_group <= 64 && E % n_group == 0,
                  "n_group must divide E and be <= 64 (E=%d, n_group=%d)", E, n_group);
    MOE_CHECK_ARG(topk_group >= 1 && topk_group <= n_group, "bad topk_group %d", topk_group);
    MOE_CHECK_ARG((long)topk_group * (E / n_group) >= K,
                  "topk_group * group size must be >= top_k");
  }
  hipStream_t st = (hipStream_t)stream;
  const int P = (E + 63) / 64;
  LogitsSide side{};
  MapJob mj{};
  // The mapping in the top-k launch: ids only, one 256-token chunk (the decode form
  // of blockwise_mapping), E <= 512 (the top-k kernel at 1024 threads keeps its
  // per-lane arrays in registers); otherwise the caller runs blockwise_mapping.
  const bool do_map =
      fuse != nullptr && fuse->tpid != nullptr && fuse->b2e != nullptr && fuse->map_ws != nullptr &&
      T <= kChunk && P <= 8 && fuse->B > 0 && fuse->N == moe_num_blocks(T, K, E, fuse->B) &&
      fuse->map_ws_bytes >= map_ws_bytes(T, E) &&
      (fuse->to.tiles == nullptr ||
       (fuse->to.num_tiles && fuse->to.mt > 0 && fuse->to.max_tiles > 0 && fuse->to.n_shared >= 0 &&
        (!fuse->to.span || fuse->to.seg))) &&
      (!fuse->to.compact || (fuse->to.tiles != nullptr && fuse->to.row_shared >= 0));
  if (do_map) {
    mj.B = fuse->B;
    mj.N = fuse->N;
    mj.tpid = fuse->tpid;
    mj.b2e = fuse->b2e;
    mj.cond = fuse->cond;
    mj.counts = fuse->counts;
    mj.inv = fuse->inv;
    mj.ws = carve_map_ws(fuse->map_ws, T, E);
    mj.to = fuse->to;
    side.zero = mj.ws.status + 1;  // the top-k launch's workgroup counter
  }
  // The quantization in the logits launch (codes as moe_act_quant_1x128's, or as
  // moe_act_quant_mx's; the MX form only as extra workgroups of the 64 x 64 form).
  const bool do_quant = fuse != nullptr && fuse->xq != nullptr && fuse->xs != nullptr &&
                        ((uintptr_t)fuse->xq & 7) == 0 && !quant_by_norm &&
                        (fuse->quant_mx ? H % 32 == 0 && !pl.wide : H % MOE_GROUP == 0);
  if (do_quant) {
    side.qq = fuse->xq;
    side.qs = fuse->xs;
    side.qmx = fuse->quant_mx;
    if (ride) side.norm = fuse->norm;  // ride implies do_quant and the 64 x 64 form
    if (!pl.wide) {  // extra workgroups; the wide form quantizes as it loads x
      side.qx = (const uint16_t*)x_bf16;
      if (fuse->quant_mx) {
        const long chunks = (long)T * H / 8;
        side.qgroups = chunks;
        side.qnblk = (int)std::max(1L, std::min<long>((chunks + 255) / 256, 4096));
      } else {
        const long groups = (long)T * (H / MOE_GROUP);
        side.qgroups = groups;
        side.qnblk = (int)std::max(1L, std::min<long>((groups + 15) / 16, 2048));
      }
      side.qblk0 = (int)logits_blocks(pl, T, E);
    }
  }
  float* part = ks > 1 ? (float*)workspace : nullptr;
  launch_router_logits(pl, x_bf16, w_bf16, bias, T, H, E, part ? part : logits, st, side);
  // Split-K: the top-k kernel sums the partials (+ bias) and writes the logits;
  // one split: the logits kernel wrote them with the bias.
  const float* lin = part ? nullptr : logits;
  const float* lbias = part ? bias : nullptr;
  float* lout = part ? logits : nullptr;
  if (do_map) {
    // One token per workgroup up to 64 tokens, so the partial sums of a token take
    // one memory round trip on 1024 threads; at most four tokens per workgroup above.
    const int tpb = T <= 64 ? 1 : (T + 63) / 64;
    const dim3 grid((T + tpb - 1) / tpb);
#define MOE_TOPK_MAP(PMV)                                                                          \
  hipLaunchKernelGGL((router_topk_kernel<PMV, true>), grid, dim3(1024), 0, st, lin, corr_bias, T, E, \
                     K, order, scoring, n_group, topk_group, renorm, renorm_eps, routed_scale, ids,  \
                     weights, nullptr, part, ks, lbias, lout, tpb, mj)
    if (P <= 1)
      MOE_TOPK_MAP(1);
    else if (P <= 2)
      MOE_TOPK_MAP(2);
    else if (P <= 4)
      MOE_TOPK_MAP(4);
    else
      MOE_TOPK_MAP(8);
#undef MOE_TOPK_MAP
  } else {
#define MOE_TOPK_FUSED(PMV)                                                                        \
  hipLaunchKernelGGL((router_topk_kernel<PMV, false>), dim3((T + 3) / 4), dim3(256), 0, st, lin,    \
                     corr_bias, T, E, K, order, scoring, n_group, topk_group, renorm, renorm_eps,   \
                     routed_scale, ids, weights, nullptr, part, ks, lbias, lout, 4, MapJob{})
    if (P <= 1)
      MOE_TOPK_FUSED(1);
    else if (P <= 2)
      MOE_TOPK_FUSED(2);
    else if (P <= 4)
      MOE_TOPK_FUSED(4);
    else if (P <= 8)
      MOE_TOPK_FUSED(8);
    else
      MOE_TOPK_FUSED(kTopkMaxP);
#undef MOE_TOPK_FUSED
  }
  if (fuse != nullptr) {
    fuse->quant_done = do_quant || quant_by_norm;
    fuse->map_done = do_map;
  }
  MOE_API_END();
}
