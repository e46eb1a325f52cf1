// RMSNorm and the fp32-operand router logits GEMM.
//
// RMSNorm follows the two reference forms:
//   router.py:681-688 (_torch_rms_norm): y = (x * rsqrt(mean(x^2) + eps)) * gamma
//   moe_block_tkg.py:135-151: the same over the first hidden_actual columns, the
//   padded columns set to 0, output cast back to the input dtype.
// Both run in fp32; mean = sum / n, rsqrt = 1 / sqrt (IEEE division and square
// root, each correctly rounded).
//
// The fp32 logits GEMM serves router() when its operands are not bf16-exact:
// router.py:236 casts hidden_states to the computation dtype (fp32) before the
// optional RMSNorm, so with gamma (or fp32 inputs) F.linear runs on fp32
// operands (router.py:418-424). It uses v_mfma_f32_16x16x4f32.
#include "moe_common.h"
#include "moe_internal.h"

namespace moe {

__device__ __forceinline__ float ld_act(const void* p, size_t i, int is_f32) {
  return is_f32 ? ((const float*)p)[i] : bf16_bits_to_f32(((const uint16_t*)p)[i]);
}

// One workgroup (256 threads) per row. The sum of squares is reduced in a
// fixed order (per-thread strided sums, then a wave butterfly, then the four
// wave sums in order), so the result is deterministic.
__global__ __launch_bounds__(256) void rms_norm_kernel(const void* __restrict__ x, int x_f32,
                                                       const float* __restrict__ gamma, int H,
                                                       int ha, float eps, void* __restrict__ out,
                                                       int out_f32) {
  __shared__ float s_part[4];
  const size_t row = (size_t)blockIdx.x * H;
  float ss = 0.f;
  for (int c = threadIdx.x; c < ha; c += 256) {
    const float v = ld_act(x, row + c, x_f32);
    ss += v * v;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
  if ((threadIdx.x & 63) == 0) s_part[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float tot = ((s_part[0] + s_part[1]) + s_part[2]) + s_part[3];
  const float r = 1.0f / sqrtf(tot / (float)ha + eps);
  for (int c = threadIdx.x; c < H; c += 256) {
    float y = 0.f;
    if (c < ha) y = (ld_act(x, row + c, x_f32) * r) * gamma[c];
    if (out_f32)
      ((float*)out)[row + c] = y;
    else
      ((uint16_t*)out)[row + c] = f32_to_bf16_bits(y);
  }
}

// Vector RMSNorm for H % 8 == 0: one workgroup per row holds the row in registers
// as 16-byte chunks of 8 values (chunk c = thread + 256 j, j < NJ), so the row is
// read once.
// The sum of squares runs in a fixed order: each thread over its chunks and their 8
// values in order, a wave butterfly, then the four wave sums in order.
// RES: the row is first v = bf16(x + residual) (written to res_out: the next residual
// stream). QUANT (H % 128 == 0): the bf16 normalized row is also quantized 1x128 to
// e4m3fn, one group per 16-lane segment, with act_quant's arithmetic. rms_norm and the
// fused prologue both run this kernel, so the prologue's normalized row is bit-identical
// to moe_rms_norm's and its codes to moe_act_quant_1x128 of that row.
constexpr int kNormMaxChunks = 8;  // H <= 256 * 8 * 8 = 16384
template <bool XF32, bool OF32, bool RES, bool QUANT, int NJ>
__global__ __launch_bounds__(256) void rms_norm_vec_kernel(
    const void* __restrict__ x, const uint16_t* __restrict__ res, const float* __restrict__ gamma,
    int H, int ha, float eps, void* __restrict__ out, uint16_t* __restrict__ res_out,
    uint8_t* __restrict__ q, float* __restrict__ qs) {
  __shared__ float s_part[4];
  const int tid = threadIdx.x, nch = H >> 3;
  const size_t base = (size_t)blockIdx.x * H;
  float v[NJ][8];
  float4 gv[NJ][2];  // gamma, loaded with the row so its latency overlaps
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int c = tid + 256 * j;
    if (c < nch) {
      gv[j][0] = *(const float4*)(gamma + 8 * c);
      gv[j][1] = *(const float4*)(gamma + 8 * c + 4);
      if (XF32) {
        const float4 a = *(const float4*)((const float*)x + base + 8 * c);
        const float4 b = *(const float4*)((const float*)x + base + 8 * c + 4);
        v[j][0] = a.x; v[j][1] = a.y; v[j][2] = a.z; v[j][3] = a.w;
        v[j][4] = b.x; v[j][5] = b.y; v[j][6] = b.z; v[j][7] = b.w;
      } else {
        bf16x8_to_f32(*(const int4*)((const uint16_t*)x + base + 8 * c), v[j]);
      }
      if (RES) norm_residual8(v[j], *(const int4*)(res + base + 8 * c));
      ss = norm_sumsq8(ss, v[j], 8 * c, ha);
    }
  }
  ss = norm_wave_sum(ss);
  if ((tid & 63) == 0) s_part[tid >> 6] = ss;
  __syncthreads();
  const float rn = norm_factor(s_part, ha, eps);
  const int G = H / MOE_GROUP;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int c = tid + 256 * j;
    if (c >= nch) continue;  // whole 16-lane segments leave together when H % 128 == 0
    float y[8];
    norm_apply8(v[j], rn, gv[j][0], gv[j][1], 8 * c, ha, y);
    if (RES) {
      uint32_t w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        w[i] = bf16x2(v[j][2 * i], v[j][2 * i + 1]);
      *(int4*)(res_out + base + 8 * c) = make_int4((int)w[0], (int)w[1], (int)w[2], (int)w[3]);
    }
    if (OF32) {
      *(float4*)((float*)out + base + 8 * c) = make_float4(y[0], y[1], y[2], y[3]);
      *(float4*)((float*)out + base + 8 * c + 4) = make_float4(y[4], y[5], y[6], y[7]);
    } else {
      uint32_t w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        w[i] = bf16x2(y[2 * i], y[2 * i + 1]);
      *(int4*)((uint16_t*)out + base + 8 * c) = make_int4((int)w[0], (int)w[1], (int)w[2], (int)w[3]);
      if (QUANT) {
        float yb[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          yb[2 * i] = __uint_as_float(w[i] << 16);
          yb[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
        }
        quant8_1x128(yb, q + base + 8 * c, qs + (size_t)blockIdx.x * G + (c >> 4), (tid & 15) == 0);
      }
    }
  }
}

// logits[t, e] = sum_h x[t, h] * w[e, h]   (fp32 x; fp32 or bf16 w; fp32 accumulate)
//
// Workgroup tile: 64 tokens x 64 experts, 4 waves; wave w owns experts
// [16w, 16w + 16) for the 64 tokens (4 row tiles). K advances 64 per step in 16
// MFMAs of K = 4. In sub-step s lane l (group g = l/16) supplies K position
// g*16 + s of the step for row / column l%16; A and B use the same mapping, so
// each lane's 16 weight values of a step are contiguous (vector loads) and the
// 16 MFMAs together cover all 64 positions. blockIdx.z splits K as in the bf16
// kernel.
template <typename WT>
__global__ __launch_bounds__(256) void router_logits_f32_kernel(
    const float* __restrict__ x, const WT* __restrict__ w, const float* __restrict__ bias, int T,
    int H, int E, int kchunk, float* __restrict__ out) {
  __shared__ float sx[64][64 + 1];  // +1: rows land on distinct banks
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t0 = blockIdx.x * 64, e0 = blockIdx.y * 64;
  const int k_begin = blockIdx.z * kchunk;
  const int k_end = min(H, k_begin + kchunk);
  const int g = lane >> 4, r16 = lane & 15;

  int erow = e0 + wave * 16 + r16;
  const bool erow_ok = erow < E;
  if (!erow_ok) erow = E - 1;
  const WT* wrow = w + (size_t)erow * H;

  v4f acc[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) acc[m] = (v4f){0.f, 0.f, 0.f, 0.f};

  for (int k0 = k_begin; k0 < k_end; k0 += 64) {
    // x tile: 64 rows x 64 floats = 1024 float4, 4 per thread.
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int idx = threadIdx.x + c * 256;
      const int row = idx >> 4, col = (idx & 15) * 4;
      float4 v = {0.f, 0.f, 0.f, 0.f};
      if (t0 + row < T) v = *(const float4*)(x + (size_t)(t0 + row) * H + k0 + col);
      sx[row][col] = v.x;
      sx[row][col + 1] = v.y;
      sx[row][col + 2] = v.z;
      sx[row][col + 3] = v.w;
    }
    float b[16];
    if constexpr (sizeof(WT) == 4) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 v = *(const float4*)(wrow + k0 + g * 16 + q * 4);
        b[4 * q] = v.x;
        b[4 * q + 1] = v.y;
        b[4 * q + 2] = v.z;
        b[4 * q + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int4 v = *(const int4*)(wrow + k0 + g * 16 + q * 8);
        const uint32_t u[4] = {(uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          b[8 * q + 2 * j] = __uint_as_float(u[j] << 16);
          b[8 * q + 2 * j + 1] = __uint_as_float(u[j] & 0xFFFF0000u);
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < 16; ++s) {
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const float a = sx[m * 16 + r16][g * 16 + s];
        acc[m] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b[s], acc[m], 0, 0, 0);
      }
    }
    __syncthreads();
  }
  // C layout: lane l, register i -> row 4*(l/16)+i of the 16-row tile, column l%16.
  if (!erow_ok) return;
  const int e = e0 + wave * 16 + r16;
  const float bv = (bias != nullptr && gridDim.z == 1) ? bias[e] : 0.f;
  float* o = out + (size_t)blockIdx.z * T * E;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = t0 + m * 16 + g * 4 + i;
      if (t < T) o[(size_t)t * E + e] = acc[m][i] + bv;
    }
  }
}

// Sums the split-K partials in split order (+ bias).
__global__ void router_logits_f32_reduce(const float* __restrict__ part,
                                         const float* __restrict__ bias, int T, int E, int ksplit,
                                         float* __restrict__ out) {
  const size_t n = (size_t)T * E;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x) {
    float s = 0.f;
    for (int k = 0; k < ksplit; ++k) s += part[(size_t)k * n + i];
    if (bias != nullptr) s += bias[i % E];
    out[i] = s;
  }
}

// Launch rms_norm_vec_kernel with the smallest chunk count per thread that covers H.
template <bool XF32, bool OF32, bool RES, bool QUANT>
static void launch_rms_norm_vec(int T, int H, hipStream_t st, const void* x, const uint16_t* res,
                                const float* gamma, int ha, float eps, void* out,
                                uint16_t* res_out, uint8_t* q, float* qs) {
  const int nj = (H / 8 + 255) / 256;
  if (nj <= 1)
    hipLaunchKernelGGL((rms_norm_vec_kernel<XF32, OF32, RES, QUANT, 1>), dim3(T), dim3(256), 0, st, x, res,
                       gamma, H, ha, eps, out, res_out, q, qs);
  else if (nj <= 2)
    hipLaunchKernelGGL((rms_norm_vec_kernel<XF32, OF32, RES, QUANT, 2>), dim3(T), dim3(256), 0, st, x, res,
                       gamma, H, ha, eps, out, res_out, q, qs);
  else if (nj <= 4)
    hipLaunchKernelGGL((rms_norm_vec_kernel<XF32, OF32, RES, QUANT, 4>), dim3(T), dim3(256), 0, st, x, res,
                       gamma, H, ha, eps, out, res_out, q, qs);
  else
    hipLaunchKernelGGL((rms_norm_vec_kernel<XF32, OF32, RES, QUANT, kNormMaxChunks>), dim3(T), dim3(256), 0,
                       st, x, res, gamma, H, ha, eps, out, res_out, q, qs);
}

}  // namespace moe

using namespace moe;

extern "C" int moe_rms_norm(const void* x, int x_is_f32, const float* gamma, int T, int H,
                            int hidden_actual, float eps, void* out, int out_is_f32,
                            void* stream) {
  MOE_API_BEGIN("moe_rms_norm");
  MOE_CHECK_ARG(x && gamma && out, "null pointer argument");
  MOE_CHECK_ARG(T >= 0 && H > 0, "bad sizes T=%d H=%d", T, H);
  MOE_CHECK_ARG(hidden_actual >= 1 && hidden_actual <= H,
                "hidden_actual must be in [1, H=%d], got %d", H, hidden_actual);
  MOE_CHECK_ARG(eps >= 0.f, "eps must be >= 0");
  if (T == 0) return MOE_OK;
  hipStream_t st = (hipStream_t)stream;
  const bool vec = H % 8 == 0 && H <= 256 * 8 * kNormMaxChunks && ((uintptr_t)x & 15) == 0 &&
                   ((uintptr_t)out & 15) == 0 && ((uintptr_t)gamma & 15) == 0;
  if (!vec) {
    hipLaunchKernelGGL(rms_norm_kernel, dim3(T), dim3(256), 0, st, x, x_is_f32 ? 1 : 0, gamma, H,
                       hidden_actual, eps, out, out_is_f32 ? 1 : 0);
  } else if (x_is_f32 && out_is_f32) {
    launch_rms_norm_vec<true, true, false, false>(T, H, st, x, nullptr, gamma, hidden_actual, eps, out, nullptr,
                                                  nullptr, nullptr);
  } else if (x_is_f32) {
    launch_rms_norm_vec<true, false, false, false>(T, H, st, x, nullptr, gamma, hidden_actual, eps, out, nullptr,
                                                  nullptr, nullptr);
  } else if (out_is_f32) {
    launch_rms_norm_vec<false, true, false, false>(T, H, st, x, nullptr, gamma, hidden_actual, eps, out, nullptr,
                                                  nullptr, nullptr);
  } else {
    launch_rms_norm_vec<false, false, false, false>(T, H, st, x, nullptr, gamma, hidden_actual, eps, out, nullptr,
                                                  nullptr, nullptr);
  }
  MOE_API_END();
}

extern "C" int moe_rms_norm_quant(const void* x_bf16, const void* residual_bf16, const float* gamma,
                                  int T, int H, int hidden_actual, float eps, void* xn_bf16,
                                  void* residual_out_bf16, uint8_t* q, float* s, void* stream) {
  MOE_API_BEGIN("moe_rms_norm_quant");
  MOE_CHECK_ARG(x_bf16 && gamma && xn_bf16 && q && s, "null pointer argument");
  MOE_CHECK_ARG((residual_bf16 == nullptr) == (residual_out_bf16 == nullptr),
                "residual and residual_out must be given together");
  MOE_CHECK_ARG(T >= 0 && H > 0 && H % 128 == 0, "H must be a positive multiple of 128 (T=%d H=%d)", T, H);
  MOE_CHECK_ARG(hidden_actual >= 1 && hidden_actual <= H,
                "hidden_actual must be in [1, H=%d], got %d", H, hidden_actual);
  MOE_CHECK_ARG(eps >= 0.f, "eps must be >= 0");
  MOE_CHECK_SUPPORTED(H <= 256 * 8 * kNormMaxChunks, "H must be at most %d, got %d",
                      256 * 8 * kNormMaxChunks, H);
  MOE_CHECK_ARG(((uintptr_t)x_bf16 & 15) == 0 && ((uintptr_t)xn_bf16 & 15) == 0 &&
                    ((uintptr_t)residual_bf16 & 15) == 0 && ((uintptr_t)residual_out_bf16 & 15) == 0 &&
                    ((uintptr_t)gamma & 15) == 0 && ((uintptr_t)q & 7) == 0,
                "x, residual, xn, residual_out and gamma must be 16-byte aligned, q 8-byte aligned");
  if (T == 0) return MOE_OK;
  if (residual_bf16 != nullptr)
    launch_rms_norm_vec<false, false, true, true>(T, H, (hipStream_t)stream, x_bf16,
                                                  (const uint16_t*)residual_bf16, gamma, hidden_actual,
                                                  eps, xn_bf16, (uint16_t*)residual_out_bf16, q, s);
  else
    launch_rms_norm_vec<false, false, false, true>(T, H, (hipStream_t)stream, x_bf16, nullptr, gamma,
                                                   hidden_actual, eps, xn_bf16, nullptr, q, s);
  MOE_API_END();
}

extern "C" int moe_router_logits_f32(const float* x, const void* router_w, int w_is_f32,
                                     const float* bias, int T, int H, int E, float* logits,
                                     void* workspace, size_t workspace_bytes, void* stream) {
  MOE_API_BEGIN("moe_router_logits_f32");
  MOE_CHECK_ARG(x && router_w && logits, "null pointer argument");
  MOE_CHECK_ARG(T >= 0 && H > 0 && E > 0, "bad sizes T=%d H=%d E=%d", T, H, E);
  MOE_CHECK_ARG(H % 64 == 0, "H must be a multiple of 64, got %d", H);
  MOE_CHECK_ARG(((uintptr_t)x & 15) == 0 && ((uintptr_t)router_w & 15) == 0,
                "x and w must be 16-byte aligned");
  if (T == 0) return MOE_OK;
  hipStream_t st = (hipStream_t)stream;
  int ks = router_logits_splits(T, H, E);
  int kchunk = ((H / 64 + ks - 1) / ks) * 64;
  ks = (H + kchunk - 1) / kchunk;
  dim3 grid((T + 63) / 64, (E + 63) / 64, ks);
  float* dst = logits;
  if (ks > 1) {
    const size_t need = (size_t)ks * T * E * sizeof(float);
    MOE_CHECK_ARG(workspace != nullptr && workspace_bytes >= need,
                  "workspace too small: need %zu bytes", need);
    dst = (float*)workspace;
  }
  if (w_is_f32)
    hipLaunchKernelGGL(router_logits_f32_kernel<float>, grid, dim3(256), 0, st, x,
                       (const float*)router_w, bias, T, H, E, kchunk, dst);
  else
    hipLaunchKernelGGL(router_logits_f32_kernel<uint16_t>, grid, dim3(256), 0, st, x,
                       (const uint16_t*)router_w, bias, T, H, E, kchunk, dst);
  if (ks > 1) {
    const size_t n = (size_t)T * E;
    const int blocks = (int)std::min<size_t>((n + 255) / 256, 4096);
    hipLaunchKernelGGL(router_logits_f32_reduce, dim3(blocks), dim3(256), 0, st, dst, bias, T, E, ks,
                       logits);
  }
  MOE_API_END();
}
