// 1x128 fp8 activation quantization and the weighted unpermute-combine.
#include <type_traits>

#include "moe_common.h"
#include "moe_internal.h"

namespace moe {

// One wave per (row, 128-column group), quant_pair_1x128; each wave loads 8 of
// its groups at a time (all in flight together) before quantizing them.
__global__ __launch_bounds__(256) void act_quant_kernel(const uint16_t* __restrict__ x, int rows,
                                                        int cols, uint8_t* __restrict__ q,
                                                        float* __restrict__ s) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int G = cols / MOE_GROUP;
  const long total = (long)rows * G;
  const long nwaves = (long)gridDim.x * 4;
  for (long g0 = (long)blockIdx.x * 4 + wave; g0 < total; g0 += 8 * nwaves) {
    uint32_t pr[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const long gi = g0 + u * nwaves;
      pr[u] = (gi < total) ? *(const uint32_t*)(x + gi * MOE_GROUP + 2 * lane) : 0u;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const long gi = g0 + u * nwaves;  // group gi = row * G + column group: offset gi * 128
      if (gi < total) quant_pair_1x128(pr[u], q + gi * MOE_GROUP, s + gi, lane);
    }
  }
}

// Vector form for 16-byte aligned x and 8-byte aligned q (act_quant_vec_body).
__global__ __launch_bounds__(256) void act_quant_vec_kernel(const uint16_t* __restrict__ x, long groups,
                                                            uint8_t* __restrict__ q,
                                                            float* __restrict__ s) {
  act_quant_vec_body(x, groups, q, s, blockIdx.x, gridDim.x);
}

// out[t] = sum_s w[t,s] * y[inv[t,s]] (inv >= 0) + sum_j y[NB + j*T + t], fp32 accumulation.
// One workgroup per (token, column chunk), 8 bf16 (16 B) per thread. The token's live
// rows are listed in slot order (ballot compaction, so the order and the fp32 sums
// are the same as a sequential scan), then each thread sums its 8 columns over the
// rows, with the loads of up to 16 rows in flight.
__global__ __launch_bounds__(256) void combine_kernel(const uint16_t* __restrict__ y,
                                                      const int32_t* __restrict__ inv,
                                                      const float* __restrict__ w, int S, int T,
                                                      int H, long NB, int n_shared, int col_chunk,
                                                      uint16_t* __restrict__ out) {
  __shared__ long s_row[1024 + 16];
  __shared__ float s_w[1024 + 16];
  __shared__ int s_wave_n[4];
  const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int n = 0;
  for (int s0 = 0; s0 < S; s0 += 256) {
    const int s = s0 + tid;
    const int p = (s < S) ? inv[(size_t)t * S + s] : -1;
    const unsigned long long live = __ballot(p >= 0);
    if (lane == 0) s_wave_n[wave] = __popcll(live);
    __syncthreads();
    int before = n;
    for (int q = 0; q < wave; ++q) before += s_wave_n[q];
    if (p >= 0) {
      const int pos = before + __popcll(live & ((1ull << lane) - 1ull));
      s_row[pos] = p;
      s_w[pos] = (w != nullptr) ? w[(size_t)t * S + s] : 1.f;
    }
    n += s_wave_n[0] + s_wave_n[1] + s_wave_n[2] + s_wave_n[3];
    __syncthreads();
  }
  if (tid < n_shared) {
    s_row[n + tid] = NB + (long)tid * T + t;
    s_w[n + tid] = 1.f;
  }
  n += n_shared;
  __syncthreads();
  const int c_begin = blockIdx.y * col_chunk, c_end = min(H / 8, c_begin + col_chunk);
  for (int c = c_begin + tid; c < c_end; c += blockDim.x) {
    float acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0.f;
    // Rows r0 .. r0 + NR - 1, all NR loads in flight (unconditional: a load under a
    // branch would be waited for at the join), then summed in row order.
    auto rows = [&](auto nr, int r0) {
      constexpr int NR = decltype(nr)::value;
      int4 v[NR];
#pragma unroll
      for (int q = 0; q < NR; ++q) v[q] = *(const int4*)(y + (size_t)s_row[r0 + q] * H + c * 8);
#pragma unroll
      for (int q = 0; q < NR; ++q) {
        const float wt = s_w[r0 + q];
        const uint32_t u[4] = {(uint32_t)v[q].x, (uint32_t)v[q].y, (uint32_t)v[q].z, (uint32_t)v[q].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc[2 * i] += wt * bf16_bits_to_f32((uint16_t)(u[i] & 0xffffu));
          acc[2 * i + 1] += wt * bf16_bits_to_f32((uint16_t)(u[i] >> 16));
        }
      }
    };
    // Up to 16 rows at a time, all their loads in flight (workgroup-uniform counts,
    // no repeated loads): one memory round trip for a token's top-8 plus shared rows.
    for (int r0 = 0; r0 < n; r0 += 16) {
      switch (min(16, n - r0)) {
#define MOE_ROWS(NRV)                                     \
  case NRV:                                               \
    rows(std::integral_constant<int, NRV>{}, r0);         \
    break;
        MOE_ROWS(1) MOE_ROWS(2) MOE_ROWS(3) MOE_ROWS(4) MOE_ROWS(5) MOE_ROWS(6) MOE_ROWS(7)
        MOE_ROWS(8) MOE_ROWS(9) MOE_ROWS(10) MOE_ROWS(11) MOE_ROWS(12) MOE_ROWS(13)
        MOE_ROWS(14) MOE_ROWS(15) MOE_ROWS(16)
#undef MOE_ROWS
      }
    }
    int4 o;
    o.x = (int)bf16x2(acc[0], acc[1]);
    o.y = (int)bf16x2(acc[2], acc[3]);
    o.z = (int)bf16x2(acc[4], acc[5]);
    o.w = (int)bf16x2(acc[6], acc[7]);
    *(int4*)(out + (size_t)t * H + c * 8) = o;
  }
}

}  // namespace moe

using namespace moe;

extern "C" int moe_act_quant_1x128(const void* x_bf16, int rows, int cols, uint8_t* q,
                                   float* scales, void* stream) {
  MOE_API_BEGIN("moe_act_quant_1x128");
  MOE_CHECK_ARG(x_bf16 && q && scales, "null pointer argument");
  MOE_CHECK_ARG(rows >= 0 && cols > 0 && cols % MOE_GROUP == 0,
                "cols must be a positive multiple of 128, got %d", cols);
  MOE_CHECK_ARG(((uintptr_t)x_bf16 & 3) == 0 && ((uintptr_t)q & 1) == 0, "misaligned x or q");
  if (rows == 0) return MOE_OK;
  long groups = (long)rows * (cols / MOE_GROUP);
  if (((uintptr_t)x_bf16 & 15) == 0 && ((uintptr_t)q & 7) == 0) {
    const int grid = (int)std::max(1L, std::min<long>((groups + 15) / 16, 2048));
    hipLaunchKernelGGL(act_quant_vec_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t*)x_bf16, groups, q, scales);
  } else {
    int grid = (int)std::min<long>((groups + 3) / 4, 2048);
    hipLaunchKernelGGL(act_quant_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t*)x_bf16, rows, cols, q, scales);
  }
  MOE_API_END();
}

extern "C" int moe_combine(const void* y_bf16, const int32_t* inv, const float* w, int S, int T,
                           int H, int NB, int n_shared, void* out_bf16, void* stream) {
  MOE_API_BEGIN("moe_combine");
  MOE_CHECK_ARG(y_bf16 && out_bf16 && (inv || S == 0), "null pointer argument");
  MOE_CHECK_ARG(T >= 0 && H > 0 && H % 8 == 0 && S >= 0 && S <= 1024 && n_shared >= 0 &&
                    n_shared <= 16 && NB >= 0,
                "bad sizes T=%d H=%d S=%d n_shared=%d", T, H, S, n_shared);
  MOE_CHECK_ARG(((uintptr_t)y_bf16 & 15) == 0 && ((uintptr_t)out_bf16 & 15) == 0,
                "y and out must be 16-byte aligned");
  if (T == 0) return MOE_OK;
  // Enough (token, column chunk) workgroups to cover the chip: at least 512.
  const int chunks = H / 8;
  int splits = std::max(1, std::min((512 + T - 1) / T, (chunks + 127) / 128));
  const int col_chunk = (chunks + splits - 1) / splits;
  splits = (chunks + col_chunk - 1) / col_chunk;
  hipLaunchKernelGGL(combine_kernel, dim3(T, splits), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)y_bf16, inv, w, S, T, H, (long)NB, n_shared, col_chunk,
                     (uint16_t*)out_bf16);
  MOE_API_END();
}
