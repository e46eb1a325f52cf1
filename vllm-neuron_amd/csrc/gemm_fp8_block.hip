// Prefill-sized FP8-blockwise expert GEMMs ("block" kernels, gfx950).
//
// Same math as gemm_fp8.hip (reference: moe_cte.py:557-588, DeepSeek-V3 128x128
// block-scaled fp8 weights), organised for experts that receive hundreds of
// rows, where the layer becomes MFMA-bound:
//
//  * one workgroup (8 waves) computes a 256-row x 256-column tile: the rows are
//    up to 256 consecutive slots of one expert, the columns 256 weight rows
//    (gate_up: 128 gate rows + the matching 128 up rows; down: 256 outputs);
//  * both operands are staged through LDS, two stages of 128 K each, loaded with
//    global_load_lds_dwordx4 (no register staging); 16-byte chunks are XOR-
//    swizzled by row so the 32-lane fragment reads hit distinct banks;
//  * wave w owns rows [32 w, +32) and all 256 columns as 8
//    v_mfma_f32_32x32x64_f8f6f4 tiles; per 128-K scale block two MFMAs form the
//    raw product, then acc += part * (s_a[row] * s_w) promotes it in fp32 (the
//    combined scale per row and column half is precomputed into LDS);
//  * for gate_up a wave holds the gate and the up columns of the same 128 h
//    columns, so SiLU(g) * u, the row amax of the 1x128 quantization group and
//    the requantization are wave-local;
//  * work items (row tile, column tile) are enumerated expert by expert, column
//    tile by column tile, and mapped so that one XCD runs the items of one
//    expert together: the row tiles of an expert share each weight tile through
//    the XCD's L2, and the column tiles share the activation rows.
//
// Fragment lane layout (32x32x64): lane l supplies row l%32 and the 32 bytes
// [h*64 + (l/32)*32, +32) of the 128-wide K block for MFMA h in {0, 1}; A and B
// use the same mapping. Accumulator: lane l, register r holds
// D[8*(r/4) + 4*(l/32) + r%4][l%32].
#include "moe_common.h"
#include "moe_internal.h"

typedef float v16f __attribute__((ext_vector_type(16)));

namespace moe {

constexpr int kBM = 256, kBN = 256, kBK = 128;
constexpr int kBlkThreads = 512;
constexpr int kStageA = kBM * kBK;                     // 32 KB
constexpr int kStageB = kBN * kBK;                     // 32 KB
constexpr int kStageBytes = kStageA + kStageB + 2 * kBM * 4;  // + s_a * s_w per row, per column half
constexpr int kBlkLds = 2 * kStageBytes;               // 132 KB

struct BlkArgs {
  const uint8_t* a;
  const float* as;
  const uint8_t* w;
  const float* ws;
  const uint8_t* wsh;
  const float* wssh;
  const int32_t* tpid;
  const int4* tiles;   // {expert, first slot, rows, 0}
  const int2* seg;     // {first tile of the expert, tiles of the expert}
  const int32_t* num_tiles;
  uint8_t* hq;
  float* hs;
  uint16_t* y;
  int T, H, I, E, nsh;
  long NB;
};

__device__ __forceinline__ v16f mfma32_fp8(const v8i& a, const v8i& b, const v16f& c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;

__device__ __forceinline__ void load_lds16(const void* g, uint8_t* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(g, (lds_ptr_t)lds_wave_base, 16, 0, 0);
}

__device__ __forceinline__ void wait_vm0() {
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
}

// Logical 16-byte chunk c of row r lives at chunk c ^ (r & 7).
__device__ __forceinline__ int swz(int row, int chunk) { return chunk ^ (row & 7); }

__device__ __forceinline__ v8i lds_frag32(const uint8_t* base, int row, int c0) {
  const uint8_t* rp = base + row * kBK;
  int4 lo = *(const int4*)(rp + swz(row, c0) * 16);
  int4 hi = *(const int4*)(rp + swz(row, c0 + 1) * 16);
  return (v8i){lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
}

template <int KIND>
__global__ __launch_bounds__(kBlkThreads) void expert_gemm_block_kernel(BlkArgs p) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[kBlkLds];
  __shared__ int sSrc[kBM];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int Kdim = (KIND == 0) ? p.H : p.I;
  const int KB = Kdim / kBK;
  const int NT = (KIND == 0) ? p.I / 128 : p.H / kBN;

  // XCD-aware item index: workgroup b runs on XCD b % 8; XCD x takes the
  // contiguous item range [x * per, (x + 1) * per).
  const int count = p.num_tiles[0] * NT;
  const int per = (count + 7) / 8;
  const int j = blockIdx.x >> 3;
  if (j >= per) return;
  const int L = (blockIdx.x & 7) * per + j;
  if (L >= count) return;
  const int2 sg = p.seg[L / NT];
  const int r0 = L - NT * sg.x;
  const int nt = r0 / sg.y;
  const int tile = sg.x + (r0 - nt * sg.y);
  if (tile >= p.num_tiles[0]) return;  // truncated tile list
  const int4 td = p.tiles[tile];
  const int e = td.x, nrows = td.z;
  const long slot0 = td.y;
  if (e < 0 || e >= p.E + p.nsh) return;
  const bool is_sh = e >= p.E;
  const int ej = is_sh ? e - p.E : e;

  for (int r = tid; r < kBM; r += kBlkThreads) {
    int src = -1;
    if (r < nrows) {
      const long slot = slot0 + r;
      if (KIND == 0) {
        long s = is_sh ? slot - p.NB - (long)ej * p.T : (long)p.tpid[slot];
        src = (s >= 0 && s < p.T) ? (int)s : -1;
      } else {
        src = (int)slot;
      }
    }
    sSrc[r] = src;
  }
  __syncthreads();

  // Loader assignment: wave w fills the 1 KB regions 4w..4w+3 of each operand
  // (8 rows per region); lane l writes region byte l*16 = row l/8, stored chunk l%8.
  const uint8_t* wb;
  const float* wsb;
  if (KIND == 0) {
    wb = (is_sh ? p.wsh : p.w) + (size_t)ej * 2 * p.I * p.H;
    wsb = (is_sh ? p.wssh : p.ws) + (size_t)ej * (2 * p.I / 128) * KB;
  } else {
    wb = (is_sh ? p.wsh : p.w) + (size_t)ej * p.H * p.I;
    wsb = (is_sh ? p.wssh : p.ws) + (size_t)ej * (p.H / 128) * KB;
  }
  uint32_t oa[4], ob[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 32 * wave + 8 * i + (lane >> 3);
    const int c = swz(row, lane & 7);
    const int src = sSrc[row];
    oa[i] = (uint32_t)((src >= 0 ? src : 0) * Kdim + c * 16);
    int wrow;
    if (KIND == 0)
      wrow = (row < 128) ? nt * 128 + row : p.I + nt * 128 + (row - 128);
    else
      wrow = nt * kBN + row;
    ob[i] = (uint32_t)(wrow * Kdim + c * 16);
  }
  // Threads 0..255 own one row's activation scale; threads 256..511 duplicate it
  // for the second column half. Each writes s_a[row] * s_w[half] per stage.
  const int srow = tid & (kBM - 1), shalf = tid >> 8;
  const float* asp = (sSrc[srow] >= 0) ? p.as + (size_t)sSrc[srow] * KB : nullptr;
  const float* swr;  // weight-scale row of column half `shalf`
  if (KIND == 0)
    swr = wsb + (size_t)(shalf == 0 ? nt : p.I / 128 + nt) * KB;
  else
    swr = wsb + (size_t)(nt * 2 + shalf) * KB;
  const uint8_t* abase = p.a;

  auto issue = [&](int stage, int kb) {
    uint8_t* sa = smem + stage * kStageBytes;
    uint8_t* sb = sa + kStageA;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      load_lds16(abase + oa[i] + (size_t)kb * kBK, sa + (4 * wave + i) * 1024);
      load_lds16(wb + ob[i] + (size_t)kb * kBK, sb + (4 * wave + i) * 1024);
    }
  };
  auto scale_of = [&](int kb) -> float { return asp ? asp[kb] * swr[kb] : 0.f; };
  auto put_scale = [&](int stage, float v) {
    ((float*)(smem + stage * kStageBytes + kStageA + kStageB))[shalf * kBM + srow] = v;
  };

  v16f acc[8];
#pragma unroll
  for (int n = 0; n < 8; ++n)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[n][r] = 0.f;

  const bool active = 32 * wave < nrows;  // this wave's 32-row tile holds rows
  const int g2 = lane >> 5, l32 = lane & 31;
  const int arow = 32 * wave + l32;

  issue(0, 0);
  float asn = scale_of(0);
  wait_vm0();
  put_scale(0, asn);
  __syncthreads();

  for (int kb = 0; kb < KB; ++kb) {
    const int cur = kb & 1;
    if (kb + 1 < KB) {
      issue(cur ^ 1, kb + 1);
      asn = scale_of(kb + 1);
    }
    if (active) {
      const uint8_t* sa = smem + cur * kStageBytes;
      const uint8_t* sb = sa + kStageA;
      const float* ssc = (const float*)(sb + kStageB);
      const v8i a0 = lds_frag32(sa, arow, 2 * g2);
      const v8i a1 = lds_frag32(sa, arow, 4 + 2 * g2);
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        v16f cs;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const v4f s4 = *(const v4f*)&ssc[hh * kBM + 32 * wave + 8 * q + 4 * g2];
#pragma unroll
          for (int i = 0; i < 4; ++i) cs[4 * q + i] = s4[i];
        }
#pragma unroll
        for (int n = 0; n < 4; ++n) {
          const int brow = 128 * hh + 32 * n + l32;
          const v8i b0 = lds_frag32(sb, brow, 2 * g2);
          const v8i b1 = lds_frag32(sb, brow, 4 + 2 * g2);
          v16f part = mfma32_fp8(a0, b0, (v16f){});
          part = mfma32_fp8(a1, b1, part);
          acc[4 * hh + n] += part * cs;
        }
      }
    }
    if (kb + 1 < KB) {
      wait_vm0();
      put_scale(cur ^ 1, asn);
    }
    __syncthreads();
  }

  if (!active) return;
  if (KIND == 0) {
    const int GI = p.I / 128;
    float amax[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) amax[r] = 0.f;
#pragma unroll
    for (int n = 0; n < 4; ++n)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float g = acc[n][r], u = acc[n + 4][r];
        const float h = g / (1.0f + __expf(-g)) * u;
        acc[n][r] = h;
        amax[r] = fmaxf(amax[r], fabsf(h));
      }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float m = amax[r];
#pragma unroll
      for (int o = 16; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
      amax[r] = m;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = 32 * wave + 8 * (r >> 2) + 4 * g2 + (r & 3);
      if (row < nrows && sSrc[row] >= 0) {
        const long slot = slot0 + row;
        const float sc = fmaxf(amax[r], 0x1.b7cdfep-34f) / 448.0f;
#pragma unroll
        for (int n = 0; n < 4; ++n) {
          const float yv = fminf(fmaxf(acc[n][r] / sc, -448.0f), 448.0f);
          p.hq[(size_t)slot * p.I + nt * 128 + 32 * n + l32] = (uint8_t)f32_to_e4m3fn(yv);
        }
        if (l32 == 0) p.hs[(size_t)slot * GI + nt] = sc;
      }
    }
  } else {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = 32 * wave + 8 * (r >> 2) + 4 * g2 + (r & 3);
      if (row < nrows) {
        const long slot = slot0 + row;
#pragma unroll
        for (int n = 0; n < 8; ++n)
          p.y[(size_t)slot * p.H + nt * kBN + 32 * n + l32] = f32_to_bf16_bits(acc[n][r]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Block tiles: per expert segment (consecutive blocks with one expert id), the
// slot range from its first block to its last valid slot, cut into chunks of
// 256 rows; seg[t] = {first tile of the segment, tiles in the segment}.
// Shared experts j: ceil(T/256) tiles over slots [NB + j*T, NB + (j+1)*T).
// One workgroup; per-block last-valid lengths go through global scratch.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void build_block_tiles_kernel(
    const int32_t* __restrict__ tpid, const int32_t* __restrict__ b2e, int N, int B, int T, int E,
    int n_shared, int* __restrict__ vlen, int* __restrict__ cnt, int4* __restrict__ tiles,
    int2* __restrict__ seg, int max_tiles, int32_t* __restrict__ num_tiles) {
  __shared__ int s_part[1024];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int b = wave; b < N; b += 16) {
    const int32_t* blk = tpid + (long)b * B;
    int v = 0;
    for (int s = lane; s < B; s += 64)
      if (blk[s] >= 0) v = s + 1;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o, 64));
    if (lane == 0) vlen[b] = v;
  }
  __syncthreads();
  __threadfence_block();
  // chunks per segment start
  for (int b = tid; b < N; b += blockDim.x) {
    int c = 0;
    if (b == 0 || b2e[b] != b2e[b - 1]) {
      int last = -1;
      for (int q = b; q < N && b2e[q] == b2e[b]; ++q)
        if (vlen[q] > 0) last = q;
      if (last >= 0) {
        long s1 = (long)last * B + vlen[last];
        c = (int)((s1 - (long)b * B + kBM - 1) / kBM);
      }
    }
    cnt[b] = c;
  }
  __syncthreads();
  __threadfence_block();
  // exclusive scan of cnt in chunks of 1024
  int base = 0;
  for (int b0 = 0; b0 < N; b0 += 1024) {
    const int b = b0 + tid;
    const int v = (b < N) ? cnt[b] : 0;
    s_part[tid] = v;
    __syncthreads();
    for (int o = 1; o < 1024; o <<= 1) {
      int t = (tid >= o) ? s_part[tid - o] : 0;
      __syncthreads();
      s_part[tid] += t;
      __syncthreads();
    }
    if (b < N && v > 0) {
      const int off = base + s_part[tid] - v;
      int last = b;
      for (int q = b; q < N && b2e[q] == b2e[b]; ++q)
        if (vlen[q] > 0) last = q;
      const long s0 = (long)b * B, s1 = (long)last * B + vlen[last];
      for (int c = 0; c < v; ++c) {
        const int idx = off + c;
        if (idx < max_tiles) {
          tiles[idx] = make_int4(b2e[b], (int)(s0 + (long)c * kBM), (int)min((long)kBM, s1 - s0 - (long)c * kBM), 0);
          seg[idx] = make_int2(off, v);
        }
      }
    }
    base += s_part[1023];
    __syncthreads();
  }
  const int per = (T + kBM - 1) / kBM;
  const long NB = (long)N * B;
  for (int i = tid; i < n_shared * per; i += blockDim.x) {
    const int jj = i / per, m = i - jj * per;
    const int idx = base + i;
    if (idx < max_tiles) {
      tiles[idx] = make_int4(E + jj, (int)(NB + (long)jj * T + (long)m * kBM), min(kBM, T - m * kBM), 0);
      seg[idx] = make_int2(base + jj * per, per);
    }
  }
  if (tid == 0) num_tiles[0] = min(base + n_shared * per, max_tiles);
}

template <int KIND>
static void launch_block(const BlkArgs& a, int max_tiles, hipStream_t st) {
  const int NT = (KIND == 0) ? a.I / 128 : a.H / kBN;
  long items = (long)max_tiles * NT;
  items = (items + 7) / 8 * 8;
  hipLaunchKernelGGL(expert_gemm_block_kernel<KIND>, dim3((unsigned)items), dim3(kBlkThreads), 0, st, a);
}

}  // namespace moe

using namespace moe;

extern "C" int moe_max_block_tiles(int T, int K, int E, int N, int B, int n_shared) {
  if (T <= 0 || K <= 0 || E <= 0 || N <= 0 || B <= 0 || n_shared < 0) return 0;
  const long routed = ((long)N * B + kBM - 1) / kBM + std::min(E, N);
  return (int)(routed + (long)n_shared * ((T + kBM - 1) / kBM));
}

extern "C" size_t moe_block_tiles_workspace_bytes(int N, int max_tiles) {
  if (N <= 0 || max_tiles <= 0) return 0;
  return (size_t)N * 8 + (size_t)max_tiles * 24 + 256;
}

extern "C" int moe_build_block_tiles(const int32_t* token_position_to_id,
                                     const int32_t* block_to_expert, int N, int B, int T, int E,
                                     int n_shared, int32_t* tiles, int max_tiles,
                                     int32_t* num_tiles, void* workspace, size_t workspace_bytes,
                                     void* stream) {
  MOE_API_BEGIN("moe_build_block_tiles");
  MOE_CHECK_ARG(token_position_to_id && block_to_expert && tiles && num_tiles && workspace,
                "null pointer argument");
  MOE_CHECK_ARG(N > 0 && B > 0 && T > 0 && E > 0 && n_shared >= 0 && max_tiles > 0, "bad sizes");
  MOE_CHECK_ARG(workspace_bytes >= moe_block_tiles_workspace_bytes(N, max_tiles),
                "workspace too small");
  // tiles buffer holds int4 tiles followed by int2 segments: max_tiles * 24 bytes
  int* vlen = (int*)workspace;
  int* cnt = vlen + N;
  hipLaunchKernelGGL(build_block_tiles_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream,
                     token_position_to_id, block_to_expert, N, B, T, E, n_shared, vlen, cnt,
                     (int4*)tiles, (int2*)(tiles + 4 * (size_t)max_tiles), max_tiles, num_tiles);
  MOE_API_END();
}

static int block_gemm_common_checks(const char* _moe_fn, int T, int H, int I, int E, int NB,
                                    int max_tiles) {
  MOE_CHECK_ARG(T > 0 && E > 0 && NB >= 0 && max_tiles > 0, "bad sizes");
  MOE_CHECK_ARG(H > 0 && H % 256 == 0 && I > 0 && I % 128 == 0,
                "H must be a multiple of 256 and I of 128 (H=%d I=%d)", H, I);
  return MOE_OK;
}

extern "C" int moe_expert_gate_up_block(const uint8_t* xq, const float* xs, int T, int H, int I,
                                        int E, const uint8_t* w13, const float* w13_scale,
                                        const uint8_t* w13_shared, const float* w13_shared_scale,
                                        int n_shared, const int32_t* token_position_to_id, int NB,
                                        const int32_t* tiles, const int32_t* num_tiles,
                                        int max_tiles, uint8_t* hq, float* hs, void* stream) {
  MOE_API_BEGIN("moe_expert_gate_up_block");
  MOE_CHECK_ARG(xq && xs && w13 && w13_scale && token_position_to_id && tiles && num_tiles && hq && hs,
                "null pointer argument");
  int rc = block_gemm_common_checks(_moe_fn, T, H, I, E, NB, max_tiles);
  if (rc != MOE_OK) return rc;
  MOE_CHECK_ARG(n_shared == 0 || (w13_shared && w13_shared_scale), "shared weights missing");
  MOE_CHECK_ARG(((uintptr_t)xq & 15) == 0 && ((uintptr_t)w13 & 15) == 0, "misaligned operands");
  BlkArgs a{};
  a.a = xq;
  a.as = xs;
  a.w = w13;
  a.ws = w13_scale;
  a.wsh = w13_shared;
  a.wssh = w13_shared_scale;
  a.tpid = token_position_to_id;
  a.tiles = (const int4*)tiles;
  a.seg = (const int2*)(tiles + 4 * (size_t)max_tiles);
  a.num_tiles = num_tiles;
  a.hq = hq;
  a.hs = hs;
  a.T = T;
  a.H = H;
  a.I = I;
  a.E = E;
  a.nsh = n_shared;
  a.NB = NB;
  launch_block<0>(a, max_tiles, (hipStream_t)stream);
  MOE_API_END();
}

extern "C" int moe_expert_down_block(const uint8_t* hq, const float* hs, int T, int H, int I, int E,
                                     const uint8_t* w2, const float* w2_scale,
                                     const uint8_t* w2_shared, const float* w2_shared_scale,
                                     int n_shared, int NB, const int32_t* tiles,
                                     const int32_t* num_tiles, int max_tiles, void* y_bf16,
                                     void* stream) {
  MOE_API_BEGIN("moe_expert_down_block");
  MOE_CHECK_ARG(hq && hs && w2 && w2_scale && tiles && num_tiles && y_bf16, "null pointer argument");
  int rc = block_gemm_common_checks(_moe_fn, T, H, I, E, NB, max_tiles);
  if (rc != MOE_OK) return rc;
  MOE_CHECK_ARG(n_shared == 0 || (w2_shared && w2_shared_scale), "shared weights missing");
  MOE_CHECK_ARG(((uintptr_t)hq & 15) == 0 && ((uintptr_t)w2 & 15) == 0, "misaligned operands");
  BlkArgs a{};
  a.a = hq;
  a.as = hs;
  a.w = w2;
  a.ws = w2_scale;
  a.wsh = w2_shared;
  a.wssh = w2_shared_scale;
  a.tiles = (const int4*)tiles;
  a.seg = (const int2*)(tiles + 4 * (size_t)max_tiles);
  a.num_tiles = num_tiles;
  a.y = (uint16_t*)y_bf16;
  a.T = T;
  a.H = H;
  a.I = I;
  a.E = E;
  a.nsh = n_shared;
  a.NB = NB;
  launch_block<1>(a, max_tiles, (hipStream_t)stream);
  MOE_API_END();
}
