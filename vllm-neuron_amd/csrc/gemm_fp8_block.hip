// Prefill-sized FP8-blockwise expert GEMMs ("block" kernels, gfx950).
//
// Same math as gemm_fp8.hip (reference: moe_cte.py:557-588, DeepSeek-V3 128x128
// block-scaled fp8 weights), organised for experts that receive hundreds of
// rows, where the layer becomes MFMA-bound:
//
//  * one workgroup (8 waves) computes a 128-row x 256-column tile: the rows are
//    up to 128 consecutive slots of one expert, the columns 256 weight rows
//    (gate_up: 128 gate rows + the matching 128 up rows; down: 256 outputs);
//  * both operands are staged through LDS in three stages of 128 K each (two K
//    blocks of lookahead), loaded with global_load_lds_dwordx4 (no register
//    staging); 16-byte chunks are XOR-swizzled by row pairs so 16-lane fragment
//    reads hit distinct banks of the 64-bank LDS;
//  * wave (wm, wn) owns rows [32 wm, +32) and 128 columns as 2 x 8 tiles of
//    v_mfma_f32_16x16x128_f8f6f4: one MFMA per tile covers a whole 128-K scale
//    block, so the 16 products of a K block are independent and issue back to
//    back; acc += part * (s_a[row] * s_w) promotes each in fp32 (the combined
//    scale per row and column half is precomputed into LDS);
//  * for gate_up wave column half wn holds gate and up columns [64 wn, +64) of
//    the tile's 128 h columns, so SiLU(g) * u is wave-local and only the row
//    amax of the 1x128 quantization group is combined across the two halves;
//  * work items (row tile, column tile) are enumerated expert by expert, column
//    tile by column tile, and mapped so that one XCD runs the items of one
//    expert together: the row tiles of an expert share each weight tile through
//    the XCD's L2, and the column tiles share the activation rows.
//
// Fragment lane layout (16x16x128): lane l supplies row l%16 and the bytes
// [(l/16)*16, +16) and [64 + (l/16)*16, +16) of the 128-wide K block, the same
// mapping for A and B. Accumulator: lane l, register i holds D[4*(l/16) + i][l%16].
#include "moe_common.h"
#include "moe_internal.h"

typedef float v16f __attribute__((ext_vector_type(16)));

namespace moe {

constexpr int kBM = 128, kBN = 256, kBK = 128;
constexpr int kBlkThreads = 512;
constexpr int kStages = 3;
constexpr int kStageA = kBM * kBK;  // 16 KB
constexpr int kStageB = kBN * kBK;  // 32 KB
constexpr int kDmaPerWave = (kStageA + kStageB) / 1024 / 8;  // 6 x 1 KB regions per wave

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

__device__ __forceinline__ v4f mfma16_fp8(const v8i& a, const v8i& b) {
  const v4f z = {0.f, 0.f, 0.f, 0.f};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, z, 0, 0, 0, 0, 0, 0);
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;

__device__ __forceinline__ void load_lds16(const void* g, uint8_t* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(g, (lds_ptr_t)lds_wave_base, 16, 0, 0);
}

// s_waitcnt vmcnt(N), other counters untouched (gfx9 encoding: vmcnt[3:0] | [15:14]).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

// Workgroup barrier that waits only for this wave's LDS operations (lgkmcnt),
// leaving the look-ahead direct-to-LDS loads in flight; __syncthreads() would
// also drain vmcnt. LDS-DMA data is covered by the explicit vmcnt waits.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt/expcnt untouched
  __builtin_amdgcn_s_barrier();
}

// Logical 16-byte chunk c of row r lives at chunk c ^ ((r >> 1) & 7): any 16
// consecutive rows read at one logical chunk touch 16 distinct 16-byte bank
// groups of the 64-bank LDS (two 128-byte rows span the banks once).
__device__ __forceinline__ int swz(int row, int chunk) { return chunk ^ ((row >> 1) & 7); }

// 16x16x128 operand fragment of `row`: logical chunks g and g + 4 (g = lane / 16).
__device__ __forceinline__ v8i lds_frag16(const uint8_t* base, int row, int g) {
  const uint8_t* rp = base + row * kBK;
  int4 lo = *(const int4*)(rp + swz(row, g) * 16);
  int4 hi = *(const int4*)(rp + swz(row, g + 4) * 16);
  return (v8i){lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
}

template <int KIND>
__global__ __launch_bounds__(kBlkThreads) void expert_gemm_block_kernel(BlkArgs p) {
  // Pipeline stages as distinct objects, so the compiler can tell that fragment
  // reads of one stage do not alias the direct-to-LDS loads in flight into another.
  __shared__ __attribute__((aligned(16))) uint8_t sT0[kStageA + kStageB];  // A tile, then B tile
  __shared__ __attribute__((aligned(16))) uint8_t sT1[kStageA + kStageB];
  __shared__ __attribute__((aligned(16))) uint8_t sT2[kStageA + kStageB];
  __shared__ __attribute__((aligned(16))) float sS0[2 * kBM];
  __shared__ __attribute__((aligned(16))) float sS1[2 * kBM];
  __shared__ __attribute__((aligned(16))) float sS2[2 * kBM];
  __shared__ int sSrc[kBM];
  __shared__ float sRed[2][kBM];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 3, wn = wave >> 2;
  const int Kdim = (KIND == 0) ? p.H : p.I;
  const int KB = Kdim / kBK;
  const int NT = (KIND == 0) ? p.I / 128 : p.H / kBN;

  // XCD-aware item index: workgroup b runs on XCD b % 8; XCD x takes the
  // contiguous item range [x * per, (x + 1) * per).
  const int count = p.num_tiles[0] * NT;
  const int per = (count + 7) / 8;
  const int jx = blockIdx.x >> 3;
  if (jx >= per) return;
  const int L = (blockIdx.x & 7) * per + jx;
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
        long sv = is_sh ? slot - p.NB - (long)ej * p.T : (long)p.tpid[slot];
        src = (sv >= 0 && sv < p.T) ? (int)sv : -1;
      } else {
        src = (int)slot;
      }
    }
    sSrc[r] = src;
  }
  __syncthreads();

  const uint8_t* wb;
  const float* wsb;
  if (KIND == 0) {
    wb = (is_sh ? p.wsh : p.w) + (size_t)ej * 2 * p.I * p.H;
    wsb = (is_sh ? p.wssh : p.ws) + (size_t)ej * (2 * p.I / 128) * KB;
  } else {
    wb = (is_sh ? p.wsh : p.w) + (size_t)ej * p.H * p.I;
    wsb = (is_sh ? p.wssh : p.ws) + (size_t)ej * (p.H / 128) * KB;
  }
  // Loader: 48 regions of 1 KB (A: 16, B: 32), 6 per wave: A regions 2w, 2w+1 and
  // B regions 4w..4w+3. Lane l writes region byte l*16 = row l/8, stored chunk l%8.
  uint32_t off[kDmaPerWave];
#pragma unroll
  for (int i = 0; i < kDmaPerWave; ++i) {
    if (i < 2) {
      const int row = 8 * (2 * wave + i) + (lane >> 3);
      const int src = sSrc[row];
      off[i] = (uint32_t)((src >= 0 ? src : 0) * Kdim + swz(row, lane & 7) * 16);
    } else {
      const int row = 8 * (4 * wave + i - 2) + (lane >> 3);
      int wrow;
      if (KIND == 0)
        wrow = (row < 128) ? nt * 128 + row : p.I + nt * 128 + (row - 128);
      else
        wrow = nt * kBN + row;
      off[i] = (uint32_t)(wrow * Kdim + swz(row, lane & 7) * 16);
    }
  }
  const uint8_t* abase = p.a;
  // Scale writers: threads 0..255 own (row tid % 128, column half tid / 128) and
  // store s_a[row] * s_w[half] for each stage.
  const int srow = tid & (kBM - 1), shalf = (tid >> 7) & 1;
  const bool swriter = tid < 2 * kBM;
  const float amask = (swriter && sSrc[srow] >= 0) ? 1.f : 0.f;
  const float* asp = p.as + (size_t)(sSrc[srow] >= 0 ? sSrc[srow] : 0) * KB;
  const float* swr;
  if (KIND == 0)
    swr = wsb + (size_t)(shalf == 0 ? nt : p.I / 128 + nt) * KB;
  else
    swr = wsb + (size_t)(nt * 2 + shalf) * KB;

  auto issue = [&](uint8_t* sa, int kb) {
    uint8_t* sb = sa + kStageA;
#pragma unroll
    for (int i = 0; i < kDmaPerWave; ++i) {
      if (i < 2)
        load_lds16(abase + off[i] + (size_t)kb * kBK, sa + (2 * wave + i) * 1024);
      else
        load_lds16(wb + off[i] + (size_t)kb * kBK, sb + (4 * wave + i - 2) * 1024);
    }
  };

  // Accumulators: 2 row tiles (16 rows) x 8 column tiles (16 columns), v_mfma 16x16x128.
  v4f acc[2][8];
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int n = 0; n < 8; ++n) acc[m][n] = (v4f){0.f, 0.f, 0.f, 0.f};

  const bool active = 32 * wm < nrows;  // this wave's 32 rows hold at least one row
  const int g = lane >> 4, l16 = lane & 15;
  // B rows of this wave's eight 16-column tiles. gate_up: tiles 0-3 gate columns
  // [64 wn, +64), tiles 4-7 the matching up columns; down: columns [128 wn, +128).
  int brow[8];
#pragma unroll
  for (int n = 0; n < 8; ++n) {
    if (KIND == 0)
      brow[n] = (n < 4) ? 64 * wn + 16 * n + l16 : 128 + 64 * wn + 16 * (n - 4) + l16;
    else
      brow[n] = 128 * wn + 16 * n + l16;
  }

  auto compute = [&](const uint8_t* sa, const float* ssc) {
    const uint8_t* sb = sa + kStageA;
    v8i a[2];
    v4f cs[2][2];  // [row tile][column half]
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      a[m] = lds_frag16(sa, 32 * wm + 16 * m + l16, g);
      const int r4 = 32 * wm + 16 * m + 4 * g;
      cs[m][0] = *(const v4f*)&ssc[((KIND == 0) ? 0 : wn) * kBM + r4];
      cs[m][1] = (KIND == 0) ? *(const v4f*)&ssc[kBM + r4] : cs[m][0];
    }
    // Two batches of four column tiles. The fragments of batch 1 are requested
    // before the MFMAs of batch 0 issue, and each batch's eight MFMAs are
    // independent, so the MFMA pipe is fed back to back while earlier results
    // get their fp32 promotion. Both row tiles are always computed (branch-free;
    // a partial last tile wastes at most 16 rows).
    v8i b0[4], b1[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) b0[j] = lds_frag16(sb, brow[j], g);
#pragma unroll
    for (int j = 0; j < 4; ++j) b1[j] = lds_frag16(sb, brow[4 + j], g);
#pragma unroll
    for (int bt = 0; bt < 2; ++bt) {
      v4f part[2][4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const v8i& b = bt == 0 ? b0[j] : b1[j];
        part[0][j] = mfma16_fp8(a[0], b);
        part[1][j] = mfma16_fp8(a[1], b);
      }
      const int hf = (KIND == 0) ? bt : 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[0][4 * bt + j] += part[0][j] * cs[0][hf];
        acc[1][4 * bt + j] += part[1][j] * cs[1][hf];
      }
    }
    // Schedule: all LDS fragment reads, the first 8 MFMAs, then each remaining
    // MFMA followed by the 4 promotion FMAs of an earlier product.
    __builtin_amdgcn_sched_group_barrier(0x100, 24, 0);  // DS reads
    __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);   // MFMA
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // VALU
    }
    __builtin_amdgcn_sched_group_barrier(0x002, 40, 0);   // VALU
  };

  // Raw scales ride a 3-slot register ring indexed by the unrolled step position
  // (no loop-carried copies, which would wait on the loads in flight).
  float ra[3] = {0.f, 0.f, 0.f}, rw[3] = {0.f, 0.f, 0.f};
  issue(sT0, 0);
  if (KB > 1) issue(sT1, 1);
  ra[0] = asp[0];
  rw[0] = swr[0];
  ra[1] = asp[min(1, KB - 1)];
  rw[1] = swr[min(1, KB - 1)];
  wait_vm<0>();
  if (swriter) sS0[shalf * kBM + srow] = ra[0] * rw[0] * amask;
  __syncthreads();

  // pos = kb % 3; na_: stage of block kb + 2; n1s: scale slot of block kb + 1
  auto step = [&](int kb, int pos, const uint8_t* ca, const float* cs_, uint8_t* na_,
                  float* n1s) {
    // Every step issues the same 8 vector-memory ops (past the last block it
    // re-reads block KB - 1 into a stage that is not read again), so the
    // in-order vmcnt wait below is exact on every path.
    const int kn = min(kb + 2, KB - 1);
    ra[(pos + 2) % 3] = asp[kn];
    rw[(pos + 2) % 3] = swr[kn];
    issue(na_, kn);
    __builtin_amdgcn_sched_barrier(0);
    if (active) compute(ca, cs_);
    __builtin_amdgcn_sched_barrier(0);
    // Issue order per step: 2 scale loads, then 6 tile loads. Block kb + 1's tile
    // loads (previous step) are followed by this step's 8 ops.
    wait_vm<2 + kDmaPerWave>();
    if (kb + 1 < KB && swriter) n1s[shalf * kBM + srow] = ra[(pos + 1) % 3] * rw[(pos + 1) % 3] * amask;
    __builtin_amdgcn_sched_barrier(0);
    lds_barrier();
    __builtin_amdgcn_sched_barrier(0);
  };
  for (int kb = 0; kb < KB; kb += 3) {
    step(kb, 0, sT0, sS0, sT2, sS1);
    if (kb + 1 < KB) step(kb + 1, 1, sT1, sS1, sT0, sS2);
    if (kb + 2 < KB) step(kb + 2, 2, sT2, sS2, sT1, sS0);
  }
  __syncthreads();

  // Accumulator layout (16x16): lane l, register i holds D[4*(l/16) + i][l%16].
  if (KIND == 0) {
    // h = SiLU(gate) * up for this wave's 64 h columns; the row amax of the 1x128
    // group combines the two column-half waves through LDS.
    const int GI = p.I / 128;
    float amax[2][4];
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float mx = 0.f;
#pragma unroll
        for (int n = 0; n < 4; ++n) {
          const float gt = acc[m][n][i], up = acc[m][n + 4][i];
          const float h = gt / (1.0f + __expf(-gt)) * up;
          acc[m][n][i] = h;
          mx = fmaxf(mx, fabsf(h));
        }
#pragma unroll
        for (int o = 8; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
        amax[m][i] = mx;
        if (l16 == 0) sRed[wn][32 * wm + 16 * m + 4 * g + i] = mx;
      }
    __syncthreads();
    if (active) {
#pragma unroll
      for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = 32 * wm + 16 * m + 4 * g + i;
          if (row < nrows && sSrc[row] >= 0) {
            const long slot = slot0 + row;
            const float sc = fmaxf(fmaxf(sRed[0][row], sRed[1][row]), 0x1.b7cdfep-34f) / 448.0f;
#pragma unroll
            for (int n = 0; n < 4; ++n) {
              const float yv = fminf(fmaxf(acc[m][n][i] / sc, -448.0f), 448.0f);
              p.hq[(size_t)slot * p.I + nt * 128 + 64 * wn + 16 * n + l16] = (uint8_t)f32_to_e4m3fn(yv);
            }
            if (wn == 0 && l16 == 0) p.hs[(size_t)slot * GI + nt] = sc;
          }
        }
    }
    (void)amax;
  } else if (active) {
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 32 * wm + 16 * m + 4 * g + i;
        if (row < nrows) {
          const long slot = slot0 + row;
#pragma unroll
          for (int n = 0; n < 8; ++n)
            p.y[(size_t)slot * p.H + nt * kBN + 128 * wn + 16 * n + l16] = f32_to_bf16_bits(acc[m][n][i]);
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
