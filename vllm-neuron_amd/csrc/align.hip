// Align-by-expert ("blockwise") mapping and the expert row-tile list.
//
// Reference: vllm_neuron/functional/moe/moe_blockwise.py:25-157 (API),
// :325-437 (torch flow). The slot of (token t, expert e) is
//   block_offset[e] * B + #{t' < t : t' routed to e},
// i.e. every expert owns ceil(count/B) consecutive blocks and lists its tokens
// in ascending token order.
//
// Three deterministic passes, no global atomics on the data path:
//  1. map_count  : one workgroup per 256-token chunk builds an LDS bitmask
//                  [E][256 bits] of (token, expert) pairs and writes the
//                  per-chunk expert histogram (popcounts); it also fills
//                  token_position_to_id with -1.
//  2. map_scan   : one workgroup scans the histograms over chunks (per-chunk
//                  base) and over experts (block offsets), and writes
//                  expert_counts, block_to_expert and conditions.
//  3. map_scatter: rebuilds the chunk bitmask; the rank of t inside its chunk
//                  is a popcount of the bits below it; writes the slots.
#include "mapping.h"

namespace moe {

__global__ __launch_bounds__(256) void map_count_kernel(
    const int32_t* __restrict__ ids, const float* __restrict__ aff,
    const uint8_t* __restrict__ pmask, float* __restrict__ aff_masked, int T, int K, int E,
    int nchunks, long nb_total, int32_t* __restrict__ tpid, MapWs ws) {
  __shared__ uint32_t bm[kMapMaxE][8];
  // token_position_to_id := -1 (grid-stride, all workgroups)
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < nb_total;
       i += (long)gridDim.x * blockDim.x)
    tpid[i] = -1;
  if (blockIdx.x == 0 && threadIdx.x == 0) ws.status[0] = 0;
  const int chunk = blockIdx.x;
  if (chunk >= nchunks) return;  // workgroup-uniform
  const int t0 = chunk * kChunk;
  if (aff != nullptr && aff_masked != nullptr) {
    for (int i = threadIdx.x; i < kChunk * E; i += blockDim.x) {
      int tl = i / E, t = t0 + tl;
      if (t >= T) break;
      size_t o = (size_t)t * E + (i - tl * E);
      float m = (pmask == nullptr || pmask[t] != 0) ? 1.f : 0.f;
      aff_masked[o] = aff[o] * m;
    }
  }
  build_chunk_mask(bm, ids, aff, T, K, E, t0, nullptr);
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    int c = 0;
#pragma unroll
    for (int w = 0; w < 8; ++w) c += __popc(bm[e][w]);
    ws.chunk_counts[(size_t)chunk * E + e] = c;
  }
}

__global__ __launch_bounds__(1024) void map_scan_kernel(int T, int E, int B, int N, int nchunks,
                                                        int32_t* __restrict__ expert_counts,
                                                        int32_t* __restrict__ block_to_expert,
                                                        int32_t* __restrict__ conditions,
                                                        MapWs ws, TileOut to) {
  __shared__ int s_blk[kMapMaxE];
  __shared__ int s_cnt[kMapMaxE];
  __shared__ int s_cex[kMapMaxE];
  __shared__ int s_tile[kMapMaxE];
  __shared__ int s_wave[16];
  const int tid = threadIdx.x;
  int run = 0;
  if (tid < E) {
    for (int c = 0; c < nchunks; ++c) {
      int v = ws.chunk_counts[(size_t)c * E + tid];
      ws.chunk_base[(size_t)c * E + tid] = run;
      run += v;
    }
  }
  finish_mapping(T, E, B, N, run, expert_counts, block_to_expert, conditions, ws.block_off,
                 ws.count_off, to, s_blk, s_cnt, s_cex, s_tile, s_wave);
}

// The whole mapping in one workgroup, for ids and at most one 256-token chunk
// (decode): fill, bitmask, counts, scan, tiles and scatter without the three
// launches of the chunked path. Same outputs, same slot order.
__global__ __launch_bounds__(1024) void map_small_kernel(
    const int32_t* __restrict__ ids, int T, int K, int E, int B, int N,
    int32_t* __restrict__ tpid, int32_t* __restrict__ block_to_expert,
    int32_t* __restrict__ conditions, int32_t* __restrict__ expert_counts,
    int32_t* __restrict__ inv_pos, MapWs ws, TileOut to) {
  __shared__ uint32_t bm[kMapMaxE][8];
  __shared__ int s_blk[kMapMaxE];
  __shared__ int s_cnt[kMapMaxE];
  __shared__ int s_cex[kMapMaxE];
  __shared__ int s_tile[kMapMaxE];
  __shared__ int s_wave[16];
  map_small_body(ids, nullptr, T, K, E, B, N, tpid, block_to_expert, conditions, expert_counts,
                 inv_pos, ws, to, bm, s_blk, s_cnt, s_cex, s_tile, s_wave);
}

// inv_rows: inv_pos receives compact rows (count_off[e] + rank in the expert)
// instead of slots.
__global__ __launch_bounds__(256) void map_scatter_kernel(
    const int32_t* __restrict__ ids, const float* __restrict__ aff, int T, int K, int E, int B,
    long nb_total, int32_t* __restrict__ tpid, int32_t* __restrict__ inv_pos, int inv_rows,
    MapWs ws) {
  __shared__ uint32_t bm[kMapMaxE][8];
  const int chunk = blockIdx.x, t0 = chunk * kChunk;
  build_chunk_mask(bm, ids, aff, T, K, E, t0, ws.status);
  // rank of token t0 + tl among the tokens of expert e (all chunks)
  auto rank_of = [&](int e, int tl) -> int {
    int rank = 0;
    const int wq = tl >> 5;
    for (int w = 0; w < wq; ++w) rank += __popc(bm[e][w]);
    rank += __popc(bm[e][wq] & ((1u << (tl & 31)) - 1u));
    return ws.chunk_base[(size_t)chunk * E + e] + rank;
  };
  auto slot_of = [&](int e, int tl) -> long { return (long)ws.block_off[e] * B + rank_of(e, tl); };
  if (ids != nullptr) {
    for (int i = threadIdx.x; i < kChunk * K; i += blockDim.x) {
      int tl = i / K, t = t0 + tl;
      if (t >= T) break;
      size_t o = (size_t)t * K + (i - tl * K);
      int e = ids[o];
      int out = -1;
      if (e >= 0 && e < E) {
        long s = slot_of(e, tl);
        if (s < nb_total) {
          tpid[s] = t;
          out = inv_rows ? ws.count_off[e] + rank_of(e, tl) : (int)s;
        } else {
          atomicAdd(ws.status, 1);
        }
      }
      if (inv_pos != nullptr) inv_pos[o] = out;
    }
  } else {
    for (int i = threadIdx.x; i < kChunk * E; i += blockDim.x) {
      int tl = i / E, t = t0 + tl;
      if (t >= T) break;
      int e = i - tl * E;
      if (aff[(size_t)t * E + e] != 0.f) {
        long s = slot_of(e, tl);
        if (s < nb_total) tpid[s] = t;
        else atomicAdd(ws.status, 1);
      }
    }
  }
}

// inv[t, e] = slot, for a mapping given by token_position_to_id / block_to_expert.
__global__ void invert_fill_kernel(int32_t* inv, long n) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x)
    inv[i] = -1;
}

__global__ void invert_scatter_kernel(const int32_t* __restrict__ tpid,
                                      const int32_t* __restrict__ b2e, int N, int B, int T, int E,
                                      int32_t* __restrict__ inv) {
  long nb = (long)N * B;
  for (long s = (long)blockIdx.x * blockDim.x + threadIdx.x; s < nb; s += (long)gridDim.x * blockDim.x) {
    int t = tpid[s];
    int e = b2e[s / B];
    if (t >= 0 && t < T && e >= 0 && e < E) inv[(size_t)t * E + e] = (int)s;
  }
}

// ---------------------------------------------------------------------------
// Row tiles: for every block, the slots up to its last valid entry, cut into
// tiles of `mt` rows; then n_shared * ceil(T/mt) tiles for the shared experts.
// One workgroup of 1024 threads; blocks are processed 4096 at a time.
// ---------------------------------------------------------------------------
constexpr int kTileChunk = 4096;

__global__ __launch_bounds__(1024) void build_tiles_kernel(
    const int32_t* __restrict__ tpid, const int32_t* __restrict__ b2e, int N, int B, int T, int E,
    int n_shared, int mt, int4* __restrict__ tiles, int max_tiles, int32_t* __restrict__ num_tiles) {
  __shared__ int s_vlen[kTileChunk];
  __shared__ int s_cnt[kTileChunk];
  __shared__ int s_part[1024];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int base = 0;
  for (int b0 = 0; b0 < N; b0 += kTileChunk) {
    const int nb = min(kTileChunk, N - b0);
    for (int bl = wave; bl < nb; bl += 16) {
      const int32_t* blk = tpid + (long)(b0 + bl) * B;
      int v = 0;
      for (int s = lane; s < B; s += 64)
        if (blk[s] >= 0) v = s + 1;
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o, 64));
      if (lane == 0) {
        s_vlen[bl] = v;
        s_cnt[bl] = (v + mt - 1) / mt;
      }
    }
    __syncthreads();
    // exclusive scan of s_cnt[0..nb): 4 entries per thread, then Hillis-Steele.
    int loc[4], sum = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      int i = tid * 4 + q;
      loc[q] = (i < nb) ? s_cnt[i] : 0;
      sum += loc[q];
    }
    s_part[tid] = sum;
    __syncthreads();
    for (int o = 1; o < 1024; o <<= 1) {
      int v = (tid >= o) ? s_part[tid - o] : 0;
      __syncthreads();
      s_part[tid] += v;
      __syncthreads();
    }
    const int chunk_total = s_part[1023];
    int run = s_part[tid] - sum;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      int i = tid * 4 + q;
      if (i < nb) {
        const int b = b0 + i, e = b2e[b];
        for (int j = 0; j < loc[q]; ++j) {
          int idx = base + run + j;
          if (idx < max_tiles)
            tiles[idx] = make_int4(e, b * B + j * mt, min(mt, s_vlen[i] - j * mt), b * B + j * mt);
        }
        run += loc[q];
      }
    }
    base += chunk_total;
    __syncthreads();
  }
  const int per = (T + mt - 1) / mt;
  const long nb_total = (long)N * B;
  for (int i = tid; i < n_shared * per; i += blockDim.x) {
    int j = i / per, m = i - j * per;
    int idx = base + i;
    if (idx < max_tiles) {
      const int s0 = (int)(nb_total + (long)j * T + (long)m * mt);
      tiles[idx] = make_int4(E + j, s0, min(mt, T - m * mt), s0);
    }
  }
  if (tid == 0) num_tiles[0] = min(base + n_shared * per, max_tiles);
}

}  // namespace moe

using namespace moe;

extern "C" int moe_num_blocks(int T, int K, int E, int B) {
  if (T <= 0 || K <= 0 || E <= 0 || B <= 0) return 0;
  long total = (long)T * std::min(K, E);
  long num = total - (E - 1);
  // ceil division that matches math.ceil for negative numerators
  long q = num >= 0 ? (num + B - 1) / B : -((-num) / B);
  long n = q + E - 1;
  return (int)std::min(n, total);
}

extern "C" size_t moe_mapping_workspace_bytes(int T, int E) {
  if (T < 0 || E <= 0) return 0;
  return map_ws_bytes(std::max(T, 1), E);
}

int moe::blockwise_mapping(const int32_t* ids, const float* affinities,
                           const uint8_t* padding_mask, int T, int K, int E, int B, int N,
                           int32_t* token_position_to_id, int32_t* block_to_expert,
                           int32_t* conditions, int32_t* expert_counts, int32_t* inv_pos,
                           float* affinities_masked, void* workspace, size_t workspace_bytes,
                           const TileOut& to, void* stream) {
  MOE_API_BEGIN("moe_blockwise_mapping");
  MOE_CHECK_ARG(to.tiles == nullptr || (to.num_tiles && to.mt > 0 && to.max_tiles > 0 &&
                                        to.n_shared >= 0 && (!to.span || to.seg)),
                "bad tile output");
  MOE_CHECK_ARG(!to.compact || (to.tiles != nullptr && ids != nullptr && to.row_shared >= 0),
                "compact rows need ids and a tile list");
  MOE_CHECK_ARG((ids != nullptr) != (affinities != nullptr),
                "exactly one of ids / affinities must be given");
  MOE_CHECK_ARG(token_position_to_id && block_to_expert && workspace, "null pointer argument");
  MOE_CHECK_ARG(T > 0 && K > 0 && E > 0 && B > 0, "bad sizes T=%d K=%d E=%d B=%d", T, K, E, B);
  MOE_CHECK_SUPPORTED(E <= kMapMaxE, "at most %d experts supported, got %d", kMapMaxE, E);
  MOE_CHECK_ARG(N == moe_num_blocks(T, K, E, B), "N=%d does not match the block formula (%d)", N,
                moe_num_blocks(T, K, E, B));
  MOE_CHECK_ARG(workspace_bytes >= map_ws_bytes(T, E), "workspace too small: need %zu bytes",
                map_ws_bytes(T, E));
  MOE_CHECK_ARG(ids != nullptr || inv_pos == nullptr, "inv_pos requires ids");
  hipStream_t st = (hipStream_t)stream;
  MapWs ws = carve_map_ws(workspace, T, E);
  const int nch = (T + kChunk - 1) / kChunk;
  const long nbt = (long)N * B;
  int grid1 = std::max(nch, (int)std::min<long>(1024, (nbt + 255) / 256));
  if (ids != nullptr && nch == 1) {
    hipLaunchKernelGGL(map_small_kernel, dim3(1), dim3(1024), 0, st, ids, T, K, E, B, N,
                       token_position_to_id, block_to_expert, conditions, expert_counts, inv_pos, ws,
                       to);
    MOE_API_END();
  }
  hipLaunchKernelGGL(map_count_kernel, dim3(grid1), dim3(256), 0, st, ids, affinities,
                     padding_mask, affinities_masked, T, K, E, nch, nbt, token_position_to_id, ws);
  hipLaunchKernelGGL(map_scan_kernel, dim3(1), dim3(1024), 0, st, T, E, B, N, nch, expert_counts,
                     block_to_expert, conditions, ws, to);
  hipLaunchKernelGGL(map_scatter_kernel, dim3(nch), dim3(256), 0, st, ids, affinities, T, K, E, B,
                     nbt, token_position_to_id, inv_pos, to.compact, ws);
  MOE_API_END();
}

extern "C" int moe_blockwise_mapping(const int32_t* ids, const float* affinities,
                                     const uint8_t* padding_mask, int T, int K, int E, int B,
                                     int N, int32_t* token_position_to_id,
                                     int32_t* block_to_expert, int32_t* conditions,
                                     int32_t* expert_counts, int32_t* inv_pos,
                                     float* affinities_masked, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  return moe::blockwise_mapping(ids, affinities, padding_mask, T, K, E, B, N,
                                token_position_to_id, block_to_expert, conditions, expert_counts,
                                inv_pos, affinities_masked, workspace, workspace_bytes, TileOut{},
                                stream);
}

extern "C" int moe_mapping_status(const void* workspace, void* stream, int* dropped) {
  MOE_API_BEGIN("moe_mapping_status");
  MOE_CHECK_ARG(workspace && dropped, "null pointer argument");
  int32_t v = 0;
  MOE_CHECK_HIP(hipMemcpyAsync(&v, workspace, sizeof(v), hipMemcpyDeviceToHost, (hipStream_t)stream));
  MOE_CHECK_HIP(hipStreamSynchronize((hipStream_t)stream));
  *dropped = v;
  return MOE_OK;
}

extern "C" int moe_invert_mapping(const int32_t* token_position_to_id,
                                  const int32_t* block_to_expert, int N, int B, int T, int E,
                                  int32_t* inv, void* stream) {
  MOE_API_BEGIN("moe_invert_mapping");
  MOE_CHECK_ARG(token_position_to_id && block_to_expert && inv, "null pointer argument");
  MOE_CHECK_ARG(N > 0 && B > 0 && T > 0 && E > 0, "bad sizes");
  hipStream_t st = (hipStream_t)stream;
  long n = (long)T * E, nb = (long)N * B;
  hipLaunchKernelGGL(invert_fill_kernel, dim3((int)std::min<long>(2048, (n + 255) / 256)),
                     dim3(256), 0, st, inv, n);
  hipLaunchKernelGGL(invert_scatter_kernel, dim3((int)std::min<long>(2048, (nb + 255) / 256)),
                     dim3(256), 0, st, token_position_to_id, block_to_expert, N, B, T, E, inv);
  MOE_API_END();
}

extern "C" int moe_max_tiles(int T, int K, int E, int N, int B, int n_shared, int mt) {
  if (T <= 0 || K <= 0 || E <= 0 || N <= 0 || B <= 0 || mt <= 0 || n_shared < 0) return 0;
  long per_block = (B + mt - 1) / mt;
  long routed = std::min((long)N * per_block, ((long)T * std::min(K, E) + mt - 1) / mt + N);
  return (int)(routed + (long)n_shared * ((T + mt - 1) / mt));
}

extern "C" int moe_build_tiles(const int32_t* token_position_to_id, const int32_t* block_to_expert,
                               int N, int B, int T, int E, int n_shared, int mt, int32_t* tiles,
                               int max_tiles, int32_t* num_tiles, void* stream) {
  MOE_API_BEGIN("moe_build_tiles");
  MOE_CHECK_ARG(token_position_to_id && block_to_expert && tiles && num_tiles,
                "null pointer argument");
  MOE_CHECK_ARG(N > 0 && B > 0 && T > 0 && E > 0 && n_shared >= 0 && max_tiles > 0, "bad sizes");
  MOE_CHECK_ARG(mt == 16 || mt == 32 || mt == 64 || mt == 128, "mt must be 16/32/64/128, got %d",
                mt);
  hipLaunchKernelGGL(build_tiles_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream,
                     token_position_to_id, block_to_expert, N, B, T, E, n_shared, mt,
                     (int4*)tiles, max_tiles, num_tiles);
  MOE_API_END();
}
