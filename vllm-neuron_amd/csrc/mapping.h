// Device code of the align-by-expert mapping shared by the mapping kernels
// (align.hip) and the top-k kernel that ends in the mapping (router.hip), plus the
// layout of the mapping workspace.
//
// Reference: vllm_neuron/functional/moe/moe_blockwise.py:25-157 (API),
// :325-437 (torch flow). The slot of (token t, expert e) is
//   block_offset[e] * B + #{t' < t : t' routed to e}.
#pragma once

#include "moe_common.h"
#include "moe_internal.h"

namespace moe {

constexpr int kChunk = 256;    // tokens per chunk (256 bits = 8 words per expert)
constexpr int kMapMaxE = 1024;  // LDS bitmask capacity

struct MapWs {
  int32_t* status;       // [4]: dropped pairs at [0]
  int32_t* chunk_counts;  // [nchunks, E]
  int32_t* chunk_base;    // [nchunks, E]
  int32_t* block_off;     // [E]
  int32_t* count_off;     // [E] exclusive prefix of the counts (compact rows)
};

static inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static inline MapWs carve_map_ws(void* ws, int T, int E) {
  int nch = (T + kChunk - 1) / kChunk;
  char* p = (char*)ws;
  MapWs m;
  m.status = (int32_t*)p;
  p += 256;
  m.chunk_counts = (int32_t*)p;
  p += align256((size_t)nch * E * 4);
  m.chunk_base = (int32_t*)p;
  p += align256((size_t)nch * E * 4);
  m.block_off = (int32_t*)p;
  p += align256((size_t)E * 4);
  m.count_off = (int32_t*)p;
  return m;
}

static inline size_t map_ws_bytes(int T, int E) {
  int nch = (T + kChunk - 1) / kChunk;
  return 256 + 2 * align256((size_t)nch * E * 4) + 2 * align256((size_t)E * 4);
}

static __device__ __forceinline__ void build_chunk_mask(uint32_t (*bm)[8], const int32_t* ids,
                                                 const float* aff, int T, int K, int E, int t0,
                                                 int32_t* status) {
  for (int i = threadIdx.x; i < E * 8; i += blockDim.x) bm[i >> 3][i & 7] = 0u;
  __syncthreads();
  if (ids != nullptr) {
    for (int i = threadIdx.x; i < kChunk * K; i += blockDim.x) {
      int tl = i / K, t = t0 + tl;
      if (t >= T) break;
      int e = ids[(size_t)t * K + (i - tl * K)];
      if (e >= 0 && e < E) {
        atomicOr(&bm[e][tl >> 5], 1u << (tl & 31));
      } else if (e >= E && status != nullptr) {
        atomicAdd(status, 1);
      }
    }
  } else {
    for (int i = threadIdx.x; i < kChunk * E; i += blockDim.x) {
      int tl = i / E, t = t0 + tl;
      if (t >= T) break;
      int e = i - tl * E;
      if (aff[(size_t)t * E + e] != 0.f) atomicOr(&bm[e][tl >> 5], 1u << (tl & 31));
    }
  }
  __syncthreads();
}


// Inclusive sum over the 1024 threads of a workgroup (wave scans, then the
// 16 wave totals); s_wave holds 16 ints.
// Wave-inclusive part by DPP moves (no LDS round trips): row_shr 1, 2, 4, 8 within
// each row of 16 lanes (lanes shifted in from outside the row add 0), then row 0's
// total into row 1 and row 2's into row 3 (row_bcast:15), and the total of rows 0-1
// into rows 2-3 (row_bcast:31).
template <int CTRL, int ROW_MASK>
static __device__ __forceinline__ int dpp_add_in(int v) {
  return v + __builtin_amdgcn_update_dpp(0, v, CTRL, ROW_MASK, 0xF, true);
}
static __device__ __forceinline__ int block_inclusive_sum(int v, int* s_wave) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v = dpp_add_in<0x111, 0xF>(v);
  v = dpp_add_in<0x112, 0xF>(v);
  v = dpp_add_in<0x114, 0xF>(v);
  v = dpp_add_in<0x118, 0xF>(v);
  v = dpp_add_in<0x142, 0xA>(v);
  v = dpp_add_in<0x143, 0xC>(v);
  if (lane == 63) s_wave[wave] = v;
  __syncthreads();
  // the totals of the waves before this one: all 16 entries read together, one
  // wait (s_wave holds 16; entries of absent waves are read and masked off)
  int add = 0;
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const int w = s_wave[q];
    add += (q < wave) ? w : 0;
  }
  __syncthreads();
  return v + add;
}

// Cut points of a block-tile list over the 8 XCDs: hdr[1 + x], x = 0..8, is the first
// tile of XCD x's range and hdr[9] = n. The ranges hold whole experts (the sibling
// tiles of an expert share its weight tiles in one XCD's L2) and about equal cost,
// a tile costing 3 + ceil(rows / 64): the fixed work of its K steps plus one unit
// per 64-row MFMA group, the split of the block kernels' time by tile height. A
// split into equal item counts left the XCD with the tallest tiles up to 10 %
// behind the others. Every range holds at most block_tiles_cap(max_tiles) tiles, the
// share of the launch grid each XCD gets (cuts are clamped to that, off expert
// boundaries if need be), so every item has a workgroup. Whole workgroup of 1024
// threads, after the tile list's stores (this workgroup's) are complete.
static __host__ __device__ inline int block_tiles_cap(int max_tiles) {
  return max(3 * max_tiles / 16, (max_tiles + 7) / 8);
}
static __device__ void block_tile_cuts(const int4* __restrict__ tiles, int n, int max_tiles,
                                       int32_t* __restrict__ hdr, int* s_wave) {
  __shared__ unsigned long long s_best[8];
  __shared__ long s_tot;
  const int tid = threadIdx.x;
  auto cost = [&](int t) { return 3 + (tiles[t].z + 63) / 64; };
  if (tid < 8) s_best[tid] = ~0ull;
  int part = 0;
  for (int t = tid; t < n; t += blockDim.x) part += cost(t);
  const int inc = block_inclusive_sum(part, s_wave);
  if (tid == (int)blockDim.x - 1) s_tot = inc;
  __syncthreads();
  const long C = s_tot;
  long base = 0;
  for (int t0 = 0; t0 < n; t0 += blockDim.x) {
    const int t = t0 + tid;
    const int c = t < n ? cost(t) : 0;
    const int ci = block_inclusive_sum(c, s_wave);
    const long excl = base + ci - c;
    if (t < n && (t == 0 || tiles[t].x != tiles[t - 1].x)) {
      for (int x = 1; x < 8; ++x) {
        const long d = 8 * excl - (long)x * C;
        atomicMin(&s_best[x], ((unsigned long long)(d < 0 ? -d : d) << 20) | (unsigned)t);
      }
    }
    if (tid == (int)blockDim.x - 1) s_tot = ci;  // the chunk's total
    __syncthreads();
    base += s_tot;
    __syncthreads();
  }
  if (tid == 0) {
    const int cap = block_tiles_cap(max_tiles);  // 8 cap >= max_tiles >= n
    int prev = 0;
    hdr[1] = 0;
    for (int x = 1; x < 8; ++x) {
      int v = s_best[x] == ~0ull ? n : (int)(s_best[x] & 0xFFFFF);
      // monotone, at most cap tiles in this range and at most cap in each later one
      v = min(max(v, max(prev, n - (8 - x) * cap)), min(prev + cap, n));
      hdr[1 + x] = v;
      prev = v;
    }
    hdr[9] = n;
  }
}

// Everything after the per-expert counts: block offsets (exclusive scan of
// ceil(count/B)), expert_counts, block_to_expert, conditions and the optional tile
// list. Thread tid < E holds run = count of expert tid. Leaves the inclusive
// block scan in s_blk, the counts in s_cnt and, for compact rows, the exclusive
// count scan in s_cex (and count_off); 1024 threads.
// SMALL (at most 256 tokens, so at most 256 blocks and tiles per expert): each
// expert's thread writes its own blocks and tiles, with no binary search over the
// scans; with fewer than 2^16 ids (ids_bound = T * K, which bounds every total)
// the block and tile counts are scanned together, 16 bits each, and with fewer
// than 2^10 the expert counts join them (compact rows), 10 bits each.
template <bool SMALL = false>
static __device__ void finish_mapping(int T, int E, int B, int N, int run, int32_t* __restrict__ expert_counts,
                               int32_t* __restrict__ block_to_expert, int32_t* __restrict__ conditions,
                               int32_t* __restrict__ block_off, int32_t* __restrict__ count_off,
                               const TileOut& to, int* s_blk, int* s_cnt, int* s_cex, int* s_tile,
                               int* s_wave, long ids_bound = 1L << 30) {
  const int tid = threadIdx.x;
  const bool pack = SMALL && ids_bound < 65536;  // workgroup-uniform
  const int mt = to.mt, tpb = (to.tiles != nullptr) ? (B + mt - 1) / mt : 0;
  // tiles of expert tid: per block ceil(rows/mt) tiles (row tiles), or ceil(c_e/mt)
  // tiles running across the expert's blocks (block tiles, span = 1)
  auto tiles_of = [&](int c) {
    return to.span ? (c + mt - 1) / mt : (c / B) * tpb + (c % B + mt - 1) / mt;
  };
  int blk = 0, ntl = 0;
  if (tid < E) {
    if (expert_counts != nullptr) expert_counts[tid] = run;
    blk = (run + B - 1) / B;
    if (SMALL && to.tiles != nullptr) ntl = tiles_of(run);
  }
  int cum, tcum_small = 0, ccum_small = 0;
  const bool pack3 = pack && to.compact && ids_bound < 1024;  // workgroup-uniform
  if (pack3) {
    const int all = block_inclusive_sum(blk | (ntl << 10) | (run << 20), s_wave);
    cum = all & 0x3ff;
    tcum_small = (all >> 10) & 0x3ff;
    ccum_small = all >> 20;
  } else if (pack) {
    const int both = block_inclusive_sum(blk | (ntl << 16), s_wave);
    cum = both & 0xffff;
    tcum_small = both >> 16;
  } else {
    cum = block_inclusive_sum(blk, s_wave);
  }
  int cex = 0;
  if (tid < E) {
    if (block_off != nullptr) block_off[tid] = cum - blk;  // exclusive
    s_blk[tid] = cum;                                      // inclusive cumulative blocks
    s_cnt[tid] = run;
  }
  if (to.compact) {  // workgroup-uniform
    const int ccum = pack3 ? ccum_small : block_inclusive_sum(run, s_wave);
    cex = ccum - run;
    if (tid < E) {
      s_cex[tid] = cex;
      if (count_off != nullptr) count_off[tid] = cex;
    }
  }
  __syncthreads();
  const int total = s_blk[E - 1];
  // block_to_expert[b] = #{ e < E-1 : cum[e] <= b }   (cum non-decreasing): the
  // expert whose blocks [cum[e] - blk_e, cum[e]) hold b, and E - 1 from total on
  if (SMALL) {
    if (tid < E) {
      for (int b = cum - blk; b < cum && b < N; ++b) {
        block_to_expert[b] = tid;
        if (conditions != nullptr) conditions[b] = 1;
      }
    }
    for (int b = total + tid; b < N; b += blockDim.x) {
      block_to_expert[b] = E - 1;
      if (conditions != nullptr) conditions[b] = 0;
    }
  } else {
    for (int b = tid; b < N; b += blockDim.x) {
      int lo = 0, hi = E - 1;  // search in cum[0 .. E-2]
      while (lo < hi) {
        int mid = (lo + hi) >> 1;
        if (s_blk[mid] <= b) lo = mid + 1;
        else hi = mid;
      }
      block_to_expert[b] = lo;
      if (conditions != nullptr) conditions[b] = (b < total) ? 1 : 0;
    }
  }
  if (to.tiles == nullptr) return;  // workgroup-uniform
  // Tile list from the counts. Expert e owns slots [off_e*B, off_e*B + c_e),
  // so its tiles follow without reading token_position_to_id: per block
  // ceil(rows/mt) tiles (row tiles), or ceil(c_e/mt) tiles running across the
  // expert's blocks (block tiles, span = 1).
  int nt = ntl;
  if (!SMALL && tid < E) nt = tiles_of(run);
  const int tcum = pack ? tcum_small : block_inclusive_sum(nt, s_wave);
  if (tid < E) s_tile[tid] = tcum;
  __syncthreads();
  const int ntiles = s_tile[E - 1];
  // Tile i of expert e (local index loc): row tiles per block, or block tiles
  // sharing the expert's rows equally.
  auto put_tile = [&](int i, int e, int first, int loc, int c, int cum_e, int tcum_e, int cex_e) {
    const long base = (long)(cum_e - (c + B - 1) / B) * B;
    if (to.span) {
      // the expert's ceil(c / mt) tiles share its rows equally, so sibling tiles
      // advance through K at the same rate and share each weight block in L2
      const int ntl_e = tcum_e - first, h = (c + ntl_e - 1) / ntl_e;
      const long in_e = (long)loc * h;  // first slot of the tile, relative to the expert
      const long row = to.compact ? cex_e + in_e : base + in_e;
      to.tiles[i] = make_int4(e, (int)(base + in_e), min(h, c - loc * h), (int)row);
      to.seg[i] = make_int2(first, ntl_e);
    } else {
      const int j = loc / tpb, m = loc - j * tpb;
      const int rows = min(B, c - j * B);
      const long in_e = (long)j * B + m * mt;
      const long row = to.compact ? cex_e + in_e : base + in_e;
      to.tiles[i] = make_int4(e, (int)(base + in_e), min(mt, rows - m * mt), (int)row);
    }
  };
  if (SMALL) {
    if (tid < E) {
      const int first = tcum - nt;
      for (int i = first; i < tcum && i < to.max_tiles; ++i) put_tile(i, tid, first, i - first, run, cum, tcum, cex);
    }
  }
  for (int i = tid; !SMALL && i < ntiles && i < to.max_tiles; i += blockDim.x) {
    int lo = 0, hi = E - 1;  // first e with s_tile[e] > i
    while (lo < hi) {
      int mid = (lo + hi) >> 1;
      if (s_tile[mid] <= i) lo = mid + 1;
      else hi = mid;
    }
    const int e = lo, first = (e > 0) ? s_tile[e - 1] : 0;
    put_tile(i, e, first, i - first, s_cnt[e], s_blk[e], s_tile[e], to.compact ? s_cex[e] : 0);
  }
  const int per = (T + mt - 1) / mt;
  const int hsh = to.span ? (T + per - 1) / per : mt;  // equal block-tile heights
  const long nb_total = (long)N * B;
  const long row_sh = to.compact ? to.row_shared : nb_total;
  for (int i = tid; i < to.n_shared * per; i += blockDim.x) {
    const int j = i / per, m = i - j * per, idx = ntiles + i;
    if (idx < to.max_tiles) {
      const long in_sh = (long)j * T + (long)m * hsh;
      to.tiles[idx] = make_int4(E + j, (int)(nb_total + in_sh), min(hsh, T - m * hsh), (int)(row_sh + in_sh));
      if (to.span) to.seg[idx] = make_int2(ntiles + j * per, per);
    }
  }
  if (tid == 0) to.num_tiles[0] = min(ntiles + to.n_shared * per, to.max_tiles);
  if (to.span) {  // block tiles: the XCD ranges (the tile stores above are this workgroup's)
    __syncthreads();
    __threadfence_block();
    block_tile_cuts(to.tiles, min(ntiles + to.n_shared * per, to.max_tiles), to.max_tiles,
                    to.num_tiles, s_wave);
  }
}

// The whole mapping in one workgroup of 1024 threads, for ids and at most one
// 256-token chunk (decode): fill, bitmask, counts, scan, tiles and scatter. The LDS
// arrays hold E entries (bm: E rows of 8 words); s_wave holds 16. s_ids (optional):
// the T*K ids already in this workgroup's LDS.
static __device__ void map_small_body(const int32_t* __restrict__ ids, const int* s_ids, int T, int K,
                                      int E, int B, int N, int32_t* __restrict__ tpid,
                                      int32_t* __restrict__ block_to_expert,
                                      int32_t* __restrict__ conditions,
                                      int32_t* __restrict__ expert_counts,
                                      int32_t* __restrict__ inv_pos, const MapWs& ws,
                                      const TileOut& to, uint32_t (*bm)[8], int* s_blk, int* s_cnt,
                                      int* s_cex, int* s_tile, int* s_wave) {
  const int tid = threadIdx.x, nthr = blockDim.x;
  const int TK = T * K;
  const long nb_total = (long)N * B;
  // Up to 2 pairs per thread (i = tid + u * nthr) the ids live in registers, loaded
  // before this body stores anything: every later wait for them would also wait
  // for the stores issued before it (stores count in vmcnt), and no global load
  // follows the fill.
  const bool reg = TK <= 2 * nthr;  // workgroup-uniform
  int my_e[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int i = tid + u * nthr;
    my_e[u] = -1;
    if (reg && i < TK) my_e[u] = (s_ids != nullptr) ? s_ids[i] : ids[i];
  }
  auto fill = [&]() {
    long filled = 0;
    if (((uintptr_t)tpid & 15) == 0) {  // 16-byte stores while they fit
      filled = nb_total & ~3L;
      for (long i = tid; i < filled / 4; i += nthr) ((int4*)tpid)[i] = make_int4(-1, -1, -1, -1);
    }
    for (long i = filled + tid; i < nb_total; i += nthr) tpid[i] = -1;
  };
  if (reg) {
    // bitmask and count of ids >= E from the registers, then the fill; the
    // barriers below order the fill and the status store before the scatter
    for (int i = tid; i < E * 8; i += nthr) bm[i >> 3][i & 7] = 0u;
    if (tid == 0) s_wave[0] = 0;
    __syncthreads();
    int drop = 0;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int i = tid + u * nthr, e = my_e[u];
      if (i < TK) {
        const int tl = i / K;
        if (e >= 0 && e < E) atomicOr(&bm[e][tl >> 5], 1u << (tl & 31));
        else if (e >= E) ++drop;
      }
    }
    if (drop != 0) atomicAdd(&s_wave[0], drop);
    fill();
    __syncthreads();
    // s_wave[0] is next written by lane 63 of this same wave (the scans below)
    if (tid == 0) ws.status[0] = s_wave[0];
  } else {
    fill();
    if (tid == 0) ws.status[0] = 0;
    __syncthreads();  // the fill and the status reset land before the scatter below
    build_chunk_mask(bm, ids, nullptr, T, K, E, 0, ws.status);
  }
  int run = 0;
  if (tid < E) {
#pragma unroll
    for (int w = 0; w < 8; ++w) run += __popc(bm[tid][w]);
  }
  finish_mapping<true>(T, E, B, N, run, expert_counts, block_to_expert, conditions, ws.block_off,
                       nullptr, to, s_blk, s_cnt, s_cex, s_tile, s_wave, (long)T * K);
  auto scatter = [&](int i, int e) {
    const int t = i / K;
    int out = -1;
    if (e >= 0 && e < E) {
      int rank = 0;
      const int wq = t >> 5;
      for (int w = 0; w < wq; ++w) rank += __popc(bm[e][w]);
      rank += __popc(bm[e][wq] & ((1u << (t & 31)) - 1u));
      const long slot = (long)(s_blk[e] - (s_cnt[e] + B - 1) / B) * B + rank;
      if (slot < nb_total) {
        tpid[slot] = t;
        out = to.compact ? s_cex[e] + rank : (int)slot;
      } else {
        atomicAdd(ws.status, 1);
      }
    }
    if (inv_pos != nullptr) inv_pos[i] = out;
  };
  if (reg) {
#pragma unroll
    for (int u = 0; u < 2; ++u)
      if (tid + u * nthr < TK) scatter(tid + u * nthr, my_e[u]);
  } else {
    for (int i = tid; i < TK; i += nthr) scatter(i, ids[i]);
  }
}

// map_small_body's outputs for one token (T = 1) with row tiles (to.span == 0), with no
// barrier. The token's K ids (s_ids: 16-byte aligned LDS, K <= 64) are distinct experts
// or negative (the top-k selection names each expert at most once), so each selected
// expert e has one row, and with rank(e) = #{selected experts < e}: block rank(e), slot
// rank(e) * B holding token 0, compact row rank(e) and tile rank(e); blocks past the
// selected ones belong to E - 1 with condition 0, and the shared experts' tiles follow.
// Every thread scans the K ids and plays three parts: expert e = tid (E <= blockDim.x),
// pair k = tid and block b = tid (N <= T K <= 64); the waves then fill the slots block by
// block. Every output address is written once.
static __device__ void map_one_token(const int* s_ids, int K, int E, int B, int N,
                                     int32_t* __restrict__ tpid, int32_t* __restrict__ block_to_expert,
                                     int32_t* __restrict__ conditions,
                                     int32_t* __restrict__ expert_counts, int32_t* __restrict__ inv_pos,
                                     const MapWs& ws, const TileOut& to) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nwaves = blockDim.x >> 6;
  const int my = tid < K ? s_ids[tid] : -1;  // pair tid's expert
  int m = 0, dropped = 0, below = 0, rank = 0;
  bool mine = false;
  for (int k0 = 0; k0 < K; k0 += 4) {
    const int4 o4 = *(const int4*)(s_ids + k0);  // entries past K are not used
    const int o[4] = {o4.x, o4.y, o4.z, o4.w};
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const bool live = k0 + u < K;
      const bool ok = live && o[u] >= 0 && o[u] < E;
      m += ok ? 1 : 0;
      dropped += (live && o[u] >= E) ? 1 : 0;
      below += (ok && o[u] < tid) ? 1 : 0;
      rank += (ok && o[u] < my) ? 1 : 0;
      mine = mine || (ok && o[u] == tid);
    }
  }
  if (tid < E) {
    if (expert_counts != nullptr) expert_counts[tid] = mine ? 1 : 0;
    ws.block_off[tid] = below;
  }
  const bool sel = my >= 0 && my < E;  // false past K
  const bool fits = sel && rank < N;    // always, with N from moe_num_blocks; else dropped
  if (tid < K && inv_pos != nullptr) inv_pos[tid] = fits ? (to.compact ? rank : rank * B) : -1;
  if (fits) {
    block_to_expert[rank] = my;
    if (conditions != nullptr) conditions[rank] = 1;
  }
  if (tid >= m && tid < N) {
    block_to_expert[tid] = E - 1;
    if (conditions != nullptr) conditions[tid] = 0;
  }
  const long NB = (long)N * B;
  if (to.tiles != nullptr) {
    if (sel && rank < to.max_tiles) to.tiles[rank] = make_int4(my, rank * B, 1, to.compact ? rank : rank * B);
    const long row_sh = to.compact ? to.row_shared : NB;
    if (tid < to.n_shared && m + tid < to.max_tiles)
      to.tiles[m + tid] = make_int4(E + tid, (int)(NB + tid), 1, (int)(row_sh + tid));
    if (tid == 0) to.num_tiles[0] = min(m + to.n_shared, to.max_tiles);
  }
  const int unfit = (int)__popcll(__ballot(sel && !fits));  // pairs are threads 0..K-1: wave 0
  if (tid == 0) ws.status[0] = dropped + unfit;
  // slots, block by block: the first slot of block b < m holds token 0, the rest are empty
  const bool vec = ((uintptr_t)tpid & 15) == 0 && B % 4 == 0;  // uniform
  for (int b = wave; b < N; b += nwaves) {
    int32_t* blk = tpid + (long)b * B;
    const int first = b < m ? 0 : -1;
    if (vec) {
      for (int i = 4 * lane; i < B; i += 256) *(int4*)(blk + i) = make_int4(i == 0 ? first : -1, -1, -1, -1);
    } else {
      for (int i = lane; i < B; i += 64) blk[i] = i == 0 ? first : -1;
    }
  }
}

}  // namespace moe
