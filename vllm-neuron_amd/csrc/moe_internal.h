// Host-side plumbing shared by the C-ABI entry points: error strings, argument
// checks and launch-shape helpers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <algorithm>

#include "moe_fp8.h"

namespace moe {

void set_error(const char* fn, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

// K splits for the router logits GEMM: aim for >= 1024 workgroups (4 per CU
// fit, and the loop is latency-bound), each split at least 256 columns of H.
inline int router_logits_splits(int T, int H, int E) {
  long base = (long)((T + 63) / 64) * ((E + 63) / 64);
  long ks = (1024 + base - 1) / base;
  long kmax = std::max(1, H / 256);
  return (int)std::max(1L, std::min(ks, kmax));
}


// Rows per tile of the 256x256 expert GEMM kernels.
constexpr int kBlockTileRows = 256;

// Compute units of the current device (cached per device; 256 on MI355X), for
// persistent grids of one workgroup per CU.
inline int device_cu_count() {
  constexpr int kMaxDev = 64;
  static int cached[kMaxDev];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) return 256;
  int n = __atomic_load_n(&cached[dev], __ATOMIC_RELAXED);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    __atomic_store_n(&cached[dev], n, __ATOMIC_RELAXED);
  }
  return n;
}

// Tile list written by the mapping's scan kernel from the expert counts
// (tiles == nullptr: none). Row tiles stay inside one block; block tiles
// (span = 1) run across an expert's blocks and carry seg = (first tile of the
// expert, its tile count). Shared-expert tiles follow the routed ones.
// A tile is {expert, first slot, rows, first hq / y row}. With compact = 0 the
// rows are the slots themselves; with compact = 1 the routed rows are packed
// expert after expert (expert e's i-th slot is row sum_{e' < e} count_e' + i),
// the shared expert j's token t is row row_shared + j * T + t, and inv_pos
// receives these rows instead of slots.
struct TileOut {
  int4* tiles;
  int2* seg;
  int32_t* num_tiles;
  int max_tiles;
  int mt;
  int span;
  int n_shared;
  int compact;
  long row_shared;
};

// The pre-MoE RMSNorm of the layer's rows (with gamma set): v = x, or bf16(x +
// residual) written to res_out as the next residual stream; the rows normalized
// over their first ha columns.
struct NormRide {
  const uint16_t* res;
  const float* gamma;
  uint16_t* res_out;
  int ha;
  float eps;
};

// Up to this many tokens the norm rides in the router logits launch: every
// workgroup of that launch reads the token rows and computes their norm factors
// itself (at most 16384 columns).
constexpr int kNormRideT = 4;
constexpr int kNormRideMaxH = 16384;

// Work that router_logits_topk may fold into its launches for the layer: the
// quantization of x into xq / xs (when xq is set: 1x128 fp8 codes and fp32 scales,
// or with quant_mx MXFP8 codes and E8M0 scale bytes) and blockwise_mapping of the
// ids it selects (when tpid is set; ids only, no padding mask, inv_pos = inv,
// workspace map_ws, tile list `to`). With norm.gamma set, x is normalized first:
// inside the logits launch where it can ride (then the quantization rides too),
// otherwise by moe_rms_norm_quant into xn (its 1x128 codes land in xq / xs), which
// the router then reads. On return quant_done / map_done say which it did; the
// caller runs the rest itself (from xn when the norm was requested).
struct RouterFuse {
  uint8_t* xq;
  void* xs;
  int quant_mx;
  NormRide norm;
  void* xn;
  int B, N;
  int32_t *tpid, *b2e, *cond, *counts, *inv;
  void* map_ws;
  size_t map_ws_bytes;
  TileOut to;
  bool quant_done, map_done;
};

// moe_router_logits followed by moe_router_topk (no affinities output), with the
// split-K reduce folded into the top-k kernel; for callers that already checked
// the arguments of both.
int router_logits_topk(const void* x_bf16, const void* w_bf16, const float* bias, int T, int H,
                       int E, float* logits, void* workspace, size_t workspace_bytes,
                       const float* corr_bias, int K, int order, int scoring, int n_group,
                       int topk_group, int renorm, float renorm_eps, float routed_scale,
                       int32_t* ids, float* weights, void* stream, RouterFuse* fuse = nullptr);

// moe_expert_gate_up for the layer, whose tiles its own mapping wrote: at one token
// every slot of a tile holds token 0, and the kernel loads no token ids.
int layer_gate_up(const uint8_t* xq, const float* xs, int T, int H, int I, int E, const uint8_t* w13,
                  const float* w13_scale, const uint8_t* w13_shared, const float* w13_shared_scale,
                  int n_shared, const int32_t* tpid, int NB, const int32_t* tiles,
                  const int32_t* num_tiles, int max_tiles, int mt, uint8_t* hq, float* hs,
                  void* stream);

// moe_expert_gate_up_mx / moe_expert_down_mx for the layer, whose tiles its own
// mapping wrote: at one token (one row per tile, token 0) the MXFP4 GEMMs with K =
// 3072 load each wave's fragments for the whole K into registers at once.
int layer_gate_up_mx(const uint8_t* xq, const uint8_t* xs, int T, int H, int I, int E, int wfmt,
                     const uint8_t* w13, const uint8_t* w13_scale, const float* b13,
                     const uint8_t* w13_shared, const uint8_t* w13_shared_scale,
                     const float* b13_shared, int n_shared, const int32_t* token_position_to_id,
                     int NB, const int32_t* tiles, const int32_t* num_tiles, int max_tiles, int mt,
                     int act, float gate_lo, float gate_hi, float up_lo, float up_hi, uint8_t* hq,
                     uint8_t* hs, void* stream);
int layer_down_mx(const uint8_t* hq, const uint8_t* hs, int T, int H, int I, int E, int wfmt,
                  const uint8_t* w2, const uint8_t* w2_scale, const float* b2,
                  const uint8_t* w2_shared, const uint8_t* w2_shared_scale, const float* b2_shared,
                  int n_shared, int NB, const int32_t* tiles, const int32_t* num_tiles,
                  int max_tiles, int mt, void* y_bf16, void* stream);

// moe_expert_down_mx followed by moe_combine (no shared experts) in one launch for the
// layer at one token with MXFP4 w2 and I = 3072 (K <= 8 pairs; ids, inv and weights of
// the token's pairs, inv the compact rows of hq): the same output bits without the y
// rows. *done says whether it ran; otherwise the caller runs both.
int layer_down_combine_mx(const uint8_t* hq, const uint8_t* hs, int T, int H, int I, int E, int K,
                          int wfmt, const uint8_t* w2, const uint8_t* w2_scale, const float* b2,
                          const int32_t* ids, const int32_t* inv, const float* weights,
                          void* out_bf16, void* stream, bool* done);

// moe_blockwise_mapping plus an optional tile list (same checks and errors).
int blockwise_mapping(const int32_t* ids, const float* affinities, const uint8_t* padding_mask,
                      int T, int K, int E, int B, int N, int32_t* token_position_to_id,
                      int32_t* block_to_expert, int32_t* conditions, int32_t* expert_counts,
                      int32_t* inv_pos, float* affinities_masked, void* workspace,
                      size_t workspace_bytes, const TileOut& to, void* stream);

}  // namespace moe

#define MOE_API_BEGIN(name)   \
  const char* _moe_fn = name; \
  moe::clear_error();

#define MOE_CHECK_ARG(cond, ...)            \
  do {                                      \
    if (!(cond)) {                          \
      moe::set_error(_moe_fn, __VA_ARGS__); \
      return MOE_ERR_ARG;                   \
    }                                       \
  } while (0)

#define MOE_CHECK_SUPPORTED(cond, ...)      \
  do {                                      \
    if (!(cond)) {                          \
      moe::set_error(_moe_fn, __VA_ARGS__); \
      return MOE_ERR_UNSUPPORTED;           \
    }                                       \
  } while (0)

#define MOE_CHECK_HIP(expr)                                                              \
  do {                                                                                   \
    hipError_t _e = (expr);                                                              \
    if (_e != hipSuccess) {                                                              \
      moe::set_error(_moe_fn, "%s failed: %s", #expr, hipGetErrorString(_e));            \
      return MOE_ERR_HIP;                                                                \
    }                                                                                    \
  } while (0)

#define MOE_API_END()                                                                    \
  do {                                                                                   \
    hipError_t _e = hipGetLastError();                                                   \
    if (_e != hipSuccess) {                                                              \
      moe::set_error(_moe_fn, "kernel launch failed: %s", hipGetErrorString(_e));        \
      return MOE_ERR_HIP;                                                                \
    }                                                                                    \
    return MOE_OK;                                                                       \
  } while (0)
