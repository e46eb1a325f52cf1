// C-ABI glue: error strings, version, and the whole-layer forward that chains
// the kernels on one stream with a caller-provided workspace.
#include <stdarg.h>
#include <stdio.h>

#include <mutex>

#include "moe_common.h"
#include "moe_internal.h"

namespace moe {

static thread_local char g_err[1024] = {0};

void set_error(const char* fn, const char* fmt, ...) {
  int n = snprintf(g_err, sizeof(g_err), "%s: ", fn);
  if (n < 0 || n >= (int)sizeof(g_err)) return;
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err + n, sizeof(g_err) - n, fmt, ap);
  va_end(ap);
}

void clear_error() { g_err[0] = 0; }

// Rows per expert tile (see use_block for the measurements): 16-row tiles up to 4
// routed rows per expert on average, 32 up to 24, 64 up to 48 (the MX layer, which
// has no block kernels, past 32), else 128.
static int choose_mt(int T, int K, int E) {
  long avg = ((long)T * std::min(K, E) + E - 1) / E;
  if (avg <= 4) return 16;
  if (avg <= 24) return 32;
  if (avg <= 48) return 64;
  return 128;
}

// The MX row-tile kernels stop at 64-row tiles: at 128 rows the MXFP4 form of the
// kernel spills registers, and larger tiles only save L2 reads of the weights.
static int choose_mt_mx(int T, int K, int E) { return std::min(choose_mt(T, K, E), 64); }

struct LayerWs {
  uint16_t* xn;  // normalized rows (bf16), when the layer normalizes
  float* logits;
  void* router_ws;
  size_t router_ws_bytes;
  int32_t* ids;
  float* weights;
  int32_t* tpid;
  int32_t* b2e;
  int32_t* cond;
  int32_t* counts;
  int32_t* inv;
  void* map_ws;
  size_t map_ws_bytes;
  uint8_t* xq;
  float* xs;
  int32_t* tiles;
  int32_t* num_tiles;
  uint8_t* hq;
  float* hs;
  uint16_t* y;
  int32_t* btiles;
  int32_t* bnum;
  size_t bytes;
};

// The 256x256 ("block") kernels take over above 32 rows per expert on average.
// Expert GEMM time (gate_up + down) on the DeepSeek-V3 layer by rows per expert,
// ms, row tiles of 16 / 32 / 64 rows against the block kernels: 4 rows 1.81 /
// 1.81 / 1.93 vs 2.05; 8: 1.95 / 1.92 / 2.08 vs 2.15; 16: 2.30 / 2.03 / 2.13 vs
// 2.29; 24: 2.78 / 2.11 / 2.19 vs 2.37; 32: 3.32 / 2.36 / 2.28 vs 2.42; 48: - /
// 2.95 / 2.47 vs 2.51; 64: - / 3.58 / 3.01 vs 2.60. On the Kimi-K2 layer at 42.7
// rows the block kernels lead (whole layer 3.90 against 3.95-4.00 ms), hence 32.
static bool use_block(int T, int K, int E) {
  return ((long)T * std::min(K, E) + E - 1) / E > 32;
}

static inline size_t al(size_t x) { return (x + 255) & ~(size_t)255; }

// Routed rows held by the layer's hq / y buffers: every routed (token, expert)
// pair has a row (packed expert by expert), then n_shared * T shared rows.
static inline long routed_rows(int T, int K, int E) { return (long)T * std::min(K, E); }

// Carves the workspace (base may be null to size it).
static LayerWs carve(char* base, int T, int H, int I, int E, int K, int n_sh, int B, bool norm) {
  LayerWs w{};
  const int N = moe_num_blocks(T, K, E, B);
  const long NB = (long)N * B;
  const long P = routed_rows(T, K, E) + (long)n_sh * T;
  // tile list sized for the smaller of the two layers' tile heights (more tiles)
  const int mt = choose_mt_mx(T, K, E);
  const int max_tiles = moe_max_tiles(T, K, E, N, B, n_sh, mt);
  size_t off = 0;
  auto take = [&](size_t bytes) -> char* {
    char* p = base ? base + off : nullptr;
    off += al(bytes);
    return p;
  };
  if (norm) w.xn = (uint16_t*)take((size_t)T * H * 2);
  w.logits = (float*)take((size_t)T * E * 4);
  w.router_ws_bytes = moe_router_logits_workspace_bytes(T, H, E);
  w.router_ws = take(w.router_ws_bytes);
  w.ids = (int32_t*)take((size_t)T * K * 4);
  w.weights = (float*)take((size_t)T * K * 4);
  w.tpid = (int32_t*)take((size_t)NB * 4);
  w.b2e = (int32_t*)take((size_t)N * 4);
  w.cond = (int32_t*)take((size_t)N * 4);
  w.counts = (int32_t*)take((size_t)E * 4);
  w.inv = (int32_t*)take((size_t)T * K * 4);
  w.map_ws_bytes = moe_mapping_workspace_bytes(T, E);
  w.map_ws = take(w.map_ws_bytes);
  w.xq = (uint8_t*)take((size_t)T * H);
  w.xs = (float*)take((size_t)T * (H / 128) * 4);
  w.tiles = (int32_t*)take((size_t)max_tiles * 16);
  w.num_tiles = (int32_t*)take(16);
  w.hq = (uint8_t*)take((size_t)P * I);
  w.hs = (float*)take((size_t)P * (I / 128) * 4);
  w.y = (uint16_t*)take((size_t)P * H * 2);
  if (use_block(T, K, E)) {
    const int mbt = moe_max_block_tiles(T, K, E, N, B, n_sh);
    w.btiles = (int32_t*)take((size_t)mbt * 24);
    w.bnum = (int32_t*)take(MOE_BLOCK_TILES_HEADER * 4);  // count + XCD ranges
  }
  w.bytes = off;
  return w;
}

}  // namespace moe

using namespace moe;

extern "C" int moe_abi_version(void) { return MOE_FP8_ABI_VERSION; }

extern "C" const char* moe_last_error(void) { return g_err; }

extern "C" size_t moe_layer_workspace_bytes(int T, int H, int I, int E, int K, int n_shared, int B,
                                            int norm) {
  if (T <= 0 || H <= 0 || I <= 0 || E <= 0 || K <= 0 || n_shared < 0 || B <= 0) return 0;
  return carve(nullptr, T, H, I, E, K, n_shared, B, norm != 0).bytes;
}

// RouterFuse for the layer's mapping (no quantization).
static RouterFuse map_fuse(const LayerWs& w, int B, int N, const TileOut& to) {
  RouterFuse fz{};
  fz.B = B;
  fz.N = N;
  fz.tpid = w.tpid;
  fz.b2e = w.b2e;
  fz.cond = w.cond;
  fz.counts = w.counts;
  fz.inv = w.inv;
  fz.map_ws = w.map_ws;
  fz.map_ws_bytes = w.map_ws_bytes;
  fz.to = to;
  return fz;
}

// The layer forward of both entry points: `workspace` is the caller's buffer or
// this device's static scratch. _moe_fn names the entry point in error messages.
static int layer_forward_impl(const char* _moe_fn, const void* x_bf16, const void* residual_bf16,
                              const float* gamma, float eps, int hidden_actual, int T, int H,
                              int I, int E, int K, int n_shared, const void* router_w_bf16,
                              const float* router_bias, const float* corr_bias, int order,
                              int scoring, int n_group, int topk_group, int renorm,
                              float renorm_eps, float routed_scale, const uint8_t* w13,
                              const float* w13_scale, const uint8_t* w2, const float* w2_scale,
                              const uint8_t* w13_shared, const float* w13_shared_scale,
                              const uint8_t* w2_shared, const float* w2_shared_scale, int B,
                              void* out_bf16, void* residual_out_bf16, int32_t* ids_out,
                              float* weights_out, float* logits_out, void* workspace,
                              size_t workspace_bytes, void* stream) {
  MOE_CHECK_ARG(x_bf16 && router_w_bf16 && w13 && w13_scale && w2 && w2_scale && out_bf16 && workspace,
                "null pointer argument");
  MOE_CHECK_ARG(T > 0 && E > 0 && K > 0 && K <= E && B > 0 && n_shared >= 0,
                "bad sizes T=%d E=%d K=%d B=%d", T, E, K, B);
  MOE_CHECK_ARG(H % 256 == 0 && I % 128 == 0, "H must be a multiple of 256 and I of 128");
  MOE_CHECK_ARG((residual_bf16 == nullptr) == (residual_out_bf16 == nullptr),
                "residual and residual_out must be given together");
  MOE_CHECK_ARG(gamma != nullptr || residual_bf16 == nullptr,
                "the residual add is fused into the norm: residual needs gamma");
  const bool norm = gamma != nullptr;
  const size_t need = moe_layer_workspace_bytes(T, H, I, E, K, n_shared, B, norm);
  MOE_CHECK_ARG(workspace_bytes >= need, "workspace too small: need %zu bytes, got %zu", need,
                workspace_bytes);
  MOE_CHECK_ARG(((uintptr_t)workspace & 255) == 0, "workspace must be 256-byte aligned");
  LayerWs w = carve((char*)workspace, T, H, I, E, K, n_shared, B, norm);
  const int N = moe_num_blocks(T, K, E, B);
  const long NB = (long)N * B;
  const long R = routed_rows(T, K, E);
  MOE_CHECK_SUPPORTED(NB + (long)n_shared * T < (1L << 31), "too many slots");
  const int mt = choose_mt(T, K, E);
  const int max_tiles = moe_max_tiles(T, K, E, N, B, n_shared, mt);
  float* logits = logits_out ? logits_out : w.logits;
  int32_t* ids = ids_out ? ids_out : w.ids;
  float* wts = weights_out ? weights_out : w.weights;

  char saved[1024];
  int rc;
#define MOE_STEP(call)                                         \
  rc = (call);                                                 \
  if (rc != MOE_OK) {                                          \
    snprintf(saved, sizeof(saved), "%s", moe_last_error());    \
    moe::set_error(_moe_fn, "%s", saved);                      \
    return rc;                                                 \
  }
  // The mapping also writes the expert tile list, from the counts.
  const bool block = use_block(T, K, E);
  const int mbt = block ? moe_max_block_tiles(T, K, E, N, B, n_shared) : 0;
  TileOut to{};
  if (block) {
    to.tiles = (int4*)w.btiles;
    to.seg = (int2*)(w.btiles + 4 * (size_t)mbt);
    to.num_tiles = w.bnum;
    to.max_tiles = mbt;
    to.mt = kBlockTileRows;
    to.span = 1;
  } else {
    to.tiles = (int4*)w.tiles;
    to.num_tiles = w.num_tiles;
    to.max_tiles = max_tiles;
    to.mt = mt;
  }
  to.n_shared = n_shared;
  to.compact = 1;  // hq / y hold only the routed and shared rows
  to.row_shared = R;
  // Pre-MoE RMSNorm (with the residual add) and the 1x128 quantization of the
  // normalized rows: up to a few tokens inside the logits launch, else in one pass
  // before it (router_logits_topk). Decode sizes: the quantization rides in the
  // logits launch and the mapping ends the top-k launch (router_logits_topk says
  // which it did).
  RouterFuse fz = map_fuse(w, B, N, to);
  fz.xq = w.xq;
  fz.xs = w.xs;
  if (norm) {
    fz.norm = NormRide{(const uint16_t*)residual_bf16, gamma, (uint16_t*)residual_out_bf16,
                       hidden_actual > 0 ? hidden_actual : H, eps};
    fz.xn = w.xn;
  }
  MOE_STEP(router_logits_topk(x_bf16, router_w_bf16, router_bias, T, H, E, logits, w.router_ws,
                              w.router_ws_bytes, corr_bias, K, order, scoring, n_group, topk_group,
                              renorm, renorm_eps, routed_scale, ids, wts, stream, &fz));
  if (!fz.map_done)
    MOE_STEP(blockwise_mapping(ids, nullptr, nullptr, T, K, E, B, N, w.tpid, w.b2e, w.cond, w.counts,
                               w.inv, nullptr, w.map_ws, w.map_ws_bytes, to, stream));
  // (with the norm the quantization is always done: in the logits launch or by the norm)
  if (!fz.quant_done) MOE_STEP(moe_act_quant_1x128(x_bf16, T, H, w.xq, w.xs, stream));
  if (block) {
    MOE_STEP(moe_expert_gate_up_block(w.xq, w.xs, T, H, I, E, w13, w13_scale, nullptr, w13_shared,
                                      w13_shared_scale, nullptr, n_shared, w.tpid, (int)NB, w.btiles,
                                      w.bnum, mbt, w.hq, w.hs, stream));
    MOE_STEP(moe_expert_down_block(w.hq, w.hs, T, H, I, E, w2, w2_scale, nullptr, w2_shared,
                                   w2_shared_scale, nullptr, n_shared, (int)NB, w.btiles, w.bnum, mbt,
                                   w.y, stream));
  } else {
    MOE_STEP(layer_gate_up(w.xq, w.xs, T, H, I, E, w13, w13_scale, w13_shared, w13_shared_scale,
                           n_shared, w.tpid, (int)NB, w.tiles, w.num_tiles, max_tiles, mt, w.hq, w.hs,
                           stream));
    MOE_STEP(moe_expert_down(w.hq, w.hs, T, H, I, E, w2, w2_scale, nullptr, w2_shared,
                             w2_shared_scale, nullptr, n_shared, (int)NB, w.tiles, w.num_tiles,
                             max_tiles, mt, w.y,
                             stream));
  }
  MOE_STEP(moe_combine(w.y, w.inv, wts, K, T, H, (int)R, n_shared, out_bf16, stream));
#undef MOE_STEP
  return MOE_OK;
}

extern "C" int moe_layer_forward(const void* x_bf16, const void* residual_bf16,
                                 const float* gamma, float eps, int hidden_actual, int T, int H,
                                 int I, int E, int K, int n_shared, const void* router_w_bf16,
                                 const float* router_bias, const float* corr_bias, int order,
                                 int scoring, int n_group, int topk_group, int renorm,
                                 float renorm_eps, float routed_scale, const uint8_t* w13,
                                 const float* w13_scale, const uint8_t* w2, const float* w2_scale,
                                 const uint8_t* w13_shared, const float* w13_shared_scale,
                                 const uint8_t* w2_shared, const float* w2_shared_scale, int B,
                                 void* out_bf16, void* residual_out_bf16, int32_t* ids_out,
                                 float* weights_out, float* logits_out, void* workspace,
                                 size_t workspace_bytes, void* stream) {
  MOE_API_BEGIN("moe_layer_forward");
  return layer_forward_impl(_moe_fn, x_bf16, residual_bf16, gamma, eps, hidden_actual, T, H, I, E,
                            K, n_shared, router_w_bf16, router_bias, corr_bias, order, scoring,
                            n_group, topk_group, renorm, renorm_eps, routed_scale, w13, w13_scale,
                            w2, w2_scale, w13_shared, w13_shared_scale, w2_shared,
                            w2_shared_scale, B, out_bf16, residual_out_bf16, ids_out, weights_out,
                            logits_out, workspace, workspace_bytes, stream);
}

// ---------------------------------------------------------------------------
// Allocation-free layer forward. Its workspace is `scratch`, one static array per
// GPU that the code object's loader places in device memory and that lives until
// the process ends. In host code `scratch` names a host-side shadow, not device
// memory, so its device address is looked up once per device with
// hipGetSymbolAddress (with that device current) and only that address is handed
// to kernels. Calls on one GPU share the array: they must not overlap (same
// stream or otherwise ordered), and nothing in it has to start at zero (every
// kernel of the layer writes what it later reads; the mapping clears its own
// status word).
// ---------------------------------------------------------------------------
static __device__ __align__(256) uint8_t scratch[MOE_NOALLOC_SCRATCH_BYTES];

namespace moe {

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_dev[kMaxDevices];

// Device address of this device's `scratch` (looked up on the first call per device).
static int scratch_address(const char* _moe_fn, void** out) {
  int dev = -1;
  MOE_CHECK_HIP(hipGetDevice(&dev));
  MOE_CHECK_SUPPORTED(dev >= 0 && dev < kMaxDevices, "device %d beyond %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_dev[dev] == nullptr) {
    void* p = nullptr;
    MOE_CHECK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    MOE_CHECK_ARG(p != nullptr && ((uintptr_t)p & 255) == 0, "bad scratch address");
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return MOE_OK;
}

}  // namespace moe

extern "C" int moe_layer_forward_noalloc(
    const void* x_bf16, const void* residual_bf16, const float* gamma, float eps,
    int hidden_actual, int T, int H, int I, int E, int K, int n_shared, const void* router_w_bf16,
    const float* router_bias, const float* corr_bias, int order, int scoring, int n_group,
    int topk_group, int renorm, float renorm_eps, float routed_scale, const uint8_t* w13,
    const float* w13_scale, const uint8_t* w2, const float* w2_scale, const uint8_t* w13_shared,
    const float* w13_shared_scale, const uint8_t* w2_shared, const float* w2_shared_scale, int B,
    void* out_bf16, void* residual_out_bf16, int32_t* ids_out, float* weights_out,
    float* logits_out, void* stream) {
  MOE_API_BEGIN("moe_layer_forward_noalloc");
  MOE_CHECK_ARG(T > 0 && H > 0 && I > 0 && E > 0 && K > 0 && B > 0 && n_shared >= 0,
                "bad sizes T=%d H=%d I=%d E=%d K=%d B=%d", T, H, I, E, K, B);
  const size_t need = moe_layer_workspace_bytes(T, H, I, E, K, n_shared, B, gamma != nullptr);
  MOE_CHECK_SUPPORTED(need <= (size_t)MOE_NOALLOC_SCRATCH_BYTES,
                      "this layer call needs %zu bytes of scratch; the static scratch holds %zu "
                      "(use moe_layer_forward with a workspace)",
                      need, (size_t)MOE_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  const int rc = scratch_address(_moe_fn, &ws);
  if (rc != MOE_OK) return rc;
  return layer_forward_impl(_moe_fn, x_bf16, residual_bf16, gamma, eps, hidden_actual, T, H, I, E,
                            K, n_shared, router_w_bf16, router_bias, corr_bias, order, scoring,
                            n_group, topk_group, renorm, renorm_eps, routed_scale, w13, w13_scale,
                            w2, w2_scale, w13_shared, w13_shared_scale, w2_shared,
                            w2_shared_scale, B, out_bf16, residual_out_bf16, ids_out, weights_out,
                            logits_out, ws, (size_t)MOE_NOALLOC_SCRATCH_BYTES, stream);
}

// ---------------------------------------------------------------------------
// The layer with MX experts (GPT-OSS): [residual add ->] [RMSNorm ->] router ->
// top-k -> mapping (compact rows) -> MXFP8 quantization -> MX gate_up (bias,
// clamps, activation) -> MX down (bias) -> combine. Same workspace as
// moe_layer_forward without shared experts (the MX scale bytes take the room of
// the 1x128 fp32 scales).
// ---------------------------------------------------------------------------
extern "C" int moe_layer_forward_mx(
    const void* x_bf16, const void* residual_bf16, const float* gamma, float eps,
    int hidden_actual, int T, int H, int I, int E, int K, const void* router_w_bf16,
    const float* router_bias, int order, int scoring, int renorm, float renorm_eps,
    float routed_scale, int wfmt, const uint8_t* w13, const uint8_t* w13_scale, const float* b13,
    const uint8_t* w2, const uint8_t* w2_scale, const float* b2, int act, float gate_lo,
    float gate_hi, float up_lo, float up_hi, int B, void* out_bf16, void* residual_out_bf16,
    int32_t* ids_out, float* weights_out, float* logits_out, void* workspace,
    size_t workspace_bytes, void* stream) {
  MOE_API_BEGIN("moe_layer_forward_mx");
  MOE_CHECK_ARG(x_bf16 && router_w_bf16 && w13 && w13_scale && w2 && w2_scale && out_bf16 && workspace,
                "null pointer argument");
  MOE_CHECK_ARG(T > 0 && E > 0 && K > 0 && K <= E && B > 0, "bad sizes T=%d E=%d K=%d B=%d", T, E,
                K, B);
  MOE_CHECK_ARG(H % 256 == 0 && I % 128 == 0, "H must be a multiple of 256 and I of 128 (pad them)");
  MOE_CHECK_ARG(order == MOE_ORDER_TOPK_ACT || order == MOE_ORDER_ACT_TOPK,
                "the MX layer routes with the TOPK_ACT or ACT_TOPK order");
  MOE_CHECK_ARG((residual_bf16 == nullptr) == (residual_out_bf16 == nullptr),
                "residual and residual_out must be given together");
  MOE_CHECK_ARG(gamma != nullptr || residual_bf16 == nullptr,
                "the residual add is fused into the norm: residual needs gamma");
  const bool norm = gamma != nullptr;
  const size_t need = moe_layer_workspace_bytes(T, H, I, E, K, 0, B, norm);
  MOE_CHECK_ARG(workspace_bytes >= need, "workspace too small: need %zu bytes, got %zu", need,
                workspace_bytes);
  MOE_CHECK_ARG(((uintptr_t)workspace & 255) == 0, "workspace must be 256-byte aligned");
  LayerWs w = carve((char*)workspace, T, H, I, E, K, 0, B, norm);
  const int N = moe_num_blocks(T, K, E, B);
  const long NB = (long)N * B;
  const long R = routed_rows(T, K, E);
  MOE_CHECK_SUPPORTED(NB < (1L << 31), "too many slots");
  const int mt = choose_mt_mx(T, K, E);
  const int max_tiles = moe_max_tiles(T, K, E, N, B, 0, mt);
  float* logits = logits_out ? logits_out : w.logits;
  int32_t* ids = ids_out ? ids_out : w.ids;
  float* wts = weights_out ? weights_out : w.weights;
  uint8_t* xs = (uint8_t*)w.xs;  // T * H/32 bytes of E8M0 scales
  uint8_t* hs = (uint8_t*)w.hs;  // P * I/32 bytes

  char saved[1024];
  int rc;
#define MOE_STEP(call)                                         \
  rc = (call);                                                 \
  if (rc != MOE_OK) {                                          \
    snprintf(saved, sizeof(saved), "%s", moe_last_error());    \
    moe::set_error(_moe_fn, "%s", saved);                      \
    return rc;                                                 \
  }
  TileOut to{};
  to.tiles = (int4*)w.tiles;
  to.num_tiles = w.num_tiles;
  to.max_tiles = max_tiles;
  to.mt = mt;
  to.compact = 1;
  to.row_shared = R;
  // Residual add + RMSNorm: up to a few tokens inside the logits launch, else in a
  // pass of its own before it (whose 1x128 codes land in xq and are replaced below).
  // Decode sizes: the MXFP8 quantization rides in the logits launch and the
  // mapping ends the top-k launch (router_logits_topk says which it did).
  RouterFuse fz = map_fuse(w, B, N, to);
  fz.xq = w.xq;
  fz.xs = xs;
  fz.quant_mx = 1;
  if (norm) {
    fz.norm = NormRide{(const uint16_t*)residual_bf16, gamma, (uint16_t*)residual_out_bf16,
                       hidden_actual > 0 ? hidden_actual : H, eps};
    fz.xn = w.xn;
  }
  const void* xr = norm ? w.xn : x_bf16;  // what the router read, unless the norm rode
  MOE_STEP(router_logits_topk(x_bf16, router_w_bf16, router_bias, T, H, E, logits, w.router_ws,
                              w.router_ws_bytes, nullptr, K, order, scoring, 1, 1, renorm,
                              renorm_eps, routed_scale, ids, wts, stream, &fz));
  if (!fz.map_done)
    MOE_STEP(blockwise_mapping(ids, nullptr, nullptr, T, K, E, B, N, w.tpid, w.b2e, w.cond, w.counts,
                               w.inv, nullptr, w.map_ws, w.map_ws_bytes, to, stream));
  if (!fz.quant_done) MOE_STEP(moe_act_quant_mx(xr, T, H, w.xq, xs, stream));
  MOE_STEP(layer_gate_up_mx(w.xq, xs, T, H, I, E, wfmt, w13, w13_scale, b13, nullptr, nullptr,
                            nullptr, 0, w.tpid, (int)NB, w.tiles, w.num_tiles, max_tiles, mt, act,
                            gate_lo, gate_hi, up_lo, up_hi, w.hq, hs, stream));
  bool fused = false;
  MOE_STEP(layer_down_combine_mx(w.hq, hs, T, H, I, E, K, wfmt, w2, w2_scale, b2, ids, w.inv, wts,
                                 out_bf16, stream, &fused));
  if (!fused) {
    MOE_STEP(layer_down_mx(w.hq, hs, T, H, I, E, wfmt, w2, w2_scale, b2, nullptr, nullptr, nullptr,
                           0, (int)NB, w.tiles, w.num_tiles, max_tiles, mt, w.y, stream));
    MOE_STEP(moe_combine(w.y, w.inv, wts, K, T, H, (int)R, 0, out_bf16, stream));
  }
#undef MOE_STEP
  return MOE_OK;
}
