/*
 * moe_fp8.h - C ABI of the MI355X (gfx950) FP8-blockwise fused-MoE layer.
 *
 * Every entry point takes plain device pointers and sizes, enqueues its work
 * on the given HIP stream (a hipStream_t passed as void*, NULL = the default
 * stream) and returns immediately: MOE_OK (0) or a negative status whose
 * message moe_last_error() returns (thread-local). No entry point allocates
 * or frees device memory; callers pass outputs and a workspace sized by the
 * matching *_workspace_bytes function. Functions are re-entrant; calls on
 * different streams may run concurrently as long as they do not share a
 * workspace.
 *
 * Tensor layouts (row-major, C order):
 *   x            [T, H]      bf16 hidden states
 *   router_w     [E, H]      bf16 router weight (the HF / reference parameter,
 *                            whose transpose the reference passes as [H, E])
 *   w13          [E, 2I, H]  e4m3fn codes, gate rows [0, I) then up rows [I, 2I)
 *   w13_scale    [E, 2I/128, H/128]  fp32 block scale (checkpoint weight_scale_inv)
 *   w2           [E, H, I]   e4m3fn codes
 *   w2_scale     [E, H/128, I/128]   fp32 block scale
 *   shared-expert tensors: the same per expert, n_shared experts of intermediate I
 *
 * The reference interface each function replaces is cited beside it
 * (paths inside jinhuang12/vllm-neuron).
 */
#ifndef MOE_FP8_H
#define MOE_FP8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOE_FP8_ABI_VERSION 3

/* status codes */
#define MOE_OK 0
#define MOE_ERR_ARG (-1)         /* bad argument / shape (reference: ValueError)              */
#define MOE_ERR_UNSUPPORTED (-2) /* valid but unsupported config (reference: NotImplementedError) */
#define MOE_ERR_HIP (-3)         /* HIP runtime / launch failure (reference: RuntimeError)    */

/* router computation orders (router.py:19-69 RouterComputationOrder, plus grouped) */
#define MOE_ORDER_TOPK_ACT 0 /* linear -> topk -> act on the k values     (router.py:384-441) */
#define MOE_ORDER_ACT_TOPK 1 /* linear -> act on all E -> topk (-> renorm) (router.py:444-504) */
#define MOE_ORDER_GROUPED 2  /* DeepSeek-V3 grouped top-k with selection-only correction bias */

/* router activation (RouterActFnType) */
#define MOE_SCORING_SOFTMAX 0
#define MOE_SCORING_SIGMOID 1

int moe_abi_version(void);
const char* moe_last_error(void);

/* ---- router ------------------------------------------------------------- */

/* logits[T,E] = x[T,H] . router_w[E,H]^T (+ bias[E]); bf16 operands, fp32
 * accumulation. Replaces the F.linear of router.py:419-424 (and the disabled
 * nkilib router_topk call, router.py:774-795). H % 64 == 0. */
size_t moe_router_logits_workspace_bytes(int T, int H, int E);
int moe_router_logits(const void* x_bf16, const void* router_w_bf16, const float* bias, int T,
                      int H, int E, float* logits, void* workspace, size_t workspace_bytes,
                      void* stream);

/* The same product with fp32 hidden states (router_w fp32 if w_is_f32, else
 * bf16; [E,H]); fp32 v_mfma_f32_16x16x4f32, fp32 accumulation. For router()
 * when its operands are not bf16-exact: router.py:236 casts hidden_states to
 * the fp32 computation dtype before the optional RMSNorm (router.py:409-410),
 * so F.linear (router.py:418-424) sees fp32 operands. Workspace size as
 * moe_router_logits_workspace_bytes. H % 64 == 0. */
int moe_router_logits_f32(const float* x, const void* router_w, int w_is_f32, const float* bias,
                          int T, int H, int E, float* logits, void* workspace,
                          size_t workspace_bytes, void* stream);

/* RMSNorm over rows of x [T,H] (bf16, or fp32 if x_is_f32):
 * y = (x * 1/sqrt(mean(x[:hidden_actual]^2) + eps)) * gamma for columns <
 * hidden_actual, 0 beyond; fp32 math, out bf16 (or fp32 if out_is_f32).
 * gamma fp32 [H]. Replaces _torch_rms_norm (router.py:681-688) and the
 * RMSNorm step of moe_block_tkg (moe_block_tkg.py:135-151). */
int moe_rms_norm(const void* x, int x_is_f32, const float* gamma, int T, int H, int hidden_actual,
                 float eps, void* out, int out_is_f32, void* stream);

/* Decode prologue, fused: v = x (or bf16(x + residual) when residual is given,
 * written to residual_out as the next residual stream), xn = RMSNorm(v) exactly
 * as moe_rms_norm with bf16 output, and q/s = the 1x128 e4m3fn quantization of
 * xn exactly as moe_act_quant_1x128. All bf16 [T,H]; q [T,H]; s fp32 [T,H/128].
 * H % 128 == 0. Replaces the RMSNorm step of moe_block_tkg (moe_block_tkg.py:
 * 135-151) with its fused residual add (moe_block_tkg.py:341,421-428; the
 * pre-norm sum model_mxfp4.py:1589-1609) and the norm + quantize prologue of
 * rmsnorm_router_topk_tkg.py:247-343. */
int moe_rms_norm_quant(const void* x_bf16, const void* residual_bf16, const float* gamma, int T,
                       int H, int hidden_actual, float eps, void* xn_bf16, void* residual_out_bf16,
                       uint8_t* q, float* s, void* stream);

/* Top-k selection + activation (+ renorm, * routed_scale) from fp32 logits.
 * ids/weights [T,K] in descending key order (ties -> lower expert index);
 * affinities [T,E] (optional, NULL to skip) is the dense scatter the reference
 * returns (router.py:437-441). corr_bias [E] (optional) is used by
 * MOE_ORDER_GROUPED for selection only. renorm != 0 divides by
 * (sum_k w + renorm_eps). E <= 1024, K <= 64.
 * Replaces router.py:384-566 and moe_block_tkg.py:165-205. */
int moe_router_topk(const float* logits, const float* corr_bias, int T, int E, int K, int order,
                    int scoring, int n_group, int topk_group, int renorm, float renorm_eps,
                    float routed_scale, int32_t* ids, float* weights, float* affinities,
                    void* stream);

/* ---- blockwise (align-by-expert) mapping -------------------------------- */

/* N = min(ceil((T*min(K,E) - (E-1)) / B) + E - 1, T*min(K,E))  (moe_blockwise.py:376-382) */
int moe_num_blocks(int T, int K, int E, int B);
size_t moe_mapping_workspace_bytes(int T, int E);

/* Builds the reference mapping (moe_blockwise.py:25-157, torch flow :325-437):
 * token_position_to_id [N*B] (token id or -1), block_to_expert [N],
 * conditions [N], plus expert_counts [E].
 * Input is either ids [T,K] (each row distinct experts, -1 = unused slot) or
 * affinities [T,E] (selected where != 0). With ids, inv_pos [T,K] (optional)
 * receives the slot of (t, ids[t,k]). With affinities, affinities_masked
 * [T*E] (optional) receives affinities * padding_mask (padding_mask [T] bytes,
 * optional, nonzero = real token; moe_blockwise.py:480-498).
 * Out-of-range ids or more routed pairs than N*B holds are dropped and counted
 * in the workspace status word (moe_mapping_status). */
int moe_blockwise_mapping(const int32_t* ids, const float* affinities, const uint8_t* padding_mask,
                          int T, int K, int E, int B, int N, int32_t* token_position_to_id,
                          int32_t* block_to_expert, int32_t* conditions, int32_t* expert_counts,
                          int32_t* inv_pos, float* affinities_masked, void* workspace,
                          size_t workspace_bytes, void* stream);

/* Synchronizes `stream` and returns, in *dropped, the number of routed pairs
 * the last moe_blockwise_mapping on this workspace had to drop (0 = valid). */
int moe_mapping_status(const void* workspace, void* stream, int* dropped);

/* inv[T,E] = slot of (t, e) in token_position_to_id, -1 if (t, e) is not
 * routed. Used when a caller hands moe_cte a mapping built elsewhere
 * (moe_cte.py:35-94 receives only token_position_to_id / block_to_expert). */
int moe_invert_mapping(const int32_t* token_position_to_id, const int32_t* block_to_expert, int N,
                       int B, int T, int E, int32_t* inv, void* stream);

/* ---- fp8 activation quantization --------------------------------------- */

/* Per row, per 128 columns: s = max(amax, 1e-10) / 448, q = RNE_e4m3fn(clamp(x/s, +-448)).
 * No reference counterpart on a CPU path (closest: the MX activation quantizer
 * of rmsnorm_router_topk_tkg.py:288-343). cols % 128 == 0. */
int moe_act_quant_1x128(const void* x_bf16, int rows, int cols, uint8_t* q, float* scales,
                        void* stream);

/* ---- expert row tiles ---------------------------------------------------- */

/* A tile is {expert, first slot, rows, first row} (int32 x4): at most `mt`
 * consecutive slots of one block of token_position_to_id; shared experts
 * j < n_shared get tiles over slots [N*B + j*T, N*B + (j+1)*T) with expert id
 * E + j. "first row" is the row of hq / hs / y the tile's first slot uses; the
 * tile builders here set it to the slot itself, so these buffers have
 * N*B + n_shared*T rows. */
int moe_max_tiles(int T, int K, int E, int N, int B, int n_shared, int mt);
int moe_build_tiles(const int32_t* token_position_to_id, const int32_t* block_to_expert, int N,
                    int B, int T, int E, int n_shared, int mt, int32_t* tiles, int max_tiles,
                    int32_t* num_tiles, void* stream);

/* ---- expert GEMMs (fp8 MFMA, 128x128 block scales in the accumulator) ---- */

/* hq[slot, :I] / hs[slot, :I/128] = quant_1x128(SiLU(x W_g^T) * (x W_u^T)) for every
 * slot of every tile, x rows gathered by token_position_to_id (shared slots map
 * to token slot - N*B - j*T). hq/hs have N*B + n_shared*T rows.
 * Replaces the gate_up half of nkilib moe_cte (moe_cte.py:356-421) and of
 * _torch_moe_impl (moe_cte.py:557-575), SiLU activation. mt in {16,32,64,128}.
 *
 * Weight dequantization: code * w13_scale[e, row/128, k/128] (128x128 blocks),
 * times w13_channel_scale[e, row] when that pointer is not NULL ([E, 2I] fp32,
 * gate rows then up rows; w13_shared_channel_scale likewise [n_shared, 2I]). The
 * channel scales carry the reference's FP8 per-channel ("row") weight scales
 * ([E, 1, 2I] in moe_cte, moe_cte.py:178-181; [E, 2, I] in moe_tkg,
 * moe_tkg.py:87-89) and, expanded along the rows, its static scales ([E, 2, 1]);
 * pass all-ones block scales with them. */
int moe_expert_gate_up(const uint8_t* xq, const float* xs, int T, int H, int I, int E,
                       const uint8_t* w13, const float* w13_scale,
                       const float* w13_channel_scale, const uint8_t* w13_shared,
                       const float* w13_shared_scale, const float* w13_shared_channel_scale,
                       int n_shared, const int32_t* token_position_to_id, int NB,
                       const int32_t* tiles, const int32_t* num_tiles, int max_tiles, int mt,
                       uint8_t* hq, float* hs, void* stream);

/* y[slot, :H] = bf16(hq[slot] W_d^T) per tile slot (unweighted).
 * Replaces the down projection of moe_cte (moe_cte.py:585-588). Channel scales as
 * moe_expert_gate_up: w2_channel_scale [E, H] (the reference's [E, 1, H] /
 * [E, H] row scales, moe_cte.py:186-188, moe_tkg.py:90-91, or its [E, 1] static
 * scale expanded), w2_shared_channel_scale [n_shared, H]; NULL for none. */
int moe_expert_down(const uint8_t* hq, const float* hs, int T, int H, int I, int E,
                    const uint8_t* w2, const float* w2_scale, const float* w2_channel_scale,
                    const uint8_t* w2_shared, const float* w2_shared_scale,
                    const float* w2_shared_channel_scale, int n_shared, int NB,
                    const int32_t* tiles, const int32_t* num_tiles, int max_tiles, int mt,
                    void* y_bf16, void* stream);

/* Prefill-sized variants ("block" kernels): one workgroup computes 256 slots
 * of one expert x 256 weight rows with 16x16x128 fp8 MFMA tiles, both operands
 * staged through LDS. Their tile list holds up to 256 consecutive slots of one
 * expert per tile: `tiles` is max_tiles * 24 bytes (int32x4 tiles followed by
 * int32x2 {first tile, tile count} of each tile's expert), built by
 * moe_build_block_tiles with a scratch workspace of
 * moe_block_tiles_workspace_bytes(N, max_tiles). Its `num_tiles` is a header of
 * MOE_BLOCK_TILES_HEADER int32: the tile count, then the first tile of each XCD's
 * range (9 values: ranges of whole experts with about equal work), which the block
 * GEMMs read. Same outputs as
 * moe_expert_gate_up / moe_expert_down (same replaced reference interface,
 * moe_cte.py:356-421 and :557-588); the layer uses them when the average
 * expert receives more than 32 rows. */
#define MOE_BLOCK_TILES_HEADER 16
int moe_max_block_tiles(int T, int K, int E, int N, int B, int n_shared);
size_t moe_block_tiles_workspace_bytes(int N, int max_tiles);
int moe_build_block_tiles(const int32_t* token_position_to_id, const int32_t* block_to_expert,
                          int N, int B, int T, int E, int n_shared, int32_t* tiles, int max_tiles,
                          int32_t* num_tiles, void* workspace, size_t workspace_bytes,
                          void* stream);
int moe_expert_gate_up_block(const uint8_t* xq, const float* xs, int T, int H, int I, int E,
                             const uint8_t* w13, const float* w13_scale,
                             const float* w13_channel_scale, const uint8_t* w13_shared,
                             const float* w13_shared_scale,
                             const float* w13_shared_channel_scale, int n_shared,
                             const int32_t* token_position_to_id, int NB, const int32_t* tiles,
                             const int32_t* num_tiles, int max_tiles, uint8_t* hq, float* hs,
                             void* stream);
int moe_expert_down_block(const uint8_t* hq, const float* hs, int T, int H, int I, int E,
                          const uint8_t* w2, const float* w2_scale, const float* w2_channel_scale,
                          const uint8_t* w2_shared, const float* w2_shared_scale,
                          const float* w2_shared_channel_scale, int n_shared, int NB,
                          const int32_t* tiles, const int32_t* num_tiles, int max_tiles,
                          void* y_bf16, void* stream);

/* ---- weighted unpermute-combine ----------------------------------------- */

/* out[t] = bf16( sum_{s<S, inv[t,s]>=0} w[t,s] * y[inv[t,s]]  +  sum_{j<n_shared} y[NB + j*T + t] ),
 * fp32 accumulation in s order then j order. POST_SCALE accumulate of
 * moe_cte.py:603-606 and the scatter-add combine of topk_reduce.py:144-159. */
int moe_combine(const void* y_bf16, const int32_t* inv, const float* w, int S, int T, int H, int NB,
                int n_shared, void* out_bf16, void* stream);

/* ---- whole layer --------------------------------------------------------- */

/* [residual add ->] [RMSNorm ->] router -> top-k -> mapping -> act quant ->
 * gate_up -> down -> combine, on one stream.
 *   gamma [H] fp32 (NULL: no norm, x is already normalized): the layer's own
 *     pre-MoE RMSNorm over the first hidden_actual columns (<= 0: all H), as
 *     moe_rms_norm; the router and the experts read the normalized bf16 rows.
 *     GptOssExperts.forward_prefill normalizes first (model_bf16.py:1359) and
 *     forward_decode passes the norm weight as gamma to moe_block_tkg
 *     (model_bf16.py:1276, moe_block_tkg.py:135-151).
 *   residual [T,H] bf16 (optional, needs gamma) is added first; the bf16 sum
 *     goes to residual_out [T,H], the (out, residual_sum) form of the MXFP4
 *     layer (model_mxfp4.py:1362-1377, :1584-1609).
 * ids/weights/logits outputs are optional (NULL to skip). The layer forward of
 * the reference MoE block (GptOssExperts.forward, model_bf16.py:1221-1232 ->
 * forward_prefill :1347-1484 / forward_decode :1309-1345; fused decode
 * moe_block_tkg.py:306-591) with DeepSeek-style fp8-blockwise experts.
 * The workspace holds the expert rows compacted: T*min(K,E) routed rows plus
 * n_shared*T shared rows of h and y (norm != 0 adds T*H*2 bytes of normalized
 * rows). */
size_t moe_layer_workspace_bytes(int T, int H, int I, int E, int K, int n_shared, int B, int norm);
int moe_layer_forward(const void* x_bf16, const void* residual_bf16, const float* gamma,
                      float eps, int hidden_actual, int T, int H, int I, int E, int K,
                      int n_shared, const void* router_w_bf16, const float* router_bias,
                      const float* corr_bias, int order, int scoring, int n_group,
                      int topk_group, int renorm, float renorm_eps, float routed_scale,
                      const uint8_t* w13, const float* w13_scale, const uint8_t* w2,
                      const float* w2_scale, const uint8_t* w13_shared,
                      const float* w13_shared_scale, const uint8_t* w2_shared,
                      const float* w2_shared_scale, int B, void* out_bf16,
                      void* residual_out_bf16, int32_t* ids_out, float* weights_out,
                      float* logits_out, void* workspace, size_t workspace_bytes, void* stream);

/* moe_layer_forward without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops that
 * forbid allocation). No counterpart in the reference. Its workspace is a static
 * device array of MOE_NOALLOC_SCRATCH_BYTES, one per GPU, reserved when the
 * library's code object loads on that GPU (whether or not this entry is ever
 * called, so it costs 64 MiB per GPU also to callers that only use the workspace
 * entry points) and held until the process ends; the call allocates nothing. Calls
 * whose moe_layer_workspace_bytes exceeds it return MOE_ERR_UNSUPPORTED (64 MiB
 * covers the DeepSeek-V3 / Kimi-K2 layers up to about 320 tokens). All calls on
 * one GPU share the array: calls that overlap on one GPU (unordered streams,
 * host threads) race and must be serialized by the caller. The device current
 * on the calling thread must be the stream's device. */
#define MOE_NOALLOC_SCRATCH_BYTES (64 << 20)
int moe_layer_forward_noalloc(const void* x_bf16, const void* residual_bf16, const float* gamma,
                              float eps, int hidden_actual, int T, int H, int I, int E, int K,
                              int n_shared, const void* router_w_bf16, const float* router_bias,
                              const float* corr_bias, int order, int scoring, int n_group,
                              int topk_group, int renorm, float renorm_eps, float routed_scale,
                              const uint8_t* w13, const float* w13_scale, const uint8_t* w2,
                              const float* w2_scale, const uint8_t* w13_shared,
                              const float* w13_shared_scale, const uint8_t* w2_shared,
                              const float* w2_shared_scale, int B, void* out_bf16,
                              void* residual_out_bf16, int32_t* ids_out, float* weights_out,
                              float* logits_out, void* stream);

/* ---- MX (microscaling) experts ------------------------------------------- */

/* OCP MX formats (MX v1.0): 32 consecutive values along K share one E8M0 scale
 * byte (2^(b - 127)). Expert weights are MXFP4 (E2M1, two codes per byte, the low
 * nibble first: the HF GPT-OSS packing) or MXFP8 (E4M3); activations are MXFP8.
 * Layouts: w13 [E, 2I, H/2] (fp4) or [E, 2I, H] (fp8), gate rows [0, I) then up
 * rows; w13_scale [E, 2I, H/32]; w2 [E, H, I/2] or [E, H, I]; w2_scale
 * [E, H, I/32]; biases fp32 b13 [E, 2I], b2 [E, H] (optional). The reference holds
 * GPT-OSS's MXFP4 experts in a Trainium tiling (moe_cte.py:122-130, :178-191;
 * model/gpt_oss/weight_loaders_mxfp4.py:301-560), converted from the same HF
 * checkpoint tensors this layout stacks. */
#define MOE_MX_FP8 0
#define MOE_MX_FP4 1
#define MOE_ACT_SILU 0
#define MOE_ACT_SWISH 1 /* g * sigmoid(1.702 g), moe_cte.py:459-461 */

/* MXFP8 quantization of bf16 rows [rows, cols] (cols % 32 == 0): e =
 * max(floor(log2(amax)) - 8, -127) per 32-value block, scale byte e + 127,
 * codes RNE_e4m3(clamp(x * 2^-e, +-448)). The activation quantization of the MX
 * path (the reference quantizes hidden rows to MX inside its fused prefill
 * kernel, model_mxfp4.py:1584-1605). */
int moe_act_quant_mx(const void* x_bf16, int rows, int cols, uint8_t* q, uint8_t* scales,
                     void* stream);

/* MX gate_up over row tiles (tiles as moe_build_tiles, mt in {16, 32, 64}; 128
 * returns MOE_ERR_UNSUPPORTED): gate = clamp(x W_g^T + b_g,
 * gate_lo, gate_hi), up = clamp(x W_u^T + b_u, up_lo, up_hi) (NaN limit = none),
 * h = act(gate) * up, written MXFP8-quantized per 32 columns (hq [rows, I] codes,
 * hs [rows, I/32] scale bytes). Replaces the gate/up half of nkilib's
 * shard_on_block_mx moe_cte (moe_cte.py:356-421) with the math of _torch_moe_impl
 * (moe_cte.py:557-575: biases :562-564, clamps :567-571, Swish :459-461). */
int moe_expert_gate_up_mx(const uint8_t* xq, const uint8_t* xs, int T, int H, int I, int E,
                          int wfmt, const uint8_t* w13, const uint8_t* w13_scale,
                          const float* b13, const uint8_t* w13_shared,
                          const uint8_t* w13_shared_scale, const float* b13_shared, int n_shared,
                          const int32_t* token_position_to_id, int NB, const int32_t* tiles,
                          const int32_t* num_tiles, int max_tiles, int mt, int act, float gate_lo,
                          float gate_hi, float up_lo, float up_hi, uint8_t* hq, uint8_t* hs,
                          void* stream);

/* MX down: y[row, :H] = bf16(h W_d^T + b_d) per tile row (unweighted; mt as the MX
 * gate_up). Replaces the
 * down projection and its bias of moe_cte (moe_cte.py:585-591). */
int moe_expert_down_mx(const uint8_t* hq, const uint8_t* hs, int T, int H, int I, int E, int wfmt,
                       const uint8_t* w2, const uint8_t* w2_scale, const float* b2,
                       const uint8_t* w2_shared, const uint8_t* w2_shared_scale,
                       const float* b2_shared, int n_shared, int NB, const int32_t* tiles,
                       const int32_t* num_tiles, int max_tiles, int mt, void* y_bf16,
                       void* stream);

/* The MoE layer with MX experts (GPT-OSS: MXFP4 experts with biases, Swish and
 * clamps): [residual add ->] [RMSNorm (gamma) ->] router logits (+ router_bias) ->
 * top-k (orders TOPK_ACT / ACT_TOPK) -> mapping -> MXFP8 activations -> MX gate_up
 * -> MX down -> weighted combine. Arguments as moe_layer_forward and
 * moe_expert_gate_up_mx; no shared experts. Workspace:
 * moe_layer_workspace_bytes(T, H, I, E, K, 0, B, gamma != NULL). Replaces
 * GptOssExperts.forward of the MXFP4 model (model_mxfp4.py:1362-1377: prefill
 * :1584-1769 fused norm + router + shard_on_block_mx moe_cte; decode
 * moe_block_tkg with the same activation, clamps and biases, model_bf16.py:
 * 1274-1307). */
int moe_layer_forward_mx(const void* x_bf16, const void* residual_bf16, const float* gamma,
                         float eps, int hidden_actual, int T, int H, int I, int E, int K,
                         const void* router_w_bf16, const float* router_bias, int order,
                         int scoring, int renorm, float renorm_eps, float routed_scale, int wfmt,
                         const uint8_t* w13, const uint8_t* w13_scale, const float* b13,
                         const uint8_t* w2, const uint8_t* w2_scale, const float* b2, int act,
                         float gate_lo, float gate_hi, float up_lo, float up_hi, int B,
                         void* out_bf16, void* residual_out_bf16, int32_t* ids_out,
                         float* weights_out, float* logits_out, void* workspace,
                         size_t workspace_bytes, void* stream);

/* ---- diagnostics ----------------------------------------------------------- */

/* shape 0: c[16,16] = decode(a[16,128]) . decode(b[16,128])^T through one
 * v_mfma_f32_16x16x128_f8f6f4; shape 1: c[32,32] = decode(a[32,128]) .
 * decode(b[32,128])^T through two v_mfma_f32_32x32x64_f8f6f4; each with the
 * operand/accumulator lane mapping the expert GEMMs use. No reference
 * counterpart: it pins the gfx950 fp8 MFMA data layout for the tests. */
int moe_selftest_mfma_fp8(const uint8_t* a, const uint8_t* b, float* c, int shape, void* stream);

/* For every fp32 bit pattern u in [first, first + count) (u < 2^31) whose value
 * v has |v| <= 448: the e4m3fn codes of v and -v from the gfx950 conversion
 * instruction against the integer round-to-nearest-even encoder. Writes
 * out[0..blocks) = mismatch counts and out[blocks..2*blocks) = the smallest
 * mismatching pattern per workgroup (0xffffffff if none). No reference
 * counterpart: it pins the hardware encoder the quantizers use. */
int moe_selftest_fp8_encode(uint32_t first, uint32_t count, uint32_t* out, int blocks,
                            void* stream);

/* For every fp32 bit pattern in [first, first + count) (first + count <= 2^32):
 * the bf16 conversion instruction the output stages use against the integer
 * round-to-nearest-even encoder (a NaN has to stay a NaN). Output as
 * moe_selftest_fp8_encode. No reference counterpart. */
int moe_selftest_bf16_encode(uint32_t first, uint32_t count, uint32_t* out, int blocks,
                             void* stream);

/* The quantizers divide by a shared scale with one reciprocal and a correction
 * step; this compares it with the IEEE division: equal e4m3 codes of the clamped
 * quotients, and equal fp32 quotients wherever their magnitude is at least 2^-10
 * (below that both encode to a signed zero). Mode 0:
 * u in [first, first + count) (u < 2^31) is the pair (bf16 group amax u >> 16,
 * bf16 value u & 0xffff), used when both are finite and |value| <= amax, with
 * the quantizer's scale max(amax, 1e-10) / 448 as divisor. Mode 1: u seeds a
 * random fp32 amax in [2^-40, 2^40) and a value of magnitude at most amax.
 * Output as moe_selftest_fp8_encode. No reference counterpart. */
int moe_selftest_quant_div(int mode, uint32_t first, uint32_t count, uint32_t* out, int blocks,
                           void* stream);

/* One scaled MFMA with the MX GEMMs' lane mapping: c[16,16] = A . B^T with A
 * [16,128] fp8 codes and scale bytes sa [16,4], B [16,128] values as fp4 (packed
 * [16,64] bytes) or fp8 ([16,128]) with sb [16,4]. No reference counterpart: it
 * pins the gfx950 scaled-MFMA data and scale layout for the tests. */
int moe_selftest_mfma_mx(const uint8_t* a, const uint8_t* sa, const uint8_t* b, const uint8_t* sb,
                         int wfmt, float* c, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MOE_FP8_H */
