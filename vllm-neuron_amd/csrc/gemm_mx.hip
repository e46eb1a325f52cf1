// MX (OCP Microscaling) expert GEMMs for gfx950: MXFP4 or MXFP8 expert weights,
// MXFP8 activations, E8M0 scales per 32 values along K applied by the MFMA itself.
//
//   gate_up: h = mxfp8( act(clamp(x W_g^T + b_g)) * clamp(x W_u^T + b_u) )   per slot
//   down   : y = bf16( h W_d^T + b_d )                                      per slot
//
// Reference: the GPT-OSS expert MLP (model/gpt_oss/model_mxfp4.py:1019-1211,
// weights in MXFP4; model_bf16.py:1274-1307, :1450-1470: Swish, clamps, biases),
// run by nkilib's shard_on_block_mx kernels on Trainium-3 (moe_cte.py:122-130,
// :178-191) with the math of the CPU fallback _torch_moe_impl (moe_cte.py:440-612).
//
// Operand layout of v_mfma_scale_f32_16x16x128_f8f6f4 (pinned on the GPU by
// moe_selftest_mfma_mx against the oracle): lane l supplies row l % 16; with g =
// l / 16, an fp8 operand holds the K values [16 g, +16) and [64 + 16 g, +16) of the
// 128-wide K block (8 registers), an fp4 operand the K values [32 g, +32) (4
// registers, two values per byte, the lower K in the low nibble). The scale
// operand of lane l is the E8M0 byte of row l % 16 and K block [32 g, +32),
// whatever the data layout. So the per-32 scales are applied inside the MFMA and
// no per-block fp32 multiply is left for the VALU.
//
// Work decomposition as in gemm_fp8.hip: a work item is (row tile, N tile); a
// row tile holds up to MT consecutive slots of one expert; a workgroup (4 waves)
// owns 256 weight rows (gate_up: 128 gate rows + the matching 128 up rows, so a
// wave holds 32 h columns = one MX block of h; down: 256 output columns). Weight
// fragments stream from HBM into registers through a PD-deep ring (each weight
// byte is read by exactly one lane); activation rows and their scale bytes are
// gathered into LDS (double buffered).
#include <math.h>

#include <type_traits>

#include "moe_common.h"
#include "moe_internal.h"

namespace moe {

constexpr int kFmtFp8 = 0;  // MFMA format codes (cbsz / blgp) of the scaled instruction
constexpr int kFmtFp4 = 4;

struct MxArgs {
  const uint8_t* a;    // fp8 activations: x [T, H] (gate_up) or h [rows, I] (down)
  const uint8_t* as;   // their E8M0 scales [rows, K/32]
  const uint8_t* w;    // routed weights, packed (fp4: K/2 bytes per row; fp8: K)
  const uint8_t* ws;   // routed weight scales [E, rows_w, K/32]
  const float* bias;   // routed bias [E, rows_w] (fp32) or null
  const uint8_t* wsh;  // shared-expert weights / scales / bias
  const uint8_t* wssh;
  const float* bsh;
  const int32_t* tpid;
  const int4* tiles;  // {expert, first slot, rows, first hq / y row}
  const int32_t* num_tiles;
  uint8_t* hq;
  uint8_t* hs;
  uint16_t* y;
  int T, H, I, E, nsh;
  long NB;
  int act;  // 0 SiLU, 1 Swish (g * sigmoid(1.702 g))
  float gate_lo, gate_hi, up_lo, up_hi;
};

// E8M0 exponent e of an MX block with magnitude maximum amax (OCP MX v1.0 6.3):
// floor(log2(amax)) - 8 (8 = emax of e4m3), at least -127; the scale byte is
// e + 127 and the elements are v * 2^-e (a power of two: exact), clamped to +-448
// and rounded to nearest even. amax = 0 or subnormal gives e = -127.
__device__ __forceinline__ int mx_exponent(float amax) {
  const int ef = (int)((__float_as_uint(amax) >> 23) & 0xffu);
  return max(ef - 135, -127);
}

// 2^-e for e in [-127, 119] (the range mx_exponent returns for finite input).
__device__ __forceinline__ float mx_inv_scale(int e) { return __uint_as_float((uint32_t)(127 - e) << 23); }

__device__ __forceinline__ uint32_t mx_e4m3x2(float a, float b, float f) {
  return e4m3x2(fminf(fmaxf(a * f, -448.0f), 448.0f), fminf(fmaxf(b * f, -448.0f), 448.0f));
}

__device__ __forceinline__ v4f mfma_mx(const v8i& a, const v8i& b, const v4f& c, int sa, int sb,
                                      std::integral_constant<int, kFmtFp8>) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, kFmtFp8, kFmtFp8, 0, sa, 0, sb);
}
__device__ __forceinline__ v4f mfma_mx(const v8i& a, const v8i& b, const v4f& c, int sa, int sb,
                                      std::integral_constant<int, kFmtFp4>) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, kFmtFp8, kFmtFp4, 0, sa, 0, sb);
}

// Lane fragment of a row for one 128-wide K block, p = row block + 16 g: fp4, the 16
// bytes at p (K values [32 g, +32); the upper half of the operand unused); fp8, the
// 16 bytes at p and at p + 64 (K values [16 g, +16) and [64 + 16 g, +16)).
template <int FMT>
__device__ __forceinline__ v8i load_frag(const uint8_t* p) {
  const int4 lo = *(const int4*)p;
  if (FMT == kFmtFp4) return (v8i){lo.x, lo.y, lo.z, lo.w, 0, 0, 0, 0};
  const int4 hi = *(const int4*)(p + 64);
  return (v8i){lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
}

__device__ __forceinline__ float mx_act(float g, int act) {
  // hardware reciprocal (about 1 ulp): h only feeds the MXFP8 quantization
  const float k = act ? -1.702f : -1.0f;
  return g * __builtin_amdgcn_rcpf(1.0f + __expf(k * g));
}

template <int MT, int KIND, int PD, int WFMT>
__global__ __launch_bounds__(256) void expert_gemm_mx_kernel(MxArgs p) {
  constexpr int MS = MT / 16;
  constexpr int ACH = MT * 8;             // 16-byte chunks per A tile per K block
  constexpr int APT = (ACH + 255) / 256;  // chunks per thread
  constexpr int LDA = 128 + 16;           // padded LDS row (bytes)
  constexpr int WKB = (WFMT == kFmtFp4) ? 64 : 128;  // weight bytes per row per K block
  __shared__ __attribute__((aligned(16))) uint8_t sA[2][MT * LDA];
  __shared__ __attribute__((aligned(16))) uint32_t sAs[2][MT];  // 4 scale bytes per row
  __shared__ long sSrc[MT];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, r16 = lane & 15;
  const int Kdim = (KIND == 0) ? p.H : p.I;
  const int KB = Kdim / 128;
  const int KS = Kdim / 32;  // scale bytes per row
  const int NT = (KIND == 0) ? p.I / 128 : p.H / 256;
  const int total = p.num_tiles[0] * NT;
  const std::integral_constant<int, WFMT> wfmt{};

  for (int wi = blockIdx.x; wi < total; wi += gridDim.x) {
    const int tile = wi / NT, nt = wi - tile * NT;
    const int4 td = p.tiles[tile];
    const int e = td.x, nrows = td.z;
    const long slot0 = td.y, row0 = td.w;
    if (e < 0 || e >= p.E + p.nsh) continue;  // workgroup-uniform: malformed tile
    const bool is_sh = e >= p.E;
    const int ej = is_sh ? e - p.E : e;

    if (tid < MT) {
      long src = -1;
      if (tid < nrows) {
        const long slot = slot0 + tid;
        if (KIND == 0) {
          src = is_sh ? slot - p.NB - (long)ej * p.T : (long)p.tpid[slot];
          if (src >= p.T) src = -1;  // token ids outside [0, T) are padding
        } else {
          src = row0 + tid;
        }
      }
      sSrc[tid] = src;
    }
    __syncthreads();

    // Activation chunks: every load is issued unconditionally (rows without a
    // source read row 0 and are zeroed), so the loads in flight stay countable.
    const uint8_t* aptr[APT];
    int aoff[APT];
    bool alive[APT];
#pragma unroll
    for (int c = 0; c < APT; ++c) {
      const int chunk = tid + 256 * c;
      aptr[c] = p.a;
      aoff[c] = -1;
      alive[c] = false;
      if (chunk < ACH) {
        const int row = chunk >> 3, col = (chunk & 7) * 16;
        aoff[c] = row * LDA + col;
        const long src = sSrc[row];
        if (src >= 0) {
          aptr[c] = p.a + (size_t)src * Kdim + col;
          alive[c] = true;
        }
      }
    }
    const bool as_alive = tid < MT && sSrc[tid] >= 0;
    const uint8_t* asp = as_alive ? p.as + (size_t)sSrc[tid] * KS : p.as;

    const size_t wrow_bytes = (size_t)Kdim * WKB / 128;
    const int rows_w = (KIND == 0) ? 2 * p.I : p.H;
    const uint8_t* wb = (is_sh ? p.wsh : p.w) + (size_t)ej * rows_w * wrow_bytes;
    const uint8_t* wsb = (is_sh ? p.wssh : p.ws) + (size_t)ej * rows_w * KS;
    const float* bb = is_sh ? p.bsh : p.bias;
    if (bb != nullptr) bb += (size_t)ej * rows_w;
    int wrow[4];
    const uint8_t* bp[4];
    const uint32_t* sp[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (KIND == 0)
        wrow[j] = (j < 2) ? nt * 128 + wave * 32 + j * 16 + r16
                          : p.I + nt * 128 + wave * 32 + (j - 2) * 16 + r16;
      else
        wrow[j] = nt * 256 + wave * 64 + j * 16 + r16;
      bp[j] = wb + (size_t)wrow[j] * wrow_bytes + g * 16;
      sp[j] = (const uint32_t*)(wsb + (size_t)wrow[j] * KS);  // KS % 4 == 0: dword aligned
    }

    v8i bq[PD][4];
    uint32_t bsq[PD][4];
    int4 aq[PD][APT];
    uint32_t asq[PD];

    auto load_stage = [&](int s, int kb) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        bq[s][j] = load_frag<WFMT>(bp[j] + (size_t)kb * WKB);
        bsq[s][j] = sp[j][kb];  // the 4 scale bytes of the K block; lane uses byte g
      }
#pragma unroll
      for (int c = 0; c < APT; ++c)
        aq[s][c] = *(const int4*)(aptr[c] + (alive[c] ? (size_t)kb * 128 : 0));
      asq[s] = *(const uint32_t*)(asp + (as_alive ? (size_t)kb * 4 : 0));
    };
    auto store_A = [&](int buf, int s) {
#pragma unroll
      for (int c = 0; c < APT; ++c)
        if (aoff[c] >= 0) *(int4*)&sA[buf][aoff[c]] = alive[c] ? aq[s][c] : make_int4(0, 0, 0, 0);
      if (tid < MT) sAs[buf][tid] = as_alive ? asq[s] : 0x7f7f7f7fu;  // scale 1 for zero rows
    };

    v4f acc[MS][4];
#pragma unroll
    for (int ms = 0; ms < MS; ++ms)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[ms][j] = (v4f){0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (int s = 0; s < PD - 1; ++s) load_stage(s, min(s, KB - 1));
    store_A(0, 0);
    __syncthreads();

    auto kstep = [&](int kb, int s) {
      load_stage((s + PD - 1) % PD, min(kb + PD - 1, KB - 1));
      const int buf = kb & 1;
#pragma unroll
      for (int ms = 0; ms < MS; ++ms) {
        const v8i a = load_frag<kFmtFp8>(&sA[buf][(ms * 16 + r16) * LDA + g * 16]);
        const int sa = (int)(sAs[buf][ms * 16 + r16] >> (8 * g));
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[ms][j] = mfma_mx(a, bq[s][j], acc[ms][j], sa, (int)(bsq[s][j] >> (8 * g)), wfmt);
      }
      if (kb + 1 < KB) store_A((kb + 1) & 1, (s + 1) % PD);
      lds_barrier();  // orders the activation double buffer; weight prefetches stay in flight
    };
    int kb0 = 0;
    for (; kb0 + PD <= KB; kb0 += PD) {
#pragma unroll
      for (int s = 0; s < PD; ++s) kstep(kb0 + s, s);
    }
#pragma unroll
    for (int s = 0; s < PD - 1; ++s)
      if (kb0 + s < KB) kstep(kb0 + s, s);

    // Accumulator layout: lane l, register i holds D[4 * (l / 16) + i][l % 16]
    // (row of the tile, weight row of the fragment).
    if (KIND == 0) {
      const int GI = p.I / 32;
      float bgate[2] = {0.f, 0.f}, bup[2] = {0.f, 0.f};
      if (bb != nullptr) {
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          bgate[jj] = bb[wrow[jj]];
          bup[jj] = bb[wrow[jj + 2]];
        }
      }
#pragma unroll
      for (int ms = 0; ms < MS; ++ms) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float m = 0.f;
#pragma unroll
          for (int jj = 0; jj < 2; ++jj) {
            const float gt = fminf(fmaxf(acc[ms][jj][i] + bgate[jj], p.gate_lo), p.gate_hi);
            const float up = fminf(fmaxf(acc[ms][jj + 2][i] + bup[jj], p.up_lo), p.up_hi);
            const float h = mx_act(gt, p.act) * up;
            acc[ms][jj][i] = h;
            m = fmaxf(m, fabsf(h));
          }
          // the wave's 32 h columns of this row are one MX block
          m = group16_max_f32(m);
          const int row = ms * 16 + 4 * g + i;
          const int ex = mx_exponent(m);
          if (sSrc[row] >= 0) {
            const float f = mx_inv_scale(ex);
            const uint32_t c2 = mx_e4m3x2(acc[ms][0][i], acc[ms][1][i], f);
            uint8_t* const hrow = p.hq + (size_t)(row0 + row) * p.I + nt * 128 + wave * 32 + r16;
            hrow[0] = (uint8_t)c2;
            hrow[16] = (uint8_t)(c2 >> 8);
            if (r16 == 0) p.hs[(size_t)(row0 + row) * GI + nt * 4 + wave] = (uint8_t)(ex + 127);
          }
        }
      }
    } else {
      float bd[4] = {0.f, 0.f, 0.f, 0.f};
      if (bb != nullptr) {
#pragma unroll
        for (int j = 0; j < 4; ++j) bd[j] = bb[wrow[j]];
      }
#pragma unroll
      for (int ms = 0; ms < MS; ++ms) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = ms * 16 + 4 * g + i;
          if (row < nrows) {
            const long yrow = row0 + row;
#pragma unroll
            for (int j = 0; j < 4; ++j)
              p.y[(size_t)yrow * p.H + wrow[j]] = (uint16_t)bf16x2(acc[ms][j][i] + bd[j], 0.f);
          }
        }
      }
    }
    __syncthreads();
  }
}

// MXFP8 quantization of bf16 rows: lane q of a 4-lane group holds 8 consecutive
// values of one 32-value block (one 16-byte load), the block amax is combined over
// the group, and the group writes 32 codes and one scale byte.
__global__ __launch_bounds__(256) void mx_act_quant_kernel(const uint16_t* __restrict__ x, long chunks,
                                                           uint8_t* __restrict__ q,
                                                           uint8_t* __restrict__ s) {
  const long stride = (long)gridDim.x * blockDim.x;
  for (long c0 = (long)blockIdx.x * blockDim.x; c0 < chunks; c0 += stride) {
    const long c = c0 + threadIdx.x;  // whole 4-lane groups share the bound (chunks % 4 == 0)
    float v[8];
    float a = 0.f;
    if (c < chunks) {
      bf16x8_to_f32(*(const int4*)(x + c * 8), v);
#pragma unroll
      for (int i = 0; i < 8; ++i) a = fmaxf(a, fabsf(v[i]));
    }
    a = fmaxf(a, __shfl_xor(a, 1, MOE_WAVE));
    a = fmaxf(a, __shfl_xor(a, 2, MOE_WAVE));
    if (c < chunks) {
      const int ex = mx_exponent(a);
      const float f = mx_inv_scale(ex);
      const uint32_t lo = mx_e4m3x2(v[0], v[1], f) | (mx_e4m3x2(v[2], v[3], f) << 16);
      const uint32_t hi = mx_e4m3x2(v[4], v[5], f) | (mx_e4m3x2(v[6], v[7], f) << 16);
      *(uint2*)(q + c * 8) = make_uint2(lo, hi);
      if ((c & 3) == 0) s[c >> 2] = (uint8_t)(ex + 127);
    }
  }
}

// One scaled MFMA with the GEMM's lane mapping: c[16,16] = A[16,128] . B[16,128]^T,
// A fp8 with scale bytes sa[16,4], B fp4 (packed, [16,64] bytes) or fp8 ([16,128])
// with sb[16,4].
template <int WFMT>
__global__ void selftest_mfma_mx_kernel(const uint8_t* a, const uint8_t* sa, const uint8_t* b,
                                        const uint8_t* sb, float* c) {
  const int lane = threadIdx.x, g = lane >> 4, r16 = lane & 15;
  constexpr int WKB = (WFMT == kFmtFp4) ? 64 : 128;
  const v8i fa = load_frag<kFmtFp8>(a + r16 * 128 + g * 16);
  const v8i fb = load_frag<WFMT>(b + r16 * WKB + g * 16);
  const v4f z = {0.f, 0.f, 0.f, 0.f};
  const v4f d = mfma_mx(fa, fb, z, sa[r16 * 4 + g], sb[r16 * 4 + g], std::integral_constant<int, WFMT>{});
#pragma unroll
  for (int i = 0; i < 4; ++i) c[(4 * g + i) * 16 + r16] = d[i];
}

template <int KIND, int WFMT>
static int launch_mx(const MxArgs& a, int max_tiles, int mt, hipStream_t st) {
  const int NT = (KIND == 0) ? a.I / 128 : a.H / 256;
  const long items = (long)max_tiles * NT;
  const int grid = (int)std::max(1L, std::min(items, 4096L));
  switch (mt) {
    case 16:
      hipLaunchKernelGGL((expert_gemm_mx_kernel<16, KIND, 3, WFMT>), dim3(grid), dim3(256), 0, st, a);
      break;
    case 32:
      hipLaunchKernelGGL((expert_gemm_mx_kernel<32, KIND, 3, WFMT>), dim3(grid), dim3(256), 0, st, a);
      break;
    case 64:
      hipLaunchKernelGGL((expert_gemm_mx_kernel<64, KIND, 2, WFMT>), dim3(grid), dim3(256), 0, st, a);
      break;
    case 128:
      hipLaunchKernelGGL((expert_gemm_mx_kernel<128, KIND, 2, WFMT>), dim3(grid), dim3(256), 0, st, a);
      break;
    default:
      return MOE_ERR_ARG;
  }
  return MOE_OK;
}

}  // namespace moe

using namespace moe;

static int mx_common_checks(const char* _moe_fn, int T, int H, int I, int E, int NB,
                            int max_tiles, int mt, int wfmt, int n_shared) {
  MOE_CHECK_ARG(T > 0 && E > 0 && NB >= 0 && max_tiles > 0 && n_shared >= 0, "bad sizes");
  MOE_CHECK_ARG(H > 0 && H % 256 == 0 && I > 0 && I % 128 == 0,
                "H must be a multiple of 256 and I of 128 (H=%d I=%d); pad them", H, I);
  MOE_CHECK_ARG(mt == 16 || mt == 32 || mt == 64 || mt == 128, "mt must be 16/32/64/128");
  MOE_CHECK_ARG(wfmt == MOE_MX_FP4 || wfmt == MOE_MX_FP8, "weight format must be MOE_MX_FP4 or MOE_MX_FP8");
  return MOE_OK;
}

static inline float lim(float v, float dflt) { return isnan(v) ? dflt : v; }

extern "C" int moe_act_quant_mx(const void* x_bf16, int rows, int cols, uint8_t* q, uint8_t* scales,
                                void* stream) {
  MOE_API_BEGIN("moe_act_quant_mx");
  MOE_CHECK_ARG(x_bf16 && q && scales, "null pointer argument");
  MOE_CHECK_ARG(rows >= 0 && cols > 0 && cols % 32 == 0, "cols must be a positive multiple of 32, got %d",
                cols);
  MOE_CHECK_ARG(((uintptr_t)x_bf16 & 15) == 0 && ((uintptr_t)q & 7) == 0,
                "x must be 16-byte and q 8-byte aligned");
  if (rows == 0) return MOE_OK;
  const long chunks = (long)rows * cols / 8;
  const int grid = (int)std::max(1L, std::min<long>((chunks + 255) / 256, 4096));
  hipLaunchKernelGGL(mx_act_quant_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)x_bf16, chunks, q, scales);
  MOE_API_END();
}

extern "C" int moe_expert_gate_up_mx(const uint8_t* xq, const uint8_t* xs, int T, int H, int I, int E,
                                     int wfmt, const uint8_t* w13, const uint8_t* w13_scale,
                                     const float* b13, const uint8_t* w13_shared,
                                     const uint8_t* w13_shared_scale, const float* b13_shared,
                                     int n_shared, const int32_t* token_position_to_id, int NB,
                                     const int32_t* tiles, const int32_t* num_tiles, int max_tiles,
                                     int mt, int act, float gate_lo, float gate_hi, float up_lo,
                                     float up_hi, uint8_t* hq, uint8_t* hs, void* stream) {
  MOE_API_BEGIN("moe_expert_gate_up_mx");
  MOE_CHECK_ARG(xq && xs && w13 && w13_scale && token_position_to_id && tiles && num_tiles && hq && hs,
                "null pointer argument");
  int rc = mx_common_checks(_moe_fn, T, H, I, E, NB, max_tiles, mt, wfmt, n_shared);
  if (rc != MOE_OK) return rc;
  MOE_CHECK_ARG(n_shared == 0 || (w13_shared && w13_shared_scale), "shared weights missing");
  MOE_CHECK_ARG(act == MOE_ACT_SILU || act == MOE_ACT_SWISH, "act must be MOE_ACT_SILU or MOE_ACT_SWISH");
  MOE_CHECK_ARG(((uintptr_t)xq & 15) == 0 && ((uintptr_t)w13 & 15) == 0 && ((uintptr_t)xs & 3) == 0 &&
                    ((uintptr_t)w13_scale & 3) == 0,
                "xq and w13 must be 16-byte aligned, the scales 4-byte aligned");
  MxArgs a{};
  a.a = xq;
  a.as = xs;
  a.w = w13;
  a.ws = w13_scale;
  a.bias = b13;
  a.wsh = w13_shared;
  a.wssh = w13_shared_scale;
  a.bsh = b13_shared;
  a.tpid = token_position_to_id;
  a.tiles = (const int4*)tiles;
  a.num_tiles = num_tiles;
  a.hq = hq;
  a.hs = hs;
  a.T = T;
  a.H = H;
  a.I = I;
  a.E = E;
  a.nsh = n_shared;
  a.NB = NB;
  a.act = act;
  a.gate_lo = lim(gate_lo, -INFINITY);
  a.gate_hi = lim(gate_hi, INFINITY);
  a.up_lo = lim(up_lo, -INFINITY);
  a.up_hi = lim(up_hi, INFINITY);
  rc = (wfmt == MOE_MX_FP4) ? launch_mx<0, kFmtFp4>(a, max_tiles, mt, (hipStream_t)stream)
                            : launch_mx<0, kFmtFp8>(a, max_tiles, mt, (hipStream_t)stream);
  MOE_CHECK_ARG(rc == MOE_OK, "bad mt %d", mt);
  MOE_API_END();
}

extern "C" int moe_expert_down_mx(const uint8_t* hq, const uint8_t* hs, int T, int H, int I, int E,
                                  int wfmt, const uint8_t* w2, const uint8_t* w2_scale,
                                  const float* b2, const uint8_t* w2_shared,
                                  const uint8_t* w2_shared_scale, const float* b2_shared,
                                  int n_shared, int NB, const int32_t* tiles,
                                  const int32_t* num_tiles, int max_tiles, int mt, void* y_bf16,
                                  void* stream) {
  MOE_API_BEGIN("moe_expert_down_mx");
  MOE_CHECK_ARG(hq && hs && w2 && w2_scale && tiles && num_tiles && y_bf16, "null pointer argument");
  int rc = mx_common_checks(_moe_fn, T, H, I, E, NB, max_tiles, mt, wfmt, n_shared);
  if (rc != MOE_OK) return rc;
  MOE_CHECK_ARG(n_shared == 0 || (w2_shared && w2_shared_scale), "shared weights missing");
  MOE_CHECK_ARG(((uintptr_t)hq & 15) == 0 && ((uintptr_t)w2 & 15) == 0 && ((uintptr_t)hs & 3) == 0 &&
                    ((uintptr_t)w2_scale & 3) == 0,
                "hq and w2 must be 16-byte aligned, the scales 4-byte aligned");
  MxArgs a{};
  a.a = hq;
  a.as = hs;
  a.w = w2;
  a.ws = w2_scale;
  a.bias = b2;
  a.wsh = w2_shared;
  a.wssh = w2_shared_scale;
  a.bsh = b2_shared;
  a.tiles = (const int4*)tiles;
  a.num_tiles = num_tiles;
  a.y = (uint16_t*)y_bf16;
  a.T = T;
  a.H = H;
  a.I = I;
  a.E = E;
  a.nsh = n_shared;
  a.NB = NB;
  rc = (wfmt == MOE_MX_FP4) ? launch_mx<1, kFmtFp4>(a, max_tiles, mt, (hipStream_t)stream)
                            : launch_mx<1, kFmtFp8>(a, max_tiles, mt, (hipStream_t)stream);
  MOE_CHECK_ARG(rc == MOE_OK, "bad mt %d", mt);
  MOE_API_END();
}

extern "C" int moe_selftest_mfma_mx(const uint8_t* a, const uint8_t* sa, const uint8_t* b,
                                    const uint8_t* sb, int wfmt, float* c, void* stream) {
  MOE_API_BEGIN("moe_selftest_mfma_mx");
  MOE_CHECK_ARG(a && sa && b && sb && c, "null pointer argument");
  MOE_CHECK_ARG(wfmt == MOE_MX_FP4 || wfmt == MOE_MX_FP8, "bad weight format");
  if (wfmt == MOE_MX_FP4)
    hipLaunchKernelGGL(selftest_mfma_mx_kernel<kFmtFp4>, dim3(1), dim3(64), 0, (hipStream_t)stream, a,
                       sa, b, sb, c);
  else
    hipLaunchKernelGGL(selftest_mfma_mx_kernel<kFmtFp8>, dim3(1), dim3(64), 0, (hipStream_t)stream, a,
                       sa, b, sb, c);
  MOE_API_END();
}
