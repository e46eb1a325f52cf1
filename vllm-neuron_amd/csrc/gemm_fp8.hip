// FP8-blockwise grouped expert GEMMs for gfx950 (OCP e4m3fn MFMA).
//
//   gate_up: h = quant_1x128( SiLU(x W_g^T) * (x W_u^T) )   per routed slot
//   down   : y = bf16( h W_d^T )                              per routed slot
//
// Reference: the blockwise expert MLP of nkilib moe_cte called at
// vllm_neuron/functional/moe/moe_cte.py:356-421, whose CPU fallback
// _torch_moe_impl (moe_cte.py:465-612) defines the math: gate/up projections
// (:557-559), SiLU(gate) * up (:574-575), down projection (:585-588). The fp8
// 128x128 block-scale dequantization is DeepSeek-V3's checkpoint format.
//
// Work decomposition: a work item is (row tile, N tile). A row tile holds up
// to MT consecutive slots of one expert (moe_build_tiles) and names the first
// row of hq / y its slots use (the slot itself, or a compacted row in the
// layer, whose buffers hold only the routed rows). Each wave owns 64 weight
// rows (four 16-row MFMA column tiles). gate_up workgroups (4 waves) own 256
// weight rows: 128 gate rows and the matching 128 up rows, so one workgroup sees
// a whole 128-column quantization group of h. down workgroups own 256 output
// columns (4 waves), or 128 (2 waves) for tiles of up to 32 rows: two of those
// fit a CU, so one workgroup's start-up (tile metadata, the first blocks' round
// trip) and epilogue overlap the other's weight stream.
//
// K loop: one v_mfma_f32_16x16x128_f8f6f4 per 128-wide K block (exactly one
// scale block), accumulated in fp32 as acc += mfma(a, b) * (s_a[row] * s_w).
// Weights, gathered activation rows and their scales stream into a PD-stage LDS
// ring with direct-to-LDS loads (see expert_gemm_kernel below).
//
// Operand lane layout: lane l supplies row l%16 and the 32 bytes
// [(l/16)*16, +16) and [64 + (l/16)*16, +16) of the K block. A and B use the
// same mapping, so the hardware's K order inside the block does not matter.
// Accumulator layout: lane l, register i holds D[4*(l/16) + i][l%16].
#include "moe_common.h"
#include "moe_internal.h"

namespace moe {

struct GemmArgs {
  const uint8_t* a;   // xq [T, H] (gate_up) or hq [rows, I] (down)
  const float* as;    // activation scales [rows, K/128]
  const uint8_t* w;   // routed weights
  const float* ws;    // routed weight scales
  const uint8_t* wsh;  // shared-expert weights
  const float* wssh;   // shared-expert weight scales
  const int32_t* tpid;
  const int4* tiles;
  const int32_t* num_tiles;
  uint8_t* hq;
  float* hs;
  uint16_t* y;
  // optional per-output-channel weight scales ([E, 2I] gate_up / [E, H] down, and
  // the shared experts'): multiplied into each output column after the K loop
  const float* cs;
  const float* cssh;
  int T, H, I, E, nsh;
  long NB;
  // gate_up: every routed and shared slot of a tile holds token 0 (the layer at one
  // token, whose own mapping wrote the tiles), so no token ids are loaded
  int tok0;
};

__device__ __forceinline__ v4f mfma_fp8(const v8i& a, const v8i& b) {
  const v4f z = {0.f, 0.f, 0.f, 0.f};
  // format codes 0/0 = e4m3 x e4m3; zero scale operands select the unscaled instruction
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, z, 0, 0, 0, 0, 0, 0);
}

__device__ __forceinline__ v8i load_frag_global(const uint8_t* p) {
  int4 lo = *(const int4*)p;
  int4 hi = *(const int4*)(p + 64);
  return (v8i){lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
}

// ---------------------------------------------------------------------------
// The row-tile kernel. Weight rows stream with global_load_lds_dwordx4 in which
// eight lanes cover one 128-byte row segment, so every load instruction reads
// eight whole cache lines. Loading the MFMA operand layout straight into
// registers reads, per instruction, the halves of sixteen lines instead, which
// measured at about half the stream rate per workgroup (2.7 against 5.5 TB/s
// with 144 workgroups streaming 264 MB), the regime of decode with few
// tokens. The activation tile and its scales arrive the same way, so a K
// step's loads are all direct-to-LDS and one vmcnt wait per step covers a stage.
//
// LDS per stage: wave w's 64 weight rows (8 KB: eight 1 KB loads of 8 rows),
// the tile's activation rows (1 KB per 8 rows) and its 1x128 scales. Rows keep
// the XOR chunk swizzle (swz), so the 16-row fragment reads are conflict-free.
// Weights are wave-private (a wave reads only the rows it loads); activations
// and scales are shared, ordered by one barrier per step. Every wave issues the
// same number of loads per stage (NV; waves without activation rows to load
// repeat row 0 into a spare slot), so the wait for the oldest stage is a
// compile-time vmcnt.
// ---------------------------------------------------------------------------
constexpr int kRowTileMaxKB = 128;  // K <= 16384

// A step's fragment reads, each group in one asm statement that also waits for
// its data: the compiler does not see these as reads of memory that
// direct-to-LDS loads write, so it does not drain the loads in flight into the
// other stages before them (it cannot tell the stages apart across the loop),
// and the registers are complete when the statement ends.
//   weights: 4 column tiles x (lo, hi) at b_lo / b_hi + 2048 j; activations
//   (lo, hi) at a_lo / a_hi; the row group's 4 activation scales at sp.
__device__ __forceinline__ void lds_read_b_a(uint32_t b_lo, uint32_t b_hi, uint32_t a_lo,
                                             uint32_t a_hi, uint32_t sp, v4i (&b)[8], v4i& al,
                                             v4i& ah, v4i& sa) {
  asm volatile(
      "ds_read_b128 %0, %11\n\t"
      "ds_read_b128 %1, %12\n\t"
      "ds_read_b128 %2, %11 offset:2048\n\t"
      "ds_read_b128 %3, %12 offset:2048\n\t"
      "ds_read_b128 %4, %11 offset:4096\n\t"
      "ds_read_b128 %5, %12 offset:4096\n\t"
      "ds_read_b128 %6, %11 offset:6144\n\t"
      "ds_read_b128 %7, %12 offset:6144\n\t"
      "ds_read_b128 %8, %13\n\t"
      "ds_read_b128 %9, %14\n\t"
      "ds_read_b128 %10, %15\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(b[0]), "=&v"(b[1]), "=&v"(b[2]), "=&v"(b[3]), "=&v"(b[4]), "=&v"(b[5]),
        "=&v"(b[6]), "=&v"(b[7]), "=&v"(al), "=&v"(ah), "=&v"(sa)
      : "v"(b_lo), "v"(b_hi), "v"(a_lo), "v"(a_hi), "v"(sp)
      : "memory");
}
__device__ __forceinline__ void lds_read_a(uint32_t a_lo, uint32_t a_hi, uint32_t sp, v4i& al,
                                           v4i& ah, v4i& sa) {
  asm volatile(
      "ds_read_b128 %0, %3\n\t"
      "ds_read_b128 %1, %4\n\t"
      "ds_read_b128 %2, %5\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(al), "=&v"(ah), "=&v"(sa)
      : "v"(a_lo), "v"(a_hi), "v"(sp)
      : "memory");
}

// One pipeline stage. Each stage is its own LDS object: the compiler then tells
// the fragment reads of one stage from the direct-to-LDS loads in flight into the
// others (it tracks such loads per LDS object) and does not drain them all.
template <int MT, int NW>
struct RowTileStage {
  uint8_t b[NW][8192];                      // wave w's 64 weight rows x 128 bytes
  uint8_t a[MT / 8 + 1][1024];              // activation rows, 8 per slot (+ a spare slot)
  float as[(MT + 63) / 64 + 1][64];         // activation scales (+ a spare slot)
};

template <int MT, int KIND, int PD, int NW>
__global__ __launch_bounds__(64 * NW) void expert_gemm_kernel(GemmArgs p) {
  constexpr int MS = MT / 16;
  constexpr int AQ = MT / 8;                // activation loads (8 rows) per stage
  constexpr int NA = (AQ + NW - 1) / NW;    // ... per wave (spare ones go to slot AQ)
  constexpr int NSQ = (MT + 63) / 64;       // scale loads (64 rows) per stage
  constexpr int NV = 8 + NA + 1;            // direct-to-LDS loads per wave per stage
  static_assert(PD >= 2 && PD <= 4 && (PD - 2) * NV < 64, "pipeline depth");
  using Stage = RowTileStage<MT, NW>;
  static_assert(NW == 4 || (KIND == 1 && NW == 2), "waves per workgroup");
  static_assert(NW * 64 >= MT, "one thread per tile row");
  __shared__ __attribute__((aligned(1024))) Stage st0;
  __shared__ __attribute__((aligned(1024))) Stage st1;
  __shared__ __attribute__((aligned(1024))) Stage st2;
  __shared__ __attribute__((aligned(1024))) Stage st3;
  __shared__ float sWs[2][kRowTileMaxKB];
  __shared__ long sSrc[MT];
  __shared__ float sRed[4][MT];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, r16 = lane & 15;
  const int Kdim = (KIND == 0) ? p.H : p.I;
  const int KB = Kdim / MOE_GROUP;
  const int NT = (KIND == 0) ? p.I / 128 : p.H / (64 * NW);
  const int total = p.num_tiles[0] * NT;

  for (int wi = blockIdx.x; wi < total; wi += gridDim.x) {
    const int tile = wi / NT, nt = wi - tile * NT;
    const int4 td = p.tiles[tile];
    const int e = td.x, nrows = td.z;
    const long slot0 = td.y;
    const long row0 = td.w;  // first hq / y row of the tile
    if (e < 0 || e >= p.E + p.nsh) continue;  // workgroup-uniform: malformed tile
    const bool is_sh = e >= p.E;
    const int ej = is_sh ? e - p.E : e;

    const uint8_t* wb;
    const float* wsb;
    if (KIND == 0) {
      wb = (is_sh ? p.wsh : p.w) + (size_t)ej * 2 * p.I * p.H;
      wsb = (is_sh ? p.wssh : p.ws) + (size_t)ej * (2 * p.I / 128) * KB;
    } else {
      wb = (is_sh ? p.wsh : p.w) + (size_t)ej * p.H * p.I;
      wsb = (is_sh ? p.wssh : p.ws) + (size_t)ej * (p.H / 128) * KB;
    }
    // Sources of the tile's rows: the token (gate_up) or the h row (down); -1 padding.
    // Down rows and one-token gate_up rows need no load (direct), so then the first
    // stages go out right after the tile descriptor, with the weight block scales,
    // instead of one round trip later behind the token ids and a barrier.
    const bool direct = KIND == 1 || p.tok0 != 0;  // workgroup-uniform
    auto direct_src = [&](int r) -> long { return r < nrows ? (KIND == 0 ? 0L : row0 + r) : -1L; };
    auto fill_tables = [&]() {
      if (tid < MT) {
        long src = -1;
        if (direct) {
          src = direct_src(tid);
        } else if (tid < nrows) {
          const long slot = slot0 + tid;
          src = is_sh ? slot - p.NB - (long)ej * p.T : (long)p.tpid[slot];
          if (src >= p.T) src = -1;  // token ids outside [0, T) are treated as padding
        }
        sSrc[tid] = src;
      }
      // weight block scales of the tile's two 128-row halves: gate / up blocks
      // (gate_up) or the two output blocks (down)
      for (int i = tid; i < (KIND == 0 ? 2 : NW / 2) * KB; i += 64 * NW) {
        const int h = i / KB, kb = i - h * KB;
        const int rb = (KIND == 0) ? (h == 0 ? nt : p.I / 128 + nt) : nt * (NW / 2) + h;
        sWs[h][kb] = wsb[(size_t)rb * KB + kb];
      }
      __syncthreads();
    };
    if (!direct) fill_tables();

    // Load sources. Weight load i of wave w: rows [8i, 8i + 8) of the wave's 64
    // (16-row column tile j = i / 2), lane l -> row 8 (i & 1) + l / 8 of the
    // column tile, stored chunk l % 8 = logical chunk swz(row, l % 8).
    uint32_t boff[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int j = i >> 1, rr = (i & 1) * 8 + (lane >> 3);
      int row;
      if (KIND == 0)
        row = (j < 2) ? nt * 128 + wave * 32 + j * 16 + rr
                      : p.I + nt * 128 + wave * 32 + (j - 2) * 16 + rr;
      else
        row = nt * 64 * NW + wave * 64 + j * 16 + rr;
      boff[i] = (uint32_t)row * (uint32_t)Kdim + (uint32_t)swz(rr, lane & 7) * 16;
    }
    // Activation load a of wave w: tile rows [8q, 8q + 8), q = w NA + a (q >= AQ:
    // a spare load of row 0 into slot AQ). Rows without a source read row 0; their
    // products are never stored.
    const uint8_t* aptr[NA];
    int aslot[NA];
#pragma unroll
    for (int a = 0; a < NA; ++a) {
      const int q = wave * NA + a;
      const int r = q * 8 + (lane >> 3);
      long src = 0;
      if (q < AQ) {
        const long sr = direct ? direct_src(r) : sSrc[r];
        if (sr >= 0) src = sr;
      }
      aslot[a] = q < AQ ? q : AQ;
      aptr[a] = p.a + (size_t)src * Kdim + swz(r, lane & 7) * 16;
    }
    // Scale load: wave w < NSQ fills the scales of rows [64 w, 64 w + 64).
    long ssrc = 0;
    {
      const int r = wave * 64 + lane;
      if (wave < NSQ && r < MT) {
        const long sr = direct ? direct_src(r) : sSrc[r];
        if (sr >= 0) ssrc = sr;
      }
    }
    const float* asp = p.as + (size_t)ssrc * KB;
    const int sslot = wave < NSQ ? wave : NSQ;

    auto issue = [&](Stage& S, int kb) {
#pragma unroll
      for (int i = 0; i < 8; ++i) load_lds16_nt(wb + boff[i] + (size_t)kb * MOE_GROUP, &S.b[wave][i * 1024]);
#pragma unroll
      for (int a = 0; a < NA; ++a) load_lds16(aptr[a] + (size_t)kb * MOE_GROUP, &S.a[aslot[a]][0]);
      load_lds4(asp + kb, (uint8_t*)&S.as[sslot][0]);
    };

    v4f acc[MS][4];
#pragma unroll
    for (int ms = 0; ms < MS; ++ms)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[ms][j] = (v4f){0.f, 0.f, 0.f, 0.f};

    // Fragment reads: row r16 of a 16-row group sits in load slot 2m + r16 / 8 at
    // byte (r16 % 8) * 128; its logical chunks g and 4 + g are stored swizzled.
    const int fr = (r16 >> 3) * 1024 + (r16 & 7) * 128;
    const int o_lo = fr + swz(r16, g) * 16, o_hi = fr + swz(r16, 4 + g) * 16;
    auto cat = [](const v4i& lo, const v4i& hi) -> v8i {
      return (v8i){lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
    };

    // Step kb: wait for block kb (stage cur), then load block kb + PD - 1 into the
    // stage block kb - 1 used (nxt; past the end, the last block again into a
    // stage that is not read again, so the waits stay exact) and multiply block kb.
    auto step = [&](int kb, Stage& cur, Stage& nxt) {
      __builtin_amdgcn_sched_barrier(0);
      wait_vm<(PD - 2) * NV>();      // this wave's share of block kb has landed
      __builtin_amdgcn_s_barrier();  // ... every wave's, and block kb - 1 is consumed
      __builtin_amdgcn_sched_barrier(0);
      issue(nxt, min(kb + PD - 1, KB - 1));
      __builtin_amdgcn_sched_barrier(0);
      const float sw0 = (KIND == 0) ? sWs[0][kb] : sWs[wave >> 1][kb];
      const float sw1 = (KIND == 0) ? sWs[1][kb] : sw0;
      const uint32_t bw = lds_addr(&cur.b[wave][0]), aw = lds_addr(&cur.a[0][0]);
      v4i bq[8];
      v8i b[4];
#pragma unroll
      for (int ms = 0; ms < MS; ++ms) {
        v4i alo, ahi, sai;
        const uint32_t sp = lds_addr(&cur.as[(ms * 16) >> 6][(ms * 16 + 4 * g) & 63]);
        if (ms == 0) {
          lds_read_b_a(bw + o_lo, bw + o_hi, aw + o_lo, aw + o_hi, sp, bq, alo, ahi, sai);
#pragma unroll
          for (int j = 0; j < 4; ++j) b[j] = cat(bq[2 * j], bq[2 * j + 1]);
        } else {
          lds_read_a(aw + 2048 * ms + o_lo, aw + 2048 * ms + o_hi, sp, alo, ahi, sai);
        }
        const v8i a = cat(alo, ahi);
        const v4f sa = {__int_as_float(sai.x), __int_as_float(sai.y), __int_as_float(sai.z), __int_as_float(sai.w)};
        const v4f c0 = sa * sw0;
        const v4f c1 = sa * sw1;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const v4f part = mfma_fp8(a, b[j]);
          acc[ms][j] += part * ((KIND == 0 && j >= 2) ? c1 : c0);
        }
      }
    };
    wait_vm<0>();  // no earlier load is still landing in a stage buffer
    issue(st0, 0);
    if (PD >= 3) issue(st1, min(1, KB - 1));
    if (PD >= 4) issue(st2, min(2, KB - 1));
    // direct: the scale loads follow the stages, and the wait for them before their
    // LDS stores (the compiler's, which counts only its own loads: vmcnt 0) covers the
    // first stages as well, so the first step's wait stays exact
    if (direct) fill_tables();
    for (int kb = 0; kb < KB; kb += PD) {
      if (PD == 2) {
        step(kb, st0, st1);
        if (kb + 1 < KB) step(kb + 1, st1, st0);
      } else if (PD == 3) {
        step(kb, st0, st2);
        if (kb + 1 < KB) step(kb + 1, st1, st0);
        if (kb + 2 < KB) step(kb + 2, st2, st1);
      } else {
        step(kb, st0, st3);
        if (kb + 1 < KB) step(kb + 1, st1, st0);
        if (kb + 2 < KB) step(kb + 2, st2, st1);
        if (kb + 3 < KB) step(kb + 3, st3, st2);
      }
    }
    wait_vm<0>();  // the tail's repeated loads land before the stages are reused

    // Per-output-channel weight scales, 1 when absent (a multiply by 1 is exact):
    // accumulator column j of this wave is weight row nt * 128 + 32 wave + 16 j + r16
    // (gate, j < 2; the up rows follow I later) or nt * 64 NW + 64 wave + 16 j + r16 (down).
    float cw[4] = {1.f, 1.f, 1.f, 1.f};
    if (const float* csb = is_sh ? p.cssh : p.cs) {
      csb += (size_t)ej * ((KIND == 0) ? 2 * p.I : p.H);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        cw[j] = csb[(KIND == 0) ? ((j < 2 ? 0 : p.I) + nt * 128 + wave * 32 + (j & 1) * 16 + r16)
                                : (nt * 64 * NW + wave * 64 + j * 16 + r16)];
    }

    if (KIND == 0) {
      // h = SiLU(gate) * up, written over the gate accumulators.
#pragma unroll
      for (int ms = 0; ms < MS; ++ms) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float m = 0.f;
#pragma unroll
          for (int jj = 0; jj < 2; ++jj) {
            const float gt = acc[ms][jj][i] * cw[jj], up = acc[ms][jj + 2][i] * cw[jj + 2];
            // hardware reciprocal (about 1 ulp): h only feeds the 1x128 fp8 quantization
            const float h = gt * __builtin_amdgcn_rcpf(1.0f + __expf(-gt)) * up;
            acc[ms][jj][i] = h;
            m = fmaxf(m, fabsf(h));
          }
          m = group16_max_f32(m);
          if (r16 == 0) sRed[wave][ms * 16 + 4 * g + i] = m;
        }
      }
      __syncthreads();
      const int GI = p.I / MOE_GROUP;
#pragma unroll
      for (int ms = 0; ms < MS; ++ms) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = ms * 16 + 4 * g + i;
          const float amax = fmaxf(fmaxf(sRed[0][row], sRed[1][row]), fmaxf(sRed[2][row], sRed[3][row]));
          const float sc = fmaxf(amax, 0x1.b7cdfep-34f) / 448.0f;
          if (sSrc[row] >= 0) {
            const long hrow_i = row0 + row;
            const float rs = 1.0f / sc;
            const uint32_t c2 = e4m3x2(fminf(fmaxf(div_by(acc[ms][0][i], sc, rs), -448.0f), 448.0f),
                                       fminf(fmaxf(div_by(acc[ms][1][i], sc, rs), -448.0f), 448.0f));
            uint8_t* const hrow = p.hq + (size_t)hrow_i * p.I + nt * 128 + wave * 32 + r16;
            hrow[0] = (uint8_t)c2;
            hrow[16] = (uint8_t)(c2 >> 8);
            if (wave == 0 && r16 == 0) p.hs[(size_t)hrow_i * GI + nt] = sc;
          }
        }
      }
    } else {
#pragma unroll
      for (int ms = 0; ms < MS; ++ms) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = ms * 16 + 4 * g + i;
          if (row < nrows) {
            const long yrow = row0 + row;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const int col = nt * 64 * NW + wave * 64 + j * 16 + r16;
              p.y[(size_t)yrow * p.H + col] = (uint16_t)bf16x2(acc[ms][j][i] * cw[j], 0.f);
            }
          }
        }
      }
    }
    __syncthreads();
  }
}

// Single-wave checks of the fragment mappings:
//   16x16: c[16,16] = a[16,128] . b[16,128]^T with the mapping above;
//   32x32: c[32,32] = a[32,128] . b[32,128]^T with the block-kernel mapping
//          (lane l: row l%32, bytes [h*64 + (l/32)*32, +32) for MFMA h).
typedef float v16f_t __attribute__((ext_vector_type(16)));

__global__ void selftest_mfma_kernel(const uint8_t* a, const uint8_t* b, float* c, int shape) {
  const int lane = threadIdx.x;
  if (shape == 0) {
    const int g = lane >> 4, r16 = lane & 15;
    const v8i fa = load_frag_global(a + r16 * 128 + g * 16);
    const v8i fb = load_frag_global(b + r16 * 128 + g * 16);
    const v4f d = mfma_fp8(fa, fb);
#pragma unroll
    for (int i = 0; i < 4; ++i) c[(4 * g + i) * 16 + r16] = d[i];
  } else {
    const int g2 = lane >> 5, l32 = lane & 31;
    v16f_t d = {};
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int4* pa = (const int4*)(a + l32 * 128 + h * 64 + g2 * 32);
      const int4* pb = (const int4*)(b + l32 * 128 + h * 64 + g2 * 32);
      const v8i fa = (v8i){pa[0].x, pa[0].y, pa[0].z, pa[0].w, pa[1].x, pa[1].y, pa[1].z, pa[1].w};
      const v8i fb = (v8i){pb[0].x, pb[0].y, pb[0].z, pb[0].w, pb[1].x, pb[1].y, pb[1].z, pb[1].w};
      d = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fa, fb, d, 0, 0, 0, 0, 0, 0);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) c[(8 * (r >> 2) + 4 * g2 + (r & 3)) * 32 + l32] = d[r];
  }
}

template <int KIND>
static int launch_gemm(const GemmArgs& a, int max_tiles, int mt, hipStream_t st) {
  // down at 16 and 32 rows: 128 weight rows per workgroup (2 waves), so two
  // workgroups share a CU and one's start-up overlaps the other's weight stream
  constexpr int NWD = (KIND == 1) ? 2 : 4;
  const int nw = (mt <= 32) ? NWD : 4;
  const int NT = (KIND == 0) ? a.I / 128 : a.H / (64 * nw);
  const long items = (long)max_tiles * NT;
  const int grid = (int)std::max(1L, std::min(items, 4096L * 4 / nw));
  switch (mt) {
    case 16:
      hipLaunchKernelGGL((expert_gemm_kernel<16, KIND, 3, NWD>), dim3(grid), dim3(64 * NWD), 0, st, a);
      break;
    case 32:
      hipLaunchKernelGGL((expert_gemm_kernel<32, KIND, 3, NWD>), dim3(grid), dim3(64 * NWD), 0, st, a);
      break;
    case 64:
      hipLaunchKernelGGL((expert_gemm_kernel<64, KIND, 3, 4>), dim3(grid), dim3(256), 0, st, a);
      break;
    case 128:
      hipLaunchKernelGGL((expert_gemm_kernel<128, KIND, 2, 4>), dim3(grid), dim3(256), 0, st, a);
      break;
    default:
      return MOE_ERR_ARG;
  }
  return MOE_OK;
}

}  // namespace moe

using namespace moe;

#define MOE_CHECK_ALIGN16(ptr) \
  MOE_CHECK_ARG(((uintptr_t)(ptr)&15) == 0, "%s must be 16-byte aligned", #ptr)

// moe_expert_gate_up; tok0: every slot of a tile holds token 0 (T = 1 and tiles from
// the layer's own mapping), so the kernel loads no token ids.
static int gate_up_entry(const uint8_t* xq, const float* xs, int T, int H, int I, int E,
                         const uint8_t* w13, const float* w13_scale, const float* w13_channel_scale,
                         const uint8_t* w13_shared, const float* w13_shared_scale,
                         const float* w13_shared_channel_scale, int n_shared,
                         const int32_t* token_position_to_id, int NB, const int32_t* tiles,
                         const int32_t* num_tiles, int max_tiles, int mt, uint8_t* hq, float* hs,
                         void* stream, int tok0) {
  MOE_API_BEGIN("moe_expert_gate_up");
  MOE_CHECK_ARG(xq && xs && w13 && w13_scale && token_position_to_id && tiles && num_tiles && hq && hs,
                "null pointer argument");
  MOE_CHECK_ARG(T > 0 && E > 0 && NB >= 0 && max_tiles > 0, "bad sizes");
  MOE_CHECK_ARG(H > 0 && H % 128 == 0 && I > 0 && I % 128 == 0,
                "H and I must be positive multiples of 128 (H=%d I=%d)", H, I);
  MOE_CHECK_SUPPORTED(H <= 128 * kRowTileMaxKB && I <= 128 * kRowTileMaxKB && 2L * I * H < (1L << 32),
                      "H and I up to %d and one expert's weights under 4 GiB (H=%d I=%d)",
                      128 * kRowTileMaxKB, H, I);
  MOE_CHECK_ARG(n_shared == 0 || (w13_shared && w13_shared_scale), "shared weights missing");
  MOE_CHECK_ARG(mt == 16 || mt == 32 || mt == 64 || mt == 128, "mt must be 16/32/64/128");
  MOE_CHECK_ALIGN16(xq);
  MOE_CHECK_ALIGN16(w13);
  MOE_CHECK_ARG(n_shared == 0 || ((uintptr_t)w13_shared & 15) == 0, "w13_shared misaligned");
  GemmArgs a{};
  a.a = xq;
  a.as = xs;
  a.w = w13;
  a.ws = w13_scale;
  a.wsh = w13_shared;
  a.wssh = w13_shared_scale;
  a.cs = w13_channel_scale;
  a.cssh = w13_shared_channel_scale;
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
  a.tok0 = (tok0 != 0 && T == 1) ? 1 : 0;
  if (launch_gemm<0>(a, max_tiles, mt, (hipStream_t)stream) != MOE_OK)
    MOE_CHECK_ARG(false, "bad mt %d", mt);
  MOE_API_END();
}

extern "C" int moe_expert_gate_up(const uint8_t* xq, const float* xs, int T, int H, int I, int E,
                                  const uint8_t* w13, const float* w13_scale,
                                  const float* w13_channel_scale, const uint8_t* w13_shared,
                                  const float* w13_shared_scale,
                                  const float* w13_shared_channel_scale, int n_shared,
                                  const int32_t* token_position_to_id, int NB,
                                  const int32_t* tiles, const int32_t* num_tiles, int max_tiles,
                                  int mt, uint8_t* hq, float* hs, void* stream) {
  return gate_up_entry(xq, xs, T, H, I, E, w13, w13_scale, w13_channel_scale, w13_shared,
                       w13_shared_scale, w13_shared_channel_scale, n_shared, token_position_to_id, NB,
                       tiles, num_tiles, max_tiles, mt, hq, hs, stream, 0);
}

int moe::layer_gate_up(const uint8_t* xq, const float* xs, int T, int H, int I, int E,
                       const uint8_t* w13, const float* w13_scale, const uint8_t* w13_shared,
                       const float* w13_shared_scale, int n_shared, const int32_t* tpid, int NB,
                       const int32_t* tiles, const int32_t* num_tiles, int max_tiles, int mt,
                       uint8_t* hq, float* hs, void* stream) {
  return gate_up_entry(xq, xs, T, H, I, E, w13, w13_scale, nullptr, w13_shared, w13_shared_scale,
                       nullptr, n_shared, tpid, NB, tiles, num_tiles, max_tiles, mt, hq, hs, stream, 1);
}

extern "C" int moe_expert_down(const uint8_t* hq, const float* hs, int T, int H, int I, int E,
                               const uint8_t* w2, const float* w2_scale,
                               const float* w2_channel_scale, const uint8_t* w2_shared,
                               const float* w2_shared_scale, const float* w2_shared_channel_scale,
                               int n_shared, int NB,
                               const int32_t* tiles, const int32_t* num_tiles, int max_tiles,
                               int mt, void* y_bf16, void* stream) {
  MOE_API_BEGIN("moe_expert_down");
  MOE_CHECK_ARG(hq && hs && w2 && w2_scale && tiles && num_tiles && y_bf16, "null pointer argument");
  MOE_CHECK_ARG(T > 0 && E > 0 && NB >= 0 && max_tiles > 0, "bad sizes");
  MOE_CHECK_ARG(H > 0 && H % 256 == 0 && I > 0 && I % 128 == 0,
                "H must be a multiple of 256 and I of 128 (H=%d I=%d)", H, I);
  MOE_CHECK_SUPPORTED(H <= 128 * kRowTileMaxKB && I <= 128 * kRowTileMaxKB && 2L * I * H < (1L << 32),
                      "H and I up to %d and one expert's weights under 4 GiB (H=%d I=%d)",
                      128 * kRowTileMaxKB, H, I);
  MOE_CHECK_ARG(n_shared == 0 || (w2_shared && w2_shared_scale), "shared weights missing");
  MOE_CHECK_ARG(mt == 16 || mt == 32 || mt == 64 || mt == 128, "mt must be 16/32/64/128");
  MOE_CHECK_ALIGN16(hq);
  MOE_CHECK_ALIGN16(w2);
  MOE_CHECK_ARG(n_shared == 0 || ((uintptr_t)w2_shared & 15) == 0, "w2_shared misaligned");
  GemmArgs a{};
  a.a = hq;
  a.as = hs;
  a.w = w2;
  a.ws = w2_scale;
  a.wsh = w2_shared;
  a.wssh = w2_shared_scale;
  a.cs = w2_channel_scale;
  a.cssh = w2_shared_channel_scale;
  a.tiles = (const int4*)tiles;
  a.num_tiles = num_tiles;
  a.y = (uint16_t*)y_bf16;
  a.T = T;
  a.H = H;
  a.I = I;
  a.E = E;
  a.nsh = n_shared;
  a.NB = NB;
  if (launch_gemm<1>(a, max_tiles, mt, (hipStream_t)stream) != MOE_OK)
    MOE_CHECK_ARG(false, "bad mt %d", mt);
  MOE_API_END();
}

// Every fp32 bit pattern u in [first, first + count) with |value| <= 448, both
// signs: the conversion instruction against the integer encoder. Workgroup b
// writes its mismatch count to out[b] and its smallest mismatching pattern (or
// 0xffffffff) to out[gridDim.x + b].
__global__ __launch_bounds__(256) void selftest_fp8_encode_kernel(uint32_t first, uint32_t count,
                                                                  uint32_t* out) {
  __shared__ uint32_t s_n[256], s_min[256];
  uint32_t n = 0, mn = 0xffffffffu;
  const uint32_t stride = gridDim.x * blockDim.x;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < count; i += stride) {
    const uint32_t u = first + i;
    const float v = __uint_as_float(u & 0x7fffffffu);
    if (!(v <= 448.0f)) continue;
    const uint32_t hw = e4m3x2(v, -v);
    const uint32_t sw = f32_to_e4m3fn(v) | (f32_to_e4m3fn(-v) << 8);
    if (hw != sw) {
      ++n;
      mn = min(mn, u);
    }
  }
  s_n[threadIdx.x] = n;
  s_min[threadIdx.x] = mn;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) {
      s_n[threadIdx.x] += s_n[threadIdx.x + o];
      s_min[threadIdx.x] = min(s_min[threadIdx.x], s_min[threadIdx.x + o]);
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    out[blockIdx.x] = s_n[0];
    out[gridDim.x + blockIdx.x] = s_min[0];
  }
}

// div_by against the IEEE division: a mismatch is a different e4m3 code of the
// clamped quotient, or a different fp32 quotient of magnitude at least 2^-10 (the
// smallest with a nonzero code; far below it the correction step's residual can
// underflow, for subnormal values, and the quotient is then only within one ulp).
// Mode 0: index u in [first, first + count)
// (u < 2^31) is the pair (bf16 group amax m = u >> 16, bf16 value v = u & 0xffff)
// of the 1x128 quantizer, skipped unless both are finite and |v| <= m; the
// divisor is max(m, 1e-10) / 448. Mode 1: index u seeds a random fp32 amax in
// [2^-40, 2^40) and a random fp32 value of magnitude at most amax. Same output
// layout as the encoder check.
__global__ __launch_bounds__(256) void selftest_quant_div_kernel(int mode, uint32_t first,
                                                                 uint32_t count, uint32_t* out) {
  __shared__ uint32_t s_n[256], s_min[256];
  uint32_t n = 0, mn = 0xffffffffu;
  const uint32_t stride = gridDim.x * blockDim.x;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < count; i += stride) {
    const uint32_t u = first + i;
    float v, m;
    if (mode == 0) {
      m = bf16_bits_to_f32((uint16_t)((u >> 16) & 0x7fffu));
      v = bf16_bits_to_f32((uint16_t)(u & 0xffffu));
      if (!(fabsf(v) <= m) || !(m < INFINITY)) continue;
    } else {
      uint32_t h = u * 0x9E3779B1u;  // integer hash of the index
      h ^= h >> 15;
      h *= 0x85EBCA77u;
      h ^= h >> 13;
      uint32_t h2 = h * 0xC2B2AE3Du;
      h2 ^= h2 >> 16;
      const uint32_t em = 87u + (h % 80u);  // amax exponent field: 2^-40 .. 2^39
      m = __uint_as_float((em << 23) | (h2 & 0x7fffffu));
      const uint32_t ev = em - (h2 >> 23) % 40u;  // value up to 39 binades below
      v = __uint_as_float(((h >> 31) << 31) | (ev << 23) | ((h2 * 0x27d4eb2du) & 0x7fffffu));
      if (fabsf(v) > m) v = copysignf(m, v);
    }
    const float sc = fmaxf(m, 0x1.b7cdfep-34f) / 448.0f;
    const float rs = 1.0f / sc;
    const float qi = v / sc, qf = div_by(v, sc, rs);
    const uint32_t ci = e4m3x2(fminf(fmaxf(qi, -448.0f), 448.0f), 0.f);
    const uint32_t cf = e4m3x2(fminf(fmaxf(qf, -448.0f), 448.0f), 0.f);
    if (ci != cf || (fabsf(qi) >= 0x1p-10f && __float_as_uint(qi) != __float_as_uint(qf))) {
      ++n;
      mn = min(mn, u);
    }
  }
  s_n[threadIdx.x] = n;
  s_min[threadIdx.x] = mn;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) {
      s_n[threadIdx.x] += s_n[threadIdx.x + o];
      s_min[threadIdx.x] = min(s_min[threadIdx.x], s_min[threadIdx.x + o]);
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    out[blockIdx.x] = s_n[0];
    out[gridDim.x + blockIdx.x] = s_min[0];
  }
}

extern "C" int moe_selftest_quant_div(int mode, uint32_t first, uint32_t count, uint32_t* out,
                                      int blocks, void* stream) {
  MOE_API_BEGIN("moe_selftest_quant_div");
  MOE_CHECK_ARG(out && blocks > 0 && blocks <= 65536 && (mode == 0 || mode == 1), "bad arguments");
  MOE_CHECK_ARG((uint64_t)first + count <= 0x80000000ull, "range must lie in [0, 2^31)");
  hipLaunchKernelGGL(selftest_quant_div_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream,
                     mode, first, count, out);
  MOE_API_END();
}

// Every fp32 bit pattern u in [first, first + count): the bf16 conversion
// instruction against the integer encoder (a NaN only has to stay a NaN). Same
// output layout as the e4m3 check.
__global__ __launch_bounds__(256) void selftest_bf16_encode_kernel(uint32_t first, uint32_t count,
                                                                   uint32_t* out) {
  __shared__ uint32_t s_n[256], s_min[256];
  uint32_t n = 0, mn = 0xffffffffu;
  const uint32_t stride = gridDim.x * blockDim.x;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < count; i += stride) {
    const uint32_t u = first + i;
    const float v = __uint_as_float(u);
    const uint32_t hw = bf16x2(v, 0.f) & 0xffffu;
    const uint32_t sw = f32_to_bf16_bits(v);
    const bool same = (v != v) ? ((hw & 0x7fffu) > 0x7f80u) : (hw == sw);
    if (!same) {
      ++n;
      mn = min(mn, u);
    }
  }
  s_n[threadIdx.x] = n;
  s_min[threadIdx.x] = mn;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) {
      s_n[threadIdx.x] += s_n[threadIdx.x + o];
      s_min[threadIdx.x] = min(s_min[threadIdx.x], s_min[threadIdx.x + o]);
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    out[blockIdx.x] = s_n[0];
    out[gridDim.x + blockIdx.x] = s_min[0];
  }
}

extern "C" int moe_selftest_bf16_encode(uint32_t first, uint32_t count, uint32_t* out, int blocks,
                                        void* stream) {
  MOE_API_BEGIN("moe_selftest_bf16_encode");
  MOE_CHECK_ARG(out && blocks > 0 && blocks <= 65536, "bad arguments");
  MOE_CHECK_ARG((uint64_t)first + count <= 0x100000000ull, "range must lie in [0, 2^32)");
  hipLaunchKernelGGL(selftest_bf16_encode_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream,
                     first, count, out);
  MOE_API_END();
}

extern "C" int moe_selftest_fp8_encode(uint32_t first, uint32_t count, uint32_t* out, int blocks,
                                       void* stream) {
  MOE_API_BEGIN("moe_selftest_fp8_encode");
  MOE_CHECK_ARG(out && blocks > 0 && blocks <= 65536, "bad arguments");
  MOE_CHECK_ARG((uint64_t)first + count <= 0x80000000ull, "range must lie in [0, 2^31)");
  hipLaunchKernelGGL(selftest_fp8_encode_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream,
                     first, count, out);
  MOE_API_END();
}

extern "C" int moe_selftest_mfma_fp8(const uint8_t* a, const uint8_t* b, float* c, int shape,
                                     void* stream) {
  MOE_API_BEGIN("moe_selftest_mfma_fp8");
  MOE_CHECK_ARG(a && b && c, "null pointer argument");
  MOE_CHECK_ARG(shape == 0 || shape == 1, "shape must be 0 (16x16x128) or 1 (32x32x64)");
  MOE_CHECK_ALIGN16(a);
  MOE_CHECK_ALIGN16(b);
  hipLaunchKernelGGL(selftest_mfma_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, a, b, c,
                     shape);
  MOE_API_END();
}
