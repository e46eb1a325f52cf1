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
// row tile holds up to MT consecutive slots of one expert; a workgroup (NW = 4
// waves, or 2 for one-token decode, which would otherwise leave CUs idle) owns
// 64 NW weight rows (gate_up: 32 NW gate rows + the matching up rows, so a wave
// holds 32 h columns = one MX block of h; down: 64 NW output columns). Weight
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
  // the layer at one token (tiles from its own mapping: one row each, token 0)
  int one;
};

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

// ---------------------------------------------------------------------------
// The MX row-tile kernel. Like the fp8 row-tile kernel, every operand arrives by
// direct-to-LDS loads into a PD-stage ring whose stages are separate LDS objects,
// eight lanes per 128-byte weight row segment so each load instruction reads
// eight whole cache lines. A stage is one 128-byte segment of each weight row:
// two 128-K blocks of MXFP4 (64 bytes each) or one of MXFP8, with the matching
// MXFP8 activation rows and the E8M0 scale dwords of both operands. Every wave
// issues the same number of loads per stage (NV; spare loads go to spare slots),
// so the wait for the oldest stage is a compile-time vmcnt; the fragment reads
// are asm statements that wait for their own data (see gemm_fp8.hip).
// ---------------------------------------------------------------------------
template <int MT, int WFMT, bool TBL, int NW>
struct MxStage {
  static constexpr int KPS = (WFMT == kFmtFp4) ? 2 : 1;  // 128-K blocks per stage
  static constexpr int AQ = MT / 8;                     // activation loads per K block
  static constexpr int NSQ = (MT + 63) / 64;            // activation scale loads per K block
  uint8_t b[NW][8192];                 // wave w's 64 weight rows x 128 bytes
  uint32_t bs[TBL ? 1 : NW][KPS][64];   // their scale dwords (row 16 j + r of the wave; unused
                                       // with the per-item scale table)
  uint8_t a[KPS * AQ + 1][1024];       // activation rows: slot kk * AQ + q = rows 8q.. of block kk
  uint32_t as[KPS][NSQ + 1][64];       // activation scale dwords per 64-row group (+ a spare)
};

// Per-item weight scale table (K <= 4096): the E8M0 bytes of each wave's 64
// weight rows for the whole K, one 128-byte LDS row per weight row. Loaded once
// per work item with 16-byte direct-to-LDS loads (whole row segments) instead of
// one 4-byte load per row and stage, whose 64 distinct lines per instruction
// cost the load path more than the stage's weight tile. The table's 16-byte
// pieces are XOR-swizzled by row so a fragment's 16 rows hit distinct banks.
constexpr int kMxTblMaxK = 4096;

// Weight fragments of four 16-row column tiles (j at +2048 j), their four scale
// dwords (at +64 j), one activation fragment (lo / hi) and its scale dword, read
// in one statement that waits for its data. fp4 weights: one 16-byte chunk per
// tile (the MFMA's fp4 operand); fp8 weights: two.
// SST: byte stride between the column tiles' scale dwords (64 in a stage, 2048 in
// the per-item table).
template <int SST>
__device__ __forceinline__ void mx_read_w4(uint32_t b, uint32_t bs, uint32_t a_lo, uint32_t a_hi,
                                           uint32_t as, v4i (&w)[4], int (&ws)[4], v4i& al,
                                           v4i& ah, int& sa) {
  asm volatile(
      "ds_read_b128 %0, %11\n\t"
      "ds_read_b128 %1, %11 offset:2048\n\t"
      "ds_read_b128 %2, %11 offset:4096\n\t"
      "ds_read_b128 %3, %11 offset:6144\n\t"
      "ds_read_b32 %4, %12\n\t"
      "ds_read_b32 %5, %12 offset:%16\n\t"
      "ds_read_b32 %6, %12 offset:%17\n\t"
      "ds_read_b32 %7, %12 offset:%18\n\t"
      "ds_read_b128 %8, %13\n\t"
      "ds_read_b128 %9, %14\n\t"
      "ds_read_b32 %10, %15\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2]), "=&v"(w[3]), "=&v"(ws[0]), "=&v"(ws[1]),
        "=&v"(ws[2]), "=&v"(ws[3]), "=&v"(al), "=&v"(ah), "=&v"(sa)
      : "v"(b), "v"(bs), "v"(a_lo), "v"(a_hi), "v"(as), "n"(SST), "n"(2 * SST), "n"(3 * SST)
      : "memory");
}
template <int SST>
__device__ __forceinline__ void mx_read_w8(uint32_t b_lo, uint32_t b_hi, uint32_t bs, uint32_t a_lo,
                                           uint32_t a_hi, uint32_t as, v4i (&w)[8], int (&ws)[4],
                                           v4i& al, v4i& ah, int& sa) {
  asm volatile(
      "ds_read_b128 %0, %15\n\t"
      "ds_read_b128 %1, %16\n\t"
      "ds_read_b128 %2, %15 offset:2048\n\t"
      "ds_read_b128 %3, %16 offset:2048\n\t"
      "ds_read_b128 %4, %15 offset:4096\n\t"
      "ds_read_b128 %5, %16 offset:4096\n\t"
      "ds_read_b128 %6, %15 offset:6144\n\t"
      "ds_read_b128 %7, %16 offset:6144\n\t"
      "ds_read_b32 %8, %17\n\t"
      "ds_read_b32 %9, %17 offset:%21\n\t"
      "ds_read_b32 %10, %17 offset:%22\n\t"
      "ds_read_b32 %11, %17 offset:%23\n\t"
      "ds_read_b128 %12, %18\n\t"
      "ds_read_b128 %13, %19\n\t"
      "ds_read_b32 %14, %20\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2]), "=&v"(w[3]), "=&v"(w[4]), "=&v"(w[5]),
        "=&v"(w[6]), "=&v"(w[7]), "=&v"(ws[0]), "=&v"(ws[1]), "=&v"(ws[2]), "=&v"(ws[3]),
        "=&v"(al), "=&v"(ah), "=&v"(sa)
      : "v"(b_lo), "v"(b_hi), "v"(bs), "v"(a_lo), "v"(a_hi), "v"(as), "n"(SST), "n"(2 * SST),
        "n"(3 * SST)
      : "memory");
}
__device__ __forceinline__ void mx_read_a(uint32_t a_lo, uint32_t a_hi, uint32_t as, v4i& al,
                                          v4i& ah, int& sa) {
  asm volatile(
      "ds_read_b128 %0, %3\n\t"
      "ds_read_b128 %1, %4\n\t"
      "ds_read_b32 %2, %5\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(al), "=&v"(ah), "=&v"(sa)
      : "v"(a_lo), "v"(a_hi), "v"(as)
      : "memory");
}

// One work item's load sources (per lane).
template <int NA>
struct MxSrc {
  const uint8_t* wb;          // expert weights
  const uint8_t* wsb;         // expert weight scales
  uint32_t boff[8];           // weight rows of the lane's eight loads
  uint32_t bsoff;             // weight scale row of the lane's per-stage scale loads
  const uint8_t* aptr[NA];    // activation rows
  const uint8_t* asp;         // activation scale row
};

// 4-byte global load whose completion the caller's later vmcnt waits cover (the
// compiler does not count it, so it adds no wait that would drain the ring);
// vm_ready() marks the point after such a wait from which the value is used.
__device__ __forceinline__ int gload_i32(const void* p) {
  int v;
  asm volatile("global_load_dword %0, %1, off" : "=v"(v) : "v"(p) : "memory");
  return v;
}
__device__ __forceinline__ void vm_ready(int& v) { asm volatile("" : "+v"(v)); }

// Persistent streaming form: workgroup b runs items b, b + G, ... (G = grid) and
// keeps its load ring going across them. During item j's first step the next
// item's token ids and biases are requested; PD - 1 stages before item j ends
// the ring moves on to item j + 1, so item j's epilogue runs with item j + 1's
// first stages in flight. With the scale table, each wave reloads its own table
// rows for item j + 1 right after its last multiply of item j (no other wave
// reads them); with three stages the ring's second block of item j + 1 is issued
// after that reload, so the first step's wait covers the table as well. Items
// with fewer stages than the ring depth drain between items instead.
template <int MT, int KIND, int PD, int WFMT, bool TBL, int NW>
__global__ __launch_bounds__(64 * NW) void expert_gemm_mx_kernel(MxArgs p) {
  using Stage = MxStage<MT, WFMT, TBL, NW>;
  static_assert(NW == 4 || NW == 2, "waves per workgroup");
  constexpr int MS = MT / 16;
  constexpr int KPS = Stage::KPS, AQ = Stage::AQ, NSQ = Stage::NSQ;
  constexpr int NA = (KPS * AQ + NW - 1) / NW;  // activation loads per wave per stage
  constexpr int NV = 8 + (TBL ? 0 : KPS) + NA + KPS;  // direct-to-LDS loads per wave per stage
  static_assert(PD >= 2 && PD <= 6 && (PD - 2) * NV < 64, "pipeline depth");
  __shared__ __attribute__((aligned(1024))) Stage st[PD];
  __shared__ __attribute__((aligned(16))) uint8_t sTbl[TBL ? NW * 64 * 128 : 16];
  __shared__ long sSrc[2][MT];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, r16 = lane & 15;
  const int Kdim = (KIND == 0) ? p.H : p.I;
  const int KS = Kdim / 32;               // scale bytes per row
  const int NSTG = Kdim / (128 * KPS);    // stages (K % (128 KPS) == 0, checked by the entry points)
  const int NT = (KIND == 0) ? p.I / (32 * NW) : p.H / (64 * NW);
  const int total = p.num_tiles[0] * NT;
  const int G = gridDim.x;
  const std::integral_constant<int, WFMT> wfmt{};
  int wi = blockIdx.x;
  if (wi >= total) return;
  // crossing step NSTG - PD + 1 >= 1 follows the token loads; a ring deeper than
  // three stages (one item per workgroup) drains between items instead
  const bool stream = PD <= 3 && NSTG >= PD;
  const size_t wrow_bytes = (size_t)Kdim * ((WFMT == kFmtFp4) ? 64 : 128) / 128;
  const int rows_w = (KIND == 0) ? 2 * p.I : p.H;

  // Work item descriptor (workgroup-uniform); an expert out of range (only in a
  // malformed tile list) runs as expert 0 with no rows.
  struct ItemDesc {
    int e, nrows, nt;
    long slot0, row0;
  };
  typedef __attribute__((address_space(4))) const int* const_int_ptr;
  const const_int_ptr ctiles = (const_int_ptr)p.tiles;  // scalar loads: no vmcnt
  auto desc = [&](int w) {
    ItemDesc d;
    const int tile = w / NT;
    d.nt = w - tile * NT;
    const int4 td = make_int4(ctiles[4 * tile], ctiles[4 * tile + 1], ctiles[4 * tile + 2],
                              ctiles[4 * tile + 3]);
    const bool ok = td.x >= 0 && td.x < p.E + p.nsh;
    d.e = ok ? td.x : 0;
    d.nrows = ok ? td.z : 0;
    d.slot0 = td.y;
    d.row0 = td.w;
    return d;
  };
  // weight row of column tile j, row r of the tile, for this wave
  auto wrow_of = [&](const ItemDesc& d, int j, int r) -> int {
    if (KIND == 0)
      return (j < 2) ? d.nt * 32 * NW + wave * 32 + j * 16 + r
                     : p.I + d.nt * 32 * NW + wave * 32 + (j - 2) * 16 + r;
    return d.nt * 64 * NW + wave * 64 + j * 16 + r;
  };
  // token (gate_up) or h row (down) of tile row r; -1 for padding. tp: the
  // token-position entry (gate_up, routed experts).
  auto row_src = [&](const ItemDesc& d, int r, long tp) -> long {
    if (r >= d.nrows) return -1;
    if (KIND == 1) return d.row0 + r;
    const long s = (d.e >= p.E) ? d.slot0 + r - p.NB - (long)(d.e - p.E) * p.T : tp;
    return (s >= 0 && s < p.T) ? s : -1;  // token ids outside [0, T) are padding
  };
  auto tp_ptr = [&](const ItemDesc& d, int r) -> const int32_t* {  // gate_up only
    return p.tpid + ((d.e < p.E && r < d.nrows) ? d.slot0 + r : 0);
  };
  auto tp_read = [&](const ItemDesc& d, int r) -> long { return KIND == 0 ? (long)*tp_ptr(d, r) : 0; };
  auto bias_ptr = [&](const ItemDesc& d) -> const float* {
    const bool sh = d.e >= p.E;
    const float* bb = sh ? p.bsh : p.bias;
    return bb == nullptr ? nullptr : bb + (size_t)(sh ? d.e - p.E : d.e) * rows_w;
  };
  // rows behind the lane's activation loads (slot sl = wave NA + a: block kk = sl /
  // AQ, rows 8 (sl % AQ) + lane / 8; sl >= KPS AQ: a spare load of row 0)
  auto a_row = [&](int a) {
    const int sl = wave * NA + a;
    return ((sl < KPS * AQ) ? sl % AQ : 0) * 8 + (lane >> 3);
  };
  auto a_live = [&](int a) { return wave * NA + a < KPS * AQ; };
  const int s_row = wave * 64 + lane;
  const bool s_live = wave < NSQ && s_row < MT;
  int aslot[NA], akk[NA];
#pragma unroll
  for (int a = 0; a < NA; ++a) {
    const int sl = wave * NA + a;
    aslot[a] = (sl < KPS * AQ) ? sl : KPS * AQ;
    akk[a] = (sl < KPS * AQ) ? sl / AQ : 0;
  }
  const int sslot = wave < NSQ ? wave : NSQ;
  auto sources = [&](const ItemDesc& d, const long (&ta)[NA], long tsc) {
    MxSrc<NA> s;
    const bool sh = d.e >= p.E;
    const int ej = sh ? d.e - p.E : d.e;
    s.wb = (sh ? p.wsh : p.w) + (size_t)ej * rows_w * wrow_bytes;
    s.wsb = (sh ? p.wssh : p.ws) + (size_t)ej * rows_w * KS;
    // weight load i: rows 8 (i & 1) + l / 8 of column tile i / 2, stored chunk l % 8
    // = logical chunk swz(row, l % 8) of the row's 128-byte segment
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int rr = (i & 1) * 8 + (lane >> 3);
      s.boff[i] = (uint32_t)wrow_of(d, i >> 1, rr) * (uint32_t)wrow_bytes + (uint32_t)swz(rr, lane & 7) * 16;
    }
    // weight scale dword of row (j = l / 16, r = l % 16): byte offset of the row
    s.bsoff = (uint32_t)wrow_of(d, lane >> 4, lane & 15) * (uint32_t)KS;
#pragma unroll
    for (int a = 0; a < NA; ++a) {
      const long src = (a_live(a) && ta[a] >= 0) ? ta[a] : 0;  // no source: row 0, never stored
      s.aptr[a] = p.a + (size_t)src * Kdim + swz(a_row(a), lane & 7) * 16;
    }
    s.asp = p.as + (size_t)(tsc >= 0 ? tsc : 0) * KS;
    return s;
  };
  // Loads of stage t (K blocks [KPS t, KPS t + KPS)).
  auto issue = [&](const MxSrc<NA>& s, Stage& S, int t) {
    const size_t kb0 = (size_t)t * KPS;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      // decode tiles (<= 32 rows: one tile per expert) stream each weight once: the
      // non-temporal hint (GPT-OSS-120B 64 tokens -7 %); taller tiles re-read them
      if constexpr (MT <= 32)
        load_lds16_nt(s.wb + s.boff[i] + (size_t)t * 128, &S.b[wave][i * 1024]);
      else
        load_lds16(s.wb + s.boff[i] + (size_t)t * 128, &S.b[wave][i * 1024]);
    }
    if constexpr (!TBL) {
#pragma unroll
      for (int kk = 0; kk < KPS; ++kk)
        load_lds4(s.wsb + s.bsoff + (kb0 + kk) * 4, (uint8_t*)&S.bs[TBL ? 0 : wave][kk][0]);
    }
#pragma unroll
    for (int a = 0; a < NA; ++a) load_lds16(s.aptr[a] + (kb0 + akk[a]) * 128, &S.a[aslot[a]][0]);
#pragma unroll
    for (int kk = 0; kk < KPS; ++kk) load_lds4(s.asp + (kb0 + kk) * 4, (uint8_t*)&S.as[kk][sslot][0]);
  };
  // The item's weight scale table (this wave's 64 rows): LDS chunk c = 64 i + lane
  // of the wave's region is stored chunk c % 8 of row c / 8 and holds the row's
  // scale bytes [16 pc, +16), pc = (c % 8) ^ (row % 8), so the 16 rows of a
  // fragment read spread over the LDS banks (KS <= 128 and KS % 16 == 0, checked
  // at launch; pieces past KS re-read piece 0 and are never read back).
  auto load_table = [&](const ItemDesc& d, const MxSrc<NA>& s) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int c = 64 * i + lane, row = c >> 3, pc = (c & 7) ^ (row & 7);
      const int off = (16 * pc < KS) ? 16 * pc : 0;
      if constexpr (MT <= 32)
        load_lds16_nt(s.wsb + (size_t)wrow_of(d, row >> 4, row & 15) * KS + off, sTbl + wave * 8192 + i * 1024);
      else
        load_lds16(s.wsb + (size_t)wrow_of(d, row >> 4, row & 15) * KS + off, sTbl + wave * 8192 + i * 1024);
    }
  };
  // bias of the lane's four weight rows (column tile j, row r16), loaded with
  // gload_i32: the epilogue's use must not make the compiler wait for the ring's
  // loads. The caller makes the loads complete (a wait) before bias_ready.
  auto bias_issue = [&](const ItemDesc& d, int (&b)[4]) {
    const float* bb = bias_ptr(d);
#pragma unroll
    for (int j = 0; j < 4; ++j) b[j] = bb != nullptr ? gload_i32(bb + wrow_of(d, j, r16)) : 0;
  };
  auto bias_ready = [&](int (&b)[4], float (&f)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      vm_ready(b[j]);
      f[j] = __int_as_float(b[j]);
    }
  };

  // ---- first item: plain loads, its tables, the ring's first stages
  ItemDesc cd = desc(wi);
  MxSrc<NA> cs;
  float cbias[4];
  {
    long ta[NA];
#pragma unroll
    for (int a = 0; a < NA; ++a) ta[a] = a_live(a) ? row_src(cd, a_row(a), tp_read(cd, a_row(a))) : -1;
    const long tsc = s_live ? row_src(cd, s_row, tp_read(cd, s_row)) : -1;
    if (tid < MT) sSrc[0][tid] = row_src(cd, tid, tp_read(cd, tid));
    cs = sources(cd, ta, tsc);
  }
  int cbi[4];
  bias_issue(cd, cbi);
  __syncthreads();  // the first item's token table (and its bias loads: vmcnt 0)
  bias_ready(cbi, cbias);
  if constexpr (TBL) load_table(cd, cs);
#pragma unroll
  for (int i = 0; i < PD - 1; ++i) issue(cs, st[i], min(i, NSTG - 1));

  const int fr = (r16 >> 3) * 1024 + (r16 & 7) * 128;
  auto cat = [](const v4i& lo, const v4i& hi) -> v8i {
    return (v8i){lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
  };

  int sc = 0;   // ring stage of the stage being multiplied
  int par = 0;  // parity of the current item's token table
  for (;;) {
    const int wn = wi + G;
    const bool has_next = wn < total;
    const bool xfer = stream && has_next;  // the ring runs into the next item
    ItemDesc nd = cd;
    MxSrc<NA> ns = cs;
    float nbias[4] = {0.f, 0.f, 0.f, 0.f};
    int mta[NA], mts = 0, mte = 0, mbi[4] = {0, 0, 0, 0};
    if (xfer) nd = desc(wn);
    const float* nbp = xfer ? bias_ptr(nd) : nullptr;

    v4f acc[MS][4];
#pragma unroll
    for (int ms = 0; ms < MS; ++ms)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[ms][j] = (v4f){0.f, 0.f, 0.f, 0.f};

    for (int t = 0; t < NSTG; ++t) {
      __builtin_amdgcn_sched_barrier(0);
      wait_vm<(PD - 2) * NV>();      // this wave's share of stage t has landed
      __builtin_amdgcn_s_barrier();  // ... every wave's, and stage t - 1 is consumed
      __builtin_amdgcn_sched_barrier(0);
      if (xfer && t == 0) {
        // the next item's token ids and biases, ahead of this step's loads
#pragma unroll
        for (int a = 0; a < NA; ++a) mta[a] = KIND == 0 ? gload_i32(tp_ptr(nd, a_row(a))) : 0;
        if (KIND == 0) {
          mts = gload_i32(tp_ptr(nd, s_row));
          mte = gload_i32(tp_ptr(nd, tid));
        }
        if (nbp != nullptr) {
#pragma unroll
          for (int j = 0; j < 4; ++j) mbi[j] = gload_i32(nbp + wrow_of(nd, j, r16));
        }
      }
      const int kn = t + PD - 1;  // stage the ring loads now
      Stage& nxt = st[sc == 0 ? PD - 1 : sc - 1];
      // with the table and three stages, the ring's second stage of the next item
      // waits until after this item's last multiply (see above)
      const bool defer = TBL && PD == 3 && xfer && kn == NSTG + 1;
      if (kn < NSTG) {
        issue(cs, nxt, kn);
      } else if (xfer) {
        if (kn == NSTG) {
          // the next item's sources and token table (its token loads have landed:
          // at least one step's wait has passed since they were issued)
          long nta[NA];
#pragma unroll
          for (int a = 0; a < NA; ++a) {
            vm_ready(mta[a]);
            nta[a] = a_live(a) ? row_src(nd, a_row(a), mta[a]) : -1;
          }
          vm_ready(mts);
          vm_ready(mte);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            vm_ready(mbi[j]);
            nbias[j] = nbp != nullptr ? __int_as_float(mbi[j]) : 0.f;
          }
          ns = sources(nd, nta, s_live ? row_src(nd, s_row, mts) : -1);
          if (tid < MT) sSrc[par ^ 1][tid] = row_src(nd, tid, mte);
        }
        if (!defer) issue(ns, nxt, min(kn - NSTG, NSTG - 1));
      } else {
        issue(cs, nxt, NSTG - 1);  // keeps the counts exact; lands in a stage not read again
      }
      __builtin_amdgcn_sched_barrier(0);
      Stage& cur = st[sc];
      const uint32_t bw = lds_addr(&cur.b[wave][0]);
#pragma unroll
      for (int kk = 0; kk < KPS; ++kk) {
        const uint32_t aw = lds_addr(&cur.a[kk * AQ][0]);
        // scale dword of row r16 of column tile 0, K block kb = KPS t + kk (table:
        // piece kb / 4 of the row stored at chunk (kb / 4) ^ (r16 % 8))
        const int kbs = t * KPS + kk;
        const uint32_t bsw = TBL ? lds_addr(sTbl) + wave * 8192 + r16 * 128 +
                                       ((((kbs >> 2) ^ (r16 & 7))) << 4) + ((kbs & 3) << 2)
                                 : lds_addr(&cur.bs[TBL ? 0 : wave][kk][r16]);
        constexpr int SST = TBL ? 2048 : 64;
        v8i b[4];
        int bsc[4];
#pragma unroll
        for (int ms = 0; ms < MS; ++ms) {
          v4i alo, ahi;
          int sa;
          const uint32_t a_lo = aw + 2048 * ms + fr + swz(r16, g) * 16;
          const uint32_t a_hi = aw + 2048 * ms + fr + swz(r16, 4 + g) * 16;
          const uint32_t asw = lds_addr(&cur.as[kk][(ms * 16) >> 6][(ms * 16 + r16) & 63]);
          if (ms == 0) {
            if (WFMT == kFmtFp4) {
              v4i w[4];
              mx_read_w4<SST>(bw + fr + swz(r16, kk * 4 + g) * 16, bsw, a_lo, a_hi, asw, w, bsc,
                              alo, ahi, sa);
#pragma unroll
              for (int j = 0; j < 4; ++j) b[j] = (v8i){w[j].x, w[j].y, w[j].z, w[j].w, 0, 0, 0, 0};
            } else {
              v4i w[8];
              mx_read_w8<SST>(bw + fr + swz(r16, g) * 16, bw + fr + swz(r16, 4 + g) * 16, bsw, a_lo,
                              a_hi, asw, w, bsc, alo, ahi, sa);
#pragma unroll
              for (int j = 0; j < 4; ++j) b[j] = cat(w[2 * j], w[2 * j + 1]);
            }
          } else {
            mx_read_a(a_lo, a_hi, asw, alo, ahi, sa);
          }
          const v8i a = cat(alo, ahi);
          const int sab = (int)((uint32_t)sa >> (8 * g));
#pragma unroll
          for (int j = 0; j < 4; ++j)
            acc[ms][j] = mfma_mx(a, b[j], acc[ms][j], sab, (int)((uint32_t)bsc[j] >> (8 * g)), wfmt);
          // keeps each row group's MFMAs next to its reads (the scheduler would
          // otherwise hold every group's fragments live at once)
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      sc = (sc == PD - 1) ? 0 : sc + 1;
    }
    if (xfer && TBL) {
      // this wave has read its table rows for the last time in this item
      load_table(nd, ns);
      // the deferred second stage of the next item: global step s_last + 2, whose
      // ring stage is (sc + 1) % 3 now that sc has moved past the last step
      if (PD == 3) issue(ns, st[sc == PD - 1 ? 0 : sc + 1], min(1, NSTG - 1));
    }

    // Epilogue. Accumulator layout: lane l, register i holds D[4 * (l / 16) + i][l % 16]
    // (row of the tile, weight row of the fragment).
    const long row0 = cd.row0;
    const int nt = cd.nt;
    int wrow[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) wrow[j] = wrow_of(cd, j, r16);
    if (KIND == 0) {
      const int GI = p.I / 32;
#pragma unroll
      for (int ms = 0; ms < MS; ++ms) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float m = 0.f;
#pragma unroll
          for (int jj = 0; jj < 2; ++jj) {
            const float gt = fminf(fmaxf(acc[ms][jj][i] + cbias[jj], p.gate_lo), p.gate_hi);
            const float up = fminf(fmaxf(acc[ms][jj + 2][i] + cbias[jj + 2], p.up_lo), p.up_hi);
            const float h = mx_act(gt, p.act) * up;
            acc[ms][jj][i] = h;
            m = fmaxf(m, fabsf(h));
          }
          // the wave's 32 h columns of this row are one MX block
          m = group16_max_f32(m);
          const int row = ms * 16 + 4 * g + i;
          const int ex = mx_exponent(m);
          if (sSrc[par][row] >= 0) {
            const float f = mx_inv_scale(ex);
            const uint32_t c2 = mx_e4m3x2(acc[ms][0][i], acc[ms][1][i], f);
            uint8_t* const hrow = p.hq + (size_t)(row0 + row) * p.I + nt * 32 * NW + wave * 32 + r16;
            hrow[0] = (uint8_t)c2;
            hrow[16] = (uint8_t)(c2 >> 8);
            if (r16 == 0) p.hs[(size_t)(row0 + row) * GI + nt * NW + wave] = (uint8_t)(ex + 127);
          }
        }
      }
    } else {
#pragma unroll
      for (int ms = 0; ms < MS; ++ms) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = ms * 16 + 4 * g + i;
          if (row < cd.nrows) {
            const long yrow = row0 + row;
#pragma unroll
            for (int j = 0; j < 4; ++j)
              p.y[(size_t)yrow * p.H + wrow[j]] = (uint16_t)bf16x2(acc[ms][j][i] + cbias[j], 0.f);
          }
        }
      }
    }

    if (!has_next) break;
    wi = wn;
    par ^= 1;
    if (xfer) {
      cd = nd;
      cs = ns;
#pragma unroll
      for (int j = 0; j < 4; ++j) cbias[j] = nbias[j];
    } else {
      // drain mode: the ring's tail loads land, then the next item starts afresh
      wait_vm<0>();
      __syncthreads();
      cd = desc(wi);
      long ta[NA];
#pragma unroll
      for (int a = 0; a < NA; ++a) ta[a] = a_live(a) ? row_src(cd, a_row(a), tp_read(cd, a_row(a))) : -1;
      const long tsc = s_live ? row_src(cd, s_row, tp_read(cd, s_row)) : -1;
      if (tid < MT) sSrc[par][tid] = row_src(cd, tid, tp_read(cd, tid));
      cs = sources(cd, ta, tsc);
      bias_issue(cd, cbi);
      __syncthreads();  // (and the bias loads: vmcnt 0)
      bias_ready(cbi, cbias);
      if constexpr (TBL) load_table(cd, cs);
      sc = 0;
#pragma unroll
      for (int i = 0; i < PD - 1; ++i) issue(cs, st[i], min(i, NSTG - 1));
    }
  }
  wait_vm<0>();  // no load is still landing in LDS when the workgroup ends
}

// MXFP8 quantization of bf16 rows (mx_act_quant_body).
__global__ __launch_bounds__(256) void mx_act_quant_kernel(const uint16_t* __restrict__ x, long chunks,
                                                           uint8_t* __restrict__ q,
                                                           uint8_t* __restrict__ s) {
  mx_act_quant_body(x, chunks, q, s, blockIdx.x, gridDim.x);
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

// ---------------------------------------------------------------------------
// One-token MX GEMM for the layer (T = 1, MXFP4 weights, K = 128 KB): a work item is
// one tile (one row) and 32 NW weight rows, one wave per 32 rows (gate_up: 16 gate rows
// and the matching 16 up rows, so a pair of waves holds one 32-column MX block of h;
// down: 32 output columns). Each wave owns two 16-row column tiles and loads all of
// their MFMA fragments for the whole K into registers at once: 2 x KB fragment loads
// (16 bytes per lane each) and KB / 2 scale loads per wave, all in flight (the counter
// holds 63), one memory round trip where the ring kernel chains its stages. The token's row and its E8M0 bytes go
// to LDS once. Every load is a plain load, so the compiler orders the waits and the
// MFMAs start as the first fragments land. Same scaled MFMAs in the same K order and
// the same epilogue arithmetic as expert_gemm_mx_kernel (the MX block maximum of h
// combines the pair of waves that hold its 32 columns), so the outputs are the same
// bits.
// ---------------------------------------------------------------------------
template <int KIND, int KB, int NW>
__global__ __launch_bounds__(64 * NW) void expert_gemm_mx_one_kernel(MxArgs p) {
  static_assert(KB % 4 == 0 && 2 * KB + KB / 2 <= 60, "fragment and scale loads in flight per wave");
  static_assert(KIND == 1 || NW % 2 == 0, "gate_up: whole MX blocks of h per workgroup");
  constexpr int K = 128 * KB;
  constexpr int NA = (K / 16 + 64 * NW - 1) / (64 * NW);  // 16-byte pieces of the row per thread
  __shared__ __attribute__((aligned(16))) uint8_t sA[K];       // the row's MXFP8 codes
  __shared__ __attribute__((aligned(16))) uint8_t sAS[K / 32];  // its E8M0 bytes
  __shared__ float sMax[NW];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, r16 = lane & 15;
  const int NT = (KIND == 0) ? p.I / (16 * NW) : p.H / (32 * NW);
  const int tile = blockIdx.x / NT, nt = blockIdx.x - tile * NT;
  if (tile >= p.num_tiles[0]) return;  // whole workgroup
  const int4 td = p.tiles[tile];
  const int e = td.x;
  if (e < 0 || e >= p.E + p.nsh) return;  // whole workgroup: malformed tile
  const bool is_sh = e >= p.E;
  const int ej = is_sh ? e - p.E : e;
  const long row0 = td.w;  // the tile's hq / y row
  const int rows_w = (KIND == 0) ? 2 * p.I : p.H;
  // weight rows of the wave's column tiles: gate_up, gate row c and up row I + c of
  // h column c = 16 (NW nt + wave) + r16; down, output columns 32 (NW nt + wave) + 16 t + r16
  const int col0 = (KIND == 0) ? 16 * (NW * nt + wave) : 32 * (NW * nt + wave);
  int wr[2];
  if (KIND == 0) {
    wr[0] = col0 + r16;
    wr[1] = p.I + wr[0];
  } else {
    wr[0] = col0 + r16;
    wr[1] = wr[0] + 16;
  }
  const uint8_t* wb = (is_sh ? p.wsh : p.w) + (size_t)ej * rows_w * (K / 2);
  const uint8_t* wsb = (is_sh ? p.wssh : p.ws) + (size_t)ej * rows_w * (K / 32);
  const float* bb = is_sh ? p.bsh : p.bias;
  // the token's row (gate_up: token 0 of x; down: the tile's h row) and its scales
  const long a_row = (KIND == 0) ? 0 : row0;
  const uint8_t* ap = p.a + (size_t)a_row * K;
  const uint8_t* asp = p.as + (size_t)a_row * (K / 32);
  int4 av[NA], asv = make_int4(0, 0, 0, 0);
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    const int c = tid + i * 64 * NW;
    av[i] = (c < K / 16) ? *(const int4*)(ap + c * 16) : make_int4(0, 0, 0, 0);
  }
  if (tid < K / 512) asv = *(const int4*)(asp + tid * 16);
  // weight scales first (K blocks 4q .. 4q + 3 of the row in piece q), then the
  // fragments in K order: the first MFMAs wait only for the first loads
  int4 ws4[2][KB / 4];
#pragma unroll
  for (int q = 0; q < KB / 4; ++q)
#pragma unroll
    for (int t = 0; t < 2; ++t) ws4[t][q] = *(const int4*)(wsb + (size_t)wr[t] * (K / 32) + q * 16);
  int4 wf[KB][2];  // fp4 fragment: row wr[t], K values [128 kb + 32 g, +32)
#pragma unroll
  for (int kb = 0; kb < KB; ++kb)
#pragma unroll
    for (int t = 0; t < 2; ++t) wf[kb][t] = *(const int4*)(wb + (size_t)wr[t] * (K / 2) + kb * 64 + g * 16);
  float bia[2] = {0.f, 0.f};
  if (bb != nullptr) {
#pragma unroll
    for (int t = 0; t < 2; ++t) bia[t] = bb[(size_t)ej * rows_w + wr[t]];
  }
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    const int c = tid + i * 64 * NW;
    if (c < K / 16) *(int4*)(sA + c * 16) = av[i];
  }
  if (tid < K / 512) *(int4*)(sAS + tid * 16) = asv;
  __syncthreads();

  // A operand: row 0 of the MFMA is the token (lanes r16 == 0), the other rows zero
  v4f acc[2] = {(v4f){0.f, 0.f, 0.f, 0.f}, (v4f){0.f, 0.f, 0.f, 0.f}};
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    const int4 lo = *(const int4*)(sA + kb * 128 + 16 * g);
    const int4 hi = *(const int4*)(sA + kb * 128 + 64 + 16 * g);
    const uint32_t sad = *(const uint32_t*)(sAS + kb * 4);
    const bool tok = r16 == 0;
    const v8i a = tok ? (v8i){lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w} : (v8i){0, 0, 0, 0, 0, 0, 0, 0};
    const int sa = tok ? (int)(sad >> (8 * g)) : 127;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int4 w4 = ws4[t][kb >> 2];
      const int q = kb & 3;  // compile-time after unrolling
      const uint32_t sw = (uint32_t)(q == 0 ? w4.x : q == 1 ? w4.y : q == 2 ? w4.z : w4.w);
      const v8i b = (v8i){wf[kb][t].x, wf[kb][t].y, wf[kb][t].z, wf[kb][t].w, 0, 0, 0, 0};
      acc[t] = mfma_mx(a, b, acc[t], sa, (int)(sw >> (8 * g)), std::integral_constant<int, kFmtFp4>{});
    }
  }

  // The MFMA reads the operands of all 64 lanes whatever EXEC holds, and the compiler
  // does not treat it as convergent: with the results used only by lanes 0..15 it
  // would move the whole K loop into the branch below, where the operand set-up (the
  // zeroed rows, the scale bytes) runs on those lanes alone and the other lanes feed
  // the MFMAs stale registers. The empty asm takes the accumulators on every lane
  // here, ahead of any branch.
#pragma unroll
  for (int t = 0; t < 2; ++t) asm volatile("" : "+v"(acc[t]));

  // Epilogue: the token's outputs are register 0 of lanes 0..15 (row 0 of the tile,
  // weight row r16 of each column tile).
  if (KIND == 0) {
    float h = 0.f;
    if (g == 0) {
      const float gt = fminf(fmaxf(acc[0][0] + bia[0], p.gate_lo), p.gate_hi);
      const float up = fminf(fmaxf(acc[1][0] + bia[1], p.up_lo), p.up_hi);
      h = mx_act(gt, p.act) * up;
    }
    // the MX block of h columns [32 b, +32) is waves 2 b and 2 b + 1 (mod NW)
    const float m = group16_max_f32(fabsf(h));
    if (lane == 0) sMax[wave] = m;
    __syncthreads();
    const int ex = mx_exponent(fmaxf(sMax[wave], sMax[wave ^ 1]));
    if (g == 0) {
      const uint32_t c2 = mx_e4m3x2(h, 0.f, mx_inv_scale(ex));
      p.hq[(size_t)row0 * p.I + col0 + r16] = (uint8_t)c2;
      if (r16 == 0 && (wave & 1) == 0) p.hs[(size_t)row0 * (p.I / 32) + col0 / 32] = (uint8_t)(ex + 127);
    }
  } else if (g == 0) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
      p.y[(size_t)row0 * p.H + wr[t]] = (uint16_t)bf16x2(acc[t][0] + bia[t], 0.f);
  }
}

// ---------------------------------------------------------------------------
// Down and combine in one launch for the layer at one token (MXFP4 w2, I = 128 KB,
// no shared experts): out = bf16(sum over the token's live pairs k, in pair order, of
// w_k * bf16(h_k W2[e_k]^T + b2[e_k])), the sum moe_combine takes over the y rows the
// down GEMM writes. A workgroup owns 16 output columns and runs one wave per pair
// (K <= 8): wave k loads pair k's h row (the row inv[k] of hq) and its E8M0 bytes into
// LDS, and its expert's 16 weight rows for the whole K into registers (24 fragment
// and 6 scale loads), as expert_gemm_mx_one_kernel does; the MFMAs and the y rounding
// are the down kernel's, the pair sum (fused multiply-adds from zero, live pairs in
// order) the combine kernel's, so the output is the same bits without the y rows or
// the combine launch. Pairs with no row (inv < 0) add nothing, as in the combine.
// ---------------------------------------------------------------------------
constexpr int kDownCombineMaxK = 8;

template <int KB>
__global__ __launch_bounds__(64 * kDownCombineMaxK) void down_combine_mx_one_kernel(
    const uint8_t* __restrict__ hq, const uint8_t* __restrict__ hs, const uint8_t* __restrict__ w2,
    const uint8_t* __restrict__ w2s, const float* __restrict__ b2, const int32_t* __restrict__ ids,
    const int32_t* __restrict__ inv, const float* __restrict__ wts, int H, int E, int K,
    uint16_t* __restrict__ out) {
  static_assert(KB % 4 == 0, "scale pieces of four K blocks");
  constexpr int K_ = 128 * KB;
  __shared__ __attribute__((aligned(16))) uint8_t sA[kDownCombineMaxK][K_];
  __shared__ __attribute__((aligned(16))) uint8_t sAS[kDownCombineMaxK][K_ / 32];
  __shared__ float sY[kDownCombineMaxK][16];
  __shared__ float sW[kDownCombineMaxK];  // the pair's weight, 0 for a pair with no row
  const int tid = threadIdx.x, lane = tid & 63, k = tid >> 6;  // wave k: pair k
  const int g = lane >> 4, r16 = lane & 15;
  const int col = blockIdx.x * 16 + r16;  // output column of lane r16
  // the pair's compact row and expert, the same on every lane of the wave
  const int row = __builtin_amdgcn_readfirstlane(inv[k]);
  const int e = __builtin_amdgcn_readfirstlane(ids[k]);
  const bool live = row >= 0 && e >= 0 && e < E;
  int4 av[(K_ / 16 + 63) / 64], asv = make_int4(0, 0, 0, 0);
  int4 ws4[KB / 4];
  int4 wf[KB];
  float bia = 0.f;
  if (live) {
    const uint8_t* ap = hq + (size_t)row * K_;
#pragma unroll
    for (int i = 0; i < (K_ / 16 + 63) / 64; ++i) {
      const int c = lane + 64 * i;
      av[i] = (c < K_ / 16) ? *(const int4*)(ap + c * 16) : make_int4(0, 0, 0, 0);
    }
    if (lane < K_ / 512) asv = *(const int4*)(hs + (size_t)row * (K_ / 32) + lane * 16);
    const uint8_t* wsb = w2s + ((size_t)e * H + col) * (K_ / 32);
#pragma unroll
    for (int q = 0; q < KB / 4; ++q) ws4[q] = *(const int4*)(wsb + q * 16);
    const uint8_t* wb = w2 + ((size_t)e * H + col) * (K_ / 2) + g * 16;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) wf[kb] = *(const int4*)(wb + kb * 64);
    if (b2 != nullptr) bia = b2[(size_t)e * H + col];
#pragma unroll
    for (int i = 0; i < (K_ / 16 + 63) / 64; ++i) {
      const int c = lane + 64 * i;
      if (c < K_ / 16) *(int4*)(&sA[k][c * 16]) = av[i];
    }
    if (lane < K_ / 512) *(int4*)(&sAS[k][lane * 16]) = asv;
  }
  __syncthreads();
  v4f acc = (v4f){0.f, 0.f, 0.f, 0.f};
  float y = 0.f;  // bf16-rounded y of column col for pair k (0 without a row)
  if (live) {
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      const int4 lo = *(const int4*)(&sA[k][kb * 128 + 16 * g]);
      const int4 hi = *(const int4*)(&sA[k][kb * 128 + 64 + 16 * g]);
      const uint32_t sad = *(const uint32_t*)(&sAS[k][kb * 4]);
      const bool tok = r16 == 0;
      const v8i a = tok ? (v8i){lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w} : (v8i){0, 0, 0, 0, 0, 0, 0, 0};
      const int sa = tok ? (int)(sad >> (8 * g)) : 127;
      const int4 w4 = ws4[kb >> 2];
      const int q = kb & 3;
      const uint32_t sw = (uint32_t)(q == 0 ? w4.x : q == 1 ? w4.y : q == 2 ? w4.z : w4.w);
      const v8i b = (v8i){wf[kb].x, wf[kb].y, wf[kb].z, wf[kb].w, 0, 0, 0, 0};
      acc = mfma_mx(a, b, acc, sa, (int)(sw >> (8 * g)), std::integral_constant<int, kFmtFp4>{});
    }
    // the MFMAs read every lane: keep them out of the lanes-0..15 branch below
    asm volatile("" : "+v"(acc));
    y = bf16_bits_to_f32((uint16_t)bf16x2(acc[0] + bia, 0.f));
  }
  if (g == 0) sY[k][r16] = y;
  if (lane == 0) sW[k] = (row >= 0) ? wts[k] : 0.f;
  __syncthreads();
  if (k == 0 && g == 0) {
    float o = 0.f;
    for (int j = 0; j < K; ++j)
      if (inv[j] >= 0) o = __builtin_fmaf(sW[j], sY[j][r16], o);  // the combine's live pairs, in order
    out[col] = (uint16_t)bf16x2(o, 0.f);
  }
}

template <int KIND, int WFMT>
static int launch_mx(const MxArgs& a, int max_tiles, int mt, hipStream_t st) {
  // The layer at one token with MXFP4 weights and K = 3072: the register kernel, one
  // workgroup per work item. Gate_up items are two MX blocks of h (196 KB of weight
  // rows), down items 64 output columns (98 KB): the time follows the bytes of the
  // busiest CU, and smaller items (more than one per CU) measured no faster.
  const int Kone = (KIND == 0) ? a.H : a.I;
  constexpr int NW1 = (KIND == 0) ? 4 : 2;
  if (a.one && a.T == 1 && WFMT == kFmtFp4 && mt == 16 && Kone == 128 * 24 && a.I % (16 * NW1) == 0 &&
      a.H % (32 * NW1) == 0) {
    const long items = (long)max_tiles * ((KIND == 0) ? a.I / (16 * NW1) : a.H / (32 * NW1));
    hipLaunchKernelGGL((expert_gemm_mx_one_kernel<KIND, 24, NW1>), dim3((unsigned)items), dim3(64 * NW1),
                       0, st, a);
    return MOE_OK;
  }
  // otherwise the ring kernel: one persistent workgroup per CU (the ring's LDS allows
  // one), each running every G-th work item; 16-row tiles whose 2-wave half-width
  // items still fit one per CU (one token) run those instead, twice as many workgroups
  const int cus = device_cu_count();
  const int nt4 = (KIND == 0) ? a.I / 128 : a.H / 256;
  const bool half = mt == 16 && 2L * max_tiles * nt4 <= cus;
  const int NT = half ? 2 * nt4 : nt4;
  const long items = (long)max_tiles * NT;
  const int grid = (int)std::max(1L, std::min(items, (long)cus));
  // the per-item scale table for K <= 4096 in whole 16-byte pieces per row
  // (K % 512 == 0), and for the tiles whose LDS has room
  const int Kdim = (KIND == 0) ? a.H : a.I;
  const bool tbl = Kdim <= kMxTblMaxK && Kdim % 512 == 0;
#define MOE_MX(MTV, PDV, TBLV, NWV) \
  hipLaunchKernelGGL((expert_gemm_mx_kernel<MTV, KIND, PDV, WFMT, TBLV, NWV>), dim3(grid), dim3(64 * NWV), 0, st, a)
  switch (mt) {
    case 16:
      if (half) {
        // one item per workgroup: six stages in flight, since a half-width item at
        // one token is a short chain of K steps rather than a byte stream
        if (tbl)
          MOE_MX(16, 6, true, 2);
        else
          MOE_MX(16, 6, false, 2);
      } else if (tbl) {
        MOE_MX(16, 3, true, 4);
      } else {
        MOE_MX(16, 3, false, 4);
      }
      break;
    case 32:
      if (tbl)
        MOE_MX(32, 2, true, 4);
      else
        MOE_MX(32, 3, false, 4);
      break;
    case 64:
      if (tbl)
        MOE_MX(64, 2, true, 4);
      else
        MOE_MX(64, 2, false, 4);
      break;
    default:
      return MOE_ERR_ARG;
  }
#undef MOE_MX
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
  // a 128-row MXFP4 tile needs more than the 512 registers of a lane (it would spill)
  MOE_CHECK_SUPPORTED(mt != 128, "MX expert tiles stop at 64 rows (mt=128 is not built)");
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

static int moe_expert_gate_up_mx_impl(const uint8_t* xq, const uint8_t* xs, int T, int H, int I, int E,
                                      int wfmt, const uint8_t* w13, const uint8_t* w13_scale,
                                      const float* b13, const uint8_t* w13_shared,
                                      const uint8_t* w13_shared_scale, const float* b13_shared,
                                      int n_shared, const int32_t* token_position_to_id, int NB,
                                      const int32_t* tiles, const int32_t* num_tiles, int max_tiles,
                                      int mt, int act, float gate_lo, float gate_hi, float up_lo,
                                      float up_hi, uint8_t* hq, uint8_t* hs, void* stream, int one) {
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
  a.one = one;
  rc = (wfmt == MOE_MX_FP4) ? launch_mx<0, kFmtFp4>(a, max_tiles, mt, (hipStream_t)stream)
                            : launch_mx<0, kFmtFp8>(a, max_tiles, mt, (hipStream_t)stream);
  MOE_CHECK_ARG(rc == MOE_OK, "bad mt %d", mt);
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
  return moe_expert_gate_up_mx_impl(xq, xs, T, H, I, E, wfmt, w13, w13_scale, b13, w13_shared,
                                    w13_shared_scale, b13_shared, n_shared, token_position_to_id,
                                    NB, tiles, num_tiles, max_tiles, mt, act, gate_lo, gate_hi,
                                    up_lo, up_hi, hq, hs, stream, 0);
}

int moe::layer_gate_up_mx(const uint8_t* xq, const uint8_t* xs, int T, int H, int I, int E,
                          int wfmt, const uint8_t* w13, const uint8_t* w13_scale,
                          const float* b13, const uint8_t* w13_shared,
                          const uint8_t* w13_shared_scale, const float* b13_shared,
                          int n_shared, const int32_t* token_position_to_id, int NB,
                          const int32_t* tiles, const int32_t* num_tiles, int max_tiles,
                          int mt, int act, float gate_lo, float gate_hi, float up_lo,
                          float up_hi, uint8_t* hq, uint8_t* hs, void* stream) {
  return moe_expert_gate_up_mx_impl(xq, xs, T, H, I, E, wfmt, w13, w13_scale, b13, w13_shared,
                                    w13_shared_scale, b13_shared, n_shared, token_position_to_id,
                                    NB, tiles, num_tiles, max_tiles, mt, act, gate_lo, gate_hi,
                                    up_lo, up_hi, hq, hs, stream, T == 1);
}

static int moe_expert_down_mx_impl(const uint8_t* hq, const uint8_t* hs, int T, int H, int I, int E,
                                   int wfmt, const uint8_t* w2, const uint8_t* w2_scale,
                                   const float* b2, const uint8_t* w2_shared,
                                   const uint8_t* w2_shared_scale, const float* b2_shared,
                                   int n_shared, int NB, const int32_t* tiles,
                                   const int32_t* num_tiles, int max_tiles, int mt, void* y_bf16,
                                   void* stream, int one) {
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
  a.one = one;
  rc = (wfmt == MOE_MX_FP4) ? launch_mx<1, kFmtFp4>(a, max_tiles, mt, (hipStream_t)stream)
                            : launch_mx<1, kFmtFp8>(a, max_tiles, mt, (hipStream_t)stream);
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
  return moe_expert_down_mx_impl(hq, hs, T, H, I, E, wfmt, w2, w2_scale, b2, w2_shared,
                                 w2_shared_scale, b2_shared, n_shared, NB, tiles, num_tiles,
                                 max_tiles, mt, y_bf16, stream, 0);
}

int moe::layer_down_combine_mx(const uint8_t* hq, const uint8_t* hs, int T, int H, int I, int E,
                               int K, int wfmt, const uint8_t* w2, const uint8_t* w2_scale,
                               const float* b2, const int32_t* ids, const int32_t* inv,
                               const float* weights, void* out_bf16, void* stream, bool* done) {
  MOE_API_BEGIN("moe_expert_down_mx");
  *done = false;
  if (T != 1 || wfmt != MOE_MX_FP4 || I != 128 * 24 || K < 1 || K > kDownCombineMaxK || H % 16 != 0 ||
      ((uintptr_t)hq & 15) != 0 || ((uintptr_t)hs & 15) != 0 || ((uintptr_t)w2 & 15) != 0 ||
      ((uintptr_t)w2_scale & 15) != 0)
    return MOE_OK;  // not this form: the caller runs down and the combine
  MOE_CHECK_ARG(hq && hs && w2 && w2_scale && ids && inv && weights && out_bf16 && E > 0,
                "null pointer argument");
  hipLaunchKernelGGL(down_combine_mx_one_kernel<24>, dim3((unsigned)(H / 16)), dim3(64 * K), 0,
                     (hipStream_t)stream, hq, hs, w2, w2_scale, b2, ids, inv, weights, H, E, K,
                     (uint16_t*)out_bf16);
  *done = true;
  MOE_API_END();
}

int moe::layer_down_mx(const uint8_t* hq, const uint8_t* hs, int T, int H, int I, int E,
                       int wfmt, const uint8_t* w2, const uint8_t* w2_scale,
                       const float* b2, const uint8_t* w2_shared,
                       const uint8_t* w2_shared_scale, const float* b2_shared,
                       int n_shared, int NB, const int32_t* tiles,
                       const int32_t* num_tiles, int max_tiles, int mt, void* y_bf16,
                       void* stream) {
  return moe_expert_down_mx_impl(hq, hs, T, H, I, E, wfmt, w2, w2_scale, b2, w2_shared,
                                 w2_shared_scale, b2_shared, n_shared, NB, tiles, num_tiles,
                                 max_tiles, mt, y_bf16, stream, T == 1);
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
