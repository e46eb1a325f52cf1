// Prefill-sized FP8-blockwise expert GEMMs ("block" kernels, gfx950).
//
// Same math as gemm_fp8.hip (reference: moe_cte.py:557-588, DeepSeek-V3 128x128
// block-scaled fp8 weights), organised for experts that receive hundreds of
// rows, where the layer becomes MFMA-bound:
//
//  * one workgroup (8 waves) computes a 256-row x 256-column tile: the rows are
//    up to 256 consecutive slots of one expert, the columns 256 weight rows
//    (gate_up: 128 gate rows + the matching 128 up rows; down: 256 outputs).
//    Per 128-K step the tile moves 64 KB through L1 for 16.8 MFLOP;
//  * both operands are staged through LDS, loaded with global_load_lds_dwordx4
//    (no register staging): the weight (B) tiles in a ring of three 128-K stages
//    (two blocks in flight, for the HBM stream), the token (A) tile in one stage
//    refilled as soon as every wave holds its fragments (two barriers per K
//    step). 16-byte chunks are XOR-swizzled by row pairs so 16-lane fragment
//    reads hit distinct banks of the 64-bank LDS;
//  * wave (wm, wn) owns rows [64 wm, +64) and 128 columns as 4 x 8 tiles of
//    v_mfma_f32_16x16x128_f8f6f4: one MFMA per tile covers a whole 128-K scale
//    block. The block scales s_k = s_a[row, k] * s_w[k] are folded into the
//    running accumulator: acc = acc * (s_{k-1} / s_k) + A_k B_k, and the result
//    is acc * s_last, which equals sum_k s_k A_k B_k (one fp32 multiply per
//    accumulator element per K block, no separate partial products). The
//    ratios are computed once per (row, column half) per K block into LDS, one
//    block ahead, from activation scales loaded two blocks ahead;
//  * for gate_up wave column half wn holds gate and up columns [64 wn, +64) of
//    the tile's 128 h columns, so SiLU(g) * u is wave-local and only the row
//    amax of the 1x128 quantization group is combined across the two halves;
//  * work items (row tile, column tile) are enumerated expert by expert, column
//    tile by column tile, and mapped so that one XCD runs the items of one
//    expert together: the row tiles of an expert share each weight tile through
//    the XCD's L2, and the column tiles share the activation rows. An expert's
//    ceil(rows / 256) row tiles split its rows equally, so sibling tiles advance
//    through K at the same pace and read each weight block once from HBM (a
//    256-row tile next to a short remainder tile left it behind: 12.3 GB read
//    for 7.6 GB of weights at 8192 tokens, 9.6 GB with equal tiles);
//  * the next token tile is loaded once the current one has been read, and the
//    weight tile two blocks ahead is spread among the current block's MFMAs.
//
// Fragment lane layout (16x16x128): lane l supplies row l%16 and the bytes
// [(l/16)*16, +16) and [64 + (l/16)*16, +16) of the 128-wide K block, the same
// mapping for A and B. Accumulator: lane l, register i holds D[4*(l/16) + i][l%16].
#include "mapping.h"
#include "moe_common.h"
#include "moe_internal.h"

namespace moe {

constexpr int kBM = 256, kBN = 256, kBK = 128;
static_assert(kBM == kBlockTileRows, "block tile rows");
constexpr int kBlkThreads = 512;
constexpr int kStageA = kBM * kBK;  // 32 KB
constexpr int kStageB = kBN * kBK;  // 32 KB
constexpr int kDmaPerWave = (kStageA + kStageB) / 1024 / 8;  // 8 x 1 KB regions per wave
// Activation scales: two buffers x two copies (one per column half) x 256 rows x
// four K blocks (fp32); every fourth step one 16-byte load per row brings the
// next four blocks' scales.
constexpr int kStageSA = 2 * 2 * kBM * 16;
constexpr int kMaxKB = 128;  // K <= 16384

struct BlkArgs {
  const uint8_t* a;
  const float* as;
  const uint8_t* w;
  const float* ws;
  const uint8_t* wsh;
  const float* wssh;
  const int32_t* tpid;
  const int4* tiles;   // {expert, first slot, rows, first hq / y row}
  const int2* seg;     // {first tile of the expert, tiles of the expert}
  const int32_t* num_tiles;
  uint8_t* hq;
  float* hs;
  uint16_t* y;
  const float* cs;    // optional per-output-channel weight scales (routed, shared)
  const float* cssh;
  int T, H, I, E, nsh;
  long NB;
};

__device__ __forceinline__ v4f mfma16_fp8_acc(const v8i& a, const v8i& b, const v4f& c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}


// The workgroup's LDS, allocated once by the kernel. The pipeline stages are
// distinct objects, so the compiler can tell that fragment reads of one stage do
// not alias the direct-to-LDS loads in flight into another.
struct BlkLds {
  uint8_t* ta;                     // A tile of the current block (one stage)
  uint8_t *tb0, *tb1, *tb2;        // B tiles: three-stage ring
  uint8_t* sa;                     // A scales (loaded two blocks ahead), one copy per column half
  uint8_t* dummy;                  // 256 bytes per wave for loads that only keep the count
  float *r0, *r1;                  // scale ratios per (half, row) of even / odd blocks
  float* last;                     // last block scale per (half, row)
  int* src;                        // token (gate_up) or slot (down) of each tile row
  float (*red)[kBM];               // row amax of the two column halves
  float (*w)[kMaxKB];              // weight block scales of the two column halves
};

// LDS reads in asm. The compiler cannot tell a direct-to-LDS load into another
// stage from one into the stage read here once the K loop merges its paths, and
// would wait for every load in flight before a plain read. Reads that finish
// inside their statement wait for themselves; lds_frag_issue leaves its reads in
// flight until lds_frag_wait, which takes the same registers (LDS reads complete
// in order, so waiting for all of them is exact).
template <int OFF>
__device__ __forceinline__ void lds_frag_issue(uint32_t lo_addr, uint32_t hi_addr, v4i& lo, v4i& hi) {
  asm volatile(
      "ds_read_b128 %0, %2 offset:%4\n\t"
      "ds_read_b128 %1, %3 offset:%4"
      : "=&v"(lo), "=&v"(hi)
      : "v"(lo_addr), "v"(hi_addr), "n"(OFF)
      : "memory");
}
__device__ __forceinline__ void lds_frag_wait(v4i& lo, v4i& hi) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(lo), "+v"(hi) : : "memory");
}
template <int OFF>
__device__ __forceinline__ void lds_v4_issue(uint32_t addr, v4i& v) {
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=&v"(v) : "v"(addr), "n"(OFF) : "memory");
}
__device__ __forceinline__ void lds_v4_wait(v4i& v) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(v) : : "memory");
}
// MF A fragments at rows 0, 16, 32, 48 of the wave's row group: all reads, one wait.
template <int MF>
__device__ __forceinline__ void lds_frags_a(uint32_t lo_addr, uint32_t hi_addr, v4i (&lo)[MF],
                                            v4i (&hi)[MF]) {
  if constexpr (MF == 1) {
    asm volatile(
        "ds_read_b128 %0, %2\n\tds_read_b128 %1, %3\n\ts_waitcnt lgkmcnt(0)"
        : "=&v"(lo[0]), "=&v"(hi[0]) : "v"(lo_addr), "v"(hi_addr) : "memory");
  } else if constexpr (MF == 2) {
    asm volatile(
        "ds_read_b128 %0, %4\n\tds_read_b128 %1, %5\n\t"
        "ds_read_b128 %2, %4 offset:2048\n\tds_read_b128 %3, %5 offset:2048\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(lo[0]), "=&v"(hi[0]), "=&v"(lo[1]), "=&v"(hi[1]) : "v"(lo_addr), "v"(hi_addr)
        : "memory");
  } else if constexpr (MF == 3) {
    asm volatile(
        "ds_read_b128 %0, %6\n\tds_read_b128 %1, %7\n\t"
        "ds_read_b128 %2, %6 offset:2048\n\tds_read_b128 %3, %7 offset:2048\n\t"
        "ds_read_b128 %4, %6 offset:4096\n\tds_read_b128 %5, %7 offset:4096\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(lo[0]), "=&v"(hi[0]), "=&v"(lo[1]), "=&v"(hi[1]), "=&v"(lo[2]), "=&v"(hi[2])
        : "v"(lo_addr), "v"(hi_addr)
        : "memory");
  } else {
    static_assert(MF == 4, "1 to 4 fragments");
    asm volatile(
        "ds_read_b128 %0, %8\n\tds_read_b128 %1, %9\n\t"
        "ds_read_b128 %2, %8 offset:2048\n\tds_read_b128 %3, %9 offset:2048\n\t"
        "ds_read_b128 %4, %8 offset:4096\n\tds_read_b128 %5, %9 offset:4096\n\t"
        "ds_read_b128 %6, %8 offset:6144\n\tds_read_b128 %7, %9 offset:6144\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(lo[0]), "=&v"(hi[0]), "=&v"(lo[1]), "=&v"(hi[1]), "=&v"(lo[2]), "=&v"(hi[2]),
          "=&v"(lo[3]), "=&v"(hi[3])
        : "v"(lo_addr), "v"(hi_addr)
        : "memory");
  }
}
__device__ __forceinline__ void lds_st32(uint32_t addr, int v) {
  asm volatile("ds_write_b32 %0, %1" : : "v"(addr), "v"(v) : "memory");
}
__device__ __forceinline__ float lds_f32(uint32_t addr) {
  float v;
  asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(addr) : "memory");
  return v;
}
__device__ __forceinline__ v8i cat8(const v4i& lo, const v4i& hi) {
  return (v8i){lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
}

// One work item: tile rows [slot0, slot0 + nrows) of expert e against column
// tile nt; they use hq / y rows [rbase, rbase + nrows). MF is the number of 16-row fragments per wave: the four row groups
// hold 16 * MF rows each, so a tile of up to 64 * MF rows keeps all eight waves
// (two per SIMD) busy and its MFMA, ratio and fragment-read work scales with MF.
template <int KIND, int MF>
__device__ __forceinline__ void block_item(const BlkArgs& p, const BlkLds& s, const int e,
                                           const long slot0, const long rbase, const int nrows,
                                           const int nt) {
  uint8_t* const sTA = s.ta;
  uint8_t* const sTB0 = s.tb0;
  uint8_t* const sTB1 = s.tb1;
  uint8_t* const sTB2 = s.tb2;
  uint8_t* const sSA = s.sa;
  uint8_t* const sDummy = s.dummy;
  float* const sR0 = s.r0;
  float* const sR1 = s.r1;
  float* const sLast = s.last;
  int* const sSrc = s.src;
  float(*const sRed)[kBM] = s.red;
  float(*const sW)[kMaxKB] = s.w;
  constexpr int RG = 16 * MF;  // rows per row group

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  // Row group wm, column half wn. Waves run on SIMD wave % 4, so the two column
  // halves of a row group sit on different SIMDs.
  const int wm = wave >> 1, wn = wave & 1;
  const int Kdim = (KIND == 0) ? p.H : p.I;
  const int KB = Kdim / kBK;
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
  // Loader: regions of 1 KB, B: 32 (regions 4w..4w+3 of wave w), A: 8 MF (the
  // tile's 64 MF rows, regions MF w..MF w + MF - 1; a partial tile loads no rows
  // its row groups do not read). Lane l writes region byte l*16 = row l/8, stored
  // chunk l%8.
  uint32_t off[kDmaPerWave];
#pragma unroll
  for (int i = 4; i < kDmaPerWave; ++i) {
    const int row = 8 * (4 * wave + (i & 3)) + (lane >> 3);
    // Tile row -> weight row. Column tile n of a wave reads tile rows 16 n + j,
    // and they hold output columns 4 j + n (gate_up, per 64-column wave half) or
    // 8 j + n (down, per 128-column half): lane j then holds consecutive output
    // columns and stores them directly (4 fp8 codes or 8 bf16 values).
    int wrow;
    if (KIND == 0) {
      const int r = row & 127;
      const int hc = (r & 64) + 4 * (r & 15) + ((r >> 4) & 3);
      wrow = (row < 128) ? nt * 128 + hc : p.I + nt * 128 + hc;
    } else {
      wrow = nt * kBN + (row & 128) + 8 * (row & 15) + ((row >> 4) & 7);
    }
    off[i] = (uint32_t)(wrow * Kdim + swz(row, lane & 7) * 16);
  }

  // The loads that do not depend on each other are in flight together: block 0's
  // B tile (issued first), each tile row's token (gate_up) or slot (down) and the
  // weight block scales (2 KB <= 256 values); the A rows need the tokens. The LDS
  // stores and reads around them are asm so the compiler does not add waits for
  // the B tile's loads.
#pragma unroll
  for (int i = 4; i < kDmaPerWave; ++i) load_lds16(wb + off[i], sTB0 + (4 * wave + i - 4) * 1024);
  const int srow = 64 * wm + lane, shalf = wn;  // the scale writer's row and half (below)
  // Activation scale buffers. For gate_up with K blocks in multiples of four
  // (sgrp), buffer (g & 1) holds blocks [4g, 4g + 4) as [half][row][4] fp32, loaded
  // by one 16-byte load per row (gathered token rows: one 4-byte load per row and
  // block makes every instruction touch 64 lines); otherwise (down's rows are
  // consecutive) buffer (kb & 1) holds block kb as [half][row] fp32. Wave (wm, wn)
  // fills rows 64 wm + lane of copy wn.
  const bool sgrp = KIND == 0 && (KB & 3) == 0;
  auto sa_dst_of = [&](int buf) -> uint8_t* {
    return sSA + ((buf * 2 + wn) * kBM + 64 * wm) * (sgrp ? 16 : 4);
  };
  if constexpr (KIND == 1) {
    // down: tile row r is h row rbase + r, so block 0's A tile and scales need no
    // lookup and join the first round trip
#pragma unroll
    for (int i = 0; i < MF; ++i) {
      const int row = 8 * (MF * wave + i) + (lane >> 3);
      const uint32_t rs = (uint32_t)(row < nrows ? rbase + row : rbase);
      off[i] = rs * (uint32_t)Kdim + (uint32_t)(swz(row, lane & 7) * 16);
      load_lds16(p.a + off[i], sTA + (MF * wave + i) * 1024);
    }
    const uint32_t rs = (uint32_t)(srow < nrows ? rbase + srow : rbase);
    if (sgrp)
      load_lds16((const uint8_t*)p.as + rs * (uint32_t)(KB * 4), sa_dst_of(0));
    else
      load_lds4((const uint8_t*)p.as + rs * (uint32_t)(KB * 4), sa_dst_of(0));
  }
  __builtin_amdgcn_sched_barrier(0);
  const int whf = tid < KB ? 0 : 1, wkb = min(tid, 2 * KB - 1) - whf * KB;
  const int wr = (KIND == 0) ? (whf == 0 ? nt : p.I / 128 + nt) : nt * 2 + whf;
  const float wsv = wsb[(size_t)wr * KB + wkb];
  const int trow = min(tid, nrows - 1);  // nrows in [1, kBM]
  long sv = (KIND == 0) ? (is_sh ? slot0 + trow - p.NB - (long)ej * p.T : (long)p.tpid[slot0 + trow])
                        : rbase + trow;
  if (KIND == 0 && (sv < 0 || sv >= p.T)) sv = -1;
  const int src = tid < nrows ? (int)sv : -1;
  if (tid < kBM) lds_st32(lds_addr(sSrc) + 4 * tid, src);
  if (tid < 2 * KB) lds_st32(lds_addr(&sW[whf][wkb]), __float_as_int(wsv));
  lds_barrier();
  if constexpr (KIND == 0) {
#pragma unroll
    for (int i = 0; i < MF; ++i) {
      const int row = 8 * (MF * wave + i) + (lane >> 3);
      const int rs = __float_as_int(lds_f32(lds_addr(sSrc) + 4 * row));
      off[i] = (uint32_t)(rs >= 0 ? rs : 0) * (uint32_t)Kdim + (uint32_t)(swz(row, lane & 7) * 16);
    }
  }
  const uint8_t* abase = p.a;
  // Scale writers: every thread owns one (row, column half) and keeps the
  // previous block's scale; invalid rows use scale 1 (never stored). A zero
  // block scale (an all-zero weight block) repeats the previous scale: that
  // block's products are zero. The activation scales of a block reach LDS with
  // the B tile of the same block, two blocks ahead of its MFMAs (one 4-byte
  // direct-to-LDS load per wave: wave (wm, wn) fills rows 64 wm + lane of the copy
  // for column half wn); the weight scales are staged once per tile.
  // Thread (wave (wm, wn), lane j) owns row 64 wm + j and half wn: the rows its
  // own wave's scale load fills, so its own vmcnt wait covers them.
  const int ssrc = __float_as_int(lds_f32(lds_addr(sSrc) + 4 * srow));
  const bool svalid = ssrc >= 0;
  // Byte offsets of operand rows fit 32 bits: the entry points reject larger operands.
  const uint32_t off_sa = (uint32_t)(svalid ? ssrc : 0) * (uint32_t)(KB * 4);
  // the writer's own scale of block kb (its own wave loaded it)
  auto sa_own = [&](int kb) -> uint32_t {
    return sgrp ? lds_addr(sSA) + (uint32_t)((((((kb >> 2) & 1) * 2 + shalf) * kBM + srow) * 16) + (kb & 3) * 4)
                : lds_addr(sSA) + (uint32_t)((((kb & 1) * 2 + shalf) * kBM + srow) * 4);
  };
  float s_prev = 0.f;
  auto ratio = [&](float sa, float sw) {
    float s = svalid ? sa * sw : 1.f;
    if (s == 0.f) s = (s_prev != 0.f) ? s_prev : 1.f;
    const float r = s_prev / s;
    s_prev = s;
    return r;
  };

  // Loads of a block: the A group (the tile's rows, exactly kAGroup loads per wave;
  // rows past the tile's end re-read row 0, never stored) and the B group (the
  // block's activation scales, then the B tile: exactly kBGroup loads per wave).
  // Fixed counts keep every vmcnt wait exact.
  constexpr int kAGroup = MF;  // the tile's 64 MF rows: MF 1 KB loads per wave
  constexpr int kBLoads = kDmaPerWave - 4;
  constexpr int kBGroup = kBLoads + 1;
  auto issue_a = [&](int kb) {
#pragma unroll
    for (int i = 0; i < kAGroup; ++i)
      load_lds16(abase + off[i] + (size_t)kb * kBK, sTA + (MF * wave + i) * 1024);
  };
  // Load i of block kb's B group into stage sb (i = 0: the scales; grouped, only
  // at a group's first block, otherwise a 4-byte load of one line into the
  // wave's dummy area so every group has the same count).
  auto issue_b = [&](uint8_t* sb, int i, int kb) {
    if (i == 0) {
      if (!sgrp)
        load_lds4((const uint8_t*)p.as + off_sa + (size_t)kb * 4, sa_dst_of(kb & 1));
      else if ((kb & 3) == 0)
        load_lds16((const uint8_t*)p.as + off_sa + (size_t)kb * 4, sa_dst_of((kb >> 2) & 1));
      else
        load_lds4((const uint8_t*)p.as, sDummy + wave * 256);
    } else {
      load_lds16(wb + off[3 + i] + (size_t)kb * kBK, sb + (4 * wave + i - 1) * 1024);
    }
  };

  // Accumulators: MF row tiles (16 rows) x 8 column tiles (16 columns).
  v4f acc[MF][8];
#pragma unroll
  for (int m = 0; m < MF; ++m)
#pragma unroll
    for (int n = 0; n < 8; ++n) acc[m][n] = (v4f){0.f, 0.f, 0.f, 0.f};

  const bool active = RG * wm < nrows;  // this wave's row group holds at least one row
  const int g = lane >> 4, l16 = lane & 15;
  // Fragment reads. Every fragment starts at a 16-aligned row, so row l16 of it
  // has swizzle (l16 >> 1) & 7 whatever the tile: a fragment is one per-lane
  // offset (f_lo / f_hi) plus a constant, and the reads use immediate offsets.
  const uint32_t f_lo = l16 * kBK + ((g ^ ((l16 >> 1) & 7)) << 4);
  const uint32_t f_hi = l16 * kBK + (((g + 4) ^ ((l16 >> 1) & 7)) << 4);
  const uint32_t a_lo = lds_addr(sTA) + RG * wm * kBK + f_lo;
  const uint32_t a_hi = lds_addr(sTA) + RG * wm * kBK + f_hi;
  // B rows of this wave's eight 16-column tiles. gate_up: tiles 0-3 gate columns
  // [64 wn, +64), tiles 4-7 the matching up columns; down: columns [128 wn, +128).
  const uint32_t b_wave = (KIND == 0 ? 64 * wn : 128 * wn) * kBK;
  constexpr int kBRow[8] = {0, 16, 32, 48, (KIND == 0) ? 128 : 64, (KIND == 0) ? 144 : 80,
                            (KIND == 0) ? 160 : 96, (KIND == 0) ? 176 : 112};
  static_assert(16 * kBK == 2048, "A fragment stride");
  auto read_a = [&](v8i (&a)[MF]) {
    v4i lo[MF], hi[MF];
    lds_frags_a<MF>(a_lo, a_hi, lo, hi);
#pragma unroll
    for (int m = 0; m < MF; ++m) a[m] = cat8(lo[m], hi[m]);
  };
  // B fragment of column tile n: issued here, completed by lds_frag_wait.
  // Ratios of MF 16-row fragments (4 rows per lane, fragment m at +64 m bytes).
  auto issue_ratios = [&](uint32_t addr, v4i (&r)[MF]) {
#pragma unroll
    for (int m = 0; m < MF; ++m) {
      switch (m) {
        case 0: lds_v4_issue<0>(addr, r[m]); break;
        case 1: lds_v4_issue<64>(addr, r[m]); break;
        case 2: lds_v4_issue<128>(addr, r[m]); break;
        default: lds_v4_issue<192>(addr, r[m]); break;
      }
    }
  };
  auto wait_ratios = [&](v4i (&r)[MF], v4f (&f)[MF]) {
#pragma unroll
    for (int m = 0; m < MF; ++m) {
      lds_v4_wait(r[m]);
      f[m] = (v4f){__int_as_float(r[m].x), __int_as_float(r[m].y), __int_as_float(r[m].z),
                   __int_as_float(r[m].w)};
    }
  };
  auto issue_bfrag = [&](uint32_t lo_addr, uint32_t hi_addr, int n, v4i& lo, v4i& hi) {
    switch (n) {
      case 0: lds_frag_issue<kBRow[0] * kBK>(lo_addr, hi_addr, lo, hi); break;
      case 1: lds_frag_issue<kBRow[1] * kBK>(lo_addr, hi_addr, lo, hi); break;
      case 2: lds_frag_issue<kBRow[2] * kBK>(lo_addr, hi_addr, lo, hi); break;
      case 3: lds_frag_issue<kBRow[3] * kBK>(lo_addr, hi_addr, lo, hi); break;
      case 4: lds_frag_issue<kBRow[4] * kBK>(lo_addr, hi_addr, lo, hi); break;
      case 5: lds_frag_issue<kBRow[5] * kBK>(lo_addr, hi_addr, lo, hi); break;
      case 6: lds_frag_issue<kBRow[6] * kBK>(lo_addr, hi_addr, lo, hi); break;
      default: lds_frag_issue<kBRow[7] * kBK>(lo_addr, hi_addr, lo, hi); break;
    }
  };

  // Ratios of block kb + 1 (scales of block kb + 1 landed) into sr.
  // Grouped scales: the writer's row holds four blocks' scales in one 16-byte piece;
  // the piece is read whole at each group's first block (64 lanes, 1 KB contiguous:
  // conflict-free) and kept, instead of one 4-byte read per block (16-byte lane
  // stride: four lanes per bank).
  v4i s4 = {0, 0, 0, 0};
  auto store_ratio = [&](float* sr, int kb) {
    float sa;
    if (sgrp) {
      if ((kb & 3) == 0) {
        lds_v4_issue<0>(sa_own(kb), s4);
        lds_v4_wait(s4);
      }
      const int k3 = kb & 3;
      sa = __int_as_float(k3 == 0 ? s4.x : k3 == 1 ? s4.y : k3 == 2 ? s4.z : s4.w);
    } else {
      sa = lds_f32(sa_own(kb));
    }
    (shalf ? sr + kBM : sr)[srow] = ratio(sa, sW[shalf][kb]);
  };

  // One K step: the MFMAs of block kb (B tile in stage cb, ratios in cr). On entry
  // the A tile and the B tile of block kb have been issued and the B group of
  // block kb + 1 may still be in flight.
  //  1. wait for all but the last B group, barrier: A(kb) and B(kb) have landed,
  //     the ratios of block kb are visible, and every wave is done with the B
  //     stage about to be refilled;
  //  2. read this wave's A fragments, issue the MFMAs of column tile 0;
  //  3. barrier: the A stage is free; issue the A group of block kb + 1;
  //  4. after column tile 1 the scales of block kb + 1 (the oldest loads in flight
  //     but the A group) have landed: the scale writers store block kb + 1's
  //     ratios into nr, which the next step's first barrier publishes;
  //  5. the B group of block kb + 2 (into stage nb) is spread among the
  //     remaining MFMAs.
  // Past the last block the loads re-read block KB - 1 into stages that are not
  // read again, so every step issues the same loads and the waits stay exact.
  auto step = [&](int kb, const uint8_t* cb, const float* cr, uint8_t* nb, float* nr) {
    wait_vm<kBGroup>();
    lds_barrier();
    const int kb2 = min(kb + 2, KB - 1);
    if (active) {
      const uint32_t b_lo = lds_addr(cb) + b_wave + f_lo, b_hi = lds_addr(cb) + b_wave + f_hi;
      // ratios of the column half in use: gate, then up (gate_up)
      const uint32_t r_addr = lds_addr(cr) + 4 * (((KIND == 0) ? 0 : wn) * kBM + RG * wm + 4 * g);
      v4i rq[MF];
      v4f rr[MF];
      issue_ratios(r_addr, rq);
      v4i blo, bhi;
      issue_bfrag(b_lo, b_hi, 0, blo, bhi);
      v8i a[MF];
      read_a(a);  // waits for the ratio and B reads issued before it too
      wait_ratios(rq, rr);
      lds_frag_wait(blo, bhi);
      v8i b = cat8(blo, bhi);
      __builtin_amdgcn_sched_barrier(0);
      // B fragments double-buffered: the reads of column tile n + 1 (and, at the
      // gate / up boundary, the up-half ratios) are issued before the MFMAs of
      // tile n and waited for after them.
#pragma unroll
      for (int n = 0; n < 8; ++n) {
        v4i nlo, nhi;
        if (n + 1 < 8) issue_bfrag(b_lo, b_hi, n + 1, nlo, nhi);
        v4i uq[MF];
        if (KIND == 0 && n == 3) issue_ratios(r_addr + 4 * kBM, uq);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int m = 0; m < MF; ++m) {
          const v4f c = acc[m][n] * rr[m];
          acc[m][n] = mfma16_fp8_acc(a[m], b, c);
        }
        __builtin_amdgcn_sched_barrier(0);
        if (n == 0) {
          lds_barrier();
          issue_a(min(kb + 1, KB - 1));
        }
        if (n == 1) {
          wait_vm<kBGroup - 1 + kAGroup>();
          if (kb + 1 < KB) store_ratio(nr, kb + 1);
        }
        if (n >= 2 && n < 2 + kBGroup) issue_b(nb, n - 2, kb2);
        __builtin_amdgcn_sched_barrier(0);
        if (KIND == 0 && n == 3) wait_ratios(uq, rr);
        if (n + 1 < 8) {
          lds_frag_wait(nlo, nhi);
          b = cat8(nlo, nhi);
        }
      }
    } else {
      lds_barrier();
      issue_a(min(kb + 1, KB - 1));
      wait_vm<kBGroup - 1 + kAGroup>();
      if (kb + 1 < KB) store_ratio(nr, kb + 1);
#pragma unroll
      for (int i = 0; i < kBGroup; ++i) issue_b(nb, i, kb2);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  // Prologue (block 0's B tile, and for down its A tile and scales, are on their
  // way): A(0) and block 0's scales, block 0's ratios, which the first step's
  // barrier publishes, and the B group of block 1.
  if constexpr (KIND == 0) {
    issue_a(0);
    issue_b(sTB0, 0, 0);
  }
  wait_vm<0>();
  store_ratio(sR0, 0);  // s_prev = 0: the accumulators start at 0
  // the scale buffer is refilled only after its reader has read it
#pragma unroll
  for (int i = 0; i < kBGroup; ++i) issue_b(sTB1, i, min(1, KB - 1));
  for (int kb = 0; kb < KB; kb += 6) {
    step(kb, sTB0, sR0, sTB2, sR1);
    if (kb + 1 < KB) step(kb + 1, sTB1, sR1, sTB0, sR0);
    if (kb + 2 < KB) step(kb + 2, sTB2, sR0, sTB1, sR1);
    if (kb + 3 < KB) step(kb + 3, sTB0, sR1, sTB2, sR0);
    if (kb + 4 < KB) step(kb + 4, sTB1, sR0, sTB0, sR1);
    if (kb + 5 < KB) step(kb + 5, sTB2, sR1, sTB1, sR0);
  }
  wait_vm<0>();  // no load is still landing in LDS past this point
  (shalf ? sLast + kBM : sLast)[srow] = s_prev;
  __syncthreads();

  // Accumulator layout (16x16): lane l, register i holds D[4*(l/16) + i][l%16];
  // with the tile's weight-row order, acc[m][n][i] of lane l is output column
  // 4 (l % 16) + n (gate_up, n < 4) or 8 (l % 16) + n (down) of the wave's half.
  // Per-output-channel weight scales, when given, multiply each column first
  // (workgroup-uniform branch).
  if (const float* csb = is_sh ? p.cssh : p.cs) {
    csb += (size_t)ej * ((KIND == 0) ? 2 * p.I : p.H);
    float c[8];
#pragma unroll
    for (int n = 0; n < 8; ++n)
      c[n] = csb[(KIND == 0) ? ((n < 4 ? 0 : p.I) + nt * 128 + 64 * wn + 4 * l16 + (n & 3))
                             : (nt * kBN + 128 * wn + 8 * l16 + n)];
#pragma unroll
    for (int m = 0; m < MF; ++m)
#pragma unroll
      for (int n = 0; n < 8; ++n) acc[m][n] *= c[n];
  }
  if (KIND == 0) {
    // h = SiLU(gate) * up for this wave's 64 h columns; the row amax of the 1x128
    // group combines the two column-half waves through LDS.
    const int GI = p.I / 128;
#pragma unroll
    for (int m = 0; m < MF; ++m)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = RG * wm + 16 * m + 4 * g + i;
        const float sg_ = sLast[row], su = sLast[kBM + row];
        float mx = 0.f;
#pragma unroll
        for (int n = 0; n < 4; ++n) {
          const float gt = acc[m][n][i] * sg_, up = acc[m][n + 4][i] * su;
          // hardware reciprocal (about 1 ulp): h only feeds the 1x128 fp8 quantization
          const float h = gt * __builtin_amdgcn_rcpf(1.0f + __expf(-gt)) * up;
          acc[m][n][i] = h;
          mx = fmaxf(mx, fabsf(h));
        }
#pragma unroll
        for (int o = 8; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
        if (l16 == 0) sRed[wn][row] = mx;
      }
    __syncthreads();
    if (active) {
#pragma unroll
      for (int m = 0; m < MF; ++m)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = RG * wm + 16 * m + 4 * g + i;
          const float sc = fmaxf(fmaxf(sRed[0][row], sRed[1][row]), 0x1.b7cdfep-34f) / 448.0f;
          const float rs = 1.0f / sc;
          float y[4];
#pragma unroll
          for (int n = 0; n < 4; ++n) y[n] = fminf(fmaxf(div_by(acc[m][n][i], sc, rs), -448.0f), 448.0f);
          const uint32_t c4 = e4m3x2(y[0], y[1]) | (e4m3x2(y[2], y[3]) << 16);
          if (row < nrows && sSrc[row] >= 0) {
            *(uint32_t*)(p.hq + (size_t)(rbase + row) * p.I + nt * 128 + 64 * wn + 4 * l16) = c4;
            if (wn == 0 && l16 == 0) p.hs[(size_t)(rbase + row) * GI + nt] = sc;
          }
        }
    }
  } else if (active) {
#pragma unroll
    for (int m = 0; m < MF; ++m)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = RG * wm + 16 * m + 4 * g + i;
        const float sl = sLast[wn * kBM + row];
        int4 o;
        o.x = (int)bf16x2(acc[m][0][i] * sl, acc[m][1][i] * sl);
        o.y = (int)bf16x2(acc[m][2][i] * sl, acc[m][3][i] * sl);
        o.z = (int)bf16x2(acc[m][4][i] * sl, acc[m][5][i] * sl);
        o.w = (int)bf16x2(acc[m][6][i] * sl, acc[m][7][i] * sl);
        if (row < nrows) *(int4*)(p.y + (size_t)(rbase + row) * p.H + nt * kBN + 128 * wn + 8 * l16) = o;
      }
  }
}

template <int KIND>
__global__ __launch_bounds__(kBlkThreads) void expert_gemm_block_kernel(BlkArgs p) {
  __shared__ __attribute__((aligned(16))) uint8_t sTA[kStageA];
  __shared__ __attribute__((aligned(16))) uint8_t sTB0[kStageB];
  __shared__ __attribute__((aligned(16))) uint8_t sTB1[kStageB];
  __shared__ __attribute__((aligned(16))) uint8_t sTB2[kStageB];
  __shared__ __attribute__((aligned(16))) uint8_t sSA[kStageSA];
  __shared__ __attribute__((aligned(16))) uint8_t sDummy[8 * 256];
  __shared__ __attribute__((aligned(16))) float sR0[2 * kBM];
  __shared__ __attribute__((aligned(16))) float sR1[2 * kBM];
  __shared__ __attribute__((aligned(16))) float sLast[2 * kBM];
  __shared__ int sSrc[kBM];
  __shared__ float sRed[2][kBM];
  __shared__ float sW[2][kMaxKB];
  const BlkLds s{sTA, sTB0, sTB1, sTB2, sSA, sDummy, sR0, sR1, sLast, sSrc, sRed, sW};

  // XCD-aware item index: workgroup b runs on XCD b % 8, and XCD x takes the items
  // of tiles [cut[x], cut[x + 1]) of the list's header (whole experts, about equal
  // cost; see block_tile_cuts), in order. A range holds at most
  // block_tiles_cap(max_tiles) tiles, and the grid gives each XCD that many items'
  // workgroups.
  const int NT = (KIND == 0) ? p.I / 128 : p.H / kBN;
  const int x = blockIdx.x & 7;
  const int L = p.num_tiles[1 + x] * NT + (int)(blockIdx.x >> 3);
  if (L >= p.num_tiles[2 + x] * NT) return;
  const int2 sg = p.seg[L / NT];
  const int r0 = L - NT * sg.x;
  const int nt = r0 / sg.y;
  const int tile = sg.x + (r0 - nt * sg.y);
  if (tile >= p.num_tiles[0]) return;  // truncated tile list
  const int4 td = p.tiles[tile];
  const int e = td.x, nrows = td.z;
  if (e < 0 || e >= p.E + p.nsh || nrows <= 0) return;
  // Row groups sized to the tile (workgroup-uniform branch).
  if (nrows > 192)
    block_item<KIND, 4>(p, s, e, td.y, td.w, nrows, nt);
  else if (nrows > 128)
    block_item<KIND, 3>(p, s, e, td.y, td.w, nrows, nt);
  else if (nrows > 64)
    block_item<KIND, 2>(p, s, e, td.y, td.w, nrows, nt);
  else
    block_item<KIND, 1>(p, s, e, td.y, td.w, nrows, nt);
}

// ---------------------------------------------------------------------------
// Block tiles: per expert segment (consecutive blocks with one expert id), the
// slot range from its first block to its last valid slot, cut into chunks of
// 256 rows; seg[t] = {first tile of the segment, tiles in the segment}.
// Shared experts j: ceil(T/256) tiles over slots [NB + j*T, NB + (j+1)*T).
// num_tiles[0] = the tile count, num_tiles[1..9] = the XCD ranges.
// One workgroup; per-block last-valid lengths go through global scratch.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void build_block_tiles_kernel(
    const int32_t* __restrict__ tpid, const int32_t* __restrict__ b2e, int N, int B, int T, int E,
    int n_shared, int* __restrict__ vlen, int* __restrict__ cnt, int4* __restrict__ tiles,
    int2* __restrict__ seg, int max_tiles, int32_t* __restrict__ num_tiles) {
  __shared__ int s_part[1024];
  __shared__ int s_wave[16];
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
      const long h = (s1 - s0 + v - 1) / v;  // equal heights (sibling tiles share weight blocks in L2)
      for (int c = 0; c < v; ++c) {
        const int idx = off + c;
        if (idx < max_tiles) {
          tiles[idx] = make_int4(b2e[b], (int)(s0 + (long)c * h), (int)min(h, s1 - s0 - (long)c * h),
                                 (int)(s0 + (long)c * h));
          seg[idx] = make_int2(off, v);
        }
      }
    }
    base += s_part[1023];
    __syncthreads();
  }
  const int per = (T + kBM - 1) / kBM;
  const int hsh = (T + per - 1) / per;
  const long NB = (long)N * B;
  for (int i = tid; i < n_shared * per; i += blockDim.x) {
    const int jj = i / per, m = i - jj * per;
    const int idx = base + i;
    if (idx < max_tiles) {
      const int s0 = (int)(NB + (long)jj * T + (long)m * hsh);
      tiles[idx] = make_int4(E + jj, s0, min(hsh, T - m * hsh), s0);
      seg[idx] = make_int2(base + jj * per, per);
    }
  }
  if (tid == 0) num_tiles[0] = min(base + n_shared * per, max_tiles);
  __syncthreads();
  __threadfence_block();  // the tile stores above are this workgroup's
  block_tile_cuts(tiles, min(base + n_shared * per, max_tiles), max_tiles, num_tiles, s_wave);
}

template <int KIND>
static void launch_block(const BlkArgs& a, int max_tiles, hipStream_t st) {
  // each XCD's range holds at most block_tiles_cap(max_tiles) tiles
  const int NT = (KIND == 0) ? a.I / 128 : a.H / kBN;
  const long items = 8L * block_tiles_cap(max_tiles) * NT;
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

// a_rows x a_cols: the gathered operand (x for gate_up, h for down), addressed with
// 32-bit byte offsets inside the kernel.
static int block_gemm_common_checks(const char* _moe_fn, int T, int H, int I, int E, int NB,
                                    int max_tiles, long a_rows, int a_cols) {
  MOE_CHECK_ARG(T > 0 && E > 0 && NB >= 0 && max_tiles > 0, "bad sizes");
  MOE_CHECK_ARG(H > 0 && H % 256 == 0 && I > 0 && I % 128 == 0,
                "H must be a multiple of 256 and I of 128 (H=%d I=%d)", H, I);
  MOE_CHECK_SUPPORTED(H / 128 <= kMaxKB && I / 128 <= kMaxKB,
                      "H and I must be at most %d (H=%d I=%d)", 128 * kMaxKB, H, I);
  MOE_CHECK_SUPPORTED((unsigned long)a_rows * (unsigned long)a_cols < (1UL << 32),
                      "activation operand of %ld rows x %d bytes exceeds 4 GiB", a_rows, a_cols);
  return MOE_OK;
}

extern "C" int moe_expert_gate_up_block(const uint8_t* xq, const float* xs, int T, int H, int I,
                                        int E, const uint8_t* w13, const float* w13_scale,
                                        const float* w13_channel_scale, const uint8_t* w13_shared,
                                        const float* w13_shared_scale,
                                        const float* w13_shared_channel_scale, int n_shared,
                                        const int32_t* token_position_to_id, int NB,
                                        const int32_t* tiles, const int32_t* num_tiles,
                                        int max_tiles, uint8_t* hq, float* hs, void* stream) {
  MOE_API_BEGIN("moe_expert_gate_up_block");
  MOE_CHECK_ARG(xq && xs && w13 && w13_scale && token_position_to_id && tiles && num_tiles && hq && hs,
                "null pointer argument");
  int rc = block_gemm_common_checks(_moe_fn, T, H, I, E, NB, max_tiles, T, H);
  if (rc != MOE_OK) return rc;
  MOE_CHECK_ARG(n_shared == 0 || (w13_shared && w13_shared_scale), "shared weights missing");
  MOE_CHECK_ARG(((uintptr_t)xq & 15) == 0 && ((uintptr_t)w13 & 15) == 0 && ((uintptr_t)hq & 15) == 0,
                "xq, w13 and hq must be 16-byte aligned");
  BlkArgs a{};
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
                                     const float* w2_channel_scale, const uint8_t* w2_shared,
                                     const float* w2_shared_scale,
                                     const float* w2_shared_channel_scale, int n_shared, int NB,
                                     const int32_t* tiles,
                                     const int32_t* num_tiles, int max_tiles, void* y_bf16,
                                     void* stream) {
  MOE_API_BEGIN("moe_expert_down_block");
  MOE_CHECK_ARG(hq && hs && w2 && w2_scale && tiles && num_tiles && y_bf16, "null pointer argument");
  int rc = block_gemm_common_checks(_moe_fn, T, H, I, E, NB, max_tiles,
                                    (long)NB + (long)n_shared * T, I);
  if (rc != MOE_OK) return rc;
  MOE_CHECK_ARG(n_shared == 0 || (w2_shared && w2_shared_scale), "shared weights missing");
  MOE_CHECK_ARG(((uintptr_t)hq & 15) == 0 && ((uintptr_t)w2 & 15) == 0 && ((uintptr_t)y_bf16 & 15) == 0,
                "hq, w2 and y must be 16-byte aligned");
  BlkArgs a{};
  a.a = hq;
  a.as = hs;
  a.w = w2;
  a.ws = w2_scale;
  a.wsh = w2_shared;
  a.wssh = w2_shared_scale;
  a.cs = w2_channel_scale;
  a.cssh = w2_shared_channel_scale;
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
