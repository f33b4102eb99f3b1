// Tiled int8-weight GEMM for M above the decode range, both modes of the int8 Linear:
//   W8A16: y[m,n] = bf16(s[n] * sum_k x[m,k] q[n,k])               bf16 x, fp32 accumulation
//   W8A8:  acc[m,n] = sum_k xq[m,k] q[n,k] exactly in int32;  y = bf16((acc * sx[m]) * s[n])
//
// MFMA-bound. A block of WGM x WGN = 8 waves (two per SIMD, so one wave's LDS reads and
// dequantization overlap the other's MFMAs) computes a BM (tokens) x BN (weight rows) tile of y
// over K in 64-wide steps; wave (wm, wn) owns a WM x WN sub-tile (128 x 64 for the big tile) of
// 16x16 MFMA tiles whose A operand is a packed 1 KB weight tile (16 rows x 64 K-bytes, already
// in operand order) and whose B operand is 16 tokens of x. Per stage a wave dequantizes its
// weight tiles once, then walks its token tiles, reading each x fragment from LDS once.
//
// Data movement (per 64-wide K step, "stage"):
//  * x rows and the block's packed weight tiles travel HBM/L2 -> LDS by direct-to-LDS buffer
//    loads (16 bytes per lane, 1 KB per wave instruction) into a ring of NST stage slots, NST-1
//    stages ahead of the MFMAs. Waits are static vmcnt counts: every stage issues the same loads
//    (out-of-range ones read zeros and move no data). The loads are issued by dma16_lds, which
//    the compiler does not track, so the only waits on them are the ones written here.
//  * Weights stay int8 in LDS (half the footprint and fill traffic of bf16); in W8A16 each wave
//    dequantizes its WN/16 tiles after the LDS read (exact: |q| <= 127), 1.5 VALU ops per
//    weight, shared by the WM/16 token tiles it multiplies. With one wave row (WGM = 1) the
//    weights travel one stage ahead of x and each stage's dequantization runs under the
//    previous stage's MFMAs (WAHEAD).
//  * Decode tiles (one block row, M <= 64) and the 128 x 128 tile in a launch of one block row
//    load weights with the streaming (nt) cache policy: each weight byte is read by one block.
//  * x rows are stored 16-byte-chunk swizzled (chunk c of row r at c ^ swz(r)) so the fragment
//    reads of 16 rows at one K offset have no LDS bank conflicts (tiled_swz).
//  * One barrier per stage: after it, the stage's loads from every wave have landed and every
//    wave has finished reading the slot the next loads overwrite. The 256 x 256 tiles instead
//    run their two wave rows half a phase apart, two barriers per phase, so one wave's MFMAs run
//    while the other wave of its SIMD reads (ping-pong: PING in W8A8, pairs of stages per phase;
//    PW in W8A16, one stage per phase).
//  * Output: each lane stores its four bf16 of a 16 x 16 tile directly (8 bytes), except in
//    256 x 256 launches of three or more rounds of blocks (W8A16) or more than one round without
//    an int32 output (W8A8), where the tile is staged in the stage ring once the K loop is done
//    and written as whole rows (STAGE_Y).
//
// Tile order. Blocks are dispatched round-robin over the 8 XCDs; the tile index is remapped so
// each XCD runs a contiguous range of tiles, in groups of kGroupM token blocks x consecutive
// weight panels (token blocks fastest within a group). The ~32 blocks resident at once on one
// XCD then form a 4 x 8 rectangle of tiles whose x and weight panels they share through that
// XCD's L2: per tile step, a quarter of the operand bytes come from beyond L2 compared with a
// 32 x 1 strip.
//
// Summation order: the K steps in increasing order, two K=32 MFMAs per step (W8A16) in a fixed
// chain per output; it depends only on K, or with K splits (65..256 tokens over a narrow weight,
// 257..1024 over a deep, narrow one: tiled_splits) on the split count too: each range's steps in
// order, then the ranges added in order by a second pass. int32 accumulation (W8A8) is exact in
// any order.
//
// Fused gate/up (GLU): with the weight in the gate/up layout (lse_common.h) a block's first row
// tile is even and a wave's TN row tiles are an even-aligned run, so its tiles j (even, gate) and
// j + 1 (up) hold the same output columns in the same lanes; the epilogue writes
// h = bf16(silu(g) * u) for them.
#include <algorithm>
#include <type_traits>

#include "lse_common.h"

namespace lse {

struct TiledArgs {
  const void* x;     // W8A16: bf16 (M rows, stride ldx); W8A8: int8 xq (M rows, stride ldx)
  int64_t ldx;       // elements
  const int8_t* qp;  // packed weight tiles
  const float* s;    // (N) per-channel scales
  const float* sx;   // (M) per-token scales, W8A8 only
  uint16_t* y;       // (M, N) bf16, stride ldy; may be null in W8A8
  int64_t ldy;
  int32_t* acc;      // (M, N) int32 contiguous, W8A8 only; may be null
  int M, N, K;
  int nsteps;        // ceil(K / 64)
  int nrb;           // ceil(N / 16)
  int mblocks, nblocks;
  int glu;           // gate/up layout: I, the output columns (N = 16 nrb packed rows); else 0
  int glu_up;        //   and the offset of the up scales from the gate scales in s
  int splits;        // > 1 (no gate/up): K split into ranges of ssteps steps, raw partial sums
  int ssteps;        //   (fp32, or int32 in W8A8) to part, added by the decode kernel's second
  void* part;        //   pass; [splits][M][16 nrb]
};

constexpr int kGroupM = 4;
constexpr int kTiledThreads = 512;  // 8 waves in every wave layout

template <bool I8>
__device__ __forceinline__ int tiled_swz(int r) {
  // A fragment read (ds_read_b128) takes one logical chunk of 16 consecutive rows per lane
  // group. Measured on MI355X with SQ_LDS_BANK_CONFLICT, these swizzles read with no conflict:
  // bf16 rows (128 bytes, 8 chunks) (r & 7) ^ ((r >> 3) & 1), int8 rows (64 bytes, 4 chunks)
  // (r >> 1) & 3. (The (r >> 1) & 7 and (r >> 2) & 3 spreads, conflict-free on a plain model of
  // 64 four-byte banks served 16 lanes at a time, cost 4 conflict cycles per read.)
  return I8 ? (r >> 1) & 3 : (r & 7) ^ ((r >> 3) & 1);
}

// NT: weights loaded with the streaming cache policy (decode tiles, where each weight byte is
// read by one block only). BFW: bf16 weights (the lm_head kept in bf16) in the 2 KB-per-step
// tile layout, whose two 1 KB halves are the lo / hi operands an int8 tile dequantizes to: the
// tiles are read from LDS as they are, with no scales, y = bf16(sum).
template <bool I8, int BM, int BN, int WGM, int WGN, int NST, bool GLU, bool NT = false,
          bool BFW = false, bool STAGE_Y = false>
__global__ void __launch_bounds__(64 * WGM * WGN)
tiled_gemm_kernel(TiledArgs a) {
  using Acc = std::conditional_t<I8, i32x4, f32x4>;
  static_assert(!BFW || (!I8 && !GLU), "bf16 weights: plain W16A16 only");
  static_assert(!STAGE_Y || (!GLU && !BFW && (!I8 || (BM == 256 && BN == 256 && WGM == 2))),
                "staged output: plain W8A16, or the W8A8 256 x 256 tile");
  constexpr int W = WGM * WGN;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int TM = WM / 16, TN = WN / 16;
  constexpr int ESZ = I8 ? 1 : 2;
  constexpr int XROW = 64 * ESZ;            // bytes of one x row per stage
  constexpr int XCH = XROW / 16;            // 16-byte chunks per row
  constexpr int XBYTES = BM * XROW;         // x bytes per stage
  constexpr int WTILES = BN / 16;           // weight tiles per stage
  constexpr int WH = BFW ? 2 : 1;           // 1 KB pieces per weight tile and stage
  constexpr int XI = XBYTES / (W * 1024);   // direct-to-LDS loads per wave per stage, x
  // ... weights: WTILES WH pieces of 1 KB over W waves; when W does not divide them (192-row
  // tiles: 12 over 8) the last loads fall past the tiles, read zeros into padding and move no data.
  constexpr int WI = (WTILES * WH + W - 1) / W;
  constexpr int LOADS = XI + WI;
  static_assert(TM >= 1 && TN >= 1, "wave grid must tile the block");
  static_assert(XBYTES % (W * 1024) == 0, "whole 1 KB x loads per wave");
  static_assert(NST >= 3 && NST <= 4, "three or four stage slots");
  static_assert((NST - 2) * LOADS < 64, "vmcnt holds at most 63");
  static_assert(!GLU || TN % 2 == 0, "gate/up wave tiles hold whole pairs of row tiles");
  // W8A16 with one wave row (each weight tile read and dequantized by one wave): weights are
  // loaded a stage ahead of x and dequantized under the previous stage's MFMAs. On MI355X
  // 1-8 % faster for the 256 x 256 tile and up to 8 % for 64 x 128 at M = 512; with two wave
  // rows (2 x 4) it measured 3-5 % slower, so those keep the plain schedule.
  constexpr bool WAHEAD = !I8 && !BFW && WGM == 1;
  // W8A8 256 x 256 (2 x 4 waves of 128 x 64, 32 MFMAs per wave and stage): the two wave rows
  // run the K loop half a pair of stages apart (ping-pong, below). On MI355X at M = 512..4096
  // over the Llama-3-8B shapes 3-12 % faster than the common schedule with one stage per phase,
  // bit-identical, and two stages per phase another 1-3 % (ten of ten cases, alternated); on
  // the 128 x 256, 256 x 128 and 128 x 128 tiles (16 or 8 MFMAs per wave and stage, shorter than
  // a wave's reads and DMA issue) ping-pong measured 2-20 % slower, so they keep the common
  // schedule.
  constexpr bool PING = I8 && BM == 256 && BN == 256 && WGM == 2 && WGN == 4 && !NT;
  // W8A16 256 x 256 (2 x 4 waves of 128 x 64, 64 MFMAs per wave and stage): the same two wave
  // rows half a stage apart, one stage per phase (PW, below).
  constexpr bool PW = !I8 && !BFW && BM == 256 && BN == 256 && WGM == 2 && WGN == 4 && !NT;

  // One LDS array per stage slot (x image, then the weight tiles and their padding); with
  // STAGE_Y one array of all NST slots, which the epilogue reuses for the block's output tile.
  constexpr int SLOT = (XBYTES + WI * W * 1024) / 16;
  __shared__ uint4 st0[STAGE_Y ? NST * SLOT : SLOT], st1[STAGE_Y ? 1 : SLOT],
      st2[STAGE_Y ? 1 : SLOT], st3[!STAGE_Y && NST > 3 ? SLOT : 1];
  auto xslot = [&](int i) -> uint4* {
    if constexpr (STAGE_Y) return st0 + i * SLOT;
    switch (i) {
      case 0: return st0;
      case 1: return st1;
      case 2: return st2;
      default: return st3;
    }
  };
  auto wslot = [&](int i) -> uint4* { return xslot(i) + XBYTES / 16; };

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WGN, wn = wave % WGN;
  const int r16 = lane & 15, g = lane >> 4;

  // XCD-aware tile order (see the header comment): XCD x = b % 8 receives blocks x, x + 8, ...;
  // give it the contiguous tile range starting at the tiles of XCDs before it.
  // K range of this block: all of K, or with splits > 1 its split's steps (blockIdx % splits).
  const int S = a.splits > 1 ? a.splits : 1;
  const int sp = blockIdx.x % S;
  const int kbeg = sp * (S > 1 ? a.ssteps : 0);
  const int kend = S > 1 ? min(kbeg + a.ssteps, a.nsteps) : a.nsteps;
  const int T = a.mblocks * a.nblocks;
  const int b = blockIdx.x / S, xcd = b & 7, l = b >> 3, q8 = T >> 3, rem = T & 7;
  const int t = xcd * q8 + min(xcd, rem) + l;
  const int group = t / (kGroupM * a.nblocks), first_bm = group * kGroupM;
  const int gm = min(a.mblocks - first_bm, kGroupM);
  const int tg = t - group * kGroupM * a.nblocks;
  const int bm = first_bm + tg % gm, bn = tg / gm;
  const int m0 = bm * BM, n0 = bn * BN, rb0 = n0 / 16;

  // The scales the block's epilogue applies, staged in LDS by direct-to-LDS loads issued before
  // the stage prologue (every later wait covers them): per-channel scales of its BN output rows
  // (gate/up: gate and up scales of its BN / 2 output columns) and in W8A8 the per-token scales
  // of its BM rows; a 1 KB load each, zeros past N and M. Read from global memory after the last
  // MFMA they were a string of dependent small loads: on MI355X the W8A8 256 x 256 tile took
  // 447 against 497 us for gate_up at M = 4096 (70 against 77 at 512), o_proj 70 against 77,
  // down_proj 202 against 212; the other tiles 0-4 % less. Same values.
  // (Not the 96-row tile: it fills exactly half the LDS, two blocks per CU, and reads its scales
  // from global memory.)
  constexpr bool SCL = !BFW && BM != 96;
  constexpr int SC_UP = 256, SC_X = GLU ? 512 : 256;
  __shared__ float sc_lds[SCL ? SC_X + (I8 ? 256 : 0) : 1];
  // Scale of output row (column) n / gate and up scales of output column n / token scale of m.
  auto scale_n = [&](int n) { return SCL ? sc_lds[n - n0] : a.s[n]; };
  auto scale_gate = [&](int n) { return SCL ? sc_lds[n - 16 * (rb0 >> 1)] : a.s[n]; };
  auto scale_up = [&](int n) {
    return SCL ? sc_lds[SC_UP + n - 16 * (rb0 >> 1)] : a.s[a.glu_up + n];
  };
  auto scale_m = [&](int m) { return SCL ? sc_lds[SC_X + m - m0] : a.sx[m]; };
  if constexpr (SCL) {
    if (S == 1) {
      const int c0 = GLU ? 16 * (rb0 >> 1) : n0;  // first output column (gate/up: of the gate half)
      const int ncols = GLU ? a.glu : a.N;
      const uint32_t cbytes = (uint32_t)max(0, ncols - c0) * 4u;
      if (wave == 0) dma16_lds<0>(make_rsrc4(a.s + c0, cbytes), lds_addr(sc_lds), 16u * lane);
      if (GLU && wave == 1)
        dma16_lds<0>(make_rsrc4(a.s + a.glu_up + c0, cbytes), lds_addr(sc_lds + SC_UP), 16u * lane);
      if (I8 && wave == 2)
        dma16_lds<0>(make_rsrc4(a.sx + m0, (uint32_t)max(0, a.M - m0) * 4u), lds_addr(sc_lds + SC_X),
                     16u * lane);
    }
  }
  // Buffer resources based at the block's first row / row tile, so 32-bit offsets suffice.
  const int rows = min(BM, a.M - m0);
  const u32x4 xres = make_rsrc4(static_cast<const char*>(a.x) + (int64_t)m0 * a.ldx * ESZ,
                                (uint32_t)(((int64_t)(rows - 1) * a.ldx + a.K) * ESZ));
  const int rtiles = min(WTILES, a.nrb - rb0);
  const u32x4 qres = make_rsrc4(a.qp + (int64_t)rb0 * a.nsteps * kTileBytes * WH,
                                (uint32_t)rtiles * (uint32_t)a.nsteps * kTileBytes * WH);

  // Lane l of load i of a stage fills byte 1024 (wave + W i) + 16 l of the slot's x image: row
  // r = RPL (wave + W i) + l / XCH (RPL = 1024 / XROW rows per load), physical chunk l % XCH,
  // which holds logical chunk (l % XCH) ^ swz(r). W RPL is a multiple of 16, so swz(r) is the same
  // for every i and the lane's K byte is fixed; only the row moves, by W RPL per load.
  constexpr int RPL = 1024 / XROW;
  static_assert((W * RPL) % 16 == 0, "swizzle must not depend on the load index");
  const int x_r0 = RPL * wave + lane / XCH;
  const int x_kb = 16 * ((lane % XCH) ^ tiled_swz<I8>(x_r0));
  const int64_t x_step = (int64_t)W * RPL * a.ldx * ESZ;
  const uint32_t x_base = (uint32_t)((int64_t)x_r0 * a.ldx * ESZ + x_kb);
  // LDS byte addresses of this wave's first x piece and first weight tile in each slot; load i
  // goes W KB further.
  uint32_t x_lds[NST], w_lds[NST];
#pragma unroll
  for (int i = 0; i < NST; ++i) {
    x_lds[i] = lds_addr(xslot(i) + 64 * wave);
    w_lds[i] = lds_addr(wslot(i) + 64 * wave);
  }
  // Stage kt (an index within the block's K range) of x / of the weights into slot `slot`.
  auto load_x = [&](int kt, int slot) {
    kt += kbeg;
    const bool kv = kt < kend && XROW * kt + x_kb < a.K * ESZ;
    uint32_t xo[XI];
#pragma unroll
    for (int i = 0; i < XI; ++i) {
      const bool rv = x_r0 + W * RPL * i < rows;
      xo[i] = kv && rv ? x_base + (uint32_t)(i * x_step) + XROW * kt : kOutOfRange;
    }
    dma16_lds_seq<1024 * W>(xres, x_lds[slot], xo, std::make_integer_sequence<int, XI>{});
  };
  // Load i of a wave fills 1 KB piece p = wave + W i of the slot's weight part: half p % WH of
  // tile p / WH (with bf16 weights tile t's lo half lands at piece 2 t, its hi half at 2 t + 1).
  auto load_w = [&](int kt, int slot) {
    kt += kbeg;
    const bool live = kt < kend;
    uint32_t wo[WI];
#pragma unroll
    for (int i = 0; i < WI; ++i) {
      const int piece = wave + W * i, tile = piece / WH, half = piece % WH;
      wo[i] = live && tile < rtiles
                  ? ((uint32_t)tile * (uint32_t)a.nsteps + (uint32_t)kt) * (kTileBytes * WH) +
                        kTileBytes * half + 16u * lane
                  : kOutOfRange;
    }
    dma16_lds_seq<1024 * W, NT>(qres, w_lds[slot], wo, std::make_integer_sequence<int, WI>{});
  };

  Acc acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = Acc{0, 0, 0, 0};

  auto compute = [&](int slot) {
    const uint4* xs = xslot(slot);
    const uint4* ws = wslot(slot) + 64 * WH * wn * TN + lane;
    if constexpr (I8) {
      uint4 wv[TN];
#pragma unroll
      for (int j = 0; j < TN; ++j) wv[j] = ws[64 * j];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int r = wm * WM + 16 * i + r16;
        const uint4 xv = xs[r * XCH + (g ^ tiled_swz<I8>(r))];
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma_i8(wv[j], xv, acc[i][j]);
      }
    } else {
      bf16x8 lo[TN], hi[TN];
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        if constexpr (BFW) {
          lo[j] = as_bf16x8(ws[128 * j]);
          hi[j] = as_bf16x8(ws[128 * j + 64]);
        } else {
          dequant16(ws[64 * j], lo[j], hi[j]);
        }
      }
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int r = wm * WM + 16 * i + r16;
        const int sw = tiled_swz<I8>(r);
        const uint4 x0 = xs[r * XCH + ((2 * g) ^ sw)];
        const uint4 x1 = xs[r * XCH + ((2 * g + 1) ^ sw)];
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          acc[i][j] = mfma16x16x32(lo[j], as_bf16x8(x0), acc[i][j]);
          acc[i][j] = mfma16x16x32(hi[j], as_bf16x8(x1), acc[i][j]);
        }
      }
    }
  };

  const int nloc = kend - kbeg;  // K steps of this block
  // The K loop runs groups of NST steps (slot i of a group is a constant). With GROUPS_CLEAN,
  // whole groups run with no test inside (in the one-row W8A16 schedule the weight registers
  // then rotate without copies) and only a last, partial group tests which steps lie in the
  // block's range; otherwise every step tests. Measured on MI355X against testing every step:
  // W8A8 tiles 0-6 % faster, W8A16 64 x 128 one-row tiles up to 6 % faster, while the W8A16
  // 2 x 4 and 32 x 128 tiles ran 2-13 % slower with it.
  constexpr bool GROUPS_CLEAN = I8 || (WAHEAD && BM == 64);
  auto run_steps = [&](auto&& step) {
    int kt0 = 0;
    if constexpr (GROUPS_CLEAN) {
      for (; kt0 + NST <= nloc; kt0 += NST) {
#pragma unroll
        for (int i = 0; i < NST; ++i) step(kt0 + i, i, true);
      }
      if (kt0 >= nloc) return;
    }
    for (; kt0 < nloc; kt0 += NST) {
#pragma unroll
      for (int i = 0; i < NST; ++i) step(kt0 + i, i, kt0 + i < nloc);
    }
  };
  if constexpr (WAHEAD) {
    // Weights one stage ahead of x: iteration kt issues x of stage kt + NST - 1 and the weights
    // of stage kt + NST (into the weight half of slot kt % NST, whose stage-kt tiles were
    // dequantized during iteration kt - 1), runs stage kt's MFMAs on weights dequantized during
    // iteration kt - 1, and dequantizes stage kt + 1's weights between them. The wait keeps the
    // same NST - 2 load groups in flight as the plain schedule.
    bf16x8 lo[TN], hi[TN];
    load_w(0, 0);
#pragma unroll
    for (int i = 0; i < NST - 1; ++i) {
      load_x(i, i);
      load_w(i + 1, (i + 1) % NST);
    }
    __builtin_amdgcn_s_waitcnt(vmcnt_imm((NST - 2) * LOADS));
    __builtin_amdgcn_s_barrier();
    {
      const uint4* ws = wslot(0) + 64 * wn * TN + lane;
#pragma unroll
      for (int j = 0; j < TN; ++j) dequant16(ws[64 * j], lo[j], hi[j]);
    }
    auto step = [&](int kt, int i, bool live) {
      // x of stage kt and weights of stage kt + 1 landed for every wave after the barrier, and
      // every wave's reads of the slot the loads below overwrite have completed.
      __builtin_amdgcn_s_waitcnt(vmcnt_lgkm0_imm((NST - 2) * LOADS));
      __builtin_amdgcn_s_barrier();
      load_x(kt + NST - 1, (i + NST - 1) % NST);
      load_w(kt + NST, i);
      if (live) {
        const uint4* xs = xslot(i);
        const uint4* wsn = wslot((i + 1) % NST) + 64 * wn * TN + lane;
        uint4 wraw[TN];
#pragma unroll
        for (int j = 0; j < TN; ++j) wraw[j] = wsn[64 * j];
        bf16x8 lo_n[TN], hi_n[TN];
#pragma unroll
        for (int ii = 0; ii < TM; ++ii) {
          const int r = wm * WM + 16 * ii + r16;
          const int sw = tiled_swz<I8>(r);
          const uint4 x0 = xs[r * XCH + ((2 * g) ^ sw)];
          const uint4 x1 = xs[r * XCH + ((2 * g + 1) ^ sw)];
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            acc[ii][j] = mfma16x16x32(lo[j], as_bf16x8(x0), acc[ii][j]);
            acc[ii][j] = mfma16x16x32(hi[j], as_bf16x8(x1), acc[ii][j]);
          }
          if (ii == 0) {
#pragma unroll
            for (int j = 0; j < TN; ++j) dequant16(wraw[j], lo_n[j], hi_n[j]);
          }
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          lo[j] = lo_n[j];
          hi[j] = hi_n[j];
        }
      }
    };
    run_steps(step);
  } else if constexpr (PING) {
    // Ping-pong: the wave rows alternate. Each SIMD holds one wave of each row; while row 0
    // issues its 64 MFMAs of a pair of K stages, row 1 reads its fragments of that pair (and the
    // reverse a phase later), so the matrix core sees one wave's MFMA run after the other's
    // instead of both waves stalling on LDS reads and the barrier together. Pair q is stages
    // 2q, 2q+1 in slots 2(q & 1), 2(q & 1) + 1. Row 1 starts one barrier late; every wave then
    // passes two barriers per pair (after its reads, after its MFMAs) and row 0 one more at the
    // end, so both rows pass the same count. Phases (c = barrier count): row 0 reads pair q while
    // row 1 multiplies pair q - 1, then row 0 multiplies pair q while row 1 reads it.
    //  * The loads split by wave row, so that no wave's DMA can overwrite LDS another wave of its
    //    row still reads: row 0 fills the x image (wave w: 1 KB pieces w + 4 i, i < 4), each
    //    row-1 wave the four weight tiles its wave column reads, which only it and the row-0
    //    wave of that column read. (Split as in the common schedule, a row-1 wave's DMA raced
    //    the other row-1 waves' fragment reads of the x rows it had loaded; seen only when the
    //    DMA read past K, whose zeros land at once.)
    //  * Row 0 issues x of pair q + 1 at the top of its reading phase of pair q, into the slots
    //    of pair q - 1, which row 1 finished reading at the barrier that opened the phase; it
    //    waits for that DMA (vmcnt 0) after its MFMAs of pair q, before the barrier that opens
    //    its reads of pair q + 1.
    //  * Row 1 issues the weights of pair q + 2 at the end of its reading phase of pair q, into
    //    the slots of pair q, which the row-0 wave of its column read in the phase before; its
    //    wait there (all but that pair) lands the weights of pair q + 1 before the same barrier.
    static_assert(NST == 4 && XI + WI == 4 && TN == 4 && XBYTES == 4 * 4096 && WH == 1,
                  "ping-pong: two pairs of slots, four 1 KB loads per wave and stage");
    const bool row1 = wm == 1;
    const uint32_t x_step4 = (uint32_t)(4 * RPL) * (uint32_t)a.ldx;
    auto load_x4 = [&](int kt, int slot) {
      kt += kbeg;
      const bool kv = kt < kend && XROW * kt + x_kb < a.K;
      uint32_t xo[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        xo[i] = kv && x_r0 + 4 * RPL * i < rows ? x_base + i * x_step4 + XROW * kt : kOutOfRange;
      dma16_lds_seq<4096>(xres, x_lds[slot], xo, std::make_integer_sequence<int, 4>{});
    };
    auto load_w4 = [&](int kt, int slot) {
      kt += kbeg;
      uint32_t wo[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int tile = TN * wn + i;
        wo[i] = kt < kend && tile < rtiles
                    ? ((uint32_t)tile * (uint32_t)a.nsteps + (uint32_t)kt) * kTileBytes + 16u * lane
                    : kOutOfRange;
      }
      dma16_lds_seq<1024>(qres, lds_addr(wslot(slot) + 64 * TN * wn), wo,
                          std::make_integer_sequence<int, 4>{});
    };
    auto load4 = [&](int kt, int slot) {
      if (row1)
        load_w4(kt, slot);
      else
        load_x4(kt, slot);
    };
    load4(0, 0);
    load4(1, 1);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    __builtin_amdgcn_s_barrier();
    if (row1) {
      load_w4(2, 2);
      load_w4(3, 3);
      __builtin_amdgcn_s_barrier();
    }
    __builtin_amdgcn_sched_barrier(0);
    auto pair = [&](int q, auto slot_pair, bool live0, bool live1) {
      constexpr int sb = 2 * decltype(slot_pair)::value;  // slots of pair q
      constexpr int so = 2 - sb;                          // slots of pairs q - 1 and q + 1
      if (!row1) {
        load_x4(2 * q + 2, so);
        load_x4(2 * q + 3, so + 1);
      }
      uint4 wv[2][TN], xv[2][TM];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint4* xs = xslot(sb + h);
        const uint4* ws = wslot(sb + h) + 64 * wn * TN + lane;
#pragma unroll
        for (int j = 0; j < TN; ++j) wv[h][j] = ws[64 * j];
#pragma unroll
        for (int ii = 0; ii < TM; ++ii) {
          const int r = wm * WM + 16 * ii + r16;
          xv[h][ii] = xs[r * XCH + (g ^ tiled_swz<I8>(r))];
        }
      }
      __builtin_amdgcn_s_waitcnt(vmcnt_lgkm0_imm(63));
      if (row1) {
        load_w4(2 * q + 4, sb);
        load_w4(2 * q + 5, sb + 1);
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(8));
      }
      // The fences keep the compiler from moving MFMAs or reads across the phase barriers.
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        if (h == 0 ? live0 : live1) {
#pragma unroll
          for (int ii = 0; ii < TM; ++ii)
#pragma unroll
            for (int j = 0; j < TN; ++j) acc[ii][j] = mfma_i8(wv[h][j], xv[h][ii], acc[ii][j]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      if (!row1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
    };
    for (int q0 = 0; 2 * q0 < nloc; q0 += 2) {
      pair(q0, std::integral_constant<int, 0>{}, 2 * q0 < nloc, 2 * q0 + 1 < nloc);
      pair(q0 + 1, std::integral_constant<int, 1>{}, 2 * q0 + 2 < nloc, 2 * q0 + 3 < nloc);
    }
    if (!row1) __builtin_amdgcn_s_barrier();
  } else if constexpr (PW) {
    // W8A16 ping-pong, one stage per phase: wave row 1 starts one barrier late, then each wave
    // alternates a memory phase (its DMA share of stage kt + NST - 1, its fragment reads of
    // stage kt, the dequantization of its first weight tile) and an MFMA phase (64 MFMAs, with
    // the other three tiles dequantized between the MFMAs of the tiles before them, two VALU ops
    // after each MFMA), two barriers per stage. Every DMA is issued at the top of a memory phase,
    // into the slot of stage kt - 1, which both rows finished reading before the barrier that
    // opened the phase; a wave's wait (all but its newest stage) lands its share of stage
    // kt + 1 before the barrier that opens row 0's reads of it. Same summation order as the
    // 1 x 8 layout (each output adds its K stages in order, lo then hi half), so bit-identical.
    // The dequantization is duplicated over the two rows but runs beside MFMAs of the same wave;
    // the x fragment reads per stage halve (160 against 272 KB of LDS reads per block).
    static_assert(NST == 3 && TN == 4 && TM == 8, "W8A16 256 x 256 ping-pong");
    const bool row1 = wm == 1;
#pragma unroll
    for (int i = 0; i < NST - 1; ++i) {
      load_x(i, i);
      load_w(i, i);
    }
    __builtin_amdgcn_s_waitcnt(vmcnt_imm((NST - 2) * LOADS));
    __builtin_amdgcn_s_barrier();
    if (row1) __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    auto step = [&](int kt, int i, bool live) {
      load_x(kt + NST - 1, (i + NST - 1) % NST);
      load_w(kt + NST - 1, (i + NST - 1) % NST);
      const uint4* xs = xslot(i);
      const uint4* ws = wslot(i) + 64 * wn * TN + lane;
      uint4 wraw[TN], x0[TM], x1[TM];
#pragma unroll
      for (int j = 0; j < TN; ++j) wraw[j] = ws[64 * j];
#pragma unroll
      for (int ii = 0; ii < TM; ++ii) {
        const int r = wm * WM + 16 * ii + r16;
        const int sw = tiled_swz<I8>(r);
        x0[ii] = xs[r * XCH + ((2 * g) ^ sw)];
        x1[ii] = xs[r * XCH + ((2 * g + 1) ^ sw)];
      }
      bf16x8 lo[TN], hi[TN];
      dequant16(wraw[0], lo[0], hi[0]);
      __builtin_amdgcn_s_waitcnt(vmcnt_lgkm0_imm(63));
      if (row1) __builtin_amdgcn_s_waitcnt(vmcnt_imm((NST - 2) * LOADS));
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
      if (live) {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          if (j + 1 < TN) dequant16(wraw[j + 1], lo[j + 1], hi[j + 1]);
#pragma unroll
          for (int ii = 0; ii < TM; ++ii) {
            acc[ii][j] = mfma16x16x32(lo[j], as_bf16x8(x0[ii]), acc[ii][j]);
            acc[ii][j] = mfma16x16x32(hi[j], as_bf16x8(x1[ii]), acc[ii][j]);
          }
        }
        // One MFMA, then two VALU ops of the next tile's dequantization. On MI355X the MFMA
        // phase took 1259-1329 clocks against 1400-1449 with each tile dequantized just before
        // its MFMAs, the compiler's own order.
#pragma unroll
        for (int k = 0; k < 2 * TM * TN; ++k) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      if (!row1) __builtin_amdgcn_s_waitcnt(vmcnt_imm((NST - 2) * LOADS));
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
    };
    run_steps(step);
    if (!row1) __builtin_amdgcn_s_barrier();
  } else {
    // Prologue: stages 0 .. NST-2 in flight.
#pragma unroll
    for (int i = 0; i < NST - 1; ++i) {
      load_x(i, i);
      load_w(i, i);
    }
    auto step = [&](int kt, int i, bool live) {
      // This wave's loads of stage kt landed (the NST-2 later stages may still be in flight)
      // and its reads of slot (i - 1) completed; after the barrier every wave's have, so the
      // loads below may overwrite slot (i - 1). Waiting for the reads here (lgkmcnt 0) costs
      // 0-2 % on MI355X against letting the barrier pass reads still in flight.
      __builtin_amdgcn_s_waitcnt(vmcnt_lgkm0_imm((NST - 2) * LOADS));
      __builtin_amdgcn_s_barrier();
      load_x(kt + NST - 1, (i + NST - 1) % NST);
      load_w(kt + NST - 1, (i + NST - 1) % NST);
      if (live) compute(i);
    };
    run_steps(step);
  }

  // The last stages' loads (past K: they write zeros into their slots) are drained before the
  // epilogue.
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));

  // Epilogue. D tile (i, j): lane holds weight rows 4 g + r (r = 0..3) of token r16.
  if constexpr (!GLU) {
    if (S > 1) {  // raw partial sums of split sp, rows padded to 16 nrb (whole 16-byte stores)
      Acc* part = static_cast<Acc*>(a.part);
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int m = m0 + wm * WM + 16 * i + r16;
        if (m >= a.M) continue;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int n = n0 + wn * WN + 16 * j + 4 * g;
          if (n < 16 * a.nrb) part[(((int64_t)sp * a.M + m) * (16 * a.nrb) + n) / 4] = acc[i][j];
        }
      }
      return;
    }
  }
  const bool yvec = a.y && (a.ldy & 3) == 0 && ((uintptr_t)a.y & 7) == 0;
  if constexpr (GLU) {
    // Row tile rb = rb0 + wn TN + j (even j: gate) covers output columns 16 (rb / 2) + 4 g + r.
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int m = m0 + wm * WM + 16 * i + r16;
      if (m >= a.M) continue;
      const float sxm = I8 ? scale_m(m) : 0.0f;
#pragma unroll
      for (int j = 0; j < TN; j += 2) {
        const int n = 16 * ((rb0 + wn * TN + j) >> 1) + 4 * g;
        if (n >= a.glu) continue;
        const int cnt = min(4, a.glu - n);
        float sg[4], su[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          sg[r] = r < cnt ? scale_gate(n + r) : 0.0f;
          su[r] = r < cnt ? scale_up(n + r) : 0.0f;
        }
        store_glu4<I8>(a.y, a.ldy, m, n, cnt, acc[i][j], acc[i][j + 1], sg, su, sxm, yvec);
      }
    }
    return;
  }
  if constexpr (STAGE_Y && I8) {
    // W8A8 (no int32 output): each wave's 128 x 64 bf16 tile goes through its own 16 KB of the
    // ring (rows of 128 bytes whose 16-byte chunks are XOR-swizzled by row) and out as whole
    // 128-byte row segments, 8 rows per store, with the nontemporal policy; the direct stores
    // below write 32-byte pieces of 16 rows each. Same values. On MI355X over launches of more
    // than one round of blocks 3-11 % faster (gate_up at M = 2048 / 4096: 253 -> 229 /
    // 457 -> 408 us); with one round up to 8 % slower, so the host picks it for longer launches.
    static_assert(WN == 64 && W * WM * WN * 2 <= NST * SLOT * 16, "per-wave staging fits the ring");
    if (a.y && (a.ldy & 7) == 0 && ((uintptr_t)a.y & 15) == 0 && !a.acc) {
      __syncthreads();  // every wave's reads of the ring have completed (loads drained above)
      char* ys = reinterpret_cast<char*>(st0 + wave * (WM * 128 / 16));
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int row = 16 * i + r16, m = m0 + wm * WM + row;
        const float sxm = m < a.M ? scale_m(m) : 0.0f;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int n = n0 + wn * WN + 16 * j + 4 * g;
          float o[4];
#pragma unroll
          for (int r = 0; r < 4; ++r)
            o[r] = scaled<I8>(acc[i][j], r, n + r < a.N ? scale_n(n + r) : 0.0f, sxm);
          const int chunk = (2 * j + (g >> 1)) ^ (row & 7);
          *reinterpret_cast<uint2*>(ys + row * 128 + chunk * 16 + 8 * (g & 1)) =
              make_uint2(pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]));
        }
      }
      // A wave's LDS accesses complete in order, so its reads below see its writes above.
#pragma unroll
      for (int k = 0; k < WM / 8; ++k) {
        const int row = 8 * k + (lane >> 3), c = lane & 7;
        const int m = m0 + wm * WM + row, n = n0 + wn * WN + 8 * c;
        const u32x4 v = *reinterpret_cast<const u32x4*>(ys + row * 128 + ((c ^ (row & 7)) * 16));
        if (m >= a.M || n >= a.N) continue;
        uint16_t* out = a.y + (int64_t)m * a.ldy + n;
        if (n + 8 <= a.N) {
          __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(out));
        } else {
          const uint16_t* e = reinterpret_cast<const uint16_t*>(&v);
          for (int t = 0; t < a.N - n; ++t) out[t] = e[t];
        }
      }
      return;
    }
  } else if constexpr (STAGE_Y) {
    // The block's bf16 tile goes through LDS (rows padded by 16 bytes, which spreads the
    // 16-row column writes over the banks) and out as whole rows of 16-byte stores. Same values
    // as the direct stores below, which remain for a y not 16-byte aligned row by row.
    constexpr int YROW = BN * 2 + 16;
    static_assert(BM * YROW <= NST * SLOT * 16, "the output tile fits the stage ring");
    if (a.y && (a.ldy & 7) == 0 && ((uintptr_t)a.y & 15) == 0) {
      char* ys = reinterpret_cast<char*>(st0);
      __syncthreads();  // every wave's reads of the ring have completed (loads drained above)
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int ml = wm * WM + 16 * i + r16;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int nl = wn * WN + 16 * j + 4 * g, n = n0 + nl;
          float o[4];
#pragma unroll
          for (int r = 0; r < 4; ++r)
            o[r] = scaled<false>(acc[i][j], r, n + r < a.N ? scale_n(n + r) : 0.0f, 0.0f);
          *reinterpret_cast<uint2*>(ys + ml * YROW + nl * 2) =
              make_uint2(pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]));
        }
      }
      __syncthreads();
      constexpr int CPR = BN / 8;  // 16-byte chunks per row
      const int cols = min(BN, a.N - n0);
      for (int c = threadIdx.x; c < BM * CPR; c += 64 * W) {
        const int r = c / CPR, nl = 8 * (c % CPR);
        if (r >= rows || nl >= cols) continue;
        const uint4 v = *reinterpret_cast<const uint4*>(ys + r * YROW + nl * 2);
        uint16_t* out = a.y + (int64_t)(m0 + r) * a.ldy + n0 + nl;
        if (nl + 8 <= cols) {
          *reinterpret_cast<uint4*>(out) = v;
        } else {
          const uint16_t* e = reinterpret_cast<const uint16_t*>(&v);
          for (int t = 0; t < cols - nl; ++t) out[t] = e[t];
        }
      }
      return;
    }
  }
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int m = m0 + wm * WM + 16 * i + r16;
    if (m >= a.M) continue;
    const float sxm = I8 ? scale_m(m) : 0.0f;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = n0 + wn * WN + 16 * j + 4 * g;
      if (n >= a.N) continue;
      const int cnt = min(4, a.N - n);
      float sc[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) sc[r] = BFW ? 1.0f : r < cnt ? scale_n(n + r) : 0.0f;
      store_out4<I8>(a.y, a.ldy, a.acc, a.N, m, n, cnt, acc[i][j], sc, sxm, yvec);
    }
  }
}

// ---- host side -----------------------------------------------------------------------------

struct TiledShape {
  int bm, bn;
};

template <bool I8, int BM, int BN, bool GLU>
static const void* tiled_fn() {
  // LDS per block: NST x (x stage + weight stage) <= 160 KB; 128 x 128 tiles keep two blocks
  // per CU. Wave layout 2 x 4, except the W8A16 128 x 256 tile: there 1 x 8 (128 x 32 per wave)
  // dequantizes each weight tile in one wave instead of two, on MI355X 9-12 % faster (it reads
  // twice the x fragments, which the conflict-free swizzle and LDS's 256 bytes per clock of
  // b128 reads absorb). The W8A16 256 x 256 tile ran 1 x 8 as well (2-9 % faster than 2 x 4
  // with the common schedule) until its ping-pong schedule (PW), which on MI355X through the
  // library is 2-3 % faster at M = 8192 and 0-3 % at 512 and 2048 (alternated, one box). In
  // W8A8 (no dequantization) 2 x 4 stays faster. Stage slots: 3 for bf16 x (4 would not fit the 256 x 256 tile, and
  // measured no faster on the others), 4 for int8 x (with the 256 x 256 tile's ping-pong schedule
  // 1-2 % faster than 3).
  constexpr int nst = I8 ? 4 : 3;
  constexpr int wgm = (!I8 && BN == 256 && BM != 256) ? 1 : 2;
  static_assert(64 * wgm * (8 / wgm) == kTiledThreads, "8 waves");
  return reinterpret_cast<const void*>(
      &tiled_gemm_kernel<I8, BM, BN, wgm, 8 / wgm, nst, GLU>);
}

// `decode`: a decode route's tile (one block row, M <= 64), whose weights stream with the nt
// cache policy: on MI355X 7-12 % faster for the decode kernel's large weights, which share
// that policy, and 5-8 % for the 32 x 128 tile over gate_up. The split-K route keeps the default
// policy for its W8A16 64 x 128 tile (down_proj at 64 tokens: 7 % slower with nt).
// `one_row`: a launch of one block row (M <= BM), where each weight tile is read by one block only;
// the 128 x 128 tile then streams its weights with the nt policy too. Measured on MI355X over
// gate_up (plain and fused, K 4096, N 28672) at 65, 96 and 128 tokens: 4-10 % faster in 10 of the
// 12 cases of both modes in a harness (fused W8A16 at 65 tokens 42.7 -> 38.9 us, fused W8A8
// 28.3 -> 25.6 us), plain W8A16 gate_up -5 % to +4 %; in the bench's mid-range figures (random
// activations) W8A8 gate_up 2-4 % faster and W8A16 unchanged. With two block rows (M > 128) nt
// measured 8-14 % slower.
//
// `stage_y`, W8A8: a 256 x 256 launch (no gate/up, no int32 output) of more than one round of
// blocks, whose waves write their output tiles through LDS (STAGE_Y with I8).
// `stage_y`, W8A16: a 256 x 256 launch (no gate/up) of at least kStageYRounds rounds of blocks,
// whose output tiles go out through LDS as whole rows (STAGE_Y). Measured on MI355X against the
// direct stores, bit-identical: q/k/v at M = 8192 (3 rounds) 319 -> 311 us, gate_up at 8192 (14
// rounds) 1460 -> 1425 us, at 2048 (3.5 rounds) 410 -> 397 us; with one or two rounds unchanged
// or up to 1 % slower (o_proj, down_proj at 8192; at one K step 22.9 -> 30.6 us), and no gain
// in W8A8.
constexpr int kStageYRounds = 3;

template <bool I8, bool GLU>
static const void* tiled_kernel_for(const TiledShape& sh, bool decode = false,
                                    bool one_row = false, bool stage_y = false) {
  if (decode) {
    if constexpr (!I8) {
      if (sh.bm == 64)
        return reinterpret_cast<const void*>(
            &tiled_gemm_kernel<false, 64, 128, 1, 4, 4, GLU, true>);
      if (sh.bm == 32)
        return reinterpret_cast<const void*>(
            &tiled_gemm_kernel<false, 32, 128, 1, 4, 4, GLU, true>);
    } else {
      if (sh.bm == 64)
        return reinterpret_cast<const void*>(&tiled_gemm_kernel<true, 64, 128, 2, 2, 4, GLU, true>);
    }
  }
  if constexpr (!I8) {
    // 96 x 128 (65..96 tokens, one block row, so the weights stream with nt): four waves of
    // 96 x 32.
    if (sh.bm == 96)
      return reinterpret_cast<const void*>(&tiled_gemm_kernel<false, 96, 128, 1, 4, 4, GLU, true>);
    // 64 x 128 (narrow prefill; 33..64 tokens over a wide weight, launch_w8a16_wide_decode) and
    // 32 x 128 (17..32 tokens over a wide weight): four waves of BM x 32.
    if (sh.bm == 64)
      return reinterpret_cast<const void*>(&tiled_gemm_kernel<false, 64, 128, 1, 4, 4, GLU>);
    if (sh.bm == 32)
      return reinterpret_cast<const void*>(&tiled_gemm_kernel<false, 32, 128, 1, 4, 4, GLU>);
  } else {
    // 64 x 128 for narrow W8A8 prefill: four waves of 32 x 64 (2 x 2 measured 1-8 % faster
    // than 1 x 4 on MI355X).
    if (sh.bm == 64)
      return reinterpret_cast<const void*>(&tiled_gemm_kernel<true, 64, 128, 2, 2, 4, GLU>);
  }
  if (sh.bm == 256 && sh.bn == 256) {
    if constexpr (!I8 && !GLU) {
      if (stage_y)
        return reinterpret_cast<const void*>(
            &tiled_gemm_kernel<false, 256, 256, 2, 4, 3, false, false, false, true>);
    } else if constexpr (I8 && !GLU) {
      if (stage_y)
        return reinterpret_cast<const void*>(
            &tiled_gemm_kernel<true, 256, 256, 2, 4, 4, false, false, false, true>);
    }
    return tiled_fn<I8, 256, 256, GLU>();
  }
  if (sh.bm == 256 && sh.bn == 192) {
    if constexpr (I8 || GLU) return nullptr;  // W8A16 without gate/up only (tiled_shape)
    else return tiled_fn<false, 256, 192, false>();
  }
  if (sh.bm == 256 && sh.bn == 128) return tiled_fn<I8, 256, 128, GLU>();
  if (sh.bm == 128 && sh.bn == 256) return tiled_fn<I8, 128, 256, GLU>();
  if (one_row)
    return reinterpret_cast<const void*>(
        &tiled_gemm_kernel<I8, 128, 128, 2, 4, I8 ? 4 : 3, GLU, true>);
  return tiled_fn<I8, 128, 128, GLU>();
}

// The tile that minimizes the time of the busiest CU: ceil(tiles / CUs) x tile area / relative
// efficiency (big tiles need fewer LDS bytes per MFMA; small tiles fill the CUs when there are
// few tiles). A 128 x 128 tile keeps two blocks per CU, so its efficiency is the one measured
// with two resident. Efficiencies relative to 256 x 256, measured on MI355X at M = 8192 (many
// rounds), per mode, except the 64 x 128 tile's, fitted at M = 256..2048 where it competes. On
// the Llama-3-8B prefill shapes timed (qkv, o_proj, gate_up, down at M = 256 to 2048, gate_up at
// 8192) this picks the fastest tile, or one within 6 % (qkv at M = 512).
// The 64 x 128 tile (four waves) fills the CUs when M is a few hundred and N is narrow, e.g.
// o_proj and down at M = 256..512: 16-25 % faster than 128 x 128 there, in both modes.
// The 256 x 192 tile (2 x 4 waves of 128 x 48) gives 6144-row weights (the fused q/k/v) one
// round of 256 blocks at M = 2048: on MI355X W8A16 97.6 us there against 103-114 us for the
// 128 x 128 tiles, 0.92 of the 256 x 256 tile's rate at M = 8192. Only W8A16 non-gate/up
// launches consider it (tiled_shape).
// The 96 x 128 tile (four waves of 96 x 32, W8A16) holds 65..96 tokens in one block row with
// a quarter less padding than 128 x 128: on MI355X over gate_up (K 4096, N 28672) at 65 / 80 / 96
// tokens 36-37 / 33.5 / 33.8 us against 38.3 / 38.5 / 39.5 us, fused gate_up 31.5-32.6 against
// 37.6-38.8 us. Measured only there, so only launches of one such block row consider it.
constexpr int kTileCands = 7;
constexpr TiledShape kTileCand[kTileCands] = {{256, 256}, {256, 128}, {128, 256}, {128, 128},
                                              {64, 128},  {256, 192}, {96, 128}};
constexpr double kTileEff16[kTileCands] = {1.0, 0.86, 0.87, 0.835, 0.6, 0.92, 0.75};
// (256 x 192 and 96 x 128 serve W8A16 only.)
// W8A8 re-measured once its 256 x 256 tile ran ping-pong with LDS-staged scales (averages over
// the four shapes at M = 8192: 256 x 128 0.76, 128 x 256 0.80, 128 x 128 0.72); the picks that
// changed (gate_up at M = 384, q/k/v at 2048, o_proj and down_proj at 3072: 256 x 256 instead of
// 128 x 128) measured 11-19 % faster.
constexpr double kTileEff8[kTileCands] = {1.0, 0.76, 0.80, 0.72, 0.6, 0.926, 0.75};

// One round of candidate i on every CU, in the cost model's units.
template <bool I8>
static double tile_round_cost(int i) {
  return (double)kTileCand[i].bm * kTileCand[i].bn / (I8 ? kTileEff8 : kTileEff16)[i];
}

template <bool I8>
static TiledShape tiled_shape(int64_t M, int64_t N, int cus, double* cost_out = nullptr,
                              bool glu = false) {
  TiledShape best = kTileCand[0];
  double best_cost = 1e300;
  for (int i = 0; i < kTileCands; ++i) {
    // 256 x 192: W8A16 only (in W8A8 on par at M = 2048, 3-9 % slower than the bulk-and-tail
    // launches at 4096), and never for gate/up (2 x 4 waves of 3 row tiles: not pairs).
    if (kTileCand[i].bn == 192 && (I8 || glu)) continue;
    if (kTileCand[i].bm == 96 && (I8 || M > 96)) continue;  // W8A16, one block row only
    const int64_t blocks = ceil_div(M, kTileCand[i].bm) * ceil_div(N, kTileCand[i].bn);
    const double cost = (double)ceil_div(blocks, (int64_t)cus) * tile_round_cost<I8>(i);
    if (cost < best_cost * 0.999) {
      best_cost = cost;
      best = kTileCand[i];
    }
  }
  if (cost_out) *cost_out = best_cost;
  return best;
}

static int device_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
    (void)hipGetLastError();
    return 256;
  }
  return cus;
}

// One launch of tile shape `sh` over packed weight rows [n0, n0 + n) (a multiple of 32 rows in
// the gate/up layout, so it starts at a gate/up pair): the operands are offset to that range.
// glu > 0: the gate/up layout of two (glu, K) matrices, N = 2 x 16 ceil(glu / 16) packed rows.
template <bool I8>
static int launch_tiled_range(const TiledShape& sh, bool decode, const void* x, int64_t ldx,
                              const int8_t* qp, const float* s, const float* sx, uint16_t* y,
                              int64_t ldy, int32_t* acc, int64_t M, int64_t N, int64_t K,
                              int64_t glu, int64_t n0, int64_t n, hipStream_t stream) {
  const int threads = sh.bm <= 96 ? 256 : kTiledThreads;  // the 96-, 64- and 32-row tiles: 4 waves
  TiledArgs a{};
  a.x = x;
  a.ldx = ldx;
  a.qp = qp + (n0 / kTileRows) * ceil_div(K, kTileK) * kTileBytes;
  a.s = s + (glu > 0 ? n0 / 2 : n0);
  a.sx = sx;
  a.y = y ? y + (glu > 0 ? n0 / 2 : n0) : nullptr;
  a.ldy = ldy;
  a.acc = acc;  // whole-range launches only (acc rows are N long)
  a.M = (int)M;
  a.N = (int)n;
  a.K = (int)K;
  a.nsteps = (int)ceil_div(K, kTileK);
  a.nrb = (int)ceil_div(n, kTileRows);
  a.mblocks = (int)ceil_div(M, sh.bm);
  a.nblocks = (int)ceil_div(n, sh.bn);
  a.glu = glu > 0 ? (int)(glu - n0 / 2) : 0;
  a.glu_up = (int)glu;
  const int64_t blocks = (int64_t)a.mblocks * a.nblocks;
  if (blocks > 0x7fffffff) return LSE_E_RANGE;
  void* args[] = {&a};
  const bool one_row = a.mblocks == 1;
  const bool stage_y =
      glu == 0 && !decode && sh.bm == 256 && sh.bn == 256 &&
      (I8 ? !acc && blocks > (int64_t)device_cus()
          : blocks >= (int64_t)kStageYRounds * device_cus());
  const void* fn = glu > 0 ? tiled_kernel_for<I8, true>(sh, decode, one_row)
                            : tiled_kernel_for<I8, false>(sh, decode, one_row, stage_y);
  if (!fn) return LSE_E_RANGE;
  const hipError_t e =
      hipLaunchKernel(fn, dim3((unsigned)blocks), dim3(threads), args, 0, stream);
  return e == hipSuccess ? launch_status() : (int)e;
}

int launch_skinny_reduce_parts(bool i8, const void* part, const float* s, const float* sx,
                               uint16_t* y, int64_t ldy, int32_t* acc, int64_t M, int64_t N,
                               int splits, hipStream_t stream);  // skinny.hip

// K splits just above the decode range. At 65..256 tokens a narrow weight gives few tiles
// (down_proj at M = 65: 64 tiles of 64 x 128 for 256 CUs, each over all 14336 of K), so the tiled
// kernel splits K into S ranges whose raw partial sums the decode kernel's second pass adds in
// split order, as the decode route does for down_proj. S depends on the token class (65..128 or
// 129..256, priced at its largest M), N, K and the CU count only, never on M inside the class,
// so a row's bits do not depend on the batch around it. S is the larger of the count that fills
// the CUs with 64-row tiles and the count that keeps each range to at most 16 K steps (W8A16) or
// 48 (W8A8, whose steps cost half as much), capped at 8, at one 256-row block row per CU, at 8
// K steps per range and at kSplitPartBytes of partials for the class's largest M. Fitted on
// MI355X by a sweep of S (1..8) and the tile (64, 128, 256 rows) over q/k/v, o_proj and
// down_proj at 65..256 tokens: summed over those cases, 1.3 % (W8A16) and 0.8 % (W8A8) above the
// best S per class with the best tile per M, and 8 % below a rule that only fills the CUs with
// the cost model's tile. Gate/up (GLU) tiles never split.
constexpr int64_t kSplitPartBytes = 32 << 20;  // the noalloc scratch holds every call's partials

// 257..1024 tokens over a deep, narrow weight (at least 128 K steps: the MLP down projection):
// the cost model's tiles give one block per CU (or fewer), each over all of K, and such a block
// hides little of its per-step latency. Splitting K fills the CUs with 256 x 128 tiles over S
// ranges instead: S = 4 at 257..512 tokens (both modes) and S = 2 at 513..1024 (W8A16), fixed
// per class, taken when the class's largest M gives at most one round of blocks and its partials
// fit kSplitPartBytes. Measured on MI355X, down_proj (K 14336, N 4096) at M = 512: 94.6 -> 75.1 us
// (W8A16), 63.6 -> 51.0 us (W8A8); at M = 1024: 143.4 -> 132.4 us (W8A16; W8A8 gained nothing).
// The shallow projections (K 4096) measured slower with every split and tile tried.
static int tiled_deep_splits(bool i8, int64_t M, int64_t N, int64_t steps, int cus) {
  if (steps < 128 || M > (i8 ? 512 : 1024)) return 1;
  const int64_t cm = M <= 512 ? 512 : 1024;
  const int64_t splits = cm == 512 ? 4 : 2;
  if (ceil_div(cm, 256) * ceil_div(N, 128) * splits > cus) return 1;
  if (splits * cm * kTileRows * ceil_div(N, kTileRows) * 4 > kSplitPartBytes) return 1;
  return (int)splits;
}

static int tiled_splits(bool i8, int64_t M, int64_t N, int64_t K, int cus) {
  if (M <= LSE_DECODE_MAX_M) return 1;
  if (M > 256) return tiled_deep_splits(i8, M, N, ceil_div(K, kTileK), cus);
  const int64_t cm = M <= 128 ? 128 : 256;
  const int64_t nb = ceil_div(N, 128), steps = ceil_div(K, kTileK);
  int64_t splits = std::max(cus / (ceil_div(cm, 64) * nb), steps / (i8 ? 48 : 16));
  splits = std::min({splits, (int64_t)8, cus / nb, steps / 8,
                     kSplitPartBytes / (cm * kTileRows * ceil_div(N, kTileRows) * 4)});
  return (int)std::max<int64_t>(1, splits);
}

// The tile of a split launch: the smallest of 64, 128 and 256 rows whose blocks (all splits)
// fit one round on the CUs, else the cost model's. On MI355X that took down_proj at 129..256
// tokens (8 splits) from 64 x 128 tiles at two splits, 50-55 us, to one 256 x 128 block row,
// 39-47 us (W8A16).
template <bool I8>
static TiledShape split_tile(int64_t M, int64_t N, int splits, int cus) {
  const int64_t nb = ceil_div(N, 128);
  for (int bm : {64, 128, 256})
    if (ceil_div(M, (int64_t)bm) * nb * splits <= cus) return TiledShape{bm, 128};
  return tiled_shape<I8>(M, N, cus);
}

int64_t tiled_workspace_bytes(bool i8, int64_t M, int64_t N, int64_t K) {
  const int splits = tiled_splits(i8, M, N, K, device_cus());
  return splits > 1 ? (int64_t)splits * M * kTileRows * ceil_div(N, kTileRows) * 4 : 0;
}

// The cost model's tile over all N, except when a big tile's blocks leave a partial last round on
// the CUs (gate_up at M = 2048: 896 tiles of 256 x 256 for 256 CUs, 3.5 rounds) and re-tiling the
// columns of that round fills them better: then the full rounds run as one launch and the
// remaining columns, with the cost model's tile for them, as a second (gate_up at M = 2048: 768
// tiles of 256 x 256, then 256 of 128 x 256 over the last 4096 rows). Every output sums its K
// steps in increasing order whatever the tile, so the split changes no result. K splits
// (tiled_splits > 1, workspace `ws`) take precedence over it.
// `wide_decode`: the 32 x 128 or 64 x 128 tile of launch_w8a16_wide_decode instead of the cost
// model's.
template <bool I8>
static int launch_tiled(const void* x, int64_t ldx, const int8_t* qp, const float* s,
                        const float* sx, uint16_t* y, int64_t ldy, int32_t* acc, int64_t M,
                        int64_t N, int64_t K, int64_t glu, hipStream_t stream,
                        bool wide_decode = false, void* ws = nullptr, int64_t ws_bytes = 0) {
  if (glu > 0) N = 2 * kTileRows * ceil_div(glu, kTileRows);
  if (wide_decode) {
    const TiledShape sh{(I8 || M > 32) ? 64 : 32, 128};
    return launch_tiled_range<I8>(sh, true, x, ldx, qp, s, sx, y, ldy, acc, M, N, K, glu, 0, N,
                                  stream);
  }
  const int cus = device_cus();
  const int splits = glu > 0 ? 1 : tiled_splits(I8, M, N, K, cus);
  if (splits > 1) {
    if (!ws || ws_bytes < (int64_t)splits * M * kTileRows * ceil_div(N, kTileRows) * 4)
      return LSE_E_WORKSPACE;
    const TiledShape sh = split_tile<I8>(M, N, splits, cus);
    const int64_t mblocks = ceil_div(M, sh.bm);
    const int64_t blocks = mblocks * ceil_div(N, sh.bn);
    TiledArgs a{};
    a.x = x;
    a.ldx = ldx;
    a.qp = qp;
    a.s = s;
    a.sx = sx;
    a.y = y;
    a.ldy = ldy;
    a.acc = acc;
    a.M = (int)M;
    a.N = (int)N;
    a.K = (int)K;
    a.nsteps = (int)ceil_div(K, kTileK);
    a.nrb = (int)ceil_div(N, kTileRows);
    a.mblocks = (int)mblocks;
    a.nblocks = (int)ceil_div(N, sh.bn);
    a.splits = splits;
    a.ssteps = (int)ceil_div(a.nsteps, splits);
    a.part = ws;
    void* args[] = {&a};
    const hipError_t e =
        hipLaunchKernel(tiled_kernel_for<I8, false>(sh, false),
                        dim3((unsigned)(blocks * splits)),
                        dim3(sh.bm <= 64 ? 256 : kTiledThreads), args, 0, stream);
    if (e != hipSuccess) return (int)e;
    if (int st = launch_status()) return st;
    return launch_skinny_reduce_parts(I8, ws, s, sx, y, ldy, acc, M, N, splits, stream);
  }
  double cost = 0.0;
  const TiledShape sh = tiled_shape<I8>(M, N, cus, &cost, glu > 0);
  // Bulk and tail: a 256-row or 256-column tile whose blocks leave a partial last round after
  // at least one full one runs its full rounds over the first columns, and the cost model's tile
  // for the rest of N runs as a second launch; taken when some such pair is modelled at least
  // 3 % under the one launch (the cheapest pair). On MI355X: gate_up at M = 2048 (256 x 256
  // bulk, 128 x 256 tail) 467 -> 444 us; qkv at M = 4096, in place of 128 x 256 tiles, 198 ->
  // 184 us (W8A16) and 121 -> 114 us (W8A8). A 128 x 128 bulk with a 64 x 128 tail (qkv at
  // M = 1024) measured 15 % slower than the model said, so smaller bulk tiles are not tried.
  double best = 0.97 * cost;
  int64_t best_bulk = 0;
  TiledShape bulk_sh{}, tail_sh{};
  for (int i = 0; i < 3 && !acc; ++i) {
    const TiledShape c = kTileCand[i];
    const int64_t mb = ceil_div(M, c.bm);
    const int64_t blocks = mb * ceil_div(N, c.bn);
    const int64_t full = blocks / cus;  // whole rounds of candidate i
    if (full < 1 || blocks % cus == 0 || (full * cus) % mb) continue;
    const int64_t n_bulk = full * cus / mb * c.bn;
    if (n_bulk >= N) continue;
    double tail_cost = 0.0;
    const TiledShape t = tiled_shape<I8>(M, N - n_bulk, cus, &tail_cost, glu > 0);
    const double total = full * tile_round_cost<I8>(i) + tail_cost;
    if (total < best) {
      best = total;
      best_bulk = n_bulk;
      bulk_sh = c;
      tail_sh = t;
    }
  }
  if (best_bulk > 0) {
    if (int st = launch_tiled_range<I8>(bulk_sh, false, x, ldx, qp, s, sx, y, ldy, nullptr, M,
                                        N, K, glu, 0, best_bulk, stream))
      return st;
    return launch_tiled_range<I8>(tail_sh, false, x, ldx, qp, s, sx, y, ldy, nullptr, M, N, K,
                                  glu, best_bulk, N - best_bulk, stream);
  }
  return launch_tiled_range<I8>(sh, false, x, ldx, qp, s, sx, y, ldy, acc, M, N, K, glu, 0, N,
                                stream);
}

int launch_w8a16_gemm(const uint16_t* x, int64_t ldx, const int8_t* qp, const float* s,
                      uint16_t* y, int64_t ldy, int64_t M, int64_t N, int64_t K, void* ws,
                      int64_t ws_bytes, hipStream_t stream) {
  return launch_tiled<false>(x, ldx, qp, s, nullptr, y, ldy, nullptr, M, N, K, 0, stream, false,
                             ws, ws_bytes);
}

// The decode kernel's 17..32- and 33..64-token classes over a wide weight (the MLP gate/up
// projection, fused or not; chosen by the decode dispatch). Each block owns a 32 x 128 or
// 64 x 128 output tile (the class's padded token count) over the whole K, so there is no
// cross-wave reduction of K partial sums, and its four waves share one activation stage per K
// step through LDS. On MI355X, gate_up (K 4096, N 28672) takes 26 us against 31 us for the
// decode kernel at 32 tokens, and 33 us against 41 us at 64. Every output is the K steps summed
// in increasing order, as for every tile shape, so rows do not depend on M or on the other rows.
int launch_w8a16_wide_decode(const uint16_t* x, int64_t ldx, const int8_t* qp, const float* s,
                             uint16_t* y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                             int64_t glu, hipStream_t stream) {
  return launch_tiled<false>(x, ldx, qp, s, nullptr, y, ldy, nullptr, M, glu > 0 ? 0 : N, K, glu,
                             stream, true);
}

// bf16 weights (the lm_head kept in bf16, in the layout of lse_pack_bf16_weight) where the decode
// kernel would reduce many partial tiles (17..64 tokens over a wide weight) or cannot run (more
// than 64 tokens): one block row of BM x 128 tiles up to 256 tokens (BM = 32, 64, 128 or 256, the
// smallest that holds M; four waves of BM x 32 up to 64, eight waves of 64 x 32 above), then
// 256 x 128 tiles over ceil(M / 256) block rows. No scales, y = bf16(sum). With one block row
// the weights stream with the nt policy; beyond, the block rows share them through L2. Every
// output sums its K steps in increasing order, two MFMAs per step, whatever the tile, so a row's
// bits depend on N and K only (not on M or on other rows). On MI355X over the Llama-3 lm_head
// (N 128256, K 4096) at 64 tokens: 191 us against 236 us for the decode kernel.
int launch_bf16_tiled(const uint16_t* x, int64_t ldx, const uint16_t* wp, uint16_t* y,
                      int64_t ldy, int64_t M, int64_t N, int64_t K, hipStream_t stream) {
  const int bm = M <= 32 ? 32 : M <= 64 ? 64 : M <= 128 ? 128 : 256;
  TiledArgs a{};
  a.x = x;
  a.ldx = ldx;
  a.qp = reinterpret_cast<const int8_t*>(wp);
  a.y = y;
  a.ldy = ldy;
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.nsteps = (int)ceil_div(K, kTileK);
  a.nrb = (int)ceil_div(N, kTileRows);
  a.mblocks = (int)ceil_div(M, bm);
  a.nblocks = (int)ceil_div(N, 128);
  const int64_t blocks = (int64_t)a.mblocks * a.nblocks;
  if (blocks > 0x7fffffff) return LSE_E_RANGE;
  const void* fn;
  switch (bm) {
    case 32: fn = reinterpret_cast<const void*>(
                 &tiled_gemm_kernel<false, 32, 128, 1, 4, 4, false, true, true>);
             break;
    case 64: fn = reinterpret_cast<const void*>(
                 &tiled_gemm_kernel<false, 64, 128, 1, 4, 4, false, true, true>);
             break;
    case 128: fn = reinterpret_cast<const void*>(
                  &tiled_gemm_kernel<false, 128, 128, 2, 4, 3, false, true, true>);
              break;
    default: fn = a.mblocks == 1 ? reinterpret_cast<const void*>(
                                       &tiled_gemm_kernel<false, 256, 128, 2, 4, 3, false, true, true>)
                                 : reinterpret_cast<const void*>(
                                       &tiled_gemm_kernel<false, 256, 128, 2, 4, 3, false, false, true>);
  }
  void* args[] = {&a};
  const hipError_t e =
      hipLaunchKernel(fn, dim3((unsigned)blocks), dim3(bm <= 64 ? 256 : 512), args, 0, stream);
  return e == hipSuccess ? launch_status() : (int)e;
}

// The decode kernel's deep, narrow class at 17..64 tokens (at most 256 row tiles and at least 128
// K steps: the MLP down projection; chosen by the decode dispatch). Tiles of the tiled kernel
// over one of 8 K ranges per block fill the CUs (8 x 32 blocks for down_proj) without the decode
// kernel's cross-wave reduction; the raw partial sums are added in split order by the decode
// kernel's second pass. W8A16: 32 x 128 or 64 x 128 tiles (class 17..32 or 33..64); on MI355X
// down_proj (K 14336, N 4096) takes 18.7 us against 21.3 us at 32 tokens and 21.5 us against
// 25.7 us at 64. W8A8: 64 x 128 tiles (int32 partials: exact, any order).
constexpr int kDeepSplits = 8;

int64_t deep_decode_part_bytes(int64_t M, int64_t N) {
  return (int64_t)kDeepSplits * M * kTileRows * ceil_div(N, kTileRows) * 4;
}

template <bool I8>
static int launch_deep_decode(const void* x, int64_t ldx, const int8_t* qp, const float* s,
                              const float* sx, uint16_t* y, int64_t ldy, int32_t* acc, int64_t M,
                              int64_t N, int64_t K, void* ws, int64_t ws_bytes,
                              hipStream_t stream) {
  if (!ws || ws_bytes < deep_decode_part_bytes(M, N)) return LSE_E_WORKSPACE;
  const TiledShape sh{(I8 || M > 32) ? 64 : 32, 128};
  TiledArgs a{};
  a.x = x;
  a.ldx = ldx;
  a.qp = qp;
  a.s = s;
  a.sx = sx;
  a.y = y;
  a.ldy = ldy;
  a.acc = acc;
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.nsteps = (int)ceil_div(K, kTileK);
  a.nrb = (int)ceil_div(N, kTileRows);
  a.mblocks = (int)ceil_div(M, sh.bm);
  a.nblocks = (int)ceil_div(N, sh.bn);
  a.splits = kDeepSplits;
  a.ssteps = (int)ceil_div(a.nsteps, kDeepSplits);
  a.part = ws;
  void* args[] = {&a};
  const hipError_t e =
      hipLaunchKernel(tiled_kernel_for<I8, false>(sh, I8 || sh.bm == 32),
                      dim3((unsigned)(a.mblocks * a.nblocks * kDeepSplits)), dim3(256), args, 0,
                      stream);
  if (e != hipSuccess) return (int)e;
  if (int st = launch_status()) return st;
  return launch_skinny_reduce_parts(I8, ws, s, sx, y, ldy, acc, M, N, kDeepSplits, stream);
}

int launch_w8a16_deep_decode(const uint16_t* x, int64_t ldx, const int8_t* qp, const float* s,
                             uint16_t* y, int64_t ldy, int64_t M, int64_t N, int64_t K, void* ws,
                             int64_t ws_bytes, hipStream_t stream) {
  return launch_deep_decode<false>(x, ldx, qp, s, nullptr, y, ldy, nullptr, M, N, K, ws,
                                   ws_bytes, stream);
}

int launch_w8a8_deep_decode(const int8_t* xq, const float* sx, const int8_t* qp, const float* s,
                            uint16_t* y, int64_t ldy, int32_t* acc, int64_t M, int64_t N,
                            int64_t K, void* ws, int64_t ws_bytes, hipStream_t stream) {
  return launch_deep_decode<true>(xq, K, qp, s, sx, y, ldy, acc, M, N, K, ws, ws_bytes, stream);
}

// W8A8 counterpart of launch_w8a16_wide_decode (17..64 tokens over a wide weight, plain or
// gate/up): 64 x 128 int8 tiles over the whole K.
int launch_w8a8_wide_decode(const int8_t* xq, const float* sx, const int8_t* qp, const float* s,
                            uint16_t* y, int64_t ldy, int32_t* acc, int64_t M, int64_t N,
                            int64_t K, int64_t glu, hipStream_t stream) {
  return launch_tiled<true>(xq, K, qp, s, sx, y, ldy, acc, M, glu > 0 ? 0 : N, K, glu, stream,
                            true);
}

int launch_w8a8_gemm(const int8_t* xq, const float* sx, const int8_t* qp, const float* s,
                     uint16_t* y, int64_t ldy, int32_t* acc, int64_t M, int64_t N, int64_t K,
                     void* ws, int64_t ws_bytes, hipStream_t stream) {
  return launch_tiled<true>(xq, K, qp, s, sx, y, ldy, acc, M, N, K, 0, stream, false, ws,
                            ws_bytes);
}

int launch_w8a16_gemm_glu(const uint16_t* x, int64_t ldx, const int8_t* qp, const float* s,
                          uint16_t* h, int64_t ldh, int64_t M, int64_t I, int64_t K,
                          hipStream_t stream) {
  return launch_tiled<false>(x, ldx, qp, s, nullptr, h, ldh, nullptr, M, 0, K, I, stream);
}

int launch_w8a8_gemm_glu(const int8_t* xq, const float* sx, const int8_t* qp, const float* s,
                         uint16_t* h, int64_t ldh, int64_t M, int64_t I, int64_t K,
                         hipStream_t stream) {
  return launch_tiled<true>(xq, K, qp, s, sx, h, ldh, nullptr, M, 0, K, I, stream);
}

}  // namespace lse
