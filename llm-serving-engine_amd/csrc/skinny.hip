// Skinny int8-weight GEMM for the decode range (M <= 64), both modes of the int8 Linear:
//   W8A16: y[m,n] = bf16(s[n] * sum_k x[m,k] q[n,k])               bf16 x, fp32 accumulation
//   W8A8:  acc[m,n] = sum_k xq[m,k] q[n,k] exactly in int32;  y = bf16((acc * sx[m]) * s[n])
//
// The kernel is a weight stream: every weight byte is read once from HBM, in packed tiles
// (lse_common.h) so that each 128-bit load of a wave is one contiguous 1 KB tile, with the
// streaming (nt) cache policy so the stream does not evict the activations and scales.
//
// Work decomposition.
//  * A panel is RT row tiles (16 * RT weight rows). The K steps split into S ranges of `ssteps`
//    steps; a work unit is (split, panel), numbered split-major. Each workgroup takes a
//    contiguous range of whole units (split as evenly as whole units allow, or, on a paired grid,
//    each CU's share split between the two workgroups it holds) and streams them one after
//    another.
//  * Within a unit the W waves split the unit's 64-wide K steps round-robin (wave w takes steps
//    w, w + W, ...; a "super-step" is one step of every wave). A wave multiplies each activation
//    fragment against all RT row tiles of the panel, so activations are read 2M/(16 RT) times
//    per weight byte: wide panels keep that traffic (from L2) below the weight stream (from
//    HBM), and splitting K keeps enough units to fill every CU when panels are wide. At the end
//    of a unit the waves' partial sums are added through LDS in wave order; with S = 1 they are
//    scaled and stored, with S > 1 stored raw to a workspace that skinny_reduce adds over the
//    splits in split order before the same epilogue.
//  * Every summation order depends only on (N, K, the token class of M, the grid), never on M
//    inside a class or on other rows: results are deterministic and a row's output is the same
//    inside any batch of its class. No atomics.
//  * Fused gate/up (GLU): the weight is in the gate/up layout (lse_common.h) and panels hold an
//    even number of row tiles, so every panel holds matching gate and up rows; the final
//    reduction adds slice pairs (gate tile, up tile) in one wave, which writes
//    h = bf16(silu(g) * u) for its I output columns. No K splits.
//  * 17..64 tokens over a wide weight (at least 1024 row tiles, the MLP gate/up) do not run here:
//    the decode dispatch sends them to 32 x 128 or 64 x 128 tiles of the tiled kernel
//    (skinny_wide_tiled); nor over a deep, narrow one (the split-K class, down_proj), which runs
//    as 8 K ranges of such tiles whose partials skinny_reduce adds (skinny_deep_tiled).
//  * bf16 weights (BFW, the lm_head kept in bf16): each 64-wide K step of a row tile is two
//    1 KB tiles already in bf16 operand form (the "lo" and "hi" halves that dequantization
//    produces from an int8 tile, layout in lse_common.h), loaded instead of dequantized; no
//    scales, y = bf16(sum).
//
// Activations reach the MFMAs from LDS, never by gathering 16 token rows per load from global
// memory (that pattern runs at a fraction of the cache bandwidth):
//  * staged whole (XLDS): all M x K activations are copied to LDS once per workgroup with
//    row-contiguous direct-to-LDS loads, when they fit, rows zero-padded to whole K steps and
//    16-byte chunks XOR-swizzled by token so fragment reads are conflict-free;
//  * otherwise streamed through a ring of DX LDS slots per wave: each wave copies the 16 MT token
//    rows x 64 K-columns of its own next steps with row-contiguous direct-to-LDS loads that run
//    DX-1 steps ahead of its MFMAs, so no other wave is involved and no barrier is needed.
//
// Pipelining. Loads are range-checked buffer loads: rows past N, K past the end, tokens past M
// and steps past the workgroup's range read zeros without a memory request, so every step issues
// the same loads, and a ring of DW register stages keeps DW-1 steps of weights in flight behind
// static wait counts. The scales (and staged activations) go to LDS while the ring's first loads
// are in flight.
#include <algorithm>
#include <type_traits>

#include "lse_common.h"

namespace lse {

constexpr int kSkinnyScaleLds = 2048;         // scales staged per workgroup (floats)
constexpr int kSkinnyXLdsBytes = 128 * 1024;  // activations staged whole up to this size

struct SkinnyArgs {
  const void* x;        // W8A16: bf16 (M rows, stride ldx); W8A8: int8 xq (M rows, stride ldx)
  int64_t ldx;          // elements
  const int8_t* qp;     // packed weight tiles
  const float* s;       // (N) per-channel scales
  const float* sx;      // (M) per-token scales, W8A8 only
  uint16_t* y;          // (M, N) bf16, stride ldy; may be null in W8A8
  int64_t ldy;
  int32_t* acc;         // (M, N) int32 contiguous, W8A8 only; may be null
  int M, N, K;
  int nsteps;           // ceil(K / 64)
  int nrb;              // ceil(N / 16)
  int panels;           // ceil(nrb / RT)
  int splits;           // S, ranges the K steps split into
  int ssteps;           // steps per range: ceil(nsteps / S)
  int units;            // panels * splits
  int NSU;              // super-steps per unit: ceil(ssteps / W) rounded up to a multiple of DW
  void* part;           // S > 1: raw partial sums [S][M][16 nrb], fp32 (W8A16) or int32 (W8A8)
  int glu;              // gate/up layout: I, the output columns (N = 16 nrb packed rows); else 0
  int pairs;            // > 0: workgroups i and i + pairs share a CU and split its units
};

// Register stage of the weight ring: one 1 KB tile per row tile of the panel.
template <int RT, int WN>
struct SkinnyWStage {
  uint4 w[RT * WN];  // WN 1 KB tiles per row tile: 1 (int8) or 2 (bf16 lo, hi)
};

// XOR swizzle of a streamed activation step image (16 MT token rows of XROW = 64 ESZ bytes,
// 16-byte chunks): chunk c of row m sits at c ^ xstep_swz(m). A fragment read takes one logical
// chunk of 16 consecutive rows; rows are 128 (bf16) or 64 (int8) bytes. Measured on MI355X with
// SQ_LDS_BANK_CONFLICT, these swizzles read with no conflict (the same ones as the tiled
// kernel's): bf16 (m & 7) ^ ((m >> 3) & 1), int8 (m >> 1) & 3.
template <int ESZ>
__host__ __device__ constexpr int xstep_swz(int m) {
  return ESZ == 2 ? (m & 7) ^ ((m >> 3) & 1) : (m >> 1) & 3;
}

// Bytes of one whole-staged activation row: K rounded up to whole 64-wide steps.
__host__ __device__ constexpr int skinny_x_row(int K, int esz) { return ((K + 63) / 64) * 64 * esz; }

// XOR swizzle of a staged row's 16-byte chunks: chunk c of token row m sits at c ^ swz(m), with
// swz(m) below the largest power of two (at most 16) dividing the chunks per row, so the
// swizzle stays inside the row and 16 consecutive rows read at one K offset spread over banks.
__host__ __device__ constexpr int skinny_swz_mask(int chunks_per_row) {
  return ((chunks_per_row & -chunks_per_row) < 16 ? (chunks_per_row & -chunks_per_row) : 16) - 1;
}

template <bool I8, int MT, int RT, int W, int DW, int DX, bool XLDS, bool GLU, bool BFW = false,
          bool QX = false, bool PAIR = false>
__global__ void __launch_bounds__(64 * W)
skinny_kernel(SkinnyArgs a) {
  using Acc = std::conditional_t<I8, i32x4, f32x4>;
  static_assert(!BFW || (!I8 && !GLU), "bf16 weights: plain W16A16 only");
  // QX: x is bf16 and the kernel quantizes it per token while staging it (W8A8 in one launch).
  static_assert(!QX || (I8 && XLDS && MT == 1 && !GLU && !BFW), "quantizing staging: W8A8, M <= 16");
  constexpr int WN = BFW ? 2 : 1;  // 1 KB weight tiles per row tile and step
  constexpr int SLICES = RT * MT;               // 16x16 output tiles of a panel
  constexpr int ESZ = I8 ? 1 : 2;               // activation element bytes
  constexpr int XL = I8 ? 1 : 2;                // 16-byte activation pieces per token tile and step
  // A single accumulator chain in W8A16 splits into two (one per dequantized half), so the two
  // MFMAs of a step do not wait on each other.
  constexpr int NACC = (!I8 && SLICES == 1) ? 2 : 1;
  static_assert(!XLDS || MT == 1, "activations are staged whole for one token tile only");
  static_assert(DW % DX == 0, "the activation ring index must repeat with the weight ring's");
  static_assert(!GLU || RT % 2 == 0, "gate/up panels hold whole pairs of row tiles");
  // Streamed activations: a wave's ring slot holds the 16 MT token rows x 64 K-columns of one of
  // its steps, row-major (XROW bytes a row), 16-byte chunks XOR-swizzled by token (chunk c of row
  // m sits at c ^ xstep_swz(m)); the wave fills it with XI pieces of 1 KB.
  constexpr int XROW = 64 * ESZ;                // bytes of one token row of a step
  constexpr int XI = XLDS ? 0 : MT * ESZ;       // 1 KB pieces per wave per step
  constexpr int kWaitX = (DX - 1) * (RT * WN + XI);  // loads issued after a step's activations
  static_assert(XLDS || kWaitX < 64, "vmcnt holds at most 63");
  // Each ring slot (all waves' parts) is its own array, so the compiler can tell the slot a
  // direct-to-LDS load fills from the slot the MFMAs read, and leaves those waits to the explicit
  // s_waitcnt.
  constexpr int XWAVE = 16 * MT * XROW / 16;    // uint4 per wave per slot
  constexpr int XSLOT = XLDS ? 1 : W * XWAVE;
  // Slices reduced per pass through LDS: all W waves' partials of RS slices (1 KB each) at once,
  // as many as the LDS left by the activation ring and the scales holds (whole gate/up pairs).
  constexpr int kRedBudget = 160 * 1024 - DX * XSLOT * 16 - kSkinnyScaleLds * 4;
  constexpr int RS0 = W < SLICES ? W : SLICES;
  constexpr int RS1 = RS0 * W * 1024 <= kRedBudget ? RS0 : kRedBudget / (W * 1024);
  constexpr int RS = GLU ? RS1 & ~1 : RS1;
  static_assert(RS >= (GLU ? 2 : 1), "no LDS left for the cross-wave reduction");

  __shared__ Acc red[W][RS][64];
  __shared__ float s_lds[kSkinnyScaleLds];
  __shared__ unsigned qx_amax[QX ? 16 : 1];  // QX: each token row's max |x|, as float bits
  __shared__ uint4 xs0[XSLOT], xs1[DX > 1 ? XSLOT : 1], xs2[DX > 2 ? XSLOT : 1],
      xs3[DX > 3 ? XSLOT : 1];
  static_assert(XLDS || DX <= 4, "at most four activation slots");
  extern __shared__ __attribute__((aligned(16))) unsigned char x_lds[];  // XLDS
  auto xslot = [&](int i) -> uint4* {
    switch (i) {
      case 0: return xs0;
      case 1: return xs1;
      case 2: return xs2;
      default: return xs3;
    }
  };

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: scalar math
  const int r16 = lane & 15;
  const int g = lane >> 4;
  const int G = gridDim.x;
  // Units [u_first, u_end) of this workgroup: an even spread of whole units over the grid, or
  // (PAIR, a grid of exactly 2 a.pairs workgroups, two resident per CU) one over a.pairs CU slots:
  // the dispatcher gives every CU its first workgroup before any CU its second, so workgroups i
  // and i + a.pairs share a CU and split that CU's units, the first taking the larger half.
  const bool second = PAIR && (int)blockIdx.x >= a.pairs;
  const unsigned slot = second ? blockIdx.x - (unsigned)a.pairs : blockIdx.x;
  const unsigned nslots = PAIR ? (unsigned)a.pairs : (unsigned)G;
  const int s0 = slot * a.units / nslots, s1 = (slot + 1) * a.units / nslots;
  const int smid = s0 + ((s1 - s0 + 1) >> 1);
  const int u_first = second ? smid : s0;
  const int u_end = PAIR && !second ? smid : s1;
  const bool split = a.splits > 1;

  const BufferRsrc qres =
      make_rsrc(a.qp, (uint32_t)a.nrb * (uint32_t)a.nsteps * (uint32_t)(kTileBytes * WN));
  const BufferRsrc xres = make_rsrc(a.x, (uint32_t)(((int64_t)(a.M - 1) * a.ldx + a.K) * ESZ));
  float sxv[MT];
#pragma unroll
  for (int b = 0; b < MT; ++b) {
    const int m = 16 * b + r16;
    sxv[b] = (I8 && !QX && m < a.M) ? a.sx[m] : 0.0f;  // QX: set while staging
  }

  // Staged inputs, issued before the weight ring: with S = 1 (units are panels) the scales of
  // rows [16 RT u_first, 16 RT u_end) (through registers), and with XLDS all activations, copied straight to LDS: piece i of the
  // image is bytes [1024 i, 1024 i + 1024), lane l fills byte 1024 i + 16 l, which is physical
  // chunk pc of row m and holds logical chunk pc ^ swz(m); tokens past M and K past the end read
  // zeros, so the image needs no bounds checks when read.
  // Scales are staged per packed row: in the gate/up layout packed row 16 rb + r is gate
  // (rb even) or up (rb odd) row 16 (rb / 2) + r, whose scale is s[(rb & 1) I + 16 (rb / 2) + r].
  const int srow0 = 16 * RT * u_first;
  const int nsc = split || BFW ? 0 : min(16 * RT * u_end, a.N) - srow0;
  constexpr int kScPerThread = (kSkinnyScaleLds + 64 * W - 1) / (64 * W);
  float sc_stage[kScPerThread];
#pragma unroll
  for (int i = 0; i < kScPerThread; ++i) {
    const int r = threadIdx.x + 64 * W * i;
    int src = srow0 + r;
    bool valid = r < nsc;
    if constexpr (GLU) {
      const int rb = src >> 4, o = 16 * (rb >> 1) + (src & 15);
      valid = valid && o < a.glu;
      src = (rb & 1) * a.glu + o;
    }
    sc_stage[i] = valid ? a.s[src] : 0.0f;
  }
  const int xrow_bytes = skinny_x_row(a.K, ESZ);
  const int xswz = skinny_swz_mask(xrow_bytes / 16);
  if constexpr (XLDS && !QX) {
    const int total = (a.M * xrow_bytes + 1023) / 1024;
    for (int piece = wave; piece < total; piece += W) {
      const int o = 1024 * piece + 16 * lane;
      const int m = o / xrow_bytes, pc = (o % xrow_bytes) / 16;
      const int kb = 16 * (pc ^ (m & xswz));
      const uint32_t off =
          m < a.M && kb < a.K * ESZ ? (uint32_t)((int64_t)m * a.ldx * ESZ + kb) : kOutOfRange;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          xres, (__attribute__((address_space(3))) void*)(x_lds + 1024 * piece), 16, off, 0, 0, 0);
    }
  }
  // Scales to LDS, and (XLDS) every wave's activation pieces landed; the weight ring's prologue
  // loads, issued after, stay in flight.
  auto store_staged = [&]() {
#pragma unroll
    for (int i = 0; i < kScPerThread; ++i) {
      const int r = threadIdx.x + 64 * W * i;
      if (r < kSkinnyScaleLds) s_lds[r] = sc_stage[i];
    }
    if constexpr (XLDS && !QX) __builtin_amdgcn_s_waitcnt(vmcnt_imm((DW - 1) * RT * WN));
    if constexpr (QX) {
      // Per-token quantization of the bf16 rows into the staged int8 image, bit for bit what
      // quantize_act_rows computes: each row's max |x| (an LDS atomic max on the float bits,
      // which order like the values since they are >= 0), then every element quantized with the
      // row's scale (with_row_quantizer: quant1's results), written at its swizzled position (chunk pc of row m holds logical chunk
      // pc ^ (m & xswz); K is a multiple of 16, so a 16-element chunk is wholly in or out).
      // Work item c is physical chunk c of the staged image (16 int8 of row c / rch), i.e. 16
      // bf16 of x (logical chunk pc ^ (m & xswz), zeros past K). A thread keeps its first QR
      // items' x in registers between the amax pass and the quantizing pass, so x is read
      // from memory once when it fits (M x K up to 16 x 512 x QR elements).
      if (threadIdx.x < 16) qx_amax[threadIdx.x] = 0u;
      __syncthreads();
      const uint16_t* xb = static_cast<const uint16_t*>(a.x);
      const int rch = xrow_bytes / 16;  // 16-byte chunks per staged row
      const int items = a.M * rch;
      auto load_item = [&](int c, uint4& v0, uint4& v1) {
        const int m = c / rch, pc = c - m * rch;
        const int k16 = 16 * (pc ^ (m & xswz));
        v0 = v1 = make_uint4(0, 0, 0, 0);
        if (k16 < a.K) {
          const uint16_t* src = xb + (int64_t)m * a.ldx + k16;
          v0 = *reinterpret_cast<const uint4*>(src);
          v1 = *reinterpret_cast<const uint4*>(src + 8);
        }
      };
      auto amax_item = [&](int c, const uint4& v0, const uint4& v1) {
        const uint32_t w8[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
        float mx = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          mx = fmaxf(mx, fabsf(__builtin_bit_cast(float, w8[j] << 16)));
          mx = fmaxf(mx, fabsf(__builtin_bit_cast(float, w8[j] & 0xffff0000u)));
        }
        atomicMax(&qx_amax[c / rch], __builtin_bit_cast(unsigned, mx));
      };
      auto quant_item = [&](int c, const uint4& v0, const uint4& v1) {
        const float scale = row_scale(__builtin_bit_cast(float, qx_amax[c / rch]));
        const uint32_t w8[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
        with_row_quantizer(scale, [&](auto q) {
          uint32_t packed[4] = {0, 0, 0, 0};
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const uint32_t lo = (uint8_t)q(__builtin_bit_cast(float, w8[j] << 16));
            const uint32_t hi = (uint8_t)q(__builtin_bit_cast(float, w8[j] & 0xffff0000u));
            packed[j >> 1] |= (lo | (hi << 8)) << (16 * (j & 1));
          }
          *reinterpret_cast<uint4*>(x_lds + 16 * c) =
              make_uint4(packed[0], packed[1], packed[2], packed[3]);
        });
      };
      constexpr int QR = 2;
      uint4 kv0[QR], kv1[QR];
#pragma unroll
      for (int it = 0; it < QR; ++it) {
        const int c = threadIdx.x + 64 * W * it;
        if (c < items) {
          load_item(c, kv0[it], kv1[it]);
          amax_item(c, kv0[it], kv1[it]);
        }
      }
      for (int c = threadIdx.x + 64 * W * QR; c < items; c += 64 * W) {
        uint4 v0, v1;
        load_item(c, v0, v1);
        amax_item(c, v0, v1);
      }
      __syncthreads();
#pragma unroll
      for (int it = 0; it < QR; ++it) {
        const int c = threadIdx.x + 64 * W * it;
        if (c < items) quant_item(c, kv0[it], kv1[it]);
      }
      for (int c = threadIdx.x + 64 * W * QR; c < items; c += 64 * W) {
        uint4 v0, v1;
        load_item(c, v0, v1);
        quant_item(c, v0, v1);
      }
      sxv[0] = r16 < a.M ? row_scale(__builtin_bit_cast(float, qx_amax[r16])) : 0.0f;
    }
    __syncthreads();
  };

  // Weight load cursor: unit lu (panel lp of split lsp), super-step lsu within it.
  int lu = u_first, lp = u_first % a.panels, lsp = u_first / a.panels, lsu = 0;
  auto load_w = [&](SkinnyWStage<RT, WN>& st) {
    const int jr = W * lsu + wave;
    const int j = lsp * a.ssteps + jr;
    const bool kv = lu < u_end && jr < a.ssteps && j < a.nsteps;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int rb = lp * RT + rt;
      const uint32_t off =
          ((uint32_t)rb * (uint32_t)a.nsteps + (uint32_t)j) * (kTileBytes * WN) + 16u * lane;
#pragma unroll
      for (int h = 0; h < WN; ++h)
        st.w[WN * rt + h] =
            buffer_load16<kLoadStream>(qres, kv && rb < a.nrb ? off + kTileBytes * h : kOutOfRange);
    }
    if (++lsu == a.NSU) {
      lsu = 0;
      ++lu;
      if (++lp == a.panels) {
        lp = 0;
        ++lsp;
      }
    }
  };
  // Activation load cursor (activations depend on the step only, not on the panel). Piece i of
  // this wave's part of a slot covers bytes [1024 i, 1024 i + 1024): lane l fills byte
  // 1024 i + 16 l, physical chunk pc of token row m, which holds logical chunk pc ^ xstep_swz(m).
  // Tokens past M, K past the end and steps past the range read zeros.
  int xu = u_first, xp = u_first % a.panels, xsp = u_first / a.panels, xsu = 0;
  auto load_x = [&](int slot) {
    const int jr = W * xsu + wave;
    const int j = xsp * a.ssteps + jr;
    const bool live = xu < u_end && jr < a.ssteps && j < a.nsteps;
#pragma unroll
    for (int i = 0; i < XI; ++i) {
      const int o = 1024 * i + 16 * lane;
      const int m = o / XROW, pc = (o % XROW) / 16;
      const int kb = XROW * j + 16 * (pc ^ xstep_swz<ESZ>(m));
      const uint32_t off = live && m < a.M && kb < a.K * ESZ
                               ? (uint32_t)((int64_t)m * a.ldx * ESZ + kb)
                               : kOutOfRange;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          xres,
          (__attribute__((address_space(3))) void*)(xslot(slot) + wave * XWAVE + 64 * i), 16, off,
          0, 0, 0);
    }
    if (++xsu == a.NSU) {
      xsu = 0;
      ++xu;
      if (++xp == a.panels) {
        xp = 0;
        ++xsp;
      }
    }
  };

  Acc acc[RT][MT][NACC];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int b = 0; b < MT; ++b)
#pragma unroll
      for (int c = 0; c < NACC; ++c) acc[rt][b][c] = Acc{0, 0, 0, 0};

  // One step: the wave's K step of super-step su of a unit of split sp, from weight stage st and
  // ring slot `slot`.
  // XLDS: this lane's token row (tokens past M re-read row M-1; their outputs are dropped).
  const int x_m = min(r16, a.M - 1);
  const unsigned char* x_row_base = x_lds + x_m * xrow_bytes;
  const int x_swz = x_m & xswz;
  auto compute = [&](const SkinnyWStage<RT, WN>& st, int slot, int sp, int su) {
    uint4 xv[MT][XL];
    if constexpr (XLDS) {
      // A padding step past the unit's range or the last K step (NSU is rounded up to the ring
      // depth) re-reads step 0; its weights are zero.
      const int jr = W * su + wave;
      const int j = sp * a.ssteps + jr;
      const int c0 = (jr < a.ssteps && j < a.nsteps ? j : 0) * 4 * ESZ + XL * g;
#pragma unroll
      for (int h = 0; h < XL; ++h)
        xv[0][h] = *reinterpret_cast<const uint4*>(x_row_base + 16 * ((c0 + h) ^ x_swz));
    } else {
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(kWaitX));  // this step's pieces landed
      const unsigned char* base =
          reinterpret_cast<const unsigned char*>(xslot(slot) + wave * XWAVE);
#pragma unroll
      for (int b = 0; b < MT; ++b) {
        const int m = min(16 * b + r16, a.M - 1);  // tokens past M re-read row M-1
#pragma unroll
        for (int h = 0; h < XL; ++h) {
          // Lane group g takes 16 consecutive K elements of the step: XL chunks of 16 bytes.
          const int c = XL * g + h;
          xv[b][h] = *reinterpret_cast<const uint4*>(base + m * XROW + 16 * (c ^ xstep_swz<ESZ>(m)));
        }
      }
    }
    if constexpr (I8) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int b = 0; b < MT; ++b) acc[rt][b][0] = mfma_i8(st.w[rt], xv[b][0], acc[rt][b][0]);
    } else {
      bf16x8 lo[RT], hi[RT];
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        if constexpr (BFW) {
          lo[rt] = as_bf16x8(st.w[2 * rt]);
          hi[rt] = as_bf16x8(st.w[2 * rt + 1]);
        } else {
          dequant16(st.w[rt], lo[rt], hi[rt]);
        }
      }
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int b = 0; b < MT; ++b)
          acc[rt][b][0] = mfma16x16x32(lo[rt], as_bf16x8(xv[b][0]), acc[rt][b][0]);
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int b = 0; b < MT; ++b)
          acc[rt][b][NACC - 1] = mfma16x16x32(hi[rt], as_bf16x8(xv[b][1]), acc[rt][b][NACC - 1]);
    }
  };

  // One lane's four outputs of a unit: rows n..n+3 of token m of slice `slice` of panel p.
  // S = 1: scaled and stored; S > 1: raw, to split sp's part of the workspace (rows padded to
  // 16 nrb, so every tile stores whole).
  const bool yvec = a.y && (a.ldy & 3) == 0 && ((uintptr_t)a.y & 7) == 0;
  auto store_out = [&](int p, int sp, int slice, Acc v) {
    const int rt = slice % RT, b = slice / RT;
    const int m = 16 * b + r16;
    const int rb = p * RT + rt;
    const int n = 16 * rb + 4 * g;
    if (split) {
      if (m < a.M && rb < a.nrb)
        *reinterpret_cast<Acc*>(static_cast<char*>(a.part) +
                                (((int64_t)sp * a.M + m) * (16 * a.nrb) + n) * 4) = v;
      return;
    }
    if (m >= a.M || n >= a.N) return;
    const int cnt = min(4, a.N - n);
    float sc[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) sc[r] = BFW ? 1.0f : r < cnt ? s_lds[n + r - srow0] : 0.0f;
    store_out4<I8>(a.y, a.ldy, a.acc, a.N, m, n, cnt, v, sc, sxv[b], yvec);
  };
  // Gate/up: slice `slice` (an even row tile rt of token tile b) holds gate rows of output
  // columns 16 (rb / 2) + 4 g + r, slice + 1 the up rows of the same columns.
  auto store_glu = [&](int p, int slice, Acc vg, Acc vu) {
    const int rt = slice % RT, b = slice / RT;
    const int m = 16 * b + r16;
    const int rb = p * RT + rt;
    const int n = 16 * (rb >> 1) + 4 * g;
    if (m >= a.M || n >= a.glu) return;
    const int cnt = min(4, a.glu - n);
    const int pr = 16 * rb + 4 * g - srow0;  // packed row of the first gate output
    float sg[4], su[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      sg[r] = r < cnt ? s_lds[pr + r] : 0.0f;
      su[r] = r < cnt ? s_lds[pr + 16 + r] : 0.0f;
    }
    store_glu4<I8>(a.y, a.ldy, m, n, cnt, vg, vu, sg, su, sxv[b], yvec);
  };

  // Storage of the partial sums of a reduction pass: wave w's 1 KB of pass slice sl (all lanes'
  // Acc) at slice_ptr(sl, w). Slices below RS live in `red`. In a workgroup's last unit the
  // activation ring is idle (its remaining loads move no data), so slices from RS on take each
  // wave's part of the ring slots, CPS per slot: one or two passes instead of up to eight.
  constexpr int CPS = XLDS ? 0 : XWAVE / 64;
  constexpr int RSW0 = RS + DX * CPS;
  constexpr int RSW = GLU ? RSW0 & ~1 : RSW0;
  auto slice_ptr = [&](int sl, int w) -> Acc* {
    if (sl < RS) return &red[w][sl][0];
    constexpr int cps = CPS > 0 ? CPS : 1;
    const int j = (sl - RS) / cps, c = (sl - RS) % cps;
    return reinterpret_cast<Acc*>(xslot(j) + w * XWAVE + 64 * c);
  };

  // End of a unit (panel p of split sp), with CAP slices of storage per pass: pass i adds slices
  // [i CAP, i CAP + CAP) over the waves in wave order (the order does not depend on CAP); wave w
  // keeps slices i CAP + w, i CAP + w + W, ... and stores them (gate/up: the pairs 2 w, 2 w + 1,
  // 2 (w + W), ... of the pass).
  auto unit_end = [&](int p, int sp, auto cap) {
    constexpr int CAP = decltype(cap)::value;
    constexpr int NP = (SLICES + CAP - 1) / CAP;
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      __syncthreads();  // the previous pass's (or unit's) reads of the storage are done
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int b = 0; b < MT; ++b) {
          const int sl = rt + RT * b - CAP * i;
          if (sl < 0 || sl >= CAP) continue;
          Acc v = acc[rt][b][0];
          if constexpr (NACC == 2) v += acc[rt][b][1];
          slice_ptr(sl, wave)[lane] = v;
        }
      __syncthreads();
      if constexpr (GLU) {
        for (int sl = 2 * wave; sl < CAP && sl + CAP * i < SLICES; sl += 2 * W) {
          Acc vg = slice_ptr(sl, 0)[lane], vu = slice_ptr(sl + 1, 0)[lane];
#pragma unroll
          for (int w2 = 1; w2 < W; ++w2) {
            vg += slice_ptr(sl, w2)[lane];
            vu += slice_ptr(sl + 1, w2)[lane];
          }
          store_glu(p, sl + CAP * i, vg, vu);
        }
      } else {
        for (int sl = wave; sl < CAP && sl + CAP * i < SLICES; sl += W) {
          Acc v = slice_ptr(sl, 0)[lane];
#pragma unroll
          for (int w2 = 1; w2 < W; ++w2) v += slice_ptr(sl, w2)[lane];
          store_out(p, sp, sl + CAP * i, v);
        }
      }
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int b = 0; b < MT; ++b)
#pragma unroll
        for (int c = 0; c < NACC; ++c) acc[rt][b][c] = Acc{0, 0, 0, 0};
  };

  if (u_first >= u_end) return;
  SkinnyWStage<RT, WN> wr[DW];
  // Prologue in the steady state's issue order (weights of step t + DW - 1, then activations of
  // unit t + DX - 1), so the activation wait count is the same at every step.
#pragma unroll
  for (int i = 0; i < DW - 1; ++i) {
    load_w(wr[i]);
    if constexpr (!XLDS) {
      if (i >= DW - DX) load_x(i - (DW - DX));
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  store_staged();
  for (int u = u_first; u < u_end; ++u) {
    const int p = u % a.panels, sp = u / a.panels;
    // NSU is a multiple of DW, so every unit starts at ring stage 0.
    for (int su = 0; su < a.NSU; su += DW) {
#pragma unroll
      for (int i = 0; i < DW; ++i) {
        load_w(wr[(i + DW - 1) % DW]);
        if constexpr (!XLDS) load_x((i + DX - 1) % DX);
        __builtin_amdgcn_sched_barrier(0);
        compute(wr[i], i % DX, sp, su + i);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if constexpr (RSW > RS) {
      if (u + 1 == u_end) {
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));  // the ring's last loads have landed
        unit_end(p, sp, std::integral_constant<int, RSW>{});
        continue;
      }
    }
    unit_end(p, sp, std::integral_constant<int, RS>{});
  }
}

// Second pass of a split launch: y (and acc) from the S raw partial sums of each output, added in
// split order. One thread per token and group of four rows; the workspace rows are 16 nrb long.
// S is a template argument so a thread issues all S loads before its first add and waits for one
// memory round trip, not S of them; the partials are read once, with the streaming policy. On
// MI355X down_proj at 17 tokens (8 splits) 17.6 -> 16.0 us, o_proj at 128 (4 splits) 16.7 -> 15.1.
template <bool I8, int S>
__global__ void __launch_bounds__(256)
skinny_reduce(SkinnyArgs a) {
  using Acc = std::conditional_t<I8, i32x4, f32x4>;
  const int groups = 4 * a.nrb;  // four-row groups per token
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (int64_t)a.M * groups) return;
  const int m = (int)(t / groups);
  const int n = 4 * (int)(t - (int64_t)m * groups);
  if (n >= a.N) return;
  const int64_t split_stride = (int64_t)a.M * 16 * a.nrb;
  const Acc* src = reinterpret_cast<const Acc*>(static_cast<const char*>(a.part) +
                                                ((int64_t)m * 16 * a.nrb + n) * 4);
  Acc p[S];
#pragma unroll
  for (int sp = 0; sp < S; ++sp) p[sp] = __builtin_nontemporal_load(src + sp * split_stride / 4);
  Acc v = p[0];
#pragma unroll
  for (int sp = 1; sp < S; ++sp) v += p[sp];
  const int cnt = min(4, a.N - n);
  float sc[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) sc[r] = r < cnt ? a.s[n + r] : 0.0f;
  const bool yvec = a.y && (a.ldy & 3) == 0 && ((uintptr_t)a.y & 7) == 0;
  store_out4<I8>(a.y, a.ldy, a.acc, a.N, m, n, cnt, v, sc, I8 ? a.sx[m] : 0.0f, yvec);
}

template <bool I8>
static const void* skinny_reduce_fn(int splits) {
  switch (splits) {
    case 2: return reinterpret_cast<const void*>(&skinny_reduce<I8, 2>);
    case 3: return reinterpret_cast<const void*>(&skinny_reduce<I8, 3>);
    case 4: return reinterpret_cast<const void*>(&skinny_reduce<I8, 4>);
    case 5: return reinterpret_cast<const void*>(&skinny_reduce<I8, 5>);
    case 6: return reinterpret_cast<const void*>(&skinny_reduce<I8, 6>);
    case 7: return reinterpret_cast<const void*>(&skinny_reduce<I8, 7>);
    case 8: return reinterpret_cast<const void*>(&skinny_reduce<I8, 8>);
    default: return nullptr;
  }
}

// ---- host side -----------------------------------------------------------------------------

// Kernel configuration: token tiles MT (the class of M), row tiles per panel RT, waves W, ring
// depths, K splits S (measured per class and shape on MI355X). MT, RT, W and S fix every summation order, so they depend on the class, N,
// K and the CU count only, never on M inside a class. Staged (XLDS) and streamed activations feed
// the same MFMAs in the same order, so the choice between them (by M and K) changes no result.
struct SkinnyShape {
  int mt, rt, w, dw;
  bool xlds;
  int splits;
};

template <bool I8, int MT, int RT, int W, int DW, int DX, bool XLDS, bool GLU = false,
          bool BFW = false, bool QX = false>
static const void* skinny_fn() {
  return reinterpret_cast<const void*>(&skinny_kernel<I8, MT, RT, W, DW, DX, XLDS, GLU, BFW, QX>);
}

// The paired-grid form of the M <= 16 kernel with staged activations (skinny_plan_for).
template <bool I8>
static const void* skinny_paired_fn() {
  return reinterpret_cast<const void*>(
      &skinny_kernel<I8, 1, 1, 8, 4, 1, true, false, false, false, true>);
}

// Panel height for 17..64 tokens: each panel re-reads the activations from L2, so panels are as
// tall as the row-tile count allows while still giving every CU work (measured on MI355X: 64-row
// panels from 1024 row tiles up, 32-row panels from 384).
static int skinny_rt(int64_t N) {
  const int64_t nrb = ceil_div(N, kTileRows);
  return nrb >= 1024 ? 4 : nrb >= 384 ? 2 : 1;
}

// Few row tiles and a deep K (the MLP down projection): one panel per CU would read all of the
// activations once per 16 rows. Four K splits of 64-row panels cut that traffic fourfold, and
// the partial sums (4 x M x N fp32) stay small next to the weights, so the second pass that adds
// them is cheap. Wider N would make the partial sums, and that pass, too large to pay off.
static bool skinny_split_k(int64_t N, int64_t K) {
  return ceil_div(N, kTileRows) <= 256 && ceil_div(K, kTileK) >= 128;
}

// N counts packed rows (2 x 16 ceil(I / 16) in the gate/up layout, whose panels hold at least
// one pair of row tiles and are never split over K).
template <bool I8>
static SkinnyShape skinny_shape(int64_t M, int64_t N, int64_t K, bool glu = false,
                                bool nosplit = false) {
  if (M <= 16) {
    const bool fits = M * (size_t)skinny_x_row((int)K, I8 ? 1 : 2) <= (size_t)kSkinnyXLdsBytes;
    // A weight ring of 2 when every wave has at most one K step (K <= 512): the 4-deep ring
    // would run three padding steps whose out-of-range loads still cross the memory pipeline.
    // On MI355X the trivial call (M 1, K 64, N 16) 3.82 -> 3.43 us per graph-replayed launch.
    // The ring depth changes no summation order (padding steps add zero products).
    const int dw = !glu && fits && ceil_div(ceil_div(K, kTileK), 8) <= 1 ? 2 : 4;
    return {1, glu ? 2 : 1, 8, dw, fits, 1};
  }
  const int mt = M <= 32 ? 2 : 4;
  if (!glu && !nosplit && skinny_split_k(N, K)) return {mt, 4, 4, 4, false, 4};
  const int rt = std::max(skinny_rt(N), glu ? 2 : 1);
  // 17..32 tokens over single-row-tile panels (o_proj, k/v): one wave per SIMD with 4-deep
  // activation rings keeps more activation bytes in flight than two waves with 2-deep ones; on
  // MI355X in W8A16 7-10 % faster (o_proj 8.4 against 9.2 us at 32 tokens). W8A8 likewise above
  // 64 row tiles (o_proj 7.20 against 7.79 us at 32 tokens, the tensor-parallel o_proj and
  // down_proj shards 6-12 %); k/v (64 row tiles, 64 workgroups) keeps eight waves (3-7 % faster
  // at 17 tokens).
  if (mt == 2) {
    const bool four = rt == 4 || (rt == 1 && (!I8 || ceil_div(N, kTileRows) > 64));
    return {2, rt, four ? 4 : 8, 4, false, 1};
  }
  // 64 tokens: two waves per SIMD (eight per workgroup); a weight ring of 4 for single row
  // tiles (o_proj: 5 % faster than one wave per SIMD), 2 for 32- and 64-row panels.
  return rt == 1 ? SkinnyShape{4, 1, 8, 4, false, 1} : SkinnyShape{4, rt, 8, 2, false, 1};
}

template <bool I8, bool GLU = false, bool BFW = false>
static const void* skinny_kernel_for(const SkinnyShape& sh) {
  if constexpr (GLU) {
    if (sh.mt == 1)
      return sh.xlds ? skinny_fn<I8, 1, 2, 8, 4, 1, true, true>()
                     : skinny_fn<I8, 1, 2, 8, 4, 4, false, true>();
  } else {
    if (sh.mt == 1) {
      if (sh.dw == 2) return skinny_fn<I8, 1, 1, 8, 2, 1, true, false, BFW>();  // xlds
      return sh.xlds ? skinny_fn<I8, 1, 1, 8, 4, 1, true, false, BFW>()
                     : skinny_fn<I8, 1, 1, 8, 4, 4, false, false, BFW>();
    }
    if (sh.rt == 1) {
      if (sh.mt == 2)
        return sh.w == 4 ? skinny_fn<I8, 2, 1, 4, 4, 4, false, false, BFW>()
                         : skinny_fn<I8, 2, 1, 8, 4, 4, false, false, BFW>();
      return skinny_fn<I8, 4, 1, 8, 4, 2, false, false, BFW>();
    }
    if constexpr (!BFW)
      if (sh.mt == 4 && sh.rt == 4 && sh.w == 4) return skinny_fn<I8, 4, 4, 4, 4, 2, false>();
  }
  if (sh.mt == 2) {
    if (sh.rt == 2) return skinny_fn<I8, 2, 2, 8, 4, 2, false, GLU, BFW>();
    return skinny_fn<I8, 2, 4, 4, 4, 4, false, GLU, BFW>();
  }
  if (sh.rt == 2) return skinny_fn<I8, 4, 2, 8, 2, 2, false, GLU, BFW>();
  return skinny_fn<I8, 4, 4, 8, 2, 2, false, GLU, BFW>();
}

struct SkinnyPlan {
  SkinnyShape sh;
  const void* fn;
  SkinnyArgs a;       // shape fields only
  int grid;
  size_t x_lds;
  int64_t part_bytes;  // workspace for the raw partial sums (0 when S = 1)
};

static int skinny_device_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return cus;
}

// Whole units per workgroup, spread as evenly as whole units allow over the resident
// workgroups; with S = 1 the scales of a workgroup's panels must fit its LDS array.
static int skinny_grid(int units, int rt, bool split, int resident) {
  int64_t per = ceil_div(units, resident);
  if (!split) per = std::min<int64_t>(per, kSkinnyScaleLds / (16 * rt));
  return (int)ceil_div(units, per);
}

// The plan of one call for a given configuration: kernel, unit counts, grid and workspace size.
template <bool I8>
static SkinnyPlan skinny_plan_for(const SkinnyShape& sh, const void* fn, int64_t M, int64_t N,
                                  int64_t K, const void* paired_fn = nullptr) {
  SkinnyPlan pl;
  pl.sh = sh;
  pl.fn = fn;
  pl.x_lds = sh.xlds ? ceil_div(M * (int64_t)skinny_x_row((int)K, I8 ? 1 : 2), 1024) * 1024 : 0;
  SkinnyArgs& a = pl.a;
  a = SkinnyArgs{};
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.nsteps = (int)ceil_div(K, kTileK);
  a.nrb = (int)ceil_div(N, kTileRows);
  a.panels = (int)ceil_div(a.nrb, sh.rt);
  a.splits = sh.splits;
  a.ssteps = (int)ceil_div(a.nsteps, sh.splits);
  a.units = a.panels * sh.splits;
  a.NSU = (int)(ceil_div(ceil_div(a.ssteps, sh.w), sh.dw) * sh.dw);
  const int resident = persistent_blocks(fn, 64 * sh.w, pl.x_lds);
  pl.grid = skinny_grid(a.units, sh.rt, sh.splits > 1, resident);
  // With two workgroups resident per CU and at least two units per CU, whole units spread over
  // the workgroups leave some CUs a unit more than others (gate_up at M <= 16: 1792 units as 448
  // workgroups of 4, so 192 CUs stream 8 units and 64 stream 4, against 7 each); a paired grid
  // gives every CU the same share, split 4 + 3 between its two workgroups.
  const int cus = paired_fn && resident > 0 ? skinny_device_cus() : 0;
  if (sh.splits == 1 && cus > 0 && resident >= 2 * cus && a.units >= 2 * cus &&
      ceil_div(ceil_div(a.units, cus), 2) <= kSkinnyScaleLds / (16 * sh.rt) &&
      ceil_div(a.units, pl.grid) * ceil_div(pl.grid, cus) > ceil_div(a.units, cus)) {
    a.pairs = cus;
    pl.grid = 2 * cus;
    pl.fn = paired_fn;  // the same kernel's paired form: same resources, so the same residency
  }
  pl.part_bytes = sh.splits > 1 ? (int64_t)sh.splits * M * 16 * a.nrb * 4 : 0;
  return pl;
}

// glu > 0: the gate/up layout of two (glu, K) matrices (N is then ignored). bfw: bf16 weights.
template <bool I8>
static SkinnyPlan skinny_plan(int64_t M, int64_t N, int64_t K, int64_t glu = 0,
                              bool bfw = false) {
  if (glu > 0) N = 2 * kTileRows * ceil_div(glu, kTileRows);
  const SkinnyShape sh = skinny_shape<I8>(M, N, K, glu > 0, bfw);
  const void* fn = glu > 0 ? skinny_kernel_for<I8, true>(sh)
                   : bfw   ? skinny_kernel_for<false, false, true>(sh)
                           : skinny_kernel_for<I8>(sh);
  const bool pairable = glu == 0 && !bfw && sh.mt == 1 && sh.xlds && sh.dw == 4;
  SkinnyPlan pl =
      skinny_plan_for<I8>(sh, fn, M, N, K, pairable ? skinny_paired_fn<I8>() : nullptr);
  pl.a.glu = (int)glu;
  return pl;
}

// Launches a planned call: the unit kernel, then (S > 1) the reduction over the splits. The
// workspace `part` must hold pl.part_bytes.
template <bool I8>
static int skinny_launch(SkinnyPlan& pl, void* part, hipStream_t stream) {
  SkinnyArgs& a = pl.a;
  a.part = part;
  void* args[] = {&a};
  const void* red = pl.sh.splits > 1 ? skinny_reduce_fn<I8>(pl.sh.splits) : nullptr;
  if (pl.sh.splits > 1 && !red) return LSE_E_RANGE;
  hipError_t e = hipLaunchKernel(pl.fn, dim3((unsigned)pl.grid), dim3(64 * pl.sh.w), args,
                                 pl.x_lds, stream);
  if (e == hipSuccess && red) {
    const int64_t threads = (int64_t)a.M * 4 * a.nrb;
    e = hipLaunchKernel(red, dim3((unsigned)ceil_div(threads, 256)), dim3(256), args, 0, stream);
  }
  return e == hipSuccess ? launch_status() : (int)e;
}

int64_t deep_decode_part_bytes(int64_t M, int64_t N);  // tiled.hip
int launch_w8a16_deep_decode(const uint16_t* x, int64_t ldx, const int8_t* qp, const float* s,
                             uint16_t* y, int64_t ldy, int64_t M, int64_t N, int64_t K, void* ws,
                             int64_t ws_bytes, hipStream_t stream);  // tiled.hip
int launch_w8a8_deep_decode(const int8_t* xq, const float* sx, const int8_t* qp, const float* s,
                            uint16_t* y, int64_t ldy, int32_t* acc, int64_t M, int64_t N,
                            int64_t K, void* ws, int64_t ws_bytes, hipStream_t stream);  // tiled.hip
int launch_w8a8_wide_decode(const int8_t* xq, const float* sx, const int8_t* qp, const float* s,
                            uint16_t* y, int64_t ldy, int32_t* acc, int64_t M, int64_t N,
                            int64_t K, int64_t glu, hipStream_t stream);  // tiled.hip

// 17..64 tokens over a deep, narrow weight (this kernel's split-K class: the MLP down
// projection): 8 K ranges of tiles of the tiled kernel, whose partial sums skinny_reduce adds.
// Chosen by the token class, N and K only, in both modes.
static bool skinny_deep_tiled(int64_t M, int64_t N, int64_t K) {
  return M > 16 && skinny_split_k(N, K);
}

int64_t xs_part_bytes(int64_t M, int64_t N, int64_t K);  // xsplit.hip
int launch_w8a16_xs(const uint16_t* x, int64_t ldx, const int8_t* qp, const float* s,
                    uint16_t* y, int64_t ldy, int64_t M, int64_t N, int64_t K, void* ws,
                    int64_t ws_bytes, hipStream_t stream);  // xsplit.hip

// 17..64 tokens over at most 64 row tiles (the k and v projections, tensor-parallel q/k/v
// shards): the stationary-slice kernel (xsplit.hip), W8A16, when a K range's activations fit its
// LDS. Chosen by the token class, N and K only.
static bool skinny_xs(int64_t M, int64_t N, int64_t K) {
  return M > 16 && ceil_div(N, kTileRows) <= 64 && !skinny_split_k(N, K) &&
         xs_part_bytes(M, N, K) >= 0;
}

// The second pass for the tiled kernel's split partial sums (the same [S][M][16 nrb] layout):
// fp32 partials and y in W8A16, int32 partials, y and acc in W8A8.
int launch_skinny_reduce_parts(bool i8, const void* part, const float* s, const float* sx,
                               uint16_t* y, int64_t ldy, int32_t* acc, int64_t M, int64_t N,
                               int splits, hipStream_t stream) {
  SkinnyArgs a{};
  a.M = (int)M;
  a.N = (int)N;
  a.nrb = (int)ceil_div(N, kTileRows);
  a.splits = splits;
  a.part = const_cast<void*>(part);
  a.s = s;
  a.sx = sx;
  a.y = y;
  a.ldy = ldy;
  a.acc = acc;
  void* args[] = {&a};
  const int64_t threads = M * 4 * a.nrb;
  const void* fn = i8 ? skinny_reduce_fn<true>(splits) : skinny_reduce_fn<false>(splits);
  if (!fn) return LSE_E_RANGE;
  const hipError_t e =
      hipLaunchKernel(fn, dim3((unsigned)ceil_div(threads, 256)), dim3(256), args, 0, stream);
  return e == hipSuccess ? launch_status() : (int)e;
}

int64_t skinny_workspace_bytes(bool i8, int64_t M, int64_t N, int64_t K) {
  if (skinny_deep_tiled(M, N, K)) return deep_decode_part_bytes(M, N);
  if (!i8 && skinny_xs(M, N, K)) return xs_part_bytes(M, N, K);
  return i8 ? skinny_plan<true>(M, N, K).part_bytes : skinny_plan<false>(M, N, K).part_bytes;
}

int launch_w8a16_wide_decode(const uint16_t* x, int64_t ldx, const int8_t* qp, const float* s,
                             uint16_t* y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                             int64_t glu, hipStream_t stream);  // tiled.hip

// 17..64 tokens over a wide weight (64-row panels in this kernel, never split): a 32 x 128 or
// 64 x 128 tile of the tiled kernel instead (64 x 128 in W8A8). Here this kernel's waves split each
// panel's K steps and then add 8 or 16 partial tiles each through LDS; with 17 or more tokens
// that reduction and the per-wave activation rings cost more than they save, while a tile over
// the whole K shares one activation stage among its waves. Chosen by the token class and N only,
// like every decode configuration.
static bool skinny_wide_tiled(int64_t M, int64_t N) {
  return M > 16 && ceil_div(N, kTileRows) >= 1024;
}

template <bool I8>
static int skinny_run(const void* x, int64_t ldx, const int8_t* qp, const float* s,
                      const float* sx, uint16_t* y, int64_t ldy, int32_t* acc, int64_t M,
                      int64_t N, int64_t K, int64_t glu, void* ws, int64_t ws_bytes,
                      hipStream_t stream, bool bfw = false) {
  const int64_t rows = glu > 0 ? 2 * kTileRows * ceil_div(glu, kTileRows) : N;
  if constexpr (!I8) {
    if (!bfw && skinny_wide_tiled(M, rows))
      return launch_w8a16_wide_decode(static_cast<const uint16_t*>(x), ldx, qp, s, y, ldy, M, N,
                                      K, glu, stream);
    if (!bfw && glu == 0 && skinny_deep_tiled(M, N, K))
      return launch_w8a16_deep_decode(static_cast<const uint16_t*>(x), ldx, qp, s, y, ldy, M, N,
                                      K, ws, ws_bytes, stream);
    if (!bfw && glu == 0 && skinny_xs(M, N, K))
      return launch_w8a16_xs(static_cast<const uint16_t*>(x), ldx, qp, s, y, ldy, M, N, K, ws,
                             ws_bytes, stream);
  } else {
    const int8_t* xq = static_cast<const int8_t*>(x);
    if (skinny_wide_tiled(M, rows))
      return launch_w8a8_wide_decode(xq, sx, qp, s, y, ldy, acc, M, N, K, glu, stream);
    if (glu == 0 && skinny_deep_tiled(M, N, K))
      return launch_w8a8_deep_decode(xq, sx, qp, s, y, ldy, acc, M, N, K, ws, ws_bytes, stream);
  }
  SkinnyPlan pl = skinny_plan<I8>(M, N, K, glu, bfw);
  if (ws_bytes < pl.part_bytes || (pl.part_bytes && !ws)) return LSE_E_WORKSPACE;
  SkinnyArgs& a = pl.a;
  a.x = x;
  a.ldx = ldx;
  a.qp = qp;
  a.s = s;
  a.sx = sx;
  a.y = y;
  a.ldy = ldy;
  a.acc = acc;
  return skinny_launch<I8>(pl, ws, stream);
}

int launch_w8a16_skinny(const uint16_t* x, int64_t ldx, const int8_t* qp, const float* s,
                        uint16_t* y, int64_t ldy, int64_t M, int64_t N, int64_t K, void* ws,
                        int64_t ws_bytes, hipStream_t stream) {
  return skinny_run<false>(x, ldx, qp, s, nullptr, y, ldy, nullptr, M, N, K, 0, ws, ws_bytes,
                           stream);
}

int launch_w8a8_skinny(const int8_t* xq, const float* sx, const int8_t* qp, const float* s,
                       uint16_t* y, int64_t ldy, int32_t* acc, int64_t M, int64_t N, int64_t K,
                       void* ws, int64_t ws_bytes, hipStream_t stream) {
  return skinny_run<true>(xq, K, qp, s, sx, y, ldy, acc, M, N, K, 0, ws, ws_bytes, stream);
}

int launch_w8a16_skinny_glu(const uint16_t* x, int64_t ldx, const int8_t* qp, const float* s,
                            uint16_t* h, int64_t ldh, int64_t M, int64_t I, int64_t K,
                            hipStream_t stream) {
  return skinny_run<false>(x, ldx, qp, s, nullptr, h, ldh, nullptr, M, 0, K, I, nullptr, 0,
                           stream);
}

// W8A8 from bf16 activations in one launch, for M <= 16 tokens whose int8 rows fit the staged
// image: the decode kernel quantizes x per token while staging it (QX). Results are bit-identical
// to lse_quantize_act_per_token followed by the decode kernel.
bool w8a8_quantizing_supported(int64_t M, int64_t K) {
  return M >= 1 && M <= 16 && M * (int64_t)skinny_x_row((int)K, 1) <= kSkinnyXLdsBytes;
}

int launch_w8a8_skinny_quantizing(const uint16_t* x, int64_t ldx, const int8_t* qp,
                                  const float* s, uint16_t* y, int64_t ldy, int32_t* acc,
                                  int64_t M, int64_t N, int64_t K, hipStream_t stream) {
  const SkinnyShape sh = skinny_shape<true>(M, N, K);
  if (sh.mt != 1 || !sh.xlds || sh.splits != 1) return LSE_E_ALGO;
  SkinnyPlan pl = skinny_plan_for<true>(
      sh,
      sh.dw == 2 ? skinny_fn<true, 1, 1, 8, 2, 1, true, false, false, true>()
                 : skinny_fn<true, 1, 1, 8, 4, 1, true, false, false, true>(),
      M, N, K);
  SkinnyArgs& a = pl.a;
  a.x = x;
  a.ldx = ldx;
  a.qp = qp;
  a.s = s;
  a.sx = nullptr;
  a.y = y;
  a.ldy = ldy;
  a.acc = acc;
  return skinny_launch<true>(pl, nullptr, stream);
}

int launch_w8a8_skinny_glu(const int8_t* xq, const float* sx, const int8_t* qp, const float* s,
                           uint16_t* h, int64_t ldh, int64_t M, int64_t I, int64_t K,
                           hipStream_t stream) {
  return skinny_run<true>(xq, K, qp, s, sx, h, ldh, nullptr, M, 0, K, I, nullptr, 0, stream);
}

}  // namespace lse

namespace lse {

int launch_bf16_tiled(const uint16_t* x, int64_t ldx, const uint16_t* wp, uint16_t* y,
                      int64_t ldy, int64_t M, int64_t N, int64_t K, hipStream_t stream);  // tiled.hip

// bf16 weights: this kernel up to 16 tokens (and up to 64 over narrow weights), the tiled
// kernel's bf16 tiles where this kernel's gate_up-class rule sends int8 weights to tiles
// (17..64 tokens over at least 1024 row tiles, the lm_head) and beyond 64 tokens.
int launch_bf16_skinny(const uint16_t* x, int64_t ldx, const uint16_t* wp, uint16_t* y,
                       int64_t ldy, int64_t M, int64_t N, int64_t K, hipStream_t stream) {
  if (M > LSE_DECODE_MAX_M || skinny_wide_tiled(M, N))
    return launch_bf16_tiled(x, ldx, wp, y, ldy, M, N, K, stream);
  return skinny_run<false>(x, ldx, reinterpret_cast<const int8_t*>(wp), nullptr, nullptr, y, ldy,
                           nullptr, M, N, K, 0, nullptr, 0, stream, true);
}

}  // namespace lse
