// Skinny int8-weight GEMM for the decode range (M <= 64), both modes of the int8 Linear:
//   W8A16: y[m,n] = bf16(s[n] * sum_k x[m,k] q[n,k])               bf16 x, fp32 accumulation
//   W8A8:  acc[m,n] = sum_k xq[m,k] q[n,k] exactly in int32;  y = bf16((acc * sx[m]) * s[n])
//
// The kernel is a weight stream: every weight byte is read once from HBM, in packed tiles
// (lse_common.h) so that each 128-bit load of a wave is one contiguous 1 KB tile.
//
// Work decomposition.
//  * A panel is RT row tiles (16 * RT weight rows). Each workgroup takes a contiguous range of
//    whole panels (the panels split as evenly as whole panels allow) and streams them one after
//    another.
//  * Within a panel the W waves split the 64-wide K steps round-robin (wave w takes steps w,
//    w + W, ...; a "unit" is one step of every wave). A wave multiplies each activation fragment
//    against all RT row tiles of the panel, so activations are read 2M/(16 RT) times per weight
//    byte. At the end of a panel the waves' partial sums are added through LDS in wave order,
//    scaled and stored.
//  * Every summation order depends only on (N, K, the token class of M, the grid), never on M
//    inside a class or on other rows: results are deterministic and a row's output is the same
//    inside any batch of its class. No atomics.
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
  int NSU;              // units per panel: ceil(nsteps / W) rounded up to a multiple of DW
};

// Register stage of the weight ring: one 1 KB tile per row tile of the panel.
template <int RT>
struct SkinnyWStage {
  uint4 w[RT];
};

// s_waitcnt immediate that waits for all but the `n` most recent vector-memory operations
// (vmcnt = n, expcnt and lgkmcnt left at their maxima).
__host__ __device__ constexpr int vmcnt_imm(int n) {
  return (n & 15) | 0x70 | 0xF00 | ((n >> 4) << 14);
}

// Bytes of one whole-staged activation row: K rounded up to whole 64-wide steps.
__host__ __device__ constexpr int skinny_x_row(int K, int esz) { return ((K + 63) / 64) * 64 * esz; }

// XOR swizzle of a staged row's 16-byte chunks: chunk c of token row m sits at c ^ swz(m), with
// swz(m) below the largest power of two (at most 16) dividing the chunks per row, so the
// swizzle stays inside the row and 16 consecutive rows read at one K offset spread over banks.
__host__ __device__ constexpr int skinny_swz_mask(int chunks_per_row) {
  return ((chunks_per_row & -chunks_per_row) < 16 ? (chunks_per_row & -chunks_per_row) : 16) - 1;
}

template <bool I8, int MT, int RT, int W, int DW, int DX, bool XLDS>
__global__ void __launch_bounds__(64 * W)
skinny_kernel(SkinnyArgs a) {
  using Acc = std::conditional_t<I8, i32x4, f32x4>;
  constexpr int SLICES = RT * MT;               // 16x16 output tiles of a panel
  constexpr int SPW = (SLICES + W - 1) / W;     // epilogue slices per wave
  constexpr int ESZ = I8 ? 1 : 2;               // activation element bytes
  constexpr int XL = I8 ? 1 : 2;                // 16-byte activation pieces per token tile and step
  // A single accumulator chain in W8A16 splits into two (one per dequantized half), so the two
  // MFMAs of a step do not wait on each other.
  constexpr int NACC = (!I8 && SLICES == 1) ? 2 : 1;
  static_assert(W % RT == 0, "a wave's epilogue slices share one row tile");
  static_assert(!XLDS || MT == 1, "activations are staged whole for one token tile only");
  static_assert(DW % DX == 0, "the activation ring index must repeat with the weight ring's");
  // Streamed activations: a wave's ring slot holds the 16 MT token rows x 64 K-columns of one of
  // its steps, row-major (XROW bytes a row), 16-byte chunks XOR-swizzled by token (chunk c of row
  // m sits at c ^ (m % XCH)); the wave fills it with XI pieces of 1 KB.
  constexpr int XROW = 64 * ESZ;                // bytes of one token row of a step
  constexpr int XCH = XROW / 16;                // chunks per row
  constexpr int XI = XLDS ? 0 : MT * ESZ;       // 1 KB pieces per wave per step
  constexpr int kWaitX = (DX - 1) * (RT + XI);  // loads issued after a step's activations
  static_assert(XLDS || kWaitX < 64, "vmcnt holds at most 63");
  constexpr int RSLOTS = W < SLICES ? W : SLICES;  // slices reduced per pass through LDS

  __shared__ Acc red[W][RSLOTS][64];
  __shared__ float s_lds[kSkinnyScaleLds];
  // Each ring slot (all waves' parts) is its own array, so the compiler can tell the slot a
  // direct-to-LDS load fills from the slot the MFMAs read, and leaves those waits to the explicit
  // s_waitcnt.
  constexpr int XWAVE = 16 * MT * XROW / 16;    // uint4 per wave per slot
  constexpr int XSLOT = XLDS ? 1 : W * XWAVE;
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
  const int p_first = blockIdx.x * a.panels / G;
  const int p_end = (blockIdx.x + 1) * a.panels / G;

  const BufferRsrc qres = make_rsrc(a.qp, (uint32_t)a.nrb * (uint32_t)a.nsteps * kTileBytes);
  const BufferRsrc xres = make_rsrc(a.x, (uint32_t)(((int64_t)(a.M - 1) * a.ldx + a.K) * ESZ));
  float sxv[MT];
#pragma unroll
  for (int b = 0; b < MT; ++b) {
    const int m = 16 * b + r16;
    sxv[b] = (I8 && m < a.M) ? a.sx[m] : 0.0f;
  }

  // Staged inputs, issued before the weight ring: the scales of rows [16 RT p_first, 16 RT p_end)
  // (through registers), and with XLDS all activations, copied straight to LDS: piece i of the
  // image is bytes [1024 i, 1024 i + 1024), lane l fills byte 1024 i + 16 l, which is physical
  // chunk pc of row m and holds logical chunk pc ^ swz(m); tokens past M and K past the end read
  // zeros, so the image needs no bounds checks when read.
  const int srow0 = 16 * RT * p_first;
  const int nsc = min(16 * RT * p_end, a.N) - srow0;
  constexpr int kScPerThread = (kSkinnyScaleLds + 64 * W - 1) / (64 * W);
  float sc_stage[kScPerThread];
#pragma unroll
  for (int i = 0; i < kScPerThread; ++i) {
    const int r = threadIdx.x + 64 * W * i;
    sc_stage[i] = r < nsc ? a.s[srow0 + r] : 0.0f;
  }
  const int xrow_bytes = skinny_x_row(a.K, ESZ);
  const int xswz = skinny_swz_mask(xrow_bytes / 16);
  if constexpr (XLDS) {
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
    if constexpr (XLDS) __builtin_amdgcn_s_waitcnt(vmcnt_imm((DW - 1) * RT));
    __syncthreads();
  };

  // Weight load cursor: panel lp, unit lsu within it.
  int lp = p_first, lsu = 0;
  auto load_w = [&](SkinnyWStage<RT>& st) {
    const int j = W * lsu + wave;
    const bool kv = lp < p_end && j < a.nsteps;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int rb = lp * RT + rt;
      const uint32_t off =
          ((uint32_t)rb * (uint32_t)a.nsteps + (uint32_t)j) * kTileBytes + 16u * lane;
      st.w[rt] = buffer_load16(qres, kv && rb < a.nrb ? off : kOutOfRange);
    }
    if (++lsu == a.NSU) {
      lsu = 0;
      ++lp;
    }
  };
  // Activation load cursor (activations depend on the step only, not on the panel). Piece i of
  // this wave's part of a slot covers bytes [1024 i, 1024 i + 1024): lane l fills byte
  // 1024 i + 16 l, physical chunk pc of token row m, which holds logical chunk pc ^ (m % XCH).
  // Tokens past M, K past the end and steps past the range read zeros.
  int xp = p_first, xsu = 0;
  auto load_x = [&](int slot) {
    const int j = W * xsu + wave;
    const bool live = xp < p_end && j < a.nsteps;
#pragma unroll
    for (int i = 0; i < XI; ++i) {
      const int o = 1024 * i + 16 * lane;
      const int m = o / XROW, pc = (o % XROW) / 16;
      const int kb = XROW * j + 16 * (pc ^ (m & (XCH - 1)));
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
      ++xp;
    }
  };

  Acc acc[RT][MT][NACC];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int b = 0; b < MT; ++b)
#pragma unroll
      for (int c = 0; c < NACC; ++c) acc[rt][b][c] = Acc{0, 0, 0, 0};

  // One step: the wave's K step of unit su, from weight stage st and ring slot `slot`.
  // XLDS: this lane's token row (tokens past M re-read row M-1; their outputs are dropped).
  const int x_m = min(r16, a.M - 1);
  const unsigned char* x_row_base = x_lds + x_m * xrow_bytes;
  const int x_swz = x_m & xswz;
  auto compute = [&](const SkinnyWStage<RT>& st, int slot, int su) {
    uint4 xv[MT][XL];
    if constexpr (XLDS) {
      // A padding step past the last K step (NSU is rounded up to the ring depth) re-reads step
      // 0; its weights are zero.
      const int j = W * su + wave;
      const int c0 = (j < a.nsteps ? j : 0) * 4 * ESZ + XL * g;
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
          xv[b][h] = *reinterpret_cast<const uint4*>(base + m * XROW + 16 * (c ^ (m & (XCH - 1))));
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
      for (int rt = 0; rt < RT; ++rt) dequant16(st.w[rt], lo[rt], hi[rt]);
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

  // Scales and stores one lane's four outputs (rows n..n+3 of token m of panel p's slice).
  const bool yvec = a.y && (a.ldy & 3) == 0 && ((uintptr_t)a.y & 7) == 0;
  auto store_out = [&](int p, int slice, Acc v) {
    const int rt = slice % RT, b = slice / RT;
    const int m = 16 * b + r16;
    const int n = 16 * (p * RT + rt) + 4 * g;
    if (m >= a.M || n >= a.N) return;
    const int cnt = min(4, a.N - n);
    float o[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float sc = r < cnt ? s_lds[n + r - srow0] : 0.0f;
      if constexpr (I8)
        o[r] = ((float)v[r] * sxv[b]) * sc;
      else
        o[r] = v[r] * sc;
    }
    if constexpr (I8) {
      if (a.acc) {
        int32_t* dst = a.acc + (int64_t)m * a.N + n;
        if (cnt == 4 && (a.N & 3) == 0) {
          *reinterpret_cast<i32x4*>(dst) = v;
        } else {
          for (int r = 0; r < cnt; ++r) dst[r] = v[r];
        }
      }
      if (!a.y) return;
    }
    uint16_t* out = a.y + (int64_t)m * a.ldy + n;
    if (cnt == 4 && yvec) {
      *reinterpret_cast<uint2*>(out) = make_uint2(pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]));
    } else {
      for (int r = 0; r < cnt; ++r) out[r] = f32_to_bf16(o[r]);
    }
  };

  // End of panel p: pass i adds slices [i W, i W + RSLOTS) over the waves in wave order; wave w
  // keeps slice i W + w, scales and stores it.
  auto panel_end = [&](int p) {
#pragma unroll
    for (int i = 0; i < SPW; ++i) {
      __syncthreads();  // the previous pass's (or panel's) reads of red are done
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int b = 0; b < MT; ++b) {
          const int sl = rt + RT * b - W * i;
          if (sl < 0 || sl >= RSLOTS) continue;
          Acc v = acc[rt][b][0];
          if constexpr (NACC == 2) v += acc[rt][b][1];
          red[wave][sl][lane] = v;
        }
      __syncthreads();
      const int slice = wave + W * i;
      if (slice < SLICES) {
        Acc v = red[0][wave][lane];
#pragma unroll
        for (int w2 = 1; w2 < W; ++w2) v += red[w2][wave][lane];
        store_out(p, slice, v);
      }
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int b = 0; b < MT; ++b)
#pragma unroll
        for (int c = 0; c < NACC; ++c) acc[rt][b][c] = Acc{0, 0, 0, 0};
  };

  if (p_first >= p_end) return;
  SkinnyWStage<RT> wr[DW];
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
  for (int p = p_first; p < p_end; ++p) {
    // NSU is a multiple of DW, so every panel starts at ring stage 0.
    for (int su = 0; su < a.NSU; su += DW) {
#pragma unroll
      for (int i = 0; i < DW; ++i) {
        load_w(wr[(i + DW - 1) % DW]);
        if constexpr (!XLDS) load_x((i + DX - 1) % DX);
        __builtin_amdgcn_sched_barrier(0);
        compute(wr[i], i % DX, su + i);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    panel_end(p);
  }
}

// ---- host side -----------------------------------------------------------------------------

// Kernel configuration: token tiles MT (the class of M), row tiles per panel RT, waves W, ring
// depths. W, RT and MT fix every summation order, so they depend on the class and on N only,
// never on M inside a class. Panels of 64 rows (RT = 4) when there are enough of them to fill the
// CUs, 32 rows when there are half as many, else single row tiles; larger panels read the
// activations fewer times per weight byte. Staged (XLDS) and streamed activations feed the same
// MFMAs in the same order, so the choice between them (by M and K) changes no result.
struct SkinnyShape {
  int mt, rt, w, dw;
  bool xlds;
};

template <bool I8, int MT, int RT, int W, int DW, int DX, bool XLDS>
static const void* skinny_fn() {
  return reinterpret_cast<const void*>(&skinny_kernel<I8, MT, RT, W, DW, DX, XLDS>);
}

static int skinny_rt(int64_t N) {
  const int64_t nrb = ceil_div(N, kTileRows);
  return nrb >= 1024 ? 4 : nrb >= 384 ? 2 : 1;
}

template <bool I8>
static SkinnyShape skinny_shape(int64_t M, int64_t N, int64_t K) {
  if (M <= 16) {
    const bool fits = M * (size_t)skinny_x_row((int)K, I8 ? 1 : 2) <= (size_t)kSkinnyXLdsBytes;
    return {1, 1, 8, 4, fits};
  }
  const int rt = skinny_rt(N);
  if (M <= 32) return {2, rt, rt == 4 ? 4 : 8, 4, false};
  return {4, rt, 4, 4, false};
}

template <bool I8>
static const void* skinny_kernel_for(const SkinnyShape& sh) {
  if (sh.mt == 1) {
    return sh.xlds ? skinny_fn<I8, 1, 1, 8, 4, 1, true>() : skinny_fn<I8, 1, 1, 8, 4, 4, false>();
  }
  if (sh.mt == 2) {
    if (sh.rt == 1) return skinny_fn<I8, 2, 1, 8, 4, 4, false>();
    if (sh.rt == 2) return skinny_fn<I8, 2, 2, 8, 4, 2, false>();
    return skinny_fn<I8, 2, 4, 4, 4, 4, false>();
  }
  if (sh.rt == 1) return skinny_fn<I8, 4, 1, 4, 4, 4, false>();
  if (sh.rt == 2) return skinny_fn<I8, 4, 2, 4, 4, 4, false>();
  return skinny_fn<I8, 4, 4, 4, 4, 2, false>();
}

struct SkinnyPlan {
  SkinnyShape sh;
  const void* fn;
  SkinnyArgs a;  // shape fields only
  int grid;
  size_t x_lds;
};

// Whole panels per workgroup, spread as evenly as whole panels allow over the resident
// workgroups; the scales of a workgroup's panels must fit its LDS array.
static int skinny_grid(int panels, int rt, int resident) {
  const int kmax = kSkinnyScaleLds / (16 * rt);
  const int per = (int)std::min<int64_t>(ceil_div(panels, resident), kmax);
  return (int)ceil_div(panels, per);
}

template <bool I8>
static SkinnyPlan skinny_plan(int64_t M, int64_t N, int64_t K) {
  SkinnyPlan pl;
  pl.sh = skinny_shape<I8>(M, N, K);
  pl.fn = skinny_kernel_for<I8>(pl.sh);
  pl.x_lds = pl.sh.xlds ? ceil_div(M * (int64_t)skinny_x_row((int)K, I8 ? 1 : 2), 1024) * 1024 : 0;
  SkinnyArgs& a = pl.a;
  a = SkinnyArgs{};
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.nsteps = (int)ceil_div(K, kTileK);
  a.nrb = (int)ceil_div(N, kTileRows);
  a.panels = (int)ceil_div(a.nrb, pl.sh.rt);
  a.NSU = (int)(ceil_div(ceil_div(a.nsteps, pl.sh.w), pl.sh.dw) * pl.sh.dw);
  pl.grid = skinny_grid(a.panels, pl.sh.rt, persistent_blocks(pl.fn, 64 * pl.sh.w, pl.x_lds));
  return pl;
}

template <bool I8>
static int launch_skinny(const void* x, int64_t ldx, const int8_t* qp, const float* s,
                         const float* sx, uint16_t* y, int64_t ldy, int32_t* acc, int64_t M,
                         int64_t N, int64_t K, hipStream_t stream) {
  SkinnyPlan pl = skinny_plan<I8>(M, N, K);
  SkinnyArgs& a = pl.a;
  a.x = x;
  a.ldx = ldx;
  a.qp = qp;
  a.s = s;
  a.sx = sx;
  a.y = y;
  a.ldy = ldy;
  a.acc = acc;
  void* args[] = {&a};
  const hipError_t e = hipLaunchKernel(pl.fn, dim3((unsigned)pl.grid), dim3(64 * pl.sh.w), args,
                                       pl.x_lds, stream);
  return e == hipSuccess ? launch_status() : (int)e;
}

int launch_w8a16_skinny(const uint16_t* x, int64_t ldx, const int8_t* qp, const float* s,
                        uint16_t* y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                        hipStream_t stream) {
  return launch_skinny<false>(x, ldx, qp, s, nullptr, y, ldy, nullptr, M, N, K, stream);
}

int launch_w8a8_skinny(const int8_t* xq, const float* sx, const int8_t* qp, const float* s,
                       uint16_t* y, int64_t ldy, int32_t* acc, int64_t M, int64_t N, int64_t K,
                       hipStream_t stream) {
  return launch_skinny<true>(xq, K, qp, s, sx, y, ldy, acc, M, N, K, stream);
}

}  // namespace lse
