// Decode GEMM with a stationary activation slice (W8A16, 17..64 tokens over a weight of at most
// 1024 rows and K of a few thousand: the k and v projections of a GQA model, tensor-parallel
// shards of q/k/v).
//
// The decode kernel gives such a weight at most 64 single-row-tile panels, so at most 64 of the
// CUs work, and every wave streams all M token rows of its K steps from L2: 8 activation bytes
// per weight byte at 64 tokens. Here a workgroup of W waves owns W row tiles (16 W weight rows)
// and one of S K ranges:
// it copies the M x (K range) activation slice into LDS once (direct-to-LDS loads, rows
// XOR-swizzled as in the tiled kernel), then each wave streams only its own row tile's weights
// through a register ring and multiplies them against the slice, with no barrier in the K loop
// and no reduction across waves. The S ranges' raw fp32 partial sums go to the workspace and the
// decode kernel's second pass (skinny_reduce) adds them in split order.
//
// Summation order per output: the range's K steps in increasing order (two K=32 MFMAs per step,
// the tiled kernel's chain), then the ranges in order. S, the wave count and the token class
// (MT token tiles: 17..32 or 33..64) depend only on the class, N, K and the CU count, never on M
// inside the class.
#include <algorithm>

#include "lse_common.h"

namespace lse {

struct XsArgs {
  const void* x;     // bf16 (M rows, stride ldx elements)
  int64_t ldx;
  const int8_t* qp;  // packed weight tiles
  void* part;        // [splits][M][16 nrb] fp32 raw partial sums
  int M, K, nsteps, nrb, splits, ssteps;
};

constexpr int kXsSliceBytes = 128 * 1024;  // LDS for the activation slice
// Four waves: for k/v (N 1024) on MI355X, 8.7 us at 64 tokens against 9.7 with eight waves
// and 10.7 in the decode kernel; 6.8 against 7.3 and 7.6 at 17. For 2048 rows and more (o_proj,
// fused q/k/v) the decode kernel stays faster at every token count (o_proj at 64 tokens 11.7 us
// against 13.3), since the second pass reads S M N 4 bytes of partials.
constexpr int kXsWaves = 4;

template <int MT, int W, int SMAX, int DW>
__global__ void __launch_bounds__(64 * W) xs_kernel(XsArgs a) {
  constexpr int MP = 16 * MT;       // token rows of the slice (the class's padded count)
  constexpr int XSTEP = MP * 128;   // bytes of one K step's image: MP rows of 64 bf16
  constexpr int PIECES = MP / 8;    // 1 KB direct-to-LDS pieces per step (8 rows each)
  static_assert(SMAX * XSTEP <= kXsSliceBytes, "slice fits the LDS budget");
  __shared__ uint4 xs[SMAX * XSTEP / 16];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane & 15, g = lane >> 4;
  // Block b: split b % S (blocks of one split share its activation slice in L2), row block b / S.
  const int S = a.splits;
  const int sp = blockIdx.x % S;
  const int rb = (blockIdx.x / S) * W + wave;  // this wave's row tile
  const int kbeg = sp * a.ssteps;
  const int nloc = min(a.ssteps, a.nsteps - kbeg);

  // The weight stream of row tile rb (none past N: a zero-length resource reads zeros).
  const uint32_t wbytes = rb < a.nrb ? (uint32_t)a.nsteps * kTileBytes : 0u;
  const BufferRsrc wres =
      make_rsrc(a.qp + (int64_t)min(rb, a.nrb - 1) * a.nsteps * kTileBytes, wbytes);
  auto wload = [&](int kt) -> uint4 {
    return buffer_load16<kLoadStream>(
        wres, kt < nloc ? (uint32_t)((kbeg + kt) * kTileBytes + 16 * lane) : kOutOfRange);
  };
  uint4 wr[DW];
#pragma unroll
  for (int i = 0; i < DW; ++i) wr[i] = wload(i);

  // The activation slice, step-major: piece p = step kt, rows 8 rg .. 8 rg + 7 (rg = p % PIECES)
  // lands at LDS byte 1024 p; lane l fills row 8 rg + l / 8, physical chunk l % 8, which holds
  // logical chunk (l % 8) ^ swz(row). Rows past M and columns past K read zeros.
  {
    const u32x4 xres =
        make_rsrc4(a.x, (uint32_t)(((int64_t)(a.M - 1) * a.ldx + a.K) * 2));
    const uint32_t base = lds_addr(xs);
    const int pieces = nloc * PIECES;
    for (int p = wave; p < pieces; p += W) {
      const int kt = p / PIECES, r = 8 * (p % PIECES) + (lane >> 3);
      const int kel = 64 * (kbeg + kt) + 8 * ((lane & 7) ^ bf16_row_swz(r));
      const uint32_t off = r < a.M && kel < a.K ? (uint32_t)(((int64_t)r * a.ldx + kel) * 2)
                                                : kOutOfRange;
      dma16_lds<0>(xres, base + 1024u * (uint32_t)p, off);
    }
  }
  // Every load so far (the slice, and the first weights) has landed; after the barrier every
  // wave's part of the slice has.
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  __builtin_amdgcn_s_barrier();

  f32x4 acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = f32x4{0, 0, 0, 0};
  for (int kt0 = 0; kt0 < nloc; kt0 += DW) {
#pragma unroll
    for (int i = 0; i < DW; ++i) {
      const int kt = kt0 + i;
      const uint4 w = wr[i];
      wr[i] = wload(kt + DW);
      if (kt < nloc) {
        bf16x8 lo, hi;
        dequant16(w, lo, hi);
        const uint4* img = xs + kt * (XSTEP / 16);
        uint4 x1[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          const int r = 16 * t + r16, sw = bf16_row_swz(r);
          acc[t] = mfma16x16x32(lo, as_bf16x8(img[r * 8 + ((2 * g) ^ sw)]), acc[t]);
          x1[t] = img[r * 8 + ((2 * g + 1) ^ sw)];
        }
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[t] = mfma16x16x32(hi, as_bf16x8(x1[t]), acc[t]);
      }
    }
  }

  // Raw partial sums of split sp: lane holds weight rows 4 g .. 4 g + 3 of token 16 t + r16.
  if (rb < a.nrb) {
    f32x4* part = static_cast<f32x4*>(a.part);
    const int64_t rowlen = 16 * (int64_t)a.nrb;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int m = 16 * t + r16;
      if (m < a.M) part[(((int64_t)sp * a.M + m) * rowlen + 16 * rb + 4 * g) / 4] = acc[t];
    }
  }
}

namespace {

struct XsPlan {
  int mt, splits, ssteps;
  int64_t blocks;
};

// S: enough ranges to give every CU a workgroup (rounded), and enough that a range's slice fits
// the LDS budget, at most 8, every range non-empty, at least 2 (else the route does not apply).
// Chosen by the class, N, K and the CU count.
bool xs_plan(int64_t M, int64_t N, int64_t K, int cus, XsPlan* p) {
  if (M <= 16 || M > LSE_DECODE_MAX_M || N <= 0 || K <= 0) return false;
  const int mt = M <= 32 ? 2 : 4;
  const int64_t smax = kXsSliceBytes / (mt * 16 * 128);
  const int64_t nrb = ceil_div(N, kTileRows), nsteps = ceil_div(K, kTileK);
  const int64_t rblocks = ceil_div(nrb, (int64_t)kXsWaves);
  int64_t s = std::max((cus + rblocks / 2) / rblocks, ceil_div(nsteps, smax));
  s = std::max<int64_t>(1, std::min<int64_t>(s, 8));
  while (s > 1 && (s - 1) * ceil_div(nsteps, s) >= nsteps) --s;  // no empty range
  const int64_t ssteps = ceil_div(nsteps, s);
  if (s < 2 || ssteps > smax) return false;  // one range: the decode kernel needs no second pass
  *p = XsPlan{mt, (int)s, (int)ssteps, rblocks * s};
  return true;
}

int device_cus_xs() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
    (void)hipGetLastError();
    return 256;
  }
  return cus;
}

}  // namespace

int launch_skinny_reduce_parts(bool i8, const void* part, const float* s, const float* sx,
                               uint16_t* y, int64_t ldy, int32_t* acc, int64_t M, int64_t N,
                               int splits, hipStream_t stream);  // skinny.hip

// Workspace of the stationary-slice route for (M, N, K), or -1 when the route does not apply.
int64_t xs_part_bytes(int64_t M, int64_t N, int64_t K) {
  XsPlan p;
  if (!xs_plan(M, N, K, device_cus_xs(), &p)) return -1;
  return (int64_t)p.splits * M * kTileRows * ceil_div(N, kTileRows) * 4;
}

int launch_w8a16_xs(const uint16_t* x, int64_t ldx, const int8_t* qp, const float* s,
                    uint16_t* y, int64_t ldy, int64_t M, int64_t N, int64_t K, void* ws,
                    int64_t ws_bytes, hipStream_t stream) {
  XsPlan p;
  if (!xs_plan(M, N, K, device_cus_xs(), &p)) return LSE_E_ALGO;
  const int64_t need = (int64_t)p.splits * M * kTileRows * ceil_div(N, kTileRows) * 4;
  if (!ws || ws_bytes < need) return LSE_E_WORKSPACE;
  if (p.blocks > 0x7fffffff) return LSE_E_RANGE;
  XsArgs a{};
  a.x = x;
  a.ldx = ldx;
  a.qp = qp;
  a.part = ws;
  a.M = (int)M;
  a.K = (int)K;
  a.nsteps = (int)ceil_div(K, kTileK);
  a.nrb = (int)ceil_div(N, kTileRows);
  a.splits = p.splits;
  a.ssteps = p.ssteps;
  void* args[] = {&a};
  const void* fn = p.mt == 2
                       ? reinterpret_cast<const void*>(&xs_kernel<2, kXsWaves, 32, 8>)
                       : reinterpret_cast<const void*>(&xs_kernel<4, kXsWaves, 16, 8>);
  const hipError_t e = hipLaunchKernel(fn, dim3((unsigned)p.blocks), dim3(64 * kXsWaves), args,
                                       0, stream);
  if (e != hipSuccess) return (int)e;
  if (int st = launch_status()) return st;
  return launch_skinny_reduce_parts(false, ws, s, nullptr, y, ldy, nullptr, M, N, p.splits,
                                    stream);
}

}  // namespace lse
