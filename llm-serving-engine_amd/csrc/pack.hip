// Row-major (N, K) int8 weight -> packed tiles of 16 rows x 64 K-bytes (layout in lse_common.h).
// One thread writes one 16-byte lane slot of a tile: 16 K-consecutive bytes of one row, which is
// one aligned 128-bit load from the row-major source (K % 16 == 0). Rows past N and K past the
// end are written as zeros, so the GEMMs can read whole tiles without edge cases.
//
// Gate/up layout (glu > 0): the source is the stacked (2 glu, K) matrix [gate; up] and packed row
// tile 2t holds gate rows 16t..16t+15, tile 2t+1 the same rows of up (zero past glu), so every
// even-aligned pair of row tiles carries matching gate and up rows for a fused SiLU-mul epilogue.
#include "lse_common.h"

namespace lse {

__global__ void __launch_bounds__(256)
pack_weight_tiles(const int8_t* __restrict__ q, int N, int K, int nsteps, int64_t slots,
                  int glu, uint4* __restrict__ qp) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= slots) return;
  const int64_t tile = t >> 6;
  const int lane = (int)(t & 63);
  const int64_t rb = tile / nsteps;
  const int j = (int)(tile - rb * nsteps);
  const int k = 64 * j + 16 * (lane >> 4);
  int64_t row;
  bool valid;
  if (glu > 0) {
    const int64_t r = 16 * (rb >> 1) + (lane & 15);  // row within gate or up
    row = (rb & 1) * glu + r;
    valid = r < glu;
  } else {
    row = 16 * rb + (lane & 15);
    valid = row < N;
  }
  uint4 v = make_uint4(0, 0, 0, 0);
  if (valid && k < K) v = *reinterpret_cast<const uint4*>(q + row * K + k);
  qp[t] = v;
}

int64_t packed_weight_bytes(int64_t N, int64_t K) {
  return ceil_div(N, kTileRows) * ceil_div(K, kTileK) * kTileBytes;
}

int64_t packed_glu_bytes(int64_t I, int64_t K) { return 2 * packed_weight_bytes(I, K); }

static int launch_pack(const int8_t* q, int64_t N, int64_t K, int64_t glu, int64_t bytes,
                       int8_t* qp, hipStream_t stream) {
  const int64_t slots = bytes / 16;
  const int64_t blocks = ceil_div(slots, 256);
  hipLaunchKernelGGL(pack_weight_tiles, dim3((unsigned)blocks), dim3(256), 0, stream, q, (int)N,
                     (int)K, (int)ceil_div(K, kTileK), slots, (int)glu,
                     reinterpret_cast<uint4*>(qp));
  return launch_status();
}

int launch_pack_weight(const int8_t* q, int64_t N, int64_t K, int8_t* qp, hipStream_t stream) {
  return launch_pack(q, N, K, 0, packed_weight_bytes(N, K), qp, stream);
}

int launch_pack_glu(const int8_t* q, int64_t I, int64_t K, int8_t* qp, hipStream_t stream) {
  return launch_pack(q, 2 * I, K, I, packed_glu_bytes(I, K), qp, stream);
}

}  // namespace lse

namespace lse {

// Row-major (N, K) bf16 (row stride ldw) -> the bf16 tile layout (lse_common.h). One thread per
// 16-byte lane slot: 8 K-consecutive bf16 of one row, one aligned 128-bit source load.
__global__ void __launch_bounds__(256)
pack_bf16_tiles(const uint16_t* __restrict__ w, int64_t ldw, int N, int K, int nsteps,
                int64_t slots, uint4* __restrict__ wp) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= slots) return;
  const int lane = (int)(t & 63);
  const int h = (int)((t >> 6) & 1);
  const int64_t step = t >> 7;  // (rb, j)
  const int64_t rb = step / nsteps;
  const int j = (int)(step - rb * nsteps);
  const int64_t row = 16 * rb + (lane & 15);
  const int k = 64 * j + 16 * (lane >> 4) + 8 * h;
  uint4 v = make_uint4(0, 0, 0, 0);
  if (row < N && k < K) v = *reinterpret_cast<const uint4*>(w + row * ldw + k);
  wp[t] = v;
}

int64_t packed_bf16_bytes(int64_t N, int64_t K) {
  return ceil_div(N, kTileRows) * ceil_div(K, kTileK) * 2 * kTileBytes;
}

int launch_pack_bf16(const uint16_t* w, int64_t ldw, int64_t N, int64_t K, uint16_t* wp,
                     hipStream_t stream) {
  const int64_t slots = packed_bf16_bytes(N, K) / 16;
  hipLaunchKernelGGL(pack_bf16_tiles, dim3((unsigned)ceil_div(slots, 256)), dim3(256), 0, stream,
                     w, ldw, (int)N, (int)K, (int)ceil_div(K, kTileK), slots,
                     reinterpret_cast<uint4*>(wp));
  return launch_status();
}

}  // namespace lse
