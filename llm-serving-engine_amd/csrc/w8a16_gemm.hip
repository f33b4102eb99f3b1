// W8A16 prefill GEMM: y[m,n] = bf16(s[n] * sum_k x[m,k] q[n,k]) for M above the decode range.
//
// MFMA-bound. A block computes a BM x BN tile of y over K in BK steps:
//  * x (bf16) and q (int8) tiles travel global → registers (128-bit loads) → LDS, double
//    buffered, so the next tile's loads are in flight while the current tile is multiplied. q
//    comes from the packed layout: a block step reads eight whole 1 KB tiles.
//  * q is dequantized to bf16 on its way into LDS, once per block (not once per wave).
//  * Each wave owns a WM x WN sub-tile built from v_mfma_f32_16x16x32_bf16, fp32 accumulate.
//  * Epilogue: scale by s[n] (fp32) and round to bf16 once.
// The K loop visits tiles in increasing k and every output's MFMA chain follows it, so the
// summation order of an element depends only on K.
#include "lse_common.h"

namespace lse {

namespace gemm16 {
constexpr int BM = 128, BN = 128, BK = 64;
constexpr int WAVES_M = 2, WAVES_N = 2;
constexpr int THREADS = 64 * WAVES_M * WAVES_N;
constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;  // 64 x 64 per wave
constexpr int TM = WM / 16, TN = WN / 16;            // 4 x 4 MFMA tiles per wave
constexpr int LDK = BK + 8;                          // bf16 row pitch in LDS (144 B: conflict-free b128 reads)
constexpr int A_CHUNKS = BM * BK / 8 / THREADS;      // uint4 (8 bf16) loads of x per thread
constexpr int B_CHUNKS = BN * BK / 16 / THREADS;     // uint4 (16 int8) loads of q per thread
}  // namespace gemm16

__global__ void __launch_bounds__(gemm16::THREADS)
w8a16_gemm_kernel(const uint16_t* __restrict__ x, int64_t ldx, const int8_t* __restrict__ q,
                  const float* __restrict__ s, uint16_t* __restrict__ y, int64_t ldy, int M, int N,
                  int K) {
  using namespace gemm16;
  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * LDK];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN * LDK];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int m_block = blockIdx.y * BM;
  const int n_block = blockIdx.x * BN;

  // Global source of each thread's chunks. Rows past M or N re-read the last row; their
  // results are never stored.
  const uint16_t* a_src[A_CHUNKS];
  int a_lds[A_CHUNKS], a_k[A_CHUNKS];
#pragma unroll
  for (int i = 0; i < A_CHUNKS; ++i) {
    const int c = tid + THREADS * i;
    const int row = c / (BK / 8), kc = c % (BK / 8);
    a_src[i] = x + (int64_t)min(m_block + row, M - 1) * ldx + kc * 8;
    a_lds[i] = row * LDK + kc * 8;
    a_k[i] = kc * 8;
  }
  // Chunk c is lane slot c % 64 of tile n_block / 16 + c / 64 at the block's K step: row
  // 16 * (c / 64) + l % 16 of the block, K offset 16 * (l / 16).
  const int nsteps = (K + 63) / 64;
  const uint4* b_src[B_CHUNKS];
  int b_lds[B_CHUNKS];
  bool b_ok[B_CHUNKS];
#pragma unroll
  for (int i = 0; i < B_CHUNKS; ++i) {
    const int c = tid + THREADS * i, t = c / 64, l = c % 64;
    const int rb = n_block / 16 + t;
    b_ok[i] = rb < (N + 15) / 16;
    b_src[i] = reinterpret_cast<const uint4*>(q) + (int64_t)(b_ok[i] ? rb : 0) * nsteps * 64 + l;
    b_lds[i] = (16 * t + (l & 15)) * LDK + 16 * (l >> 4);
  }

  uint4 a_reg[A_CHUNKS], b_reg[B_CHUNKS];
  auto load_tile = [&](int k0) {
    const bool full = k0 + BK <= K;
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i)
      a_reg[i] = (full || k0 + a_k[i] < K) ? *reinterpret_cast<const uint4*>(a_src[i] + k0)
                                           : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < B_CHUNKS; ++i)
      b_reg[i] = b_ok[i] ? b_src[i][(int64_t)(k0 / 64) * 64] : make_uint4(0, 0, 0, 0);
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) *reinterpret_cast<uint4*>(&As[buf][a_lds[i]]) = a_reg[i];
#pragma unroll
    for (int i = 0; i < B_CHUNKS; ++i) {
      bf16x8 lo, hi;
      dequant16(b_reg[i], lo, hi);
      *reinterpret_cast<bf16x8*>(&Bs[buf][b_lds[i]]) = lo;
      *reinterpret_cast<bf16x8*>(&Bs[buf][b_lds[i] + 8]) = hi;
    }
  };

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int r16 = lane & 15, g = lane >> 4;
  const int ktiles = (K + BK - 1) / BK;
  load_tile(0);
  store_tile(0);
  __syncthreads();
  for (int kt = 0; kt < ktiles; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < ktiles;
    if (more) load_tile((kt + 1) * BK);
#pragma unroll
    for (int kk = 0; kk < BK; kk += 32) {
      bf16x8 af[TM], bfr[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        af[i] = *reinterpret_cast<const bf16x8*>(
            &As[cur][(wm * WM + 16 * i + r16) * LDK + kk + 8 * g]);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        bfr[j] = *reinterpret_cast<const bf16x8*>(
            &Bs[cur][(wn * WN + 16 * j + r16) * LDK + kk + 8 * g]);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma16x16x32(af[i], bfr[j], acc[i][j]);
    }
    if (more) store_tile(cur ^ 1);
    __syncthreads();
  }

  // D tile (i, j): lane holds rows 4*(lane/16)+r of column lane%16.
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int n = n_block + wn * WN + 16 * j + r16;
    if (n >= N) continue;
    const float sc = s[n];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m_block + wm * WM + 16 * i + 4 * g + r;
        if (m < M) y[(int64_t)m * ldy + n] = f32_to_bf16(acc[i][j][r] * sc);
      }
    }
  }
}

int launch_w8a16_gemm(const uint16_t* x, int64_t ldx, const int8_t* q, const float* s, uint16_t* y,
                      int64_t ldy, int64_t M, int64_t N, int64_t K, hipStream_t stream) {
  using namespace gemm16;
  const dim3 grid((unsigned)((N + BN - 1) / BN), (unsigned)((M + BM - 1) / BM));
  hipLaunchKernelGGL(w8a16_gemm_kernel, grid, dim3(THREADS), 0, stream, x, ldx, q, s, y, ldy,
                     (int)M, (int)N, (int)K);
  return launch_status();
}

}  // namespace lse
