// W8A8 tiled GEMM for M above the decode range: acc[m,n] = sum_k xq[m,k] q[n,k] in int32
// (exact: |acc| <= 127*127*K < 2^31), then y[m,n] = bf16_rne((fp32(acc) * sx[m]) * s[n]).
// 128x128x128 block tiles of v_mfma_i32_16x16x64_i8 staged through LDS, double buffered; the
// weight tiles come from the packed layout (two 64-wide K steps per block step). Integer
// accumulation is associative, so the result is bit-exact in any order. The decode range runs
// in skinny.hip.
#include "lse_common.h"

namespace lse {

namespace gemm8 {
constexpr int BM = 128, BN = 128, BK = 128;
constexpr int WAVES_M = 2, WAVES_N = 2;
constexpr int THREADS = 64 * WAVES_M * WAVES_N;
constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
constexpr int TM = WM / 16, TN = WN / 16;
constexpr int LDK = BK + 16;                       // int8 row pitch in LDS
constexpr int A_CHUNKS = BM * BK / 16 / THREADS;   // uint4 loads of xq per thread
constexpr int B_CHUNKS = BN * BK / 16 / THREADS;   // uint4 loads of q per thread
}  // namespace gemm8

// A is xq (M rows), B is q (N rows); D tile (i, j) lane l holds rows 4*(l/16)+r of column l%16,
// so each lane owns four rows m of one column n.
__global__ void __launch_bounds__(gemm8::THREADS)
w8a8_gemm_kernel(const int8_t* __restrict__ xq, const float* __restrict__ sx,
                 const int8_t* __restrict__ q, const float* __restrict__ s,
                 uint16_t* __restrict__ y, int64_t ldy, int32_t* __restrict__ acc_out, int M, int N,
                 int K) {
  using namespace gemm8;
  __shared__ __attribute__((aligned(16))) int8_t As[2][BM * LDK];
  __shared__ __attribute__((aligned(16))) int8_t Bs[2][BN * LDK];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int m_block = blockIdx.y * BM, n_block = blockIdx.x * BN;

  const int8_t* a_src[A_CHUNKS];
  const uint4* b_src[B_CHUNKS];
  int a_lds[A_CHUNKS], b_lds[B_CHUNKS], a_k[A_CHUNKS], b_j[B_CHUNKS];
  bool b_ok[B_CHUNKS];
  const int nsteps = (K + 63) / 64;
#pragma unroll
  for (int i = 0; i < A_CHUNKS; ++i) {
    const int c = tid + THREADS * i, row = c / (BK / 16), kc = c % (BK / 16);
    a_src[i] = xq + (int64_t)min(m_block + row, M - 1) * K + kc * 16;
    a_lds[i] = row * LDK + kc * 16;
    a_k[i] = kc * 16;
  }
  // Packed weights: chunk c is lane slot c % 64 of tile (n_block / 16 + (c / 64) % 8, step
  // 2 * kt + c / 512); its 16 bytes are row 16 * tile + l % 16, K offset 16 * (l / 16) of the step.
#pragma unroll
  for (int i = 0; i < B_CHUNKS; ++i) {
    const int c = tid + THREADS * i, h = c / 512, t = (c / 64) % 8, l = c % 64;
    const int rb = n_block / 16 + t;
    b_ok[i] = rb < (N + 15) / 16;
    b_src[i] = reinterpret_cast<const uint4*>(q) + ((int64_t)(b_ok[i] ? rb : 0) * nsteps + h) * 64 + l;
    b_lds[i] = (16 * t + (l & 15)) * LDK + 64 * h + 16 * (l >> 4);
    b_j[i] = h;
  }
  uint4 a_reg[A_CHUNKS], b_reg[B_CHUNKS];
  auto load_tile = [&](int k0) {
    const bool full = k0 + BK <= K;
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i)
      a_reg[i] = (full || k0 + a_k[i] < K) ? *reinterpret_cast<const uint4*>(a_src[i] + k0)
                                           : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < B_CHUNKS; ++i) {
      const int j = k0 / 64 + b_j[i];
      b_reg[i] = b_ok[i] && j < nsteps ? b_src[i][(int64_t)(k0 / 64) * 64] : make_uint4(0, 0, 0, 0);
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) *reinterpret_cast<uint4*>(&As[buf][a_lds[i]]) = a_reg[i];
#pragma unroll
    for (int i = 0; i < B_CHUNKS; ++i) *reinterpret_cast<uint4*>(&Bs[buf][b_lds[i]]) = b_reg[i];
  };

  i32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = i32x4{0, 0, 0, 0};

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
    for (int kk = 0; kk < BK; kk += 64) {
      uint4 af[TM], bfr[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        af[i] = *reinterpret_cast<const uint4*>(&As[cur][(wm * WM + 16 * i + r16) * LDK + kk + 16 * g]);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        bfr[j] = *reinterpret_cast<const uint4*>(&Bs[cur][(wn * WN + 16 * j + r16) * LDK + kk + 16 * g]);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma_i8(af[i], bfr[j], acc[i][j]);
    }
    if (more) store_tile(cur ^ 1);
    __syncthreads();
  }

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
        if (m >= M) continue;
        const int v = acc[i][j][r];
        if (acc_out) acc_out[(int64_t)m * N + n] = v;
        if (y) y[(int64_t)m * ldy + n] = f32_to_bf16(((float)v * sx[m]) * sc);
      }
    }
  }
}

int launch_w8a8_gemm(const int8_t* xq, const float* sx, const int8_t* q, const float* s,
                     uint16_t* y, int64_t ldy, int32_t* acc, int64_t M, int64_t N, int64_t K,
                     hipStream_t stream) {
  using namespace gemm8;
  const dim3 grid((unsigned)((N + BN - 1) / BN), (unsigned)((M + BM - 1) / BM));
  hipLaunchKernelGGL(w8a8_gemm_kernel, grid, dim3(THREADS), 0, stream, xq, sx, q, s, y, ldy, acc,
                     (int)M, (int)N, (int)K);
  return launch_status();
}

}  // namespace lse
