// W8A8 GEMM: acc[m,n] = sum_k xq[m,k] q[n,k] in int32 (exact: |acc| <= 127*127*K < 2^31),
// then y[m,n] = bf16_rne((fp32(acc) * sx[m]) * s[n]).
//
// Two kernel families on v_mfma_i32_16x16x64_i8 (16x16 int32 += 16x64 int8 · 64x16 int8):
//  * decode (M <= 64): weights stream from HBM exactly as in the W8A16 decode kernel, with no
//    dequantization at all: each 128-bit weight load is one MFMA A operand.
//  * tiled GEMM (M > 64): 128x128x128 block tiles staged through LDS, double buffered.
// Integer accumulation is associative, so the result is bit-exact in any order.
#include "lse_common.h"

namespace lse {

__device__ __forceinline__ i32x4 mfma_i8(uint4 a, uint4 b, i32x4 c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4, a),
                                               __builtin_bit_cast(i32x4, b), c, 0, 0, 0);
}

// Stores one lane's four consecutive outputs n..n+3 of row m: the exact int32 accumulators
// (when requested) and the scaled bf16 values.
__device__ __forceinline__ void w8a8_store4(i32x4 v, int m, int n, int N, float sxm,
                                            const float* __restrict__ s, uint16_t* __restrict__ y,
                                            int64_t ldy, int32_t* __restrict__ acc) {
  if (n + 4 <= N) {
    if (acc) {
      int32_t* dst = acc + (int64_t)m * N + n;
      if ((N & 3) == 0) {
        *reinterpret_cast<i32x4*>(dst) = v;
      } else {
        for (int r = 0; r < 4; ++r) dst[r] = v[r];
      }
    }
    if (y) {
      const float4 sc = *reinterpret_cast<const float4*>(s + n);
      const float o[4] = {((float)v[0] * sxm) * sc.x, ((float)v[1] * sxm) * sc.y,
                          ((float)v[2] * sxm) * sc.z, ((float)v[3] * sxm) * sc.w};
      uint16_t* dst = y + (int64_t)m * ldy + n;
      if ((ldy & 3) == 0 && ((uintptr_t)y & 7) == 0) {
        *reinterpret_cast<uint2*>(dst) = make_uint2(pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]));
      } else {
        for (int r = 0; r < 4; ++r) dst[r] = f32_to_bf16(o[r]);
      }
    }
  } else {
    for (int r = 0; n + r < N; ++r) {
      if (acc) acc[(int64_t)m * N + n + r] = v[r];
      if (y) y[(int64_t)m * ldy + n + r] = f32_to_bf16(((float)v[r] * sxm) * s[n + r]);
    }
  }
}

template <int MT, int KW, int U>
__global__ void __launch_bounds__(64 * KW)
w8a8_decode_kernel(const int8_t* __restrict__ xq, const float* __restrict__ sx,
                   const int8_t* __restrict__ q, const float* __restrict__ s,
                   uint16_t* __restrict__ y, int64_t ldy, int32_t* __restrict__ acc_out, int M,
                   int N, int K) {
  __shared__ i32x4 red[KW][MT][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r16 = lane & 15, g = lane >> 4;
  const int n_block = blockIdx.x * 16;

  const int8_t* qp = q + (int64_t)min(n_block + r16, N - 1) * K + 16 * g;
  const int8_t* xp[MT];
  bool xok[MT];
#pragma unroll
  for (int b = 0; b < MT; ++b) {
    const int m = 16 * b + r16;
    xok[b] = m < M;
    xp[b] = xq + (int64_t)(xok[b] ? m : 0) * K + 16 * g;
  }
  i32x4 acc[MT];
#pragma unroll
  for (int b = 0; b < MT; ++b) acc[b] = i32x4{0, 0, 0, 0};

  struct Regs {
    uint4 w;
    uint4 x[MT];
  };
  auto load = [&](Regs& r, int step) {
    const int64_t k0 = (int64_t)step * 64;
    r.w = *reinterpret_cast<const uint4*>(qp + k0);
#pragma unroll
    for (int b = 0; b < MT; ++b)
      r.x[b] = xok[b] ? *reinterpret_cast<const uint4*>(xp[b] + k0) : make_uint4(0, 0, 0, 0);
  };
  auto compute = [&](const Regs& r) {
#pragma unroll
    for (int b = 0; b < MT; ++b) acc[b] = mfma_i8(r.w, r.x[b], acc[b]);
  };

  const int nsteps = K >> 6;
  const int mine = nsteps > wave ? (nsteps - wave + KW - 1) / KW : 0;
  const int groups = mine / U;
  Regs ra[U], rb[U];
  if (groups > 0) {
#pragma unroll
    for (int u = 0; u < U; ++u) load(ra[u], wave + KW * u);
    int gi = 0;
    for (;;) {
      const bool more = gi + 1 < groups;
      if (more) {
#pragma unroll
        for (int u = 0; u < U; ++u) load(rb[u], wave + KW * (U * (gi + 1) + u));
      }
#pragma unroll
      for (int u = 0; u < U; ++u) compute(ra[u]);
      if (!more) break;
      ++gi;
      const bool more2 = gi + 1 < groups;
      if (more2) {
#pragma unroll
        for (int u = 0; u < U; ++u) load(ra[u], wave + KW * (U * (gi + 1) + u));
      }
#pragma unroll
      for (int u = 0; u < U; ++u) compute(rb[u]);
      if (!more2) break;
      ++gi;
    }
  }
  for (int j = groups * U; j < mine; ++j) {
    load(ra[0], wave + KW * j);
    compute(ra[0]);
  }
  if ((K & 63) && wave == nsteps % KW) {
    const int64_t k0 = (int64_t)nsteps * 64;
    const bool ok = k0 + 16 * g < K;
    Regs r;
    r.w = ok ? *reinterpret_cast<const uint4*>(qp + k0) : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int b = 0; b < MT; ++b)
      r.x[b] = (ok && xok[b]) ? *reinterpret_cast<const uint4*>(xp[b] + k0) : make_uint4(0, 0, 0, 0);
    compute(r);
  }

#pragma unroll
  for (int b = 0; b < MT; ++b) red[wave][b][lane] = acc[b];
  __syncthreads();
  for (int item = threadIdx.x; item < MT * 64; item += 64 * KW) {
    const int b = item >> 6, l = item & 63;
    i32x4 sum = red[0][b][l];
#pragma unroll
    for (int w = 1; w < KW; ++w) sum += red[w][b][l];
    const int m = 16 * b + (l & 15);
    const int n = n_block + 4 * (l >> 4);
    if (m < M && n < N) w8a8_store4(sum, m, n, N, sx[m], s, y, ldy, acc_out);
  }
}

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
  const int8_t* b_src[B_CHUNKS];
  int a_lds[A_CHUNKS], b_lds[B_CHUNKS], a_k[A_CHUNKS], b_k[B_CHUNKS];
#pragma unroll
  for (int i = 0; i < A_CHUNKS; ++i) {
    const int c = tid + THREADS * i, row = c / (BK / 16), kc = c % (BK / 16);
    a_src[i] = xq + (int64_t)min(m_block + row, M - 1) * K + kc * 16;
    a_lds[i] = row * LDK + kc * 16;
    a_k[i] = kc * 16;
  }
#pragma unroll
  for (int i = 0; i < B_CHUNKS; ++i) {
    const int c = tid + THREADS * i, row = c / (BK / 16), kc = c % (BK / 16);
    b_src[i] = q + (int64_t)min(n_block + row, N - 1) * K + kc * 16;
    b_lds[i] = row * LDK + kc * 16;
    b_k[i] = kc * 16;
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
      b_reg[i] = (full || k0 + b_k[i] < K) ? *reinterpret_cast<const uint4*>(b_src[i] + k0)
                                           : make_uint4(0, 0, 0, 0);
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

template <int MT>
static int launch_w8a8_decode_mt(const int8_t* xq, const float* sx, const int8_t* q, const float* s,
                                 uint16_t* y, int64_t ldy, int32_t* acc, int64_t M, int64_t N,
                                 int64_t K, hipStream_t stream) {
  constexpr int KW = 8, U = MT == 1 ? 4 : MT == 2 ? 2 : 1;
  const dim3 grid((unsigned)((N + 15) / 16));
  hipLaunchKernelGGL((w8a8_decode_kernel<MT, KW, U>), grid, dim3(64 * KW), 0, stream, xq, sx, q, s,
                     y, ldy, acc, (int)M, (int)N, (int)K);
  return launch_status();
}

int launch_w8a8_gemm(const int8_t* xq, const float* sx, const int8_t* q, const float* s,
                     uint16_t* y, int64_t ldy, int32_t* acc, int64_t M, int64_t N, int64_t K,
                     hipStream_t stream) {
  if (M <= LSE_DECODE_MAX_M) {
    switch ((M + 15) / 16) {
      case 1: return launch_w8a8_decode_mt<1>(xq, sx, q, s, y, ldy, acc, M, N, K, stream);
      case 2: return launch_w8a8_decode_mt<2>(xq, sx, q, s, y, ldy, acc, M, N, K, stream);
      case 3: return launch_w8a8_decode_mt<3>(xq, sx, q, s, y, ldy, acc, M, N, K, stream);
      default: return launch_w8a8_decode_mt<4>(xq, sx, q, s, y, ldy, acc, M, N, K, stream);
    }
  }
  using namespace gemm8;
  const dim3 grid((unsigned)((N + BN - 1) / BN), (unsigned)((M + BM - 1) / BM));
  hipLaunchKernelGGL(w8a8_gemm_kernel, grid, dim3(THREADS), 0, stream, xq, sx, q, s, y, ldy, acc,
                     (int)M, (int)N, (int)K);
  return launch_status();
}

}  // namespace lse
