// W8A16 decode kernel (M <= 64): y[m,n] = bf16(s[n] * sum_k x[m,k] q[n,k]).
//
// HBM-bound: every weight byte is read once, so the kernel is a weight stream with the
// arithmetic hidden under it.
//  * Workgroup = KW waves over one block of 16*NA weight rows. Wave w owns the 64-wide K
//    "supersteps" w, w+KW, w+2KW, ..., so at any moment a workgroup reads one contiguous
//    64*KW-byte run of each of its rows.
//  * Lane l reads 16 bytes (one global_load_dwordx4) of row l%16 at byte 16*(l/16) of each
//    superstep: a wave load covers 16 rows x 64 bytes.
//  * Those 16 int8 → two bf16x8 A operands; x supplies the matching B operands (16 bf16 of
//    token 16*b + l%16), and two v_mfma_f32_16x16x32_bf16 per (A tile, B tile) accumulate
//    fp32. Tokens m >= M are zero operands, so M in 1..16 costs one B tile.
//  * The next group of U supersteps is loaded while the current one is converted and
//    multiplied (register double buffering).
//  * The KW per-wave partial sums are added in LDS in wave order 0..KW-1, then scaled by
//    s[n] and rounded to bf16. No atomics: the summation order of every output depends only
//    on (K, KW), and KW is chosen from (N, K), never from M.
#include "lse_common.h"

namespace lse {

template <int MT, int NA>
struct DecodeRegs {
  uint4 w[NA];
  uint4 x[MT][2];
};

template <int MT, int NA, int KW, int U>
__global__ void __launch_bounds__(64 * KW)
w8a16_decode_kernel(const uint16_t* __restrict__ x, int64_t ldx, const int8_t* __restrict__ q,
                    const float* __restrict__ s, uint16_t* __restrict__ y, int64_t ldy, int M,
                    int N, int K) {
  __shared__ f32x4 red[KW][NA * MT][64];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r16 = lane & 15;
  const int g = lane >> 4;
  const int n_block = blockIdx.x * 16 * NA;

  const int8_t* qp[NA];
#pragma unroll
  for (int a = 0; a < NA; ++a) {
    const int n = min(n_block + 16 * a + r16, N - 1);
    qp[a] = q + (int64_t)n * K + 16 * g;
  }
  const uint16_t* xp[MT];
  bool xok[MT];
#pragma unroll
  for (int b = 0; b < MT; ++b) {
    const int m = 16 * b + r16;
    xok[b] = m < M;
    xp[b] = x + (int64_t)(xok[b] ? m : 0) * ldx + 16 * g;
  }

  f32x4 acc[NA][MT];
#pragma unroll
  for (int a = 0; a < NA; ++a)
#pragma unroll
    for (int b = 0; b < MT; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto load = [&](DecodeRegs<MT, NA>& r, int step) {
    const int64_t k0 = (int64_t)step * 64;
#pragma unroll
    for (int a = 0; a < NA; ++a) r.w[a] = *reinterpret_cast<const uint4*>(qp[a] + k0);
#pragma unroll
    for (int b = 0; b < MT; ++b) {
      if (xok[b]) {
        r.x[b][0] = *reinterpret_cast<const uint4*>(xp[b] + k0);
        r.x[b][1] = *reinterpret_cast<const uint4*>(xp[b] + k0 + 8);
      } else {
        r.x[b][0] = make_uint4(0, 0, 0, 0);
        r.x[b][1] = make_uint4(0, 0, 0, 0);
      }
    }
  };
  auto compute = [&](const DecodeRegs<MT, NA>& r) {
#pragma unroll
    for (int a = 0; a < NA; ++a) {
      bf16x8 lo, hi;
      dequant16(r.w[a], lo, hi);
#pragma unroll
      for (int b = 0; b < MT; ++b) {
        acc[a][b] = mfma16x16x32(lo, as_bf16x8(r.x[b][0]), acc[a][b]);
        acc[a][b] = mfma16x16x32(hi, as_bf16x8(r.x[b][1]), acc[a][b]);
      }
    }
  };

  // This wave's supersteps: wave, wave + KW, ...; full groups of U are double buffered.
  const int nsteps = K >> 6;
  const int mine = nsteps > wave ? (nsteps - wave + KW - 1) / KW : 0;
  const int groups = mine / U;
  DecodeRegs<MT, NA> ra[U], rb[U];
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
  // K % 64 tail (K % 16 == 0): one partial superstep, taken by the wave next in line.
  if ((K & 63) && wave == nsteps % KW) {
    const int64_t k0 = (int64_t)nsteps * 64;
    DecodeRegs<MT, NA> r;
    const bool ok = k0 + 16 * g < K;
#pragma unroll
    for (int a = 0; a < NA; ++a)
      r.w[a] = ok ? *reinterpret_cast<const uint4*>(qp[a] + k0) : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int b = 0; b < MT; ++b) {
      const bool okx = ok && xok[b];
      r.x[b][0] = okx ? *reinterpret_cast<const uint4*>(xp[b] + k0) : make_uint4(0, 0, 0, 0);
      r.x[b][1] = okx ? *reinterpret_cast<const uint4*>(xp[b] + k0 + 8) : make_uint4(0, 0, 0, 0);
    }
    compute(r);
  }

  // Cross-wave reduction in fixed wave order, then the per-channel scale and bf16 store.
#pragma unroll
  for (int a = 0; a < NA; ++a)
#pragma unroll
    for (int b = 0; b < MT; ++b) red[wave][a * MT + b][lane] = acc[a][b];
  __syncthreads();
  const bool yvec = (ldy & 3) == 0 && ((uintptr_t)y & 7) == 0;
  for (int item = threadIdx.x; item < NA * MT * 64; item += 64 * KW) {
    const int ab = item >> 6;
    const int l = item & 63;
    f32x4 sum = red[0][ab][l];
#pragma unroll
    for (int w = 1; w < KW; ++w) sum += red[w][ab][l];
    const int a = ab / MT, b = ab % MT;
    const int m = 16 * b + (l & 15);
    const int n = n_block + 16 * a + 4 * (l >> 4);
    if (m >= M || n >= N) continue;
    uint16_t* out = y + (int64_t)m * ldy + n;
    if (n + 4 <= N && yvec) {
      const float4 sc = *reinterpret_cast<const float4*>(s + n);
      const uint2 v = make_uint2(pack_bf16x2(sum[0] * sc.x, sum[1] * sc.y),
                                 pack_bf16x2(sum[2] * sc.z, sum[3] * sc.w));
      *reinterpret_cast<uint2*>(out) = v;
    } else {
      for (int r = 0; r < 4 && n + r < N; ++r) out[r] = f32_to_bf16(sum[r] * s[n + r]);
    }
  }
}

// KW depends only on (N, K) so that a row's summation order never changes with M.
static int decode_waves(int64_t N, int64_t K) {
  const int64_t blocks = (N + 15) / 16;
  if (K >= 8192 || blocks <= 512) return 8;
  return 4;
}

template <int MT>
static int launch_decode_mt(const uint16_t* x, int64_t ldx, const int8_t* q, const float* s,
                            uint16_t* y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                            hipStream_t stream) {
  constexpr int NA = 1;
  // Prefetch depth (supersteps in flight per buffer). It shapes only the pipelining; the
  // order in which a wave accumulates its supersteps is the same for every U.
  constexpr int U = MT == 1 ? 4 : MT == 2 ? 2 : 1;
  const dim3 grid((unsigned)((N + 16 * NA - 1) / (16 * NA)));
  if (decode_waves(N, K) == 8) {
    hipLaunchKernelGGL((w8a16_decode_kernel<MT, NA, 8, U>), grid, dim3(512), 0, stream, x, ldx, q,
                       s, y, ldy, (int)M, (int)N, (int)K);
  } else {
    hipLaunchKernelGGL((w8a16_decode_kernel<MT, NA, 4, U>), grid, dim3(256), 0, stream, x, ldx, q,
                       s, y, ldy, (int)M, (int)N, (int)K);
  }
  return launch_status();
}

int launch_w8a16_decode(const uint16_t* x, int64_t ldx, const int8_t* q, const float* s,
                        uint16_t* y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                        hipStream_t stream) {
  switch ((M + 15) / 16) {
    case 1: return launch_decode_mt<1>(x, ldx, q, s, y, ldy, M, N, K, stream);
    case 2: return launch_decode_mt<2>(x, ldx, q, s, y, ldy, M, N, K, stream);
    case 3: return launch_decode_mt<3>(x, ldx, q, s, y, ldy, M, N, K, stream);
    case 4: return launch_decode_mt<4>(x, ldx, q, s, y, ldy, M, N, K, stream);
    default: return LSE_E_ALGO;
  }
}

}  // namespace lse
