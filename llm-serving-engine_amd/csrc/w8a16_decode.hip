// W8A16 decode kernel (M <= 64): y[m,n] = bf16(s[n] * sum_k x[m,k] q[n,k]).
//
// HBM-bound: every weight byte is read once, so the kernel is a weight stream with the
// arithmetic hidden under it.
//  * A "row block" is 16 weight rows. A workgroup of KW = 16 waves owns row blocks blockIdx.x,
//    blockIdx.x + gridDim.x, ...; the grid is sized to the CUs (persistent workgroups), so a
//    wave's load stream runs on from one row block into the next without draining.
//  * Inside a row block, wave w owns the 64-wide K "supersteps" w, w+KW, w+2KW, ..., so at any
//    moment a workgroup reads one contiguous 64*KW-byte run of each of its rows.
//  * Lane l reads 16 bytes (one buffer_load_dwordx4) of row l%16 at byte 16*(l/16) of each
//    superstep: a wave load covers 16 rows x 64 bytes.
//  * Those 16 int8 → two bf16x8 A operands; x supplies the matching B operands (16 bf16 of
//    token 16*b + l%16), and two v_mfma_f32_16x16x32_bf16 per B tile accumulate fp32 into two
//    independent accumulators (the second MFMA does not wait on the first). Tokens m >= M
//    contribute nothing to stored outputs, so M in 1..16 costs one B tile.
//  * When x (M x K bf16) fits, the workgroup copies it to LDS once and the MFMA B operands come
//    from LDS: the load stream is then weights only. Otherwise x rides in the ring next to the
//    weights.
//  * All global loads are range-checked buffer loads: rows past N, tokens past M, the K tail
//    and the ring's steps past the wave's work read zeros without touching memory. Every step
//    issues the same loads, and a ring of D register stages keeps D-1 supersteps of loads in
//    flight behind static wait counts. The stage that holds a row block's last superstep also
//    brings that block's scales s[n].
//  * At the end of a row block the per-wave partial sums are added in LDS in wave order
//    0..KW-1 (double-buffered, one barrier per block), scaled by s[n] and rounded to bf16.
//    No atomics: each output's summation order depends only on K, never on M, N or the grid.
#include <algorithm>

#include "lse_common.h"

namespace lse {

constexpr int kDecodeWaves = 16;
constexpr int kDecodeXLdsBytes = 80 * 1024;  // x staged in LDS up to this size

template <int MT, bool XLDS>
struct DecodeStage {
  uint4 w;
  uint4 x[XLDS ? 1 : MT][2];
  uint4 sc;  // float4 scales of this lane's epilogue columns (last superstep of a block only)
};

// Row pitch of x in LDS: 16 bytes of padding shift consecutive rows by four banks, so the 16
// rows a wave reads at one k land in distinct banks.
__host__ __device__ constexpr uint32_t x_lds_pitch(int K) { return 2u * K + 16u; }

template <int MT, int KW, int D, bool XLDS>
__global__ void __launch_bounds__(64 * KW)
w8a16_decode_kernel(const uint16_t* __restrict__ x, int64_t ldx, const int8_t* __restrict__ q,
                    const float* __restrict__ s, uint16_t* __restrict__ y, int64_t ldy, int M,
                    int N, int K) {
  __shared__ f32x4 red[2][KW][MT][64];
  extern __shared__ __attribute__((aligned(16))) unsigned char x_lds[];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r16 = lane & 15;
  const int g = lane >> 4;
  const int nrb = (N + 15) >> 4;
  const int G = gridDim.x;

  // All of q (N*K bytes); rows past N read zeros. Row block rb starts at byte 16*K*rb.
  const BufferRsrc qres = make_rsrc(q, (uint32_t)N * (uint32_t)K);
  const uint32_t q_lane = (uint32_t)r16 * K + 16 * g;
  const BufferRsrc sres = make_rsrc(s, (uint32_t)N * 4);
  // Activation rows 0..M-1; tokens m >= M read zeros.
  const BufferRsrc xres = make_rsrc(x, (uint32_t)(((int64_t)(M - 1) * ldx + K) * 2));
  uint32_t x_lane[MT];
#pragma unroll
  for (int b = 0; b < MT; ++b) {
    const int m = 16 * b + r16;
    x_lane[b] = m < M ? (uint32_t)(m * ldx + 16 * g) * 2 : kOutOfRange;
  }
  const uint32_t pitch = x_lds_pitch(K);
  // LDS row read by this lane: tokens past M re-read row M-1 (their outputs are not stored).
  const uint32_t x_lds_row = (uint32_t)min(r16, M - 1) * pitch;

  // x staged to LDS (XLDS): each thread fetches up to kXChunks 16-byte chunks of x before the
  // weight ring starts, and stores them to LDS after the ring's first loads are in flight, so
  // the copy's latency overlaps the first weight loads instead of preceding them.
  constexpr int kXChunks = XLDS ? (kDecodeXLdsBytes / 16 + 64 * KW - 1) / (64 * KW) : 1;
  uint4 xstage[kXChunks];
  const int chunks_per_row = K >> 3;
  if constexpr (XLDS) {
#pragma unroll
    for (int i = 0; i < kXChunks; ++i) {
      const int c = threadIdx.x + 64 * KW * i;
      const int m = c / chunks_per_row, kc = c - m * chunks_per_row;
      xstage[i] = buffer_load16(xres, m < M ? (uint32_t)(m * ldx + 8 * kc) * 2 : kOutOfRange);
    }
  }
  auto store_x_to_lds = [&]() {
    if constexpr (XLDS) {
#pragma unroll
      for (int i = 0; i < kXChunks; ++i) {
        const int c = threadIdx.x + 64 * KW * i;
        const int m = c / chunks_per_row, kc = c - m * chunks_per_row;
        if (m < M) *reinterpret_cast<uint4*>(x_lds + m * pitch + 16 * kc) = xstage[i];
      }
      __syncthreads();
    }
  };

  const int nsteps = (K + 63) >> 6;
  const int mine = nsteps > wave ? (nsteps - wave + KW - 1) / KW : 0;
  const int my_blocks = blockIdx.x < nrb ? (nrb - 1 - blockIdx.x) / G + 1 : 0;

  // Load cursor (row block, superstep index of this wave) of the next stage to fill.
  int lrb = blockIdx.x, lj = 0;
  auto load = [&](DecodeStage<MT, XLDS>& r) {
    const int kb = 64 * (wave + KW * lj);  // superstep start, in elements
    const bool ok = lrb < nrb && kb + 16 * g < K;
    const uint32_t rb_bytes = (uint32_t)lrb * 16u * (uint32_t)K;
    r.w = buffer_load16(qres, ok ? rb_bytes + q_lane + (uint32_t)kb : kOutOfRange);
    if constexpr (!XLDS) {
#pragma unroll
      for (int b = 0; b < MT; ++b) {
        const uint32_t off = ok ? x_lane[b] + (uint32_t)(2 * kb) : kOutOfRange;
        r.x[b][0] = buffer_load16(xres, off);
        r.x[b][1] = buffer_load16(xres, off + 16);
      }
    }
    const bool last = lj == mine - 1 && lrb < nrb;
    r.sc = buffer_load16(sres, last ? (uint32_t)(64 * lrb + 16 * g) : kOutOfRange);
    if (++lj == mine) {
      lj = 0;
      lrb += G;
    }
  };

  // One token tile (M <= 16) keeps two accumulators so its two MFMAs per superstep do not
  // wait on each other; wider M tiles have independent chains across tiles already and spend
  // the registers on the ring instead.
  constexpr int NACC = MT == 1 ? 2 : 1;
  f32x4 acc[MT][NACC];
#pragma unroll
  for (int b = 0; b < MT; ++b)
#pragma unroll
    for (int a = 0; a < NACC; ++a) acc[b][a] = f32x4{0.f, 0.f, 0.f, 0.f};
  // cj: this wave's superstep index within the current row block (selects x in LDS).
  auto compute = [&](const DecodeStage<MT, XLDS>& r, int cj) {
    bf16x8 lo, hi;
    if constexpr (XLDS) {
      // Lanes past the K tail read an in-row address and use zeros (their weights are zero
      // too, but a zero operand keeps 0 * inf out of the sum).
      const int kb = 64 * (wave + KW * cj) + 16 * g;
      const bool kv = kb < K;
      const unsigned char* p = x_lds + x_lds_row + 2u * (kv ? kb : 0);
      uint4 x0 = *reinterpret_cast<const uint4*>(p);
      uint4 x1 = *reinterpret_cast<const uint4*>(p + 16);
      if (!kv) x0 = x1 = make_uint4(0, 0, 0, 0);
      dequant16(r.w, lo, hi);
      acc[0][0] = mfma16x16x32(lo, as_bf16x8(x0), acc[0][0]);
      acc[0][1] = mfma16x16x32(hi, as_bf16x8(x1), acc[0][1]);
    } else {
      dequant16(r.w, lo, hi);
#pragma unroll
      for (int b = 0; b < MT; ++b) {
        acc[b][0] = mfma16x16x32(lo, as_bf16x8(r.x[b][0]), acc[b][0]);
        acc[b][NACC - 1] = mfma16x16x32(hi, as_bf16x8(r.x[b][1]), acc[b][NACC - 1]);
      }
    }
  };

  const bool yvec = (ldy & 3) == 0 && ((uintptr_t)y & 7) == 0;
  int par = 0;
  // Row block crb is complete in every wave: reduce in wave order, scale, store.
  auto finish_block = [&](int crb, const uint4& sc_bits) {
#pragma unroll
    for (int b = 0; b < MT; ++b) {
      red[par][wave][b][lane] = NACC == 2 ? acc[b][0] + acc[b][NACC - 1] : acc[b][0];
#pragma unroll
      for (int a = 0; a < NACC; ++a) acc[b][a] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    __syncthreads();
    if (threadIdx.x < MT * 64) {
      const int b = threadIdx.x >> 6;
      // Partials are read four at a time before they are added, so the LDS reads overlap; the
      // sum still runs in wave order.
      f32x4 sum = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int w0 = 0; w0 < KW; w0 += 4) {
        f32x4 part[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) part[i] = red[par][w0 + i][b][lane];
#pragma unroll
        for (int i = 0; i < 4; ++i) sum = (w0 + i == 0) ? part[0] : sum + part[i];
      }
      const int m = 16 * b + r16;
      const int n = 16 * crb + 4 * g;
      if (m < M && n < N) {
        uint16_t* out = y + (int64_t)m * ldy + n;
        if (n + 4 <= N) {
          const float4 sc = __builtin_bit_cast(float4, sc_bits);
          const float o[4] = {sum[0] * sc.x, sum[1] * sc.y, sum[2] * sc.z, sum[3] * sc.w};
          if (yvec) {
            *reinterpret_cast<uint2*>(out) =
                make_uint2(pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]));
          } else {
            for (int r = 0; r < 4; ++r) out[r] = f32_to_bf16(o[r]);
          }
        } else {
          // The last columns of a ragged N: the prefetched float4 of scales straddles N.
          for (int r = 0; n + r < N; ++r) out[r] = f32_to_bf16(sum[r] * s[n + r]);
        }
      }
    }
    par ^= 1;
  };

  if (mine > 0) {
    // Compute cursor. Every wave of the workgroup finishes the same row blocks in the same
    // order, so the barriers inside finish_block pair up across waves.
    int crb = blockIdx.x, cj = 0;
    const int items = my_blocks * mine;
    DecodeStage<MT, XLDS> ring[D];
#pragma unroll
    for (int u = 0; u < D - 1; ++u) {
      load(ring[u]);
      __builtin_amdgcn_sched_barrier(0);  // issue in ring order: slot 0 is consumed first
    }
    store_x_to_lds();
    for (int t0 = 0; t0 < items; t0 += D) {
#pragma unroll
      for (int u = 0; u < D; ++u) {
        load(ring[(u + D - 1) % D]);
        __builtin_amdgcn_sched_barrier(0);
        compute(ring[u], cj);
        // Keep the stages in program order: hoisting a later stage's conversion would wait
        // on its loads and drain the ring.
        __builtin_amdgcn_sched_barrier(0);
        if (t0 + u < items && ++cj == mine) {
          finish_block(crb, ring[u].sc);
          cj = 0;
          crb += G;
        }
      }
    }
  } else {
    // A wave with no supersteps (K < 64*KW) still takes part in every block's reduction and
    // stores its M tile, with scales loaded directly (it has no ring stage to carry them).
    store_x_to_lds();
    for (int i = 0; i < my_blocks; ++i) {
      const int crb = blockIdx.x + i * G;
      finish_block(crb, buffer_load16(sres, (uint32_t)(64 * crb + 16 * g)));
    }
  }
}

template <int MT, bool XLDS>
static int launch_decode(const uint16_t* x, int64_t ldx, const int8_t* q, const float* s,
                         uint16_t* y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                         hipStream_t stream) {
  // Ring depth: supersteps in flight per wave. It shapes only the pipelining; the order in which
  // a wave accumulates its supersteps is the same for every D.
  constexpr int D = MT == 1 ? 4 : MT == 2 ? 3 : 2;
  constexpr int KW = kDecodeWaves;
  auto kernel = w8a16_decode_kernel<MT, KW, D, XLDS>;
  const size_t lds = XLDS ? (size_t)M * x_lds_pitch((int)K) : 0;
  const int64_t nrb = (N + 15) / 16;
  const int64_t grid =
      std::min<int64_t>(nrb, persistent_blocks((const void*)kernel, 64 * KW, lds));
  hipLaunchKernelGGL(kernel, dim3((unsigned)grid), dim3(64 * KW), lds, stream, x, ldx, q, s, y,
                     ldy, (int)M, (int)N, (int)K);
  return launch_status();
}

int launch_w8a16_decode(const uint16_t* x, int64_t ldx, const int8_t* q, const float* s,
                        uint16_t* y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                        hipStream_t stream) {
  if (M <= 16 && (size_t)M * x_lds_pitch((int)K) <= (size_t)kDecodeXLdsBytes)
    return launch_decode<1, true>(x, ldx, q, s, y, ldy, M, N, K, stream);
  switch ((M + 15) / 16) {
    case 1: return launch_decode<1, false>(x, ldx, q, s, y, ldy, M, N, K, stream);
    case 2: return launch_decode<2, false>(x, ldx, q, s, y, ldy, M, N, K, stream);
    case 3: return launch_decode<3, false>(x, ldx, q, s, y, ldy, M, N, K, stream);
    case 4: return launch_decode<4, false>(x, ldx, q, s, y, ldy, M, N, K, stream);
    default: return LSE_E_ALGO;
  }
}

}  // namespace lse
