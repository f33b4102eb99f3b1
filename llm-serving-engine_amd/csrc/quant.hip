// Row-wise symmetric int8 quantizers: per output channel for weights (load time) and per
// token for activations (W8A8 first stage). Both compute, per row r,
//   scale[r] = fl32(amax_r / 127)   (IEEE division; an all-zero row gets scale 1)
//   out[r,k] = clamp(rne(fl32(v[r,k] / scale[r])), -127, 127)
// with the correctly rounded fp32 division HIP compiles `/` to, so results are bit-exact
// against any IEEE implementation of the same formula.
#include "lse_common.h"

namespace lse {

constexpr int kQuantThreads = 256;

__device__ __forceinline__ float block_max(float v, float* red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  float m = red[0];
#pragma unroll
  for (int w = 1; w < kQuantThreads / 64; ++w) m = fmaxf(m, red[w]);
  return m;
}


// Eight bf16 values (four packed pairs, low half first) quantized by `q` into eight int8 bytes.
template <typename Q>
__device__ __forceinline__ uint2 quant8(const uint32_t (&u)[4], Q q) {
  uint32_t packed[2] = {0, 0};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t lo = (uint8_t)q(__builtin_bit_cast(float, u[j] << 16));
    const uint32_t hi = (uint8_t)q(__builtin_bit_cast(float, u[j] & 0xffff0000u));
    packed[j >> 1] |= (lo | (hi << 8)) << (16 * (j & 1));
  }
  return make_uint2(packed[0], packed[1]);
}

// One workgroup per weight row; fp32 input read twice (the second pass hits L2).
__global__ void __launch_bounds__(kQuantThreads)
quantize_weight_rows(const float* __restrict__ w, int64_t ldw, int8_t* __restrict__ q,
                     float* __restrict__ s, int K) {
  __shared__ float red[kQuantThreads / 64];
  const int64_t n = blockIdx.x;
  const float* row = w + n * ldw;
  float amax = 0.0f;
  for (int k = threadIdx.x * 4; k < K; k += kQuantThreads * 4) {
    const float4 v = *reinterpret_cast<const float4*>(row + k);
    amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
  }
  const float scale = row_scale(block_max(amax, red));
  if (threadIdx.x == 0) s[n] = scale;
  int8_t* out = q + n * K;
  for (int k = threadIdx.x * 4; k < K; k += kQuantThreads * 4) {
    const float4 v = *reinterpret_cast<const float4*>(row + k);
    const uint32_t packed = (uint32_t)(uint8_t)quant1(v.x, scale) |
                            ((uint32_t)(uint8_t)quant1(v.y, scale) << 8) |
                            ((uint32_t)(uint8_t)quant1(v.z, scale) << 16) |
                            ((uint32_t)(uint8_t)quant1(v.w, scale) << 24);
    *reinterpret_cast<uint32_t*>(out + k) = packed;
  }
}

// One workgroup per token; bf16 input read twice (the second pass hits L2). Rows longer than 16384
// elements; shorter ones take quantize_act_rows_reg.
__global__ void __launch_bounds__(kQuantThreads)
quantize_act_rows(const uint16_t* __restrict__ x, int64_t ldx, int8_t* __restrict__ xq,
                  float* __restrict__ sx, int K) {
  __shared__ float red[kQuantThreads / 64];
  const int64_t m = blockIdx.x;
  const uint16_t* row = x + m * ldx;
  float amax = 0.0f;
  for (int k = threadIdx.x * 8; k < K; k += kQuantThreads * 8) {
    const uint4 v = *reinterpret_cast<const uint4*>(row + k);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      amax = fmaxf(amax, fabsf(__builtin_bit_cast(float, w[i] << 16)));
      amax = fmaxf(amax, fabsf(__builtin_bit_cast(float, w[i] & 0xffff0000u)));
    }
  }
  const float scale = row_scale(block_max(amax, red));
  if (threadIdx.x == 0) sx[m] = scale;
  int8_t* out = xq + m * K;
  with_row_quantizer(scale, [&](auto q) {
    for (int k = threadIdx.x * 8; k < K; k += kQuantThreads * 8) {
      const uint4 v = *reinterpret_cast<const uint4*>(row + k);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
      *reinterpret_cast<uint2*>(out + k) = quant8(w, q);
    }
  });
}

__device__ __forceinline__ float block_sum(float v, float* red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  const int wave = threadIdx.x >> 6;
  __syncthreads();  // red may still be read by an earlier reduction
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  float t = red[0];
#pragma unroll
  for (int w = 1; w < kQuantThreads / 64; ++w) t += red[w];
  return t;
}

// RMSNorm of one token row followed by its per-token quantization (W8A8 first stage fused into
// the decoder's input_layernorm / post_attention_layernorm). With the rounding steps of
// transformers' LlamaRMSNorm (modeling_llama.py:62-67: fp32 variance, x * rsqrt(var + eps)
// rounded to bf16, times the bf16 weight rounded to bf16):
//   r = 1 / sqrt(fl32(sum_k x^2 / K) + eps),  h_k = bf16(w_k * bf16(x_k * r))
// then sx = fl32(amax_k |h_k| / 127) and xq_k = clamp(rne(h_k / sx), -127, 127), exactly as
// quantize_act_rows does for an existing bf16 row. One workgroup per token; the row is read three
// times (sum of squares, amax, quantize), the last two from L2 (rows longer than 16384 elements;
// shorter ones take rmsnorm_quant_rows_reg). `normed` (optional) receives h.
__device__ __forceinline__ float rms_h(uint32_t xb, uint32_t wb, float r) {
  const float x = __builtin_bit_cast(float, xb);
  const float h = bf16_to_f32(f32_to_bf16(x * r));
  return bf16_to_f32(f32_to_bf16(__builtin_bit_cast(float, wb) * h));
}

__global__ void __launch_bounds__(kQuantThreads)
rmsnorm_quant_rows(const uint16_t* __restrict__ x, int64_t ldx, const uint16_t* __restrict__ w,
                   float eps, int8_t* __restrict__ xq, float* __restrict__ sx,
                   uint16_t* __restrict__ normed, int K) {
  __shared__ float red[kQuantThreads / 64];
  const int64_t m = blockIdx.x;
  const uint16_t* row = x + m * ldx;
  float ss = 0.0f;
  for (int k = threadIdx.x * 8; k < K; k += kQuantThreads * 8) {
    const uint4 v = *reinterpret_cast<const uint4*>(row + k);
    const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a = __builtin_bit_cast(float, u[i] << 16);
      const float b = __builtin_bit_cast(float, u[i] & 0xffff0000u);
      ss = __builtin_fmaf(a, a, ss);
      ss = __builtin_fmaf(b, b, ss);
    }
  }
  const float var = block_sum(ss, red) / (float)K;
  const float r = 1.0f / __builtin_sqrtf(var + eps);
  float amax = 0.0f;
  for (int k = threadIdx.x * 8; k < K; k += kQuantThreads * 8) {
    const uint4 v = *reinterpret_cast<const uint4*>(row + k);
    const uint4 g = *reinterpret_cast<const uint4*>(w + k);
    const uint32_t u[4] = {v.x, v.y, v.z, v.w}, gw[4] = {g.x, g.y, g.z, g.w};
    uint32_t hb[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float lo = rms_h(u[i] << 16, gw[i] << 16, r);
      const float hi = rms_h(u[i] & 0xffff0000u, gw[i] & 0xffff0000u, r);
      amax = fmaxf(amax, fmaxf(fabsf(lo), fabsf(hi)));
      hb[i] = pack_bf16x2(lo, hi);
    }
    if (normed) *reinterpret_cast<uint4*>(normed + m * K + k) = make_uint4(hb[0], hb[1], hb[2], hb[3]);
  }
  __syncthreads();  // the sum's reads of red are done before block_max writes it
  const float scale = row_scale(block_max(amax, red));
  if (threadIdx.x == 0) sx[m] = scale;
  int8_t* out = xq + m * K;
  with_row_quantizer(scale, [&](auto q) {
    for (int k = threadIdx.x * 8; k < K; k += kQuantThreads * 8) {
      const uint4 v = *reinterpret_cast<const uint4*>(row + k);
      const uint4 g = *reinterpret_cast<const uint4*>(w + k);
      const uint32_t u[4] = {v.x, v.y, v.z, v.w}, gw[4] = {g.x, g.y, g.z, g.w};
      uint32_t hb[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        hb[i] = pack_bf16x2(rms_h(u[i] << 16, gw[i] << 16, r),
                            rms_h(u[i] & 0xffff0000u, gw[i] & 0xffff0000u, r));
      *reinterpret_cast<uint2*>(out + k) = quant8(hb, q);
    }
  });
}

// The same for rows of at most NV x 2048 elements (hidden sizes up to 16384): thread t keeps
// elements 8 t + 2048 i (i < NV) of x and of the weight in registers, so the row is read once and
// the normed row is quantized from registers. Slots past K hold zeros, which add exact zeros to
// the sum of squares and to nothing else; the arithmetic and every order of summation are those
// of rmsnorm_quant_rows, so the results are bit-identical.
template <int NV>
__global__ void __launch_bounds__(kQuantThreads)
rmsnorm_quant_rows_reg(const uint16_t* __restrict__ x, int64_t ldx, const uint16_t* __restrict__ w,
                       float eps, int8_t* __restrict__ xq, float* __restrict__ sx,
                       uint16_t* __restrict__ normed, int K) {
  __shared__ float red[kQuantThreads / 64];
  const int64_t m = blockIdx.x;
  const uint16_t* row = x + m * ldx;
  uint32_t u[NV][4], gw[NV][4];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int k = threadIdx.x * 8 + kQuantThreads * 8 * i;
    const uint4 v = k < K ? *reinterpret_cast<const uint4*>(row + k) : make_uint4(0, 0, 0, 0);
    const uint4 g = k < K ? *reinterpret_cast<const uint4*>(w + k) : make_uint4(0, 0, 0, 0);
    u[i][0] = v.x, u[i][1] = v.y, u[i][2] = v.z, u[i][3] = v.w;
    gw[i][0] = g.x, gw[i][1] = g.y, gw[i][2] = g.z, gw[i][3] = g.w;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float a = __builtin_bit_cast(float, u[i][j] << 16);
      const float b = __builtin_bit_cast(float, u[i][j] & 0xffff0000u);
      ss = __builtin_fmaf(a, a, ss);
      ss = __builtin_fmaf(b, b, ss);
    }
  }
  const float var = block_sum(ss, red) / (float)K;
  const float r = 1.0f / __builtin_sqrtf(var + eps);
  float amax = 0.0f;
  uint32_t hb[NV][4];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int k = threadIdx.x * 8 + kQuantThreads * 8 * i;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float lo = rms_h(u[i][j] << 16, gw[i][j] << 16, r);
      const float hi = rms_h(u[i][j] & 0xffff0000u, gw[i][j] & 0xffff0000u, r);
      amax = fmaxf(amax, fmaxf(fabsf(lo), fabsf(hi)));
      hb[i][j] = pack_bf16x2(lo, hi);
    }
    if (normed && k < K)
      *reinterpret_cast<uint4*>(normed + m * K + k) = make_uint4(hb[i][0], hb[i][1], hb[i][2], hb[i][3]);
  }
  __syncthreads();  // the sum's reads of red are done before block_max writes it
  const float scale = row_scale(block_max(amax, red));
  if (threadIdx.x == 0) sx[m] = scale;
  int8_t* out = xq + m * K;
  with_row_quantizer(scale, [&](auto q) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int k = threadIdx.x * 8 + kQuantThreads * 8 * i;
      if (k < K) *reinterpret_cast<uint2*>(out + k) = quant8(hb[i], q);
    }
  });
}

int launch_rmsnorm_quantize(const uint16_t* x, int64_t ldx, const uint16_t* w, float eps,
                            int8_t* xq, float* sx, uint16_t* normed, int64_t M, int64_t K,
                            hipStream_t stream) {
  constexpr int64_t kRow = kQuantThreads * 8;  // elements per register slot of a row
  const dim3 grid((unsigned)M), block(kQuantThreads);
  if (K <= kRow)
    hipLaunchKernelGGL(rmsnorm_quant_rows_reg<1>, grid, block, 0, stream, x, ldx, w, eps, xq, sx,
                       normed, (int)K);
  else if (K <= 2 * kRow)
    hipLaunchKernelGGL(rmsnorm_quant_rows_reg<2>, grid, block, 0, stream, x, ldx, w, eps, xq, sx,
                       normed, (int)K);
  else if (K <= 4 * kRow)
    hipLaunchKernelGGL(rmsnorm_quant_rows_reg<4>, grid, block, 0, stream, x, ldx, w, eps, xq, sx,
                       normed, (int)K);
  else if (K <= 8 * kRow)
    hipLaunchKernelGGL(rmsnorm_quant_rows_reg<8>, grid, block, 0, stream, x, ldx, w, eps, xq, sx,
                       normed, (int)K);
  else
    hipLaunchKernelGGL(rmsnorm_quant_rows, grid, block, 0, stream, x, ldx, w, eps, xq, sx, normed,
                       (int)K);
  return launch_status();
}

int launch_quantize_weight(const float* w, int64_t ldw, int8_t* q, float* s, int64_t N, int64_t K,
                           hipStream_t stream) {
  hipLaunchKernelGGL(quantize_weight_rows, dim3((unsigned)N), dim3(kQuantThreads), 0, stream, w,
                     ldw, q, s, (int)K);
  return launch_status();
}

// The same for rows of at most NV x 2048 elements: thread t keeps elements 8 t + 2048 i (i < NV)
// in registers, so the row is read once. The row maximum is order-independent and each element's
// quantization is the same expression, so the results are bit-identical to quantize_act_rows.
template <int NV>
__global__ void __launch_bounds__(kQuantThreads)
quantize_act_rows_reg(const uint16_t* __restrict__ x, int64_t ldx, int8_t* __restrict__ xq,
                      float* __restrict__ sx, int K) {
  __shared__ float red[kQuantThreads / 64];
  const int64_t m = blockIdx.x;
  const uint16_t* row = x + m * ldx;
  uint32_t u[NV][4];
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int k = threadIdx.x * 8 + kQuantThreads * 8 * i;
    const uint4 v = k < K ? *reinterpret_cast<const uint4*>(row + k) : make_uint4(0, 0, 0, 0);
    u[i][0] = v.x, u[i][1] = v.y, u[i][2] = v.z, u[i][3] = v.w;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      amax = fmaxf(amax, fabsf(__builtin_bit_cast(float, u[i][j] << 16)));
      amax = fmaxf(amax, fabsf(__builtin_bit_cast(float, u[i][j] & 0xffff0000u)));
    }
  }
  const float scale = row_scale(block_max(amax, red));
  if (threadIdx.x == 0) sx[m] = scale;
  int8_t* out = xq + m * K;
  with_row_quantizer(scale, [&](auto q) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int k = threadIdx.x * 8 + kQuantThreads * 8 * i;
      if (k < K) *reinterpret_cast<uint2*>(out + k) = quant8(u[i], q);
    }
  });
}

int launch_quantize_act(const uint16_t* x, int64_t ldx, int8_t* xq, float* sx, int64_t M,
                        int64_t K, hipStream_t stream) {
  constexpr int64_t kRow = kQuantThreads * 8;  // elements per register slot of a row
  const dim3 grid((unsigned)M), block(kQuantThreads);
  if (K <= kRow)
    hipLaunchKernelGGL(quantize_act_rows_reg<1>, grid, block, 0, stream, x, ldx, xq, sx, (int)K);
  else if (K <= 2 * kRow)
    hipLaunchKernelGGL(quantize_act_rows_reg<2>, grid, block, 0, stream, x, ldx, xq, sx, (int)K);
  else if (K <= 4 * kRow)
    hipLaunchKernelGGL(quantize_act_rows_reg<4>, grid, block, 0, stream, x, ldx, xq, sx, (int)K);
  else if (K <= 8 * kRow)
    hipLaunchKernelGGL(quantize_act_rows_reg<8>, grid, block, 0, stream, x, ldx, xq, sx, (int)K);
  else
    hipLaunchKernelGGL(quantize_act_rows, grid, block, 0, stream, x, ldx, xq, sx, (int)K);
  return launch_status();
}

}  // namespace lse
