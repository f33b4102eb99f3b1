// Device-side building blocks shared by the gfx950 kernels of the int8 Linear path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "lse_int8.h"

namespace lse {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

// Sixteen int8 weights (one 128-bit load) → two bf16x8 MFMA operands. Every |q| <= 127 has at
// most 7 significant bits, so int8 → fp32 → bf16 is exact. gfx950 does this in 1.5 VALU ops
// per weight: a sign-extending byte-select convert (v_cvt_f32_i32 with SDWA) per byte and a
// two-lane pack (v_cvt_pk_bf16_f32) per pair.
__device__ __forceinline__ void dequant16(uint4 w, bf16x8& lo, bf16x8& hi) {
  f32x8 a, b;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    a[i] = (float)(int8_t)(w.x >> (8 * i));
    a[4 + i] = (float)(int8_t)(w.y >> (8 * i));
    b[i] = (float)(int8_t)(w.z >> (8 * i));
    b[4 + i] = (float)(int8_t)(w.w >> (8 * i));
  }
  lo = __builtin_convertvector(a, bf16x8);
  hi = __builtin_convertvector(b, bf16x8);
}

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

// D(16x16 fp32) += A(16x32 bf16) · B(32x16 bf16). Lane l supplies A row l%16 and B column
// l%16, each as 8 values of the 32-long contraction; lanes with equal l/16 supply matching
// slices. D lands as rows 4*(l/16)+r, r = 0..3, of column l%16.
__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// fp32 → bf16 bits, round-to-nearest-even (the hardware pack instruction rounds RNE).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __builtin_bit_cast(float, (uint32_t)b << 16);
}

// Raw buffer resource (gfx9 descriptor: base, byte count, dword3 = 0x00020000). A buffer load
// whose byte offset lies at or past the byte count returns zeros and issues no memory request;
// the kernels use this for every ragged edge instead of branching around loads.
typedef __amdgpu_buffer_rsrc_t BufferRsrc;
constexpr uint32_t kOutOfRange = 0x80000000u;  // past every resource (byte counts < 2^31)

__device__ __forceinline__ BufferRsrc make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

__device__ __forceinline__ uint4 buffer_load16(BufferRsrc r, uint32_t byte_offset) {
  typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_offset, 0, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}

__device__ __forceinline__ i32x4 mfma_i8(uint4 a, uint4 b, i32x4 c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4, a),
                                               __builtin_bit_cast(i32x4, b), c, 0, 0, 0);
}

// Packed weight layout. The (N, K) int8 matrix is cut into tiles of 16 rows x 64 K-bytes; tile
// (rb, j) is 1024 contiguous bytes at ((rb * nsteps) + j) * 1024, nsteps = ceil(K / 64), and its
// byte 16 * l + i holds q[16 * rb + l % 16][64 * j + 16 * (l / 16) + i] (zero past N or K). One
// 128-bit load per lane of a wave reads one whole tile, already in MFMA operand order: lane l
// holds 16 K-consecutive bytes of row l % 16.
constexpr int kTileRows = 16;
constexpr int kTileK = 64;
constexpr int kTileBytes = 1024;

__host__ __device__ constexpr int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Workgroups of `kernel` (launched with `threads` threads and `dyn_lds` bytes of dynamic LDS)
// that fit on the current device at once: CU count x resident workgroups per CU. Persistent
// kernels size their grid with it. Cached per (device, kernel, dyn_lds); host-side queries only,
// so it is safe during stream capture.
int persistent_blocks(const void* kernel, int threads, size_t dyn_lds = 0);

inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? LSE_OK : (int)e;
}

}  // namespace lse
