// Device-side building blocks shared by the gfx950 kernels of the int8 Linear path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

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

// XOR swizzle of the 16-byte chunks of a 128-byte bf16 activation row in LDS (64 bf16, one K
// step): chunk c of row r is stored at c ^ bf16_row_swz(r). Fragment reads of 16 consecutive rows
// at one chunk offset then hit no LDS bank twice (measured on MI355X with SQ_LDS_BANK_CONFLICT).
__host__ __device__ constexpr int bf16_row_swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

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

// Cache policy of a buffer load (the instruction's cache-policy bits): kLoadDefault, or
// kLoadStream (nt) for data read once per call, such as decode weights, so the stream does not
// claim cache lines that reused data (activations, scales) need.
constexpr int kLoadDefault = 0;
constexpr int kLoadStream = 2;

// A 16-byte global load with the streaming (nt) cache policy.
__device__ __forceinline__ uint4 load16_stream(const void* p) {
  typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 v = __builtin_nontemporal_load(static_cast<const u32x4*>(p));
  return make_uint4(v[0], v[1], v[2], v[3]);
}

template <int POLICY = kLoadDefault>
__device__ __forceinline__ uint4 buffer_load16(BufferRsrc r, uint32_t byte_offset) {
  typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_offset, 0, POLICY);
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
//
// Gate/up layout of the MLP's fused projection (two (I, K) matrices): row tile 2t holds gate rows
// 16t..16t+15 and row tile 2t+1 the same rows of up, so 2 ceil(I/16) row tiles in all; a kernel
// holding an even-aligned pair of row tiles holds matching gate and up rows.
//
// bf16 weight layout (the bf16 lm_head): the same 16-row x 64-K steps, each 2 KB: at byte
// (rb * nsteps + j) * 2048 + 1024 h + 16 l + 2 i lies w[16 rb + l % 16][64 j + 16 (l / 16) +
// 8 h + i] (zero past N and K): tile h = 0 and 1 are the "lo" and "hi" MFMA operands that
// dequantizing an int8 tile of the same step yields.
constexpr int kTileRows = 16;
constexpr int kTileK = 64;
constexpr int kTileBytes = 1024;

__host__ __device__ constexpr int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Four outputs y[m, n..n+cnt) in bf16 (RNE); one aligned 8-byte store when yvec and cnt == 4.
__device__ __forceinline__ void store_bf16x4(uint16_t* y, int64_t ldy, int m, int n, int cnt,
                                             const float (&o)[4], bool yvec) {
  uint16_t* out = y + (int64_t)m * ldy + n;
  if (cnt == 4 && yvec) {
    *reinterpret_cast<uint2*>(out) = make_uint2(pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]));
  } else {
    for (int r = 0; r < cnt; ++r) out[r] = f32_to_bf16(o[r]);
  }
}

// The scaled fp32 value of accumulator element r: W8A16 v * s, W8A8 (v * sx[m]) * s.
template <bool I8, typename Acc>
__device__ __forceinline__ float scaled(Acc v, int r, float sc, float sxm) {
  if constexpr (I8)
    return ((float)v[r] * sxm) * sc;
  else
    return v[r] * sc;
}

// The scaled output of one lane's MFMA result: `v` holds rows n..n+3 (cnt of them valid) of
// token m, `sc` their scales, sxm the token's scale (W8A8). W8A16: y = bf16(v * s[n]); W8A8:
// acc = v (int32, when acc is not null; row stride N), y = bf16((v * sx[m]) * s[n]) (when y is
// not null). yvec: y rows allow an aligned 8-byte store of four outputs.
template <bool I8, typename Acc>
__device__ __forceinline__ void store_out4(uint16_t* y, int64_t ldy, int32_t* acc, int N, int m,
                                           int n, int cnt, Acc v, const float (&sc)[4], float sxm,
                                           bool yvec) {
  float o[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) o[r] = scaled<I8>(v, r, sc[r], sxm);
  if constexpr (I8) {
    if (acc) {
      int32_t* dst = acc + (int64_t)m * N + n;
      if (cnt == 4 && (N & 3) == 0) {
        *reinterpret_cast<i32x4*>(dst) = v;
      } else {
        for (int r = 0; r < cnt; ++r) dst[r] = v[r];
      }
    }
    if (!y) return;
  }
  store_bf16x4(y, ldy, m, n, cnt, o, yvec);
}

// SiLU(v) = v * sigmoid(v) = v / (1 + e^-v) in fp32. e^-v overflows to +inf for v < -88, where
// the quotient is the correctly signed zero; the hardware exponential's few-ulp fp32 error is far
// below the bf16 rounding that follows.
__device__ __forceinline__ float silu(float v) { return v / (1.0f + __expf(-v)); }

// Gate/up epilogue of the fused MLP projection: gate and up accumulators of the same four output
// columns n..n+3 of token m (cnt valid), their scales sg and su. h = bf16(silu(g) * u) with g and
// u scaled in fp32 as store_out4 scales them, rounded once.
template <bool I8, typename Acc>
__device__ __forceinline__ void store_glu4(uint16_t* y, int64_t ldy, int m, int n, int cnt,
                                           Acc vg, Acc vu, const float (&sg)[4],
                                           const float (&su)[4], float sxm, bool yvec) {
  float o[4];
#pragma unroll
  for (int r = 0; r < 4; ++r)
    o[r] = silu(scaled<I8>(vg, r, sg[r], sxm)) * scaled<I8>(vu, r, su[r], sxm);
  store_bf16x4(y, ldy, m, n, cnt, o, yvec);
}

// s_waitcnt immediate that waits for all but the `n` most recent vector-memory operations
// (vmcnt = n, expcnt and lgkmcnt left at their maxima).
__host__ __device__ constexpr int vmcnt_imm(int n) {
  return (n & 15) | 0x70 | 0xF00 | ((n >> 4) << 14);
}

// The same with lgkmcnt = 0: also waits for every LDS read the wave has issued. Before a raw
// s_barrier that releases direct-to-LDS loads into a slot this wave was reading, the reads must
// have completed, not only issued (the compiler may place the barrier above outstanding reads).
__host__ __device__ constexpr int vmcnt_lgkm0_imm(int n) {
  return (n & 15) | 0x70 | ((n >> 4) << 14);
}

typedef __attribute__((address_space(3))) void* LdsPtr;

// Direct-to-LDS 16-byte buffer load: lane l's 16 bytes from `offset` land at lds + 16 l (lds is
// wave-uniform). An offset past the resource writes zeros and issues no memory request.
__device__ __forceinline__ void buffer_load16_lds(BufferRsrc r, void* lds, uint32_t offset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (LdsPtr)lds, 16, offset, 0, 0, 0);
}

// The same load with the buffer descriptor as four dwords, issued from inline assembly. The
// compiler then does not track the LDS write, so it inserts no waits of its own between these
// loads and later LDS reads: the caller orders them with explicit s_waitcnt vmcnt counts and
// barriers (vmcnt drops when the data is in LDS). M0 carries the LDS address and is restored.
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ u32x4 make_rsrc4(const void* base, uint32_t bytes) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  return u32x4{(uint32_t)p, (uint32_t)(p >> 32) & 0xffffu, bytes, 0x00020000u};
}

// LDS byte address of a shared-memory pointer, as a wave-uniform value.
__device__ __forceinline__ uint32_t lds_addr(const void* lds) {
  return __builtin_amdgcn_readfirstlane(
      (uint32_t)(size_t)(__attribute__((address_space(3))) const void*)lds);
}

// One load to LDS byte address base + IMM (+ 16 l for lane l); NT: the streaming (nt) cache
// policy, for data read once per call.
template <int IMM, bool NT = false>
__device__ __forceinline__ void dma16_lds(u32x4 r, uint32_t base, uint32_t offset) {
  uint32_t saved;
  if constexpr (NT) {
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_add_u32 m0, %1, %4\n\t"
        "buffer_load_dwordx4 %2, %3, 0 offen nt lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(base), "v"(offset), "s"(r), "i"(IMM)
        : "memory", "scc");
  } else {
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_add_u32 m0, %1, %4\n\t"
        "buffer_load_dwordx4 %2, %3, 0 offen lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(base), "v"(offset), "s"(r), "i"(IMM)
        : "memory", "scc");
  }
}

// N loads, load i to base + i * STEP, from offsets off[i].
template <int STEP, bool NT = false, int... I>
__device__ __forceinline__ void dma16_lds_seq(u32x4 r, uint32_t base, const uint32_t* off,
                                              std::integer_sequence<int, I...>) {
  (dma16_lds<I * STEP, NT>(r, base, off[I]), ...);
}

// Workgroups of `kernel` (launched with `threads` threads and `dyn_lds` bytes of dynamic LDS)
// that fit on the current device at once: CU count x resident workgroups per CU. Persistent
// kernels size their grid with it. Cached per (device, kernel, dyn_lds); host-side queries only,
// so it is safe during stream capture.
int persistent_blocks(const void* kernel, int threads, size_t dyn_lds = 0);

// Per-token (and per-channel) symmetric int8 quantization, shared by the quantizers and the
// decode kernel's quantizing staging: scale = fl32(amax / 127) (IEEE division; an all-zero row
// gets 1), q = clamp(rne(fl32(v / scale)), -127, 127).
__device__ __forceinline__ float row_scale(float amax) { return amax > 0.0f ? amax / 127.0f : 1.0f; }

// The same quantization of a bf16 value v from the row's reciprocal inv = fl32(1 / scale), for
// scales of at least kQuantRecipMinScale: q0 = fl32(v inv) is within an ulp of v / scale, the
// residual fma(-q0, scale, v) is exact, and fma(residual, inv, q0) is fl32(v / scale) (the
// quotient correction with a correctly rounded reciprocal of P. Markstein, IBM J. Res. Dev.
// 34(1), 1990). Three operations instead of a correctly rounded division per element. Checked
// exhaustively (tests/quant_recip_check.c): for every bf16 amax whose scale is in range and every
// bf16 v with |v| <= amax it gives quant1's result (q0 alone differs in 5304 of those 5.2e8).
constexpr float kQuantRecipMinScale = 0x1p-100f;

__device__ __forceinline__ int8_t quant1_recip(float v, float scale, float inv) {
  const float q0 = v * inv;
  const float t = __builtin_rintf(__builtin_fmaf(__builtin_fmaf(-q0, scale, v), inv, q0));
  return (int8_t)fminf(fmaxf(t, -127.0f), 127.0f);
}

__device__ __forceinline__ int8_t quant1(float v, float scale) {
  const float t = __builtin_rintf(v / scale);
  return (int8_t)fminf(fmaxf(t, -127.0f), 127.0f);
}

// Runs `body(q)` with a row's element quantizer q(v) (bf16 v): from the reciprocal of the scale
// where that gives quant1's results (scale >= kQuantRecipMinScale, every bf16 row but the
// tiniest), else by division.
template <typename F>
__device__ __forceinline__ void with_row_quantizer(float scale, F body) {
  if (scale >= kQuantRecipMinScale) {
    const float inv = 1.0f / scale;
    body([=](float v) { return quant1_recip(v, scale, inv); });
  } else {
    body([=](float v) { return quant1(v, scale); });
  }
}

inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? LSE_OK : (int)e;
}

}  // namespace lse
