// Paged attention over a shared per-layer K/V pool: the computation of the reference's
// `paged_attention_forward` / `paged_attention_2` (src/llm_serving_engine/kernels/flash_attention.py:
// 201-332), written for gfx950 matrix cores.
//
// Semantics. Entry e owns q rows [q_start[e], q_start[e] + q_len[e]) of q (H, tokens, D); its cache
// position i lives in pool block block_table[e][i / block_size], slot i % block_size. Query row m
// (cache position query_offset[e] + m) of head h attends to positions n < context_len[e] with
// n <= query_offset[e] + m, through K/V head h / (H / H_KV):
//   o[h][q_start + m] = sum_n softmax_n(scale * q . k_n) v_n.
// Like the reference, the softmax runs online in fp32 and the probabilities are rounded to bf16
// before the product with V (fp32 accumulation); the output is rounded to bf16.
//
// Work decomposition. A workgroup of four waves takes one (entry, K/V head, query tile, key
// partition). A query tile is 16 MFMA rows: 16 / G query tokens x the G query heads that share
// the K/V head (GQA), so every K/V byte a workgroup reads serves all G heads. The partition's keys
// go to the waves in tiles of 32, round-robin; each wave keeps its own online-softmax state and
// the four are merged through LDS at the end. Long contexts with few (entry, head, tile) items are
// split into key partitions whose partial results (unnormalized O, running max and sum) a second
// kernel merges; the split depends only on the shapes, never on the data.
//
// Per 32-key tile and wave:
//  * S^T = K Q^T on v_mfma_f32_16x16x32_bf16: K rows are the A operand (16 keys x 32 head dims:
//    each lane loads 16 contiguous bytes of one key row straight from the pool) and Q the B
//    operand, kept in registers. Lane l then holds the scores of keys 4 (l / 16) + r of row l % 16.
//  * Online softmax on those scores: row max and sum over the lane's 8 values and the 4 lanes
//    holding the same row (l, l ^ 16, l ^ 32, l ^ 48).
//  * O += P V: the probabilities, rounded to bf16, are already the A operand in the lane layout the
//    scores came out in, with the 32-long contraction running over keys {4 g + j, 16 + 4 g + j}
//    for lane group g; V is staged in LDS row-major (rows XOR-swizzled by 16-byte chunk so the
//    reads below are conflict-free) and read with ds_read_b64_tr_b16, whose 16-lane transpose
//    returns, for lane i of a group addressing rows kb + (s >> 2) at columns d0 + 4 (s & 3), the
//    four keys kb..kb+3 at column d0 + i: exactly the B operand for those keys.
#include <algorithm>

#include "lse_common.h"

namespace lse {

constexpr int kAttnWaves = 4;
constexpr int kAttnKeys = 32;                          // keys per wave tile
constexpr int kAttnPartKeys = kAttnWaves * kAttnKeys;  // partition lengths are multiples of this

struct PagedAttnArgs {
  const uint16_t* q;  // bf16, element (h, t, d) at h * sq_h + t * sq_t + d
  int64_t sq_h, sq_t;
  const uint16_t* k_pool;  // bf16 (blocks, block_size, H_KV, D): (b, w, h, d) at b sb + w sw + h sh + d
  const uint16_t* v_pool;
  int64_t sb, sw, sh;
  const int32_t* block_table;  // (entries, max_blocks), row stride sbt
  int64_t sbt;
  const int32_t* context_len;
  const int32_t* query_offset;
  const int32_t* q_start;
  const int32_t* q_len;
  uint16_t* o;  // bf16, same indexing as q with strides so_h, so_t
  int64_t so_h, so_t;
  int entries, H, HKV, G, block_size, max_q_len;
  int qtiles;        // ceil(max_q_len / (16 / G))
  int parts;         // key partitions
  int chunk;         // keys per partition (a multiple of kAttnPartKeys)
  float scale_log2;  // softmax scale x log2(e): scores are kept in the base-2 domain
  float* ws_o;       // parts > 1: partial O [parts][entries][H][max_q_len][D], fp32
  float* ws_ml;      // parts > 1: running max and sum [parts][entries][H][max_q_len][2]
};

typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

// 16-lane transposing LDS read (see the header comment).
__device__ __forceinline__ bf16x4 lds_read_tr16(const unsigned char* p) {
  typedef __attribute__((address_space(3))) bf16x4* LdsV4;
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
      (LdsV4)((__attribute__((address_space(3))) unsigned char*)p));
}

__device__ __forceinline__ float exp2_fast(float v) { return __builtin_amdgcn_exp2f(v); }

// The keys [pstart, pend) a workgroup covers and the tile's causal bound: the furthest position any
// of its rows attends to is query_offset + min(q_len, (qt + 1) * TQ) - 1, and never past
// context_len.
__device__ __forceinline__ int attn_end(int qo, int qlen, int ctx, int qt, int tq) {
  return min(qo + min(qlen, (qt + 1) * tq), ctx);
}

// NT: K and V stream with the nt cache policy; used when each K/V row is read by one workgroup
// only (one query tile: decode).
template <int D, bool NT>
__global__ void __launch_bounds__(64 * kAttnWaves)
paged_attn_kernel(PagedAttnArgs a) {
  static_assert(D == 128, "head_dim 128: 16 chunks of 16 bytes per K/V row");
  constexpr int W = kAttnWaves, KT = kAttnKeys, KK = D / 32, DT = D / 16;
  constexpr int VROWB = 2 * D;  // bytes of one V row in LDS
  constexpr float NEG_INF = -__builtin_huge_valf();
  // Per wave: the V tile (32 rows), reused at the end for the wave's O (16 rows x D fp32).
  static_assert(KT * VROWB == 16 * D * 4, "the V tile and the O tile share one LDS region");
  __shared__ __attribute__((aligned(16))) unsigned char vbuf[W][KT * VROWB];
  __shared__ float mbuf[W][16], lbuf[W][16];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n16 = lane & 15, grp = lane >> 4;

  int b = blockIdx.x;
  const int part = b % a.parts;
  b /= a.parts;
  const int qt = b % a.qtiles;
  b /= a.qtiles;
  const int kvh = b % a.HKV;
  const int e = b / a.HKV;
  const int G = a.G, TQ = 16 / G;
  const int qlen = a.q_len[e];
  if (qt * TQ >= qlen) return;
  const int ctx = a.context_len[e], qo = a.query_offset[e], qs = a.q_start[e];
  const int end_n = attn_end(qo, qlen, ctx, qt, TQ);
  const int pstart = part * a.chunk;
  const int pend = min(pstart + a.chunk, end_n);
  if (part > 0 && pstart >= pend) return;  // beyond the tile's keys: the merge reads no result

  // This lane's MFMA row (for Q, the scores and the softmax state): token tq, head g of the group.
  const int tq = n16 / G, gq = n16 - tq * G;
  const int m_row = qt * TQ + tq;
  const bool row_ok = m_row < qlen;
  const int qpos = qo + m_row;  // the row's cache position: it sees keys n <= qpos
  const int head = kvh * G + gq;

  bf16x8 qf[KK];
  {
    const uint16_t* qp = a.q + (int64_t)head * a.sq_h + (int64_t)(qs + min(m_row, qlen - 1)) * a.sq_t;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const uint4 v = *reinterpret_cast<const uint4*>(qp + 32 * kk + 8 * grp);
      qf[kk] = as_bf16x8(row_ok ? v : make_uint4(0, 0, 0, 0));
    }
  }
  const int32_t* bt = a.block_table + (int64_t)e * a.sbt;
  const int bs = a.block_size;
  // Element offset of key n's row (this K/V head) in the pool; keys past the partition are
  // clamped to its last key, so every load stays inside the entry's own blocks.
  auto row_off = [&](int n) -> int64_t {
    n = min(n, pend - 1);
    const int blk = bt[n / bs];
    return (int64_t)blk * a.sb + (int64_t)(n - (n / bs) * bs) * a.sw + (int64_t)kvh * a.sh;
  };

  float m_run = NEG_INF, l_run = 0.0f;
  f32x4 oacc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) oacc[t] = f32x4{0, 0, 0, 0};
  unsigned char* vb = vbuf[wave];

  for (int n0 = pstart + KT * wave; n0 < pend; n0 += KT * W) {
    // K rows of the tile's two 16-key blocks (A operand) and the V tile (16 bytes x 8 per lane:
    // row (lane / 16) + 4 i, chunk lane % 16), all issued before any use.
    uint4 kf[2][KK], vr[8];
#pragma unroll
    for (int bk = 0; bk < 2; ++bk) {
      const uint16_t* kp = a.k_pool + row_off(n0 + 16 * bk + n16) + 8 * grp;
#pragma unroll
      for (int kk = 0; kk < KK; ++kk)
        kf[bk][kk] = NT ? load16_stream(kp + 32 * kk) : *reinterpret_cast<const uint4*>(kp + 32 * kk);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint16_t* vp = a.v_pool + row_off(n0 + grp + 4 * i) + 8 * n16;
      vr[i] = NT ? load16_stream(vp) : *reinterpret_cast<const uint4*>(vp);
    }

    // Scores: lane holds keys n0 + 16 bk + 4 grp + r of row n16.
    f32x4 st[2];
#pragma unroll
    for (int bk = 0; bk < 2; ++bk) {
      st[bk] = f32x4{0, 0, 0, 0};
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) st[bk] = mfma16x16x32(as_bf16x8(kf[bk][kk]), qf[kk], st[bk]);
    }
    float s[8];
    float tmax = NEG_INF;
#pragma unroll
    for (int bk = 0; bk < 2; ++bk)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int n = n0 + 16 * bk + 4 * grp + r;
        const bool ok = row_ok && n < pend && n <= qpos;
        s[4 * bk + r] = ok ? st[bk][r] * a.scale_log2 : NEG_INF;
        tmax = fmaxf(tmax, s[4 * bk + r]);
      }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
    const float m_new = fmaxf(m_run, tmax);
    const float mref = m_new == NEG_INF ? 0.0f : m_new;  // a row with no key yet keeps p = 0
    const float alpha = exp2_fast(m_run - mref);
    float p[8], psum = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      p[i] = exp2_fast(s[i] - mref);
      psum += p[i];
    }
    psum += __shfl_xor(psum, 16);
    psum += __shfl_xor(psum, 32);
    l_run = l_run * alpha + psum;
    m_run = m_new;
    // O rows are 4 grp + r: their factors come from the lanes holding those rows.
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float ar = __shfl(alpha, 4 * grp + r);
#pragma unroll
      for (int t = 0; t < DT; ++t) oacc[t][r] *= ar;
    }
    bf16x8 pa;
#pragma unroll
    for (int i = 0; i < 8; ++i) pa[i] = (__bf16)p[i];

    // V tile to LDS: row rr = grp + 4 i, logical chunk n16 at physical chunk n16 ^ 2 (rr & 3).
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int rr = grp + 4 * i;
      *reinterpret_cast<uint4*>(vb + rr * VROWB + 16 * (n16 ^ (2 * (rr & 3)))) = vr[i];
    }
    // O += P V. Group grp reads rows kb + (n16 >> 2), kb = 4 grp (keys 0..3 of its contraction
    // slice) and 16 + 4 grp (keys 4..7), at logical columns 16 t + 4 (n16 & 3).
    const int rlo = n16 >> 2;
    const int swz = 2 * (rlo & 3);
    const int cbyte = 8 * (n16 & 1);
    const unsigned char* r0 = vb + (4 * grp + rlo) * VROWB + cbyte;
    const unsigned char* r1 = vb + (16 + 4 * grp + rlo) * VROWB + cbyte;
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      const int pc = (2 * t + ((n16 & 3) >> 1)) ^ swz;
      const bf16x4 v0 = lds_read_tr16(r0 + 16 * pc);
      const bf16x4 v1 = lds_read_tr16(r1 + 16 * pc);
      const bf16x8 vv = __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7);
      oacc[t] = mfma16x16x32(pa, vv, oacc[t]);
    }
  }

  // Merge the waves: each writes its state (O rows 4 grp + r, columns 16 t + n16) to its LDS region.
  float* ob = reinterpret_cast<float*>(vb);
  if (lane < 16) {
    mbuf[wave][lane] = m_run;
    lbuf[wave][lane] = l_run;
  }
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) ob[(4 * grp + r) * D + 16 * t + n16] = oacc[t][r];
  __syncthreads();

  // 256 threads: row = tid / 16, columns 8 c .. 8 c + 7 with c = tid % 16.
  const int row = threadIdx.x >> 4, c8 = 8 * (threadIdx.x & 15);
  const int m_out = qt * TQ + row / G;
  if (m_out >= qlen) return;
  const int h_out = kvh * G + row % G;
  float mw[W], M = NEG_INF;
#pragma unroll
  for (int w = 0; w < W; ++w) {
    mw[w] = mbuf[w][row];
    M = fmaxf(M, mw[w]);
  }
  const float Mref = M == NEG_INF ? 0.0f : M;
  float L = 0.0f, ov[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int w = 0; w < W; ++w) {
    const float f = exp2_fast(mw[w] - Mref);
    L += f * lbuf[w][row];
    const float* src = reinterpret_cast<const float*>(vbuf[w]) + row * D + c8;
#pragma unroll
    for (int i = 0; i < 8; ++i) ov[i] += f * src[i];
  }
  if (a.parts == 1) {
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    uint4 out;
    out.x = pack_bf16x2(ov[0] * inv, ov[1] * inv);
    out.y = pack_bf16x2(ov[2] * inv, ov[3] * inv);
    out.z = pack_bf16x2(ov[4] * inv, ov[5] * inv);
    out.w = pack_bf16x2(ov[6] * inv, ov[7] * inv);
    *reinterpret_cast<uint4*>(a.o + (int64_t)h_out * a.so_h + (int64_t)(qs + m_out) * a.so_t + c8) =
        out;
  } else {
    const int64_t slot =
        (((int64_t)part * a.entries + e) * a.H + h_out) * a.max_q_len + m_out;
    float* dst = a.ws_o + slot * D + c8;
    *reinterpret_cast<float4*>(dst) = make_float4(ov[0], ov[1], ov[2], ov[3]);
    *reinterpret_cast<float4*>(dst + 4) = make_float4(ov[4], ov[5], ov[6], ov[7]);
    if (c8 == 0) *reinterpret_cast<float2*>(a.ws_ml + 2 * slot) = make_float2(M, L);
  }
}

// Second pass of a split launch: one thread per (entry, head, query row, 8 columns) merges the
// partitions the row's tile covered, in partition order.
template <int D>
__global__ void __launch_bounds__(256)
paged_attn_merge(PagedAttnArgs a) {
  constexpr float NEG_INF = -__builtin_huge_valf();
  constexpr int C = D / 8;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t rows = (int64_t)a.entries * a.H * a.max_q_len;
  if (t >= rows * C) return;
  const int c8 = 8 * (int)(t % C);
  int64_t r = t / C;
  const int m = (int)(r % a.max_q_len);
  r /= a.max_q_len;
  const int h = (int)(r % a.H);
  const int e = (int)(r / a.H);
  const int qlen = a.q_len[e];
  if (m >= qlen) return;
  const int TQ = 16 / a.G;
  const int end_n = attn_end(a.query_offset[e], qlen, a.context_len[e], m / TQ, TQ);
  const int np = max(1, (end_n + a.chunk - 1) / a.chunk);
  const int64_t stride = (int64_t)a.entries * a.H * a.max_q_len;
  const int64_t base = ((int64_t)e * a.H + h) * a.max_q_len + m;
  float M = NEG_INF;
  for (int p = 0; p < np; ++p) M = fmaxf(M, a.ws_ml[2 * (base + p * stride)]);
  const float Mref = M == NEG_INF ? 0.0f : M;
  float L = 0.0f, ov[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int p = 0; p < np; ++p) {
    const int64_t slot = base + p * stride;
    const float f = exp2_fast(a.ws_ml[2 * slot] - Mref);
    L += f * a.ws_ml[2 * slot + 1];
    const float* src = a.ws_o + slot * D + c8;
#pragma unroll
    for (int i = 0; i < 8; ++i) ov[i] += f * src[i];
  }
  const float inv = L > 0.0f ? 1.0f / L : 0.0f;
  uint4 out;
  out.x = pack_bf16x2(ov[0] * inv, ov[1] * inv);
  out.y = pack_bf16x2(ov[2] * inv, ov[3] * inv);
  out.z = pack_bf16x2(ov[4] * inv, ov[5] * inv);
  out.w = pack_bf16x2(ov[6] * inv, ov[7] * inv);
  *reinterpret_cast<uint4*>(a.o + (int64_t)h * a.so_h + (int64_t)(a.q_start[e] + m) * a.so_t + c8) =
      out;
}

// ---- host side -----------------------------------------------------------------------------

struct AttnPlan {
  int qtiles, parts, chunk;
  int64_t ws_o_bytes, ws_bytes;
};

// Key partitions: one per (entry, K/V head, query tile) once those fill the CUs twice over;
// otherwise the context bound (max_blocks x block_size) is cut so they do, in partitions of at
// least 256 keys.
static AttnPlan attn_plan(int64_t entries, int64_t H, int64_t HKV, int64_t D, int64_t max_q_len,
                          int64_t max_ctx, int cus) {
  AttnPlan pl{};
  const int64_t tq = 16 / (H / HKV);
  pl.qtiles = (int)ceil_div(max_q_len, tq);
  const int64_t items = entries * HKV * pl.qtiles;
  int64_t parts = 1;
  if (items > 0 && items < 2 * (int64_t)cus) {
    parts = std::min<int64_t>(ceil_div(2 * (int64_t)cus, items), ceil_div(max_ctx, 256));
    parts = std::max<int64_t>(parts, 1);
  }
  const int64_t chunk = ceil_div(ceil_div(std::max<int64_t>(max_ctx, 1), parts), kAttnPartKeys) *
                        kAttnPartKeys;
  pl.chunk = (int)chunk;
  pl.parts = (int)ceil_div(std::max<int64_t>(max_ctx, 1), chunk);
  if (pl.parts > 1) {
    const int64_t slots = (int64_t)pl.parts * entries * H * max_q_len;
    pl.ws_o_bytes = slots * D * 4;
    pl.ws_bytes = pl.ws_o_bytes + slots * 2 * 4;
  }
  return pl;
}

static int attn_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
    (void)hipGetLastError();
    return 256;
  }
  return cus;
}

int64_t paged_attention_workspace_bytes(int64_t entries, int64_t H, int64_t HKV, int64_t D,
                                        int64_t max_q_len, int64_t max_ctx) {
  return attn_plan(entries, H, HKV, D, max_q_len, max_ctx, attn_cus()).ws_bytes;
}

int launch_paged_attention(const uint16_t* q, int64_t sq_h, int64_t sq_t, const uint16_t* k_pool,
                           const uint16_t* v_pool, int64_t sb, int64_t sw, int64_t sh,
                           const int32_t* block_table, int64_t sbt, const int32_t* context_len,
                           const int32_t* query_offset, const int32_t* q_start,
                           const int32_t* q_len, uint16_t* o, int64_t so_h, int64_t so_t,
                           int64_t entries, int64_t H, int64_t HKV, int64_t block_size,
                           int64_t max_blocks, int64_t max_q_len, float softmax_scale, void* ws,
                           int64_t ws_bytes, hipStream_t stream) {
  PagedAttnArgs a{};
  a.q = q;
  a.sq_h = sq_h;
  a.sq_t = sq_t;
  a.k_pool = k_pool;
  a.v_pool = v_pool;
  a.sb = sb;
  a.sw = sw;
  a.sh = sh;
  a.block_table = block_table;
  a.sbt = sbt;
  a.context_len = context_len;
  a.query_offset = query_offset;
  a.q_start = q_start;
  a.q_len = q_len;
  a.o = o;
  a.so_h = so_h;
  a.so_t = so_t;
  a.entries = (int)entries;
  a.H = (int)H;
  a.HKV = (int)HKV;
  a.G = (int)(H / HKV);
  a.block_size = (int)block_size;
  a.max_q_len = (int)max_q_len;
  const int64_t max_ctx = max_blocks * block_size;
  const AttnPlan pl = attn_plan(a.entries, a.H, a.HKV, 128, a.max_q_len, max_ctx, attn_cus());
  if (pl.ws_bytes > 0 && (ws_bytes < pl.ws_bytes || !ws)) return LSE_E_WORKSPACE;
  a.qtiles = pl.qtiles;
  a.parts = pl.parts;
  a.chunk = pl.chunk;
  a.scale_log2 = softmax_scale * 1.4426950408889634f;
  a.ws_o = pl.parts > 1 ? static_cast<float*>(ws) : nullptr;
  a.ws_ml = pl.parts > 1 ? reinterpret_cast<float*>(static_cast<char*>(ws) + pl.ws_o_bytes) : nullptr;
  const int64_t blocks = (int64_t)a.entries * a.HKV * pl.qtiles * pl.parts;
  if (blocks > 0x7fffffff) return LSE_E_RANGE;
  void* args[] = {&a};
  const void* fn = pl.qtiles == 1 ? reinterpret_cast<const void*>(&paged_attn_kernel<128, true>)
                                  : reinterpret_cast<const void*>(&paged_attn_kernel<128, false>);
  hipError_t err = hipLaunchKernel(fn,
                                   dim3((unsigned)blocks), dim3(64 * kAttnWaves), args, 0, stream);
  if (err == hipSuccess && pl.parts > 1) {
    const int64_t threads = (int64_t)a.entries * a.H * a.max_q_len * (128 / 8);
    err = hipLaunchKernel(reinterpret_cast<const void*>(&paged_attn_merge<128>),
                          dim3((unsigned)ceil_div(threads, 256)), dim3(256), args, 0, stream);
  }
  return err == hipSuccess ? launch_status() : (int)err;
}

}  // namespace lse
