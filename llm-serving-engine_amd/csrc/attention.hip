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
// Work decomposition. A workgroup of four waves takes one (entry, K/V head, query tile) item, or
// one key chunk of it. A query tile is 16 MFMA rows: TQ = floor(16 / G) query tokens x the G query
// heads that share the K/V head (GQA), so every K/V byte a workgroup reads serves all G heads; with
// G not dividing 16 (e.g. 24 query heads over 8 K/V heads) the last 16 - TQ G rows are idle.
//
// Canonical order of summation. A row's keys are cut into chunks of kAttnChunk positions
// (0..1023, 1024..2047, ...), fixed lengths that depend on nothing but the position. Within a chunk
// the four waves take 32-key tiles round-robin, each keeping its own online-softmax state, and the
// four states are merged in wave order; the chunks' merged states are then folded in chunk order
// (attn_fold). Whether the chunks of an item run one after another in one workgroup or as
// separate workgroups whose states a second kernel folds (the split launch, chosen from the shapes
// to fill the CUs) changes only where the arithmetic runs, never the arithmetic: a row's output is
// bit-identical whatever the batch around it, the table width or the query bucket, as for the
// reference's kernel, which never splits a row.
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
constexpr int kAttnKeys = 32;     // keys per wave tile
// Keys per chunk of the canonical order. Measured on MI355X (64 decode rows over 1025 keys, 8 over
// 8192, 256 over 512): 1024 keys is within 3 % of the best of 512, 1024 and 2048 in every case;
// 512 pays a cross-wave merge per 512 keys (+3 %), 2048 leaves long contexts too few chunks to
// split over (+13 % at 8 x 8192).
constexpr int kAttnChunk = 1024;
constexpr int kAttnMaxSplit = 64;  // chunks per item the split launch takes at most
static_assert(kAttnChunk % (kAttnWaves * kAttnKeys) == 0, "whole rounds of wave tiles per chunk");

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
  int bs_shift;      // log2(block_size) when it is a power of two, else -1
  int tq;            // query tokens per tile: floor(16 / G)
  int qtiles;        // ceil(max_q_len / tq)
  int parts;         // 1: a workgroup folds every chunk of its item; > 1: one chunk per workgroup
  float scale_log2;  // softmax scale x log2(e): scores are kept in the base-2 domain
  float* ws_o;       // parts > 1: chunk states' O [parts][entries][H][max_q_len][D], fp32
  float* ws_ml;      // parts > 1: chunk states' max and sum [parts][entries][H][max_q_len][2]
};

typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

// 16-lane transposing LDS read (see the header comment).
__device__ __forceinline__ bf16x4 lds_read_tr16(const unsigned char* p) {
  typedef __attribute__((address_space(3))) bf16x4* LdsV4;
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
      (LdsV4)((__attribute__((address_space(3))) unsigned char*)p));
}

__device__ __forceinline__ float exp2_fast(float v) { return __builtin_amdgcn_exp2f(v); }

// The tile's causal bound: the furthest position any of its rows attends to is query_offset +
// min(q_len, (qt + 1) * TQ) - 1, and never past context_len. Keys [0, attn_end) are its chunks'.
__device__ __forceinline__ int attn_end(int qo, int qlen, int ctx, int qt, int tq) {
  return min(qo + min(qlen, (qt + 1) * tq), ctx);
}

__device__ __forceinline__ int attn_chunks(int end_n) {
  return max(1, (end_n + kAttnChunk - 1) / kAttnChunk);
}

// Folds the next chunk's state (max mc in the base-2 domain, sum lc of exp2(s - mc), unnormalized
// output oc) into the running state (M, L, O) of the chunks before it. From (-inf, 0, 0) the first
// fold yields the chunk's state exactly. Explicit fused multiply-adds keep the arithmetic the same
// in every kernel that folds.
__device__ __forceinline__ void attn_fold(float& M, float& L, float (&O)[8], float mc, float lc,
                                          const float* oc) {
  const float mn = fmaxf(M, mc);
  const float ref = mn == -__builtin_huge_valf() ? 0.0f : mn;  // no key yet: keep p = 0
  const float fa = exp2_fast(M - ref), fb = exp2_fast(mc - ref);
  L = __builtin_fmaf(lc, fb, L * fa);
#pragma unroll
  for (int i = 0; i < 8; ++i) O[i] = __builtin_fmaf(oc[i], fb, O[i] * fa);
  M = mn;
}

// Eight normalized outputs in bf16 (a row that saw no key gives zeros).
__device__ __forceinline__ uint4 attn_out8(float L, const float (&O)[8]) {
  const float inv = L > 0.0f ? 1.0f / L : 0.0f;
  uint4 out;
  out.x = pack_bf16x2(O[0] * inv, O[1] * inv);
  out.y = pack_bf16x2(O[2] * inv, O[3] * inv);
  out.z = pack_bf16x2(O[4] * inv, O[5] * inv);
  out.w = pack_bf16x2(O[6] * inv, O[7] * inv);
  return out;
}

// NT: K and V stream with the nt cache policy; used when each K/V row is read by one workgroup
// only (one query tile: decode). POW2: block_size is a power of two (a shift finds a key's block).
template <int D, bool NT, bool POW2>
__global__ void __launch_bounds__(64 * kAttnWaves)
paged_attn_kernel(PagedAttnArgs a) {
  static_assert(D == 128, "head_dim 128: 16 chunks of 16 bytes per K/V row");
  constexpr int W = kAttnWaves, KT = kAttnKeys, KK = D / 32, DT = D / 16;
  constexpr int VROWB = 2 * D;  // bytes of one V row in LDS
  constexpr float NEG_INF = -__builtin_huge_valf();
  // Per wave: the V tile (32 rows), reused at the end of a chunk for the wave's O (16 rows x D
  // fp32).
  static_assert(KT * VROWB == 16 * D * 4, "the V tile and the O tile share one LDS region");
  __shared__ __attribute__((aligned(16))) unsigned char vbuf[W][KT * VROWB];
  __shared__ float mbuf[W][16], lbuf[W][16];
  // The pool blocks of the current chunk's positions (block_table entries b0 .. b0 + count - 1),
  // read once per chunk so a key's address needs no dependent global load.
  __shared__ int blk_lds[kAttnChunk + 1];

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
  const int G = a.G, TQ = a.tq;
  const int qlen = a.q_len[e];
  if (qt * TQ >= qlen) return;
  const int ctx = a.context_len[e], qo = a.query_offset[e], qs = a.q_start[e];
  const int end_n = attn_end(qo, qlen, ctx, qt, TQ);
  const int nch = attn_chunks(end_n);
  // Split launch: this workgroup's chunk only (none past the tile's keys: the fold reads no
  // state there). Otherwise every chunk of the item, folded here.
  const int c_first = a.parts > 1 ? part : 0;
  const int c_end = a.parts > 1 ? part + 1 : nch;
  if (c_first >= nch) return;

  // This lane's MFMA row (for Q, the scores and the softmax state): token tq, head gq of the group.
  // Rows from TQ G on are idle (G not dividing 16).
  const int tq = n16 / G, gq = n16 - tq * G;
  const int m_row = qt * TQ + tq;
  const bool row_ok = n16 < TQ * G && m_row < qlen;
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

  // The thread's part of a chunk merge and of the output: row `row` of the tile (token row / G,
  // head row % G), columns c8 .. c8 + 7.
  const int row = threadIdx.x >> 4, c8 = 8 * (threadIdx.x & 15);
  const int m_out = qt * TQ + row / G;
  const bool out_ok = row < TQ * G && m_out < qlen;
  const int h_out = kvh * G + row % G;
  float Mr = NEG_INF, Lr = 0.0f, Or[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  unsigned char* vb = vbuf[wave];

  for (int c = c_first; c < c_end; ++c) {
    const int pstart = c * kAttnChunk;
    const int pend = min(pstart + kAttnChunk, end_n);
    auto blk_of = [&](int n) { return POW2 ? n >> a.bs_shift : n / bs; };
    const int b0 = blk_of(pstart);
    {
      const int count = pend > pstart ? blk_of(pend - 1) - b0 + 1 : 0;
      for (int i = threadIdx.x; i < count; i += 64 * W) blk_lds[i] = bt[b0 + i];
      __syncthreads();
    }
    // Element offset of key n's row (this K/V head) in the pool; keys past the chunk are clamped
    // to its last key, so every load stays inside the entry's own blocks.
    auto row_off = [&](int n) -> int64_t {
      n = min(n, pend - 1);
      const int bi = blk_of(n);
      return (int64_t)blk_lds[bi - b0] * a.sb + (int64_t)(n - bi * bs) * a.sw +
             (int64_t)kvh * a.sh;
    };
    // K rows of a tile's two 16-key blocks (A operand) and its V tile (16 bytes x 8 per lane:
    // row (lane / 16) + 4 i, chunk lane % 16).
    uint4 kf[2][KK], vr[8];
    auto load_k = [&](int n0) {
#pragma unroll
      for (int bk = 0; bk < 2; ++bk) {
        const uint16_t* kp = a.k_pool + row_off(n0 + 16 * bk + n16) + 8 * grp;
#pragma unroll
        for (int kk = 0; kk < KK; ++kk)
          kf[bk][kk] =
              NT ? load16_stream(kp + 32 * kk) : *reinterpret_cast<const uint4*>(kp + 32 * kk);
      }
    };
    auto load_v = [&](int n0) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint16_t* vp = a.v_pool + row_off(n0 + grp + 4 * i) + 8 * n16;
        vr[i] = NT ? load16_stream(vp) : *reinterpret_cast<const uint4*>(vp);
      }
    };

    float m_run = NEG_INF, l_run = 0.0f;
    f32x4 oacc[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t) oacc[t] = f32x4{0, 0, 0, 0};

    // Each wave's tiles n0 = pstart + KT wave + KT W j. The next tile's K rows are loaded as soon
    // as the scores have consumed this tile's, and its V rows once this tile's are in LDS, so
    // they travel during this tile's softmax and P V. After the last tile these loads read the
    // chunk's last key again (row_off clamps), which keeps them unconditional and their waits
    // exact.
    if (pstart + KT * wave < pend) {
      load_k(pstart + KT * wave);
      // K before V, as in the loop, so the scores wait for K alone.
      __builtin_amdgcn_sched_barrier(0);
      load_v(pstart + KT * wave);
    }
    for (int n0 = pstart + KT * wave; n0 < pend; n0 += KT * W) {
      // Scores: lane holds keys n0 + 16 bk + 4 grp + r of row n16.
      f32x4 st[2];
#pragma unroll
      for (int bk = 0; bk < 2; ++bk) {
        st[bk] = f32x4{0, 0, 0, 0};
#pragma unroll
        for (int kk = 0; kk < KK; ++kk)
          st[bk] = mfma16x16x32(as_bf16x8(kf[bk][kk]), qf[kk], st[bk]);
      }
      load_k(n0 + KT * W);
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
      l_run = __builtin_fmaf(l_run, alpha, psum);
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
      load_v(n0 + KT * W);
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

    // Merge the waves in wave order: each writes its state (O rows 4 grp + r, columns
    // 16 t + n16) to its LDS region.
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

    float mw[W], mc = NEG_INF;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      mw[w] = mbuf[w][row];
      mc = fmaxf(mc, mw[w]);
    }
    const float mcref = mc == NEG_INF ? 0.0f : mc;
    float lc = 0.0f, oc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const float f = exp2_fast(mw[w] - mcref);
      lc = __builtin_fmaf(f, lbuf[w][row], lc);
      const float* src = reinterpret_cast<const float*>(vbuf[w]) + row * D + c8;
#pragma unroll
      for (int i = 0; i < 8; ++i) oc[i] = __builtin_fmaf(f, src[i], oc[i]);
    }
    if (a.parts > 1) {
      if (out_ok) {
        const int64_t slot = (((int64_t)c * a.entries + e) * a.H + h_out) * a.max_q_len + m_out;
        float* dst = a.ws_o + slot * D + c8;
        *reinterpret_cast<float4*>(dst) = make_float4(oc[0], oc[1], oc[2], oc[3]);
        *reinterpret_cast<float4*>(dst + 4) = make_float4(oc[4], oc[5], oc[6], oc[7]);
        if (c8 == 0) *reinterpret_cast<float2*>(a.ws_ml + 2 * slot) = make_float2(mc, lc);
      }
    } else {
      attn_fold(Mr, Lr, Or, mc, lc, oc);
    }
    if (c + 1 < c_end) __syncthreads();  // every thread read the merge storage before reuse
  }
  if (a.parts == 1 && out_ok)
    *reinterpret_cast<uint4*>(a.o + (int64_t)h_out * a.so_h + (int64_t)(qs + m_out) * a.so_t +
                              c8) = attn_out8(Lr, Or);
}

// Second pass of a split launch: one thread per (entry, head, query row, 8 columns) folds the
// states of the chunks the row's tile covered, in chunk order, as the single-pass kernel does.
template <int D>
__global__ void __launch_bounds__(256)
paged_attn_merge(PagedAttnArgs a) {
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
  const int end_n = attn_end(a.query_offset[e], qlen, a.context_len[e], m / a.tq, a.tq);
  const int np = attn_chunks(end_n);
  const int64_t stride = (int64_t)a.entries * a.H * a.max_q_len;
  const int64_t base = ((int64_t)e * a.H + h) * a.max_q_len + m;
  float M = -__builtin_huge_valf(), L = 0.0f, O[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int p = 0; p < np; ++p) {
    const int64_t slot = base + p * stride;
    attn_fold(M, L, O, a.ws_ml[2 * slot], a.ws_ml[2 * slot + 1], a.ws_o + slot * D + c8);
  }
  *reinterpret_cast<uint4*>(a.o + (int64_t)h * a.so_h + (int64_t)(a.q_start[e] + m) * a.so_t + c8) =
      attn_out8(L, O);
}

// ---- host side -----------------------------------------------------------------------------

struct AttnPlan {
  int tq, qtiles, parts;
  int64_t ws_o_bytes, ws_bytes;
};

// One workgroup per (entry, K/V head, query tile) item once those fill the CUs twice over;
// otherwise, when the table's context bound (max_blocks x block_size) spans 2..kAttnMaxSplit
// chunks, one workgroup per chunk (workgroups past a row's own chunks exit at once) and a second
// pass that folds them. The choice depends on shapes only and changes no result.
static AttnPlan attn_plan(int64_t entries, int64_t H, int64_t HKV, int64_t D, int64_t max_q_len,
                          int64_t max_ctx, int cus) {
  AttnPlan pl{};
  pl.tq = (int)(16 / (H / HKV));
  pl.qtiles = (int)ceil_div(max_q_len, pl.tq);
  const int64_t items = entries * HKV * pl.qtiles;
  const int64_t chunks = ceil_div(std::max<int64_t>(max_ctx, 1), kAttnChunk);
  pl.parts = items > 0 && items < 2 * (int64_t)cus && chunks > 1 && chunks <= kAttnMaxSplit
                 ? (int)chunks
                 : 1;
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
  a.bs_shift = -1;
  for (int s = 0; s < 31; ++s)
    if ((int64_t)1 << s == block_size) a.bs_shift = s;
  a.max_q_len = (int)max_q_len;
  const int64_t max_ctx = max_blocks * block_size;
  const AttnPlan pl = attn_plan(a.entries, a.H, a.HKV, 128, a.max_q_len, max_ctx, attn_cus());
  if (pl.ws_bytes > 0 && (ws_bytes < pl.ws_bytes || !ws)) return LSE_E_WORKSPACE;
  a.tq = pl.tq;
  a.qtiles = pl.qtiles;
  a.parts = pl.parts;
  a.scale_log2 = softmax_scale * 1.4426950408889634f;
  a.ws_o = pl.parts > 1 ? static_cast<float*>(ws) : nullptr;
  a.ws_ml = pl.parts > 1 ? reinterpret_cast<float*>(static_cast<char*>(ws) + pl.ws_o_bytes) : nullptr;
  const int64_t blocks = (int64_t)a.entries * a.HKV * pl.qtiles * pl.parts;
  if (blocks > 0x7fffffff) return LSE_E_RANGE;
  void* args[] = {&a};
  const bool pow2 = a.bs_shift >= 0;
  const void* fn =
      pl.qtiles == 1
          ? (pow2 ? reinterpret_cast<const void*>(&paged_attn_kernel<128, true, true>)
                  : reinterpret_cast<const void*>(&paged_attn_kernel<128, true, false>))
          : (pow2 ? reinterpret_cast<const void*>(&paged_attn_kernel<128, false, true>)
                  : reinterpret_cast<const void*>(&paged_attn_kernel<128, false, false>));
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
