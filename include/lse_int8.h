/*
 * lse_int8.h — C ABI of the MI355X (gfx950) int8 quantized Linear forward.
 *
 * The reference engine routes every Llama projection through `nn.Linear.forward`, i.e.
 * `F.linear(x, W)` with bias=False (torch/nn/modules/linear.py:130-134), from these call
 * sites: q/k/v in `ModelRunner._project_qkv` (src/llm_serving_engine/model/model_runner.py:322-324),
 * o_proj in `attention_output` (model_runner.py:369) and `contiguous_attention`
 * (model_runner.py:418), gate/up/down in `LlamaMLP.forward` reached from `decoder_hidden`
 * (model_runner.py:223). Its int8 switch (`ModelConfig.quantize`, src/llm_serving_engine/config.py:32)
 * stops at `raise NotImplementedError("int8 weight-only quantization")` (model_runner.py:45-46).
 * The entry points below are what a binding for that switch calls.
 *
 * Conventions shared by every entry point:
 *  - All pointers are device pointers. The caller owns every buffer; the library keeps no state
 *    beyond its compiled kernels and allocates nothing. The GEMMs of some shapes (deep decode
 *    shapes, and 65..256 tokens over a narrow weight) add partial sums of K ranges in a second
 *    pass through a caller-provided workspace of lse_workspace_bytes(...) bytes (0 for most
 *    calls); a workspace may be reused by calls that are ordered on one stream, never by calls
 *    that can overlap.
 *  - Weights travel in the packed tile layout written by lse_pack_weight: tiles of 16 rows x 64
 *    K-bytes, 1 KB each, tile (rb, j) at byte (rb * ceil(K/64) + j) * 1024, its byte 16*l + i
 *    holding q[16*rb + l%16][64*j + 16*(l/16) + i], zero past N and K. One 128-bit load per lane
 *    of a 64-wide wave reads one tile, contiguous and already in matrix-core operand order.
 *  - Matrices are row-major. `ld*` is the row stride in elements. bf16 data travels as
 *    `void*` (2 bytes per element, IEEE bfloat16 bit patterns).
 *  - `stream` is a `hipStream_t` passed as `void*`. Work is enqueued on it and never
 *    synchronised, so every entry point is safe under HIP graph capture. The null stream is
 *    accepted but callers that capture must pass their capture stream.
 *  - Return value: LSE_OK (0) on success; a negative LSE_E_* code for a rejected argument
 *    (nothing was launched); a positive hipError_t from the launch otherwise.
 *  - Results are deterministic: no atomics, and the summation order of every output element
 *    depends only on N, K, the device's CU count and the token class of the call, never on M
 *    inside the class, on other rows or on timing. Row m of y is therefore bit-identical whether
 *    it is computed alone or inside a padded batch of the same class. W8A8 sums are exact int32,
 *    so its rows are identical for every M. The W8A16 classes are M <= 16, 17..32, 33..64,
 *    65..128 and 129..256, and above 256 tokens one class, except over a deep, narrow weight
 *    (at least 128 K steps of 64, i.e. K > 8128, and few enough output tiles that the split grid
 *    fits the CUs: down_proj of Llama-3-8B on 256 CUs), where 257..512, 513..1024 and > 1024 are
 *    three. The classes align with power-of-two decode buckets (bucket(M) <= 16 exactly when
 *    M <= 16, and so on), so a graphed bucket and the eager batch it stands for compute each
 *    row identically; a caller that pads a batch must pad within its class.
 */
#ifndef LSE_INT8_H
#define LSE_INT8_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum lse_status {
  LSE_OK = 0,
  LSE_E_NULL = -1,        /* a required pointer is NULL (with a non-empty shape) */
  LSE_E_SHAPE = -2,       /* negative size, or a stride smaller than the row it holds */
  LSE_E_ALIGN = -3,       /* K, a stride or a pointer misses the alignment the kernels load with */
  LSE_E_RANGE = -4,       /* K too large for exact int32 accumulation, or a size beyond int32 grids */
  LSE_E_ALGO = -5,        /* unknown algorithm id, or one that cannot run this shape */
  LSE_E_WORKSPACE = -6,   /* workspace NULL or smaller than lse_workspace_bytes for the call */
  LSE_E_SCRATCH = -7,     /* lse_w8a16_gemm_noalloc: the call needs more workspace than the
                             library's static scratch (LSE_NOALLOC_SCRATCH_BYTES) holds */
};

/* Arithmetic mode, for lse_workspace_bytes. */
enum lse_mode {
  LSE_MODE_W8A16 = 0,
  LSE_MODE_W8A8 = 1,
};

/* Algorithm selector for lse_w8a16_gemm_algo. */
enum lse_algo {
  LSE_ALGO_AUTO = 0,      /* decode kernel for M <= LSE_DECODE_MAX_M, prefill GEMM above */
  LSE_ALGO_DECODE = 1,    /* streaming GEMV / skinny GEMM (M <= LSE_DECODE_MAX_M) */
  LSE_ALGO_PREFILL = 2,   /* LDS-tiled MFMA GEMM */
};

/* lse_query keys. */
enum lse_query_key {
  LSE_Q_ABI_VERSION = 0,  /* this header's ABI version */
  LSE_Q_K_ALIGN = 1,      /* K must be a multiple of this (bytes of an int8 row = elements) */
  LSE_Q_DECODE_MAX_M = 2, /* largest M the decode kernel takes */
  LSE_Q_MAX_K = 3,        /* largest K with exact int32 W8A8 accumulation */
  LSE_Q_GFX_ARCH = 4,     /* the code-object target, e.g. 950 */
  LSE_Q_NOALLOC_SCRATCH = 5, /* bytes of the static scratch lse_w8a16_gemm_noalloc works in */
};

#define LSE_ABI_VERSION 12
#define LSE_NOALLOC_SCRATCH_BYTES (32 << 20)
#define LSE_K_ALIGN 16
#define LSE_DECODE_MAX_M 64
#define LSE_MAX_K 133120      /* 127*127*K < 2^31 with margin; multiple of LSE_K_ALIGN */

/*
 * Per-output-channel symmetric weight quantization, run once at load time.
 *   s[n] = fl32(max_k |w[n,k]| / 127)      (IEEE division; an all-zero row gets s[n] = 1)
 *   q[n,k] = clamp(rne(fl32(w[n,k] / s[n])), -127, 127)
 * w: (N, K) fp32, row stride ldw. q: (N, K) int8, contiguous (row stride K). s: (N) fp32.
 * Replaces: the bf16 `nn.Linear.weight` that `AutoModelForCausalLM.from_pretrained` loads
 * (model_runner.py:50-52) at the int8 switch (model_runner.py:45-46).
 */
int lse_quantize_weight_per_channel(const float* w, int64_t ldw, int8_t* q, float* s,
                                    int64_t N, int64_t K, void* stream);

/* Bytes of the packed layout of an (N, K) weight: ceil(N/16) * ceil(K/64) * 1024. */
int64_t lse_packed_weight_bytes(int64_t N, int64_t K);

/*
 * Packs a row-major (N, K) int8 weight (contiguous, K % LSE_K_ALIGN == 0, 16-byte aligned) into
 * the tile layout every GEMM below reads (qp: lse_packed_weight_bytes(N, K) bytes, 16-byte
 * aligned). Load time only.
 * Replaces: nothing in the reference (its weights are row-major `nn.Linear.weight`); it is the
 * storage step of the int8 switch (model_runner.py:45-46).
 */
int lse_pack_weight(const int8_t* q, int64_t N, int64_t K, int8_t* qp, void* stream);

/*
 * Bytes of device workspace (16-byte aligned) that lse_w8a16_gemm (mode LSE_MODE_W8A16) or
 * lse_w8a8_gemm (LSE_MODE_W8A8) needs for an (M, N, K) call on the current device; 0 when the
 * call needs none, -1 for a negative size or an unknown mode. At most 64 * M * (N + 15).
 * Replaces: nothing in the reference; callers size the buffer with it, as cuBLASLt callers do.
 */
int64_t lse_workspace_bytes(int mode, int64_t M, int64_t N, int64_t K);

/*
 * W8A16 linear: y[m,n] = bf16_rne(s[n] * sum_k x[m,k] * q[n,k]), fp32 accumulation.
 * x: (M, K) bf16, row stride ldx (multiple of 8, 16-byte aligned base).
 * qp: packed (N, K) int8 weight, K % LSE_K_ALIGN == 0. s: (N) fp32.
 * y: (M, N) bf16, row stride ldy >= N (any; 8-byte stores are used when ldy % 4 == 0 and the
 *    base is 8-byte aligned, 2-byte stores otherwise).
 * workspace: workspace_bytes >= lse_workspace_bytes(LSE_MODE_W8A16, M, N, K) bytes, 16-byte
 *    aligned (may be NULL when that is 0).
 * Replaces: `F.linear(x, W)` of `nn.Linear.forward` (torch/nn/modules/linear.py:134) at
 * model_runner.py:322-324, 369, 418 and modeling_llama.py:175 (LlamaMLP.forward).
 */
int lse_w8a16_gemm(const void* x, int64_t ldx, const int8_t* qp, const float* s, void* y,
                   int64_t ldy, int64_t M, int64_t N, int64_t K, void* workspace,
                   int64_t workspace_bytes, void* stream);

/*
 * lse_w8a16_gemm without a workspace argument, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). It calls
 * no hipMalloc, hipFree or allocating routine: the workspace lse_w8a16_gemm would take lives in a
 * static device array of LSE_NOALLOC_SCRATCH_BYTES (32 MiB) that each device the library runs on
 * holds until the process ends, its device address looked up on the device's first call. A
 * call with M = 0 launches nothing and only does that lookup for the current device: a caller
 * whose first real call on a device is made under HIP graph capture makes one before it. Same
 * kernels, so y is bit-identical to lse_w8a16_gemm's. Calls that overlap on one device (two
 * streams at once) share that array and race; calls in stream order do not. Returns
 * LSE_E_SCRATCH when lse_workspace_bytes(LSE_MODE_W8A16, M, N, K) exceeds the array.
 * Replaces: nothing in the reference (it has no such caller); an addition for callers that
 * cannot allocate.
 */
int lse_w8a16_gemm_noalloc(const void* x, int64_t ldx, const int8_t* qp, const float* s,
                           void* y, int64_t ldy, int64_t M, int64_t N, int64_t K, void* stream);

/* lse_w8a16_gemm with the kernel family chosen by the caller (enum lse_algo); used to test
 * the decode and prefill kernels on identical inputs. Same contract otherwise. */
int lse_w8a16_gemm_algo(const void* x, int64_t ldx, const int8_t* qp, const float* s, void* y,
                        int64_t ldy, int64_t M, int64_t N, int64_t K, int algo, void* workspace,
                        int64_t workspace_bytes, void* stream);

/*
 * Dynamic per-token activation quantization (W8A8 first stage).
 *   sx[m] = fl32(max_k |x[m,k]| / 127)     (an all-zero row gets sx[m] = 1)
 *   xq[m,k] = clamp(rne(fl32(x[m,k] / sx[m])), -127, 127)
 * x: (M, K) bf16, row stride ldx. xq: (M, K) int8 contiguous. sx: (M) fp32.
 * Replaces: nothing in the reference; it is the activation half of the int8 path the switch at
 * model_runner.py:45-46 names.
 */
int lse_quantize_act_per_token(const void* x, int64_t ldx, int8_t* xq, float* sx,
                               int64_t M, int64_t K, void* stream);

/*
 * RMSNorm followed by per-token quantization, in one pass over each token row (the W8A8 first
 * stage fused into the decoder's norms). With the rounding steps of LlamaRMSNorm:
 *   r = 1 / sqrt(fl32(sum_k x[m,k]^2 / K) + eps),  h[m,k] = bf16(weight[k] * bf16(x[m,k] * r))
 * then sx[m] and xq[m,k] from h exactly as lse_quantize_act_per_token computes them from a bf16
 * row. The sum of squares runs in a fixed fp32 order (tree over the row), so h can differ from
 * another implementation's in the last bf16 place where x * r lies at a rounding boundary.
 * x: (M, K) bf16, row stride ldx (multiple of 8, 16-byte aligned). weight: (K) bf16, 16-byte
 * aligned. xq: (M, K) int8 contiguous. sx: (M) fp32. normed: (M, K) bf16 contiguous receiving h,
 * or NULL. K % LSE_K_ALIGN == 0.
 * Replaces: `input_layernorm` / `post_attention_layernorm` (LlamaRMSNorm.forward,
 * modeling_llama.py:62-67) at model_runner.py:222-223, followed by the activation quantization
 * of the W8A8 mode.
 */
int lse_rmsnorm_quantize(const void* x, int64_t ldx, const void* weight, float eps, int8_t* xq,
                         float* sx, void* normed, int64_t M, int64_t K, void* stream);

/*
 * W8A8 linear: acc[m,n] = sum_k xq[m,k] * q[n,k] exactly in int32;
 *   y[m,n] = bf16_rne((fp32(acc[m,n]) * sx[m]) * s[n]).
 * xq: (M, K) int8 contiguous; qp: packed (N, K) int8 weight; K % LSE_K_ALIGN == 0,
 * K <= LSE_MAX_K. y: (M, N) bf16 with row stride ldy >= N, or NULL to skip it.
 * acc: (M, N) int32 contiguous, or NULL to skip it (the bit-exact test reads it).
 * workspace: as for lse_w8a16_gemm, sized by lse_workspace_bytes(LSE_MODE_W8A8, M, N, K).
 * Replaces: `F.linear(x, W)` (torch/nn/modules/linear.py:134) at the same call sites as
 * lse_w8a16_gemm, in the dynamic per-token mode.
 */
int lse_w8a8_gemm(const int8_t* xq, const float* sx, const int8_t* qp, const float* s, void* y,
                  int64_t ldy, int32_t* acc, int64_t M, int64_t N, int64_t K, void* workspace,
                  int64_t workspace_bytes, void* stream);

/*
 * W8A8 linear from bf16 activations in one launch: y (and acc) exactly as
 * lse_quantize_act_per_token followed by lse_w8a8_gemm compute them, bit for bit, with the
 * per-token quantization done by the GEMM kernel itself (no xq / sx round trip, one launch).
 * x: (M, K) bf16, row stride ldx (multiple of 8, 16-byte aligned base); the rest as for
 * lse_w8a8_gemm. Needs no workspace. Runs when lse_w8a8_linear_supported(M, K) (small decode
 * batches: M <= 16 and M * K int8 bytes fit the kernel's staged image); otherwise returns
 * LSE_E_ALGO and the caller quantizes and calls lse_w8a8_gemm.
 * Replaces: `F.linear(x, W)` (torch/nn/modules/linear.py:134) at the decode call sites of the
 * dynamic per-token mode, where x arrives in bf16 (o_proj after attention, down_proj after the
 * SiLU-mul; model_runner.py:369, modeling_llama.py:175).
 */
int lse_w8a8_linear_supported(int64_t M, int64_t K);
int lse_w8a8_linear(const void* x, int64_t ldx, const int8_t* qp, const float* s, void* y,
                    int64_t ldy, int32_t* acc, int64_t M, int64_t N, int64_t K, void* stream);

/* Bytes of the packed gate/up layout of two (I, K) weights: 2 * ceil(I/16) * ceil(K/64) * 1024. */
int64_t lse_packed_glu_bytes(int64_t I, int64_t K);

/*
 * Packs the MLP's stacked gate/up weight, row-major (2I, K) int8 = [gate rows 0..I-1; up rows
 * 0..I-1] (contiguous, K % LSE_K_ALIGN == 0, 16-byte aligned), into the gate/up layout the GLU
 * entry points read (qp: lse_packed_glu_bytes(I, K) bytes, 16-byte aligned): packed row tile 2t
 * is the lse_pack_weight tile of gate rows 16t..16t+15, row tile 2t+1 that of the same up rows,
 * zero past I. Load time only.
 * Replaces: the separate `gate_proj.weight` and `up_proj.weight` of `LlamaMLP`
 * (modeling_llama.py:169-170) at the int8 switch (model_runner.py:45-46).
 */
int lse_pack_glu(const int8_t* q, int64_t I, int64_t K, int8_t* qp, void* stream);

/*
 * Fused gate/up projection and SiLU-mul, W8A16. For n < I, in fp32:
 *   g = s[n] * sum_k x[m,k] q[n,k],   u = s[I+n] * sum_k x[m,k] q[I+n,k],
 *   h[m,n] = bf16_rne(silu(g) * u),   silu(v) = v / (1 + e^-v),
 * q being the stacked (2I, K) weight given packed by lse_pack_glu and s its (2I) fp32 scales
 * [gate; up]. x as for lse_w8a16_gemm (K % LSE_K_ALIGN == 0). h: (M, I) bf16, row stride
 * ldh >= I. algo: enum lse_algo, as for lse_w8a16_gemm_algo. Needs no workspace.
 * Replaces: `self.act_fn(self.gate_proj(x)) * self.up_proj(x)` in `LlamaMLP.forward`
 * (modeling_llama.py:175, reached from decoder_hidden, model_runner.py:223): two GEMMs, the
 * activation and the product, each rounding to bf16, become one kernel that rounds once.
 */
int lse_w8a16_glu(const void* x, int64_t ldx, const int8_t* qp, const float* s, void* h,
                  int64_t ldh, int64_t M, int64_t I, int64_t K, int algo, void* stream);

/*
 * Fused gate/up projection and SiLU-mul, W8A8: with xq, sx from lse_quantize_act_per_token and
 * acc_g, acc_u the exact int32 sums of gate row n and up row n,
 *   g = (fp32(acc_g) * sx[m]) * s[n],   u = (fp32(acc_u) * sx[m]) * s[I+n],
 *   h[m,n] = bf16_rne(silu(g) * u).
 * Operands as for lse_w8a8_gemm (K <= LSE_MAX_K) and lse_w8a16_glu. Needs no workspace.
 * Replaces: the same LlamaMLP expression (modeling_llama.py:175) in the dynamic per-token mode.
 */
int lse_w8a8_glu(const int8_t* xq, const float* sx, const int8_t* qp, const float* s, void* h,
                 int64_t ldh, int64_t M, int64_t I, int64_t K, void* stream);

/*
 * Bytes of device workspace (16-byte aligned) lse_paged_attention needs for these sizes on the
 * current device: 0 when every (entry, K/V head, query tile) takes its whole context in one
 * workgroup, the partial results of the key partitions otherwise. -1 for invalid sizes.
 * Replaces: nothing in the reference (its Triton launch needs no scratch).
 */
int64_t lse_paged_attention_workspace_bytes(int64_t entries, int64_t H, int64_t H_KV, int64_t D,
                                            int64_t max_q_len, int64_t max_blocks,
                                            int64_t block_size);

/*
 * Paged attention of a whole batch plan at one layer against a shared K/V pool. For entry e,
 * query row m < q_len[e] (q row q_start[e] + m, cache position query_offset[e] + m) and head h:
 *   o[h][q_start[e] + m] = sum_n softmax_n(softmax_scale * q[h][q_start[e] + m] . k_n) v_n
 * over cache positions n < context_len[e] with n <= query_offset[e] + m, where position n of
 * entry e lives in pool block block_table[e][n / block_size], slot n % block_size, K/V head
 * h / (H / H_KV). fp32 online softmax; probabilities rounded to bf16 before the product with V;
 * bf16 output (a row with no position is written as zeros).
 * q, o: bf16, element (h, t, d) at h * stride_h + t * stride_t + d. k_pool, v_pool: bf16
 *   (blocks, block_size, H_KV, D), element (b, w, kh, d) at b * pool_stride_block +
 *   w * pool_stride_slot + kh * pool_stride_head + d (the same strides for both).
 * block_table: (entries, >= max_blocks) int32, row stride block_table_stride; context_len,
 *   query_offset, q_start, q_len: (entries) int32. Their values must describe positions inside
 *   the pool and rows inside q/o (the kernel reads only blocks the table names for positions
 *   below context_len), as for the reference kernel.
 * Shapes: D = 128; H a multiple of H_KV with 1 <= H / H_KV <= 16; strides multiples of 8
 *   elements and base pointers 16-byte aligned. max_q_len >= every q_len (a graphed decode may
 *   pass its bucket size). workspace as sized by lse_paged_attention_workspace_bytes.
 * Determinism: each row's keys are summed in fixed 1024-position chunks, merged in a fixed order,
 *   so a row's output does not depend on the other entries, the entry count, max_q_len or the
 *   table width (a graph bucket with q_len = 0 padding rows and a pool-wide table gives the bits
 *   an exact-width eager call gives).
 * Replaces: `paged_attention_forward` (src/llm_serving_engine/kernels/flash_attention.py:
 *   287-332, the Triton kernel `paged_attention_2` at :201-284), called from
 *   `ModelRunner.attend_paged` (model_runner.py:357-363).
 */
int lse_paged_attention(const void* q, int64_t q_stride_h, int64_t q_stride_t,
                        const void* k_pool, const void* v_pool, int64_t pool_stride_block,
                        int64_t pool_stride_slot, int64_t pool_stride_head,
                        const int32_t* block_table, int64_t block_table_stride,
                        const int32_t* context_len, const int32_t* query_offset,
                        const int32_t* q_start, const int32_t* q_len, void* o,
                        int64_t o_stride_h, int64_t o_stride_t, int64_t entries, int64_t H,
                        int64_t H_KV, int64_t D, int64_t block_size, int64_t max_blocks,
                        int64_t max_q_len, float softmax_scale, void* workspace,
                        int64_t workspace_bytes, void* stream);

/* Bytes of the bf16 tile layout of an (N, K) weight: ceil(N/16) * ceil(K/64) * 2048. */
int64_t lse_packed_bf16_weight_bytes(int64_t N, int64_t K);

/*
 * Packs a row-major (N, K) bf16 weight (row stride ldw, a multiple of 8, 16-byte aligned;
 * K % LSE_K_ALIGN == 0) into the bf16 tile layout lse_bf16_decode_gemm reads: 16 rows x 64 K
 * per step, 2 KB, byte (rb * ceil(K/64) + j) * 2048 + 1024 h + 16 l + 2 i holding
 * w[16 rb + l % 16][64 j + 16 (l / 16) + 8 h + i], zero past N and K. Load time only.
 * Replaces: the row-major bf16 `lm_head.weight` (its storage step; the reference computes
 * `get_output_embeddings()(hidden)` at model_runner.py:306-307).
 */
int lse_pack_bf16_weight(const void* w, int64_t ldw, int64_t N, int64_t K, void* wp,
                         void* stream);

/*
 * bf16 linear over the packed bf16 layout (the lm_head the int8 path keeps in bf16), built for
 * decode-sized batches and correct for any M:
 *   y[m,n] = bf16_rne(sum_k x[m,k] * w[n,k]), fp32 accumulation.
 * x: (M, K) bf16, row stride ldx (multiple of 8, 16-byte aligned). wp: lse_pack_bf16_weight
 * layout. y: (M, N) bf16, row stride ldy >= N. Deterministic as the int8 decode GEMMs are: a
 * row's bits depend on N, K and its token class (1..16, 17..32, 33..64, above 64) only.
 * Replaces: `F.linear(hidden, lm_head.weight)` in `emit_owed` (model_runner.py:306-307) and the
 * graphed decode step (decode_graph.py:140).
 */
int lse_bf16_decode_gemm(const void* x, int64_t ldx, const void* wp, void* y, int64_t ldy,
                         int64_t M, int64_t N, int64_t K, void* stream);

/* Static properties (enum lse_query_key); -1 for an unknown key. Load-time checks read these,
 * as `ModelRunner.check_custom_kernel_support` (model_runner.py:77-94) checks its kernels. */
int64_t lse_query(int key);

/* Text for a status code returned above (never NULL). */
const char* lse_status_string(int status);

#ifdef __cplusplus
}
#endif

#endif /* LSE_INT8_H */
