// extern "C" entry points of liblse_int8.so (declared in include/lse_int8.h): argument checks,
// then dispatch to the kernels. A rejected argument returns a negative status before anything is
// launched; a launch failure returns the hipError_t.
#include <algorithm>
#include <mutex>

#include "lse_common.h"

namespace lse {
int launch_quantize_weight(const float* w, int64_t ldw, int8_t* q, float* s, int64_t N, int64_t K,
                           hipStream_t stream);
int launch_quantize_act(const uint16_t* x, int64_t ldx, int8_t* xq, float* sx, int64_t M,
                        int64_t K, hipStream_t stream);
int launch_rmsnorm_quantize(const uint16_t* x, int64_t ldx, const uint16_t* w, float eps,
                            int8_t* xq, float* sx, uint16_t* normed, int64_t M, int64_t K,
                            hipStream_t stream);
int launch_pack_weight(const int8_t* q, int64_t N, int64_t K, int8_t* qp, hipStream_t stream);
int launch_pack_glu(const int8_t* q, int64_t I, int64_t K, int8_t* qp, hipStream_t stream);
int64_t packed_weight_bytes(int64_t N, int64_t K);
int64_t packed_glu_bytes(int64_t I, int64_t K);
int64_t skinny_workspace_bytes(bool i8, int64_t M, int64_t N, int64_t K);
int launch_w8a16_skinny(const uint16_t* x, int64_t ldx, const int8_t* qp, const float* s,
                        uint16_t* y, int64_t ldy, int64_t M, int64_t N, int64_t K, void* ws,
                        int64_t ws_bytes, hipStream_t stream);
int launch_w8a8_skinny(const int8_t* xq, const float* sx, const int8_t* qp, const float* s,
                       uint16_t* y, int64_t ldy, int32_t* acc, int64_t M, int64_t N, int64_t K,
                       void* ws, int64_t ws_bytes, hipStream_t stream);
bool w8a8_quantizing_supported(int64_t M, int64_t K);
int launch_w8a8_skinny_quantizing(const uint16_t* x, int64_t ldx, const int8_t* qp,
                                  const float* s, uint16_t* y, int64_t ldy, int32_t* acc,
                                  int64_t M, int64_t N, int64_t K, hipStream_t stream);
int64_t tiled_workspace_bytes(bool i8, int64_t M, int64_t N, int64_t K);
int launch_w8a16_gemm(const uint16_t* x, int64_t ldx, const int8_t* q, const float* s, uint16_t* y,
                      int64_t ldy, int64_t M, int64_t N, int64_t K, void* ws, int64_t ws_bytes,
                      hipStream_t stream);
int launch_w8a8_gemm(const int8_t* xq, const float* sx, const int8_t* q, const float* s,
                     uint16_t* y, int64_t ldy, int32_t* acc, int64_t M, int64_t N, int64_t K,
                     void* ws, int64_t ws_bytes, hipStream_t stream);
int launch_w8a16_skinny_glu(const uint16_t* x, int64_t ldx, const int8_t* qp, const float* s,
                            uint16_t* h, int64_t ldh, int64_t M, int64_t I, int64_t K,
                            hipStream_t stream);
int launch_w8a8_skinny_glu(const int8_t* xq, const float* sx, const int8_t* qp, const float* s,
                           uint16_t* h, int64_t ldh, int64_t M, int64_t I, int64_t K,
                           hipStream_t stream);
int launch_w8a16_gemm_glu(const uint16_t* x, int64_t ldx, const int8_t* qp, const float* s,
                          uint16_t* h, int64_t ldh, int64_t M, int64_t I, int64_t K,
                          hipStream_t stream);
int launch_w8a8_gemm_glu(const int8_t* xq, const float* sx, const int8_t* qp, const float* s,
                         uint16_t* h, int64_t ldh, int64_t M, int64_t I, int64_t K,
                         hipStream_t stream);
int64_t packed_bf16_bytes(int64_t N, int64_t K);
int launch_pack_bf16(const uint16_t* w, int64_t ldw, int64_t N, int64_t K, uint16_t* wp,
                     hipStream_t stream);
int launch_bf16_skinny(const uint16_t* x, int64_t ldx, const uint16_t* wp, uint16_t* y,
                       int64_t ldy, int64_t M, int64_t N, int64_t K, hipStream_t stream);
int64_t paged_attention_workspace_bytes(int64_t entries, int64_t H, int64_t HKV, int64_t D,
                                        int64_t max_q_len, int64_t max_ctx);
int launch_paged_attention(const uint16_t* q, int64_t sq_h, int64_t sq_t, const uint16_t* k_pool,
                           const uint16_t* v_pool, int64_t sb, int64_t sw, int64_t sh,
                           const int32_t* block_table, int64_t sbt, const int32_t* context_len,
                           const int32_t* query_offset, const int32_t* q_start,
                           const int32_t* q_len, uint16_t* o, int64_t so_h, int64_t so_t,
                           int64_t entries, int64_t H, int64_t HKV, int64_t block_size,
                           int64_t max_blocks, int64_t max_q_len, float softmax_scale, void* ws,
                           int64_t ws_bytes, hipStream_t stream);
}  // namespace lse

namespace lse {

int persistent_blocks(const void* kernel, int threads, size_t dyn_lds) {
  // A fixed table, so no launch path allocates (host or device); past its size the occupancy
  // query simply runs again.
  struct Entry {
    int device;
    const void* kernel;
    size_t dyn_lds;
    int blocks;
  };
  constexpr int kEntries = 512;
  static std::mutex mu;
  static Entry cache[kEntries];
  static int used = 0;
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return 1;
  std::lock_guard<std::mutex> lock(mu);
  for (int i = 0; i < used; ++i) {
    const Entry& e = cache[i];
    if (e.device == device && e.kernel == kernel && e.dyn_lds == dyn_lds) return e.blocks;
  }
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, dyn_lds) !=
          hipSuccess) {
    (void)hipGetLastError();
    return 256;
  }
  const int blocks = std::max(1, cus * std::max(1, per_cu));
  if (used < kEntries) cache[used++] = Entry{device, kernel, dyn_lds, blocks};
  return blocks;
}

}  // namespace lse

namespace {

constexpr int64_t kMaxGridX = 2147483647;
constexpr int64_t kMaxRows = 2147483647;  // row indices are int inside the kernels
constexpr uint32_t kBufferLimit = lse::kOutOfRange;  // byte extent of a buffer resource

bool aligned(const void* p, uintptr_t bytes) { return ((uintptr_t)p % bytes) == 0; }

// Checks shared by every GEMM-shaped entry point: sizes, K alignment and range, scale vector.
int check_common(const int8_t* q, const float* s, int64_t M, int64_t N, int64_t K) {
  if (M < 0 || N < 0 || K < 0 || M > kMaxRows || N > kMaxRows) return LSE_E_SHAPE;
  if (K % LSE_K_ALIGN) return LSE_E_ALIGN;
  if (K > LSE_MAX_K) return LSE_E_RANGE;
  if (M == 0 || N == 0) return LSE_OK;
  if (!q || !s) return LSE_E_NULL;
  if (!aligned(q, 16) || !aligned(s, 16)) return LSE_E_ALIGN;
  return LSE_OK;
}

int check_bf16_matrix(const void* p, int64_t ld, int64_t rows, int64_t cols, int elem_align) {
  if (rows == 0 || cols == 0) return LSE_OK;
  if (!p) return LSE_E_NULL;
  if (ld < cols) return LSE_E_SHAPE;
  if (ld % elem_align || !aligned(p, 2 * elem_align)) return LSE_E_ALIGN;
  return LSE_OK;
}

// y[m, :] = 0 when K == 0: the empty sum. Written as a plain kernel so the call stays
// capture-safe (no memset node).
__global__ void zero_rows(uint16_t* y, int64_t ldy, int64_t M, int64_t N) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < M * N) y[(i / N) * ldy + i % N] = 0;
}

int zero_output(void* y, int64_t ldy, int64_t M, int64_t N, hipStream_t stream) {
  const int64_t total = M * N;
  const int64_t blocks = (total + 255) / 256;
  if (blocks > kMaxGridX) return LSE_E_RANGE;
  hipLaunchKernelGGL(zero_rows, dim3((unsigned)blocks), dim3(256), 0, stream, (uint16_t*)y, ldy, M,
                     N);
  return lse::launch_status();
}

__global__ void zero_i32(int32_t* p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

// The packed weight and the 32-bit buffer offsets the kernels address it with.
int check_packed(int64_t N, int64_t K) {
  return lse::packed_weight_bytes(N, K) < (int64_t)kBufferLimit ? LSE_OK : LSE_E_RANGE;
}

int check_packed_glu(int64_t I, int64_t K) {
  return lse::packed_glu_bytes(I, K) < (int64_t)kBufferLimit ? LSE_OK : LSE_E_RANGE;
}

}  // namespace

extern "C" {

int lse_quantize_weight_per_channel(const float* w, int64_t ldw, int8_t* q, float* s, int64_t N,
                                    int64_t K, void* stream) {
  if (N < 0 || K < 0 || N > kMaxGridX) return LSE_E_SHAPE;
  if (K % LSE_K_ALIGN) return LSE_E_ALIGN;
  if (N == 0) return LSE_OK;
  if (!s || (K > 0 && (!w || !q))) return LSE_E_NULL;
  if (K > 0 && ldw < K) return LSE_E_SHAPE;
  if (K > 0 && (ldw % 4 || !aligned(w, 16) || !aligned(q, 16))) return LSE_E_ALIGN;
  return lse::launch_quantize_weight(w, ldw, q, s, N, K, (hipStream_t)stream);
}

int lse_quantize_act_per_token(const void* x, int64_t ldx, int8_t* xq, float* sx, int64_t M,
                               int64_t K, void* stream) {
  if (M < 0 || K < 0 || M > kMaxGridX) return LSE_E_SHAPE;
  if (K % LSE_K_ALIGN) return LSE_E_ALIGN;
  if (M == 0) return LSE_OK;
  if (!sx || (K > 0 && !xq)) return LSE_E_NULL;
  if (int st = check_bf16_matrix(x, ldx, M, K, 8)) return st;
  if (K > 0 && !aligned(xq, 16)) return LSE_E_ALIGN;
  return lse::launch_quantize_act((const uint16_t*)x, ldx, xq, sx, M, K, (hipStream_t)stream);
}

int lse_rmsnorm_quantize(const void* x, int64_t ldx, const void* weight, float eps, int8_t* xq,
                         float* sx, void* normed, int64_t M, int64_t K, void* stream) {
  if (M < 0 || K < 0 || M > kMaxGridX) return LSE_E_SHAPE;
  if (K % LSE_K_ALIGN) return LSE_E_ALIGN;
  if (M == 0 || K == 0) return LSE_OK;
  if (!weight || !xq || !sx) return LSE_E_NULL;
  if (int st = check_bf16_matrix(x, ldx, M, K, 8)) return st;
  if (!aligned(weight, 16) || !aligned(xq, 16) || (normed && !aligned(normed, 16)))
    return LSE_E_ALIGN;
  if (!(eps >= 0.0f)) return LSE_E_SHAPE;
  return lse::launch_rmsnorm_quantize((const uint16_t*)x, ldx, (const uint16_t*)weight, eps, xq,
                                      sx, (uint16_t*)normed, M, K, (hipStream_t)stream);
}

int64_t lse_packed_weight_bytes(int64_t N, int64_t K) {
  if (N < 0 || K < 0) return -1;
  return lse::packed_weight_bytes(N, K);
}

int lse_pack_weight(const int8_t* q, int64_t N, int64_t K, int8_t* qp, void* stream) {
  if (N < 0 || K < 0 || N > kMaxRows) return LSE_E_SHAPE;
  if (K % LSE_K_ALIGN) return LSE_E_ALIGN;
  if (N == 0 || K == 0) return LSE_OK;
  if (!q || !qp) return LSE_E_NULL;
  if (!aligned(q, 16) || !aligned(qp, 16)) return LSE_E_ALIGN;
  if (int st = check_packed(N, K)) return st;
  return lse::launch_pack_weight(q, N, K, qp, (hipStream_t)stream);
}

int64_t lse_packed_glu_bytes(int64_t I, int64_t K) {
  if (I < 0 || K < 0) return -1;
  return lse::packed_glu_bytes(I, K);
}

int lse_pack_glu(const int8_t* q, int64_t I, int64_t K, int8_t* qp, void* stream) {
  if (I < 0 || K < 0 || 2 * I > kMaxRows) return LSE_E_SHAPE;
  if (K % LSE_K_ALIGN) return LSE_E_ALIGN;
  if (I == 0 || K == 0) return LSE_OK;
  if (!q || !qp) return LSE_E_NULL;
  if (!aligned(q, 16) || !aligned(qp, 16)) return LSE_E_ALIGN;
  if (int st = check_packed_glu(I, K)) return st;
  return lse::launch_pack_glu(q, I, K, qp, (hipStream_t)stream);
}

int64_t lse_workspace_bytes(int mode, int64_t M, int64_t N, int64_t K) {
  if (M < 0 || N < 0 || K < 0 || (mode != LSE_MODE_W8A16 && mode != LSE_MODE_W8A8)) return -1;
  // Split-K partial sums: the decode kernel's (M <= 64) or the tiled kernel's (65..256 tokens
  // over a narrow weight). The tiled kernel needs none at M <= 64, so the bound holds for either
  // algorithm; shapes the entry points reject need none.
  if (M == 0 || N == 0 || K == 0 || M > kMaxRows || N > kMaxRows || K > LSE_MAX_K ||
      K % LSE_K_ALIGN)
    return 0;
  const bool i8 = mode == LSE_MODE_W8A8;
  return M <= LSE_DECODE_MAX_M ? lse::skinny_workspace_bytes(i8, M, N, K)
                               : lse::tiled_workspace_bytes(i8, M, N, K);
}

int lse_w8a16_gemm_algo(const void* x, int64_t ldx, const int8_t* qp, const float* s, void* y,
                        int64_t ldy, int64_t M, int64_t N, int64_t K, int algo, void* workspace,
                        int64_t workspace_bytes, void* stream) {
  if (int st = check_common(qp, s, M, N, K)) return st;
  if (algo < LSE_ALGO_AUTO || algo > LSE_ALGO_PREFILL) return LSE_E_ALGO;
  if (algo == LSE_ALGO_DECODE && M > LSE_DECODE_MAX_M) return LSE_E_ALGO;
  if (M == 0 || N == 0) return LSE_OK;
  if (int st = check_bf16_matrix(y, ldy, M, N, 1)) return st;
  hipStream_t st = (hipStream_t)stream;
  if (K == 0) return zero_output(y, ldy, M, N, st);
  if (int e = check_bf16_matrix(x, ldx, M, K, 8)) return e;
  if (int e = check_packed(N, K)) return e;
  if (algo == LSE_ALGO_AUTO) algo = M <= LSE_DECODE_MAX_M ? LSE_ALGO_DECODE : LSE_ALGO_PREFILL;
  if (workspace_bytes < 0 || (workspace && !aligned(workspace, 16))) return LSE_E_WORKSPACE;
  if (algo == LSE_ALGO_DECODE) {
    // The decode kernel addresses x through a 32-bit buffer resource.
    if (((M - 1) * ldx + K) * 2 >= (int64_t)kBufferLimit) return LSE_E_RANGE;
    return lse::launch_w8a16_skinny((const uint16_t*)x, ldx, qp, s, (uint16_t*)y, ldy, M, N, K,
                                    workspace, workspace_bytes, st);
  }
  // The tiled kernel addresses a block's 256 rows of x through a 32-bit buffer resource.
  if (256 * ldx * 2 >= (int64_t)kBufferLimit) return LSE_E_RANGE;
  return lse::launch_w8a16_gemm((const uint16_t*)x, ldx, qp, s, (uint16_t*)y, ldy, M, N, K,
                                workspace, workspace_bytes, st);
}

int lse_w8a16_gemm(const void* x, int64_t ldx, const int8_t* qp, const float* s, void* y,
                   int64_t ldy, int64_t M, int64_t N, int64_t K, void* workspace,
                   int64_t workspace_bytes, void* stream) {
  return lse_w8a16_gemm_algo(x, ldx, qp, s, y, ldy, M, N, K, LSE_ALGO_AUTO, workspace,
                             workspace_bytes, stream);
}

int lse_w8a8_gemm(const int8_t* xq, const float* sx, const int8_t* qp, const float* s, void* y,
                  int64_t ldy, int32_t* acc, int64_t M, int64_t N, int64_t K, void* workspace,
                  int64_t workspace_bytes, void* stream) {
  if (int st = check_common(qp, s, M, N, K)) return st;
  if (M == 0 || N == 0) return LSE_OK;
  if (!sx) return LSE_E_NULL;
  if (y) {
    if (int st = check_bf16_matrix(y, ldy, M, N, 1)) return st;
  }
  if (acc && !aligned(acc, 16)) return LSE_E_ALIGN;
  hipStream_t st = (hipStream_t)stream;
  if (K == 0) {
    if (acc) {
      hipLaunchKernelGGL(zero_i32, dim3((unsigned)((M * N + 255) / 256)), dim3(256), 0, st, acc,
                         M * N);
      if (int e = lse::launch_status()) return e;
    }
    return y ? zero_output(y, ldy, M, N, st) : LSE_OK;
  }
  if (!xq) return LSE_E_NULL;
  if (!aligned(xq, 16)) return LSE_E_ALIGN;
  if (int e = check_packed(N, K)) return e;
  if (workspace_bytes < 0 || (workspace && !aligned(workspace, 16))) return LSE_E_WORKSPACE;
  if (M <= LSE_DECODE_MAX_M) {
    if (M * K >= (int64_t)kBufferLimit) return LSE_E_RANGE;
    return lse::launch_w8a8_skinny(xq, sx, qp, s, (uint16_t*)y, ldy, acc, M, N, K, workspace,
                                   workspace_bytes, st);
  }
  if (256 * K >= (int64_t)kBufferLimit) return LSE_E_RANGE;
  return lse::launch_w8a8_gemm(xq, sx, qp, s, (uint16_t*)y, ldy, acc, M, N, K, workspace,
                               workspace_bytes, st);
}

int lse_w8a8_linear_supported(int64_t M, int64_t K) {
  return K > 0 && K % LSE_K_ALIGN == 0 && K <= LSE_MAX_K && lse::w8a8_quantizing_supported(M, K);
}

int lse_w8a8_linear(const void* x, int64_t ldx, const int8_t* qp, const float* s, void* y,
                    int64_t ldy, int32_t* acc, int64_t M, int64_t N, int64_t K, void* stream) {
  if (int st = check_common(qp, s, M, N, K)) return st;
  if (M == 0 || N == 0) return LSE_OK;
  if (!lse_w8a8_linear_supported(M, K)) return LSE_E_ALGO;
  if (y) {
    if (int st = check_bf16_matrix(y, ldy, M, N, 1)) return st;
  }
  if (acc && !aligned(acc, 16)) return LSE_E_ALIGN;
  if (int e = check_bf16_matrix(x, ldx, M, K, 8)) return e;
  if (int e = check_packed(N, K)) return e;
  return lse::launch_w8a8_skinny_quantizing((const uint16_t*)x, ldx, qp, s, (uint16_t*)y, ldy,
                                            acc, M, N, K, (hipStream_t)stream);
}

int lse_w8a16_glu(const void* x, int64_t ldx, const int8_t* qp, const float* s, void* h,
                  int64_t ldh, int64_t M, int64_t I, int64_t K, int algo, void* stream) {
  if (I < 0 || 2 * I > kMaxRows) return LSE_E_SHAPE;
  if (int st = check_common(qp, s, M, 2 * I, K)) return st;
  if (algo < LSE_ALGO_AUTO || algo > LSE_ALGO_PREFILL) return LSE_E_ALGO;
  if (algo == LSE_ALGO_DECODE && M > LSE_DECODE_MAX_M) return LSE_E_ALGO;
  if (M == 0 || I == 0) return LSE_OK;
  if (int st = check_bf16_matrix(h, ldh, M, I, 1)) return st;
  hipStream_t st = (hipStream_t)stream;
  if (K == 0) return zero_output(h, ldh, M, I, st);  // silu(0) * 0
  if (int e = check_bf16_matrix(x, ldx, M, K, 8)) return e;
  if (int e = check_packed_glu(I, K)) return e;
  if (algo == LSE_ALGO_AUTO) algo = M <= LSE_DECODE_MAX_M ? LSE_ALGO_DECODE : LSE_ALGO_PREFILL;
  if (algo == LSE_ALGO_DECODE) {
    if (((M - 1) * ldx + K) * 2 >= (int64_t)kBufferLimit) return LSE_E_RANGE;
    return lse::launch_w8a16_skinny_glu((const uint16_t*)x, ldx, qp, s, (uint16_t*)h, ldh, M, I,
                                        K, st);
  }
  if (256 * ldx * 2 >= (int64_t)kBufferLimit) return LSE_E_RANGE;
  return lse::launch_w8a16_gemm_glu((const uint16_t*)x, ldx, qp, s, (uint16_t*)h, ldh, M, I, K,
                                    st);
}

int lse_w8a8_glu(const int8_t* xq, const float* sx, const int8_t* qp, const float* s, void* h,
                 int64_t ldh, int64_t M, int64_t I, int64_t K, void* stream) {
  if (I < 0 || 2 * I > kMaxRows) return LSE_E_SHAPE;
  if (int st = check_common(qp, s, M, 2 * I, K)) return st;
  if (M == 0 || I == 0) return LSE_OK;
  if (!sx) return LSE_E_NULL;
  if (int st = check_bf16_matrix(h, ldh, M, I, 1)) return st;
  hipStream_t st = (hipStream_t)stream;
  if (K == 0) return zero_output(h, ldh, M, I, st);
  if (!xq) return LSE_E_NULL;
  if (!aligned(xq, 16)) return LSE_E_ALIGN;
  if (int e = check_packed_glu(I, K)) return e;
  if (M <= LSE_DECODE_MAX_M) {
    if (M * K >= (int64_t)kBufferLimit) return LSE_E_RANGE;
    return lse::launch_w8a8_skinny_glu(xq, sx, qp, s, (uint16_t*)h, ldh, M, I, K, st);
  }
  if (256 * K >= (int64_t)kBufferLimit) return LSE_E_RANGE;
  return lse::launch_w8a8_gemm_glu(xq, sx, qp, s, (uint16_t*)h, ldh, M, I, K, st);
}

namespace {

// Sizes lse_paged_attention accepts (see include/lse_int8.h).
int check_attention_sizes(int64_t entries, int64_t H, int64_t HKV, int64_t D, int64_t max_q_len,
                          int64_t max_blocks, int64_t block_size) {
  if (entries < 0 || H < 1 || HKV < 1 || max_q_len < 0 || max_blocks < 0 || block_size < 1 ||
      entries > kMaxRows || H > 65536 || max_q_len > kMaxRows)
    return LSE_E_SHAPE;
  if (D != 128 || H % HKV) return LSE_E_SHAPE;
  if (H / HKV > 16) return LSE_E_SHAPE;  // a query tile holds at least one token's group
  if (max_blocks * block_size > kMaxRows) return LSE_E_RANGE;
  return LSE_OK;
}

}  // namespace

int64_t lse_paged_attention_workspace_bytes(int64_t entries, int64_t H, int64_t H_KV, int64_t D,
                                            int64_t max_q_len, int64_t max_blocks,
                                            int64_t block_size) {
  if (check_attention_sizes(entries, H, H_KV, D, max_q_len, max_blocks, block_size)) return -1;
  if (entries == 0 || max_q_len == 0) return 0;
  return lse::paged_attention_workspace_bytes(entries, H, H_KV, D, max_q_len,
                                              max_blocks * block_size);
}

int lse_paged_attention(const void* q, int64_t q_stride_h, int64_t q_stride_t,
                        const void* k_pool, const void* v_pool, int64_t pool_stride_block,
                        int64_t pool_stride_slot, int64_t pool_stride_head,
                        const int32_t* block_table, int64_t block_table_stride,
                        const int32_t* context_len, const int32_t* query_offset,
                        const int32_t* q_start, const int32_t* q_len, void* o,
                        int64_t o_stride_h, int64_t o_stride_t, int64_t entries, int64_t H,
                        int64_t H_KV, int64_t D, int64_t block_size, int64_t max_blocks,
                        int64_t max_q_len, float softmax_scale, void* workspace,
                        int64_t workspace_bytes, void* stream) {
  if (int st = check_attention_sizes(entries, H, H_KV, D, max_q_len, max_blocks, block_size))
    return st;
  if (entries == 0 || max_q_len == 0) return LSE_OK;
  if (!q || !k_pool || !v_pool || !block_table || !context_len || !query_offset || !q_start ||
      !q_len || !o)
    return LSE_E_NULL;
  if (q_stride_h < 0 || q_stride_t < 0 || o_stride_h < 0 || o_stride_t < 0 ||
      pool_stride_block < 0 || pool_stride_slot < 0 || pool_stride_head < 0 ||
      block_table_stride < max_blocks)
    return LSE_E_SHAPE;
  const int64_t strides[] = {q_stride_h, q_stride_t, o_stride_h, o_stride_t, pool_stride_block,
                             pool_stride_slot, pool_stride_head};
  for (int64_t s : strides)
    if (s % 8) return LSE_E_ALIGN;
  if (!aligned(q, 16) || !aligned(o, 16) || !aligned(k_pool, 16) || !aligned(v_pool, 16) ||
      !aligned(block_table, 4) || !aligned(context_len, 4) || !aligned(query_offset, 4) ||
      !aligned(q_start, 4) || !aligned(q_len, 4))
    return LSE_E_ALIGN;
  if (workspace_bytes < 0 || (workspace && !aligned(workspace, 16))) return LSE_E_WORKSPACE;
  return lse::launch_paged_attention(
      (const uint16_t*)q, q_stride_h, q_stride_t, (const uint16_t*)k_pool,
      (const uint16_t*)v_pool, pool_stride_block, pool_stride_slot, pool_stride_head, block_table,
      block_table_stride, context_len, query_offset, q_start, q_len, (uint16_t*)o, o_stride_h,
      o_stride_t, entries, H, H_KV, block_size, max_blocks, max_q_len, softmax_scale, workspace,
      workspace_bytes, (hipStream_t)stream);
}

int64_t lse_packed_bf16_weight_bytes(int64_t N, int64_t K) {
  if (N < 0 || K < 0) return -1;
  return lse::packed_bf16_bytes(N, K);
}

int lse_pack_bf16_weight(const void* w, int64_t ldw, int64_t N, int64_t K, void* wp,
                         void* stream) {
  if (N < 0 || K < 0 || N > kMaxRows) return LSE_E_SHAPE;
  if (K % LSE_K_ALIGN) return LSE_E_ALIGN;
  if (N == 0 || K == 0) return LSE_OK;
  if (!w || !wp) return LSE_E_NULL;
  if (int st = check_bf16_matrix(w, ldw, N, K, 8)) return st;
  if (!aligned(wp, 16)) return LSE_E_ALIGN;
  if (lse::packed_bf16_bytes(N, K) >= (int64_t)kBufferLimit) return LSE_E_RANGE;
  return lse::launch_pack_bf16((const uint16_t*)w, ldw, N, K, (uint16_t*)wp, (hipStream_t)stream);
}

int lse_bf16_decode_gemm(const void* x, int64_t ldx, const void* wp, void* y, int64_t ldy,
                         int64_t M, int64_t N, int64_t K, void* stream) {
  if (M < 0 || N < 0 || K < 0 || N > kMaxRows) return LSE_E_SHAPE;
  if (K % LSE_K_ALIGN) return LSE_E_ALIGN;
  if (M == 0 || N == 0) return LSE_OK;
  if (!wp) return LSE_E_NULL;
  if (!aligned(wp, 16)) return LSE_E_ALIGN;
  if (int st = check_bf16_matrix(y, ldy, M, N, 1)) return st;
  hipStream_t st = (hipStream_t)stream;
  if (K == 0) return zero_output(y, ldy, M, N, st);
  if (int e = check_bf16_matrix(x, ldx, M, K, 8)) return e;
  if (lse::packed_bf16_bytes(N, K) >= (int64_t)kBufferLimit) return LSE_E_RANGE;
  if (((M - 1) * ldx + K) * 2 >= (int64_t)kBufferLimit) return LSE_E_RANGE;
  return lse::launch_bf16_skinny((const uint16_t*)x, ldx, (const uint16_t*)wp, (uint16_t*)y, ldy,
                                 M, N, K, st);
}

int64_t lse_query(int key) {
  switch (key) {
    case LSE_Q_ABI_VERSION: return LSE_ABI_VERSION;
    case LSE_Q_K_ALIGN: return LSE_K_ALIGN;
    case LSE_Q_DECODE_MAX_M: return LSE_DECODE_MAX_M;
    case LSE_Q_MAX_K: return LSE_MAX_K;
    case LSE_Q_GFX_ARCH: return 950;
    case LSE_Q_NOALLOC_SCRATCH: return LSE_NOALLOC_SCRATCH_BYTES;
    default: return -1;
  }
}

const char* lse_status_string(int status) {
  switch (status) {
    case LSE_OK: return "ok";
    case LSE_E_NULL: return "a required pointer is NULL";
    case LSE_E_SHAPE: return "negative size or a stride smaller than its row";
    case LSE_E_ALIGN: return "K, a stride or a pointer is not aligned as the kernels require";
    case LSE_E_RANGE: return "size out of range (int32 accumulation or grid limits)";
    case LSE_E_ALGO: return "unknown algorithm, or one that cannot run this shape";
    case LSE_E_WORKSPACE: return "workspace missing, misaligned or smaller than lse_workspace_bytes";
    case LSE_E_SCRATCH:
      return "the call needs more workspace than lse_w8a16_gemm_noalloc's static scratch "
             "(LSE_NOALLOC_SCRATCH_BYTES) holds";
    default: return status > 0 ? hipGetErrorString((hipError_t)status) : "unknown status";
  }
}

}  // extern "C"
