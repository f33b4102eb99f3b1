// lse_w8a16_gemm_noalloc: the W8A16 linear for callers that cannot allocate device memory (code
// under HIP graph capture that may not grow a pool, tight serving loops, harnesses that forbid
// hipMalloc). It is lse_w8a16_gemm with its workspace (the split-K partial sums some decode
// shapes add in a second pass) taken from `scratch`, a file-scope device array of a fixed size,
// instead of from the caller.
//
// Each device holds its own copy of `scratch` at its own address, kept until the process ends.
// In host code the array's name is only a host-side stand-in, so its device address is looked up
// once per device with hipGetSymbolAddress, with that device current, and only that address is
// ever passed to a kernel; a call with M = 0 does only that lookup, for callers that capture
// their first real call into a graph. Every call on a device shares the device's array and
// leaves the last call's partial sums in it: calls that overlap on one device (two streams at
// once) race. Nothing needs clearing between calls: each call writes every partial sum it reads
// before reading it.
#include <mutex>

#include "lse_common.h"

namespace {

constexpr int64_t kScratchBytes = LSE_NOALLOC_SCRATCH_BYTES;
__device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex scratch_mu;
void* scratch_addr[kMaxDevices];  // device address of `scratch` per device, once looked up

// The current device's address of `scratch`, looked up on the device's first call.
int device_scratch(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return LSE_E_RANGE;
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (!scratch_addr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!p) return LSE_E_NULL;
    scratch_addr[dev] = p;
  }
  *out = scratch_addr[dev];
  return LSE_OK;
}

}  // namespace

extern "C" {

int lse_w8a16_gemm_noalloc(const void* x, int64_t ldx, const int8_t* qp, const float* s, void* y,
                           int64_t ldy, int64_t M, int64_t N, int64_t K, void* stream) {
  const int64_t need = lse_workspace_bytes(LSE_MODE_W8A16, M, N, K);
  if (need < 0) return LSE_E_SHAPE;
  if (need > kScratchBytes) return LSE_E_SCRATCH;
  void* ws = nullptr;
  // A call with M = 0 launches nothing and only looks the current device's address up, so a
  // caller can do that before it starts a graph capture.
  if (M == 0) return device_scratch(&ws);
  if (N > 0) {
    if (int st = device_scratch(&ws)) return st;
  }
  return lse_w8a16_gemm(x, ldx, qp, s, y, ldy, M, N, K, need > 0 ? ws : nullptr, need, stream);
}

}  // extern "C"
