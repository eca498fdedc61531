// The allocation-free form of f16_gemv_argmax_rows (include/q8gemv.h), for
// callers that cannot call hipMalloc: code under HIP graph capture, tight
// serving loops, harnesses that forbid allocation.
//
// The argmax key that the caller's `workspace` holds in f16_gemv_argmax_rows
// lives here in a file-scope device array, one copy per GPU, held until the
// process ends.  q8gemv_init looks up its address on the current device
// (hipGetSymbolAddress) and zero-fills it; the entry point then passes that
// address to the same two kernels as the workspace form.  The finalize kernel
// leaves the key zero again after every call, so each call starts from zero.
//
// Every call on one GPU shares that GPU's array: calls that overlap on one GPU
// (different streams, no ordering between them) race on the key and may
// return each other's token.
#include <hip/hip_runtime.h>

#include <mutex>

#include "q8gemv.h"
#include "shim_internal.h"

// The scratch: bytes 0-7 are the 64-bit argmax key, the rest is the 256-byte
// workspace the kernels are specified against (vocab_argmax_workspace_bytes).
// The size is fixed: no input size changes what the kernels use of it.
constexpr size_t kNoallocScratchBytes = 256;
static __device__ __align__(256) uint8_t scratch[kNoallocScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_scratch[kMaxDevices];  // device address of `scratch` on each device, set once

}  // namespace

namespace q8_shim {

int noalloc_setup(int device) {
  if (device < 0 || device >= kMaxDevices)
    return error(Q8_ERR_BAD_ARGUMENT, "device index beyond the allocation-free scratch table");
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_scratch[device] != nullptr) return Q8_OK;
  // `scratch` in host code is only a stand-in for the symbol; the device
  // address comes from the runtime, per device.
  void* ptr = nullptr;
  hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return hip_error(e, "hipGetSymbolAddress(scratch)");
  if (ptr == nullptr) return error(Q8_ERR_HIP, "hipGetSymbolAddress(scratch) gave a null address");
  e = hipMemset(ptr, 0, kNoallocScratchBytes);
  if (e != hipSuccess) return hip_error(e, "hipMemset(scratch)");
  g_scratch[device] = ptr;
  return Q8_OK;
}

}  // namespace q8_shim

extern "C" int f16_gemv_argmax_rows_noalloc(const void* w_f16, int64_t n_rows, const void* x_f16,
                                            void* logits_f16, int32_t* token, void* stream) {
  int rc = q8_shim::validate_f16_argmax(w_f16, n_rows, x_f16, logits_f16, token);
  if (rc) return rc;
  if ((rc = q8_shim::noalloc_ready())) return rc;
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return q8_shim::hip_error(e, "hipGetDevice");
  void* ptr = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_mu);
    if (dev >= 0 && dev < kMaxDevices) ptr = g_scratch[dev];
  }
  if (ptr == nullptr)
    return q8_shim::error(Q8_ERR_NOT_INITIALIZED,
                          "the allocation-free scratch is not set up on the current device "
                          "(call q8gemv_init with it current)");
  return q8_shim::launch_f16_argmax(w_f16, n_rows, x_f16, logits_f16, token, ptr,
                                    static_cast<hipStream_t>(stream));
}
