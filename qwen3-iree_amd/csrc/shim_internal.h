// Internal interface between the C-ABI shim (q8gemv_shim.cpp) and the
// allocation-free entry point (q8gemv_noalloc.hip); not part of the ABI.
#ifndef QWEN3_SHIM_INTERNAL_H
#define QWEN3_SHIM_INTERNAL_H

#include <hip/hip_runtime_api.h>
#include <stdint.h>

namespace q8_shim {

// Sets the calling thread's error message (q8gemv_last_error) and returns code.
int error(int code, const char* msg);
int hip_error(hipError_t e, const char* what);

// Q8_OK once q8gemv_init has run and the allocation-free scratch of its
// device was set up; otherwise the status and message of what is missing.
int noalloc_ready();

// Argument checks of f16_gemv_argmax_rows other than the workspace.
int validate_f16_argmax(const void* w_f16, int64_t n_rows, const void* x_f16,
                        const void* logits_f16, const int32_t* token);

// The vocab GEMV + argmax and its finalize on `s`, the argmax key at
// `workspace` (a device address: 16-byte aligned, zero before the launch,
// zero again after the finalize).
int launch_f16_argmax(const void* w_f16, int64_t n_rows, const void* x_f16, void* logits_f16,
                      int32_t* token, void* workspace, hipStream_t s);

// Implemented in q8gemv_noalloc.hip: looks up the scratch array's address on
// `device` (which must be current) and zero-fills it; called by q8gemv_init.
int noalloc_setup(int device);

}  // namespace q8_shim

#endif
