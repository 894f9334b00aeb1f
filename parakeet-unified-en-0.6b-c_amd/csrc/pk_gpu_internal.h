// pk_gpu_internal.h - host-side services of pk_gpu_runtime.hip used by the
// other host translation units of libpk_gpu.so (not part of the C ABI).
#pragma once

#include "pk_gemm_kernels.h"

#include <hip/hip_runtime.h>

namespace pkgpu {
namespace rt {

// Set the calling thread's pk_gpu_last_error() message; returns code.
int error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// PK_GPU_EHIP with the HIP error string.
int hip_error(hipError_t e, const char* what);
// Initialise the library if needed and bind the calling thread to its
// device; *thread_stream (if given) receives the thread's own stream.
int bind(hipStream_t* thread_stream);
// Launch one weight GEMM (launch_gemm with the thread's forced config, which
// implies exact chains), mapping launch errors to pk_gpu_status codes.
int gemm(const GemmProblem& p, hipStream_t s, Tolerance tol = TOL_NONE);
// The tolerance a PK_GPU_NUMERICS_* mode allows.
Tolerance tolerance_of(int numerics);
// The calling thread's pk_gpu_force_config index (-1: the dispatcher picks).
int forced_config();

}  // namespace rt
}  // namespace pkgpu
