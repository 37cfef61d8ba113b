// launch.hpp — host-side status/error plumbing shared by the C-ABI entry points.
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/ythip.h"

namespace ythip {

// Records a formatted message as this thread's last error and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// 0 for hipSuccess; otherwise records the HIP error string and returns the
// (positive) hipError_t value.
int status_of(hipError_t e);

// Kernel dispatchers (one per translation unit).
int gemm_dispatch(int dtype_in, int dtype_out, int batch, int m, int n, int k, const void* A, int64_t sa_b,
                  int64_t rsa, int64_t csa, const void* B, int64_t sb_b, int64_t rsb, int64_t csb, void* C,
                  int64_t sc_b, int64_t rsc, int64_t csc, float alpha, float beta, hipStream_t s);

}  // namespace ythip
