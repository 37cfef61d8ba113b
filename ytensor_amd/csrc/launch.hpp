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

// Skinny GEMM / fused decode GEMV (gemv.hip): C[m, n] = alpha * A' . W^T + beta * C
// with A' built by the prologue (0: A as is, 1: RMSNorm of fp32 rows, 2: SwiGLU
// of [gate | up] rows).
struct GemvArgs {
    const void* A;  // prologue 0: T [m][k]; 1: fp32 [m][k]; 2: T [m][2k] (gate | up)
    int64_t lda;
    const float* nw;  // prologue 1: norm weight [k]
    float eps;
    const void* W;  // [n][k] rows, stride ldw
    int64_t ldw;
    void* C;
    int64_t ldc;
    int64_t sa_b, sw_b, sc_b;  // batch strides (blockIdx.y)
    int m, n, k;
    float alpha, beta;
    float* amax;  // optional: per 16-column tile (max, index) of row 0
    int hq, hd, splits;  // prologue 3: A = split-K decode partials [m][hq][splits][hd + 2]
    // prologue 3: the decode-state record whose KV_LEN (clamped to max_ctx) the
    // split kernel partitioned, so only the splits holding keys are read (NULL:
    // every split; the empty ones add exact zeros)
    const int32_t* dstate;
    int max_ctx;
};

int gemv_dispatch(int prologue, int dtype_in, int dtype_out, const GemvArgs& a, int batch, hipStream_t s);

}  // namespace ythip
