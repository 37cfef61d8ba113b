// ythip_abi.hip — the extern "C" boundary of libythip.so (include/ythip.h).
// Argument validation happens here, before anything is launched; the kernels
// themselves assume validated shapes. Error reporting mirrors the reference's
// L3/L4 checks (src/function/ops.inl:123-128, 382-387; src/ytensor_math.inl:290-292)
// but as status codes plus a thread-local message instead of exceptions.

#include <cmath>
#include <cstdarg>
#include <cstdio>

#include "launch.hpp"

namespace ythip {

static thread_local char g_last_error[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

int status_of(hipError_t e) {
    if (e == hipSuccess) return 0;
    fail(static_cast<int>(e), "HIP error %d: %s", static_cast<int>(e), hipGetErrorString(e));
    return static_cast<int>(e);
}

static bool valid_dtype(int d) { return d == YTHIP_F32 || d == YTHIP_F16 || d == YTHIP_BF16; }

}  // namespace ythip

using namespace ythip;

extern "C" {

__attribute__((visibility("default"))) int ythip_abi_version(void) { return YTHIP_ABI_VERSION; }

__attribute__((visibility("default"))) const char* ythip_last_error(void) { return g_last_error; }

__attribute__((visibility("default"))) int ythip_gemm(int dtype_in, int dtype_out, int batch, int m, int n, int k,
                                                      const void* A, int64_t sa_b, int64_t rsa, int64_t csa,
                                                      const void* B, int64_t sb_b, int64_t rsb, int64_t csb, void* C,
                                                      int64_t sc_b, int64_t rsc, int64_t csc, float alpha, float beta,
                                                      void* stream) {
    g_last_error[0] = '\0';
    if (!valid_dtype(dtype_in) || !valid_dtype(dtype_out))
        return fail(YTHIP_EINVAL, "ythip_gemm: invalid dtype %d/%d", dtype_in, dtype_out);
    if (batch < 0 || m < 0 || n < 0 || k < 0)
        return fail(YTHIP_EINVAL, "ythip_gemm: negative size (batch=%d m=%d n=%d k=%d)", batch, m, n, k);
    if (batch == 0 || m == 0 || n == 0) return 0;  // sgemm.inl:594
    if (C == nullptr) return fail(YTHIP_EINVAL, "ythip_gemm: C is NULL");
    if (k > 0 && alpha != 0.0f && (A == nullptr || B == nullptr))
        return fail(YTHIP_EINVAL, "ythip_gemm: A or B is NULL");
    return gemm_dispatch(dtype_in, dtype_out, batch, m, n, k, A, sa_b, rsa, csa, B, sb_b, rsb, csb, C, sc_b, rsc,
                         csc, alpha, beta, static_cast<hipStream_t>(stream));
}

// Host-side RoPE tables, computed as RoPECache::precompute does
// (example/qwen3/src/qwen3.cpp:161-175): float freq = 1/powf(theta, 2i/dim),
// angle = t*freq, cos/sin duplicated into both halves. HOST pointers,
// cosv/sinv [max_len][dim].
__attribute__((visibility("default"))) int ythip_rope_tables(int dim, int max_len, float theta, float* cosv,
                                                             float* sinv) {
    if (dim <= 0 || (dim & 1) || max_len < 0 || !cosv || !sinv)
        return fail(YTHIP_EINVAL, "ythip_rope_tables: bad arguments");
    const int half = dim / 2;
    for (int t = 0; t < max_len; ++t)
        for (int i = 0; i < half; ++i) {
            const float freq = 1.0f / std::pow(theta, 2.0f * i / dim);
            const float angle = t * freq;
            cosv[(size_t)t * dim + i] = cosv[(size_t)t * dim + i + half] = std::cos(angle);
            sinv[(size_t)t * dim + i] = sinv[(size_t)t * dim + i + half] = std::sin(angle);
        }
    return 0;
}

}  // extern "C"
