// ythip.hpp — C++ host mirror of YTensor's kernel API over libythip.so.
//
// The reference's L2 kernel API (yt::kernel::avx2, include/kernel/avx2/
// sgemm.hpp:51-68, hgemm.hpp:26-42, flash_attention.hpp:21-69) takes host
// pointers, element strides and sizes and returns void; errors surface in the
// L3/L4 callers as std::invalid_argument / std::runtime_error. This header
// keeps those names and argument meanings for DEVICE pointers plus a stream,
// and turns a non-zero libythip status into std::runtime_error carrying
// ythip_last_error(). Header-only; link with -lythip.
#pragma once

#include <cstdint>
#include <stdexcept>
#include <string>

#include "ythip.h"

namespace yt::kernel::hip {

inline void check(int status, const char* what) {
    if (status != 0) throw std::runtime_error(std::string(what) + ": " + ythip_last_error());
}

// yt::kernel::avx2::sgemm (sgemm.hpp:51-58): C = alpha*A.B + beta*C, element strides.
inline void sgemm(const float* A, const float* B, float* C, int m, int n, int k, float alpha, float beta,
                  int64_t rsa, int64_t csa, int64_t rsb, int64_t csb, int64_t rsc, int64_t csc,
                  void* stream = nullptr) {
    check(ythip_gemm(YTHIP_F32, YTHIP_F32, 1, m, n, k, A, 0, rsa, csa, B, 0, rsb, csb, C, 0, rsc, csc, alpha, beta,
                     stream),
          "yt::kernel::hip::sgemm");
}

// yt::kernel::avx2::matmul (sgemm.hpp:60-68): alpha = 1, beta = 0.
inline void matmul(const float* A, const float* B, float* C, int m, int n, int k, int64_t rsa, int64_t csa,
                   int64_t rsb, int64_t csb, int64_t rsc, int64_t csc, void* stream = nullptr) {
    sgemm(A, B, C, m, n, k, 1.0f, 0.0f, rsa, csa, rsb, csb, rsc, csc, stream);
}

// yt::kernel::avx2::hgemm (hgemm.hpp:26-33) for the 16-bit members of the type
// set: A/B/C hold raw float16 (YTHIP_F16) or bfloat16 (YTHIP_BF16) bits;
// accumulation is fp32 as in the reference's fp32 fast path (hgemm.inl:165-216).
inline void hgemm(int dtype, const void* A, const void* B, void* C, int m, int n, int k, float alpha, float beta,
                  int64_t rsa, int64_t csa, int64_t rsb, int64_t csb, int64_t rsc, int64_t csc,
                  void* stream = nullptr) {
    check(ythip_gemm(dtype, dtype, 1, m, n, k, A, 0, rsa, csa, B, 0, rsb, csb, C, 0, rsc, csc, alpha, beta,
                     stream),
          "yt::kernel::hip::hgemm");
}

// yt::kernel::avx2::flash_attention (flash_attention.hpp:21-44), one
// (query-block, key/value) matrix with row/column element strides, optional
// bool mask [q_len, mask_stride] and additive bias. Column strides must be 1.
inline void flash_attention(int dtype, const void* Q, const void* K, const void* V, void* O, int q_len, int kv_len,
                            int head_dim, int value_dim, float scale, int64_t rsq, int64_t csq, int64_t rsk,
                            int64_t csk, int64_t rsv, int64_t csv, int64_t rso, int64_t cso,
                            const bool* mask = nullptr, int64_t mask_stride = 0, const float* bias = nullptr,
                            int64_t rsbias = 0, int64_t csbias = 0, void* stream = nullptr) {
    if (csq != 1 || csk != 1 || csv != 1 || cso != 1)
        throw std::invalid_argument("yt::kernel::hip::flash_attention: column strides must be 1");
    const int64_t qs[4] = {0, 0, rsq, 1}, ks[4] = {0, 0, rsk, 1}, vs[4] = {0, 0, rsv, 1}, os[4] = {0, 0, rso, 1};
    check(ythip_attn_prefill(dtype, 1, 1, 1, q_len, kv_len, head_dim, value_dim, Q, qs, K, ks, V, vs, O, os, scale,
                             mask ? YTHIP_MASK_BOOL : YTHIP_MASK_NONE, reinterpret_cast<const uint8_t*>(mask),
                             mask_stride, bias, rsbias, csbias, stream),
          "yt::kernel::hip::flash_attention");
}

// The batched GQA form the qwen3 example drives through
// scaledDotProductAttention(..., FLASH_AVX2) (example/qwen3/src/qwen3.cpp:250-264):
// Q [B,Hq,q_len,d], K/V [B,Hkv,kv_len,d] with 4 strides each; causal with the
// example's offset (kv_len - q_len).
inline void sdpa_gqa(int dtype, int B, int Hq, int Hkv, int q_len, int kv_len, int d, const void* Q,
                     const int64_t q_str[4], const void* K, const int64_t k_str[4], const void* V,
                     const int64_t v_str[4], void* O, const int64_t o_str[4], float scale, bool causal,
                     void* stream = nullptr) {
    check(ythip_attn_prefill(dtype, B, Hq, Hkv, q_len, kv_len, d, d, Q, q_str, K, k_str, V, v_str, O, o_str, scale,
                             causal ? YTHIP_MASK_CAUSAL : YTHIP_MASK_NONE, nullptr, 0, nullptr, 0, 0, stream),
          "yt::kernel::hip::sdpa_gqa");
}

}  // namespace yt::kernel::hip
