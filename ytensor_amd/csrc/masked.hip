// masked.hip — masked matmul and the MATH attention backend.
//
// Reference operations replaced:
//   * yt::kernel::avx2::sgemm_masked (src/kernel/avx2/sgemm.inl:342-584) and
//     YTensor::masked_matmul (src/ytensor_math.inl:318-410, 1054-1127):
//     C = alpha * A.B + beta * C where the mask (a bool matrix, or a predicate)
//     is set, C untouched (or filled with maskedValue) elsewhere;
//   * scaledDotProductAttention with sdpaBackend::MATH (src/function/ops.inl:
//     388-418, 474-490): score = masked_matmul(q, k^T, mask, -1e9), *= scale,
//     += bias, softmax_ over keys (src/function/activation.inl:313-329:
//     max, exp(x - max), sum, divide), out = score . v, rows with no visible
//     key -> 0 (ops.inl:18-40).
// Predicate masks cross the C ABI as a kind: the causal mask of the examples
// (key j visible to row i iff j <= i + (n - m)) and the general diagonal form
// j <= i + offset (the documented predicate [](int i, int j){ return j <= i; },
// doc/en/api/function/fused.mdx:200); any other predicate is evaluated into a
// bool mask by the caller.
//
// MI355X design: both operations are a product on the matrix cores plus a
// bandwidth-bound pass over the [m, n] result. The products run on the GEMM
// kernels of gemm.hip (fp32 output into a caller workspace); the mask / blend
// and the softmax rows are one workgroup per row, and the attention weights
// are written in the input type so
// that the second product runs on the 16-bit MFMA path as in the reference,
// whose score tensor has the input type. Masked tiles are not skipped: the
// products are computed whole and the mask applied on the way out.

#include <cfloat>

#include "common.hpp"
#include "launch.hpp"

namespace ythip {

struct MaskDesc {
    int kind;  // YTHIP_MASK_NONE / CAUSAL / BOOL / DIAG
    const uint8_t* data;
    int64_t ld;
    int64_t off;  // CAUSAL and DIAG: key j visible to row i iff j <= i + off
};

__device__ __forceinline__ bool visible(const MaskDesc& mk, int i, int j) {
    if (mk.kind == YTHIP_MASK_BOOL) return mk.data[(int64_t)i * mk.ld + j] != 0;
    if (mk.kind == YTHIP_MASK_CAUSAL || mk.kind == YTHIP_MASK_DIAG) return (int64_t)j <= (int64_t)i + mk.off;
    return true;
}

// C[b] (m x n) from W[b] = A.B (fp32, row stride n): where visible,
// C = alpha * W + beta * C (W alone for alpha = 1, beta = 0, as the reference's
// zero-initialised tiles store it); elsewhere C keeps its value, or takes
// `value` when `fill` is set. scale_only: the k == 0 / alpha == 0 case of
// sgemm_masked (visible entries scaled by beta, zero for beta = 0).
template <class TO>
__global__ __launch_bounds__(256) void masked_blend_kernel(const float* __restrict__ W, void* C, int64_t sc_b,
                                                           int64_t rsc, int64_t csc, int m, int n, MaskDesc mk,
                                                           float alpha, float beta, int fill, float value,
                                                           int scale_only) {
    const int cb = (gridDim.x + m - 1) / m;  // column blocks per row
    const int i = blockIdx.x / cb;
    const int b = blockIdx.z;
    const float* wr = W ? W + ((int64_t)b * m + i) * n : nullptr;
    for (int j = (blockIdx.x - i * cb) * 256 + threadIdx.x; j < n; j += cb * 256) {
        const int64_t co = (int64_t)b * sc_b + (int64_t)i * rsc + (int64_t)j * csc;
        if (visible(mk, i, j)) {
            float v;
            if (scale_only) {
                if (beta == 1.0f) continue;
                v = beta == 0.0f ? 0.0f : beta * load_as_f32<TO>(C, co);
            } else if (alpha == 1.0f && beta == 0.0f) {
                v = wr[j];
            } else {
                v = alpha * wr[j] + beta * load_as_f32<TO>(C, co);
            }
            store_from_f32<TO>(C, co, v);
        } else if (fill) {
            store_from_f32<TO>(C, co, value);
        }
    }
}

__device__ __forceinline__ float block_max(float v, float* red) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

__device__ __forceinline__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// One attention-weight row per workgroup: row i of matrix t = (b * Hq + h) of
// the fp32 scores S [t][Lq][Lkv] -> weights P (type T, same layout).
template <class T>
__global__ __launch_bounds__(256) void math_softmax_kernel(const float* __restrict__ S, void* P, int Lq, int Lkv,
                                                           MaskDesc mk, float scale, const float* __restrict__ bias,
                                                           int64_t brs, int64_t bcs, int zero_empty) {
    __shared__ float red[4];
    const int i = blockIdx.x;
    const int64_t row = ((int64_t)blockIdx.z * gridDim.y + blockIdx.y) * Lq + i;
    const float* s = S + row * Lkv;
    auto score = [&](int j) -> float {
        float x = visible(mk, i, j) ? s[j] : -1e9f;  // masked_matmul's fill value (ops.inl:395-399)
        x *= scale;
        if (bias) x += bias[(int64_t)i * brs + (int64_t)j * bcs];
        return x;
    };
    float mx = -FLT_MAX;  // std::numeric_limits<float>::lowest()
    int any = 0;
    for (int j = threadIdx.x; j < Lkv; j += 256) {
        mx = fmaxf(mx, score(j));
        any |= visible(mk, i, j) ? 1 : 0;
    }
    mx = block_max(mx, red);
    const int any_all = __syncthreads_or(any);
    float sum = 0.f;
    for (int j = threadIdx.x; j < Lkv; j += 256) sum += expf(score(j) - mx);
    sum = block_sum(sum, red);
    const bool empty = zero_empty && !any_all;  // no visible key: the output row is zeroed
    for (int j = threadIdx.x; j < Lkv; j += 256) {
        const float p = empty ? 0.0f : expf(score(j) - mx) / sum;
        store_from_f32<T>(P, row * Lkv + j, p);
    }
}

// The same for rows of at most 256 * CACHE keys, read once: each thread keeps
// its scores, then their exponentials, in registers.
template <class T, int CACHE>
__global__ __launch_bounds__(256) void math_softmax_cached_kernel(const float* __restrict__ S, void* P, int Lq,
                                                                  int Lkv, MaskDesc mk, float scale,
                                                                  const float* __restrict__ bias, int64_t brs,
                                                                  int64_t bcs, int zero_empty) {
    __shared__ float red[4];
    const int i = blockIdx.x;
    const int64_t row = ((int64_t)blockIdx.z * gridDim.y + blockIdx.y) * Lq + i;
    const float* s = S + row * Lkv;
    float x[CACHE];
    float mx = -FLT_MAX;  // std::numeric_limits<float>::lowest()
    int any = 0;
#pragma unroll
    for (int c = 0; c < CACHE; ++c) {
        const int j = c * 256 + threadIdx.x;
        x[c] = -INFINITY;
        if (j < Lkv) {
            const bool vis = visible(mk, i, j);
            float v = vis ? s[j] : -1e9f;  // masked_matmul's fill value (ops.inl:395-399)
            v *= scale;
            if (bias) v += bias[(int64_t)i * brs + (int64_t)j * bcs];
            x[c] = v;
            mx = fmaxf(mx, v);
            any |= vis ? 1 : 0;
        }
    }
    mx = block_max(mx, red);
    const int any_all = __syncthreads_or(any);
    float sum = 0.f;
#pragma unroll
    for (int c = 0; c < CACHE; ++c) {
        x[c] = (c * 256 + (int)threadIdx.x < Lkv) ? expf(x[c] - mx) : 0.f;
        sum += x[c];
    }
    sum = block_sum(sum, red);
    const bool empty = zero_empty && !any_all;
#pragma unroll
    for (int c = 0; c < CACHE; ++c) {
        const int j = c * 256 + threadIdx.x;
        if (j < Lkv) store_from_f32<T>(P, row * Lkv + j, empty ? 0.0f : x[c] / sum);
    }
}

namespace {

template <class T>
hipError_t launch_softmax(const float* S, void* P, int B, int Hq, int Lq, int Lkv, const MaskDesc& mk, float scale,
                          const float* bias, int64_t brs, int64_t bcs, int zero_empty, hipStream_t s) {
    dim3 grid(Lq, Hq, B);
    if (Lkv <= 256 * 4)
        math_softmax_cached_kernel<T, 4><<<grid, 256, 0, s>>>(S, P, Lq, Lkv, mk, scale, bias, brs, bcs, zero_empty);
    else if (Lkv <= 256 * 16)
        math_softmax_cached_kernel<T, 16><<<grid, 256, 0, s>>>(S, P, Lq, Lkv, mk, scale, bias, brs, bcs, zero_empty);
    else
        math_softmax_kernel<T><<<grid, 256, 0, s>>>(S, P, Lq, Lkv, mk, scale, bias, brs, bcs, zero_empty);
    return hipGetLastError();
}

MaskDesc make_mask(int kind, const uint8_t* data, int64_t ld, int m, int n) {
    MaskDesc mk{kind, data, ld, 0};
    if (kind == YTHIP_MASK_CAUSAL) mk.off = (int64_t)n - m;
    if (kind == YTHIP_MASK_DIAG) {
        mk.off = ld;
        mk.data = nullptr;
    }
    return mk;
}

int check_mask(const char* who, int kind, const uint8_t* data, int64_t ld, int n) {
    if (kind < YTHIP_MASK_NONE || kind > YTHIP_MASK_DIAG) return fail(YTHIP_EINVAL, "%s: mask_kind %d", who, kind);
    if (kind == YTHIP_MASK_BOOL && (data == nullptr || ld < n))
        return fail(YTHIP_EINVAL, "%s: a bool mask needs a pointer and mask_ld >= %d", who, n);
    return 0;
}

template <class TO>
hipError_t launch_blend(const float* W, void* C, int64_t sc_b, int64_t rsc, int64_t csc, int batch, int m, int n,
                        const MaskDesc& mk, float alpha, float beta, int fill, float value, int scale_only,
                        hipStream_t s) {
    const int cb = (n + 255) / 256 < 8 ? (n + 255) / 256 : 8;
    dim3 grid((unsigned)((int64_t)m * cb), 1, batch);
    masked_blend_kernel<TO><<<grid, 256, 0, s>>>(W, C, sc_b, rsc, csc, m, n, mk, alpha, beta, fill, value,
                                                 scale_only);
    return hipGetLastError();
}

hipError_t blend(int dtype_out, const float* W, void* C, int64_t sc_b, int64_t rsc, int64_t csc, int batch, int m,
                 int n, const MaskDesc& mk, float alpha, float beta, int fill, float value, int scale_only,
                 hipStream_t s) {
    if (dtype_out == YTHIP_F32)
        return launch_blend<F32>(W, C, sc_b, rsc, csc, batch, m, n, mk, alpha, beta, fill, value, scale_only, s);
    if (dtype_out == YTHIP_BF16)
        return launch_blend<BF16>(W, C, sc_b, rsc, csc, batch, m, n, mk, alpha, beta, fill, value, scale_only, s);
    return launch_blend<F16>(W, C, sc_b, rsc, csc, batch, m, n, mk, alpha, beta, fill, value, scale_only, s);
}

int esize(int dtype) { return dtype == YTHIP_F32 ? 4 : 2; }

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

}  // namespace
}  // namespace ythip

using namespace ythip;

extern "C" {

__attribute__((visibility("default"))) size_t ythip_gemm_masked_workspace_size(int batch, int m, int n) {
    if (batch <= 0 || m <= 0 || n <= 0) return 0;
    return (size_t)batch * m * n * sizeof(float);
}

__attribute__((visibility("default"))) int ythip_gemm_masked(
    int dtype_in, int dtype_out, int batch, int m, int n, int k, const void* A, int64_t sa_b, int64_t rsa,
    int64_t csa, const void* B, int64_t sb_b, int64_t rsb, int64_t csb, void* C, int64_t sc_b, int64_t rsc,
    int64_t csc, float alpha, float beta, int mask_kind, const uint8_t* mask, int64_t mask_ld, int fill_masked,
    float masked_value, void* workspace, size_t ws_bytes, void* stream) {
    const char* who = "ythip_gemm_masked";
    if (batch < 0 || m < 0 || n < 0 || k < 0) return fail(YTHIP_EINVAL, "%s: negative size", who);
    if (batch == 0 || m == 0 || n == 0) return 0;  // sgemm.inl:351
    if (int st = check_mask(who, mask_kind, mask, mask_ld, n)) return st;
    if (!C) return fail(YTHIP_EINVAL, "%s: C is NULL", who);
    if (dtype_out != YTHIP_F32 && dtype_out != YTHIP_F16 && dtype_out != YTHIP_BF16)
        return fail(YTHIP_EINVAL, "%s: dtype_out %d", who, dtype_out);
    const MaskDesc mk = make_mask(mask_kind, mask, mask_ld, m, n);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (k == 0 || alpha == 0.0f)  // sgemm.inl:352-363 (fill still applies to the masked entries)
        return status_of(blend(dtype_out, nullptr, C, sc_b, rsc, csc, batch, m, n, mk, alpha, beta, fill_masked,
                               masked_value, 1, s));
    if (!A || !B) return fail(YTHIP_EINVAL, "%s: A or B is NULL", who);
    const size_t need = ythip_gemm_masked_workspace_size(batch, m, n);
    if (!workspace || ws_bytes < need)
        return fail(YTHIP_EINVAL, "%s: workspace of %zu bytes needed (%zu given)", who, need, ws_bytes);
    float* W = static_cast<float*>(workspace);
    if (int st = gemm_dispatch(dtype_in, YTHIP_F32, batch, m, n, k, A, sa_b, rsa, csa, B, sb_b, rsb, csb, W,
                               (int64_t)m * n, n, 1, 1.0f, 0.0f, s))
        return st;
    return status_of(blend(dtype_out, W, C, sc_b, rsc, csc, batch, m, n, mk, alpha, beta, fill_masked,
                           masked_value, 0, s));
}

__attribute__((visibility("default"))) size_t ythip_attn_math_workspace_size(int dtype, int B, int Hq, int q_len,
                                                                          int kv_len) {
    if (B <= 0 || Hq <= 0 || q_len <= 0 || kv_len <= 0) return 0;
    const size_t cells = (size_t)B * Hq * q_len * kv_len;
    return dtype == YTHIP_F32 ? cells * 4 : align256(cells * 4) + cells * 2;
}

__attribute__((visibility("default"))) int ythip_attn_math(
    int dtype, int B, int Hq, int Hkv, int q_len, int kv_len, int d, int dv, const void* Q, const int64_t q_str[4],
    const void* K, const int64_t k_str[4], const void* V, const int64_t v_str[4], void* O, const int64_t o_str[4],
    float scale, int mask_kind, const uint8_t* mask, int64_t mask_ld, const float* bias, int64_t rs_bias,
    int64_t cs_bias, void* workspace, size_t ws_bytes, void* stream) {
    const char* who = "ythip_attn_math";
    if (B < 0 || Hq < 0 || Hkv < 0 || q_len < 0 || kv_len < 0 || d < 0 || dv < 0)
        return fail(YTHIP_EINVAL, "%s: negative size", who);
    if ((int64_t)B * Hq * q_len == 0 || dv == 0) return 0;
    if (Hkv == 0 || Hq % Hkv != 0) return fail(YTHIP_EINVAL, "%s: Hq=%d not a multiple of Hkv=%d", who, Hq, Hkv);
    if (dtype != YTHIP_F32 && dtype != YTHIP_F16 && dtype != YTHIP_BF16)
        return fail(YTHIP_EINVAL, "%s: invalid dtype %d", who, dtype);
    if (!Q || !O || !q_str || !k_str || !v_str || !o_str || (kv_len > 0 && (!K || !V)))
        return fail(YTHIP_EINVAL, "%s: NULL tensor or stride array", who);
    if (int st = check_mask(who, mask_kind, mask, mask_ld, kv_len)) return st;
    if (scale == 0.0f) scale = 1.0f / sqrtf((float)d);  // src/function/ops.inl:378-381
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int es = esize(dtype);
    auto op = [&](int b, int h) { return static_cast<char*>(O) + (b * o_str[0] + h * o_str[1]) * es; };
    if (kv_len == 0) {
        // no key: score . v is an empty product, i.e. zeros (sgemm.inl:594-604)
        for (int b = 0; b < B; ++b)
            if (int st = gemm_dispatch(dtype, dtype, Hq, q_len, dv, 0, nullptr, 0, 0, 1, nullptr, 0, 0, 1, op(b, 0),
                                       o_str[1], o_str[2], o_str[3], 1.0f, 0.0f, s))
                return st;
        return 0;
    }
    const size_t need = ythip_attn_math_workspace_size(dtype, B, Hq, q_len, kv_len);
    if (!workspace || ws_bytes < need)
        return fail(YTHIP_EINVAL, "%s: workspace of %zu bytes needed (%zu given)", who, need, ws_bytes);
    const int G = Hq / Hkv;
    const size_t cells = (size_t)B * Hq * q_len * kv_len;
    float* S = static_cast<float*>(workspace);
    void* P = dtype == YTHIP_F32 ? workspace : static_cast<char*>(workspace) + align256(cells * 4);
    const int64_t mat = (int64_t)q_len * kv_len;  // one head's scores
    auto qp = [&](int b, int h) { return static_cast<const char*>(Q) + (b * q_str[0] + h * q_str[1]) * es; };
    auto kp = [&](int b, int h) { return static_cast<const char*>(K) + (b * k_str[0] + h * k_str[1]) * es; };
    auto vp = [&](int b, int h) { return static_cast<const char*>(V) + (b * v_str[0] + h * v_str[1]) * es; };
    // The G query heads of one kv head are one [G * q_len, d] matrix when
    // heads are laid out row after row; then one batched GEMM per batch entry.
    const bool q_rows = q_str[1] == (int64_t)q_len * q_str[2];
    const bool o_rows = o_str[1] == (int64_t)q_len * o_str[2];
    // 1. S = Q . K^T (fp32); K^T element (p, j) at j * k_str[2] + p * k_str[3]
    for (int b = 0; b < B; ++b) {
        for (int g = 0; g < (q_rows ? 1 : G); ++g) {
            const int rows = q_rows ? G * q_len : q_len;
            if (int st = gemm_dispatch(dtype, YTHIP_F32, Hkv, rows, kv_len, d, qp(b, g), G * q_str[1], q_str[2],
                                       q_str[3], kp(b, 0), k_str[1], k_str[3], k_str[2],
                                       S + ((int64_t)b * Hq + g) * mat, G * mat, kv_len, 1, 1.0f, 0.0f, s))
                return st;
        }
    }
    // 2. mask, scale, bias, softmax -> P (input type)
    const MaskDesc mk = make_mask(mask_kind, mask, mask_ld, q_len, kv_len);
    {
        const int zero_empty = mask_kind != YTHIP_MASK_NONE;
        hipError_t e;
        if (dtype == YTHIP_F32)
            e = launch_softmax<F32>(S, P, B, Hq, q_len, kv_len, mk, scale, bias, rs_bias, cs_bias, zero_empty, s);
        else if (dtype == YTHIP_BF16)
            e = launch_softmax<BF16>(S, P, B, Hq, q_len, kv_len, mk, scale, bias, rs_bias, cs_bias, zero_empty, s);
        else
            e = launch_softmax<F16>(S, P, B, Hq, q_len, kv_len, mk, scale, bias, rs_bias, cs_bias, zero_empty, s);
        if (int st = status_of(e)) return st;
    }
    // 3. O = P . V
    const char* Pc = static_cast<const char*>(P);
    for (int b = 0; b < B; ++b) {
        for (int g = 0; g < (o_rows ? 1 : G); ++g) {
            const int rows = o_rows ? G * q_len : q_len;
            if (int st = gemm_dispatch(dtype, dtype, Hkv, rows, dv, kv_len,
                                       Pc + (((int64_t)b * Hq + g) * mat) * es, G * mat, kv_len, 1, vp(b, 0),
                                       v_str[1], v_str[2], v_str[3], op(b, g), G * o_str[1], o_str[2], o_str[3],
                                       1.0f, 0.0f, s))
                return st;
        }
    }
    return 0;
}

}  // extern "C"
