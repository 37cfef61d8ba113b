// decoder_glue.hip — the small elementwise kernels that, with the GEMM,
// attention and RMSNorm+RoPE kernels, make a whole Qwen3 decoder step device
// resident (example/qwen3/src/qwen3.cpp:193-516):
//   * SwiGLU: act = swish(gate) * up over the fused gate_up projection
//     (Qwen3MLP::forward, qwen3.cpp:193-200; swish_ with the stable sigmoid,
//     src/function/activation.inl:631-647, src/ytensor_function.inl:43-52);
//   * embedding gather with the token ids read from device memory
//     (Qwen3Model::forward, qwen3.cpp:378-385);
//   * greedy selection: argmax over the logits that also advances the
//     decode-position counters kept in device memory.
// Nothing here takes a host-side value that changes from one decode step to
// the next, so a step can be captured once as a HIP graph and replayed.

#include <cfloat>

#include <algorithm>

#include "common.hpp"
#include "launch.hpp"

namespace ythip {

template <class T, class TO>
__global__ __launch_bounds__(256) void silu_mul_kernel(const void* gu, int64_t ld_gu, void* out, int64_t ld_out,
                                                       int n, int rows) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int r = (int)(i / n), j = (int)(i % n);
    if (r >= rows) return;
    const float a = load_as_f32<T>(gu, (int64_t)r * ld_gu + j);
    const float u = load_as_f32<T>(gu, (int64_t)r * ld_gu + n + j);
    float sig;
    if (a >= 0.0f) {
        const float z = expf(-a);
        sig = 1.0f / (1.0f + z);
    } else {
        const float z = expf(a);
        sig = z / (1.0f + z);
    }
    store_from_f32<TO>(out, (int64_t)r * ld_out + j, (a * sig) * u);
}

// silu_mul_kernel's arithmetic on 8 consecutive columns per thread (16-byte
// loads and stores; 16-bit in and out, n % 8 == 0, 16-byte aligned rows).
template <class T, class TO>
__global__ __launch_bounds__(256) void silu_mul_vec_kernel(const void* gu, int64_t ld_gu, void* out, int64_t ld_out,
                                                           int n) {
    const int r = blockIdx.y;
    const int j = (blockIdx.x * 256 + threadIdx.x) * 8;
    if (j >= n) return;
    const auto* g = static_cast<const typename T::raw*>(gu) + (int64_t)r * ld_gu + j;
    const u32x4 wa = *reinterpret_cast<const u32x4*>(g);
    const u32x4 wu = *reinterpret_cast<const u32x4*>(g + n);
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        float y[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const float a = h ? hi_as_f32(T{}, wa[e]) : lo_as_f32(T{}, wa[e]);
            const float u = h ? hi_as_f32(T{}, wu[e]) : lo_as_f32(T{}, wu[e]);
            float sig;
            if (a >= 0.0f) {
                const float z = expf(-a);
                sig = 1.0f / (1.0f + z);
            } else {
                const float z = expf(a);
                sig = z / (1.0f + z);
            }
            y[h] = (a * sig) * u;
        }
        // the scalar kernel's per-element conversion (same rounding of fp16
        // denormals as store_from_f32), then packed
        uint32_t bits[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            if constexpr (std::is_same_v<TO, BF16>) bits[h] = f32_to_bf16_bits(y[h]);
            else bits[h] = f32_to_f16_bits(y[h]);
        }
        o[e] = bits[0] | (bits[1] << 16);
    }
    *reinterpret_cast<u32x4*>(static_cast<typename TO::raw*>(out) + (int64_t)r * ld_out + j) = o;
}

// Rows whose id is outside [0, vocab) get zeros: the id is never used as an
// address. Rows beyond the grid's 65535 y-blocks are taken in a row-stride loop.
template <class T, class TO>
__global__ __launch_bounds__(256) void embedding_kernel(const void* table, const int32_t* ids, void* out,
                                                        int64_t ld_out, int n, int vocab, int rows) {
    for (int r = blockIdx.y; r < rows; r += gridDim.y) {
        const int64_t row = ids[r];
        const bool valid = row >= 0 && row < vocab;
        for (int j = blockIdx.x * 256 + threadIdx.x; j < n; j += gridDim.x * 256)
            store_from_f32<TO>(out, (int64_t)r * ld_out + j, valid ? load_as_f32<T>(table, row * n + j) : 0.0f);
    }
}

// linear's bias (src/function/ops.inl:93-104): the product is already stored
// (rounded to T); the bias is then added in T, out = T(out + bias).
template <class T>
__global__ __launch_bounds__(256) void add_bias_kernel(void* out, int64_t ld_out, const void* bias, int n, int rows) {
    const int j = blockIdx.x * 256 + threadIdx.x;
    if (j >= n) return;
    const float b = load_as_f32<T>(bias, j);
    for (int r = blockIdx.y; r < rows; r += gridDim.y) {  // rows past 65535 y-blocks: row-stride loop
        const int64_t i = (int64_t)r * ld_out + j;
        store_from_f32<T>(out, i, load_as_f32<T>(out, i) + b);
    }
}

// One workgroup scans all n logits; ties resolve to the lowest index (the
// first maximum, as a left-to-right scan finds it).
__global__ __launch_bounds__(1024) void argmax_step_kernel(const float* x, int n, int32_t* token, int32_t* history,
                                                           int32_t* state) {
    float best = -INFINITY;
    int idx = 0x7fffffff;
    for (int i = threadIdx.x; i < n; i += 1024) {
        const float v = x[i];
        if (v > best || (v == best && i < idx)) { best = v; idx = i; }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float ob = __shfl_xor(best, off, 64);
        const int oi = __shfl_xor(idx, off, 64);
        if (ob > best || (ob == best && oi < idx)) { best = ob; idx = oi; }
    }
    __shared__ float sb[16];
    __shared__ int si[16];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) { sb[wave] = best; si[wave] = idx; }
    __syncthreads();
    if (threadIdx.x == 0) {
        float b = sb[0];
        int id = si[0];
        for (int w = 1; w < 16; ++w)
            if (sb[w] > b || (sb[w] == b && si[w] < id)) { b = sb[w]; id = si[w]; }
        if (id == 0x7fffffff) id = 0;  // all NaN / empty: token 0
        token[0] = id;
        if (state != nullptr) decode_state_advance(state, history, id);
    }
}

namespace {

template <class T, class TO>
hipError_t launch_silu(int rows, int n, const void* gu, int64_t ld_gu, void* out, int64_t ld_out, hipStream_t s) {
    if constexpr (sizeof(typename T::raw) == 2 && sizeof(typename TO::raw) == 2) {
        const bool vec = n % 8 == 0 && ld_gu % 8 == 0 && ld_out % 8 == 0 && rows <= 65535 &&
                         reinterpret_cast<uintptr_t>(gu) % 16 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0;
        if (vec) {
            silu_mul_vec_kernel<T, TO><<<dim3((unsigned)((n / 8 + 255) / 256), rows), 256, 0, s>>>(gu, ld_gu, out,
                                                                                                 ld_out, n);
            return hipGetLastError();
        }
    }
    const int64_t total = (int64_t)rows * n;
    silu_mul_kernel<T, TO><<<(unsigned)((total + 255) / 256), 256, 0, s>>>(gu, ld_gu, out, ld_out, n, rows);
    return hipGetLastError();
}

template <class T, class TO>
hipError_t launch_embed(int rows, int n, int vocab, const void* table, const int32_t* ids, void* out,
                        int64_t ld_out, hipStream_t s) {
    dim3 grid((unsigned)((n + 255) / 256), (unsigned)std::min(rows, 65535));
    embedding_kernel<T, TO><<<grid, 256, 0, s>>>(table, ids, out, ld_out, n, vocab, rows);
    return hipGetLastError();
}

}  // namespace

}  // namespace ythip

using namespace ythip;

#define YTHIP_DISPATCH2(di, dout, FN, ...)                                                   \
    do {                                                                                      \
        if (di == YTHIP_BF16 && dout == YTHIP_BF16) return status_of(FN<BF16, BF16>(__VA_ARGS__)); \
        if (di == YTHIP_BF16 && dout == YTHIP_F32) return status_of(FN<BF16, F32>(__VA_ARGS__));   \
        if (di == YTHIP_F32 && dout == YTHIP_F32) return status_of(FN<F32, F32>(__VA_ARGS__));     \
        if (di == YTHIP_F32 && dout == YTHIP_BF16) return status_of(FN<F32, BF16>(__VA_ARGS__));   \
        if (di == YTHIP_F16 && dout == YTHIP_F16) return status_of(FN<F16, F16>(__VA_ARGS__));     \
        if (di == YTHIP_F16 && dout == YTHIP_F32) return status_of(FN<F16, F32>(__VA_ARGS__));     \
        if (di == YTHIP_F32 && dout == YTHIP_F16) return status_of(FN<F32, F16>(__VA_ARGS__));     \
    } while (0)

extern "C" {

__attribute__((visibility("default"))) int ythip_silu_mul(int dtype_in, int dtype_out, int rows, int n,
                                                          const void* gate_up, int64_t ld_gu, void* out,
                                                          int64_t ld_out, void* stream) {
    if (rows < 0 || n < 0) return fail(YTHIP_EINVAL, "ythip_silu_mul: negative size");
    if ((int64_t)rows * n == 0) return 0;
    if (!gate_up || !out || ld_gu < 2 * (int64_t)n || ld_out < n)
        return fail(YTHIP_EINVAL, "ythip_silu_mul: NULL pointer or leading dimension too small");
    hipStream_t s = static_cast<hipStream_t>(stream);
    YTHIP_DISPATCH2(dtype_in, dtype_out, launch_silu, rows, n, gate_up, ld_gu, out, ld_out, s);
    return fail(YTHIP_EUNSUPPORTED, "ythip_silu_mul: dtype pair %d/%d", dtype_in, dtype_out);
}

__attribute__((visibility("default"))) int ythip_embedding(int dtype_table, int dtype_out, int rows, int n,
                                                           int vocab, const void* table, const int32_t* ids,
                                                           void* out, int64_t ld_out, void* stream) {
    if (rows < 0 || n < 0 || vocab < 0) return fail(YTHIP_EINVAL, "ythip_embedding: negative size");
    if ((int64_t)rows * n == 0) return 0;
    if (!table || !ids || !out || ld_out < n)
        return fail(YTHIP_EINVAL, "ythip_embedding: NULL pointer or leading dimension too small");
    hipStream_t s = static_cast<hipStream_t>(stream);
    YTHIP_DISPATCH2(dtype_table, dtype_out, launch_embed, rows, n, vocab, table, ids, out, ld_out, s);
    return fail(YTHIP_EUNSUPPORTED, "ythip_embedding: dtype pair %d/%d", dtype_table, dtype_out);
}

__attribute__((visibility("default"))) int ythip_add_bias(int dtype, int rows, int n, void* out, int64_t ld_out,
                                                          const void* bias, void* stream) {
    if (rows < 0 || n < 0) return fail(YTHIP_EINVAL, "ythip_add_bias: negative size");
    if ((int64_t)rows * n == 0) return 0;
    if (!out || !bias || ld_out < n) return fail(YTHIP_EINVAL, "ythip_add_bias: NULL pointer or ld_out < n");
    hipStream_t s = static_cast<hipStream_t>(stream);
    dim3 grid((unsigned)((n + 255) / 256), (unsigned)std::min(rows, 65535));
    switch (dtype) {
        case YTHIP_F32: add_bias_kernel<F32><<<grid, 256, 0, s>>>(out, ld_out, bias, n, rows); break;
        case YTHIP_F16: add_bias_kernel<F16><<<grid, 256, 0, s>>>(out, ld_out, bias, n, rows); break;
        case YTHIP_BF16: add_bias_kernel<BF16><<<grid, 256, 0, s>>>(out, ld_out, bias, n, rows); break;
        default: return fail(YTHIP_EINVAL, "ythip_add_bias: invalid dtype %d", dtype);
    }
    return status_of(hipGetLastError());
}

__attribute__((visibility("default"))) int ythip_argmax_step(int n, const float* logits, int32_t* token,
                                                             int32_t* history, int32_t* state, void* stream) {
    if (n <= 0 || !logits || !token) return fail(YTHIP_EINVAL, "ythip_argmax_step: empty input or NULL pointer");
    argmax_step_kernel<<<1, 1024, 0, static_cast<hipStream_t>(stream)>>>(logits, n, token, history, state);
    return status_of(hipGetLastError());
}

}  // extern "C"
