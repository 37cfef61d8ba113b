// norm_rope.hip — RMSNorm and the fused per-head RMSNorm + RoPE for gfx950.
//
// Reference semantics:
//   rmsNorm_ (src/function/normalization.inl:256-267 -> _rmsAxes_ 33-54 and
//   _applyScale_ 88-101): y = x / sqrt(mean(x*x) + eps) * w, a division by the
//   square root (not an rsqrt multiply).
//   rope (example/qwen3/src/qwen3.cpp:522-559): rotate-half over [0, d/2) and
//   [d/2, d) with cos/sin table row = position:
//     x1' = x1*c - x2*s ;  x2' = x2*c + x1*s
//   The tables are the host's RoPECache::precompute output (qwen3.cpp:161-175)
//   so the angles are bit-identical to the CPU path.
//
// Both kernels are HBM-bound elementwise passes: one wave per (token, head)
// row of d = 128 elements (64 lanes x 2, lane l holds x[l] and x[l + d/2], the
// two halves RoPE pairs up), a wave-wide DPP/shuffle sum of squares, then one
// vectorised store.

#include "common.hpp"
#include "launch.hpp"

namespace ythip {

struct NormRopeArgs {
    const void* qkv;
    int64_t ld_qkv;
    const float* wq;
    const float* wk;
    float eps;
    const float* cos_tab;
    const float* sin_tab;
    int64_t ld_tab;
    int pos0;
    void* q;
    void* k;
    void* v;
    int64_t qs0, qs1, qs2, ks0, ks1, ks2, vs0, vs1, vs2;
    int B, S, Hq, Hkv;
    int cache_pos;
    const int32_t* dev_pos;  // when set: pos0 = cache_pos = *dev_pos (graph-replayable decode)
};

// One wave per (token, head) with d = 2 * HALF; HALF <= 64 (d <= 128).
template <class T, int HALF>
__global__ __launch_bounds__(256) void norm_rope_kernel(NormRopeArgs a) {
    const int wave = (blockIdx.x * 4) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int H = a.Hq + 2 * a.Hkv;
    const int64_t rows = (int64_t)a.B * a.S * H;
    if (wave >= rows) return;
    const int h = wave % H;
    const int64_t tok = wave / H;
    const int s = tok % a.S;
    const int b = tok / a.S;
    constexpr int D = 2 * HALF;
    const int pos0 = a.dev_pos ? a.dev_pos[0] : a.pos0;
    const int cache_pos = a.dev_pos ? a.dev_pos[0] : a.cache_pos;
    const bool active = lane < HALF;

    const auto* src = static_cast<const typename T::raw*>(a.qkv) + tok * a.ld_qkv + (int64_t)h * D;
    float x1 = 0.f, x2 = 0.f;
    if (active) {
        x1 = load_as_f32<T>(src, lane);
        x2 = load_as_f32<T>(src, lane + HALF);
    }
    void* dst;
    int64_t off;
    const float* w = nullptr;
    if (h < a.Hq) {
        dst = a.q;
        off = b * a.qs0 + h * a.qs1 + s * a.qs2;
        w = a.wq;
    } else if (h < a.Hq + a.Hkv) {
        dst = a.k;
        off = b * a.ks0 + (h - a.Hq) * a.ks1 + (int64_t)(cache_pos + s) * a.ks2;
        w = a.wk;
    } else {
        dst = a.v;
        off = b * a.vs0 + (h - a.Hq - a.Hkv) * a.vs1 + (int64_t)(cache_pos + s) * a.vs2;
        if (dst != nullptr && active) {
            store_from_f32<T>(dst, off + lane, x1);
            store_from_f32<T>(dst, off + lane + HALF, x2);
        }
        return;
    }
    if (dst == nullptr) return;
    if (w != nullptr) {
        const float ss = wave_sum(x1 * x1 + x2 * x2);
        const float den = sqrtf(ss / (float)D + a.eps);
        if (active) {
            x1 = (x1 / den) * w[lane];
            x2 = (x2 / den) * w[lane + HALF];
        }
    }
    if (a.cos_tab != nullptr && active) {
        const int64_t t = (int64_t)(pos0 + s) * a.ld_tab;
        const float c = a.cos_tab[t + lane], sn = a.sin_tab[t + lane];
        const float y1 = fmaf(x1, c, -(x2 * sn));
        const float y2 = fmaf(x2, c, x1 * sn);
        x1 = y1;
        x2 = y2;
    }
    if (active) {
        store_from_f32<T>(dst, off + lane, x1);
        store_from_f32<T>(dst, off + lane + HALF, x2);
    }
}

// Row RMSNorm for wide rows (hidden size): one 256-thread block per row.
template <class T, class TO>
__global__ __launch_bounds__(256) void rms_norm_kernel(const void* x, int64_t ldx, const float* w, float eps,
                                                       void* y, int64_t ldy, int n) {
    const int64_t row = blockIdx.x;
    const auto* xr = static_cast<const typename T::raw*>(x) + row * ldx;
    auto* yr = static_cast<typename TO::raw*>(y) + row * ldy;
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += 256) {
        const float v = load_as_f32<T>(xr, i);
        ss = fmaf(v, v, ss);
    }
    __shared__ float part[4];
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float tot = (part[0] + part[1]) + (part[2] + part[3]);
    const float den = sqrtf(tot / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += 256) store_from_f32<TO>(yr, i, (load_as_f32<T>(xr, i) / den) * w[i]);
}

namespace {

template <class T>
hipError_t launch_norm_rope(const NormRopeArgs& a, int d, hipStream_t s) {
    const int64_t rows = (int64_t)a.B * a.S * (a.Hq + 2 * a.Hkv);
    dim3 grid((unsigned)((rows + 3) / 4));
    switch (d) {
        case 64: norm_rope_kernel<T, 32><<<grid, 256, 0, s>>>(a); break;
        case 128: norm_rope_kernel<T, 64><<<grid, 256, 0, s>>>(a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <class T, class TO>
hipError_t launch_rms(int rows, int n, const void* x, int64_t ldx, const float* w, float eps, void* y, int64_t ldy,
                      hipStream_t s) {
    rms_norm_kernel<T, TO><<<rows, 256, 0, s>>>(x, ldx, w, eps, y, ldy, n);
    return hipGetLastError();
}

}  // namespace

}  // namespace ythip

using namespace ythip;

extern "C" {

__attribute__((visibility("default"))) int ythip_rmsnorm_rope(
    int dtype, int B, int S, int Hq, int Hkv, int d, const void* qkv, int64_t ld_qkv, const float* wq,
    const float* wk, float eps, const float* cos_tab, const float* sin_tab, int64_t ld_tab, int pos0, void* Qout,
    const int64_t q_str[3], void* Kout, const int64_t k_str[3], void* Vout, const int64_t v_str[3], int cache_pos,
    const int32_t* dev_pos, void* stream) {
    if (B < 0 || S < 0 || Hq < 0 || Hkv < 0) return fail(YTHIP_EINVAL, "ythip_rmsnorm_rope: negative size");
    if (d != 64 && d != 128) return fail(YTHIP_EUNSUPPORTED, "ythip_rmsnorm_rope: head dim %d (supported: 64, 128)", d);
    if ((int64_t)B * S * (Hq + 2 * Hkv) == 0) return 0;
    if (qkv == nullptr || Qout == nullptr || q_str == nullptr) return fail(YTHIP_EINVAL, "ythip_rmsnorm_rope: NULL qkv/Q");
    if ((cos_tab == nullptr) != (sin_tab == nullptr))
        return fail(YTHIP_EINVAL, "ythip_rmsnorm_rope: cos and sin must both be given or both NULL");
    if (cos_tab != nullptr && (pos0 < 0 || ld_tab < d)) return fail(YTHIP_EINVAL, "ythip_rmsnorm_rope: bad table args");
    if ((Kout != nullptr && k_str == nullptr) || (Vout != nullptr && v_str == nullptr) || cache_pos < 0)
        return fail(YTHIP_EINVAL, "ythip_rmsnorm_rope: bad K/V output args");
    if (ld_qkv < (int64_t)(Hq + 2 * Hkv) * d) return fail(YTHIP_EINVAL, "ythip_rmsnorm_rope: ld_qkv too small");
    NormRopeArgs a{};
    a.qkv = qkv; a.ld_qkv = ld_qkv; a.wq = wq; a.wk = wk; a.eps = eps;
    a.cos_tab = cos_tab; a.sin_tab = sin_tab; a.ld_tab = ld_tab; a.pos0 = pos0;
    a.q = Qout; a.k = Kout; a.v = Vout;
    a.qs0 = q_str[0]; a.qs1 = q_str[1]; a.qs2 = q_str[2];
    if (k_str) { a.ks0 = k_str[0]; a.ks1 = k_str[1]; a.ks2 = k_str[2]; }
    if (v_str) { a.vs0 = v_str[0]; a.vs1 = v_str[1]; a.vs2 = v_str[2]; }
    a.B = B; a.S = S; a.Hq = Hq; a.Hkv = Hkv; a.cache_pos = cache_pos; a.dev_pos = dev_pos;
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (dtype) {
        case YTHIP_F32: return status_of(launch_norm_rope<F32>(a, d, s));
        case YTHIP_F16: return status_of(launch_norm_rope<F16>(a, d, s));
        case YTHIP_BF16: return status_of(launch_norm_rope<BF16>(a, d, s));
        default: return fail(YTHIP_EINVAL, "ythip_rmsnorm_rope: invalid dtype %d", dtype);
    }
}

__attribute__((visibility("default"))) int ythip_rms_norm(int dtype_in, int dtype_out, int rows, int n,
                                                          const void* x, int64_t ld_x, const float* w, float eps,
                                                          void* y, int64_t ld_y, void* stream) {
    if (rows < 0 || n < 0) return fail(YTHIP_EINVAL, "ythip_rms_norm: negative size");
    if (rows == 0 || n == 0) return 0;
    if (x == nullptr || y == nullptr || w == nullptr) return fail(YTHIP_EINVAL, "ythip_rms_norm: NULL pointer");
    if (ld_x < n || ld_y < n) return fail(YTHIP_EINVAL, "ythip_rms_norm: leading dimension smaller than n");
    if (x == y && dtype_in != dtype_out) return fail(YTHIP_EINVAL, "ythip_rms_norm: in place needs one dtype");
    hipStream_t s = static_cast<hipStream_t>(stream);
#define YTHIP_RMS(TI, TOUT) return status_of(launch_rms<TI, TOUT>(rows, n, x, ld_x, w, eps, y, ld_y, s))
    if (dtype_in == YTHIP_F32 && dtype_out == YTHIP_F32) YTHIP_RMS(F32, F32);
    if (dtype_in == YTHIP_F32 && dtype_out == YTHIP_BF16) YTHIP_RMS(F32, BF16);
    if (dtype_in == YTHIP_F32 && dtype_out == YTHIP_F16) YTHIP_RMS(F32, F16);
    if (dtype_in == YTHIP_BF16 && dtype_out == YTHIP_BF16) YTHIP_RMS(BF16, BF16);
    if (dtype_in == YTHIP_BF16 && dtype_out == YTHIP_F32) YTHIP_RMS(BF16, F32);
    if (dtype_in == YTHIP_F16 && dtype_out == YTHIP_F16) YTHIP_RMS(F16, F16);
    if (dtype_in == YTHIP_F16 && dtype_out == YTHIP_F32) YTHIP_RMS(F16, F32);
#undef YTHIP_RMS
    return fail(YTHIP_EINVAL, "ythip_rms_norm: invalid dtype pair %d/%d", dtype_in, dtype_out);
}

}  // extern "C"
