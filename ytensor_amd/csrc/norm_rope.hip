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
// Both kernels are HBM-bound elementwise passes. The fused one gives each
// (token, head) row d/16 lanes with 8 rotate-half pairs each (16-byte loads and
// stores, non-temporal reads of the projection output, a shuffle sum of
// squares over the row's lanes).

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
    int cache_rows;   // K/V rows are written at (cache_pos + s) % cache_rows (a ring)
    int tab_rows;     // cos/sin rows
    int32_t* dev_state;  // when set: pos0 / cache_pos from the decode-state record (graph-replayable decode)
};

// LPR lanes per (token, head) row of d = 2 * HALF: lane j of a row holds
// x[8j .. 8j+7] and x[HALF + 8j .. HALF + 8j+7], i.e. 8 rotate-half pairs, so
// every global access is 16 bytes (bf16/fp16) and RoPE stays inside the lane.
template <class T, int HALF>
__global__ __launch_bounds__(256) void norm_rope_kernel(NormRopeArgs a) {
    using raw = typename T::raw;
    constexpr int D = 2 * HALF;
    constexpr int LPR = HALF / 8;            // lanes per row
    constexpr int RPB = 256 / LPR;           // rows per block
    const int j = threadIdx.x % LPR;
    const int H = a.Hq + 2 * a.Hkv;
    const int rows = a.B * a.S * H;          // < 2^31, checked on the host
    const int row = blockIdx.x * RPB + threadIdx.x / LPR;
    if (row >= rows) return;                 // whole rows leave together (LPR divides 64)
    const int h = row % H;
    const int tok = row / H;
    const int s = tok % a.S;
    const int b = tok / a.S;
    const int pos0 = a.dev_state ? a.dev_state[YTHIP_ST_ROPE_POS] : a.pos0;
    const int cache_pos = a.dev_state ? a.dev_state[YTHIP_ST_SLOT] : a.cache_pos;
    // A device-held position out of range is flagged and never used as an
    // address (host positions were checked before the launch).
    const bool rope_ok = pos0 >= 0 && pos0 + s < a.tab_rows;
    const bool slot_ok = cache_pos >= 0 && cache_pos < a.cache_rows;
    if (a.dev_state != nullptr && j == 0 && h == 0) {
        if (a.cos_tab != nullptr && !rope_ok) atomicOr(&a.dev_state[YTHIP_ST_ERROR], (int)YTHIP_ST_ERR_ROPE);
        if ((a.k != nullptr || a.v != nullptr) && !slot_ok)
            atomicOr(&a.dev_state[YTHIP_ST_ERROR], (int)YTHIP_ST_ERR_CACHE);
    }
    const int64_t crow = slot_ok ? (cache_pos + s) % a.cache_rows : 0;

    const raw* src = static_cast<const raw*>(a.qkv) + (int64_t)tok * a.ld_qkv + (int64_t)h * D + 8 * j;
    float x1[8], x2[8];
    auto load8 = [&](const raw* p, float (&x)[8]) {
        if constexpr (sizeof(raw) == 2) {
            const u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                x[2 * e] = lo_as_f32(T{}, w[e]);
                x[2 * e + 1] = hi_as_f32(T{}, w[e]);
            }
        } else {
            const f32x4 lo = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
            const f32x4 hi = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p) + 1);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                x[e] = lo[e];
                x[e + 4] = hi[e];
            }
        }
    };
    auto store8 = [&](raw* p, const float (&x)[8]) {
        if constexpr (sizeof(raw) == 2) {
            *reinterpret_cast<u32x4*>(p) = u32x4{pack2<T>(x[0], x[1]), pack2<T>(x[2], x[3]), pack2<T>(x[4], x[5]),
                                                 pack2<T>(x[6], x[7])};
        } else {
            reinterpret_cast<f32x4*>(p)[0] = f32x4{x[0], x[1], x[2], x[3]};
            reinterpret_cast<f32x4*>(p)[1] = f32x4{x[4], x[5], x[6], x[7]};
        }
    };
    // Every load is issued before the first use (the row, then its norm
    // weights, then its table row): vector loads retire in order, so the
    // weights and the cached tables arrive behind the row instead of costing a
    // round trip each after the reduction. v rows load them too (unused).
    load8(src, x1);
    load8(src + HALF, x2);
    const bool is_q = h < a.Hq, is_k = !is_q && h < a.Hq + a.Hkv;
    const float* w = is_q ? a.wq : a.wk;
    f32x4 wa = {}, wb = {}, wc = {}, wd = {};
    if (w != nullptr) {
        const f32x4* w1 = reinterpret_cast<const f32x4*>(w + 8 * j);
        const f32x4* w2 = reinterpret_cast<const f32x4*>(w + HALF + 8 * j);
        wa = w1[0];
        wb = w1[1];
        wc = w2[0];
        wd = w2[1];
    }
    f32x4 c0 = {}, c1 = {}, s0 = {}, s1 = {};
    if (a.cos_tab != nullptr && rope_ok) {
        const int64_t t = (int64_t)(pos0 + s) * a.ld_tab + 8 * j;
        c0 = *reinterpret_cast<const f32x4*>(a.cos_tab + t);
        c1 = *reinterpret_cast<const f32x4*>(a.cos_tab + t + 4);
        s0 = *reinterpret_cast<const f32x4*>(a.sin_tab + t);
        s1 = *reinterpret_cast<const f32x4*>(a.sin_tab + t + 4);
    }

    raw* dst;
    if (is_q) {
        dst = static_cast<raw*>(a.q) + b * a.qs0 + h * a.qs1 + s * a.qs2;
    } else if (is_k) {
        if (!slot_ok) return;
        dst = static_cast<raw*>(a.k) + b * a.ks0 + (h - a.Hq) * a.ks1 + crow * a.ks2;
    } else {
        if (a.v == nullptr || !slot_ok) return;
        dst = static_cast<raw*>(a.v) + b * a.vs0 + (h - a.Hq - a.Hkv) * a.vs1 + crow * a.vs2;
        store8(dst + 8 * j, x1);
        store8(dst + HALF + 8 * j, x2);
        return;
    }
    if (static_cast<void*>(dst) == nullptr) return;
    if (w != nullptr) {
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = fmaf(x2[e], x2[e], fmaf(x1[e], x1[e], ss));
#pragma unroll
        for (int off = LPR / 2; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, 64);
        const float den = sqrtf(ss / (float)D + a.eps);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            x1[e] = (x1[e] / den) * wa[e];
            x1[e + 4] = (x1[e + 4] / den) * wb[e];
            x2[e] = (x2[e] / den) * wc[e];
            x2[e + 4] = (x2[e + 4] / den) * wd[e];
        }
    }
    if (a.cos_tab != nullptr) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float c = e < 4 ? c0[e] : c1[e - 4], sn = e < 4 ? s0[e] : s1[e - 4];
            const float y1 = fmaf(x1[e], c, -(x2[e] * sn));
            const float y2 = fmaf(x2[e], c, x1[e] * sn);
            x1[e] = y1;
            x2[e] = y2;
        }
    }
    store8(dst + 8 * j, x1);
    store8(dst + HALF + 8 * j, x2);
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

// rms_norm_kernel with element strides (one normalised axis of any stride, the
// axes overloads of rmsNorm / rmsNorm_): the same element-to-thread assignment
// and operation order, so the same bits as the contiguous kernels.
template <class T, class TO>
__global__ __launch_bounds__(256) void rms_norm_strided_kernel(const void* x, int64_t ldx, int64_t csx,
                                                               const float* w, float eps, void* y, int64_t ldy,
                                                               int64_t csy, int n) {
    const int64_t row = blockIdx.x;
    const auto* xr = static_cast<const typename T::raw*>(x) + row * ldx;
    auto* yr = static_cast<typename TO::raw*>(y) + row * ldy;
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += 256) {
        const float v = load_as_f32<T>(xr, i * csx);
        ss = fmaf(v, v, ss);
    }
    __shared__ float part[4];
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float tot = (part[0] + part[1]) + (part[2] + part[3]);
    const float den = sqrtf(tot / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += 256)
        store_from_f32<TO>(yr, i * csy, (load_as_f32<T>(xr, i * csx) / den) * w[i]);
}

// rms_norm_kernel for n <= 256 * J: the same element-to-thread assignment and
// operation order (so the same bits), with every load of the row and its
// weights issued up front and the row kept in registers for the second pass
// (one memory round trip instead of a dependent load per loop trip, and no
// re-read). Indices past n re-read the last element, unused.
template <class T, class TO, int J>
__global__ __launch_bounds__(256) void rms_norm_reg_kernel(const void* x, int64_t ldx, const float* w, float eps,
                                                           void* y, int64_t ldy, int n) {
    const int64_t row = blockIdx.x;
    const auto* xr = static_cast<const typename T::raw*>(x) + row * ldx;
    auto* yr = static_cast<typename TO::raw*>(y) + row * ldy;
    float v[J], wv[J];
#pragma unroll
    for (int j = 0; j < J; ++j) v[j] = load_as_f32<T>(xr, min((int)threadIdx.x + 256 * j, n - 1));
#pragma unroll
    for (int j = 0; j < J; ++j) wv[j] = w[min((int)threadIdx.x + 256 * j, n - 1)];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < J; ++j)
        if ((int)threadIdx.x + 256 * j < n) ss = fmaf(v[j], v[j], ss);
    __shared__ float part[4];
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float tot = (part[0] + part[1]) + (part[2] + part[3]);
    const float den = sqrtf(tot / (float)n + eps);
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int i = threadIdx.x + 256 * j;
        if (i < n) store_from_f32<TO>(yr, i, (v[j] / den) * wv[j]);
    }
}

namespace {

template <class T>
hipError_t launch_norm_rope(const NormRopeArgs& a, int d, hipStream_t s) {
    const int64_t rows = (int64_t)a.B * a.S * (a.Hq + 2 * a.Hkv);
    switch (d) {
        case 64: norm_rope_kernel<T, 32><<<(unsigned)((rows + 63) / 64), 256, 0, s>>>(a); break;   // 4 lanes, 64 rows / block
        case 128: norm_rope_kernel<T, 64><<<(unsigned)((rows + 31) / 32), 256, 0, s>>>(a); break;  // 8 lanes, 32 rows / block
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <class T, class TO>
hipError_t launch_rms(int rows, int n, const void* x, int64_t ldx, const float* w, float eps, void* y, int64_t ldy,
                      hipStream_t s, int64_t csx = 1, int64_t csy = 1) {
    if (csx != 1 || csy != 1) {
        rms_norm_strided_kernel<T, TO><<<rows, 256, 0, s>>>(x, ldx, csx, w, eps, y, ldy, csy, n);
        return hipGetLastError();
    }
    if (n <= 1024) rms_norm_reg_kernel<T, TO, 4><<<rows, 256, 0, s>>>(x, ldx, w, eps, y, ldy, n);
    else if (n <= 2048) rms_norm_reg_kernel<T, TO, 8><<<rows, 256, 0, s>>>(x, ldx, w, eps, y, ldy, n);
    else if (n <= 4096) rms_norm_reg_kernel<T, TO, 16><<<rows, 256, 0, s>>>(x, ldx, w, eps, y, ldy, n);
    else rms_norm_kernel<T, TO><<<rows, 256, 0, s>>>(x, ldx, w, eps, y, ldy, n);
    return hipGetLastError();
}

}  // namespace

}  // namespace ythip

using namespace ythip;

extern "C" {

__attribute__((visibility("default"))) int ythip_rmsnorm_rope(
    int dtype, int B, int S, int Hq, int Hkv, int d, const void* qkv, int64_t ld_qkv, const float* wq,
    const float* wk, float eps, const float* cos_tab, const float* sin_tab, int64_t ld_tab, int tab_rows, int pos0,
    void* Qout, const int64_t q_str[3], void* Kout, const int64_t k_str[3], void* Vout, const int64_t v_str[3],
    int cache_rows, int cache_pos, int32_t* dev_state, void* stream) {
    if (B < 0 || S < 0 || Hq < 0 || Hkv < 0) return fail(YTHIP_EINVAL, "ythip_rmsnorm_rope: negative size");
    if (d != 64 && d != 128) return fail(YTHIP_EUNSUPPORTED, "ythip_rmsnorm_rope: head dim %d (supported: 64, 128)", d);
    if ((int64_t)B * S * (Hq + 2 * Hkv) == 0) return 0;
    if (qkv == nullptr || Qout == nullptr || q_str == nullptr) return fail(YTHIP_EINVAL, "ythip_rmsnorm_rope: NULL qkv/Q");
    if ((cos_tab == nullptr) != (sin_tab == nullptr))
        return fail(YTHIP_EINVAL, "ythip_rmsnorm_rope: cos and sin must both be given or both NULL");
    if (cos_tab != nullptr && (ld_tab < d || tab_rows < 0))
        return fail(YTHIP_EINVAL, "ythip_rmsnorm_rope: bad table args");
    if (cos_tab != nullptr && dev_state == nullptr && (pos0 < 0 || (int64_t)pos0 + S > tab_rows))
        return fail(YTHIP_EINVAL, "ythip_rmsnorm_rope: RoPE rows %d..%d outside the %d-row table", pos0,
                    pos0 + S - 1, tab_rows);
    if ((Kout != nullptr && k_str == nullptr) || (Vout != nullptr && v_str == nullptr))
        return fail(YTHIP_EINVAL, "ythip_rmsnorm_rope: bad K/V output args");
    if ((Kout != nullptr || Vout != nullptr) &&
        (cache_rows <= 0 || S > cache_rows || (dev_state == nullptr && (cache_pos < 0 || cache_pos >= cache_rows))))
        return fail(YTHIP_EINVAL, "ythip_rmsnorm_rope: cache row %d / %d rows for S=%d", cache_pos, cache_rows, S);
    if (ld_qkv < (int64_t)(Hq + 2 * Hkv) * d) return fail(YTHIP_EINVAL, "ythip_rmsnorm_rope: ld_qkv too small");
    if ((int64_t)B * S * (Hq + 2 * Hkv) >= (int64_t)1 << 31)
        return fail(YTHIP_EUNSUPPORTED, "ythip_rmsnorm_rope: more than 2^31 rows");
    // every access is 16 bytes wide: rows, strides and tables must keep that alignment
    {
        const int es = dtype == YTHIP_F32 ? 4 : 2;
        const int64_t v = 16 / es;  // elements per 16 bytes
        auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
        bool ok = al16(qkv) && ld_qkv % v == 0 && al16(Qout) && q_str[0] % v == 0 && q_str[1] % v == 0 &&
                  q_str[2] % v == 0;
        if (Kout) ok = ok && al16(Kout) && k_str[0] % v == 0 && k_str[1] % v == 0 && k_str[2] % v == 0;
        if (Vout) ok = ok && al16(Vout) && v_str[0] % v == 0 && v_str[1] % v == 0 && v_str[2] % v == 0;
        if (wq) ok = ok && al16(wq);
        if (wk) ok = ok && al16(wk);
        if (cos_tab) ok = ok && al16(cos_tab) && al16(sin_tab) && ld_tab % 4 == 0;
        if (!ok)
            return fail(YTHIP_EUNSUPPORTED,
                        "ythip_rmsnorm_rope: tensors, strides and tables must be 16-byte aligned");
    }
    NormRopeArgs a{};
    a.qkv = qkv; a.ld_qkv = ld_qkv; a.wq = wq; a.wk = wk; a.eps = eps;
    a.cos_tab = cos_tab; a.sin_tab = sin_tab; a.ld_tab = ld_tab; a.pos0 = pos0;
    a.q = Qout; a.k = Kout; a.v = Vout;
    a.qs0 = q_str[0]; a.qs1 = q_str[1]; a.qs2 = q_str[2];
    if (k_str) { a.ks0 = k_str[0]; a.ks1 = k_str[1]; a.ks2 = k_str[2]; }
    if (v_str) { a.vs0 = v_str[0]; a.vs1 = v_str[1]; a.vs2 = v_str[2]; }
    a.B = B; a.S = S; a.Hq = Hq; a.Hkv = Hkv; a.cache_pos = cache_pos; a.dev_state = dev_state;
    a.cache_rows = cache_rows > 0 ? cache_rows : 1;
    a.tab_rows = tab_rows;
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

__attribute__((visibility("default"))) int ythip_rms_norm_strided(int dtype_in, int dtype_out, int rows, int n,
                                                                  const void* x, int64_t ld_x, int64_t cs_x,
                                                                  const float* w, float eps, void* y, int64_t ld_y,
                                                                  int64_t cs_y, void* stream) {
    if (rows < 0 || n < 0) return fail(YTHIP_EINVAL, "ythip_rms_norm_strided: negative size");
    if (rows == 0 || n == 0) return 0;
    if (x == nullptr || y == nullptr || w == nullptr) return fail(YTHIP_EINVAL, "ythip_rms_norm_strided: NULL pointer");
    if (x == y && (dtype_in != dtype_out || ld_x != ld_y || cs_x != cs_y))
        return fail(YTHIP_EINVAL, "ythip_rms_norm_strided: in place needs one dtype and one layout");
    hipStream_t s = static_cast<hipStream_t>(stream);
#define YTHIP_RMS(TI, TOUT) return status_of(launch_rms<TI, TOUT>(rows, n, x, ld_x, w, eps, y, ld_y, s, cs_x, cs_y))
    if (dtype_in == YTHIP_F32 && dtype_out == YTHIP_F32) YTHIP_RMS(F32, F32);
    if (dtype_in == YTHIP_F32 && dtype_out == YTHIP_BF16) YTHIP_RMS(F32, BF16);
    if (dtype_in == YTHIP_F32 && dtype_out == YTHIP_F16) YTHIP_RMS(F32, F16);
    if (dtype_in == YTHIP_BF16 && dtype_out == YTHIP_BF16) YTHIP_RMS(BF16, BF16);
    if (dtype_in == YTHIP_BF16 && dtype_out == YTHIP_F32) YTHIP_RMS(BF16, F32);
    if (dtype_in == YTHIP_F16 && dtype_out == YTHIP_F16) YTHIP_RMS(F16, F16);
    if (dtype_in == YTHIP_F16 && dtype_out == YTHIP_F32) YTHIP_RMS(F16, F32);
#undef YTHIP_RMS
    return fail(YTHIP_EINVAL, "ythip_rms_norm_strided: invalid dtype pair %d/%d", dtype_in, dtype_out);
}

}  // extern "C"
