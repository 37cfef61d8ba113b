// gemv.hip — skinny GEMM (M <= 16 rows of activations against a weight
// W [N, K], i.e. the decode-time `linear`) with optional fused prologues.
//
// Reference operations replaced (example/qwen3/src/qwen3.cpp):
//   * linear(x, W) (src/function/ops.inl:84-91) for M <= 16, which the
//     reference runs as gemv_row_simd (src/kernel/avx2/sgemv.inl:443-717);
//   * rmsNorm_(x, w) feeding a linear (qwen3.cpp:271-283, 365-413; the norm is
//     src/function/normalization.inl:256-277): the normalised, bf16-rounded
//     activation is built in the GEMV's operand prologue;
//   * swish(gate) * up feeding the down projection (qwen3.cpp:193-200,
//     src/ytensor_function.inl:42-52);
//   * the greedy argmax over the LM-head logits (qwen3.cpp:465-486): the
//     epilogue leaves one (max, index) pair per 16-column tile and a one-block
//     kernel reduces them and advances the decode state.
// The prologues reproduce the standalone kernels' arithmetic exactly
// (rms_norm_kernel: same per-thread FMA order, wave butterflies and pairwise
// combination; silu_mul_kernel: same stable sigmoid), so a fused call gives
// the same bits as the unfused sequence.
//
// MI355X design: HBM-bound on the weight stream. One workgroup per 16 output
// columns; its waves split K and each wave issues all of its 16-byte weight
// loads for a round (UNR chunks per lane) before consuming any, so a single
// memory latency covers the wave's share; non-temporal loads for the weights
// (read once). v_mfma_f32_16x16x32 serves as the 16-lane dot-product reducer
// (its flops are free against the byte stream); the waves' 16 x 16 partial
// tiles are summed through LDS. Small N gets 16 waves per column tile so
// that the chip still has enough loads in flight.

#include <cfloat>
#include <type_traits>

#include "common.hpp"
#include "launch.hpp"

namespace ythip {

constexpr int GEMV_M = 16;
// Single-row GEMVs wider than this (the LM head) give each wave 4 weight rows:
// more bytes in flight per wave and a quarter of the workgroups (and of the
// prologue copies) -- measured 50 us against 97 us for the 151936 x 1024 head.
constexpr int GEMV_WIDE_N = 32768;
constexpr int GEMV_LDS_MAX = 64 * 1024;  // bytes of the staged A' (prologues 1 and 2)


// Stable sigmoid of the reference (src/ytensor_function.inl:43-52), as in silu_mul_kernel.
__device__ __forceinline__ float silu_ref(float a) {
    float sig;
    if (a >= 0.0f) {
        const float z = expf(-a);
        sig = 1.0f / (1.0f + z);
    } else {
        const float z = expf(a);
        sig = z / (1.0f + z);
    }
    return a * sig;
}

// Operand prologues of the decode GEMVs: build A' [m][k] (16-bit, row-major) in
// the dynamic LDS. load() issues the prologue's global loads into registers and
// runs BEFORE the weight loads: vector-memory loads retire in issue order, so
// the prologue's first wait then covers only its own (small, cache-resident)
// inputs and its arithmetic overlaps the weight stream. build() does the
// arithmetic (loading directly whatever did not fit in the registers) and ends
// with a barrier. All NT threads of the workgroup take part.
//   PRO 1: RMSNorm of fp32 rows (rms_norm_kernel's arithmetic and order);
//   PRO 2: swish(gate) * up of 16-bit rows [gate | up] (silu_mul_kernel's);
//   PRO 3: the split-K decode merge (attn_decode_merge's): per (row, head) the
//          max M of the splits' m, weights w_s = 2^(m_s - M) (-inf marks a split
//          merge skips) and L = sum w_s l_s, then o = sum_s w_s o_s[d] / L.
template <class T, int NT, int PRO>
struct GemvPrologue {
    using raw = typename T::raw;
    static constexpr bool EW = PRO == 1 || PRO == 2;  // elementwise prologues
    static constexpr int PJ = PRO == 2 ? 8 : 4;        // elements per thread held in registers
    static constexpr int MS = 8;                       // merge: splits held in registers
    float p0[EW ? PJ : 1], p1[EW ? PJ : 1];
    float xr[PRO == 1 ? 4 : 1];                        // RMSNorm: first reduction group of row 0
    float opre[PRO == 3 ? 2 : 1][PRO == 3 ? MS : 1];   // merge: o of this thread's 2 elements
    float mreg[PRO == 3 ? MS : 1], lreg[PRO == 3 ? MS : 1];
    int used = 0;                                      // merge: splits holding keys

    __device__ __forceinline__ void load_elem(const GemvArgs& a, int bz, int e, float& x0, float& x1) const {
        const int row = e / a.k, col = e - row * a.k;
        if constexpr (PRO == 1) {
            x0 = static_cast<const float*>(a.A)[bz * a.sa_b + (int64_t)row * a.lda + col];
            x1 = a.nw[col];
        } else {
            const raw* gp = static_cast<const raw*>(a.A) + bz * a.sa_b + (int64_t)row * a.lda;
            x0 = load_as_f32<T>(gp, col);
            x1 = load_as_f32<T>(gp, a.k + col);
        }
    }
    __device__ __forceinline__ const float* merge_src(const GemvArgs& a, int bz, int e) const {
        const int row = e / a.k, col = e - row * a.k;
        const int h = col / a.hd, d = col - h * a.hd;
        return static_cast<const float*>(a.A) + bz * a.sa_b + (int64_t)row * a.lda +
               (int64_t)h * a.splits * (a.hd + 2) + 2 + d;
    }
    __device__ __forceinline__ const float* merge_msrc(const GemvArgs& a, int bz, int rh) const {
        return static_cast<const float*>(a.A) + bz * a.sa_b + (int64_t)(rh / a.hq) * a.lda +
               (int64_t)(rh % a.hq) * a.splits * (a.hd + 2);
    }

    __device__ __forceinline__ void load(const GemvArgs& a, int bz) {
        const int tid = threadIdx.x, total = a.m * a.k;
        if constexpr (EW) {
#pragma unroll
            for (int j = 0; j < PJ; ++j) {
                p0[j] = p1[j] = 0.f;
                if (tid + j * NT < total) load_elem(a, bz, tid + j * NT, p0[j], p1[j]);
            }
        }
        if constexpr (PRO == 1) {
            const float* X = static_cast<const float*>(a.A) + bz * a.sa_b;
#pragma unroll
            for (int j = 0; j < 4; ++j) xr[j] = (tid < 256 && tid + 256 * j < a.k) ? X[tid + 256 * j] : 0.f;
        }
        if constexpr (PRO == 3) {
            const int S = a.splits, stride = a.hd + 2;
            // the split kernel's partition (decode_used); the loads below do not wait for it
            used = a.dstate != nullptr ? decode_used(max(0, min(a.dstate[YTHIP_ST_KV_LEN], a.max_ctx)), S) : S;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int e = tid + j * NT;
                const float* src = merge_src(a, bz, e < total ? e : 0);
#pragma unroll
                for (int q = 0; q < MS; ++q) opre[j][q] = (e < total && q < S) ? src[q * stride] : 0.f;
            }
            const bool owner = tid < a.m * a.hq;
            const float* msrc = merge_msrc(a, bz, owner ? tid : 0);
#pragma unroll
            for (int q = 0; q < MS; ++q) {
                mreg[q] = (owner && q < S) ? msrc[q * stride] : -INFINITY;
                lreg[q] = (owner && q < S) ? msrc[q * stride + 1] : 0.f;
            }
        }
    }

    __device__ __forceinline__ void build(const GemvArgs& a, int bz, raw* sAp) {
        const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6), total = a.m * a.k;
        if constexpr (PRO == 1) {
            __shared__ float s_part[GEMV_M][4];
            __shared__ float s_den[GEMV_M];
            // rms_norm_kernel's reduction, row by row, on the first 256 threads: the
            // sequential FMA order over i = t, t + 256, ...; a zero term leaves the
            // non-negative sum unchanged.
            const float* X = static_cast<const float*>(a.A) + bz * a.sa_b;
            for (int row = 0; row < a.m; ++row) {
                if (tid < 256) {
                    float ss = 0.f;
                    for (int i = tid; i < a.k; i += 1024) {
                        float x[4];
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            x[j] = (row == 0 && i == tid) ? xr[j]
                                                          : (i + 256 * j < a.k ? X[(int64_t)row * a.lda + i + 256 * j] : 0.f);
#pragma unroll
                        for (int j = 0; j < 4; ++j) ss = fmaf(x[j], x[j], ss);
                    }
                    ss = wave_sum(ss);
                    if (lane == 0) s_part[row][wave] = ss;
                }
            }
            __syncthreads();
            if (tid < a.m) {
                const float tot = (s_part[tid][0] + s_part[tid][1]) + (s_part[tid][2] + s_part[tid][3]);
                s_den[tid] = sqrtf(tot / (float)a.k + a.eps);
            }
            __syncthreads();
            auto finish = [&](int e, float x0, float x1) {
                const float y = (x0 / s_den[e / a.k]) * x1;
                sAp[e] = static_cast<raw>(pack2<T>(y, 0.0f) & 0xffffu);
            };
#pragma unroll
            for (int j = 0; j < PJ; ++j)
                if (tid + j * NT < total) finish(tid + j * NT, p0[j], p1[j]);
            for (int e = tid + PJ * NT; e < total; e += NT) {
                float x0, x1;
                load_elem(a, bz, e, x0, x1);
                finish(e, x0, x1);
            }
            __syncthreads();
        }
        if constexpr (PRO == 2) {
            auto finish = [&](int e, float x0, float x1) {
                const float y = silu_ref(x0) * x1;
                sAp[e] = static_cast<raw>(pack2<T>(y, 0.0f) & 0xffffu);
            };
#pragma unroll
            for (int j = 0; j < PJ; ++j)
                if (tid + j * NT < total) finish(tid + j * NT, p0[j], p1[j]);
            for (int e = tid + PJ * NT; e < total; e += NT) {
                float x0, x1;
                load_elem(a, bz, e, x0, x1);
                finish(e, x0, x1);
            }
            __syncthreads();
        }
        if constexpr (PRO == 3) {
            // splits from U on hold no key (m = -inf): their terms are skipped as
            // every empty split's is, so reading U splits gives the bits of reading S
            const int S = a.splits, U = used, hs = a.hq * S, stride = a.hd + 2;
            float* s_w = reinterpret_cast<float*>(sAp + ((total + 7) & ~7));
            float* s_L = s_w + a.m * hs;
            if (tid < a.m * a.hq) {  // this thread owns (row, head) rh = tid
                const float* msrc = merge_msrc(a, bz, tid);
                float M = -INFINITY;
#pragma unroll
                for (int q = 0; q < MS; ++q)
                    if (q < U) M = fmaxf(M, mreg[q]);
                for (int q = MS; q < U; ++q) M = fmaxf(M, msrc[q * stride]);
                float L = 0.f;
                float* w = s_w + tid * S;
#pragma unroll
                for (int q = 0; q < MS; ++q) {
                    if (q < U) {
                        float ws = -INFINITY;
                        if (M != -INFINITY && mreg[q] != -INFINITY) {
                            ws = exp2f(mreg[q] - M);
                            L = fmaf(lreg[q], ws, L);
                        }
                        w[q] = ws;
                    }
                }
                for (int q = MS; q < U; ++q) {
                    const float ms = msrc[q * stride];
                    float ws = -INFINITY;
                    if (M != -INFINITY && ms != -INFINITY) {
                        ws = exp2f(ms - M);
                        L = fmaf(msrc[q * stride + 1], ws, L);
                    }
                    w[q] = ws;
                }
                s_L[tid] = L;
            }
            __syncthreads();
            // pre: the element's first MS partial values, in registers (or not)
            auto merge_one = [&](int e, const float (&pre)[MS], bool have_pre) {
                const int row = e / a.k, col = e - row * a.k;
                const int rh = row * a.hq + col / a.hd;
                const float* src = merge_src(a, bz, e);
                const float* w = s_w + rh * S;
                float acc = 0.f;
#pragma unroll
                for (int q = 0; q < MS; ++q) {
                    if (q < U) {
                        const float ws = w[q];
                        const float o = have_pre ? pre[q] : src[q * stride];
                        if (ws != -INFINITY) acc = fmaf(o, ws, acc);
                    }
                }
                for (int q = MS; q < U; ++q) {
                    const float ws = w[q];
                    if (ws != -INFINITY) acc = fmaf(src[q * stride], ws, acc);
                }
                const float L = s_L[rh];
                const float y = L > 0.f ? acc / L : 0.f;
                sAp[e] = static_cast<raw>(pack2<T>(y, 0.0f) & 0xffffu);
            };
#pragma unroll
            for (int j = 0; j < 2; ++j)
                if (tid + j * NT < total) merge_one(tid + j * NT, opre[j], true);
            for (int e = tid + 2 * NT; e < total; e += NT) merge_one(e, opre[0], false);
            __syncthreads();
        }
    }
};

// EPI = 1 (SwiGLU epilogue): W holds 2n rows, gate rows [0, n) then up rows
// [n, 2n); a workgroup covers 8 indices i, its MFMA columns 0-7 being gate rows
// n0 + 0..7 and columns 8-15 the up rows of the same indices, so the epilogue
// rounds both to the output type (the stored gate_up of the unfused sequence),
// meets them with one lane exchange and writes swish(gate) * up (silu_mul_kernel's
// arithmetic) to C [m][n].
template <class T, class TO, int WAVES, int PRO, int EPI = 0>
__global__ __launch_bounds__(64 * WAVES) void gemv_kernel(GemvArgs a) {
    using raw = typename T::raw;
    constexpr int VEC = 16 / sizeof(raw);
    constexpr int KSTEP = 4 * VEC;  // k covered by one MFMA chunk across the 4 lane groups
    constexpr int UNR = 8;
    static_assert(PRO == 0 || sizeof(raw) == 2, "fused prologues are 16-bit");
    static_assert(EPI == 0 || PRO <= 1, "the SwiGLU epilogue takes prologue 0 or 1");
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // scalar
    const int r = lane & 15, g = lane >> 4;
    const int n0 = blockIdx.x * (EPI ? 8 : 16);
    const int bz = blockIdx.y;
    const int nsteps = (a.k + KSTEP - 1) / KSTEP;
    const int per_wave = (nsteps + WAVES - 1) / WAVES;
    const int s_begin = wave * per_wave, s_end = min(nsteps, s_begin + per_wave);
    const bool arow = r < a.m;
    bool brow;
    int wrow;
    if constexpr (EPI == 0) {
        wrow = n0 + r;
        brow = wrow < a.n;
    } else {
        brow = n0 + (r & 7) < a.n;
        wrow = (r < 8 ? 0 : a.n) + n0 + (r & 7);
    }
    const raw* __restrict__ wrp =
        static_cast<const raw*>(a.W) + bz * a.sw_b + (int64_t)(brow ? wrow : 0) * a.ldw + g * VEC;

    auto load_w = [&](int s) -> u32x4 {
        const int k = s * KSTEP + g * VEC;
        if (s < s_end && k < a.k && brow)
            return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrp + (int64_t)s * KSTEP));
        return u32x4{0u, 0u, 0u, 0u};
    };
    // Latency plan: the prologue's loads, then the first round of weight loads,
    // then the epilogue's, all before anything waits on memory.
    GemvPrologue<T, 64 * WAVES, PRO> pro;
    if constexpr (PRO != 0) pro.load(a, bz);
    u32x4 fb[UNR];
#pragma unroll
    for (int u = 0; u < UNR; ++u) fb[u] = load_w(s_begin + u);

    using oraw = typename TO::raw;
    oraw* crow = static_cast<oraw*>(a.C) + bz * a.sc_b + (int64_t)r * a.ldc;
    float cold[4] = {0.f, 0.f, 0.f, 0.f};  // C for the beta term (wave 0 stores the result)
    if (EPI == 0 && wave == 0 && arow && a.beta != 0.0f) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (n0 + 4 * g + j < a.n) cold[j] = load_as_f32<TO>(crow, n0 + 4 * g + j);
    }

    extern __shared__ u32x4 gemv_lds[];  // dynamic: m * k 16-bit values (+ prologue 3's tables)
    raw* sAp = reinterpret_cast<raw*>(gemv_lds);
    if constexpr (PRO != 0) pro.build(a, bz, sAp);

    // A operand chunk s of this lane: 8 (16-bit) or 4 (fp32) k values of row r.
    auto load_a = [&](int s) -> u32x4 {
        const int k = s * KSTEP + g * VEC;
        if (!(s < s_end && k < a.k && arow)) return u32x4{0u, 0u, 0u, 0u};
        if constexpr (PRO == 0)
            return *reinterpret_cast<const u32x4*>(static_cast<const raw*>(a.A) + bz * a.sa_b + (int64_t)r * a.lda + k);
        else
            return *reinterpret_cast<const u32x4*>(&sAp[r * a.k + k]);
    };

    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int s = s_begin; s < s_end; s += UNR) {
        if (s != s_begin) {
#pragma unroll
            for (int u = 0; u < UNR; ++u) fb[u] = load_w(s + u);
        }
        u32x4 fa[UNR];
#pragma unroll
        for (int u = 0; u < UNR; ++u) fa[u] = load_a(s + u);
#pragma unroll
        for (int u = 0; u < UNR; ++u) acc = mfma_chunk(T{}, fb[u], fa[u], acc);
    }
    // acc: lane holds C[m = r][n0 + 4g + j] partial over this wave's k range.
    __shared__ f32x4 red[WAVES][64];
    red[wave][lane] = acc;
    __syncthreads();
    if (wave != 0) return;
    f32x4 t = red[0][lane];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) t += red[w][lane];
    if constexpr (EPI == 1) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float val = a.alpha * t[j];
            if constexpr (std::is_same<TO, BF16>::value) val = bf16_bits_to_f32(f32_to_bf16_bits(val));
            if constexpr (std::is_same<TO, F16>::value) val = f16_bits_to_f32(f32_to_f16_bits(val));
            const float up = __shfl_xor(val, 32, 64);  // lane group g + 2 holds the up rows
            const int i = n0 + 4 * g + j;
            if (g < 2 && arow && i < a.n) store_from_f32<TO>(crow, i, silu_ref(val) * up);
        }
        return;
    }
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int n = n0 + 4 * g + j;
        v[j] = a.alpha * t[j];
        if (arow && n < a.n) {
            if (a.beta != 0.0f) v[j] += a.beta * cold[j];
            store_from_f32<TO>(crow, n, v[j]);
            if constexpr (std::is_same<TO, BF16>::value) v[j] = bf16_bits_to_f32(f32_to_bf16_bits(v[j]));  // as stored
            if constexpr (std::is_same<TO, F16>::value) v[j] = f16_bits_to_f32(f32_to_f16_bits(v[j]));
        }
    }
    if (a.amax != nullptr && bz == 0) {
        // row 0: lanes 0, 16, 32, 48 hold its 16 columns; lowest index wins ties, NaN never wins
        float best = -INFINITY;
        int idx = 0x7fffffff;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int n = n0 + 4 * g + j;
            if (n < a.n && (v[j] > best || (v[j] == best && n < idx))) { best = v[j]; idx = n; }
        }
#pragma unroll
        for (int off = 16; off <= 32; off <<= 1) {
            const float ob = __shfl_xor(best, off, 64);
            const int oi = __shfl_xor(idx, off, 64);
            if (ob > best || (ob == best && oi < idx)) { best = ob; idx = oi; }
        }
        if (lane == 0) {
            a.amax[2 * blockIdx.x] = best;
            a.amax[2 * blockIdx.x + 1] = __int_as_float(idx);
        }
    }
}

// 16 bytes of 16-bit weights . 16 bytes of the 16-bit operand, fp32 accumulate
// (v_dot2_f32_bf16 / v_dot2_f32_f16: the products are exact in fp32).
__device__ __forceinline__ float dot8(BF16, u32x4 w, u32x4 x, float acc) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        // element copies first: hipcc (clang 22) folds a bit_cast of a vector
        // element expression to element 0
        const uint32_t we = w[e], xe = x[e];
        acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, we), __builtin_bit_cast(bf16x2_t, xe), acc,
                                              false);
    }
    return acc;
}
__device__ __forceinline__ float dot8(F16, u32x4 w, u32x4 x, float acc) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const uint32_t we = w[e], xe = x[e];  // see dot8(BF16, ...)
        acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, we), __builtin_bit_cast(f16x2_t, xe), acc, false);
    }
    return acc;
}
__device__ __forceinline__ float dot8(F32, u32x4 w, u32x4 x, float acc) {
#pragma unroll
    for (int e = 0; e < 4; ++e) acc = fmaf(__uint_as_float(w[e]), __uint_as_float(x[e]), acc);
    return acc;
}

// Decode GEMV for ONE activation row (m == 1), the shape of every decode-step
// linear. A wave owns RPW whole weight rows: lane l takes the 16-byte chunks
// c = l, l + 64, ... of a row, so one load instruction reads 1 KB of one row
// (full 128-byte lines, unlike the MFMA layout's 64-byte pieces of 16 rows),
// all chunks of a round go out before any is used, and the row's dot product
// is the lane's in-order partial followed by one DPP wave sum. Each row is
// computed entirely inside one wave in a fixed order, so its bits do not
// depend on the workgroup shape, the prologue or the epilogue: a fused call
// and the unfused sequence it replaces agree bit for bit.
//   EPI 0: C[n] = alpha * dot + beta * C; optional per-workgroup (max, index)
//          pairs for the LM-head argmax (WAVES * RPW rows per workgroup).
//   EPI 1: RPW = 2, rows (i, n + i) of W = [gate | up]; C[i] = swish(g) * u with
//          g, u rounded to TO first (silu_mul_kernel after a 16-bit gate_up).
template <class T, class TO, int WAVES, int RPW, int PRO, int EPI, int CPL_ = 0>
__global__ __launch_bounds__(64 * WAVES) void gemv_row_kernel(GemvArgs a) {
    using raw = typename T::raw;
    constexpr int VEC = 16 / sizeof(raw);
    // chunks per lane per round (16-wave workgroups hold fewer: 128 VGPRs a lane);
    // the lane's chunk order, hence the bits, is the same for any CPL
    constexpr int CPL = CPL_ ? CPL_ : ((sizeof(raw) == 2 && WAVES < 16) ? 8 : 4);
    static_assert(PRO == 0 || sizeof(raw) == 2, "fused prologues are 16-bit");
    static_assert(EPI == 0 || (RPW == 2 && PRO <= 1), "the SwiGLU epilogue pairs a gate and an up row");
    static_assert(PRO == 0 || WAVES >= 4, "the RMSNorm prologue reduces on 256 threads");
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // scalar
    const int nch = a.k / VEC;
    int rows[RPW];
    bool rok[RPW];
#pragma unroll
    for (int j = 0; j < RPW; ++j) {
        if constexpr (EPI == 1) {
            const int i = blockIdx.x * WAVES + wave;
            rok[j] = i < a.n;
            rows[j] = j == 0 ? i : a.n + i;
        } else {
            rows[j] = (blockIdx.x * WAVES + wave) * RPW + j;
            rok[j] = rows[j] < a.n;
        }
    }
    const raw* Wp = static_cast<const raw*>(a.W);
    auto load_round = [&](int c0, u32x4 (&w)[RPW][CPL]) {
#pragma unroll
        for (int j = 0; j < RPW; ++j) {
            const raw* wr = Wp + (int64_t)(rok[j] ? rows[j] : 0) * a.ldw;
#pragma unroll
            for (int u = 0; u < CPL; ++u) {
                const int c = c0 + lane + 64 * u;
                w[j][u] = (rok[j] && c < nch) ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wr) + c)
                                              : u32x4{0u, 0u, 0u, 0u};
            }
        }
    };
    GemvPrologue<T, 64 * WAVES, PRO> pro;  // its loads go out first (see GemvPrologue)
    if constexpr (PRO != 0) pro.load(a, 0);
    u32x4 w[RPW][CPL];
    load_round(0, w);

    using oraw = typename TO::raw;
    oraw* Cp = static_cast<oraw*>(a.C);
    float cold[RPW];
#pragma unroll
    for (int j = 0; j < RPW; ++j) cold[j] = (EPI == 0 && a.beta != 0.0f && rok[j]) ? load_as_f32<TO>(Cp, rows[j]) : 0.f;

    extern __shared__ u32x4 gemv_lds[];
    raw* sAp = reinterpret_cast<raw*>(gemv_lds);
    auto load_x = [&](int c) -> u32x4 {
        if (c >= nch) return u32x4{0u, 0u, 0u, 0u};
        if constexpr (PRO == 0) return reinterpret_cast<const u32x4*>(a.A)[c];
        else return reinterpret_cast<const u32x4*>(sAp)[c];
    };
    u32x4 x[CPL];
    if constexpr (PRO == 0) {
#pragma unroll
        for (int u = 0; u < CPL; ++u) x[u] = load_x(lane + 64 * u);
    } else {
        pro.build(a, 0, sAp);
#pragma unroll
        for (int u = 0; u < CPL; ++u) x[u] = load_x(lane + 64 * u);
    }

    float acc[RPW];
#pragma unroll
    for (int j = 0; j < RPW; ++j) acc[j] = 0.f;
    for (int c0 = 0;;) {
#pragma unroll
        for (int j = 0; j < RPW; ++j)
#pragma unroll
            for (int u = 0; u < CPL; ++u) acc[j] = dot8(T{}, w[j][u], x[u], acc[j]);
        c0 += 64 * CPL;
        if (c0 >= nch) break;
        load_round(c0, w);
#pragma unroll
        for (int u = 0; u < CPL; ++u) x[u] = load_x(c0 + lane + 64 * u);
    }
    float tot[RPW];
#pragma unroll
    for (int j = 0; j < RPW; ++j) tot[j] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dpp_sum_to_lane63(acc[j])), 63));

    if constexpr (EPI == 1) {
        float g = a.alpha * tot[0], u = a.alpha * tot[1];
        if constexpr (std::is_same<TO, BF16>::value) {
            g = bf16_bits_to_f32(f32_to_bf16_bits(g));
            u = bf16_bits_to_f32(f32_to_bf16_bits(u));
        }
        if constexpr (std::is_same<TO, F16>::value) {
            g = f16_bits_to_f32(f32_to_f16_bits(g));
            u = f16_bits_to_f32(f32_to_f16_bits(u));
        }
        if (lane == 0 && rok[0]) store_from_f32<TO>(Cp, rows[0], silu_ref(g) * u);
        return;
    }
    float v[RPW];
#pragma unroll
    for (int j = 0; j < RPW; ++j) {
        v[j] = a.alpha * tot[j];
        if (a.beta != 0.0f) v[j] += a.beta * cold[j];
        if (lane == 0 && rok[j]) store_from_f32<TO>(Cp, rows[j], v[j]);
        if constexpr (std::is_same<TO, BF16>::value) v[j] = bf16_bits_to_f32(f32_to_bf16_bits(v[j]));  // as stored
        if constexpr (std::is_same<TO, F16>::value) v[j] = f16_bits_to_f32(f32_to_f16_bits(v[j]));
    }
    if (a.amax != nullptr) {
        // the workgroup's rows: lowest index wins ties, NaN never wins
        float best = -INFINITY;
        int idx = 0x7fffffff;
#pragma unroll
        for (int j = 0; j < RPW; ++j)
            if (rok[j] && (v[j] > best || (v[j] == best && rows[j] < idx))) { best = v[j]; idx = rows[j]; }
        __shared__ float s_best[WAVES];
        __shared__ int s_idx[WAVES];
        if (lane == 0) {
            s_best[wave] = best;
            s_idx[wave] = idx;
        }
        __syncthreads();
        if (tid == 0) {
            for (int w2 = 1; w2 < WAVES; ++w2)
                if (s_best[w2] > best || (s_best[w2] == best && s_idx[w2] < idx)) { best = s_best[w2]; idx = s_idx[w2]; }
            a.amax[2 * blockIdx.x] = best;
            a.amax[2 * blockIdx.x + 1] = __int_as_float(idx);
        }
    }
}

// Final greedy step over the per-tile (max, index) pairs; same tie rule and
// state update as argmax_step_kernel.
__global__ __launch_bounds__(1024) void argmax_finish_kernel(const float* parts, int n_parts, int32_t* token,
                                                             int32_t* history, int32_t* state) {
    float best = -INFINITY;
    int idx = 0x7fffffff;
    for (int i = threadIdx.x; i < n_parts; i += 1024) {
        const float v = parts[2 * i];
        const int id = __float_as_int(parts[2 * i + 1]);
        if (v > best || (v == best && id < idx)) { best = v; idx = id; }
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

// Waves per column tile. The kernel holds ~90 VGPRs (5 waves per SIMD, 20 per
// CU), so a 16-wave workgroup is alone on its CU: 16 waves while the grid fits
// the 256 CUs in one round (more loads in flight per tile), 8 waves (two
// workgroups per CU) beyond that. Depends only on the tile count, so a fused
// call and the unfused sequence it replaces sum the k partials alike.
inline bool gemv_wide(int64_t tiles) { return tiles <= 256; }

template <class T, class TO, int WAVES, int RPW, int PRO, int EPI, int CPL = 0>
hipError_t launch_row_t(const GemvArgs& a, size_t lds, hipStream_t s) {
    const int per_wg = EPI ? WAVES : WAVES * RPW;
    gemv_row_kernel<T, TO, WAVES, RPW, PRO, EPI, CPL><<<(a.n + per_wg - 1) / per_wg, 64 * WAVES, lds, s>>>(a);
    return hipGetLastError();
}

template <class T, class TO, int PRO, int EPI = 0>
hipError_t launch_gemv_t(const GemvArgs& a, int batch, hipStream_t s) {
    if (a.m == 1 && batch == 1) {
        // One activation row: the row-per-wave kernel, whose bits do not depend on
        // the workgroup shape, so each variant takes the shape measured fastest on
        // the decode shapes: 4 rows per workgroup without a prologue; 16 waves
        // where a prologue is built once per workgroup (fewer copies of it) or the
        // argmax wants 16-row tiles; 16 gate/up pairs with the SwiGLU epilogue.
        size_t lds = PRO == 0 ? 0 : (size_t)a.k * sizeof(typename T::raw);
        if (PRO == 3) lds = ((size_t)a.k + 7) / 8 * 16 + ((size_t)a.hq * a.splits + (size_t)a.hq) * 4;
        if constexpr (EPI == 1) return launch_row_t<T, TO, 16, 2, PRO, 1>(a, lds, s);
        if (a.n > GEMV_WIDE_N) {
            if (a.k / (16 / (int)sizeof(typename T::raw)) <= 128) return launch_row_t<T, TO, 4, 4, PRO, 0, 2>(a, lds, s);
            return launch_row_t<T, TO, 4, 4, PRO, 0, 4>(a, lds, s);
        }
        if (PRO != 0 || a.amax != nullptr) return launch_row_t<T, TO, 16, 1, PRO, 0>(a, lds, s);
        return launch_row_t<T, TO, 4, 1, PRO, 0>(a, lds, s);
    }
    const int tiles = EPI ? (a.n + 7) / 8 : (a.n + 15) / 16;
    size_t lds = PRO == 0 ? 0 : (size_t)a.m * a.k * sizeof(typename T::raw);
    if (PRO == 3) lds = ((size_t)a.m * a.k + 7) / 8 * 16 + ((size_t)a.m * a.hq * a.splits + (size_t)a.m * a.hq) * 4;
    if (gemv_wide((int64_t)tiles * batch))
        gemv_kernel<T, TO, 16, PRO, EPI><<<dim3(tiles, batch), 1024, lds, s>>>(a);
    else
        gemv_kernel<T, TO, 8, PRO, EPI><<<dim3(tiles, batch), 512, lds, s>>>(a);
    return hipGetLastError();
}

}  // namespace

int gemv_merge_dispatch(int dtype_in, int dtype_out, const GemvArgs& a, hipStream_t s) {
    if (dtype_in == YTHIP_BF16 && dtype_out == YTHIP_BF16) return status_of(launch_gemv_t<BF16, BF16, 3>(a, 1, s));
    if (dtype_in == YTHIP_BF16 && dtype_out == YTHIP_F32) return status_of(launch_gemv_t<BF16, F32, 3>(a, 1, s));
    if (dtype_in == YTHIP_F16 && dtype_out == YTHIP_F16) return status_of(launch_gemv_t<F16, F16, 3>(a, 1, s));
    if (dtype_in == YTHIP_F16 && dtype_out == YTHIP_F32) return status_of(launch_gemv_t<F16, F32, 3>(a, 1, s));
    return fail(YTHIP_EUNSUPPORTED, "ythip_gemv_attn_merge: unsupported dtype/dtype_out %d/%d", dtype_in, dtype_out);
}

int gemv_swiglu_dispatch(int prologue, int dtype, const GemvArgs& a, hipStream_t s) {
    if (dtype == YTHIP_BF16)
        return status_of(prologue ? launch_gemv_t<BF16, BF16, 1, 1>(a, 1, s) : launch_gemv_t<BF16, BF16, 0, 1>(a, 1, s));
    if (dtype == YTHIP_F16)
        return status_of(prologue ? launch_gemv_t<F16, F16, 1, 1>(a, 1, s) : launch_gemv_t<F16, F16, 0, 1>(a, 1, s));
    return fail(YTHIP_EUNSUPPORTED, "ythip_gemv_swiglu: weights and output must be bf16 or fp16");
}

int gemv_dispatch(int prologue, int dtype_in, int dtype_out, const GemvArgs& a, int batch, hipStream_t s) {
#define YTHIP_GEMV(TI, TOUT)                                                          \
    do {                                                                              \
        if (prologue == 0) return status_of(launch_gemv_t<TI, TOUT, 0>(a, batch, s)); \
        if constexpr (sizeof(typename TI::raw) == 2) {                                \
            if (prologue == 1) return status_of(launch_gemv_t<TI, TOUT, 1>(a, batch, s)); \
            if (prologue == 2) return status_of(launch_gemv_t<TI, TOUT, 2>(a, batch, s)); \
        }                                                                             \
        return fail(YTHIP_EUNSUPPORTED, "gemv: prologue %d needs 16-bit inputs", prologue); \
    } while (0)
    if (dtype_in == YTHIP_BF16 && dtype_out == YTHIP_BF16) YTHIP_GEMV(BF16, BF16);
    if (dtype_in == YTHIP_BF16 && dtype_out == YTHIP_F32) YTHIP_GEMV(BF16, F32);
    if (dtype_in == YTHIP_F16 && dtype_out == YTHIP_F16) YTHIP_GEMV(F16, F16);
    if (dtype_in == YTHIP_F16 && dtype_out == YTHIP_F32) YTHIP_GEMV(F16, F32);
    if (dtype_in == YTHIP_F32 && dtype_out == YTHIP_F32) YTHIP_GEMV(F32, F32);
#undef YTHIP_GEMV
    return fail(YTHIP_EUNSUPPORTED, "gemv: unsupported dtype_in/dtype_out combination %d/%d", dtype_in, dtype_out);
}

}  // namespace ythip

using namespace ythip;

extern "C" {

__attribute__((visibility("default"))) int ythip_gemv_fused(int prologue, int dtype_in, int dtype_out, int m, int n,
                                                            int k, const void* A, int64_t lda, const float* norm_w,
                                                            float eps, const void* W, int64_t ldw, void* C,
                                                            int64_t ldc, float alpha, float beta,
                                                            float* argmax_parts, void* stream) {
    if (prologue < 0 || prologue > 2) return fail(YTHIP_EINVAL, "ythip_gemv_fused: prologue %d", prologue);
    if (m < 0 || n < 0 || k < 0) return fail(YTHIP_EINVAL, "ythip_gemv_fused: negative size");
    if (m > GEMV_M) return fail(YTHIP_EUNSUPPORTED, "ythip_gemv_fused: m = %d (at most %d rows)", m, GEMV_M);
    if (m == 0 || n == 0) return 0;
    if (!A || !W || !C) return fail(YTHIP_EINVAL, "ythip_gemv_fused: NULL A, W or C");
    if (prologue == 1 && (norm_w == nullptr || dtype_in == YTHIP_F32))
        return fail(YTHIP_EINVAL, "ythip_gemv_fused: the RMSNorm prologue needs norm_w and 16-bit weights");
    const int es = dtype_in == YTHIP_F32 ? 4 : 2;
    const int vec = 16 / es;
    const int64_t a_cols = prologue == 2 ? 2 * (int64_t)k : k;
    if (k % vec || ldw % vec || (prologue == 1 ? lda % 4 : lda % vec) || lda < a_cols || ldw < k ||
        (reinterpret_cast<uintptr_t>(A) % 16) || (reinterpret_cast<uintptr_t>(W) % 16) ||
        (prologue == 1 && (reinterpret_cast<uintptr_t>(norm_w) % 16)))
        return fail(YTHIP_EUNSUPPORTED,
                    "ythip_gemv_fused: rows of A/W must be 16-byte aligned and k a multiple of %d", vec);
    if (ldc < n) return fail(YTHIP_EINVAL, "ythip_gemv_fused: ldc < n");
    if (prologue != 0 && (int64_t)m * k * es > GEMV_LDS_MAX)
        return fail(YTHIP_EUNSUPPORTED, "ythip_gemv_fused: m * k = %lld exceeds the %d-byte operand staging",
                    (long long)m * k, GEMV_LDS_MAX);
    GemvArgs a{};
    a.A = A; a.lda = lda; a.nw = norm_w; a.eps = eps;
    a.W = W; a.ldw = ldw; a.C = C; a.ldc = ldc;
    a.m = m; a.n = n; a.k = k; a.alpha = alpha; a.beta = beta;
    a.amax = argmax_parts;
    return gemv_dispatch(prologue, dtype_in, dtype_out, a, 1, static_cast<hipStream_t>(stream));
}

__attribute__((visibility("default"))) int ythip_gemv_swiglu(int prologue, int dtype, int m, int inter, int k,
                                                             const void* A, int64_t lda, const float* norm_w,
                                                             float eps, const void* W, int64_t ldw, void* C,
                                                             int64_t ldc, void* stream) {
    if (prologue < 0 || prologue > 1) return fail(YTHIP_EINVAL, "ythip_gemv_swiglu: prologue %d", prologue);
    if (m < 0 || inter < 0 || k < 0) return fail(YTHIP_EINVAL, "ythip_gemv_swiglu: negative size");
    if (m > GEMV_M) return fail(YTHIP_EUNSUPPORTED, "ythip_gemv_swiglu: m = %d (at most %d rows)", m, GEMV_M);
    if (m == 0 || inter == 0) return 0;
    if (!A || !W || !C) return fail(YTHIP_EINVAL, "ythip_gemv_swiglu: NULL A, W or C");
    if (dtype != YTHIP_BF16 && dtype != YTHIP_F16)
        return fail(YTHIP_EUNSUPPORTED, "ythip_gemv_swiglu: weights and output must be bf16 or fp16");
    if (prologue == 1 && norm_w == nullptr) return fail(YTHIP_EINVAL, "ythip_gemv_swiglu: the RMSNorm prologue needs norm_w");
    if (k % 8 || ldw % 8 || (prologue == 1 ? lda % 4 : lda % 8) || lda < k || ldw < k ||
        (reinterpret_cast<uintptr_t>(A) % 16) || (reinterpret_cast<uintptr_t>(W) % 16) ||
        (prologue == 1 && (reinterpret_cast<uintptr_t>(norm_w) % 16)))
        return fail(YTHIP_EUNSUPPORTED, "ythip_gemv_swiglu: rows of A/W must be 16-byte aligned and k a multiple of 8");
    if (ldc < inter) return fail(YTHIP_EINVAL, "ythip_gemv_swiglu: ldc < inter");
    if (prologue != 0 && (int64_t)m * k * 2 > GEMV_LDS_MAX)
        return fail(YTHIP_EUNSUPPORTED, "ythip_gemv_swiglu: m * k = %lld exceeds the %d-byte operand staging",
                    (long long)m * k, GEMV_LDS_MAX);
    GemvArgs a{};
    a.A = A; a.lda = lda; a.nw = norm_w; a.eps = eps;
    a.W = W; a.ldw = ldw; a.C = C; a.ldc = ldc;
    a.m = m; a.n = inter; a.k = k; a.alpha = 1.0f; a.beta = 0.0f;
    return gemv_swiglu_dispatch(prologue, dtype, a, static_cast<hipStream_t>(stream));
}

__attribute__((visibility("default"))) int ythip_gemv_attn_merge(int dtype, int dtype_out, int m, int n, int hq,
                                                                 int hd, int splits, const float* partials,
                                                                 int64_t ld_part, const void* W, int64_t ldw, void* C,
                                                                 int64_t ldc, float alpha, float beta,
                                                                 const int32_t* dev_state, int max_ctx, void* stream) {
    const char* who = "ythip_gemv_attn_merge";
    if (m < 0 || n < 0 || hq < 0 || hd <= 0 || splits <= 0) return fail(YTHIP_EINVAL, "%s: bad size", who);
    if (dev_state != nullptr && max_ctx <= 0) return fail(YTHIP_EINVAL, "%s: max_ctx must be positive", who);
    if (m > GEMV_M) return fail(YTHIP_EUNSUPPORTED, "%s: m = %d (at most %d rows)", who, m, GEMV_M);
    if (m == 0 || n == 0 || hq == 0) return 0;
    if (!partials || !W || !C) return fail(YTHIP_EINVAL, "%s: NULL partials, W or C", who);
    const int64_t k = (int64_t)hq * hd;
    if (hd % 8 || ldw % 8 || ldw < k || (reinterpret_cast<uintptr_t>(W) % 16) ||
        (reinterpret_cast<uintptr_t>(partials) % 4))
        return fail(YTHIP_EUNSUPPORTED, "%s: W rows must be 16-byte aligned and hd a multiple of 8", who);
    if (ld_part < (int64_t)hq * splits * (hd + 2)) return fail(YTHIP_EINVAL, "%s: ld_part too small", who);
    if (ldc < n) return fail(YTHIP_EINVAL, "%s: ldc < n", who);
    const int64_t lds = (m * k + 7) / 8 * 16 + ((int64_t)m * hq * splits + (int64_t)m * hq) * 4;
    if (lds > GEMV_LDS_MAX)
        return fail(YTHIP_EUNSUPPORTED, "%s: m * hq * hd = %lld with %d splits exceeds the %d-byte staging", who,
                    (long long)(m * k), splits, GEMV_LDS_MAX);
    GemvArgs a{};
    a.A = partials; a.lda = ld_part;
    a.W = W; a.ldw = ldw; a.C = C; a.ldc = ldc;
    a.m = m; a.n = n; a.k = (int)k; a.alpha = alpha; a.beta = beta;
    a.hq = hq; a.hd = hd; a.splits = splits;
    a.dstate = dev_state; a.max_ctx = max_ctx;
    return gemv_merge_dispatch(dtype, dtype_out, a, static_cast<hipStream_t>(stream));
}

__attribute__((visibility("default"))) int ythip_argmax_finish(const float* parts, int n_parts, int32_t* token,
                                                               int32_t* history, int32_t* state, void* stream) {
    if (n_parts <= 0 || parts == nullptr || token == nullptr)
        return fail(YTHIP_EINVAL, "ythip_argmax_finish: bad arguments");
    argmax_finish_kernel<<<1, 1024, 0, static_cast<hipStream_t>(stream)>>>(parts, n_parts, token, history, state);
    return status_of(hipGetLastError());
}

}  // extern "C"
