// ytoracle.cpp — CPU restatement of YTensor's (SnifferCaptain/ytensor v0.13)
// CPU algorithms on the MI355X hot path.
//
// TEST INFRASTRUCTURE ONLY. This library is the parity checker for the HIP
// kernels in ytensor_amd/csrc and the "port" CPU baseline in bench.py. The
// product path (libythip.so) never links, loads or calls it.
//
// Every function restates one reference algorithm, cited as file:line relative
// to the reference root. Summation orders follow the reference so that the
// fp32 results are bit-identical to YTensor's AVX2 path where the reference
// order is fixed by intrinsics (sequential FMA chains, 2x8-lane GEMV
// accumulators, the hsum_ps tree). The build uses -ffp-contract=off and
// writes every FMA the reference performs as std::fma, so the compiler cannot
// reassociate or contract differently from what is written here.
//
// Pinning (what checks each function): see tests/test_oracle_*.py.
//   - randn / bf16 / fp16: golden vectors written by the compiled reference
//     (tests/golden) plus a closed-form known-answer table.
//   - sgemm / gemv / flash / rmsnorm / rope / qwen3: bit-exact or ulp-level
//     comparison against the compiled reference (oracle/_ref) on fixtures, plus
//     closed forms (identity, permutation, small integers, single visible key,
//     Q=0 mean, decode == last prefill row) and fp64 brute force.

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <immintrin.h>
#include <limits>
#include <random>
#include <vector>

#ifdef _OPENMP
#include <omp.h>
#endif

#define OEXPORT extern "C" __attribute__((visibility("default")))

namespace {

inline uint32_t f2u(float x) { uint32_t u; std::memcpy(&u, &x, 4); return u; }
inline float u2f(uint32_t u) { float x; std::memcpy(&x, &u, 4); return x; }

// ---------------------------------------------------------------------------
// Types
// ---------------------------------------------------------------------------

// include/types/bfloat16.hpp:78-80 — "round_to_nearest_even": adds bit16>>1 and
// shifts. Not IEEE RNE (a value with bit16 = 0 and low half exactly 0x8000
// truncates; NaN is not special-cased).
inline uint16_t bf16_round(float x) {
    uint32_t u = f2u(x);
    return static_cast<uint16_t>((u + ((u & 0x00010000u) >> 1)) >> 16);
}
// include/types/bfloat16.hpp:285-291
inline float bf16_to_f32(uint16_t h) { return u2f(static_cast<uint32_t>(h) << 16); }

// include/types/float_spec.hpp:435-491 (FloatSpec<1,5,10>::fromFloat32):
// zero/subnormal fp32 -> signed 0, inf/NaN kept (NaN mantissa = 1), underflow
// (realExp <= 0) flushes to signed 0, overflow -> inf, otherwise mantissa RNE.
inline uint16_t f16_round(float x) {
    uint32_t bits = f2u(x);
    uint32_t s = (bits >> 31) & 1u, e = (bits >> 23) & 0xFFu, m = bits & 0x7FFFFFu;
    uint32_t ne, nm;
    if (e == 0) { ne = 0; nm = 0; }
    else if (e == 0xFF) { ne = 31; nm = m != 0 ? 1 : 0; }
    else {
        int real = static_cast<int>(e) - 127 + 15;
        if (real <= 0) { ne = 0; nm = 0; }
        else if (real >= 31) { ne = 31; nm = 0; }
        else {
            ne = static_cast<uint32_t>(real);
            nm = m >> 13;
            uint32_t rem = m & 0x1FFFu, half = 0x1000u;
            if (rem > half || (rem == half && (nm & 1u))) {
                nm++;
                if (nm >= 0x400u) { nm = 0; ne++; if (ne >= 31) { ne = 31; nm = 0; } }
            }
        }
    }
    return static_cast<uint16_t>((s << 15) | (ne << 10) | nm);
}
// include/types/float_spec.hpp:299-370 (toFloat32), specialised to fp16.
inline float f16_to_f32(uint16_t h) {
    uint32_t s = (h >> 15) & 1u, e = (h >> 10) & 0x1Fu, m = h & 0x3FFu, r;
    if (e == 0) {
        if (m == 0) r = s << 31;
        else {
            int shift = 0;
            while ((m & 0x200u) == 0 && shift < 10) { m <<= 1; shift++; }
            m = (m << 1) & 0x3FFu;
            int ee = 1 - shift;
            int ne = ee - 15 + 127;
            r = (ne <= 0) ? ((s << 31) | (m << 13)) : ((s << 31) | (static_cast<uint32_t>(ne) << 23) | (m << 13));
        }
    } else if (e == 31) {
        r = (s << 31) | (0xFFu << 23) | (m != 0 ? 1u : 0u);
    } else {
        r = (s << 31) | ((e - 15 + 127) << 23) | (m << 13);
    }
    return u2f(r);
}

// ---------------------------------------------------------------------------
// RNG: include/ytensor_infos.hpp:81 (global std::mt19937), ytensor_core.inl:729-732
// (seed), ytensor_core.hpp:44-58 (randn: a fresh normal_distribution<double>
// per tensor, values drawn in row-major order, then static_cast<T>).
// ---------------------------------------------------------------------------
std::mt19937 g_gen;

// ---------------------------------------------------------------------------
// hsum_ps: src/kernel/avx2/gemm_utils.inl:117-126
//   ((v0+v4)+(v1+v5)) + ((v2+v6)+(v3+v7))
// ---------------------------------------------------------------------------
inline float hsum8(const float v[8]) {
    float a0 = v[0] + v[4], a1 = v[1] + v[5], a2 = v[2] + v[6], a3 = v[3] + v[7];
    return (a0 + a1) + (a2 + a3);
}

// gemv_dot_ncols<N> for one column: src/kernel/avx2/sgemv.inl:32-52.
// Two 8-lane accumulators over 16-element steps, one 8-step, hsum(acc0+acc1),
// then a scalar tail.
inline float dot_2x8(const float* a, const float* b, int k) {
    float acc0[8] = {0}, acc1[8] = {0};
    int p = 0;
    for (; p + 16 <= k; p += 16)
        for (int l = 0; l < 8; ++l) {
            acc0[l] = std::fma(a[p + l], b[p + l], acc0[l]);
            acc1[l] = std::fma(a[p + 8 + l], b[p + 8 + l], acc1[l]);
        }
    for (; p + 8 <= k; p += 8)
        for (int l = 0; l < 8; ++l) acc0[l] = std::fma(a[p + l], b[p + l], acc0[l]);
    float t[8];
    for (int l = 0; l < 8; ++l) t[l] = acc0[l] + acc1[l];
    float s = hsum8(t);
    for (; p < k; ++p) s = std::fma(a[p], b[p], s);
    return s;
}

// sdot_contiguous: src/kernel/avx2/sdot.inl:13-35 (4 accumulators over 32-steps).
inline float dot_4x8(const float* x, const float* y, int n) {
    float acc[4][8] = {{0}};
    int i = 0;
    for (; i + 32 <= n; i += 32)
        for (int q = 0; q < 4; ++q)
            for (int l = 0; l < 8; ++l) acc[q][l] = std::fma(x[i + 8 * q + l], y[i + 8 * q + l], acc[q][l]);
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; ++l) acc[0][l] = std::fma(x[i + l], y[i + l], acc[0][l]);
    float t[8];
    for (int l = 0; l < 8; ++l) t[l] = (acc[0][l] + acc[1][l]) + (acc[2][l] + acc[3][l]);
    float s = hsum8(t);
    for (; i < n; ++i) s = std::fma(x[i], y[i], s);
    return s;
}

inline float dot_strided(const float* x, const float* y, int n, int64_t incx, int64_t incy) {
    // src/kernel/avx2/sdot.inl:5-10
    float s = 0.0f;
    for (int i = 0; i < n; ++i) s = std::fma(x[i * incx], y[i * incy], s);
    return s;
}

// ---------------------------------------------------------------------------
// M=1 GEMV: src/kernel/avx2/sgemv.inl:443-717 (gemv_row_simd)
// ---------------------------------------------------------------------------
void gemv_row(const float* A, const float* B, float* C, int n, int k, float alpha, float beta,
              int64_t csa, int64_t rsb, int64_t csb, int64_t csc) {
    if (csa == 1 && csb == 1 && rsb == n && csc == 1) {
        // gemv_row_rowmajor_block (sgemv.inl:98-230): C = beta*C, then for each
        // p: C[j] = fma(alpha*A[p], B[p][j], C[j]) in p order. Column tails
        // (width % 8) use a scalar sum of up to 8 products added to C.
        if (beta == 0.0f) std::fill(C, C + n, 0.0f);
        else if (beta != 1.0f) for (int j = 0; j < n; ++j) C[j] *= beta;
        const int vec_w = (n / 8) * 8;
        int p = 0;
        auto tail = [&](int p0, int cnt) {
            for (int j = vec_w; j < n; ++j) {
                // c += a0*b0 + a1*b1 + ... as contracted by the reference build:
                // s = fma(a0, b0, a1*b1); s = fma(a_q, b_q, s) for q >= 2; c = c + s.
                auto bq = [&](int q) { return B[static_cast<int64_t>(p0 + q) * n + j]; };
                float s = std::fma(alpha * A[p0], bq(0), (alpha * A[p0 + 1]) * bq(1));
                for (int q = 2; q < cnt; ++q) s = std::fma(alpha * A[p0 + q], bq(q), s);
                C[j] += s;
            }
        };
        for (; p + 8 <= k; p += 8) {
            for (int q = 0; q < 8; ++q) {
                float a = alpha * A[p + q];
                const float* b = B + static_cast<int64_t>(p + q) * n;
                for (int j = 0; j < vec_w; ++j) C[j] = std::fma(a, b[j], C[j]);
            }
            tail(p, 8);
        }
        for (; p + 4 <= k; p += 4) {
            for (int q = 0; q < 4; ++q) {
                float a = alpha * A[p + q];
                const float* b = B + static_cast<int64_t>(p + q) * n;
                for (int j = 0; j < vec_w; ++j) C[j] = std::fma(a, b[j], C[j]);
            }
            tail(p, 4);
        }
        for (; p < k; ++p) {
            float a = alpha * A[p];
            const float* b = B + static_cast<int64_t>(p) * n;
            for (int j = 0; j < vec_w; ++j) C[j] = std::fma(a, b[j], C[j]);
            for (int j = vec_w; j < n; ++j) C[j] = std::fma(a, b[j], C[j]);
        }
        return;
    }
    if (csa == 1 && rsb == 1 && csc == 1) {
        // gemv_row_colmajor_kernel<4> (sgemv.inl:379-425): full groups of 4
        // columns use gemv_dot_ncols<4>; leftover columns use sdot_contiguous.
        const int full = (n / 4) * 4;
#pragma omp parallel for schedule(static) if (n >= 1024)
        for (int j = 0; j < n; ++j) {
            const float* bcol = B + static_cast<int64_t>(j) * csb;
            float s = (j < full) ? dot_2x8(A, bcol, k) : dot_4x8(A, bcol, k);
            C[j] = (beta == 0.0f) ? alpha * s : alpha * s + beta * C[j];
        }
        return;
    }
    // Remaining strided layouts (sgemv.inl:459-717): sequential per-column dot
    // products. Not on the configured path; ulp-level only.
    for (int j = 0; j < n; ++j) {
        float s = dot_strided(A, B + static_cast<int64_t>(j) * csb, k, csa, rsb);
        C[j * csc] = alpha * s + beta * C[j * csc];
    }
}

// ---------------------------------------------------------------------------
// Blocked GEMM: src/kernel/avx2/sgemm.inl:268-340 (sgemm_rowmajor) and the
// exact-layout dispatch at 611-715. For alpha=1, beta=0 every exact-layout
// route (row/row/row, col/col/col, W^T cache, A^T cache) computes each output
// as one FMA chain over k = 0..K-1 starting from +0: later kc panels reload C
// and continue the chain (kernel_row_full_accum_fast, 174-202).
// Implementation (this oracle's own tiling; only the per-element chain has to
// match): B is packed into 24-column strips, k runs in blocks of 256, and a
// 4-row x 24-column register tile (12 AVX2 accumulators) advances every output
// by one FMA per k in k order; between k blocks the tile is stored and
// reloaded, which is exact. Edge rows / columns run the same chain in scalar
// std::fma. OpenMP over the row blocks of a k block.
// ---------------------------------------------------------------------------
void gemm_chain(const float* A, int64_t rsa, int64_t csa, const float* B, int64_t rsb, int64_t csb,
                float* C, int64_t rsc, int64_t csc, int m, int n, int k) {
    constexpr int MR = 4, NR = 24, KB = 256;
    const int nstrip = (n + NR - 1) / NR;
    // packed B: strip s, row p -> Bp[(s * k + p) * NR + jj], zero-padded past n
    std::vector<float> Bp(static_cast<size_t>(nstrip) * k * NR);
#pragma omp parallel for schedule(static)
    for (int sidx = 0; sidx < nstrip; ++sidx)
        for (int p = 0; p < k; ++p)
            for (int jj = 0; jj < NR; ++jj) {
                const int j = sidx * NR + jj;
                Bp[(static_cast<size_t>(sidx) * k + p) * NR + jj] = j < n ? B[p * rsb + j * csb] : 0.0f;
            }
    const bool c_row = (csc == 1);
    std::vector<float> Ctmp;
    float* Cw = C;
    int64_t ldc = rsc;
    if (!c_row) {
        Ctmp.assign(static_cast<size_t>(m) * n, 0.0f);
        Cw = Ctmp.data();
        ldc = n;
    }
    // Loop order: k block -> block of MB rows (its A panel, MB x KB, stays in
    // L2) -> 24-column strip (KB x 24 of packed B, in L1) -> 4-row tiles.
    constexpr int MB = 128;
    const int nrb = (m + MB - 1) / MB;
    for (int p0 = 0; p0 < k; p0 += KB) {
        const int p1 = std::min(k, p0 + KB);
        const bool first = (p0 == 0);
#pragma omp parallel for schedule(dynamic, 1)
        for (int rb = 0; rb < nrb; ++rb) {
            const int r0 = rb * MB, r1 = std::min(m, r0 + MB);
            const int rfull = r0 + (r1 - r0) / MR * MR;
            for (int sidx = 0; sidx < nstrip; ++sidx) {
                const int j0 = sidx * NR, nw = std::min(NR, n - j0);
                const float* bs = &Bp[static_cast<size_t>(sidx) * k * NR];
                if (nw == NR) {
                    for (int i0 = r0; i0 < rfull; i0 += MR) {
                        __m256 acc[MR][3];
#pragma GCC unroll 4
                        for (int r = 0; r < MR; ++r)
#pragma GCC unroll 3
                            for (int t = 0; t < 3; ++t)
                                acc[r][t] = first ? _mm256_setzero_ps()
                                                  : _mm256_loadu_ps(Cw + (i0 + r) * ldc + j0 + 8 * t);
                        for (int p = p0; p < p1; ++p) {
                            const __m256 b0 = _mm256_loadu_ps(bs + static_cast<size_t>(p) * NR);
                            const __m256 b1 = _mm256_loadu_ps(bs + static_cast<size_t>(p) * NR + 8);
                            const __m256 b2 = _mm256_loadu_ps(bs + static_cast<size_t>(p) * NR + 16);
#pragma GCC unroll 4
                            for (int r = 0; r < MR; ++r) {
                                const __m256 a = _mm256_set1_ps(A[(i0 + r) * rsa + p * csa]);
                                acc[r][0] = _mm256_fmadd_ps(a, b0, acc[r][0]);
                                acc[r][1] = _mm256_fmadd_ps(a, b1, acc[r][1]);
                                acc[r][2] = _mm256_fmadd_ps(a, b2, acc[r][2]);
                            }
                        }
#pragma GCC unroll 4
                        for (int r = 0; r < MR; ++r)
#pragma GCC unroll 3
                            for (int t = 0; t < 3; ++t) _mm256_storeu_ps(Cw + (i0 + r) * ldc + j0 + 8 * t, acc[r][t]);
                    }
                }
                // edge rows (and a partial last strip): the same chain, scalar
                for (int i = (nw == NR ? rfull : r0); i < r1; ++i)
                    for (int jj = 0; jj < nw; ++jj) {
                        float c = first ? 0.0f : Cw[i * ldc + j0 + jj];
                        for (int p = p0; p < p1; ++p)
                            c = std::fma(A[i * rsa + p * csa], bs[static_cast<size_t>(p) * NR + jj], c);
                        Cw[i * ldc + j0 + jj] = c;
                    }
            }
        }
    }
    if (!c_row)
        for (int i = 0; i < m; ++i)
            for (int j = 0; j < n; ++j) C[i * rsc + j * csc] = Ctmp[static_cast<size_t>(i) * n + j];
}

constexpr int KC_DEFAULT = 500;  // include/kernel/avx2/gemm_utils.hpp:55 (g_gemm_kc)

void sgemm_full(const float* A, const float* B, float* C, int m, int n, int k, float alpha, float beta,
                int64_t rsa, int64_t csa, int64_t rsb, int64_t csb, int64_t rsc, int64_t csc) {
    // src/kernel/avx2/sgemm.inl:594-609: empty and degenerate shapes.
    if (m == 0 || n == 0) return;
    if (k == 0 || alpha == 0.0f) {
        for (int i = 0; i < m; ++i)
            for (int j = 0; j < n; ++j) {
                float& c = C[i * rsc + j * csc];
                c = (beta == 0.0f) ? 0.0f : (beta != 1.0f ? c * beta : c);
            }
        return;
    }
    if (m == 1 && n == 1) {
        float s = (csa == 1 && rsb == 1) ? dot_4x8(A, B, k) : dot_strided(A, B, k, csa, rsb);
        *C = alpha * s + beta * (*C);
        return;
    }
    if (k == 1) {
        // sger (src/kernel/avx2/sger.inl:5-78): C = (alpha*x_i)*y_j [+ beta*C]
        for (int i = 0; i < m; ++i) {
            float a = alpha * A[i * rsa];
            for (int j = 0; j < n; ++j) {
                float& c = C[i * rsc + j * csc];
                c = (beta == 0.0f) ? a * B[j * csb] : std::fma(a, B[j * csb], beta * c);
            }
        }
        return;
    }
    if (m == 1) { gemv_row(A, B, C, n, k, alpha, beta, csa, rsb, csb, csc); return; }
    if (n == 1) {
        // gemv_col_simd (sgemv.inl:719-768) -> gemv_col_rowmajor_contiguous_range
        // (sgemv.inl:58-96): one 8-lane accumulator over 8-steps, hsum, FMA tail,
        // C = fma(alpha, sum, beta*C).
        for (int i = 0; i < m; ++i) {
            const float* a = A + i * rsa;
            float s;
            if (csa == 1 && rsb == 1) {
                float acc[8] = {0};
                int p = 0;
                for (; p + 8 <= k; p += 8)
                    for (int l = 0; l < 8; ++l) acc[l] = std::fma(a[p + l], B[p + l], acc[l]);
                s = hsum8(acc);
                for (; p < k; ++p) s = std::fma(a[p], B[p], s);
            } else {
                s = dot_strided(a, B, k, csa, rsb);
            }
            C[i * rsc] = std::fma(alpha, s, beta * C[i * rsc]);
        }
        return;
    }
    const bool a_exact = (csa == 1 && rsa == k) || (rsa == 1 && csa == m);
    const bool b_exact = (csb == 1 && rsb == n) || (rsb == 1 && csb == k);
    const bool c_row_exact = (csc == 1 && rsc == n);
    const bool c_col_exact = (rsc == 1 && csc == m);
    if (alpha == 1.0f && beta == 0.0f && a_exact && b_exact && (c_row_exact || c_col_exact)) {
        gemm_chain(A, rsa, csa, B, rsb, csb, C, rsc, csc, m, n, k);
        return;
    }
    // Generic path (sgemm.inl:717-787): per kc=500 panel, an FMA chain from 0
    // combined into C by the store kernels.
    const bool c_rowmajor = (csc == 1 && rsc >= n);
    std::vector<float> part(static_cast<size_t>(m) * n);
    for (int pp = 0; pp < k; pp += KC_DEFAULT) {
        const int kc = std::min(KC_DEFAULT, k - pp);
        const bool first = (pp == 0);
        gemm_chain(A + pp * csa, rsa, csa, B + pp * rsb, rsb, csb, part.data(), n, 1, m, n, kc);
        for (int i = 0; i < m; ++i)
            for (int j = 0; j < n; ++j) {
                float& c = C[i * rsc + j * csc];
                const float t = part[static_cast<size_t>(i) * n + j];
                if (c_rowmajor && alpha == 1.0f) {
                    // kernel_row_zero / kernel_row_load continue the chain; the
                    // first panel with beta != 0 pre-scales C.
                    if (first) c = (beta == 0.0f) ? t : t + c * beta;  // approximate for beta != 0
                    else c = c + t;
                } else if (c_rowmajor) {
                    // kernel_row_alphabeta (gemm_utils.inl:267-292)
                    float v = t * alpha;
                    if (first && beta != 0.0f) v = std::fma(beta, c, v);
                    else if (!first) v = v + c;
                    c = v;
                } else {
                    // kernel_row_generic_store (gemm_utils.inl:294-315)
                    float v = alpha * t;
                    v = first ? v + beta * c : v + c;
                    c = v;
                }
            }
    }
}

// ---------------------------------------------------------------------------
// Flash attention, one (batch, head) matrix.
// src/kernel/avx2/flash_attention.inl:274-443 (_flashAttentionImpl, prefill)
// and 202-272 (_flashAttentionDecodeGemvImpl, q_len == 1).
// mask: nullptr = all visible; otherwise byte mask [q_len, mask_stride].
// ---------------------------------------------------------------------------
constexpr int NR = 16;  // include/kernel/avx2/gemm_utils.hpp:48 (NR_ROW): keys per tile

struct MaskView {
    const uint8_t* data; int64_t stride;
    bool operator()(int r, int c) const { return data == nullptr || data[r * stride + c] != 0; }
};

void flash_decode(const float* Q, const float* K, const float* V, float* O, int kv_len, int hd, int dv,
                  float scale, int64_t csq, int64_t rsk, int64_t csk, int64_t rsv, int64_t csv, int64_t cso,
                  MaskView mask, const float* bias, int64_t rsb, int64_t csb) {
    (void)rsb;
    std::vector<float> s(kv_len);
    // scores = scale * (q . k_j) through gemv_row_simd(Q, K^T, ..., alpha=scale)
    gemv_row(Q, K, s.data(), kv_len, hd, scale, 0.0f, csq, csk, rsk, 1);
    float mx = -std::numeric_limits<float>::infinity();
    bool any = false;
    for (int c = 0; c < kv_len; ++c) {
        if (!mask(0, c)) { s[c] = -std::numeric_limits<float>::infinity(); continue; }
        s[c] += bias ? bias[c * csb] : 0.0f;
        mx = std::max(mx, s[c]);
        any = true;
    }
    auto zero = [&]() { for (int d = 0; d < dv; ++d) O[d * cso] = 0.0f; };
    if (!any) { zero(); return; }
    float sum = 0.0f;
    for (int c = 0; c < kv_len; ++c) {
        if (!mask(0, c)) { s[c] = 0.0f; continue; }
        s[c] = std::exp(s[c] - mx);
        sum += s[c];
    }
    if (sum == 0.0f) { zero(); return; }
    const float inv = 1.0f / sum;
    for (int c = 0; c < kv_len; ++c) s[c] *= inv;
    // O = P . V through gemv_row_simd(scores, V, ...)
    gemv_row(s.data(), V, O, dv, kv_len, 1.0f, 0.0f, 1, rsv, csv, cso);
}

void flash_prefill(const float* Q, const float* K, const float* V, float* O, int q_len, int kv_len, int hd,
                   int dv, float scale, int64_t rsq, int64_t csq, int64_t rsk, int64_t csk, int64_t rsv,
                   int64_t csv, int64_t rso, int64_t cso, MaskView mask, const float* bias, int64_t rsb,
                   int64_t csb) {
    if (q_len == 0 || kv_len == 0 || hd == 0 || dv == 0) return;
    const float NEG_INF = -std::numeric_limits<float>::infinity();
    constexpr int MR = 6;  // include/kernel/avx2/gemm_utils.hpp:47 (MR_ROW): query rows per block
    // K packed per 16-key tile as [d][16] (pack_b_generic, flash_attention.inl:302-305)
    // so each score chain over d runs for 16 keys side by side.
    const int ntiles = (kv_len + NR - 1) / NR;
    std::vector<float> kp(static_cast<size_t>(ntiles) * hd * NR, 0.0f);
    for (int t = 0; t < ntiles; ++t)
        for (int j = 0; j < NR && t * NR + j < kv_len; ++j)
            for (int d = 0; d < hd; ++d)
                kp[(static_cast<size_t>(t) * hd + d) * NR + j] = K[static_cast<int64_t>(t * NR + j) * rsk + d * csk];
    std::vector<float> qp(static_cast<size_t>(MR) * hd), acc(dv);
    // one block of MR query rows at a time, as _flashAttentionImpl's q_block loop
    // (flash_attention.inl:309-443): every key tile's 6 x 16 score tile comes from
    // one pass over the packed K (dispatch_fma_row: per element an FMA chain over
    // d from 0, here eight lanes at a time), then each row's online-softmax step.
    for (int qi = 0; qi < q_len; qi += MR) {
        const int mr = std::min(MR, q_len - qi);
        for (int i = 0; i < MR; ++i)
            for (int d = 0; d < hd; ++d)
                qp[static_cast<size_t>(i) * hd + d] = i < mr ? Q[static_cast<int64_t>(qi + i) * rsq + d * csq] : 0.0f;
        float row_max[MR], row_l[MR];
        for (int i = 0; i < mr; ++i) {
            row_max[i] = NEG_INF;
            row_l[i] = 0.0f;
            float* orow = O + static_cast<int64_t>(qi + i) * rso;
            for (int d = 0; d < dv; ++d) orow[d * cso] = 0.0f;
        }
        for (int kj = 0; kj < kv_len; kj += NR) {
            const int nr = std::min(NR, kv_len - kj);
            bool vis[MR][NR];
            bool any_block = false;
            for (int i = 0; i < mr; ++i)
                for (int j = 0; j < nr; ++j) {
                    vis[i][j] = mask(qi + i, kj + j);
                    any_block |= vis[i][j];
                }
            if (!any_block) continue;  // _flashTileAllFalse (flash_attention.inl:334-336)
            alignas(32) float score[MR][NR];
            {
                const float* kt = &kp[static_cast<size_t>(kj / NR) * hd * NR];
                __m256 c[MR][2];
                for (int i = 0; i < MR; ++i) c[i][0] = c[i][1] = _mm256_setzero_ps();
                for (int d = 0; d < hd; ++d) {
                    const __m256 b0 = _mm256_loadu_ps(kt + d * NR), b1 = _mm256_loadu_ps(kt + d * NR + 8);
                    for (int i = 0; i < MR; ++i) {
                        const __m256 a = _mm256_set1_ps(qp[static_cast<size_t>(i) * hd + d]);
                        c[i][0] = _mm256_fmadd_ps(a, b0, c[i][0]);
                        c[i][1] = _mm256_fmadd_ps(a, b1, c[i][1]);
                    }
                }
                for (int i = 0; i < MR; ++i) {
                    _mm256_store_ps(&score[i][0], c[i][0]);
                    _mm256_store_ps(&score[i][8], c[i][1]);
                }
            }
            for (int i = 0; i < mr; ++i) {
                float* orow = O + static_cast<int64_t>(qi + i) * rso;
                float prob[NR];
                bool any_vis = false;
                for (int j = 0; j < nr; ++j) any_vis |= vis[i][j];
                if (!any_vis) continue;  // the row contributes nothing to this tile (flash_attention.inl:377-379)
                // flash_attention.inl:361-398: scale (+bias), running max, exp, new l.
                float tile_max = NEG_INF;
                for (int j = 0; j < nr; ++j) {
                    if (!vis[i][j]) { prob[j] = 0.0f; continue; }
                    const float sc = bias ? score[i][j] * scale + bias[(qi + i) * rsb + (kj + j) * csb]
                                          : score[i][j] * scale;
                    prob[j] = sc;
                    tile_max = std::max(tile_max, sc);
                }
                const float prev_max = row_max[i];
                const float new_max = std::max(prev_max, tile_max);
                const float prev_scale = std::isfinite(prev_max) ? std::exp(prev_max - new_max) : 0.0f;
                float tile_sum = 0.0f;
                for (int j = 0; j < nr; ++j) {
                    if (!vis[i][j]) continue;
                    const float p = std::exp(prob[j] - new_max);
                    prob[j] = p;
                    tile_sum += p;
                }
                const float l_scaled = row_l[i] * prev_scale;  // shared with the rescale below
                const float new_l = l_scaled + tile_sum;
                if (new_l == 0.0f) continue;
                const float rescale = row_l[i] == 0.0f ? 0.0f : (l_scaled / new_l);
                // flash_attention.inl:402-404: rows whose (l, max) did not change are skipped.
                if (new_l == row_l[i] && new_max == row_max[i]) continue;
                const float inv_new_l = 1.0f / new_l;
                // _flashAccumulateRowContiguous (160-200): O = O*rescale, then FMA of
                // (p_j * inv_new_l) * v_j over the tile's keys in key order, skipping p_j == 0.
                for (int d = 0; d < dv; ++d) acc[d] = (rescale == 0.0f) ? 0.0f : orow[d * cso] * rescale;
                for (int j = 0; j < nr; ++j) {
                    if (prob[j] == 0.0f) continue;
                    const float w = prob[j] * inv_new_l;
                    const float* vr = V + static_cast<int64_t>(kj + j) * rsv;
                    int d = 0;
                    if (csv == 1) {
                        const __m256 wv = _mm256_set1_ps(w);
                        for (; d + 8 <= dv; d += 8)
                            _mm256_storeu_ps(&acc[d], _mm256_fmadd_ps(wv, _mm256_loadu_ps(vr + d), _mm256_loadu_ps(&acc[d])));
                    }
                    for (; d < dv; ++d) acc[d] = std::fma(w, vr[d * csv], acc[d]);
                }
                for (int d = 0; d < dv; ++d) orow[d * cso] = acc[d];
                row_max[i] = new_max;
                row_l[i] = new_l;
            }
        }
    }
}

}  // namespace

// ===========================================================================
// Exported C ABI (ctypes from tests/ and bench.py)
// ===========================================================================

OEXPORT int oracle_abi_version(void) { return 1; }

OEXPORT void oracle_bf16_round(const float* x, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = bf16_round(x[i]);
}
OEXPORT void oracle_bf16_to_f32(const uint16_t* x, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = bf16_to_f32(x[i]);
}
OEXPORT void oracle_f16_round(const float* x, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = f16_round(x[i]);
}
OEXPORT void oracle_f16_to_f32(const uint16_t* x, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = f16_to_f32(x[i]);
}

// YTensor<float,N>::seed(s): reseeds the shared generator.
OEXPORT void oracle_seed(uint32_t s) { g_gen.seed(s); }
// YTensor<float,N>::randn(...): n values, one fresh normal_distribution<double>.
OEXPORT void oracle_randn(float* out, int64_t n) {
    std::normal_distribution<double> dist(0.0, 1.0);
    for (int64_t i = 0; i < n; ++i) out[i] = static_cast<float>(dist(g_gen));
}

OEXPORT void oracle_sgemm(const float* A, const float* B, float* C, int m, int n, int k, float alpha, float beta,
                          int64_t rsa, int64_t csa, int64_t rsb, int64_t csb, int64_t rsc, int64_t csc) {
    sgemm_full(A, B, C, m, n, k, alpha, beta, rsa, csa, rsb, csb, rsc, csc);
}

// One-matrix flash attention with the reference's kernel signature
// (include/kernel/avx2/flash_attention.hpp:21-44); mask bytes are bools.
OEXPORT void oracle_flash_attention(const float* Q, const float* K, const float* V, float* O, int q_len,
                                    int kv_len, int head_dim, int value_dim, float scale, int64_t rsq,
                                    int64_t csq, int64_t rsk, int64_t csk, int64_t rsv, int64_t csv, int64_t rso,
                                    int64_t cso, const uint8_t* mask, int64_t mask_stride, const float* bias,
                                    int64_t rsbias, int64_t csbias) {
    MaskView mv{mask, mask_stride};
    if (q_len == 1)
        flash_decode(Q, K, V, O, kv_len, head_dim, value_dim, scale, csq, rsk, csk, rsv, csv, cso, mv, bias,
                     rsbias, csbias);
    else
        flash_prefill(Q, K, V, O, q_len, kv_len, head_dim, value_dim, scale, rsq, csq, rsk, csk, rsv, csv, rso,
                      cso, mv, bias, rsbias, csbias);
}

// Batched GQA SDPA over contiguous [B,H,S,D] tensors, as the qwen3 example
// drives it (example/qwen3/src/qwen3.cpp:252-264): q-head h reads kv-head
// h / (Hq/Hkv); causal mask ki <= (kv_len - q_len) + qi (qwen3.cpp:46-55,
// 104-126); scale 0 means 1/sqrt(D) (src/function/ops.inl:378-381).
// OpenMP over (batch, head) as broadcastInplace does (src/kernel/broadcast.inl:391-445).
OEXPORT void oracle_sdpa_gqa(const float* Q, const float* K, const float* V, float* O, int B, int Hq, int Hkv,
                             int q_len, int kv_len, int D, float scale, int causal) {
    if (scale == 0.0f) scale = 1.0f / std::sqrt(static_cast<float>(D));
    const int G = Hq / Hkv;
    std::vector<uint8_t> mask;
    if (causal) {
        mask.resize(static_cast<size_t>(q_len) * kv_len);
        const int off = kv_len - q_len;
        for (int i = 0; i < q_len; ++i)
            for (int j = 0; j < kv_len; ++j) mask[static_cast<size_t>(i) * kv_len + j] = (j <= off + i) ? 1 : 0;
    }
    const uint8_t* mp = causal ? mask.data() : nullptr;
#pragma omp parallel for schedule(dynamic, 1)
    for (int bh = 0; bh < B * Hq; ++bh) {
        const int b = bh / Hq, h = bh % Hq, kh = h / G;
        const float* q = Q + (static_cast<int64_t>(b) * Hq + h) * q_len * D;
        const float* k = K + (static_cast<int64_t>(b) * Hkv + kh) * kv_len * D;
        const float* v = V + (static_cast<int64_t>(b) * Hkv + kh) * kv_len * D;
        float* o = O + (static_cast<int64_t>(b) * Hq + h) * q_len * D;
        oracle_flash_attention(q, k, v, o, q_len, kv_len, D, D, scale, D, 1, D, 1, D, 1, D, 1, mp, kv_len,
                               nullptr, 0, 0);
    }
}

// rmsNorm_ over the last axis of a contiguous [rows, n] tensor:
// src/function/normalization.inl:256-267 -> _rmsAxes_ (33-54): mean of x*x by
// YTensor::mean(axis) (src/ytensor_math.inl:532-553, running mean
// m += (x - m)/(j+1)), then a /= sqrt(m + eps); _applyScale_ (88-101): a *= w.
OEXPORT void oracle_rms_norm(float* x, const float* w, int64_t rows, int n, float eps) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        float* a = x + r * n;
        float m = 0.0f;
        for (int j = 0; j < n; ++j) {
            const float sq = a[j] * a[j];
            m += (sq - m) / static_cast<float>(j + 1);
        }
        const float den = std::sqrt(m + eps);
        for (int j = 0; j < n; ++j) {
            a[j] /= den;
            a[j] *= w[j];
        }
    }
}

// RoPECache::precompute: example/qwen3/src/qwen3.cpp:161-175. Tables [max_len, dim].
OEXPORT void oracle_rope_precompute(int dim, int max_len, float theta, float* cosv, float* sinv) {
    const int half = dim / 2;
    for (int t = 0; t < max_len; ++t)
        for (int i = 0; i < half; ++i) {
            const float freq = 1.0f / std::pow(theta, 2.0f * i / dim);
            const float angle = t * freq;
            cosv[t * dim + i] = cosv[t * dim + i + half] = std::cos(angle);
            sinv[t * dim + i] = sinv[t * dim + i + half] = std::sin(angle);
        }
}

// ops::rope on one tensor [B,H,L,D] (contiguous): example/qwen3/src/qwen3.cpp:522-559.
// Position li reads table row li (the caller passes tables sliced to the
// positions). x1' = x1*c - x2*s ; x2' = x2*c + x1*s over halves [0,D/2), [D/2,D).
OEXPORT void oracle_rope(float* x, int B, int H, int L, int D, const float* cosv, const float* sinv) {
    const int half = D / 2;
    for (int64_t bhl = 0; bhl < static_cast<int64_t>(B) * H * L; ++bhl) {
        const int li = static_cast<int>(bhl % L);
        float* r = x + bhl * D;
        for (int d = 0; d < half; ++d) {
            const float c = cosv[li * D + d], s = sinv[li * D + d];
            const float x1 = r[d], x2 = r[d + half];
            r[d] = std::fma(x1, c, -(x2 * s));
            r[d + half] = std::fma(x2, c, x1 * s);
        }
    }
}

// ---------------------------------------------------------------------------
// Masked matmul and the MATH SDPA backend.
// ---------------------------------------------------------------------------

// sgemm_masked with a bool mask [m, n] (src/kernel/avx2/sgemm.inl:342-447): where
// the mask is set, C = alpha * (A.B) + beta * C; elsewhere C is left as it was.
// k == 0 or alpha == 0 only scales (beta == 0 writes 0) the visible entries
// (351-363). The visible products are those of sgemm (one FMA chain per
// element over each k block, as its full tiles compute them); the blend is
// alpha * dot + beta * c. Positions where the mask is clear are never read.
OEXPORT void oracle_sgemm_masked(const float* A, const float* B, float* C, int m, int n, int k, float alpha,
                                 float beta, int64_t rsa, int64_t csa, int64_t rsb, int64_t csb, int64_t rsc,
                                 int64_t csc, const uint8_t* mask) {
    if (m == 0 || n == 0) return;
    if (k == 0 || alpha == 0.0f) {
        for (int i = 0; i < m; ++i)
            for (int j = 0; j < n; ++j)
                if (mask[static_cast<size_t>(i) * n + j]) {
                    float& c = C[i * rsc + j * csc];
                    if (beta == 0.0f) c = 0.0f;
                    else if (beta != 1.0f) c *= beta;
                }
        return;
    }
    std::vector<float> prod(static_cast<size_t>(m) * n);
    sgemm_full(A, B, prod.data(), m, n, k, 1.0f, 0.0f, rsa, csa, rsb, csb, n, 1);
    for (int i = 0; i < m; ++i)
        for (int j = 0; j < n; ++j)
            if (mask[static_cast<size_t>(i) * n + j]) {
                float& c = C[i * rsc + j * csc];
                const float p = prod[static_cast<size_t>(i) * n + j];
                if (alpha == 1.0f && beta == 0.0f) c = p;
                else c = alpha * p + beta * c;
            }
}

// scaledDotProductAttention, MATH backend (src/function/ops.inl:388-418 and,
// for a predicate, 474-490), one [Lq, D] x [Lkv, D] x [Lkv, Dv] problem per
// head h of H contiguous heads:
//   score = masked_matmul(q, k^T, mask, -1e9)   (plain matmul without a mask)
//   score *= scale; score += bias
//   softmax_(score, -1): max, exp(x - max), running sum, x /= sum
//     (src/function/activation.inl:313-329)
//   out = matmul(score, v); rows whose mask has no visible key -> 0 (18-40)
// mask: bool bytes [Lq, Lkv] or NULL; diag != 0 uses the predicate
// j <= i + diag_off instead. bias [Lq, Lkv] or NULL. scale 0 -> 1/sqrt(D).
OEXPORT void oracle_sdpa_math(const float* Q, const float* K, const float* V, float* O, int H, int Lq, int Lkv,
                              int D, int Dv, float scale, const uint8_t* mask, const float* bias, int diag,
                              int diag_off) {
    if (scale == 0.0f) scale = 1.0f / std::sqrt(static_cast<float>(D));
    const bool masked = diag != 0 || mask != nullptr;
    auto visible = [&](int i, int j) -> bool {
        if (diag) return j <= i + diag_off;
        return mask == nullptr || mask[static_cast<size_t>(i) * Lkv + j] != 0;
    };
    std::vector<float> s(static_cast<size_t>(Lq) * Lkv);
    for (int h = 0; h < H; ++h) {
        const float* q = Q + static_cast<size_t>(h) * Lq * D;
        const float* k = K + static_cast<size_t>(h) * Lkv * D;
        const float* v = V + static_cast<size_t>(h) * Lkv * Dv;
        float* o = O + static_cast<size_t>(h) * Lq * Dv;
        // k^T is the view (p, j) -> k[j * D + p]: rsb = 1, csb = D
        sgemm_full(q, k, s.data(), Lq, Lkv, D, 1.0f, 0.0f, D, 1, 1, D, Lkv, 1);
        for (int i = 0; i < Lq; ++i) {
            float* row = s.data() + static_cast<size_t>(i) * Lkv;
            for (int j = 0; j < Lkv; ++j) {
                if (!visible(i, j)) row[j] = -1e9f;
                row[j] *= scale;
                if (bias) row[j] += bias[static_cast<size_t>(i) * Lkv + j];
            }
            float mx = std::numeric_limits<float>::lowest();
            for (int j = 0; j < Lkv; ++j) mx = std::max(mx, row[j]);
            float sum = 0.0f;
            for (int j = 0; j < Lkv; ++j) {
                row[j] = std::exp(row[j] - mx);
                sum += row[j];
            }
            for (int j = 0; j < Lkv; ++j) row[j] /= sum;
        }
        sgemm_full(s.data(), v, o, Lq, Dv, Lkv, 1.0f, 0.0f, Lkv, 1, Dv, 1, Dv, 1);
        if (masked)
            for (int i = 0; i < Lq; ++i) {
                bool any = false;
                for (int j = 0; j < Lkv && !any; ++j) any = visible(i, j);
                if (!any)
                    for (int d = 0; d < Dv; ++d) o[static_cast<size_t>(i) * Dv + d] = 0.0f;
            }
    }
}

OEXPORT int oracle_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
OEXPORT void oracle_set_num_threads(int t) {
#ifdef _OPENMP
    if (t > 0) omp_set_num_threads(t);
#else
    (void)t;
#endif
}

// ===========================================================================
// Qwen3 decoder (example/qwen3/src/qwen3.cpp:193-516), fp32, batch 1, greedy.
// Composition of the functions above exactly as the example composes
// yt::function::linear / rmsNorm_ / scaledDotProductAttention(FLASH_AVX2) /
// swish_ and the example's rope, KV cache and chat_only last layer.
//
// Weight buffer layout (fp32, in the configs' fill order): embed [V,H]; per
// layer: q [nh*hd,H], k [nkv*hd,H], v [nkv*hd,H] (= the fused qkv_proj,
// qwen3.cpp:326-338), o [H,nh*hd], q_norm [hd], k_norm [hd], gate [I,H],
// up [I,H] (= gate_up, 339-349), down [H,I], norm1 [H], norm2 [H]; final norm [H].
// ===========================================================================
namespace {

struct Q3Cfg { int H, L, V, I, nh, nkv, hd, max_pos; float eps, theta; };

struct Q3Layer {
    const float *qkv, *o, *qn, *kn, *gu, *down, *n1, *n2;
};

struct Q3Cache {  // KVCache (qwen3.cpp:57-126), batch 1
    std::vector<float> k, v;  // [nkv][max_len][hd]
    int cur_len = 0, write_pos = 0, total = 0, max_len = 0, nkv = 0, hd = 0;
    void init(int ml, int kvh, int d) {
        max_len = ml; nkv = kvh; hd = d;
        k.assign(static_cast<size_t>(kvh) * ml * d, 0.0f);
        v.assign(static_cast<size_t>(kvh) * ml * d, 0.0f);
    }
    // new_k/new_v: [nkv][l][hd]
    void append(const float* nk, const float* nv, int l) {
        for (int t = 0; t < l; ++t) {
            for (int h = 0; h < nkv; ++h) {
                std::memcpy(&k[(static_cast<size_t>(h) * max_len + write_pos) * hd], nk + (static_cast<size_t>(h) * l + t) * hd, hd * 4);
                std::memcpy(&v[(static_cast<size_t>(h) * max_len + write_pos) * hd], nv + (static_cast<size_t>(h) * l + t) * hd, hd * 4);
            }
            write_pos = (write_pos + 1) % max_len;
            total++;
            if (cur_len < max_len) cur_len++;
        }
    }
    // get_mask (104-126): [q_len, cur_len]
    std::vector<uint8_t> mask(int q_len) const {
        const int kv_len = cur_len;
        std::vector<uint8_t> m(static_cast<size_t>(q_len) * kv_len);
        const int start = kv_len - q_len;
        const bool full = cur_len >= max_len;
        for (int qi = 0; qi < q_len; ++qi)
            for (int ki = 0; ki < kv_len; ++ki) {
                bool vis;
                if (!full) vis = ki <= start + qi;
                else vis = ((ki - write_pos + max_len) % max_len) <= start + qi;
                m[static_cast<size_t>(qi) * kv_len + ki] = vis ? 1 : 0;
            }
        return m;
    }
};

struct Q3Model {
    Q3Cfg c;
    const float* embed;
    const float* fnorm;
    std::vector<Q3Layer> layers;
    std::vector<Q3Cache> caches;
    std::vector<float> cosv, sinv;

    // yt::function::linear: x [l, in] . W[out, in]^T
    static void linear(const float* x, const float* W, float* y, int l, int in, int out) {
        sgemm_full(x, W, y, l, out, in, 1.0f, 0.0f, in, 1, 1, in, out, 1);
    }
    void rms(float* x, const float* w, int rows, int n) const { oracle_rms_norm(x, w, rows, n, c.eps); }

    // ops::rope / rope_k on [heads][l][hd] with table rows [start, start+l)
    void rope(float* x, int heads, int l, int start) const {
        oracle_rope(x, 1, heads, l, c.hd, &cosv[static_cast<size_t>(start) * c.hd], &sinv[static_cast<size_t>(start) * c.hd]);
    }

    // qkv projection + per-head norms + RoPE, then cache append (the parts of
    // Qwen3Attention::forward / prefill_kv_only, qwen3.cpp:203-247).
    void qkv_rope_append(const Q3Layer& W, Q3Cache& cache, const float* h, int l, int start, std::vector<float>* q_out) {
        const int qs = c.nh * c.hd, ks = c.nkv * c.hd, tot = qs + 2 * ks;
        std::vector<float> qkv(static_cast<size_t>(l) * tot);
        linear(h, W.qkv, qkv.data(), l, c.H, tot);
        std::vector<float> k(static_cast<size_t>(c.nkv) * l * c.hd), v(k.size());
        for (int t = 0; t < l; ++t)
            for (int hh = 0; hh < c.nkv; ++hh)
                for (int d = 0; d < c.hd; ++d) {
                    k[(static_cast<size_t>(hh) * l + t) * c.hd + d] = qkv[static_cast<size_t>(t) * tot + qs + hh * c.hd + d];
                    v[(static_cast<size_t>(hh) * l + t) * c.hd + d] = qkv[static_cast<size_t>(t) * tot + qs + ks + hh * c.hd + d];
                }
        if (q_out) {
            q_out->assign(static_cast<size_t>(c.nh) * l * c.hd, 0.0f);
            for (int t = 0; t < l; ++t)
                for (int hh = 0; hh < c.nh; ++hh)
                    std::memcpy(&(*q_out)[(static_cast<size_t>(hh) * l + t) * c.hd], &qkv[static_cast<size_t>(t) * tot + hh * c.hd], c.hd * 4);
            rms(q_out->data(), W.qn, c.nh * l, c.hd);
        }
        rms(k.data(), W.kn, c.nkv * l, c.hd);
        if (q_out) rope(q_out->data(), c.nh, l, start);
        rope(k.data(), c.nkv, l, start);
        cache.append(k.data(), v.data(), l);
    }

    // Qwen3Attention::forward (224-269): returns o_proj output [l, H]
    std::vector<float> attention(const Q3Layer& W, Q3Cache& cache, const float* h, int l, int start) {
        std::vector<float> q;
        qkv_rope_append(W, cache, h, l, start, &q);
        const int kv_len = cache.cur_len, G = c.nh / c.nkv;
        std::vector<uint8_t> m = cache.mask(l);
        std::vector<float> att(static_cast<size_t>(l) * c.nh * c.hd);
        const float scale = 1.0f / std::sqrt(static_cast<float>(c.hd));
#pragma omp parallel for schedule(dynamic, 1)
        for (int hh = 0; hh < c.nh; ++hh) {
            const int kh = hh / G;
            std::vector<float> o(static_cast<size_t>(l) * c.hd);
            oracle_flash_attention(&q[static_cast<size_t>(hh) * l * c.hd], &cache.k[static_cast<size_t>(kh) * cache.max_len * c.hd],
                                   &cache.v[static_cast<size_t>(kh) * cache.max_len * c.hd], o.data(), l, kv_len, c.hd, c.hd,
                                   scale, c.hd, 1, c.hd, 1, c.hd, 1, c.hd, 1, m.data(), kv_len, nullptr, 0, 0);
            for (int t = 0; t < l; ++t)
                std::memcpy(&att[(static_cast<size_t>(t) * c.nh + hh) * c.hd], &o[static_cast<size_t>(t) * c.hd], c.hd * 4);
        }
        std::vector<float> out(static_cast<size_t>(l) * c.H);
        linear(att.data(), W.o, out.data(), l, c.nh * c.hd, c.H);
        return out;
    }

    // Qwen3MLP::forward (193-200) with swish_ (activation.inl:631-647,
    // _stableSigmoid ytensor_function.inl:43-52)
    std::vector<float> mlp(const Q3Layer& W, const float* h, int l) const {
        std::vector<float> gu(static_cast<size_t>(l) * 2 * c.I);
        linear(h, W.gu, gu.data(), l, c.H, 2 * c.I);
        std::vector<float> act(static_cast<size_t>(l) * c.I);
        for (int t = 0; t < l; ++t)
            for (int j = 0; j < c.I; ++j) {
                const float a = gu[static_cast<size_t>(t) * 2 * c.I + j];
                float sig;
                if (a >= 0.0f) { const float z = std::exp(-a); sig = 1.0f / (1.0f + z); }
                else { const float z = std::exp(a); sig = z / (1.0f + z); }
                act[static_cast<size_t>(t) * c.I + j] = (a * sig) * gu[static_cast<size_t>(t) * 2 * c.I + c.I + j];
            }
        std::vector<float> out(static_cast<size_t>(l) * c.H);
        linear(act.data(), W.down, out.data(), l, c.I, c.H);
        return out;
    }

    // Qwen3DecoderLayer::forward (271-283), in place on x [l, H]
    void layer(int i, std::vector<float>& x, int l, int start) {
        const Q3Layer& W = layers[i];
        std::vector<float> h1(x);
        rms(h1.data(), W.n1, l, c.H);
        std::vector<float> x2 = attention(W, caches[i], h1.data(), l, start);
        for (size_t e = 0; e < x2.size(); ++e) x2[e] += x[e];
        std::vector<float> h2(x2);
        rms(h2.data(), W.n2, l, c.H);
        std::vector<float> mo = mlp(W, h2.data(), l);
        for (size_t e = 0; e < x2.size(); ++e) x2[e] += mo[e];
        x.swap(x2);
    }

    // Qwen3Model::forward (365-413) + Qwen3ForCausalLM::forward (449-457): logits of the last token
    std::vector<float> forward(const int* ids, int l, bool chat_only) {
        int start = caches[0].cur_len > 0 ? caches[0].total : 0;
        if (start + l > c.max_pos) {
            start = caches[0].cur_len;
            if (start + l > c.max_pos) start = 0;
        }
        std::vector<float> x(static_cast<size_t>(l) * c.H);
        for (int t = 0; t < l; ++t) std::memcpy(&x[static_cast<size_t>(t) * c.H], embed + static_cast<size_t>(ids[t]) * c.H, c.H * 4);
        std::vector<float> last(c.H);
        bool done = false;
        for (int i = 0; i < c.L; ++i) {
            if (chat_only && l > 1 && i == c.L - 1) {
                const Q3Layer& W = layers[i];
                std::vector<float> h1(x);
                rms(h1.data(), W.n1, l, c.H);
                qkv_rope_append(W, caches[i], h1.data(), l - 1, start, nullptr);  // prefill_kv_only
                std::vector<float> x2 = attention(W, caches[i], &h1[static_cast<size_t>(l - 1) * c.H], 1, start + l - 1);
                for (int e = 0; e < c.H; ++e) x2[e] += x[static_cast<size_t>(l - 1) * c.H + e];
                std::vector<float> h2(x2);
                rms(h2.data(), W.n2, 1, c.H);
                std::vector<float> mo = mlp(W, h2.data(), 1);
                for (int e = 0; e < c.H; ++e) x2[e] += mo[e];
                rms(x2.data(), fnorm, 1, c.H);
                last = x2;
                done = true;
                break;
            }
            layer(i, x, l, start);
        }
        if (!done) {
            rms(x.data(), fnorm, l, c.H);
            std::memcpy(last.data(), &x[static_cast<size_t>(l - 1) * c.H], c.H * 4);
        }
        // last.matmul(embed^T): a 1 x V GEMV with B = embed^T (col-major view)
        std::vector<float> logits(c.V);
        sgemm_full(last.data(), embed, logits.data(), 1, c.V, c.H, 1.0f, 0.0f, c.H, 1, 1, c.H, c.V, 1);
        return logits;
    }
};

}  // namespace

// cfg_i: H, L, V, I, nh, nkv, hd, max_pos ; cfg_f: eps, theta
// Greedy multi-turn generation over one set of KV caches, as repeated calls of
// Qwen3ForCausalLM::generate (506-516) do (the caches persist between calls;
// argmax replaces the example's top-20 sampling): turn t runs its prompt
// forward with chat_only = true, then steps[t] - 1 single-token steps; the
// caches wrap as KVCache::append / get_mask do (57-126) once more than max_pos
// tokens were written. out_tokens / out_margins (top1 - top2 logit) get one
// entry per step of all turns in order; logits [n_logit_steps][V] (optional)
// receives the logits of the global step indices listed in logit_steps.
OEXPORT int oracle_qwen3_run(const int* cfg_i, const float* cfg_f, const float* W, int n_turns,
                             const int* prompt_lens, const int* prompts, const int* steps, int* out_tokens,
                             float* out_margins, const int* logit_steps, int n_logit_steps, float* logits) {
    Q3Model m;
    m.c = {cfg_i[0], cfg_i[1], cfg_i[2], cfg_i[3], cfg_i[4], cfg_i[5], cfg_i[6], cfg_i[7], cfg_f[0], cfg_f[1]};
    const Q3Cfg& c = m.c;
    for (int t = 0; t < n_turns; ++t)
        if (prompt_lens[t] <= 0 || prompt_lens[t] > c.max_pos || steps[t] <= 0) return -1;
    const float* p = W;
    m.embed = p;
    p += static_cast<size_t>(c.V) * c.H;
    const size_t qkv_rows = static_cast<size_t>(c.nh + 2 * c.nkv) * c.hd;
    for (int i = 0; i < c.L; ++i) {
        Q3Layer L{};
        L.qkv = p; p += qkv_rows * c.H;
        L.o = p; p += static_cast<size_t>(c.H) * c.nh * c.hd;
        L.qn = p; p += c.hd;
        L.kn = p; p += c.hd;
        L.gu = p; p += static_cast<size_t>(2) * c.I * c.H;
        L.down = p; p += static_cast<size_t>(c.H) * c.I;
        L.n1 = p; p += c.H;
        L.n2 = p; p += c.H;
        m.layers.push_back(L);
    }
    m.fnorm = p;
    m.caches.resize(c.L);
    for (auto& ch : m.caches) ch.init(c.max_pos, c.nkv, c.hd);
    m.cosv.resize(static_cast<size_t>(c.max_pos) * c.hd);
    m.sinv.resize(m.cosv.size());
    oracle_rope_precompute(c.hd, c.max_pos, c.theta, m.cosv.data(), m.sinv.data());
    int g = 0;  // global step index
    const int* pr = prompts;
    for (int t = 0; t < n_turns; ++t) {
        std::vector<int> ids(pr, pr + prompt_lens[t]);
        pr += prompt_lens[t];
        for (int step = 0; step < steps[t]; ++step, ++g) {
            std::vector<float> lg = m.forward(ids.data(), static_cast<int>(ids.size()), step == 0);
            for (int q = 0; q < n_logit_steps; ++q)
                if (logits && logit_steps[q] == g) std::memcpy(logits + static_cast<size_t>(q) * c.V, lg.data(), sizeof(float) * c.V);
            int best = 0;
            for (int j = 1; j < c.V; ++j) if (lg[j] > lg[best]) best = j;
            float second = -std::numeric_limits<float>::infinity();
            for (int j = 0; j < c.V; ++j) if (j != best && lg[j] > second) second = lg[j];
            out_tokens[g] = best;
            out_margins[g] = lg[best] - second;
            ids.assign(1, best);
        }
    }
    return 0;
}

// Single turn of oracle_qwen3_run with the first step's logits (logits0, optional [V]).
OEXPORT int oracle_qwen3_generate(const int* cfg_i, const float* cfg_f, const float* W, const int* prompt,
                                  int prompt_len, int n_steps, int* out_tokens, float* out_margins,
                                  float* logits0) {
    const int zero = 0;
    return oracle_qwen3_run(cfg_i, cfg_f, W, 1, &prompt_len, prompt, &n_steps, out_tokens, out_margins, &zero,
                            logits0 ? 1 : 0, logits0);
}
