// gemm.hip — MFMA GEMM for gfx950 (CDNA4), the device replacement of YTensor's
// blocked AVX2 sgemm / hgemm (src/kernel/avx2/sgemm.inl:268-340, 586-787;
// src/kernel/avx2/hgemm.inl:139-273).
//
// Design (MI355X-first, not a translation of the CPU Goto loop):
//  * Block tile BM x BN, k step of 128 bytes per row (64 bf16/fp16 or 32 fp32).
//    Both operands live in LDS K-contiguous, [rows][8 chunks of 16 B], so an
//    MFMA operand fragment is one ds_read_b128 per lane. A row-major B ("NN",
//    B[k][n]) stays [k][n] in LDS and its fragments are read with the gfx950
//    transposing read ds_read_b64_tr_b16, so nothing is transposed in registers.
//  * Tiles move global -> LDS by direct-to-LDS DMA (global_load_lds_dwordx4):
//    no VGPR staging. Two stages for the 256 x 256 tile (one k step in flight),
//    a 4-deep ring for the smaller tiles. The bytes each CU can pull through its
//    vector-memory path (~28 B/clk) are close to what 256 x 256 MFMA work
//    consumes, so the 256 x 256 tile is the only one that keeps up at 4096^3.
//  * LDS swizzles were chosen by measuring gfx950's LDS read rate per pattern
//    (see swz_dma / nn_blk): fragment reads are bank-conflict free.
//  * Inside a k step the A fragments stream through a 3-register ring read two
//    MFMA groups ahead, pinned by schedule barriers, so LDS latency overlaps
//    the matrix cores.
//  * MFMA operands are swapped (src0 = B rows, src1 = A rows): each lane then
//    holds 4 consecutive output columns of one row, stored as one vector.
//  * Tiles are assigned XCD-aware: the hardware places workgroup w on XCD
//    w % 8; each XCD receives a contiguous, M-grouped range of tiles so its
//    32 CUs share A and B panels in their own L2.
//  * The register-staged kernel (gemm_mfma_kernel) serves layouts the DMA path
//    cannot take (k not a multiple of the k step, 4-byte-aligned NN rows).

#include "common.hpp"
#include "launch.hpp"

namespace ythip {

struct GemmArgs {
    const void* A;
    const void* B;
    void* C;
    int m, n, k;
    int64_t rsa, rsb, csb, rsc;  // csa == 1 and csc == 1 on this path
    int64_t sa_b, sb_b, sc_b;
    float alpha, beta;
    int tiles_m, tiles_n;
    int c_vec_ok;   // C rows allow 4-element vector stores
    int c_line_ok;  // 16-bit C: 16-byte aligned base and rows (the ping-pong kernel's line stores)
};

__device__ __forceinline__ int swz(int row, int chunk) { return chunk ^ ((row ^ (row >> 3)) & 7); }

// Swizzles of the DMA-staged kernel, chosen by measuring gfx950's LDS read rate
// per access pattern (64 banks; ds_read_b128 and ds_read_b64_tr_b16):
//  * K-major tiles [row][8 x 16 B]: chunk c of row r at c ^ ((r >> 1) & 7). Rows
//    r and r+1 share one 256-byte bank window and take the same XOR, so a
//    fragment read (16 rows, one logical chunk) covers all 64 banks without
//    conflict; the previous row-XOR swizzle ran at ~60% of that rate.
//  * NN B tiles [k][n] in 32-byte column blocks: block b of k-row r at
//    b ^ h(r), h(r) = (r ^ ((r >> 3) << 2)) & mask, so the transposing reads of
//    k-rows r and r + 8 (served together) land in different blocks.
__device__ __forceinline__ int swz_dma(int row, int chunk) { return chunk ^ ((row >> 1) & 7); }
__device__ __forceinline__ int nn_blk(int row, int blk, int mask) { return blk ^ ((row ^ ((row >> 3) << 2)) & mask); }

template <class T, class TO, int BM, int BN, int WM, int WN, bool NN>
__global__ __launch_bounds__(64 * WM * WN) void gemm_mfma_kernel(GemmArgs a) {
    using raw = typename T::raw;
    constexpr int THREADS = 64 * WM * WN;
    constexpr int VEC = 16 / sizeof(raw);      // elements per 16-byte chunk
    constexpr int BK = 8 * VEC;                 // elements per k step (128 bytes)
    constexpr int WTM = BM / WM, WTN = BN / WN; // wave tile
    constexpr int FM = WTM / 16, FN = WTN / 16;
    constexpr int A_CHUNKS = BM * 8, B_CHUNKS = BN * 8;
    constexpr int A_PT = (A_CHUNKS + THREADS - 1) / THREADS;
    constexpr int B_PT = (B_CHUNKS + THREADS - 1) / THREADS;
    constexpr int NN_GROUPS = 8 * (BN / 4);     // VEC k-rows x 4 columns each
    constexpr int NN_PT = (NN_GROUPS + THREADS - 1) / THREADS;
    constexpr int STAGE = (BM + BN) * 8;        // u32x4 slots per stage

    __shared__ u32x4 lds[2 * STAGE];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;

    int tm, tn;
    tile_coords(blockIdx.x, a.tiles_m, a.tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int bz = blockIdx.y;

    const raw* __restrict__ Ap = static_cast<const raw*>(a.A) + bz * a.sa_b;
    const raw* __restrict__ Bp = static_cast<const raw*>(a.B) + bz * a.sb_b;

    const int KT = (a.k + BK - 1) / BK;

    u32x4 ra[A_PT];
    u32x4 rb[NN ? 1 : B_PT];
    // NN staging: VEC rows of 4 columns each (8 bytes for 16-bit, 16 bytes for fp32)
    using nn_row_t = typename std::conditional<sizeof(raw) == 2, u32x2, u32x4>::type;
    nn_row_t rn[NN ? NN_PT : 1][NN ? VEC : 1];

    auto load_global = [&](int kt) {
        const int k0 = kt * BK;
#pragma unroll
        for (int i = 0; i < A_PT; ++i) {
            const int id = tid + i * THREADS;
            const int r = id >> 3, c = id & 7;
            u32x4 v = {0u, 0u, 0u, 0u};
            if ((A_CHUNKS % THREADS == 0 || id < A_CHUNKS) && m0 + r < a.m && k0 + c * VEC < a.k)
                v = *reinterpret_cast<const u32x4*>(Ap + (int64_t)(m0 + r) * a.rsa + (k0 + c * VEC));
            ra[i] = v;
        }
        if constexpr (!NN) {
#pragma unroll
            for (int i = 0; i < B_PT; ++i) {
                const int id = tid + i * THREADS;
                const int r = id >> 3, c = id & 7;
                u32x4 v = {0u, 0u, 0u, 0u};
                if ((B_CHUNKS % THREADS == 0 || id < B_CHUNKS) && n0 + r < a.n && k0 + c * VEC < a.k)
                    v = *reinterpret_cast<const u32x4*>(Bp + (int64_t)(n0 + r) * a.csb + (k0 + c * VEC));
                rb[i] = v;
            }
        } else {
#pragma unroll
            for (int i = 0; i < NN_PT; ++i) {
                const int id = tid + i * THREADS;
                const int g = id % (BN / 4), kc = id / (BN / 4);
                const int col = n0 + g * 4;
                const bool ok = (NN_GROUPS % THREADS == 0 || id < NN_GROUPS) && col < a.n;
#pragma unroll
                for (int r = 0; r < VEC; ++r) {
                    const int kk = k0 + kc * VEC + r;
                    nn_row_t v = {};
                    if (ok && kk < a.k) v = *reinterpret_cast<const nn_row_t*>(Bp + (int64_t)kk * a.rsb + col);
                    rn[i][r] = v;
                }
            }
        }
    };

    auto store_lds = [&](int stage) {
        u32x4* sA = lds + stage * STAGE;
        u32x4* sB = sA + BM * 8;
#pragma unroll
        for (int i = 0; i < A_PT; ++i) {
            const int id = tid + i * THREADS;
            if (A_CHUNKS % THREADS == 0 || id < A_CHUNKS) {
                const int r = id >> 3, c = id & 7;
                sA[r * 8 + swz(r, c)] = ra[i];
            }
        }
        if constexpr (!NN) {
#pragma unroll
            for (int i = 0; i < B_PT; ++i) {
                const int id = tid + i * THREADS;
                if (B_CHUNKS % THREADS == 0 || id < B_CHUNKS) {
                    const int r = id >> 3, c = id & 7;
                    sB[r * 8 + swz(r, c)] = rb[i];
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < NN_PT; ++i) {
                const int id = tid + i * THREADS;
                if (NN_GROUPS % THREADS == 0 || id < NN_GROUPS) {
                    const int g = id % (BN / 4), kc = id / (BN / 4);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        u32x4 o;
                        if constexpr (sizeof(raw) == 2) {
                            // out[j] = column j's VEC k-values: half-word j of each row, paired.
#pragma unroll
                            for (int q = 0; q < 4; ++q) {
                                const uint32_t lo = rn[i][2 * q][j >> 1];
                                const uint32_t hi = rn[i][2 * q + 1][j >> 1];
                                o[q] = (j & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
                            }
                        } else {
#pragma unroll
                            for (int q = 0; q < 4; ++q) o[q] = rn[i][q][j];
                        }
                        const int row = g * 4 + j;
                        sB[row * 8 + swz(row, kc)] = o;
                    }
                }
            }
        }
    };

    f32x4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    load_global(0);
    store_lds(0);
    __syncthreads();

    const int lrow = lane & 15;
    const int lgrp = lane >> 4;

    for (int kt = 0; kt < KT; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < KT) load_global(kt + 1);
        const u32x4* sA = lds + cur * STAGE;
        const u32x4* sB = sA + BM * 8;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const int chunk = ks * 4 + lgrp;
            u32x4 fa[FM], fb[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                const int r = wm * WTM + i * 16 + lrow;
                fa[i] = sA[r * 8 + swz(r, chunk)];
            }
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const int r = wn * WTN + j * 16 + lrow;
                fb[j] = sB[r * 8 + swz(r, chunk)];
            }
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j) acc[i][j] = mfma_chunk(T{}, fb[j], fa[i], acc[i][j]);
        }
        if (kt + 1 < KT) store_lds(cur ^ 1);
        __syncthreads();
    }

    // Epilogue: lane holds C[m][n..n+3] for m = row lrow, n = 4*lgrp + r.
    using oraw = typename TO::raw;
    oraw* Cp = static_cast<oraw*>(a.C) + bz * a.sc_b;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
        const int m = m0 + wm * WTM + i * 16 + lrow;
        if (m >= a.m) continue;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int n = n0 + wn * WTN + j * 16 + lgrp * 4;
            if (n >= a.n) continue;
            oraw* crow = Cp + (int64_t)m * a.rsc;
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) v[r] = a.alpha * acc[i][j][r];
            const bool full = a.c_vec_ok && (n + 3 < a.n);
            if (a.beta != 0.0f) {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (n + r < a.n) v[r] += a.beta * load_as_f32<TO>(crow, n + r);
            }
            if (full) {
                if constexpr (sizeof(oraw) == 2) {
                    u32x2 p = {pack2<TO>(v[0], v[1]), pack2<TO>(v[2], v[3])};
                    *reinterpret_cast<u32x2*>(crow + n) = p;
                } else {
                    *reinterpret_cast<f32x4*>(crow + n) = f32x4{v[0], v[1], v[2], v[3]};
                }
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (n + r < a.n) store_from_f32<TO>(crow, n + r, v[r]);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// DMA-staged variant (the fast path). Tiles go global -> LDS with
// global_load_lds (16 bytes per lane, no VGPR staging); the XOR swizzle is
// applied on the global-address side because the DMA writes 64 consecutive
// 16-byte LDS slots per wave. While the matrix cores work on one LDS stage the
// DMA fills the other; fragments for the second 32-wide k step are read from
// LDS before the first step's MFMAs, and a scheduling pattern interleaves the
// LDS reads with the MFMAs.
//   NN (B row-major [k][n], 16-bit): the B tile stays [k][n] in LDS (rows of
//   BN elements, 32-byte blocks XOR-swizzled by row) and is read with
//   ds_read_b64_tr_b16: within each 16-lane group, lane j addresses the 4
//   columns 4*(j%4).. of k-row j/4 and lane i receives column i of those 4
//   k-rows -- exactly the MFMA B operand (two reads per 16x32 fragment).
// Requirements (checked on the host): k % BK == 0, 16-byte aligned rows, and
// for NN: n % 16 == 0. Rows past M / N are clamped (their outputs are never
// stored); K has no tail.
// ---------------------------------------------------------------------------

// SOFF: every operand spans less than 2^31 bytes (checked on the host): the DMA
// then goes from a wave-uniform base, moved by scalar adds per k step, plus a
// per-lane 32-bit byte offset fixed for the whole k loop (dma16_soff), and the
// LDS destination is the wave's base plus constants -- no VALU address work
// between the MFMAs of consecutive k steps.
template <class T, class TO, int BM, int BN, int WM, int WN, bool NN, int STAGES, bool SOFF>
__global__ __launch_bounds__(64 * WM * WN) void gemm_mfma_dma_kernel(GemmArgs a) {
    using raw = typename T::raw;
    constexpr int THREADS = 64 * WM * WN;
    constexpr int VEC = 16 / sizeof(raw);
    constexpr int BK = 8 * VEC;
    constexpr int WTM = BM / WM, WTN = BN / WN;
    constexpr int FM = WTM / 16, FN = WTN / 16;
    constexpr int A_PT = BM * 8 / THREADS, B_PT = BN * 8 / THREADS;
    static_assert(A_PT * THREADS == BM * 8 && B_PT * THREADS == BN * 8, "tile/thread mismatch");
    static_assert(!NN || sizeof(raw) == 2, "the transposing LDS read is 16-bit");
    constexpr int STA = BM * 8, STB = BN * 8;             // 16-byte slots per stage
    constexpr int NBLK = BN / 16;                          // NN: 32-byte blocks per k-row
    constexpr int BLK_MASK = (NBLK < 8 ? NBLK : 8) - 1;
    constexpr int MF_PER_CHUNK = sizeof(raw) == 2 ? 1 : 4;

    constexpr int PER = A_PT + B_PT;  // DMA instructions per thread per stage
    static_assert(STAGES >= 2 && STAGES <= 4 && (STAGES - 2) * PER < 64, "pipeline depth");

    __shared__ u32x4 sbuf[STAGES * (STA + STB)];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int lrow = lane & 15, lgrp = lane >> 4;

    int tm, tn;
    tile_coords(blockIdx.x, a.tiles_m, a.tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int bz = blockIdx.y;
    const raw* __restrict__ Ap = static_cast<const raw*>(a.A) + bz * a.sa_b;
    const raw* __restrict__ Bp = static_cast<const raw*>(a.B) + bz * a.sb_b;
    const int KT = a.k / BK;

    auto issue_a = [&](int kt, u32x4* sA) {
        const int k0 = kt * BK;
#pragma unroll
        for (int i = 0; i < A_PT; ++i) {
            const int slot = i * THREADS + wave * 64 + lane;
            const int r = slot >> 3;
            const int c = swz_dma(r, slot & 7);  // the swizzle is an involution on the chunk index
            const int row = min(m0 + r, a.m - 1);
            dma16_async(Ap + (int64_t)row * a.rsa + k0 + c * VEC, &sA[i * THREADS + wave * 64]);
        }
    };
    auto issue_b = [&](int kt, u32x4* sB) {
        const int k0 = kt * BK;
#pragma unroll
        for (int i = 0; i < B_PT; ++i) {
            const int slot = i * THREADS + wave * 64 + lane;
            const raw* g;
            if constexpr (!NN) {
                const int r = slot >> 3;
                const int c = swz_dma(r, slot & 7);
                const int row = min(n0 + r, a.n - 1);
                g = Bp + (int64_t)row * a.csb + k0 + c * VEC;
            } else {
                const int r = slot / (2 * NBLK), ps = slot % (2 * NBLK);
                const int lb = nn_blk(r, ps >> 1, BLK_MASK);
                g = Bp + (int64_t)(k0 + r) * a.rsb + min(n0 + lb * 16, a.n - 16) + (ps & 1) * 8;
            }
            dma16_async(g, &sB[i * THREADS + wave * 64]);
        }
    };
    // SOFF: per-lane byte offsets of the stage-0 loads (the k loop moves the base)
    uint32_t offA[SOFF ? A_PT : 1], offB[SOFF ? B_PT : 1];
    uint32_t ldsA0 = 0, ldsB0 = 0;
    if constexpr (SOFF) {
#pragma unroll
        for (int i = 0; i < A_PT; ++i) {
            const int slot = i * THREADS + wave * 64 + lane;
            const int r = slot >> 3;
            const int c = swz_dma(r, slot & 7);
            const int row = min(m0 + r, a.m - 1);
            offA[i] = (uint32_t)(((int64_t)row * a.rsa + c * VEC) * (int64_t)sizeof(raw));
        }
#pragma unroll
        for (int i = 0; i < B_PT; ++i) {
            const int slot = i * THREADS + wave * 64 + lane;
            int64_t e;
            if constexpr (!NN) {
                const int r = slot >> 3;
                const int c = swz_dma(r, slot & 7);
                e = (int64_t)min(n0 + r, a.n - 1) * a.csb + c * VEC;
            } else {
                const int r = slot / (2 * NBLK), ps = slot % (2 * NBLK);
                const int lb = nn_blk(r, ps >> 1, BLK_MASK);
                e = (int64_t)r * a.rsb + min(n0 + lb * 16, a.n - 16) + (ps & 1) * 8;
            }
            offB[i] = (uint32_t)(e * (int64_t)sizeof(raw));
        }
        ldsA0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)&sbuf[wave * 64]);
        ldsB0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)&sbuf[STAGES * STA + wave * 64]);
    }
    // DMA of k step kt into stage st
    auto issue_st = [&](int kt, int st) {
        if constexpr (SOFF) {
            const char* bA = reinterpret_cast<const char*>(Ap) + (int64_t)kt * BK * (int64_t)sizeof(raw);
            const char* bB = reinterpret_cast<const char*>(Bp) +
                             (int64_t)kt * BK * (NN ? a.rsb : (int64_t)1) * (int64_t)sizeof(raw);
#pragma unroll
            for (int i = 0; i < A_PT; ++i) dma16_soff(bA, offA[i], ldsA0 + (uint32_t)(st * STA + i * THREADS) * 16u);
#pragma unroll
            for (int i = 0; i < B_PT; ++i) dma16_soff(bB, offB[i], ldsB0 + (uint32_t)(st * STB + i * THREADS) * 16u);
        } else {
            issue_a(kt, sbuf + st * STA);
            issue_b(kt, sbuf + STAGES * STA + st * STB);
        }
    };

    f32x4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Fragment reads. A fragment (16 rows x one 16-byte chunk) is one ds_read_b128;
    // a B fragment is one ds_read_b128 (NT) or two transposing reads (NN).
    auto ldA = [&](const u32x4* sA, int ks, int i) -> u32x4 {
        const int r = wm * WTM + i * 16 + lrow;
        return sA[r * 8 + swz_dma(r, ks * 4 + lgrp)];
    };
    auto ldB = [&](const u32x4* sB, int ks, int j) -> u32x4 {
        if constexpr (!NN) {
            const int r = wn * WTN + j * 16 + lrow;
            return sB[r * 8 + swz_dma(r, ks * 4 + lgrp)];
        } else {
            const int nb = (wn * WTN + j * 16) >> 4;
            u32x4 v;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int r = ks * 32 + 8 * lgrp + 4 * h + (lrow >> 2);
                const int byte = r * (BN * 2) + (nn_blk(r, nb, BLK_MASK) << 5) + 8 * (lrow & 3);
                const u32x2 w = lds_read_tr16(sB, byte);
                v[2 * h] = w[0];
                v[2 * h + 1] = w[1];
            }
            return v;
        }
    };
    // One k step = 2 x 32 k = 2*FM A fragments (t = ks*FM + i). A fragments stream
    // through a ring of 3 registers, read two steps ahead; the B fragments of the
    // second half are read right after the first step. The schedule barriers pin
    // the order (reads for t+2, then the FN MFMAs of t), so every wait before an
    // MFMA is a partial lgkmcnt and the reads overlap the matrix work.
    constexpr int BR = NN ? 2 : 1;
    constexpr int NTS = 2 * FM;
    static_assert(FM >= 2, "the A ring needs at least 4 fragments per k step");
    auto compute = [&](const u32x4* sA, const u32x4* sB) {
        u32x4 fb[2][FN], fa[3];
#pragma unroll
        for (int j = 0; j < FN; ++j) fb[0][j] = ldB(sB, 0, j);
        fa[0] = ldA(sA, 0, 0);
        fa[1] = ldA(sA, 1 / FM, 1 % FM);
        __builtin_amdgcn_sched_group_barrier(0x100, FN * BR + 2, 0);
        static_for<0, NTS>([&](auto tc) {
            constexpr int t = decltype(tc)::value;
            constexpr int ks = t / FM, i = t % FM;
            constexpr int nrd = (t + 2 < NTS ? 1 : 0) + (t == 1 ? FN * BR : 0);
            if constexpr (t + 2 < NTS) fa[(t + 2) % 3] = ldA(sA, (t + 2) / FM, (t + 2) % FM);
            if constexpr (t == 1) {
#pragma unroll
                for (int j = 0; j < FN; ++j) fb[1][j] = ldB(sB, 1, j);
            }
#pragma unroll
            for (int j = 0; j < FN; ++j) acc[i][j] = mfma_chunk(T{}, fb[ks][j], fa[t % 3], acc[i][j]);
            if constexpr (nrd > 0) __builtin_amdgcn_sched_group_barrier(0x100, nrd, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, FN * MF_PER_CHUNK, 0);
        });
    };

    u32x4* sA = sbuf;
    u32x4* sB = sbuf + STAGES * STA;
    if constexpr (STAGES == 2) {
        // Double buffer: DMA of step kt+1 overlaps the MFMAs of step kt.
        issue_st(0, 0);
        wait_vmcnt<0>();
        __syncthreads();
        for (int kt = 0; kt < KT; ++kt) {
            const int cur = kt & 1;
            if (kt + 1 < KT) issue_st(kt + 1, cur ^ 1);
            compute(sA + cur * STA, sB + cur * STB);
            wait_vmcnt<0>();  // this wave's DMA for the next step has landed
            __syncthreads();
        }
    } else {
    // STAGES-deep ring: STAGES-1 k steps are in flight while one is computed.
#pragma unroll
    for (int st = 0; st < STAGES - 1; ++st)
        if (st < KT) issue_st(st, st);
    for (int kt = 0; kt < KT; ++kt) {
        // Stage kt has landed for this wave once at most `ahead` later stages are outstanding.
        const int ahead = min(STAGES - 2, KT - 1 - kt);
        if (STAGES > 2 && ahead >= 2) wait_vmcnt<(STAGES > 2 ? 2 : 0) * PER>();
        else if (STAGES > 2 && ahead == 1) wait_vmcnt<PER>();
        else wait_vmcnt<0>();
        __syncthreads();  // every wave's share of stage kt is in LDS; stage kt-1 is consumed
        const int nxt = kt + STAGES - 1;
        if (nxt < KT) issue_st(nxt, nxt % STAGES);
        compute(sA + (kt % STAGES) * STA, sB + (kt % STAGES) * STB);
    }
    }

    using oraw = typename TO::raw;
    oraw* Cp = static_cast<oraw*>(a.C) + bz * a.sc_b;
    if constexpr (sizeof(oraw) == 2 && BN >= 64) {
        if (a.beta == 0.0f && a.c_line_ok && m0 + BM <= a.m && n0 + BN <= a.n) {
            // A whole 16-bit tile leaves through LDS in rows of BN elements (chunk c of
            // row r at c ^ (r % CPR)): each thread stores 16-byte chunks of whole tile
            // rows, 128-byte lines and up, instead of the fragments' 8-byte pieces of
            // 16 rows (1040 x 12288 x 512: 24.6 -> 20.4 us; 512 x 6144 x 1024: 11.2 ->
            // 10.0 us). Tiles 32 wide keep the fragment stores: half lines gain nothing
            // there and the extra barriers cost.
            constexpr int CPR = BN / 8;  // 16-byte chunks per tile row
            static_assert(BM * BN * 2 <= STAGES * (STA + STB) * 16, "the C tile fits in the stages");
            char* t = reinterpret_cast<char*>(sbuf);
            __syncthreads();  // every wave is done reading the stages
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    const int r = wm * WTM + i * 16 + lrow;
                    const int cb = (wn * WTN + j * 16 + lgrp * 4) * 2;
                    *reinterpret_cast<u32x2*>(t + r * (2 * BN) + ((((cb >> 4) ^ (r & (CPR - 1))) << 4) | (cb & 15))) =
                        u32x2{pack2<TO>(a.alpha * acc[i][j][0], a.alpha * acc[i][j][1]),
                              pack2<TO>(a.alpha * acc[i][j][2], a.alpha * acc[i][j][3])};
                }
            __syncthreads();
#pragma unroll
            for (int id = tid; id < BM * CPR; id += THREADS) {
                const int r = id / CPR, c = id % CPR;
                *reinterpret_cast<u32x4*>(Cp + (int64_t)(m0 + r) * a.rsc + n0 + c * 8) =
                    *reinterpret_cast<const u32x4*>(t + r * (2 * BN) + ((c ^ (r & (CPR - 1))) << 4));
            }
            return;
        }
    }
#pragma unroll
    for (int i = 0; i < FM; ++i) {
        const int m = m0 + wm * WTM + i * 16 + lrow;
        if (m >= a.m) continue;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int n = n0 + wn * WTN + j * 16 + lgrp * 4;
            if (n >= a.n) continue;
            oraw* crow = Cp + (int64_t)m * a.rsc;
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) v[r] = a.alpha * acc[i][j][r];
            if (a.beta != 0.0f) {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (n + r < a.n) v[r] += a.beta * load_as_f32<TO>(crow, n + r);
            }
            if (a.c_vec_ok && n + 3 < a.n) {
                if constexpr (sizeof(oraw) == 2) {
                    *reinterpret_cast<u32x2*>(crow + n) = u32x2{pack2<TO>(v[0], v[1]), pack2<TO>(v[2], v[3])};
                } else {
                    *reinterpret_cast<f32x4*>(crow + n) = f32x4{v[0], v[1], v[2], v[3]};
                }
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (n + r < a.n) store_from_f32<TO>(crow, n + r, v[r]);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Ping-pong variant of the 256 x 256 DMA kernel for whole 256-row tiles.
// Waves 0-3 (group A) own tile rows 0-127, waves 4-7 (group B) rows 128-255;
// the hardware places waves w and w+4 on one SIMD. Per 64-wide k step kt, after
// one workgroup barrier,
//   group A: stages step kt+1 (DMA), reads every fragment of step kt from LDS
//            into registers (X), then runs the step's 64 MFMAs from registers at
//            raised issue priority (Y);
//   group B: runs Y(kt-1) on the fragments it read before the barrier, then
//            X(kt), and drains its LDS reads;
// so on each SIMD one wave's MFMA cluster runs while the other wave loads.
// Group A waits for its DMA of step kt+1 before the next barrier; group B's
// reads of a stage end before the barrier after which group A refills it.
// Same LDS layouts, swizzles, fragments and MFMA order as
// gemm_mfma_dma_kernel (bit-identical C).
// Requirements (host): m % 256 == 0, k % 64 == 0, every operand spans < 2^31
// bytes, and NN: n % 16 == 0 / NT: n % 256 == 0. Each DMA is a scalar base
// plus a 32-bit lane offset fixed for the kernel: A's (and NT B's) chunk
// swizzle repeats every 32 rows of a stage and NN B's block swizzle depends on
// the 8-k-row group only through its parity. A partial last column of NN
// tiles re-reads B's last 16 columns and stores only columns below N. A 16-bit
// C with beta == 0 and 16-byte aligned rows leaves through LDS as whole lines.
template <class T, class TO, bool NN>
__global__ __launch_bounds__(512, 1) void gemm_pingpong_kernel(GemmArgs a) {
    using raw = typename T::raw;
    static_assert(sizeof(raw) == 2, "16-bit operands");
    constexpr int BM = 256, BN = 256, BK = 64, GT = 256;
    constexpr int WTM = 128, WTN = 64, FM = 8, FN = 4;
    constexpr int STA = BM * 8, STB = BN * 8;        // 16-byte slots per stage
    constexpr int A_PT = STA / GT, B_PT = STB / GT;  // DMA per group-A thread per step
    constexpr int NBLK = BN / 16, BLK_MASK = 7;
    __shared__ u32x4 sbuf[2 * (STA + STB)];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool grpB = wave >= 4;
    const int wm = wave >> 2, wn = wave & 3;
    const int lrow = lane & 15, lgrp = lane >> 4;
    int tm, tn;
    tile_coords(blockIdx.x, a.tiles_m, a.tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int bz = blockIdx.y;
    const raw* __restrict__ Ap = static_cast<const raw*>(a.A) + bz * a.sa_b;
    const raw* __restrict__ Bp = static_cast<const raw*>(a.B) + bz * a.sb_b;
    const int KT = a.k / BK;
    u32x4* sA = sbuf;
    u32x4* sB = sbuf + 2 * STA;

    // DMA slot i*256 + t of a stage (t < 256: group A)
    const int t = tid & (GT - 1);
    uint32_t offA, offB0, offB1;
    {
        const int r0 = t >> 3;
        const int c = swz_dma(r0, t & 7);
        offA = (uint32_t)(((int64_t)(m0 + r0) * a.rsa + c * 8) * 2);
        if constexpr (NN) {
            // columns past N (a partial last tile column) re-read the last 16 (never stored)
            const int kr = t / (2 * NBLK), ps = t % (2 * NBLK);
            const int lb0 = nn_blk(kr, ps >> 1, BLK_MASK), lb1 = nn_blk(kr + 8, ps >> 1, BLK_MASK);
            offB0 = (uint32_t)(((int64_t)kr * a.rsb + min(n0 + lb0 * 16, a.n - 16) + (ps & 1) * 8) * 2);
            offB1 = (uint32_t)(((int64_t)kr * a.rsb + min(n0 + lb1 * 16, a.n - 16) + (ps & 1) * 8) * 2);
        } else {
            offB0 = offB1 = (uint32_t)(((int64_t)(n0 + r0) * a.csb + c * 8) * 2);
        }
    }
    const uint32_t ldsA = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)&sA[(wave & 3) * 64]);
    const uint32_t ldsB = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)&sB[(wave & 3) * 64]);
    // the DMA of step kt: A's slice, then B's
    auto issueA = [&](int kt) {
        const int st = kt & 1;
        const char* bA = reinterpret_cast<const char*>(Ap) + (int64_t)kt * BK * 2;
#pragma unroll
        for (int i = 0; i < A_PT; ++i)
            dma16_soff(bA + (int64_t)i * 32 * a.rsa * 2, offA, ldsA + (uint32_t)(st * STA + i * GT) * 16u);
    };
    auto issueB = [&](int kt) {
        const int st = kt & 1;
        const char* bB = reinterpret_cast<const char*>(Bp) + (int64_t)kt * BK * (NN ? a.rsb : (int64_t)1) * 2;
#pragma unroll
        for (int i = 0; i < B_PT; ++i) {
            const int64_t step = NN ? (int64_t)i * 8 * a.rsb * 2 : (int64_t)i * 32 * a.csb * 2;
            dma16_soff(bB + step, (i & 1) ? offB1 : offB0, ldsB + (uint32_t)(st * STB + i * GT) * 16u);
        }
    };
    // half hf of A's or B's slice of step kt
    auto issueAh = [&](int kt, int hf) {
        const int st = kt & 1;
        const char* bA = reinterpret_cast<const char*>(Ap) + (int64_t)kt * BK * 2;
#pragma unroll
        for (int i = hf * (A_PT / 2); i < (hf + 1) * (A_PT / 2); ++i)
            dma16_soff(bA + (int64_t)i * 32 * a.rsa * 2, offA, ldsA + (uint32_t)(st * STA + i * GT) * 16u);
    };
    auto issueBh = [&](int kt, int hf) {
        const int st = kt & 1;
        const char* bB = reinterpret_cast<const char*>(Bp) + (int64_t)kt * BK * (NN ? a.rsb : (int64_t)1) * 2;
#pragma unroll
        for (int i = hf * (B_PT / 2); i < (hf + 1) * (B_PT / 2); ++i) {
            const int64_t step = NN ? (int64_t)i * 8 * a.rsb * 2 : (int64_t)i * 32 * a.csb * 2;
            dma16_soff(bB + step, (i & 1) ? offB1 : offB0, ldsB + (uint32_t)(st * STB + i * GT) * 16u);
        }
    };
    auto ldA = [&](const u32x4* s, int ks, int i) -> u32x4 {
        const int r = wm * WTM + i * 16 + lrow;
        return s[r * 8 + swz_dma(r, ks * 4 + lgrp)];
    };
    auto ldB = [&](const u32x4* s, int ks, int j) -> u32x4 {
        if constexpr (!NN) {
            const int r = wn * WTN + j * 16 + lrow;
            return s[r * 8 + swz_dma(r, ks * 4 + lgrp)];
        } else {
            const int nb = (wn * WTN + j * 16) >> 4;
            u32x4 v;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int r = ks * 32 + 8 * lgrp + 4 * h + (lrow >> 2);
                const int byte = r * (BN * 2) + (nn_blk(r, nb, BLK_MASK) << 5) + 8 * (lrow & 3);
                const u32x2 w = lds_read_tr16(s, byte);
                v[2 * h] = w[0];
                v[2 * h + 1] = w[1];
            }
            return v;
        }
    };

    f32x4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    u32x4 fa[2][FM], fb[2][FN];
    // the fragments of step kt's 32-wide k chunk ks
    auto Xk = [&](int kt, int ks) {
        const u32x4* cA = sA + (kt & 1) * STA;
        const u32x4* cB = sB + (kt & 1) * STB;
#pragma unroll
        for (int j = 0; j < FN; ++j) fb[ks][j] = ldB(cB, ks, j);
#pragma unroll
        for (int i = 0; i < FM; ++i) fa[ks][i] = ldA(cA, ks, i);
    };
    auto X = [&](int kt) {
        Xk(kt, 0);
        Xk(kt, 1);
    };
    auto XB = [&](int kt, int ks) {
        const u32x4* cB = sB + (kt & 1) * STB;
#pragma unroll
        for (int j = 0; j < FN; ++j) fb[ks][j] = ldB(cB, ks, j);
    };
    auto XA = [&](int kt, int ks) {
        const u32x4* cA = sA + (kt & 1) * STA;
#pragma unroll
        for (int i = 0; i < FM; ++i) fa[ks][i] = ldA(cA, ks, i);
    };
    // the MFMA order of gemm_mfma_dma_kernel: per output fragment, k chunk 0 then 1
    auto Y = [&]() {
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j) acc[i][j] = mfma_chunk(T{}, fb[ks][j], fa[ks][i], acc[i][j]);
        __builtin_amdgcn_s_setprio(0);
    };
    constexpr int LGKM0 = 0xc07f;  // s_waitcnt lgkmcnt(0), vmcnt and expcnt not waited
    if (!grpB) {
        issueA(0);
        issueB(0);
        for (int kt = 0; kt < KT; ++kt) {
            wait_vmcnt<0>();               // this wave's share of step kt has landed
            __builtin_amdgcn_s_barrier();  // step kt in LDS; group B done with stage (kt+1)&1
            // step kt+1's DMA interleaved with step kt's fragment reads, the same
            // bits. NT: A's slice, the first k chunk, B's slice, the second (4096^3
            // NT 96.7 -> 94.6 us, the LM head 563 -> 559 us). NN, in quarters: half
            // of A's slice before each of the first chunk's B and A fragment reads,
            // then half of B's before the second chunk's (4096^3 NN 98.7 -> 98.0 ->
            // 97.0 us over the two steps)
            const bool nx = kt + 1 < KT;
            if constexpr (NN) {
                if (nx) issueAh(kt + 1, 0);
                XB(kt, 0);
                if (nx) issueAh(kt + 1, 1);
                XA(kt, 0);
                if (nx) issueBh(kt + 1, 0);
                XB(kt, 1);
                if (nx) issueBh(kt + 1, 1);
                XA(kt, 1);
            } else {
                if (nx) issueA(kt + 1);
                Xk(kt, 0);
                if (nx) issueB(kt + 1);
                Xk(kt, 1);
            }
            Y();
        }
    } else {
        for (int kt = 0; kt < KT; ++kt) {
            __builtin_amdgcn_s_barrier();
            if (kt > 0) Y();  // step kt-1, read before the barrier
            X(kt);
            __builtin_amdgcn_s_waitcnt(LGKM0);  // the stage's reads end before group A refills it
        }
        Y();
    }

    using oraw = typename TO::raw;
    oraw* Cp = static_cast<oraw*>(a.C) + bz * a.sc_b;
    if constexpr (sizeof(oraw) == 2) {
        if (a.beta == 0.0f && a.c_line_ok) {
            // Whole 128-byte lines of C. A fragment store writes 32 bytes into each
            // of 16 rows, a quarter of a line per row, and the launch then spends
            // microseconds per tile in the store path (the LM head's 18 rounds of
            // tiles lose ~10% to it). Instead each wave rounds its 128 x 64 tile into
            // 16 KiB of a free operand stage (row r at r * 128 bytes, 16-byte chunk c
            // at c ^ (r & 7)) and stores 8 whole rows per instruction. Group A's waves
            // take the stage no wave reads in the last k step and go at once; group
            // B's take the other one after a barrier that group A meets once its
            // stores are out.
            const int sl = ((KT - 1) & 1) ^ (grpB ? 0 : 1);
            const bool bhalf = (wave & 3) >= 2;  // waves 0, 1, 4, 5 use A's stage, 2, 3, 6, 7 B's
            char* wl = reinterpret_cast<char*>(bhalf ? sB + sl * STB : sA + sl * STA) + (wave & 1) * (WTM * WTN * 2);
            if (grpB) __builtin_amdgcn_s_barrier();
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    const int r = i * 16 + lrow;
                    const int cb = j * 32 + lgrp * 8;  // byte of the lane's 4 columns in the row
                    *reinterpret_cast<u32x2*>(wl + r * 128 + ((((cb >> 4) ^ (r & 7)) << 4) | (cb & 15))) =
                        u32x2{pack2<TO>(a.alpha * acc[i][j][0], a.alpha * acc[i][j][1]),
                              pack2<TO>(a.alpha * acc[i][j][2], a.alpha * acc[i][j][3])};
                }
            // the wave reads back only its own writes: LDS keeps a wave's accesses in order
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_s_waitcnt(LGKM0);
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
            for (int q = 0; q < WTM / 8; ++q) {
                const int r = q * 8 + (lane >> 3), c = lane & 7;
                const u32x4 v = *reinterpret_cast<const u32x4*>(wl + r * 128 + ((c ^ (r & 7)) << 4));
                const int n = n0 + wn * WTN + c * 8;  // n % 16 == 0: the 8 columns are all in or all out
                if (n < a.n) *reinterpret_cast<u32x4*>(Cp + (int64_t)(m0 + wm * WTM + r) * a.rsc + n) = v;
            }
            if (!grpB) __builtin_amdgcn_s_barrier();
            return;
        }
    }
#pragma unroll
    for (int i = 0; i < FM; ++i) {
        const int m = m0 + wm * WTM + i * 16 + lrow;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int n = n0 + wn * WTN + j * 16 + lgrp * 4;
            if (n >= a.n) continue;  // n % 16 == 0: the lane's 4 columns are all in or all out
            oraw* crow = Cp + (int64_t)m * a.rsc;
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) v[r] = a.alpha * acc[i][j][r];
            if (a.beta != 0.0f) {
#pragma unroll
                for (int r = 0; r < 4; ++r) v[r] += a.beta * load_as_f32<TO>(crow, n + r);
            }
            if (a.c_vec_ok) {
                if constexpr (sizeof(oraw) == 2) {
                    *reinterpret_cast<u32x2*>(crow + n) = u32x2{pack2<TO>(v[0], v[1]), pack2<TO>(v[2], v[3])};
                } else {
                    *reinterpret_cast<f32x4*>(crow + n) = f32x4{v[0], v[1], v[2], v[3]};
                }
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r) store_from_f32<TO>(crow, n + r, v[r]);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Skinny GEMM, M <= 16 (the decode GEMVs: x [1..16, K] . W^T). HBM-bound on
// the weight stream, so the design goal is bytes in flight, not MFMA reuse.
//   NT (W^T, the `linear` layout): gemv_kernel in gemv.hip.
//   NN (B [K][N] row-major): VALU; M == 1 in gemv_nn_kernel (16-byte chunks
//   of 8 k-rows per load), else lane = one output column, coalesced 2-byte
//   row loads, 8 waves split K, LDS reduction.
// ---------------------------------------------------------------------------
constexpr int SKINNY_M = 16;
constexpr int SKINNY_WAVES = 8;

template <class T, class TO>
__global__ __launch_bounds__(64 * SKINNY_WAVES) void gemm_skinny_nn_kernel(GemmArgs a) {
    using raw = typename T::raw;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = blockIdx.x * 64 + lane;
    const int bz = blockIdx.y;
    const raw* __restrict__ Ap = static_cast<const raw*>(a.A) + bz * a.sa_b;
    const raw* __restrict__ Bp = static_cast<const raw*>(a.B) + bz * a.sb_b;
    const int per_wave = (a.k + SKINNY_WAVES - 1) / SKINNY_WAVES;
    const int k_begin = wave * per_wave, k_end = min(a.k, k_begin + per_wave);
    float acc[SKINNY_M];
#pragma unroll
    for (int i = 0; i < SKINNY_M; ++i) acc[i] = 0.f;
    const bool col = n < a.n;
    const raw* bp = Bp + (col ? n : 0);
    constexpr int UNR = 8;
    int k = k_begin;
    for (; k + UNR <= k_end; k += UNR) {
        float b[UNR];
#pragma unroll
        for (int u = 0; u < UNR; ++u) b[u] = col ? load_as_f32<T>(bp, (int64_t)(k + u) * a.rsb) : 0.f;
#pragma unroll
        for (int i = 0; i < SKINNY_M; ++i) {
            if (i < a.m) {
#pragma unroll
                for (int u = 0; u < UNR; ++u) acc[i] = fmaf(load_as_f32<T>(Ap, (int64_t)i * a.rsa + k + u), b[u], acc[i]);
            }
        }
    }
    for (; k < k_end; ++k) {
        const float b = col ? load_as_f32<T>(bp, (int64_t)k * a.rsb) : 0.f;
#pragma unroll
        for (int i = 0; i < SKINNY_M; ++i)
            if (i < a.m) acc[i] = fmaf(load_as_f32<T>(Ap, (int64_t)i * a.rsa + k), b, acc[i]);
    }
    __shared__ float red[SKINNY_WAVES][SKINNY_M][64];
#pragma unroll
    for (int i = 0; i < SKINNY_M; ++i) red[wave][i][lane] = acc[i];
    __syncthreads();
    if (wave != 0 || !col) return;
    using oraw = typename TO::raw;
    for (int i = 0; i < a.m; ++i) {
        float t = 0.f;
#pragma unroll
        for (int w = 0; w < SKINNY_WAVES; ++w) t += red[w][i][lane];
        oraw* crow = static_cast<oraw*>(a.C) + bz * a.sc_b + (int64_t)i * a.rsc;
        float v = a.alpha * t;
        if (a.beta != 0.0f) v += a.beta * load_as_f32<TO>(crow, n);
        store_from_f32<TO>(crow, n, v);
    }
}

// M == 1 with row-major B [K][N] (the configs' weight layout): a workgroup owns
// CPR * VEC consecutive columns (CPR 16-byte chunks of a k-row); its 16 waves
// split K, and within a wave lane (r, c) = (lane / CPR, lane % CPR) reads chunk c
// of k-rows r, r + 64/CPR, ... (all of a wave's loads issued before the first
// use). CPR is chosen so the grid covers the CUs: narrower column tiles read
// shorter row pieces but keep more CUs streaming. Per lane VEC fp32 partials in
// k order, a butterfly over the row lanes, then a fixed-order sum of the 16
// waves' partials in LDS.
template <class T, class TO, int CPR>
__global__ __launch_bounds__(1024) void gemv_nn_kernel(GemmArgs a) {
    using raw = typename T::raw;
    constexpr int VEC = 16 / sizeof(raw), WAVES = 16, UNR = 8, RPI = 64 / CPR;  // k-rows per load
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = lane % CPR, r = lane / CPR;
    // column tiles t..t+T/8-1 on one XCD (workgroups are dealt to the 8 XCDs
    // round-robin): tiles narrower than a 128-byte line share its fetch in one L2
    int tile = blockIdx.x;
    if ((gridDim.x & 7) == 0) tile = (tile & 7) * (gridDim.x >> 3) + (tile >> 3);
    const int n0 = tile * CPR * VEC;
    const int bz = blockIdx.y;
    const raw* __restrict__ Ap = static_cast<const raw*>(a.A) + bz * a.sa_b;
    const raw* __restrict__ Bp = static_cast<const raw*>(a.B) + bz * a.sb_b + n0 + c * VEC;
    const bool col = n0 + c * VEC < a.n;  // the host guarantees n % VEC == 0
    const int kper = ((a.k + WAVES - 1) / WAVES + RPI - 1) / RPI * RPI;
    const int kb = wave * kper, ke = min(a.k, kb + kper);
    float acc[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] = 0.f;
    for (int k0 = kb; k0 < ke; k0 += RPI * UNR) {
        u32x4 w[UNR];
        float x[UNR];
#pragma unroll
        for (int u = 0; u < UNR; ++u) {
            const int kk = k0 + RPI * u + r;
            const bool ok = col && kk < ke;
            w[u] = ok ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(Bp + (int64_t)kk * a.rsb))
                      : u32x4{0u, 0u, 0u, 0u};
            x[u] = kk < ke ? load_as_f32<T>(Ap, kk) : 0.f;
        }
#pragma unroll
        for (int u = 0; u < UNR; ++u) {
            if constexpr (sizeof(raw) == 2) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t we = w[u][e];
                    acc[2 * e] = fmaf(x[u], lo_as_f32(T{}, we), acc[2 * e]);
                    acc[2 * e + 1] = fmaf(x[u], hi_as_f32(T{}, we), acc[2 * e + 1]);
                }
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[e] = fmaf(x[u], __uint_as_float(w[u][e]), acc[e]);
            }
        }
    }
#pragma unroll
    for (int off = CPR; off < 64; off <<= 1)
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[e] += __shfl_xor(acc[e], off, 64);
    __shared__ float red[WAVES][CPR * VEC];
    if (r == 0) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) red[wave][c * VEC + e] = acc[e];
    }
    __syncthreads();
    if (tid >= CPR * VEC) return;
    const int n = n0 + tid;
    if (n >= a.n) return;
    float t = 0.f;
#pragma unroll
    for (int w2 = 0; w2 < WAVES; ++w2) t += red[w2][tid];
    using oraw = typename TO::raw;
    oraw* crow = static_cast<oraw*>(a.C) + bz * a.sc_b;
    float v = a.alpha * t;
    if (a.beta != 0.0f) v += a.beta * load_as_f32<TO>(crow, n);
    store_from_f32<TO>(crow, n, v);
}

// fp32 GEMM on v_mfma_f32_16x16x4_f32 with DMA-staged tiles (configs[0], the
// reference's sgemm_rowmajor, src/kernel/avx2/sgemm.inl:268-340, and its
// transposed-B forms). Block tile BM x BN, k step BK = 32 (one 128-byte row of
// fp32), an LDS ring of STAGES steps filled by global_load_lds (two in flight
// ahead of the one being computed with 4 stages). Operands are swapped
// (src0 = B^T fragment, src1 = A fragment) so lane l holds C[m = l % 16][n =
// 4 g + 0..3], g = l / 16: one 16-byte store per output fragment.
//   A tile [BM rows][8 chunks of 16 B]: chunk c of row r at c ^ (r & 7); the
//     fragment of a 16-wide k block kb is one ds_read_b128 (chunk 4 kb + g) per
//     lane feeding 4 MFMAs.
//   B, NT (B = W^T, W [n][k] rows): the same layout as A.
//   B, NN (row-major [k][n]): [BK rows][BN / 4 chunks], chunk c of k-row r at
//     c ^ (((r >> 2) & 3) << 2); MFMA step j of lane group g reads k-row
//     16 kb + 4 g + j, one ds_read_b32 of n = 16 fn + l % 16: the four groups'
//     rows land in four bank ranges.
// Rows of A / B past m / n re-read the last row (never stored); k % 32 == 0.
template <int BM, int BN, int WM, int WN, bool NN, int STAGES>
__global__ __launch_bounds__(64 * WM * WN) void gemm_f32_kernel(GemmArgs a) {
    constexpr int THREADS = 64 * WM * WN;
    constexpr int BK = 32;
    static_assert(STAGES >= 3, "the ring keeps two k steps in flight");
    constexpr int WTM = BM / WM, WTN = BN / WN;
    constexpr int FM = WTM / 16, FN = WTN / 16;
    constexpr int STA = BM * 8;                        // 16-byte chunks of an A stage
    constexpr int STB = NN ? BK * (BN / 4) : BN * 8;   // ... of a B stage
    constexpr int A_PT = STA / THREADS, B_PT = STB / THREADS;
    static_assert(A_PT * THREADS == STA && B_PT * THREADS == STB, "tile / thread mismatch");
    static_assert(!NN || BN >= 64, "the NN swizzle needs 16 chunks per k-row");
    constexpr int PER = A_PT + B_PT;
    __shared__ u32x4 sA[STAGES * STA];
    __shared__ u32x4 sB[STAGES * STB];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r16 = lane & 15, g = lane >> 4;
    const int wm = wave / WN, wn = wave % WN;
    int tm, tn;
    tile_coords(blockIdx.x, a.tiles_m, a.tiles_n, tm, tn);
    const int bz = blockIdx.y;
    const int m0 = tm * BM, n0 = tn * BN;
    const float* Ap = static_cast<const float*>(a.A) + bz * a.sa_b;
    const float* Bp = static_cast<const float*>(a.B) + bz * a.sb_b;

    // DMA element offsets within a k step (the base moves by BK along k)
    int aoff[A_PT], boff[B_PT];  // source chunk of each DMA slot
    int64_t arow[A_PT];
#pragma unroll
    for (int i = 0; i < A_PT; ++i) {
        const int slot = i * THREADS + tid;
        const int row = slot / 8, c = slot % 8;
        aoff[i] = c ^ (row & 7);
        arow[i] = (int64_t)min(m0 + row, a.m - 1) * a.rsa;
    }
    int64_t bbase[B_PT];
#pragma unroll
    for (int i = 0; i < B_PT; ++i) {
        const int slot = i * THREADS + tid;
        if constexpr (NN) {
            constexpr int BCH = BN / 4;
            const int row = slot / BCH, c = slot % BCH;   // k-row, n chunk
            const int src = c ^ (((row >> 2) & 3) << 2);
            const int nn = min(n0 + 4 * src, a.n - 4);    // n % 4 == 0 on this path
            bbase[i] = (int64_t)row * a.rsb + nn;
            boff[i] = 0;
        } else {
            const int row = slot / 8, c = slot % 8;       // n-row, k chunk
            bbase[i] = (int64_t)min(n0 + row, a.n - 1) * a.csb;
            boff[i] = (c ^ (row & 7)) * 4;
        }
    }
    auto issue = [&](int ks) {
        const int k0 = ks * BK;
        u32x4* dA = sA + (ks % STAGES) * STA;
        u32x4* dB = sB + (ks % STAGES) * STB;
#pragma unroll
        for (int i = 0; i < A_PT; ++i) dma16_async(Ap + arow[i] + k0 + aoff[i] * 4, &dA[i * THREADS + wave * 64]);
#pragma unroll
        for (int i = 0; i < B_PT; ++i) {
            if constexpr (NN) dma16_async(Bp + bbase[i] + (int64_t)k0 * a.rsb, &dB[i * THREADS + wave * 64]);
            else dma16_async(Bp + bbase[i] + k0 + boff[i], &dB[i * THREADS + wave * 64]);
        }
    };

    f32x4 acc[FM][FN];
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) acc[fm][fn] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int nks = a.k / BK;
    constexpr int AHEAD = STAGES - 1;  // steps issued before the first one is computed
#pragma unroll
    for (int i = 0; i < AHEAD; ++i)
        if (i < nks) issue(i);
    for (int ks = 0; ks < nks; ++ks) {
        // this thread's DMA of step ks has landed (the later steps' may still fly)
        const int later = min(nks - 1 - ks, AHEAD - 1);
        if (later >= 2) wait_vmcnt<2 * PER>();
        else if (later == 1) wait_vmcnt<PER>();
        else wait_vmcnt<0>();
        __syncthreads();
        if (ks + AHEAD < nks) issue(ks + AHEAD);
        const u32x4* cA = sA + (ks % STAGES) * STA;
        const u32x4* cB = sB + (ks % STAGES) * STB;
        const float* cBf = reinterpret_cast<const float*>(cB);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            f32x4 af[FM];
#pragma unroll
            for (int fm = 0; fm < FM; ++fm) {
                const int row = wm * WTM + fm * 16 + r16;
                af[fm] = __builtin_bit_cast(f32x4, cA[row * 8 + ((4 * kb + g) ^ (row & 7))]);
            }
            if constexpr (!NN) {
                f32x4 bf[FN];
#pragma unroll
                for (int fn = 0; fn < FN; ++fn) {
                    const int row = wn * WTN + fn * 16 + r16;
                    bf[fn] = __builtin_bit_cast(f32x4, cB[row * 8 + ((4 * kb + g) ^ (row & 7))]);
                }
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
                        for (int fn = 0; fn < FN; ++fn)
                            acc[fm][fn] = __builtin_amdgcn_mfma_f32_16x16x4f32(bf[fn][j], af[fm][j], acc[fm][fn], 0, 0, 0);
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int krow = 16 * kb + 4 * g + j;  // (krow >> 2) & 3 == g
                    float bf[FN];
#pragma unroll
                    for (int fn = 0; fn < FN; ++fn) {
                        const int nl = wn * WTN + fn * 16 + r16;  // n within the tile
                        const int ch = (nl >> 2) ^ (g << 2);
                        bf[fn] = cBf[krow * BN + ch * 4 + (nl & 3)];
                    }
#pragma unroll
                    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
                        for (int fn = 0; fn < FN; ++fn)
                            acc[fm][fn] = __builtin_amdgcn_mfma_f32_16x16x4f32(bf[fn], af[fm][j], acc[fm][fn], 0, 0, 0);
                }
            }
        }
    }
    // epilogue: lane holds C[m0 + wm WTM + 16 fm + l % 16][n0 + wn WTN + 16 fn + 4 g + i]
    float* Cp = static_cast<float*>(a.C) + bz * a.sc_b;
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
        const int m = m0 + wm * WTM + fm * 16 + r16;
        if (m >= a.m) continue;
        float* crow = Cp + (int64_t)m * a.rsc;
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) {
            const int n = n0 + wn * WTN + fn * 16 + 4 * g;
            f32x4 v = acc[fm][fn] * a.alpha;
            if (a.c_vec_ok && n + 3 < a.n) {
                if (a.beta != 0.0f) v += a.beta * *reinterpret_cast<const f32x4*>(crow + n);
                *reinterpret_cast<f32x4*>(crow + n) = v;
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (n + i < a.n) crow[n + i] = a.beta != 0.0f ? v[i] + a.beta * crow[n + i] : v[i];
            }
        }
    }
}

// Any-stride fallback: one output per thread, fp32 accumulation in k order.
struct GenericArgs {
    const void* A;
    const void* B;
    void* C;
    int m, n, k;
    int64_t rsa, csa, rsb, csb, rsc, csc, sa_b, sb_b, sc_b;
    float alpha, beta;
};

template <class T, class TO>
__global__ __launch_bounds__(256) void gemm_generic_kernel(GenericArgs a) {
    const int j = blockIdx.x * 16 + (threadIdx.x & 15);
    const int i = blockIdx.y * 16 + (threadIdx.x >> 4);
    const int b = blockIdx.z;
    if (i >= a.m || j >= a.n) return;
    const int64_t ao = b * a.sa_b + i * a.rsa, bo = b * a.sb_b + j * a.csb;
    float acc = 0.0f;
    for (int p = 0; p < a.k; ++p)
        acc = fmaf(load_as_f32<T>(a.A, ao + p * a.csa), load_as_f32<T>(a.B, bo + p * a.rsb), acc);
    const int64_t co = b * a.sc_b + i * a.rsc + j * a.csc;
    float v = a.alpha * acc;
    if (a.beta != 0.0f) v += a.beta * load_as_f32<TO>(a.C, co);
    store_from_f32<TO>(a.C, co, v);
}

// C = beta * C (k == 0 or alpha == 0), sgemm.inl:594-604.
template <class TO>
__global__ __launch_bounds__(256) void gemm_scale_kernel(void* C, int m, int n, int64_t rsc, int64_t csc,
                                                         int64_t sc_b, float beta) {
    const int j = blockIdx.x * 16 + (threadIdx.x & 15);
    const int i = blockIdx.y * 16 + (threadIdx.x >> 4);
    if (i >= m || j >= n) return;
    const int64_t co = blockIdx.z * sc_b + i * rsc + j * csc;
    const float v = (beta == 0.0f) ? 0.0f : beta * load_as_f32<TO>(C, co);
    store_from_f32<TO>(C, co, v);
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
namespace {

template <class T, class TO, int BM, int BN, int WM, int WN>
hipError_t launch_tile(const GemmArgs& a0, bool nn, int batch, hipStream_t s) {
    GemmArgs a = a0;
    a.tiles_m = (a.m + BM - 1) / BM;
    a.tiles_n = (a.n + BN - 1) / BN;
    dim3 grid(a.tiles_m * a.tiles_n, batch);
    dim3 block(64 * WM * WN);
    if (nn)
        gemm_mfma_kernel<T, TO, BM, BN, WM, WN, true><<<grid, block, 0, s>>>(a);
    else
        gemm_mfma_kernel<T, TO, BM, BN, WM, WN, false><<<grid, block, 0, s>>>(a);
    return hipGetLastError();
}

template <class T, class TO, int BM, int BN, int WM, int WN, int STAGES>
hipError_t launch_dma_tile(const GemmArgs& a0, bool nn, int batch, hipStream_t s) {
    GemmArgs a = a0;
    a.tiles_m = (a.m + BM - 1) / BM;
    a.tiles_n = (a.n + BN - 1) / BN;
    dim3 grid(a.tiles_m * a.tiles_n, batch);
    dim3 block(64 * WM * WN);
    // bytes spanned by one batch entry's A and B (the DMA addresses stay inside)
    constexpr int64_t es = sizeof(typename T::raw);
    const int64_t span_a = ((int64_t)(a.m - 1) * a.rsa + a.k) * es;
    const int64_t span_b = (nn ? (int64_t)(a.k - 1) * a.rsb + a.n : (int64_t)(a.n - 1) * a.csb + a.k) * es;
    const bool soff = span_a < (int64_t(1) << 31) && span_b < (int64_t(1) << 31);
    if constexpr (sizeof(typename T::raw) == 2) {
        if (nn) {
            if (soff) gemm_mfma_dma_kernel<T, TO, BM, BN, WM, WN, true, STAGES, true><<<grid, block, 0, s>>>(a);
            else gemm_mfma_dma_kernel<T, TO, BM, BN, WM, WN, true, STAGES, false><<<grid, block, 0, s>>>(a);
            return hipGetLastError();
        }
    }
    if (soff) gemm_mfma_dma_kernel<T, TO, BM, BN, WM, WN, false, STAGES, true><<<grid, block, 0, s>>>(a);
    else gemm_mfma_dma_kernel<T, TO, BM, BN, WM, WN, false, STAGES, false><<<grid, block, 0, s>>>(a);
    return hipGetLastError();
}

template <class T, class TO>
hipError_t launch_dma(const GemmArgs& a, bool nn, int batch, hipStream_t s) {
    auto tiles = [&](int bm, int bn) {
        return (int64_t)((a.m + bm - 1) / bm) * ((a.n + bn - 1) / bn) * batch;
    };
    // Chosen from a sweep of M x N x K shapes on MI355X (bf16): the 256 x 256 tile
    // once it has most of the 256 CUs busy, 128 x 128 (two workgroups per CU) for
    // mid sizes, 64 x 64 below that; the 64 x 64 ring pays off only while its
    // grid is short of several workgroups per CU.
    if (tiles(256, 256) >= 192) {
        if constexpr (sizeof(typename T::raw) == 2) {
            // whole 256-row tiles: the ping-pong schedule (same bits)
            constexpr int64_t es = 2;
            const int64_t span_a = ((int64_t)(a.m - 1) * a.rsa + a.k) * es;
            const int64_t span_b = (nn ? (int64_t)(a.k - 1) * a.rsb + a.n : (int64_t)(a.n - 1) * a.csb + a.k) * es;
            // NT with a partial last column of tiles: the whole tiles on the
            // ping-pong kernel, the last N % 256 columns as a product of their own
            // (disjoint columns of C; B rows and C columns offset).
            if (!nn && a.m % 256 == 0 && a.n % 256 != 0 && a.n > 256 && span_a < (int64_t(1) << 31) &&
                span_b < (int64_t(1) << 31)) {
                using oraw = typename TO::raw;
                GemmArgs g = a;
                g.n = a.n / 256 * 256;
                g.tiles_m = a.m / 256;
                g.tiles_n = g.n / 256;
                gemm_pingpong_kernel<T, TO, false><<<dim3(g.tiles_m * g.tiles_n, batch), 512, 0, s>>>(g);
                const hipError_t e = hipGetLastError();
                if (e != hipSuccess) return e;
                GemmArgs r = a;
                r.n = a.n - g.n;
                r.B = static_cast<const typename T::raw*>(a.B) + (int64_t)g.n * a.csb;
                r.C = static_cast<oraw*>(a.C) + g.n;
                return launch_dma<T, TO>(r, nn, batch, s);
            }
            if (a.m % 256 == 0 && (nn ? a.n % 16 == 0 : a.n % 256 == 0) && span_a < (int64_t(1) << 31) &&
                span_b < (int64_t(1) << 31)) {
                GemmArgs g = a;
                g.tiles_m = a.m / 256;
                g.tiles_n = (a.n + 255) / 256;
                const dim3 grid(g.tiles_m * g.tiles_n, batch);
                if (nn) gemm_pingpong_kernel<T, TO, true><<<grid, 512, 0, s>>>(g);
                else gemm_pingpong_kernel<T, TO, false><<<grid, 512, 0, s>>>(g);
                return hipGetLastError();
            }
        }
        return launch_dma_tile<T, TO, 256, 256, 2, 4, 2>(a, nn, batch, s);
    }
    if (tiles(128, 128) >= 384) return launch_dma_tile<T, TO, 128, 128, 2, 2, 2>(a, nn, batch, s);
    if (tiles(64, 64) >= 768) return launch_dma_tile<T, TO, 64, 64, 2, 2, 2>(a, nn, batch, s);
    // Fewer 64 x 64 tiles than CUs: 64 x 32 tiles (two waves) put twice as many
    // workgroups, hence CUs, on the operand stream (7-10% on the Qwen3 prefill
    // projections with weights coming from HBM).
    if (tiles(64, 64) < 256) return launch_dma_tile<T, TO, 64, 32, 2, 1, 4>(a, nn, batch, s);
    return launch_dma_tile<T, TO, 64, 64, 2, 2, 4>(a, nn, batch, s);
}

template <class T, class TO>
hipError_t launch_mfma(const GemmArgs& a, bool nn, int batch, hipStream_t s) {
    auto tiles = [&](int bm, int bn) {
        return (int64_t)((a.m + bm - 1) / bm) * ((a.n + bn - 1) / bn) * batch;
    };
    if (tiles(256, 256) >= 160) return launch_tile<T, TO, 256, 256, 2, 4>(a, nn, batch, s);
    if (tiles(128, 128) >= 96) return launch_tile<T, TO, 128, 128, 2, 2>(a, nn, batch, s);
    return launch_tile<T, TO, 64, 64, 2, 2>(a, nn, batch, s);
}

template <class T, class TO>
hipError_t launch_generic(const GenericArgs& a, int batch, hipStream_t s) {
    dim3 grid((a.n + 15) / 16, (a.m + 15) / 16, batch);
    gemm_generic_kernel<T, TO><<<grid, 256, 0, s>>>(a);
    return hipGetLastError();
}

template <class TO>
hipError_t launch_scale(void* C, int m, int n, int64_t rsc, int64_t csc, int64_t sc_b, float beta, int batch,
                        hipStream_t s) {
    dim3 grid((n + 15) / 16, (m + 15) / 16, batch);
    gemm_scale_kernel<TO><<<grid, 256, 0, s>>>(C, m, n, rsc, csc, sc_b, beta);
    return hipGetLastError();
}

bool aligned(const void* p, int bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }

template <class T, class TO>
int gemm_typed(int batch, int m, int n, int k, const void* A, int64_t sa_b, int64_t rsa, int64_t csa,
               const void* B, int64_t sb_b, int64_t rsb, int64_t csb, void* C, int64_t sc_b, int64_t rsc,
               int64_t csc, float alpha, float beta, hipStream_t s) {
    using raw = typename T::raw;
    using oraw = typename TO::raw;
    constexpr int VEC = 16 / sizeof(raw);
    if (k == 0 || alpha == 0.0f) return status_of(launch_scale<TO>(C, m, n, rsc, csc, sc_b, beta, batch, s));

    const int es = sizeof(raw);
    const bool a_ok = csa == 1 && (rsa % VEC) == 0 && (sa_b % VEC) == 0 && aligned(A, 16) && (k % VEC) == 0;
    const bool nt = rsb == 1 && (csb % VEC) == 0 && (sb_b % VEC) == 0 && aligned(B, 16);
    const bool nn = !nt && csb == 1 && (rsb % 4) == 0 && (sb_b % 4) == 0 && (n % 4) == 0 && aligned(B, 4 * es);
    const bool c_ok = csc == 1;
    if (a_ok && (nt || nn) && c_ok) {
        GemmArgs g{};
        g.A = A; g.B = B; g.C = C;
        g.m = m; g.n = n; g.k = k;
        g.rsa = rsa; g.rsb = rsb; g.csb = csb; g.rsc = rsc;
        g.sa_b = sa_b; g.sb_b = sb_b; g.sc_b = sc_b;
        g.alpha = alpha; g.beta = beta;
        g.c_vec_ok = (rsc % 4 == 0) && (sc_b % 4 == 0) && aligned(C, 4 * sizeof(oraw));
        g.c_line_ok = sizeof(oraw) == 2 && (rsc % 8 == 0) && (sc_b % 8 == 0) && aligned(C, 16);
        if (m <= SKINNY_M) {
            if (nt) {
                GemvArgs v{};
                v.A = A; v.lda = rsa; v.W = B; v.ldw = csb; v.C = C; v.ldc = rsc;
                v.sa_b = sa_b; v.sw_b = sb_b; v.sc_b = sc_b;
                v.m = m; v.n = n; v.k = k; v.alpha = alpha; v.beta = beta;
                return gemv_dispatch(0, T::code, TO::code, v, batch, s);
            }
            if (m == 1 && (n % VEC) == 0 && (rsb % VEC) == 0 && (sb_b % VEC) == 0 && aligned(B, 16)) {
                auto tiles = [&](int cpr) { return (int64_t)((n + cpr * VEC - 1) / (cpr * VEC)) * batch; };
                // >= 192 workgroups: (1, 3072, 1024) 8.0 us with 96 workgroups of 32
                // columns, 7.1 us with 192 of 16 (XCD-remapped, lines shared in L2)
                if (tiles(8) >= 192)
                    gemv_nn_kernel<T, TO, 8><<<dim3((n + 8 * VEC - 1) / (8 * VEC), batch), 1024, 0, s>>>(g);
                else if (tiles(4) >= 192)
                    gemv_nn_kernel<T, TO, 4><<<dim3((n + 4 * VEC - 1) / (4 * VEC), batch), 1024, 0, s>>>(g);
                else
                    gemv_nn_kernel<T, TO, 2><<<dim3((n + 2 * VEC - 1) / (2 * VEC), batch), 1024, 0, s>>>(g);
                return status_of(hipGetLastError());
            }
            // 2..16 rows of a row-major, 16-bit B: the MFMA DMA path (one partial
            // 64-row tile per column tile) streams B at full width; the column-per-
            // lane kernel below re-reads A per k and issues 2-byte loads of B
            // ((16, 3072, 1024): ~100 us there)
            if (es == 2 && (k % (8 * VEC)) == 0 && (rsb % VEC) == 0 && (sb_b % VEC) == 0 && (n % 16) == 0 &&
                aligned(B, 16))
                return status_of(launch_dma<T, TO>(g, true, batch, s));
            gemm_skinny_nn_kernel<T, TO><<<dim3((n + 63) / 64, batch), 64 * SKINNY_WAVES, 0, s>>>(g);
            return status_of(hipGetLastError());
        }
        if constexpr (std::is_same_v<T, F32> && std::is_same_v<TO, F32>) {
            // fp32 on the DMA-staged fp32 MFMA kernel: k a multiple of its 32-wide
            // step, 16-byte aligned rows of A and of B (NT) or B's k-rows (NN)
            const bool f_nn = nn && (rsb % 4) == 0 && (sb_b % 4) == 0 && aligned(B, 16) && n >= 4;
            if (k % 32 == 0 && (nt || f_nn)) {
                auto ntiles = [&](int bm, int bn) { return (int64_t)((m + bm - 1) / bm) * ((n + bn - 1) / bn) * batch; };
                const bool big = ntiles(128, 128) >= 512;
                GemmArgs f = g;
                f.tiles_m = (m + (big ? 127 : 63)) / (big ? 128 : 64);
                f.tiles_n = (n + (big ? 127 : 63)) / (big ? 128 : 64);
                const dim3 grid(f.tiles_m * f.tiles_n, batch);
                // 1024^3 (256 tiles of 64 x 64): 8 waves of 32 x 16 and a 4-step ring,
                // 99 TFLOP/s NN; 4 waves or 3 steps 86-98, 32 x 64 or 64 x 128 tiles <= 92
                if (big) {
                    if (f_nn) gemm_f32_kernel<128, 128, 2, 4, true, 3><<<grid, 512, 0, s>>>(f);
                    else gemm_f32_kernel<128, 128, 2, 4, false, 3><<<grid, 512, 0, s>>>(f);
                } else {
                    if (f_nn) gemm_f32_kernel<64, 64, 2, 4, true, 4><<<grid, 512, 0, s>>>(f);
                    else gemm_f32_kernel<64, 64, 2, 4, false, 4><<<grid, 512, 0, s>>>(f);
                }
                return status_of(hipGetLastError());
            }
        }
        // DMA-staged fast path: whole k steps, 16-byte aligned rows everywhere.
        const bool dma_k = (k % (8 * VEC)) == 0;
        const bool dma_nt = nt;
        const bool dma_nn = nn && es == 2 && (rsb % VEC) == 0 && (sb_b % VEC) == 0 && (n % 16) == 0 &&
                            aligned(B, 16);
        if (dma_k && (dma_nt || dma_nn)) return status_of(launch_dma<T, TO>(g, nn, batch, s));
        return status_of(launch_mfma<T, TO>(g, nn, batch, s));
    }
    GenericArgs g{A, B, C, m, n, k, rsa, csa, rsb, csb, rsc, csc, sa_b, sb_b, sc_b, alpha, beta};
    return status_of(launch_generic<T, TO>(g, batch, s));
}

}  // namespace

int gemm_dispatch(int dtype_in, int dtype_out, int batch, int m, int n, int k, const void* A, int64_t sa_b,
                  int64_t rsa, int64_t csa, const void* B, int64_t sb_b, int64_t rsb, int64_t csb, void* C,
                  int64_t sc_b, int64_t rsc, int64_t csc, float alpha, float beta, hipStream_t s) {
#define YTHIP_GEMM(TI, TOUT) \
    return gemm_typed<TI, TOUT>(batch, m, n, k, A, sa_b, rsa, csa, B, sb_b, rsb, csb, C, sc_b, rsc, csc, alpha, beta, s)
    if (dtype_in == YTHIP_F32 && dtype_out == YTHIP_F32) YTHIP_GEMM(F32, F32);
    if (dtype_in == YTHIP_BF16 && dtype_out == YTHIP_BF16) YTHIP_GEMM(BF16, BF16);
    if (dtype_in == YTHIP_BF16 && dtype_out == YTHIP_F32) YTHIP_GEMM(BF16, F32);
    if (dtype_in == YTHIP_F16 && dtype_out == YTHIP_F16) YTHIP_GEMM(F16, F16);
    if (dtype_in == YTHIP_F16 && dtype_out == YTHIP_F32) YTHIP_GEMM(F16, F32);
#undef YTHIP_GEMM
    return fail(YTHIP_EUNSUPPORTED, "ythip_gemm: unsupported dtype_in/dtype_out combination %d/%d", dtype_in,
                dtype_out);
}

}  // namespace ythip
