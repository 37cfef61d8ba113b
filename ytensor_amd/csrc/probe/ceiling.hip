// ceiling.hip — roofline probes for the headline bf16 GEMM (4096^3 NN on the
// 256 x 256 ping-pong kernel of gemm.hip). Built into libythip_probe.so, apart
// from the product library: bench.py and the tests load it to measure the two
// resources that bound the GEMM, each alone, with the GEMM's grid, workgroup
// shape and per-CU work.
//
//   ceiling_mfma_kernel  the GEMM's MFMA stream on operands held in registers:
//     per wave, `steps` k steps of 64 v_mfma_f32_16x16x32_bf16 into 32 16x16
//     fp32 accumulators (a 128 x 64 wave tile, operands swapped as in the GEMM),
//     8 waves per workgroup, one workgroup per CU. No LDS and no memory traffic
//     in the loop, full-entropy operands (each MFMA takes a different A/B
//     pair), so its rate is what the matrix cores sustain under that power load.
//     The epilogue is the GEMM's: the wave tile rounded to bf16 with one 8-byte
//     store per fragment row (2048 waves x 16 KiB = the 32 MiB of a 4096^2 C).
//     out[w] = bf16(steps * A_w . B_w^T) for wave w (A_w [128][64], B_w
//     [64][64] given as [n][k]).
//   ceiling_dma_kernel  the GEMM's operand stream for an NN product: per 64-wide
//     k step, waves 0-3 move A's 256 x 64 and B's 64 x 256 bf16 slices (64 KiB)
//     global -> LDS with global_load_lds_dwordx4 from a scalar base plus fixed
//     lane offsets, into one of two 64 KiB stages, wait for them, and the
//     workgroup meets at one barrier; tiles in the GEMM's XCD-aware order. No
//     LDS reads and no MFMA in the loop: the L2 -> LDS delivery floor of the
//     GEMM's one-burst-per-step schedule. Each workgroup then sums its 128 KiB
//     of LDS (the last two k steps) as 32-bit words per 16-byte lane slot and
//     writes one u32x4 per thread, so a test can check the bytes that landed.
//
// C ABI (no header under include/: this library is measurement support, not
// part of the boundary):
//   int ythip_probe_mfma(const void* A, const void* B, void* out,
//                        int workgroups, int steps, void* stream);
//   int ythip_probe_dma(const void* A, const void* B, int m, int n, int k,
//                       void* out, void* stream);
// Return 0, -1 for invalid arguments (nothing launched), -3 for a HIP launch
// error.

#include "../common.hpp"

namespace ythip {
namespace {

__global__ __launch_bounds__(512, 1) void ceiling_mfma_kernel(const uint16_t* __restrict__ A,
                                                              const uint16_t* __restrict__ B,
                                                              uint16_t* __restrict__ out, int steps) {
    constexpr int FM = 8, FN = 4;
    const int lane = threadIdx.x & 63, lrow = lane & 15, lgrp = lane >> 4;
    const int64_t w = (int64_t)blockIdx.x * 8 + (threadIdx.x >> 6);
    const uint16_t* a = A + w * (128 * 64);
    const uint16_t* b = B + w * (64 * 64);
    // the GEMM's fragment layout: lane l holds row l % 16 of a 16-row block and
    // k = 8 * (l / 16) .. + 7 of a 32-wide k chunk
    u32x4 fa[2][FM], fb[2][FN];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
            fa[ks][i] = *reinterpret_cast<const u32x4*>(a + (i * 16 + lrow) * 64 + (ks * 4 + lgrp) * 8);
#pragma unroll
        for (int j = 0; j < FN; ++j)
            fb[ks][j] = *reinterpret_cast<const u32x4*>(b + (j * 16 + lrow) * 64 + (ks * 4 + lgrp) * 8);
    }
    f32x4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < steps; ++s) {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j) acc[i][j] = mfma_chunk(BF16{}, fb[ks][j], fa[ks][i], acc[i][j]);
    }
    // lane l holds C[i*16 + l % 16][j*16 + 4*(l / 16) + r], r = 0..3
    uint16_t* o = out + w * (128 * 64);
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
            *reinterpret_cast<u32x2*>(o + (i * 16 + lrow) * 64 + j * 16 + lgrp * 4) =
                u32x2{pack2<BF16>(acc[i][j][0], acc[i][j][1]), pack2<BF16>(acc[i][j][2], acc[i][j][3])};
}

__global__ __launch_bounds__(512, 1) void ceiling_dma_kernel(const uint16_t* __restrict__ A,
                                                             const uint16_t* __restrict__ B, int n, int k,
                                                             int tiles_m, int tiles_n, u32x4* __restrict__ out) {
    constexpr int BM = 256, BN = 256, BK = 64, GT = 256;
    constexpr int STA = BM * 8;          // A stage: 256 rows x 8 16-byte chunks
    constexpr int STB = BK * (BN / 8);   // B stage: 64 k-rows x 32 16-byte chunks
    constexpr int A_PT = STA / GT, B_PT = STB / GT;
    __shared__ u32x4 sbuf[2 * (STA + STB)];
    const int tid = threadIdx.x, wave = tid >> 6;
    int tm, tn;
    tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int KT = k / BK;
    if (wave < 4) {
        // slot i*256 + t of a stage: A row i*32 + t/8, chunk t%8; B k-row i*8 + t/32, chunk t%32
        const int t = tid;
        const uint32_t offA = (uint32_t)((((int64_t)(t >> 3)) * k + (t & 7) * 8) * 2);
        const uint32_t offB = (uint32_t)((((int64_t)(t >> 5)) * n + (t & 31) * 8) * 2);
        const uint32_t ldsA = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)&sbuf[wave * 64]);
        const uint32_t ldsB = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)&sbuf[2 * STA + wave * 64]);
        const char* a0 = reinterpret_cast<const char*>(A + (int64_t)m0 * k);
        const char* b0 = reinterpret_cast<const char*>(B + n0);
        for (int kt = 0; kt < KT; ++kt) {
            const uint32_t st = (uint32_t)(kt & 1);
            const char* bA = a0 + (int64_t)kt * BK * 2;
#pragma unroll
            for (int i = 0; i < A_PT; ++i)
                dma16_soff(bA + (int64_t)i * 32 * k * 2, offA, ldsA + (st * STA + (uint32_t)i * GT) * 16u);
            const char* bB = b0 + (int64_t)kt * BK * n * 2;
#pragma unroll
            for (int i = 0; i < B_PT; ++i)
                dma16_soff(bB + (int64_t)i * 8 * n * 2, offB, ldsB + (st * STB + (uint32_t)i * GT) * 16u);
            wait_vmcnt<0>();  // this wave's 16 DMAs of the step have landed
            __builtin_amdgcn_s_barrier();
        }
    } else {
        for (int kt = 0; kt < KT; ++kt) __builtin_amdgcn_s_barrier();
    }
    u32x4 s = u32x4{0u, 0u, 0u, 0u};
    for (int i = tid; i < 2 * (STA + STB); i += 512) s += sbuf[i];
    out[(int64_t)blockIdx.x * 512 + tid] = s;
}

}  // namespace
}  // namespace ythip

using namespace ythip;

extern "C" __attribute__((visibility("default"))) int ythip_probe_mfma(const void* A, const void* B, void* out,
                                                                       int workgroups, int steps, void* stream) {
    if (!A || !B || !out || workgroups < 1 || workgroups > 65535 || steps < 1) return -1;
    ceiling_mfma_kernel<<<workgroups, 512, 0, (hipStream_t)stream>>>(static_cast<const uint16_t*>(A),
                                                                      static_cast<const uint16_t*>(B),
                                                                      static_cast<uint16_t*>(out), steps);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

extern "C" __attribute__((visibility("default"))) int ythip_probe_dma(const void* A, const void* B, int m, int n,
                                                                      int k, void* out, void* stream) {
    if (!A || !B || !out || m < 256 || n < 256 || k < 128 || m % 256 || n % 256 || k % 64) return -1;
    const int64_t tiles = (int64_t)(m / 256) * (n / 256);
    // lane offsets are 32-bit: 31 rows of A (k elements each) and 7 k-rows of B (n each)
    if (tiles > 65535 || (31 * (int64_t)k + 64) * 2 >= (int64_t)1 << 32 || (7 * (int64_t)n + 256) * 2 >= (int64_t)1 << 32)
        return -1;
    ceiling_dma_kernel<<<(unsigned)tiles, 512, 0, (hipStream_t)stream>>>(
        static_cast<const uint16_t*>(A), static_cast<const uint16_t*>(B), n, k, m / 256, n / 256,
        static_cast<u32x4*>(out));
    return hipGetLastError() == hipSuccess ? 0 : -3;
}
