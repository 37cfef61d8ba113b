// common.hpp — shared device types and helpers for the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/ythip.h"

namespace ythip {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Storage tags: the kernels move 16-bit data as raw uint16_t bits and convert
// explicitly, so that the rounding is the one written here.
struct BF16 { using raw = uint16_t; static constexpr int code = YTHIP_BF16; };
struct F16 { using raw = uint16_t; static constexpr int code = YTHIP_F16; };
struct F32 { using raw = float; static constexpr int code = YTHIP_F32; };

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// fp32 -> bf16 with the gfx950 converter (v_cvt_pk_bf16_f32): IEEE
// round-to-nearest-even, NaN stays NaN.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    _Float16 x = __builtin_bit_cast(_Float16, static_cast<uint16_t>(h));
    return static_cast<float>(x);
}
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
    _Float16 x = static_cast<_Float16>(f);  // v_cvt_f16_f32: RNE
    return __builtin_bit_cast(uint16_t, x);
}

template <class T> __device__ __forceinline__ float load_as_f32(const void* p, int64_t i);
template <> __device__ __forceinline__ float load_as_f32<F32>(const void* p, int64_t i) {
    return static_cast<const float*>(p)[i];
}
template <> __device__ __forceinline__ float load_as_f32<BF16>(const void* p, int64_t i) {
    return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
}
template <> __device__ __forceinline__ float load_as_f32<F16>(const void* p, int64_t i) {
    return f16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
}

template <class T> __device__ __forceinline__ void store_from_f32(void* p, int64_t i, float v);
template <> __device__ __forceinline__ void store_from_f32<F32>(void* p, int64_t i, float v) {
    static_cast<float*>(p)[i] = v;
}
template <> __device__ __forceinline__ void store_from_f32<BF16>(void* p, int64_t i, float v) {
    static_cast<uint16_t*>(p)[i] = static_cast<uint16_t>(f32_to_bf16_bits(v));
}
template <> __device__ __forceinline__ void store_from_f32<F16>(void* p, int64_t i, float v) {
    static_cast<uint16_t*>(p)[i] = static_cast<uint16_t>(f32_to_f16_bits(v));
}

template <class T> __device__ __forceinline__ uint32_t pack2(float a, float b);
// Two fp32 -> one packed 16-bit pair (low half = a), one conversion instruction.
template <> __device__ __forceinline__ uint32_t pack2<BF16>(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{a, b}), bf16x2_t));
}
template <> __device__ __forceinline__ uint32_t pack2<F16>(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{a, b}), f16x2_t));
}

__device__ __forceinline__ float lo_as_f32(BF16, uint32_t w) { return bf16_bits_to_f32(w & 0xffffu); }
__device__ __forceinline__ float hi_as_f32(BF16, uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float lo_as_f32(F16, uint32_t w) { return f16_bits_to_f32(w & 0xffffu); }
__device__ __forceinline__ float hi_as_f32(F16, uint32_t w) { return f16_bits_to_f32(w >> 16); }

// MFMA on one 16-byte operand chunk per lane, 16x16 fp32 output tile.
//   16-bit: one v_mfma_f32_16x16x32_{bf16,f16}: lane l supplies row (l%16) and
//           k = 8*(l/16) + 0..7 of the 32-wide k block.
//   fp32  : four v_mfma_f32_16x16x4_f32, lane l supplies row (l%16) and
//           k = 4*(l/16) + j on step j; together the 16 k of the block.
// Any k assignment is valid as long as both operands use the same one.
__device__ __forceinline__ f32x4 mfma_chunk(BF16, u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_chunk(F16, u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
}
__device__ __forceinline__ f32x4 mfma_chunk(F32, u32x4 a, u32x4 b, f32x4 c) {
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a[0]), __uint_as_float(b[0]), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a[1]), __uint_as_float(b[1]), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a[2]), __uint_as_float(b[2]), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a[3]), __uint_as_float(b[3]), c, 0, 0, 0);
    return c;
}

// Tile order of the GEMM grids, XCD-aware: the hardware places workgroup w on
// XCD w % 8, so (when the tile count is a multiple of 8) w is remapped to give
// each XCD a contiguous range of tiles, taken 4 tile-rows at a time so that an
// XCD's L2 holds the A panels its 32 CUs reuse.
__device__ __forceinline__ void tile_coords(int w, int tiles_m, int tiles_n, int& tm, int& tn) {
    const int T = tiles_m * tiles_n;
    if ((T & 7) == 0) {
        const int per = T >> 3;
        w = (w & 7) * per + (w >> 3);
    }
    constexpr int GROUP = 4;
    const int in_group = GROUP * tiles_n;
    const int g = w / in_group;
    const int first = g * GROUP;
    const int gsize = min(tiles_m - first, GROUP);
    const int r = w - g * in_group;
    tm = first + r % gsize;
    tn = r / gsize;
}

// Wait until at most N vector-memory operations of this wave are outstanding
// (gfx9 s_waitcnt encoding: vmcnt in bits 3:0 and 15:14; expcnt and lgkmcnt
// left at their "no wait" maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// gfx950 LDS data movers. The builtins exist only for the device target; the
// host compilation pass of a kernel that names them directly drops the kernel's
// launch stub, so they are wrapped here and compiled in the device pass only.
typedef short v4i16 __attribute__((ext_vector_type(4)));

// global -> LDS DMA of 16 bytes per lane: lane i's 16 bytes land at
// lds_wave_base + 16*i (lds_wave_base is wave-uniform).
__device__ __forceinline__ void dma16(const void* gsrc, void* lds_wave_base) {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_global_load_lds(gsrc, lds_wave_base, 16, 0, 0);
#endif
}

// The same DMA issued through inline asm. The compiler does not model an asm
// DMA, so it keeps using partial lgkmcnt waits for the ds_reads that follow
// (with the builtin it falls back to lgkmcnt(0) after every read, which
// serialises the LDS fragment loads with the MFMAs). Callers order the DMA with
// explicit vmcnt waits and barriers.
__device__ __forceinline__ void dma16_async(const void* gsrc, void* lds_wave_base) {
#if defined(__HIP_DEVICE_COMPILE__)
    const uint32_t l = (uint32_t)(uintptr_t)lds_wave_base;
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off"
                 :
                 : "v"(gsrc), "s"(__builtin_amdgcn_readfirstlane(l))
                 : "memory", "m0");
#else
    (void)gsrc; (void)lds_wave_base;
#endif
}

// The same DMA from a wave-uniform base (scalar registers) plus this lane's
// 32-bit byte offset, i.e. global_load_lds's scalar-base form: a caller that
// keeps the offsets fixed across a loop and moves only the base (and the LDS
// destination, both scalar) issues its DMA with no per-load VALU address
// arithmetic. lds_wave_base is the LDS byte address of lane 0's 16 bytes.
__device__ __forceinline__ void dma16_soff(const void* sbase, uint32_t voff, uint32_t lds_wave_base) {
#if defined(__HIP_DEVICE_COMPILE__)
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1"
                 :
                 : "v"(voff), "s"(sbase), "s"(lds_wave_base)
                 : "memory", "m0");
#else
    (void)sbase; (void)voff; (void)lds_wave_base;
#endif
}

// ds_read_b64_tr_b16: within each 16-lane group, lane j supplies the LDS byte
// address of 4 consecutive 16-bit values R[j][0..3]; lane i receives
// { R[4t + i/4][i%4] : t = 0..3 }.
__device__ __forceinline__ u32x2 lds_read_tr16(const void* lds, int byte_off) {
#if defined(__HIP_DEVICE_COMPILE__)
    typedef __attribute__((address_space(3))) v4i16 lds_v4i16_t;
    typedef __attribute__((address_space(3))) char lds_char_t;
    const v4i16 t = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)((lds_char_t*)lds + byte_off));
    return __builtin_bit_cast(u32x2, t);
#else
    (void)lds; (void)byte_off;
    return u32x2{0u, 0u};
#endif
}

// Butterfly sum over the 64 lanes of a wave (every lane gets the total).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// Sum / max over the 64 lanes with DPP row operations (quad swaps, half-row and
// row mirrors, then the row broadcasts of gfx9): the result lands in lane 63.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add(float v) {
    return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_max(float v) {
    const int ninf = __float_as_int(-INFINITY);  // rows the broadcast skips see -inf
    return fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(ninf, __float_as_int(v), CTRL, ROW_MASK, 0xf, false)));
}
__device__ __forceinline__ float dpp_sum_to_lane63(float v) {
    v = dpp_add<0xb1, 0xf>(v);   // quad_perm [1,0,3,2]
    v = dpp_add<0x4e, 0xf>(v);   // quad_perm [2,3,0,1]
    v = dpp_add<0x141, 0xf>(v);  // row_half_mirror
    v = dpp_add<0x140, 0xf>(v);  // row_mirror
    v = dpp_add<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
    v = dpp_add<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
    return v;
}
__device__ __forceinline__ float dpp_max_to_lane63(float v) {
    v = dpp_max<0xb1, 0xf>(v);
    v = dpp_max<0x4e, 0xf>(v);
    v = dpp_max<0x141, 0xf>(v);
    v = dpp_max<0x140, 0xf>(v);
    v = dpp_max<0x142, 0xa>(v);
    v = dpp_max<0x143, 0xc>(v);
    return v;
}
// Maximum over lanes l, l^16, l^32, l^48 (the four 16-lane rows of a wave),
// every lane getting the result: gfx950's v_permlane16_swap / v_permlane32_swap
// exchange rows inside the VALU (no LDS round trip). IEEE maximum: a NaN
// propagates, -inf is the identity.
__device__ __forceinline__ float max_across_rows(float v) {
    const uint32_t u = __float_as_uint(v);
    const auto p16 = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    v = __builtin_elementwise_maximum(__uint_as_float(p16[0]), __uint_as_float(p16[1]));
    const uint32_t w = __float_as_uint(v);
    const auto p32 = __builtin_amdgcn_permlane32_swap(w, w, false, false);
    return __builtin_elementwise_maximum(__uint_as_float(p32[0]), __uint_as_float(p32[1]));
}

// Sum over aligned groups of N = 8 or 16 lanes, every lane of a group getting
// its group's total (DPP: quad swaps, half-row mirror, then a rotate by 8 within
// the 16-lane row).
template <int N>
__device__ __forceinline__ float dpp_sum_group(float v) {
    static_assert(N == 8 || N == 16, "8- or 16-lane groups");
    auto dpp = [](float x, auto ctrl) {
        return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), decltype(ctrl)::value, 0xf, 0xf, false));
    };
    v += dpp(v, std::integral_constant<int, 0xb1>{});   // quad_perm [1,0,3,2]
    v += dpp(v, std::integral_constant<int, 0x4e>{});   // quad_perm [2,3,0,1]
    v += dpp(v, std::integral_constant<int, 0x141>{});  // row_half_mirror
    if constexpr (N == 16) v += dpp(v, std::integral_constant<int, 0x128>{});  // row_ror:8
    return v;
}

// The lane-63 result as a wave-uniform value.
__device__ __forceinline__ float lane63(float v) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63)); }

// Compile-time loop: f(std::integral_constant<int, i>) for i in [B, E).
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

// Elements per 16-byte chunk.
template <class T> struct Vec { static constexpr int n = 16 / sizeof(typename T::raw); };

// Decode-state record (include/ythip.h, ythip_decode_state_field): derive the
// next token's cache row, visible key count and RoPE row from TOTAL, the ring
// size and max_position_embeddings, as KVCache::append / get_mask and
// Qwen3Model::forward's start rule do (example/qwen3/src/qwen3.cpp:70-126,
// 365-375) for a one-token step.
__host__ __device__ inline void decode_state_derive(int32_t* st) {
    const int T = st[YTHIP_ST_TOTAL], L = st[YTHIP_ST_RING], P = st[YTHIP_ST_MAX_POS];
    const int cur = T < L ? T : L;  // KVCache::cur_len before the append
    st[YTHIP_ST_SLOT] = L > 0 ? T % L : 0;
    st[YTHIP_ST_KV_LEN] = T + 1 < L ? T + 1 : L;
    st[YTHIP_ST_ROPE_POS] = T + 1 <= P ? T : (cur + 1 <= P ? cur : 0);
}

// The argmax step's update (one thread): the token just run was written to the
// cache; record the new token and advance to the next one.
__device__ inline void decode_state_advance(int32_t* st, int32_t* history, int token) {
    const int g = st[YTHIP_ST_GENERATED];
    if (history != nullptr) {
        if (g >= 0 && g < st[YTHIP_ST_HISTORY]) history[g] = token;
        else st[YTHIP_ST_ERROR] |= YTHIP_ST_ERR_HISTORY;
    }
    st[YTHIP_ST_GENERATED] = g + 1;
    st[YTHIP_ST_TOTAL] += 1;
    decode_state_derive(st);
}

// Split-K decode partition. The grid holds `splits` workgroups per (batch, kv
// head), sized for the cache's capacity; the keys visible at run time, len,
// are cut into chunks of len / splits keys (rounded up), at least
// DEC_MIN_CHUNK, so a short context in a large ring fills only the first few
// splits with full chunks and the merges read only those. Splits past the last
// used one hold empty partials (m = -inf, l = 0, o = 0).
constexpr int DEC_MIN_CHUNK = 128;
__host__ __device__ inline int decode_chunk(int len, int splits) {
    const int c = splits > 0 ? (len + splits - 1) / splits : len;
    return c > DEC_MIN_CHUNK ? c : DEC_MIN_CHUNK;
}
// splits holding keys (at least 1, at most splits)
__host__ __device__ inline int decode_used(int len, int splits) {
    if (len <= 0) return 1;
    const int c = decode_chunk(len, splits), u = (len + c - 1) / c;
    return u < splits ? u : (splits > 0 ? splits : 1);
}

}  // namespace ythip
