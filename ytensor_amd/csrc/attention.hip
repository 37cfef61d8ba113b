// attention.hip — attention forward for gfx950: MFMA flash-attention prefill,
// split-context decode, and an any-layout row-wise kernel.
//
// Reference semantics (src/kernel/avx2/flash_attention.inl):
//   prefill 274-443: blockwise online softmax over key tiles, masked entries
//   excluded (not -1e9), bias added after scaling, rows with no visible key
//   give 0 (327-331); decode 202-272: scores, max, exp, sum, normalise, P.V.
//   GQA as in the qwen3 example (example/qwen3/src/qwen3.cpp:250-264): query
//   head h reads key/value head h / (Hq / Hkv).
//
// Prefill kernel (16-bit inputs, d in {64, 128}):
//   * Workgroup = 4 waves x 32 queries = 128 queries of one (batch, head);
//     key/value blocks of 64 keys double-buffered in LDS. Short prompts take
//     16 queries per wave, and without a staged mask 8 waves splitting each
//     128-key stage in two halves merged at the end; long ones with an even
//     GQA group the paired-head ping-pong kernel.
//   * S^T = K . Q^T on v_mfma_f32_16x16x32: src0 = K rows, src1 = Q rows, so
//     lane l holds 16 scores of ONE query (l % 16) -> the online softmax is
//     lane-local plus two cross-group shuffles (xor 16, 32) for the max.
//   * O^T = V^T . P^T: src0 = V^T rows (d), src1 = P (the lane's own
//     probabilities, packed to 16-bit), so each lane's accumulators belong to
//     its own query and the rescale is a per-lane scalar. V is transposed to
//     [d][key] on its way into LDS (4 keys x 8 d per thread).
//   * exp2 with log2(e) folded into the scale (exp(x) = 2^(x*log2 e)).
//   * Causal: heaviest query blocks launch first; key blocks past the diagonal
//     are never loaded; waves skip blocks entirely in their future.
// Decode kernel: one workgroup per (batch, kv head, context split) serves all
//   G = Hq/Hkv query heads of the group, so each K/V byte is read once;
//   16 lanes per key (8 elements each), DPP/shuffle dot-product reduction,
//   per-lane online softmax, then a cross-slot merge in LDS; a second kernel
//   merges the splits (log-sum-exp).

#include <algorithm>
#include <mutex>
#include <cfloat>

#include "common.hpp"
#include "launch.hpp"

namespace ythip {

constexpr float LOG2E = 1.4426950408889634f;

struct AttnArgs {
    const void* Q;
    const void* K;
    const void* V;
    void* O;
    int64_t qs0, qs1, qs2, ks0, ks1, ks2, vs0, vs1, vs2, os0, os1, os2;
    int64_t qs3, ks3, vs3, os3;  // element strides along d (1 on the MFMA path)
    int B, Hq, Hkv, Sq, Skv, D, Dv;
    int diag_off;  // causal / diagonal masks: key j visible to query i iff j <= i + diag_off
    float scale_log2;  // scale * log2(e)
    const uint8_t* mask;
    int64_t mask_ld;
    int causal;
    const float* bias;
    int64_t brs, bcs;
    int nqb;
    int balance;  // causal: the grid is resident at once, two workgroups per CU (see attn_fwd_mfma)
    uint8_t* tcls;        // byte mask's tile classes (mask_tile_class_kernel), or null
    int nkbt;             // 64-key blocks of the mask rows: ceil(Skv / 64)
    int o_line;           // O: unit d stride, 16-byte aligned base, rows and heads
    int mask_words;       // byte mask, no bias, 4-byte aligned base and rows (attn_fwd_f32)
};

// MODE 0: no mask; 1: causal; 2: byte mask and/or bias read per element;
// 3: byte mask staged per key block: the block's [BQ x BKV] mask tile is DMA'd
// into LDS with K and V (16-byte aligned rows, full key blocks; the last,
// partial block reads its bytes directly), each wave skips a block none of
// whose keys its rows see, drops the per-score masking in a block its rows
// see whole, and otherwise takes visibility from the LDS tile (the bool-mask
// call of src/kernel/avx2/flash_attention.inl:335-379 with the tile tests of
// 14-49).
// GH query heads of one GQA group share a workgroup (4 waves per head, 32
// queries per wave), so each K/V tile is staged once for GH*128 queries; the
// mask (one per query/key pair, the same for every head) then serves both.
// K and V tiles reach LDS by DMA (global_load_lds, 16 bytes per lane), both
// kept in their natural [key][d] layout:
//   K rows: 16-byte chunk c stored at c ^ (key & KMASK) -> the S^T operand is
//           one conflict-free ds_read_b128 per lane.
//   V rows: 32-byte block b stored at b ^ (key & BMASK) and read transposed by
//           ds_read_b64_tr_b16: lane j of a 16-lane group addresses 4 d-values
//           of key (kt*16 + 4*grp + j/4); lane i receives d = i of 4 keys,
//           i.e. the V^T operand in the key order P was packed in.
// Workgroup order: the hardware deals workgroups to the 8 XCDs round-robin;
// the linear id is remapped so each XCD walks a contiguous range of
// (kv head, query block) pairs -- one KV head's K/V stays in one XCD's L2 --
// and, for causal masks, the longest query blocks start first.
// KSPLIT = 2 (one head per workgroup, no staged mask): 8 waves serve the same
// query block, each stage holds 2 * BKV keys, waves 0-3 take its first BKV
// keys and waves 4-7 the second, each with its own online softmax; at the end
// waves 4-7 hand O, l and m to waves 0-3 through LDS, which merge them
// (O = a0 O0 + a1 O1, l likewise, a = 2^(m - max m)). Short prompts use it:
// the longest query block's serial chain of key blocks is halved.
template <class T, int D, int MODE, int GH, int QT, int NKT = 4, int KSPLIT = 1>
__global__ __launch_bounds__(256 * GH * KSPLIT, 2 / (GH * KSPLIT)) void attn_fwd_mfma(AttnArgs a) {
    using raw = typename T::raw;
    static_assert(KSPLIT == 1 || (KSPLIT == 2 && GH == 1 && MODE != 3), "key split: one head, no staged mask");
    constexpr int THREADS = 256 * GH * KSPLIT;
    constexpr int WQ = 16 * QT, BQ = 4 * WQ, BKV = 16 * NKT;  // QT 16-query tiles per wave, NKT 16-key tiles per block
    constexpr int SBKV = BKV * KSPLIT;  // keys per stage
    constexpr int KCH = D / 8;    // 16-byte chunks per K/V row
    constexpr int DT = D / 16;    // output d tiles
    constexpr int KS = D / 32;    // d steps of the score MFMA
    constexpr int PT = SBKV * KCH / THREADS;
    static_assert(PT * THREADS == SBKV * KCH, "tile / thread mismatch");
    constexpr int NB = D / 16;    // 32-byte blocks per V row
    constexpr int BMASK = (NB < 8 ? NB : 8) - 1;
    constexpr int STG = SBKV * KCH;  // u32x4 slots per stage
    // K chunk swizzle: with D = 128 a K row is one full 256-byte bank window, so
    // 16 consecutive keys XOR their chunk index with key & 15 and a fragment read
    // (16 keys, one logical chunk) touches all 64 banks once.
    constexpr int KMASK = KCH - 1 < 15 ? KCH - 1 : 15;
    __shared__ u32x4 sK[2 * STG];
    __shared__ u32x4 sV[2 * STG];
    constexpr int MCH = BKV / 16;                 // MODE 3: 16-byte mask chunks per row of a block
    constexpr int MSTG = BQ * MCH;                // mask chunks per stage
    constexpr int MPT = MSTG / THREADS;
    static_assert(MODE != 3 || MPT * THREADS == MSTG, "mask tile / thread mismatch");
    // SKIP (staged mask, paired heads): the mask tiles run MAHEAD = 6 blocks
    // ahead in a ring of 8, each wave tests block kb+2 during step kb and
    // publishes whether its rows see a key, and after step kb's barrier the
    // workgroup stages K/V(kb+1) only if some wave does -- an all-false block
    // costs a tile test and a barrier, no K/V DMA and no MFMA, and no wait on a
    // DMA of its own step.
    constexpr bool SKIP = MODE == 3 && GH == 2;
    constexpr int MAHEAD = 6;
    constexpr int MRING = SKIP ? 8 : 2;
    static_assert(!SKIP || THREADS == 512, "one flag byte per wave, 8 waves");
    __shared__ u32x4 sM[MODE == 3 ? MRING * MSTG : 1];
    __shared__ uint64_t sflag[SKIP ? 2 : 1];
    auto mslot = [](int kb) { return kb & (MRING - 1); };

    // (batch, kv head or head pair, query block) from the XCD-remapped id.
    const int G = a.Hq / a.Hkv;
    const int hgroups = G / GH;                 // head groups per kv head
    const int units = a.B * a.Hkv * hgroups;    // (b, kvh, head group) units
    const int total = units * a.nqb;
    int w = blockIdx.x;
    if ((total & 7) == 0) w = (w & 7) * (total >> 3) + (w >> 3);
    const int unit = w / a.nqb;
    const int qi = w % a.nqb;
    // Causal work grows with the query block; heaviest blocks launch first. When
    // the whole grid is resident at once with two workgroups per CU (balance),
    // CU k holds workgroups k and k + total/2, which the remap above gives the
    // same query block of units u and u + 1 (u even) whenever total / 8 is a
    // multiple of nqb: odd units then take their blocks lightest first, so such
    // a CU pairs a heavy block with a light one. Per unit the order stays a
    // permutation of its query blocks.
    const bool light_first = a.balance && (unit & 1);
    // the staged-mask kernel also starts from the last query block: in
    // causal-shaped masks (the KV ring's included) later rows see more keys
    // (S=2048 causal as bytes, one head per workgroup: 48.8 -> 45.4 us)
    constexpr bool HEAVY_FIRST = MODE == 1 || MODE == 3;
    const int qb = (HEAVY_FIRST && !light_first) ? (a.nqb - 1 - qi) : qi;
    const int b = unit / (a.Hkv * hgroups);
    const int rem = unit % (a.Hkv * hgroups);
    const int kvh = rem / hgroups;
    // the wave index made scalar: per-wave tests are then scalar branches
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = KSPLIT == 2 ? (wave >> 2) : 0;  // key half of each stage
    const int h = kvh * G + (rem % hgroups) * GH + (KSPLIT == 1 ? (wave >> 2) : 0);
    const int l16 = lane & 15, g = lane >> 4;
    const int q0 = qb * BQ + (wave & 3) * WQ;

    const raw* Qp = static_cast<const raw*>(a.Q) + b * a.qs0 + h * a.qs1;
    const raw* Kp = static_cast<const raw*>(a.K) + b * a.ks0 + kvh * a.ks1;
    const raw* Vp = static_cast<const raw*>(a.V) + b * a.vs0 + kvh * a.vs1;

    // Q is pre-scaled by scale*log2(e) and rounded back to T (relative error
    // 2^-9 per element, about 1e-3 on p): the scores then leave the MFMA in
    // log2 units, and since the accumulator starts at -m they leave it as
    // s - m, so p = exp2(s - m) costs one exp per score and no multiply.
    const float c = a.scale_log2;
    u32x4 qf[QT][KS];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const int q = q0 + qt * 16 + l16;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            u32x4 v = {0u, 0u, 0u, 0u};
            if (q < a.Sq) v = *reinterpret_cast<const u32x4*>(Qp + (int64_t)q * a.qs2 + ks * 32 + g * 8);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t w2 = v[e];
                v[e] = pack2<T>(lo_as_f32(T{}, w2) * c, hi_as_f32(T{}, w2) * c);
            }
            qf[qt][ks] = v;
        }
    }

    const int off = a.diag_off;  // causal: key j visible to query i iff j <= i + off
    int kv_end = a.Skv;
    if (MODE == 1) kv_end = min(a.Skv, qb * BQ + BQ + off);
    const int nkb = kv_end > 0 ? (kv_end + SBKV - 1) / SBKV : 0;  // stages

    // m is the reference point of the exponentials (log2 units), set by the
    // first block with a visible key and moved only when a block's max exceeds
    // it by more than 2^8 in probability, so the O rescale is rare; p = 2^(s - m)
    // <= 2^8 stays far from any overflow and the final O / l is independent of m.
    // l is the fourth MFMA output next to O: ones . P^T sums the packed p of
    // every key (the same rounded p that multiplies V), one result per query.
    constexpr float LAZY = 8.0f;
    constexpr uint32_t ONE2 = std::is_same_v<T, BF16> ? 0x3F803F80u : 0x3C003C00u;
    const u32x4 ones = {ONE2, ONE2, ONE2, ONE2};
    float m[QT];
    bool mset[QT];
    f32x4 lsum[QT];
    // per row: the block max above which the reference point moves (any
    // visible key before the first move, LAZY after)
    float thr[QT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        m[qt] = 0.f;
        mset[qt] = false;
        lsum[qt] = f32x4{0.f, 0.f, 0.f, 0.f};
        thr[qt] = -INFINITY;
    }
    f32x4 o[QT][DT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[qt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};

    // This thread's DMA slots within a stage: row and swizzled chunk, as element
    // offsets from the stage's first key (64-row spans are < 2^31 elements).
    auto slot_row = [&](int i) { return (i * THREADS + wave * 64 + lane) / KCH; };
    auto koff = [&](int i) {
        const int slot = i * THREADS + wave * 64 + lane, row = slot / KCH, ps = slot % KCH;
        return row * (int)a.ks2 + (ps ^ (row & KMASK)) * 8;
    };
    auto voff = [&](int i) {
        const int slot = i * THREADS + wave * 64 + lane, row = slot / KCH, ps = slot % KCH;
        return row * (int)a.vs2 + ((ps >> 1) ^ (row & BMASK)) * 16 + (ps & 1) * 8;
    };
    auto issue_mask = [&](int kb) {
        if constexpr (MODE == 3) {
            const int k0 = kb * SBKV;
            if (k0 + BKV <= a.Skv) {
                // mask rows of the query block (clamped to the last query row)
#pragma unroll
                for (int i = 0; i < MPT; ++i) {
                    const int slot = i * THREADS + wave * 64 + lane;
                    const int r = slot / MCH, c = slot % MCH;
                    const int row = min(qb * BQ + r, a.Sq - 1);
                    dma16_async(a.mask + (int64_t)row * a.mask_ld + k0 + c * 16,
                                &sM[mslot(kb) * MSTG + i * THREADS + wave * 64]);
                }
            }
        }
    };
    // Whole stages whose lane offsets fit 31 bits (every layout but huge row
    // strides) go from the stage's scalar base plus this lane's fixed byte
    // offset, kept in registers: no VALU address work per DMA. Other stages
    // recompute the offsets.
    const bool soff = (int64_t)SBKV * (a.ks2 > a.vs2 ? a.ks2 : a.vs2) * (int64_t)sizeof(raw) < (1ll << 31);
    uint32_t kbo[PT], vbo[PT];
#pragma unroll
    for (int i = 0; i < PT; ++i) {
        kbo[i] = (uint32_t)koff(i) * (uint32_t)sizeof(raw);
        vbo[i] = (uint32_t)voff(i) * (uint32_t)sizeof(raw);
    }
    const uint32_t ldsK0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)&sK[wave * 64]);
    const uint32_t ldsV0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)&sV[wave * 64]);
    auto issue = [&](int kb) {
        const int k0 = kb * SBKV;
        u32x4* dK = sK + (kb & 1) * STG;
        u32x4* dV = sV + (kb & 1) * STG;
        if (!SKIP) issue_mask(kb);
        const raw* kbase = Kp + (int64_t)k0 * a.ks2;
        const raw* vbase = Vp + (int64_t)k0 * a.vs2;
        if (k0 + SBKV <= a.Skv && soff) {
            const uint32_t lk = ldsK0 + (uint32_t)((kb & 1) * STG) * 16u;
            const uint32_t lv = ldsV0 + (uint32_t)((kb & 1) * STG) * 16u;
#pragma unroll
            for (int i = 0; i < PT; ++i) {
                dma16_soff(kbase, kbo[i], lk + (uint32_t)(i * THREADS) * 16u);
                dma16_soff(vbase, vbo[i], lv + (uint32_t)(i * THREADS) * 16u);
            }
        } else {
            // a tail stage's rows past the end re-read the last key (never used)
#pragma unroll
            for (int i = 0; i < PT; ++i) {
                const int row = slot_row(i);
                const int sh = k0 + SBKV <= a.Skv ? 0 : min(k0 + row, a.Skv - 1) - k0 - row;
                dma16_async(kbase + koff(i) + sh * (int)a.ks2, &dK[i * THREADS + wave * 64]);
                dma16_async(vbase + voff(i) + sh * (int)a.vs2, &dV[i * THREADS + wave * 64]);
            }
        }
    };

    f32x4 s[QT][NKT];
    // S^T - m = K . Q^T - m for block kb (K stage kb & 1).
    auto qk = [&](int kb) {
        const u32x4* cK = sK + (kb & 1) * STG + grp * BKV * KCH;
#pragma unroll
        for (int qt = 0; qt < QT; ++qt)
#pragma unroll
            for (int kt = 0; kt < NKT; ++kt) s[qt][kt] = f32x4{-m[qt], -m[qt], -m[qt], -m[qt]};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
            for (int kt = 0; kt < NKT; ++kt) {
                const int key = kt * 16 + l16;
                const u32x4 kf = cK[key * KCH + ((ks * 4 + g) ^ (key & KMASK))];
#pragma unroll
                for (int qt = 0; qt < QT; ++qt) s[qt][kt] = mfma_chunk(T{}, kf, qf[qt][ks], s[qt][kt]);
            }
        }
    };
    // MODE 3: this wave's view of the staged mask tile of block kb -- does any
    // key of the block reach its rows, do all of them?
    bool tile_any = true, tile_all = false;
    auto mask_tile = [&](int kb) {
        if constexpr (MODE == 3) {
            if (kb * BKV + BKV > a.Skv) {  // partial last block: not staged
                tile_any = true;
                tile_all = false;
                return;
            }
            constexpr int WCH = WQ * MCH;  // 16-byte chunks of this wave's rows
            const u32x4* t = sM + mslot(kb) * MSTG + ((wave & 3) * WQ) * MCH;
            bool any = false, all = true;
#pragma unroll
            for (int i = 0; i < (WCH + 63) / 64; ++i) {
                const int c = i * 64 + lane;
                if (c < WCH) {
                    const u32x4 v = t[c];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const uint32_t w = v[e];
                        any = any || w != 0u;
                        all = all && ((w - 0x01010101u) & ~w & 0x80808080u) == 0u;  // no zero byte
                    }
                }
            }
            tile_any = __ballot(any) != 0;
            tile_all = __ballot(!all) == 0;
        }
    };
    // Online softmax of block kb and O += V^T P^T (V stage kb & 1).
    auto softmax_pv = [&](int kb) {
        const int k0 = kb * SBKV + grp * BKV;
        const bool staged = MODE == 3 && k0 + BKV <= a.Skv;
        const bool need_mask = (MODE == 2) || (MODE == 3 && !tile_all) || (k0 + BKV > a.Skv) ||
                               (MODE == 1 && k0 + BKV - 1 > q0 + off);
        u32x4 pk[QT][NKT / 2];
        float lmax[QT];
        bool trig = false;
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
            const int qa = q0 + qt * 16 + l16;
            if (need_mask) {
#pragma unroll
                for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        float x = s[qt][kt][r];
                        const int key = k0 + kt * 16 + g * 4 + r;
                        bool vis = key < a.Skv;
                        if (MODE == 1) vis = vis && (key <= qa + off);
                        if (MODE == 3) {
                            if (staged) {
                                const uint32_t w = reinterpret_cast<const uint32_t*>(sM + mslot(kb) * MSTG)
                                    [((qa - qb * BQ) * BKV + kt * 16 + g * 4) >> 2];
                                vis = ((w >> (8 * r)) & 0xffu) != 0u;
                            } else if (vis && qa < a.Sq) {
                                vis = a.mask[(int64_t)qa * a.mask_ld + key] != 0;
                            }
                        }
                        if (MODE == 2 && vis && qa < a.Sq) {
                            if (a.mask != nullptr) vis = a.mask[(int64_t)qa * a.mask_ld + key] != 0;
                            // bias is added after scaling: log2 units, like the scores
                            if (vis && a.bias != nullptr)
                                x += a.bias[(int64_t)qa * a.brs + (int64_t)key * a.bcs] * LOG2E;
                        }
                        s[qt][kt][r] = vis ? x : -INFINITY;
                    }
            }
            // IEEE maximum (NaN-propagating) instead of fmaxf: gfx950's v_maximum3_f32
            // takes the MFMA results as they are, where fmaxf first canonicalises
            // every input (one extra VALU op per score); same value for any non-NaN row
            float mx = -INFINITY;
#pragma unroll
            for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
                for (int r = 0; r < 4; ++r) mx = __builtin_elementwise_maximum(mx, s[qt][kt][r]);
            lmax[qt] = mx;
            // the reference point of a row moves (set on its first visible block,
            // afterwards only for a block max far above it) iff one of its lanes sees this
            trig = trig || mx > thr[qt];
        }
        auto exps = [&]() {
#pragma unroll
            for (int qt = 0; qt < QT; ++qt)
#pragma unroll
                for (int kk = 0; kk < NKT / 2; ++kk) {
                    float e[8];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        e[r] = __builtin_amdgcn_exp2f(s[qt][2 * kk][r]);
                        e[4 + r] = __builtin_amdgcn_exp2f(s[qt][2 * kk + 1][r]);
                    }
                    pk[qt][kk] = u32x4{pack2<T>(e[0], e[1]), pack2<T>(e[2], e[3]), pack2<T>(e[4], e[5]),
                                       pack2<T>(e[6], e[7])};
                }
        };
        // p = 2^(s - m) with the current m, issued without waiting for the test;
        // final unless some row's reference point moves in this block.
        exps();
        if (__ballot(trig) != 0) {
            // Rare: full row max (the row's 16-lane groups), move m, rescale O
            // and l, exps again -- the same values as deciding before the exps.
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) {
                float mx = lmax[qt];
                mx = __builtin_elementwise_maximum(mx, __shfl_xor(mx, 16, 64));
                mx = __builtin_elementwise_maximum(mx, __shfl_xor(mx, 32, 64));
                const bool move = mset[qt] ? (mx > LAZY) : (mx != -INFINITY);
                const float delta = move ? mx : 0.f;
                const float alpha = (move && mset[qt]) ? __builtin_amdgcn_exp2f(-delta) : 1.0f;
                m[qt] += delta;
                mset[qt] = mset[qt] || move;
                thr[qt] = mset[qt] ? LAZY : -INFINITY;
#pragma unroll
                for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
                    for (int r = 0; r < 4; ++r) s[qt][kt][r] -= delta;
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) o[qt][dt] *= alpha;
                lsum[qt] *= alpha;
            }
            exps();
        }
        const u32x4* cV = sV + (kb & 1) * STG + grp * BKV * KCH;
#pragma unroll
        for (int kk = 0; kk < NKT / 2; ++kk) {
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                u32x4 vf;
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const int key = (2 * kk + hh) * 16 + g * 4 + (l16 >> 2);
                    const int byte = key * (D * 2) + ((dt ^ (key & BMASK)) << 5) + 8 * (l16 & 3);
                    const u32x2 w2 = lds_read_tr16(cV, byte);
                    vf[2 * hh] = w2[0];
                    vf[2 * hh + 1] = w2[1];
                }
#pragma unroll
                for (int qt = 0; qt < QT; ++qt) o[qt][dt] = mfma_chunk(T{}, vf, pk[qt][kk], o[qt][dt]);
            }
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) lsum[qt] = mfma_chunk(T{}, ones, pk[qt][kk], lsum[qt]);
        }
    };
    // Wave-uniform: does block kb hold any key visible to this wave's queries?
    auto active = [&](int kb) {
        const int k0 = kb * SBKV + grp * BKV;
        return (KSPLIT == 1 || k0 < a.Skv) && ((MODE != 1) || (k0 <= q0 + WQ - 1 + off));
    };

    if constexpr (SKIP) {
        // Flag word kb & 1 holds one byte per wave, "its rows see a key of block
        // kb": written in step kb-2, read in step kb-1 before K/V(kb) is issued.
        // A wave computes block kb only when its own test of the tile found a
        // key, which implies K/V(kb) was staged. Mask tile t is DMA'd in step t-6 into
        // the slot of tile t-8 (last read in step t-8) and waited for at the end
        // of step t-3, before the barrier after which step t-2 tests it.
        // Each wave keeps its own (any, all) for tiles kb, kb+1, kb+2 in
        // registers: every tile is tested once, two steps before its compute.
        bool any0 = false, all0 = false, any1 = false, all1 = false;
        auto publish = [&](int kb, bool& any, bool& all) {
            any = false;
            all = false;
            if (kb < nkb) {
                mask_tile(kb);
                any = tile_any;
                all = tile_all;
            }
            if (lane == 0) reinterpret_cast<uint8_t*>(&sflag[kb & 1])[wave] = any ? 1 : 0;
        };
        auto wg_vis = [&](int kb) { return kb < nkb && sflag[kb & 1] != 0; };
        // mask DMAs (MPT per thread) issued for tile t: full blocks only
        auto staged_tile = [&](int t) { return t < nkb && t * BKV + BKV <= a.Skv; };
        // wait until at most n * MPT of this wave's DMAs are in flight, LDS reads drained
        auto wait_masks = [&](int n) {
            constexpr int L0 = 7 << 4;  // expcnt not waited, lgkmcnt(0)
            if (n >= 3) __builtin_amdgcn_s_waitcnt(((3 * MPT) & 15) | (((3 * MPT) >> 4) << 14) | L0);
            else if (n == 2) __builtin_amdgcn_s_waitcnt(((2 * MPT) & 15) | (((2 * MPT) >> 4) << 14) | L0);
            else if (n == 1) __builtin_amdgcn_s_waitcnt((MPT & 15) | ((MPT >> 4) << 14) | L0);
            else __builtin_amdgcn_s_waitcnt(L0);
        };
#pragma unroll
        for (int t = 0; t < MAHEAD; ++t) issue_mask(t);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        publish(0, any0, all0);
        publish(1, any1, all1);
        __syncthreads();
        if (wg_vis(0)) issue(0);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        for (int kb = 0; kb < nkb; ++kb) {
            const bool kv = wg_vis(kb + 1);
            if (kv) issue(kb + 1);                               // the K/V stage read in step kb-1
            if (kb + MAHEAD < nkb) issue_mask(kb + MAHEAD);      // the slot of tile kb-2
            bool any2, all2;
            publish(kb + 2, any2, all2);
            tile_any = any0;
            tile_all = all0;
            if (tile_any) {
                qk(kb);
                softmax_pv(kb);
            }
            any0 = any1;
            all0 = all1;
            any1 = any2;
            all1 = all2;
            // K/V(kb+1) and mask tile kb+3 have landed once only the DMAs
            // issued after them are in flight: mask tiles kb+4..kb+6 (or only
            // kb+6 when K/V(kb+1) was issued in this step); DMAs retire in order.
            const int after = kv ? (int)staged_tile(kb + 6)
                                 : (int)staged_tile(kb + 4) + (int)staged_tile(kb + 5) + (int)staged_tile(kb + 6);
            wait_masks(after);
            __syncthreads();
        }
    } else {
        if (nkb > 0) issue(0);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();

        for (int kb = 0; kb < nkb; ++kb) {
            if (kb + 1 < nkb) issue(kb + 1);
            if (active(kb)) {
                mask_tile(kb);
                if (tile_any) {
                    qk(kb);
                    softmax_pv(kb);
                }
            }
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
        }
    }

    if constexpr (KSPLIT == 2) {
        // Every wave is past the last barrier, so the stages are free: waves 4-7
        // leave O and l (one u32x4 slot per lane) and m (-inf where none of its
        // keys was visible) for the wave with the same query rows.
        const int wl = wave & 3;
        u32x4* xo = sK;
        float* xm = reinterpret_cast<float*>(sV);
        if (grp == 1) {
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) {
                u32x4* dst = xo + ((wl * QT + qt) * (DT + 1)) * 64 + lane;
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) dst[dt * 64] = __builtin_bit_cast(u32x4, o[qt][dt]);
                dst[DT * 64] = __builtin_bit_cast(u32x4, lsum[qt]);
                xm[(wl * QT + qt) * 64 + lane] = mset[qt] ? m[qt] : -INFINITY;
            }
        }
        __syncthreads();
        if (grp == 1) return;
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
            const u32x4* src = xo + ((wl * QT + qt) * (DT + 1)) * 64 + lane;
            const float m1 = xm[(wl * QT + qt) * 64 + lane];
            float a0 = 1.f, a1 = 0.f;
            if (!mset[qt]) {
                a0 = 0.f;
                a1 = 1.f;
            } else if (m1 != -INFINITY) {
                const float mt = fmaxf(m[qt], m1);
                a0 = __builtin_amdgcn_exp2f(m[qt] - mt);
                a1 = __builtin_amdgcn_exp2f(m1 - mt);
            }
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) o[qt][dt] = o[qt][dt] * a0 + __builtin_bit_cast(f32x4, src[dt * 64]) * a1;
            lsum[qt] = lsum[qt] * a0 + __builtin_bit_cast(f32x4, src[DT * 64]) * a1;
        }
    }

    raw* Op = static_cast<raw*>(a.O) + b * a.os0 + h * a.os1;
    // Whole 128-byte lines of O (as in attn_fwd_pingpong): the wave rounds its
    // WQ x D rows into LDS -- its own merge slots with the key split, else its
    // share of the K stages, free after the loop's last barrier -- reads them
    // back in order and stores 512 / D rows per instruction. A fragment store
    // writes 8 bytes into each of 16 rows: S=2048 spent 3.1 of 33 us on them.
    constexpr int RB = 2 * D, CPR = RB / 16;  // bytes and 16-byte chunks per row
    if constexpr (KSPLIT == 2 || 4 * GH * WQ * RB <= 2 * STG * 16) {
        if (a.o_line) {
            char* wl = KSPLIT == 2 ? reinterpret_cast<char*>(sK + (wave & 3) * QT * (DT + 1) * 64)
                                   : reinterpret_cast<char*>(sK) + wave * (WQ * RB);
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // after the merge's reads of these slots
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) {
                const float L = lsum[qt][0];
                const float inv = L > 0.f ? 1.0f / L : 0.f;
                const int r = qt * 16 + l16;
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) {
                    const int cb = dt * 32 + g * 8;
                    const f32x4 v = o[qt][dt] * inv;
                    *reinterpret_cast<u32x2*>(wl + r * RB + ((((cb >> 4) ^ (r & (CPR - 1))) << 4) | (cb & 15))) =
                        u32x2{pack2<T>(v[0], v[1]), pack2<T>(v[2], v[3])};
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
            for (int it = 0; it < WQ * CPR / 64; ++it) {
                const int r = it * (64 / CPR) + lane / CPR, c = lane % CPR;
                const u32x4 v = *reinterpret_cast<const u32x4*>(wl + r * RB + ((c ^ (r & (CPR - 1))) << 4));
                const int q = q0 + r;
                if (q < a.Sq) *reinterpret_cast<u32x4*>(Op + (int64_t)q * a.os2 + c * 8) = v;
            }
            return;
        }
    }
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const float L = lsum[qt][0];
        const float inv = L > 0.f ? 1.0f / L : 0.f;
        const int q = q0 + qt * 16 + l16;
        if (q >= a.Sq) continue;
        raw* orow = Op + (int64_t)q * a.os2;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            const int d = dt * 16 + g * 4;
            const f32x4 v = o[qt][dt] * inv;
            u32x2 p = {pack2<T>(v[0], v[1]), pack2<T>(v[2], v[3])};
            *reinterpret_cast<u32x2*>(orow + d) = p;
        }
    }
}

// Paired-head ping-pong prefill (no mask or causal, 16-bit, d in {64, 128}).
// A workgroup of 8 waves serves two query heads of one GQA group over the same
// 128 queries: waves 0-3 (group A) head h0, waves 4-7 (group B) head h1, each
// wave 32 queries, the 64-key K/V tiles staged once for both. The hardware
// places waves w and w+4 on the same SIMD. Each wave alternates
//   M(j): PV(j-1) and QK(j) on the matrix cores (operand fragments read three
//         fragments ahead of their MFMAs, raised issue priority), and
//   S(j): mask, row max, reference-point update, exp2 and packing of block j,
// with group B one phase behind group A and a workgroup barrier per phase, so
// on every SIMD one wave's MFMA phase runs beside the other wave's softmax.
// Group B stages K(j+1) during its S(j-1) (phase 2j) and group A stages V(j)
// during its S(j) (phase 2j+1); each waits for its own DMA at the end of phase
// 2j+1, and both are first read in phase 2j+2. A wave issues in order and DMA
// instructions back to back wait for the address unit (about 30 bytes per
// clock per CU), so each group issues half of a block's DMA in the phase
// where it has slack. The arithmetic per score
// and its order (accumulator started at -m, lazy reference point, packed p,
// ones-MFMA row sums, O accumulated block by block) are those of
// attn_fwd_mfma with 64-key blocks.
// Key blocks a ping-pong workgroup can list under a byte mask (kv_len up to
// 64 * PP_LIST_MAX); longer masks take the staged-mask kernel.
constexpr int PP_LIST_MAX = 4096;

// Tile classes of a byte mask [Sq, Skv] (row stride ld, rows 16-byte aligned):
// for each 32-row group rg and 64-key block kb, cls[rg * nkbt + kb] has bit 0
// set when some (row, key) of the tile is visible and bit 1 when every one is
// (rows < Sq, keys < Skv). One workgroup per row group and 16 key blocks; the
// ping-pong kernel lists its blocks from these instead of reading the mask.
__global__ __launch_bounds__(256) void mask_tile_class_kernel(const uint8_t* mask, int64_t ld, int Sq, int Skv,
                                                              int nkbt, uint8_t* cls) {
    __shared__ uint32_t s_any[16], s_all[16];
    const int t = threadIdx.x, kbl = t & 15, r0 = t >> 4;
    const int rg = blockIdx.x, kb = blockIdx.y * 16 + kbl;
    if (t < 16) {
        s_any[t] = 0u;
        s_all[t] = 1u;
    }
    __syncthreads();
    bool any = false, all = true;
    if (kb < nkbt) {
        const int k0 = kb * 64;
#pragma unroll
        for (int rr = 0; rr < 2; ++rr) {
            const int row = rg * 32 + r0 + 16 * rr;
            if (row >= Sq) continue;
            const uint8_t* mr = mask + (int64_t)row * ld + k0;
            if (k0 + 64 <= Skv) {
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const u32x4 w = reinterpret_cast<const u32x4*>(mr)[c];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const uint32_t x = w[e];
                        any = any || x != 0u;
                        all = all && ((x - 0x01010101u) & ~x & 0x80808080u) == 0u;  // no zero byte
                    }
                }
            } else {
                for (int jj = 0; jj < Skv - k0; ++jj) {
                    const bool v = mr[jj] != 0;
                    any = any || v;
                    all = all && v;
                }
            }
        }
    }
    if (any) atomicOr(&s_any[kbl], 1u);
    if (!all) atomicAnd(&s_all[kbl], 0u);
    __syncthreads();
    if (t < 16 && blockIdx.y * 16 + t < nkbt)
        cls[(int64_t)rg * nkbt + blockIdx.y * 16 + t] = (uint8_t)(s_any[t] | (s_all[t] << 1));
}

template <class T, int D, int MODE>
__global__ __launch_bounds__(512, 1) void attn_fwd_pingpong(AttnArgs a) {
    using raw = typename T::raw;
    constexpr int QT = 2, NKT = 4;
    constexpr int WQ = 16 * QT, BQ = 4 * WQ, BKV = 16 * NKT;
    constexpr int KCH = D / 8;
    constexpr int DT = D / 16;
    constexpr int KS = D / 32;
    constexpr int GT = 256;  // threads of one wave group (the issuers of a tile's DMA)
    constexpr int PT = BKV * KCH / GT;
    static_assert(PT * GT == BKV * KCH, "tile / thread mismatch");
    constexpr int NB = D / 16;
    constexpr int BMASK = (NB < 8 ? NB : 8) - 1;
    constexpr int STG = BKV * KCH;
    constexpr int KMASK = KCH - 1 < 15 ? KCH - 1 : 15;
    __shared__ u32x4 sK[2 * STG];
    __shared__ u32x4 sV[2 * STG];

    const int G = a.Hq / a.Hkv;
    const int hgroups = G / 2;
    const int units = a.B * a.Hkv * hgroups;
    const int total = units * a.nqb;
    int w = blockIdx.x;
    if ((total & 7) == 0) w = (w & 7) * (total >> 3) + (w >> 3);
    const int unit = w / a.nqb;
    const int qi = w % a.nqb;
    const int qb = (MODE == 1 || MODE == 3) ? (a.nqb - 1 - qi) : qi;
    const int b = unit / (a.Hkv * hgroups);
    const int rem = unit % (a.Hkv * hgroups);
    const int kvh = rem / hgroups;
    // the wave index made scalar: every per-wave test (rows seen, tile class)
    // is then a scalar branch, not an exec-mask one
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool grpB = wave >= 4;
    const int h = kvh * G + (rem % hgroups) * 2 + (wave >> 2);
    const int l16 = lane & 15, g = lane >> 4;
    const int q0 = qb * BQ + (wave & 3) * WQ;

    const raw* Qp = static_cast<const raw*>(a.Q) + b * a.qs0 + h * a.qs1;
    const raw* Kp = static_cast<const raw*>(a.K) + b * a.ks0 + kvh * a.ks1;
    const raw* Vp = static_cast<const raw*>(a.V) + b * a.vs0 + kvh * a.vs1;

    // MODE 3: the four 32-row groups' tile classes of key block kb, 2 bits each
    // (issued before the Q loads so that the two latencies overlap)
    auto tile_classes = [&](int kb) -> uint32_t {
        uint32_t packed = 0;
        if (kb < a.nkbt) {
            const int nrg = (a.Sq + 31) / 32;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int rg = qb * 4 + i;
                if (rg < nrg) packed |= (uint32_t)a.tcls[(int64_t)rg * a.nkbt + kb] << (2 * i);
            }
        }
        return packed;
    };
    const uint32_t packed0 = MODE == 3 ? tile_classes(wave * 64 + lane) : 0u;

    // Q pre-scaled by scale*log2(e) and rounded back to T, as in attn_fwd_mfma
    const float c = a.scale_log2;
    u32x4 qf[QT][KS];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const int q = q0 + qt * 16 + l16;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            u32x4 v = {0u, 0u, 0u, 0u};
            if (q < a.Sq) v = *reinterpret_cast<const u32x4*>(Qp + (int64_t)q * a.qs2 + ks * 32 + g * 8);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t w2 = v[e];
                v[e] = pack2<T>(lo_as_f32(T{}, w2) * c, hi_as_f32(T{}, w2) * c);
            }
            qf[qt][ks] = v;
        }
    }

    const int off = a.diag_off;  // causal: key j visible to query i iff j <= i + off
    int kv_end = a.Skv;
    if (MODE == 1) kv_end = min(a.Skv, qb * BQ + BQ + off);
    int nkb = kv_end > 0 ? (kv_end + BKV - 1) / BKV : 0;  // blocks the workgroup stages
    int kv_end_w = a.Skv;
    if (MODE == 1) kv_end_w = min(a.Skv, q0 + WQ + off);
    const int nkw = kv_end_w > 0 ? (kv_end_w + BKV - 1) / BKV : 0;  // blocks this wave's rows see

    // MODE 3 (byte mask, tile classes from mask_tile_class_kernel): the workgroup
    // stages, in key order, only the blocks some of its 128 rows see; list
    // position j holds block slist[j] and the four 32-row groups' classes, 2 bits
    // each (0 none, 1 some, 3 all). K/V stages follow the position, not the block.
    constexpr int LMAX = MODE == 3 ? PP_LIST_MAX : 1;
    __shared__ uint32_t slist[LMAX];  // block | classes << 16
    __shared__ int scnt[MODE == 3 ? 8 : 1];
    if constexpr (MODE == 3) {
        int base = 0;
        for (int c0 = 0; c0 < a.nkbt; c0 += 512) {
            const int kb = c0 + wave * 64 + lane;
            const uint32_t packed = c0 == 0 ? packed0 : tile_classes(kb);
            const uint64_t bal = __ballot(packed != 0u);
            if (lane == 0) scnt[wave] = __popcll(bal);
            __syncthreads();
            int before = base, tot = 0;
#pragma unroll
            for (int w2 = 0; w2 < 8; ++w2) {
                before += w2 < wave ? scnt[w2] : 0;
                tot += scnt[w2];
            }
            if (packed != 0u) {
                const int pos = before + __popcll(bal & ((1ull << lane) - 1ull));
                slist[pos] = (uint32_t)kb | (packed << 16);
            }
            base += tot;
            __syncthreads();  // the list is complete; scnt free for the next chunk
        }
        nkb = base;
    }
    // List entry of position j (MODE 3: block | classes << 16; otherwise block j),
    // read from LDS one step before the loop needs it.
    auto entry_v = [&](int j) -> uint32_t {  // the LDS read (per lane)
        if constexpr (MODE == 3) return (j < nkb) ? slist[j] : 0u;
        else return 0u;
    };
    auto entry = [&](int j) -> uint32_t { return __builtin_amdgcn_readfirstlane(entry_v(j)); };
    auto kblock = [&](int j, uint32_t e) -> int {
        if constexpr (MODE == 3) return (int)(e & 0xffffu);
        else return j;
    };
    // this wave's 32 rows: the class of an entry (MODE 3), whether they see position j
    auto wcls = [&](uint32_t e) -> int { return (int)((e >> (16 + 2 * (wave & 3))) & 3u); };
    auto wsees = [&](int j, uint32_t e) -> bool {
        if constexpr (MODE == 3) return j >= 0 && j < nkb && wcls(e) != 0;
        else return j >= 0 && j < nkw;
    };

    constexpr float LAZY = 8.0f;
    constexpr uint32_t ONE2 = std::is_same_v<T, BF16> ? 0x3F803F80u : 0x3C003C00u;
    const u32x4 ones = {ONE2, ONE2, ONE2, ONE2};
    float m[QT];
    bool mset[QT];
    f32x4 lsum[QT];
    // per row: the block max above which the reference point moves (any
    // visible key before the first move, LAZY after)
    float thr[QT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        m[qt] = 0.f;
        mset[qt] = false;
        lsum[qt] = f32x4{0.f, 0.f, 0.f, 0.f};
        thr[qt] = -INFINITY;
    }
    f32x4 o[QT][DT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[qt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};

    // DMA slots of this thread within its wave group: row and swizzled chunk, as
    // element offsets from the block's first key
    const int gw = (tid & (GT - 1)) >> 6;
    auto slot_row = [&](int i) { return (i * GT + gw * 64 + lane) / KCH; };
    auto koff = [&](int i) {
        const int slot = i * GT + gw * 64 + lane, row = slot / KCH, ps = slot % KCH;
        return row * (int)a.ks2 + (ps ^ (row & KMASK)) * 8;
    };
    auto voff = [&](int i) {
        const int slot = i * GT + gw * 64 + lane, row = slot / KCH, ps = slot % KCH;
        return row * (int)a.vs2 + ((ps >> 1) ^ (row & BMASK)) * 16 + (ps & 1) * 8;
    };
    // Whole blocks: the DMA goes from the block's scalar base plus this lane's
    // fixed 32-bit byte offset (no VALU address work inside the loop; 64 rows
    // at a row stride below 2^24 elements span < 2^31 bytes); the LDS
    // destinations of the two stages are scalar too. A partial last block
    // clamps its rows past the end to the last key (their scores are masked).
    uint32_t kbo[PT], vbo[PT];
#pragma unroll
    for (int i = 0; i < PT; ++i) {
        kbo[i] = (uint32_t)koff(i) * (uint32_t)sizeof(raw);
        vbo[i] = (uint32_t)voff(i) * (uint32_t)sizeof(raw);
    }
    const uint32_t ldsK0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)&sK[gw * 64]);
    const uint32_t ldsV0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)&sV[gw * 64]);
    auto issue_k = [&](int j, uint32_t e) {
        const int k0 = kblock(j, e) * BKV;
        const raw* kbase = Kp + (int64_t)k0 * a.ks2;
        if (k0 + BKV <= a.Skv) {
            const uint32_t l0 = ldsK0 + (uint32_t)((j & 1) * STG) * 16u;
#pragma unroll
            for (int i = 0; i < PT; ++i) dma16_soff(kbase, kbo[i], l0 + (uint32_t)(i * GT) * 16u);
            return;
        }
        u32x4* dK = sK + (j & 1) * STG;
#pragma unroll
        for (int i = 0; i < PT; ++i) {
            const int row = slot_row(i);
            const int sh = min(k0 + row, a.Skv - 1) - k0 - row;
            dma16_async(kbase + koff(i) + sh * (int)a.ks2, &dK[i * GT + gw * 64]);
        }
    };
    auto issue_v = [&](int j, uint32_t e) {
        const int k0 = kblock(j, e) * BKV;
        const raw* vbase = Vp + (int64_t)k0 * a.vs2;
        if (k0 + BKV <= a.Skv) {
            const uint32_t l0 = ldsV0 + (uint32_t)((j & 1) * STG) * 16u;
#pragma unroll
            for (int i = 0; i < PT; ++i) dma16_soff(vbase, vbo[i], l0 + (uint32_t)(i * GT) * 16u);
            return;
        }
        u32x4* dV = sV + (j & 1) * STG;
#pragma unroll
        for (int i = 0; i < PT; ++i) {
            const int row = slot_row(i);
            const int sh = min(k0 + row, a.Skv - 1) - k0 - row;
            dma16_async(vbase + voff(i) + sh * (int)a.vs2, &dV[i * GT + gw * 64]);
        }
    };

    f32x4 s[QT][NKT];
    u32x4 pk[QT][NKT / 2];

    // M phase: O += V^T P^T for block jp (and the row sums), then S^T - m = K Q^T
    // for block jq. A unit is one K or V fragment feeding QT MFMAs; fragments are
    // read PF units ahead, the scheduling barriers keep that order.
    constexpr int PF = 3;
    auto mphase = [&](int jp, bool do_pv, int jq, bool do_qk) {
        __builtin_amdgcn_s_setprio(1);
        const u32x4* cV = sV + (jp & 1) * STG;
        const u32x4* cK = sK + (jq & 1) * STG;
        auto ldv = [&](int kk, int dt) -> u32x4 {
            u32x4 vf;
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const int key = (2 * kk + hh) * 16 + g * 4 + (l16 >> 2);
                const int byte = key * (D * 2) + ((dt ^ (key & BMASK)) << 5) + 8 * (l16 & 3);
                const u32x2 w2 = lds_read_tr16(cV, byte);
                vf[2 * hh] = w2[0];
                vf[2 * hh + 1] = w2[1];
            }
            return vf;
        };
        auto ldk = [&](int ks, int kt) -> u32x4 {
            const int key = kt * 16 + l16;
            return cK[key * KCH + ((ks * 4 + g) ^ (key & KMASK))];
        };
        if (do_pv) {
            constexpr int NU = (NKT / 2) * DT;
            u32x4 fr[PF + 1];
            static_for<0, PF>([&](auto uc) {
                constexpr int u = decltype(uc)::value;
                fr[u] = ldv(u / DT, u % DT);
            });
            __builtin_amdgcn_sched_barrier(0);
            static_for<0, NU>([&](auto uc) {
                constexpr int u = decltype(uc)::value;
                constexpr int kk = u / DT, dt = u % DT;
                if constexpr (u + PF < NU) fr[(u + PF) % (PF + 1)] = ldv((u + PF) / DT, (u + PF) % DT);
#pragma unroll
                for (int qt = 0; qt < QT; ++qt) o[qt][dt] = mfma_chunk(T{}, fr[u % (PF + 1)], pk[qt][kk], o[qt][dt]);
                if constexpr (dt == DT - 1) {
#pragma unroll
                    for (int qt = 0; qt < QT; ++qt) lsum[qt] = mfma_chunk(T{}, ones, pk[qt][kk], lsum[qt]);
                }
                __builtin_amdgcn_sched_barrier(0);
            });
        }
        if (do_qk) {
#pragma unroll
            for (int qt = 0; qt < QT; ++qt)
#pragma unroll
                for (int kt = 0; kt < NKT; ++kt) s[qt][kt] = f32x4{-m[qt], -m[qt], -m[qt], -m[qt]};
            constexpr int NU = KS * NKT;
            u32x4 fr[PF + 1];
            static_for<0, PF>([&](auto uc) {
                constexpr int u = decltype(uc)::value;
                fr[u] = ldk(u / NKT, u % NKT);
            });
            __builtin_amdgcn_sched_barrier(0);
            static_for<0, NU>([&](auto uc) {
                constexpr int u = decltype(uc)::value;
                constexpr int ks = u / NKT, kt = u % NKT;
                if constexpr (u + PF < NU) fr[(u + PF) % (PF + 1)] = ldk((u + PF) / NKT, (u + PF) % NKT);
#pragma unroll
                for (int qt = 0; qt < QT; ++qt)
                    s[qt][kt] = mfma_chunk(T{}, fr[u % (PF + 1)], qf[qt][ks], s[qt][kt]);
                __builtin_amdgcn_sched_barrier(0);
            });
        }
        __builtin_amdgcn_s_setprio(0);
    };
    // S phase of block kb: masked scores -> -inf, row max (relative to m), the
    // lazy reference point (set by the first visible block, moved only when a
    // block max exceeds it by more than LAZY in log2 units, O and l rescaled
    // then), p = exp2(s - m) packed to T.
    // MODE 3, a mixed tile (some but not all of it visible to the wave's rows):
    // its 32 x 64 mask bytes reach the wave's own LDS slot (row-major) by DMA,
    // issued with the DMA of the step before the wave's next S phase, so the
    // step-end wait covers it. kv_len % 16 == 0 on this path: a 16-byte piece
    // is wholly below kv_len or wholly past it (those re-read key 0 and are
    // masked by index); rows past Sq re-read the last row (never stored).
    __shared__ u32x4 smask[MODE == 3 ? 8 * 128 : 1];
    auto load_mw = [&](int j, uint32_t e) {
        if constexpr (MODE == 3) {
            if (!(wsees(j, e) && wcls(e) == 1)) return;
            const int kp = kblock(j, e) * BKV + 16 * (lane & 3);
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int row = min(q0 + 16 * i + (lane >> 2), a.Sq - 1);
                dma16_async(a.mask + (int64_t)row * a.mask_ld + (kp < a.Skv ? kp : 0), &smask[wave * 128 + i * 64]);
            }
        }
    };
    auto sphase = [&](int j, uint32_t e) {
        const int k0 = kblock(j, e) * BKV;
        const bool mixed = MODE == 3 && wcls(e) == 1;
        const bool msk = (k0 + BKV > a.Skv) || (MODE == 1 && k0 + BKV - 1 > q0 + off) || mixed;
        uint32_t mw[QT][NKT];  // this lane's 4 mask bytes per 16-key tile
        if constexpr (MODE == 3) {
            if (mixed) {
                const uint32_t* sm = reinterpret_cast<const uint32_t*>(&smask[wave * 128]);
#pragma unroll
                for (int qt = 0; qt < QT; ++qt)
#pragma unroll
                    for (int kt = 0; kt < NKT; ++kt) mw[qt][kt] = sm[(qt * 16 + l16) * 16 + kt * 4 + g];
            }
        }
        float lmax[QT];
        bool trig = false;
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
            const int qa = q0 + qt * 16 + l16;
            if (msk) {
#pragma unroll
                for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int key = k0 + kt * 16 + g * 4 + r;
                        bool vis = key < a.Skv;
                        if (MODE == 1) vis = vis && (key <= qa + off);
                        if constexpr (MODE == 3) vis = vis && (!mixed || ((mw[qt][kt] >> (8 * r)) & 0xffu) != 0u);
                        s[qt][kt][r] = vis ? s[qt][kt][r] : -INFINITY;
                    }
            }
            float mx = -INFINITY;
#pragma unroll
            for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
                for (int r = 0; r < 4; ++r) mx = __builtin_elementwise_maximum(mx, s[qt][kt][r]);
            lmax[qt] = mx;
            // a row's reference point moves iff one of its lanes sees this
            trig = trig || mx > thr[qt];
        }
        auto exps = [&]() {
#pragma unroll
            for (int qt = 0; qt < QT; ++qt)
#pragma unroll
                for (int kk = 0; kk < NKT / 2; ++kk) {
                    float e[8];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        e[r] = __builtin_amdgcn_exp2f(s[qt][2 * kk][r]);
                        e[4 + r] = __builtin_amdgcn_exp2f(s[qt][2 * kk + 1][r]);
                    }
                    pk[qt][kk] = u32x4{pack2<T>(e[0], e[1]), pack2<T>(e[2], e[3]), pack2<T>(e[4], e[5]),
                                       pack2<T>(e[6], e[7])};
                }
        };
        // p = 2^(s - m) with the current m, issued without waiting for the test;
        // when no lane's row moves its reference point (every block after a
        // row's first, barring a max more than LAZY above m) these are final.
        exps();
        if (__ballot(trig) != 0) {
            // Rare: full row max across the row's lanes, move m, rescale O and l,
            // exps again -- the same values as deciding before the exps.
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) {
                const float mx = max_across_rows(lmax[qt]);
                const bool move = mset[qt] ? (mx > LAZY) : (mx != -INFINITY);
                const float delta = move ? mx : 0.f;
                const float alpha = (move && mset[qt]) ? __builtin_amdgcn_exp2f(-delta) : 1.0f;
                m[qt] += delta;
                mset[qt] = mset[qt] || move;
                thr[qt] = mset[qt] ? LAZY : -INFINITY;
#pragma unroll
                for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
                    for (int r = 0; r < 4; ++r) s[qt][kt][r] -= delta;
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) o[qt][dt] *= alpha;
                lsum[qt] *= alpha;
            }
            exps();
        }
    };

    // Phase 2j: A runs M(j), B stages K(j+1) and runs S(j-1).
    // Phase 2j+1: A stages V(j) and runs S(j), B runs M(j). The K stage B fills
    // held K(j-1) and the V stage A fills held V(j-2), both last read in
    // phases 2j-2 and 2j-1. Every wave passes 2 (nkb + 1) + 1 barriers; K(0) is
    // staged by group A before the first one.
    // em, e0, ep: the entries of positions j - 1, j, j + 1 (MODE 3)
    uint32_t em = 0u, e0 = entry(0), ep = entry(1);
    if (nkb > 0 && !grpB) issue_k(0, e0);
    if (!grpB) load_mw(0, e0);
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_s_barrier();
    // The entry of position j + 2 is read in step j and made scalar after the
    // step-end wait, so the read never stalls the step.
    if (!grpB) {
        for (int j = 0; j <= nkb; ++j) {
            mphase(j - 1, wsees(j - 1, em), j, wsees(j, e0));
            __builtin_amdgcn_s_waitcnt(0);
            __builtin_amdgcn_s_barrier();
            const uint32_t en = entry_v(j + 2);
            if (j < nkb) issue_v(j, e0);
            if (wsees(j, e0)) sphase(j, e0);
            load_mw(j + 1, ep);
            __builtin_amdgcn_s_waitcnt(0);  // this wave's V(j) DMA has landed
            __builtin_amdgcn_s_barrier();
            em = e0;
            e0 = ep;
            ep = __builtin_amdgcn_readfirstlane(en);
        }
    } else {
        for (int j = 0; j <= nkb; ++j) {
            if (j + 1 < nkb) issue_k(j + 1, ep);
            const uint32_t en = entry_v(j + 2);
            if (wsees(j - 1, em)) sphase(j - 1, em);
            load_mw(j, e0);
            __builtin_amdgcn_s_barrier();
            mphase(j - 1, wsees(j - 1, em), j, wsees(j, e0));
            __builtin_amdgcn_s_waitcnt(0);  // this wave's K(j+1) DMA has landed
            __builtin_amdgcn_s_barrier();
            em = e0;
            e0 = ep;
            ep = __builtin_amdgcn_readfirstlane(en);
        }
    }

    raw* Op = static_cast<raw*>(a.O) + b * a.os0 + h * a.os1;
    if (a.o_line) {
        // Whole 128-byte lines of O: a fragment store writes 8 bytes into each of
        // 16 rows. Every wave's K/V reads ended at the loop's last barrier, so
        // each wave rounds its 32 x D rows into its own 64 D bytes of the stages
        // (row r at r * 2D bytes, 16-byte chunk c at c ^ (r % (D / 8))), reads
        // them back (LDS keeps a wave's accesses in order) and stores 512 / D rows
        // per instruction, 16 bytes per lane.
        constexpr int RB = 2 * D;     // bytes per row
        constexpr int CPR = RB / 16;  // 16-byte chunks per row
        char* wl = reinterpret_cast<char*>(wave < 4 ? sK : sV) + (wave & 3) * (WQ * RB);
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
            const float L = lsum[qt][0];
            const float inv = L > 0.f ? 1.0f / L : 0.f;
            const int r = qt * 16 + l16;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                const int cb = dt * 32 + g * 8;
                const f32x4 v = o[qt][dt] * inv;
                *reinterpret_cast<u32x2*>(wl + r * RB + ((((cb >> 4) ^ (r & (CPR - 1))) << 4) | (cb & 15))) =
                    u32x2{pack2<T>(v[0], v[1]), pack2<T>(v[2], v[3])};
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int it = 0; it < WQ * CPR / 64; ++it) {
            const int r = it * (64 / CPR) + lane / CPR, c = lane % CPR;
            const u32x4 v = *reinterpret_cast<const u32x4*>(wl + r * RB + ((c ^ (r & (CPR - 1))) << 4));
            const int q = q0 + r;
            if (q < a.Sq) *reinterpret_cast<u32x4*>(Op + (int64_t)q * a.os2 + c * 8) = v;
        }
        return;
    }
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const float L = lsum[qt][0];
        const float inv = L > 0.f ? 1.0f / L : 0.f;
        const int q = q0 + qt * 16 + l16;
        if (q >= a.Sq) continue;
        raw* orow = Op + (int64_t)q * a.os2;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            const int d = dt * 16 + g * 4;
            const f32x4 v = o[qt][dt] * inv;
            u32x2 p = {pack2<T>(v[0], v[1]), pack2<T>(v[2], v[3])};
            *reinterpret_cast<u32x2*>(orow + d) = p;
        }
    }
}

// Any layout / any dtype / d, dv <= 256: one wave per (batch, head, query row).
// Scores for the whole row are kept in LDS (kv_len <= ROW_MAX), then max,
// exp, sum and P.V in key order (the decode formulation of the reference).
constexpr int ROW_MAX = 16384;

template <class T>
__global__ __launch_bounds__(64) void attn_rowwise(AttnArgs a) {
    extern __shared__ float sc[];
    const int qi = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int kvh = h / (a.Hq / a.Hkv);
    const int lane = threadIdx.x;
    const int64_t qo = b * a.qs0 + h * a.qs1 + (int64_t)qi * a.qs2;
    const int64_t ko = b * a.ks0 + kvh * a.ks1;
    const int64_t vo = b * a.vs0 + kvh * a.vs1;
    const float scale = a.scale_log2 / LOG2E;
    const int off = a.diag_off;
    float mx = -INFINITY;
    for (int j = lane; j < a.Skv; j += 64) {
        bool vis = true;
        if (a.causal) vis = j <= qi + off;
        if (vis && a.mask != nullptr) vis = a.mask[(int64_t)qi * a.mask_ld + j] != 0;
        float x = -INFINITY;
        if (vis) {
            float acc = 0.f;
            for (int d = 0; d < a.D; ++d)
                acc = fmaf(load_as_f32<T>(a.Q, qo + d * a.qs3),
                           load_as_f32<T>(a.K, ko + (int64_t)j * a.ks2 + d * a.ks3), acc);
            x = acc * scale;
            if (a.bias != nullptr) x += a.bias[(int64_t)qi * a.brs + (int64_t)j * a.bcs];
        }
        sc[j] = x;
        mx = fmaxf(mx, x);
    }
#pragma unroll
    for (int off2 = 32; off2 >= 1; off2 >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off2, 64));
    float sum = 0.f;
    for (int j = lane; j < a.Skv; j += 64) {
        const float p = (sc[j] == -INFINITY) ? 0.f : expf(sc[j] - mx);
        sc[j] = p;
        sum += p;
    }
#pragma unroll
    for (int off2 = 32; off2 >= 1; off2 >>= 1) sum += __shfl_xor(sum, off2, 64);
    __syncthreads();
    const float inv = sum > 0.f ? 1.0f / sum : 0.f;
    const int64_t oo = b * a.os0 + h * a.os1 + (int64_t)qi * a.os2;
    for (int d = lane; d < a.Dv; d += 64) {
        float acc = 0.f;
        if (sum > 0.f)
            for (int j = 0; j < a.Skv; ++j)
                if (sc[j] != 0.f)
                    acc = fmaf(sc[j] * inv, load_as_f32<T>(a.V, vo + (int64_t)j * a.vs2 + d * a.vs3), acc);
        store_from_f32<T>(a.O, oo + d * a.os3, acc);
    }
}

// ---------------------------------------------------------------------------
// fp32 prefill on the matrix cores. The reference's flash backend is fp32-only
// (src/function/ops.inl:119-121; _flashAttentionImpl, src/kernel/avx2/
// flash_attention.inl:274-443), so this is its call's native dtype.
// ---------------------------------------------------------------------------
// v_mfma_f32_16x16x4_f32; workgroup = 8 waves x 16 queries = 128 queries of one
// (batch, head); 64-key blocks of K and V double-buffered in LDS by DMA, one
// barrier per block. Lane l: query r = l % 16 of its wave, lane group g = l / 16.
//   S^T = K . Q^T: src0 = K[key l%16][d], src1 = Q[query l%16][d] (pre-scaled by
//     scale * log2 e), d = 16b + 4g + j at step (b, j): lane l receives
//     S[query r][keys 4g .. 4g+3] of each 16-key tile, so a query's 64 scores of
//     a block sit in its 4 lanes (l, l^16, l^32, l^48) and its block maximum is
//     two row swaps (max_across_rows).
//   O^T += V^T . P^T: step (tile, j) takes the keys 16 tile + 4g + j of the four
//     lane groups, src0 = V[that key][d = 16t + l%16], src1 = the lane's own
//     probability j: lane l accumulates O[query r][d = 16t + 4g + i], so the
//     rescale by 2^(m_old - m_new) is per lane, and the softmax denominator is a
//     per-lane partial summed over the query's 4 lanes at the end.
//   LDS: K chunk c (16 bytes) of a row stored at c ^ (key & 15) -- the 16 keys
//     a quarter-wave's ds_read_b128 serves land on 16 distinct 16-byte bank
//     groups (with key & 7 they share 8: a 2-way conflict on every score
//     step); V chunk c at c ^ (((key>>2)&3)<<2)
//     -- the four lane groups' ds_read_b32 of four different keys fall in four
//     bank ranges.
// MODE 0: no mask; 1: causal / diagonal (key j visible to query i iff j <= i +
// diag_off; key blocks past the workgroup's last visible key are never loaded,
// the heaviest query blocks launch first); 2: byte mask and / or bias read per
// element. Keys at or past kv_len are masked; a query with no visible key
// gets zeros (flash_attention.inl:241-244, 327-331).
// KS = 2 (short prompts): 64-query blocks, twice the workgroups. Waves w and
// w + 4 own the same 16 queries; wave group g = w / 4 takes keys [32 g, 32 g +
// 32) of every staged block, and at the end group 1 hands its O, m and l to
// group 0 through LDS, which merges them with the log-sum-exp rule.
template <int D, int MODE, int KS = 1>
__global__ __launch_bounds__(512, 1) void attn_fwd_f32(AttnArgs a) {
    static_assert(KS == 1 || KS == 2, "key split 1 or 2");
    constexpr int NW = 8, BQ = 16 * NW / KS, BKV = 64;
    constexpr int NKT = 4 / KS;         // 16-key tiles of a block per wave
    constexpr int KCH = D / 4;          // 16-byte chunks per K / V row
    constexpr int STG = BKV * KCH;      // chunks per stage of K (or V)
    constexpr int PT = STG / (64 * NW); // DMA chunks per thread per stage
    constexpr int NB = D / 16;          // 16-wide k blocks of S, 16-wide d tiles of O
    static_assert(PT * 64 * NW == STG, "whole DMA rounds");
    __shared__ u32x4 sK[2 * STG];
    __shared__ u32x4 sV[2 * STG];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane & 15, g = lane >> 4;
    const int nqb = (a.Sq + BQ - 1) / BQ;
    const int nbh = a.B * a.Hq;
    const int rank = blockIdx.x / nbh, bh = blockIdx.x % nbh;
    // the last query blocks first: causal rows, and the rows of causal-shaped
    // byte masks (a KV ring's included), see more keys further down
    const int qb = (MODE == 1 || MODE == 2) ? nqb - 1 - rank : rank;
    const int b = bh / a.Hq, h = bh % a.Hq, kvh = h / (a.Hq / a.Hkv);
    const float* Qp = static_cast<const float*>(a.Q) + b * a.qs0 + h * a.qs1;
    const float* Kp = static_cast<const float*>(a.K) + b * a.ks0 + kvh * a.ks1;
    const float* Vp = static_cast<const float*>(a.V) + b * a.vs0 + kvh * a.vs1;
    float* Op = static_cast<float*>(a.O) + b * a.os0 + h * a.os1;
    const int wl = KS == 2 ? (wave & 3) : wave;  // row group of this wave
    const int kofs = KS == 2 ? (wave >> 2) * 32 : 0;  // first key of a block this wave takes
    const int q0 = qb * BQ + wl * 16;  // this wave's first query
    const int qrow = q0 + r;             // this lane's query
    const bool wave_rows = q0 < a.Sq;

    // key blocks the workgroup reads
    const int nkb_all = (a.Skv + BKV - 1) / BKV;
    int nkb = nkb_all;
    if constexpr (MODE == 1) {
        const int last = min(qb * BQ + BQ - 1, a.Sq - 1) + a.diag_off;
        nkb = last < 0 ? 0 : min(nkb_all, last / BKV + 1);
    }

    // Q fragments, pre-scaled into log2 units: qf[bb][j] = Q[qrow][16 bb + 4 g + j]
    f32x4 qf[NB];
    {
        const float* qp = Qp + (int64_t)min(qrow, a.Sq - 1) * a.qs2 + 4 * g;
#pragma unroll
        for (int bb = 0; bb < NB; ++bb) qf[bb] = *reinterpret_cast<const f32x4*>(qp + 16 * bb) * a.scale_log2;
    }

    // DMA slots (row and swizzled chunk) as element offsets from the block's first key
    auto slot_row = [&](int i) { return (i * 64 * NW + wave * 64 + lane) / KCH; };
    auto koff = [&](int i) {
        const int slot = i * 64 * NW + wave * 64 + lane, row = slot / KCH, c = slot % KCH;
        return row * (int)a.ks2 + (c ^ (row & 15)) * 4;
    };
    auto voff = [&](int i) {
        const int slot = i * 64 * NW + wave * 64 + lane, row = slot / KCH, c = slot % KCH;
        return row * (int)a.vs2 + (c ^ (((row >> 2) & 3) << 2)) * 4;
    };
    // Whole blocks whose lane offsets fit 31 bits go from the block's scalar
    // base plus this lane's fixed byte offset, kept in registers: no VALU
    // address work per DMA. Other blocks recompute the offsets.
    const bool soff = (int64_t)BKV * (a.ks2 > a.vs2 ? a.ks2 : a.vs2) * 4 < (1ll << 31);
    uint32_t kbo[PT], vbo[PT];
#pragma unroll
    for (int i = 0; i < PT; ++i) {
        kbo[i] = (uint32_t)koff(i) * 4u;
        vbo[i] = (uint32_t)voff(i) * 4u;
    }
    const uint32_t ldsK0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)&sK[wave * 64]);
    const uint32_t ldsV0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)&sV[wave * 64]);
    // block kb into the stage of list position j
    auto issue = [&](int j, int kb) {
        const int k0 = kb * BKV;
        u32x4* dK = sK + (j & 1) * STG;
        u32x4* dV = sV + (j & 1) * STG;
        const float* kbase = Kp + (int64_t)k0 * a.ks2;
        const float* vbase = Vp + (int64_t)k0 * a.vs2;
        if (k0 + BKV <= a.Skv && soff) {
            const uint32_t lk = ldsK0 + (uint32_t)((j & 1) * STG) * 16u;
            const uint32_t lv = ldsV0 + (uint32_t)((j & 1) * STG) * 16u;
#pragma unroll
            for (int i = 0; i < PT; ++i) {
                dma16_soff(kbase, kbo[i], lk + (uint32_t)(i * 64 * NW) * 16u);
                dma16_soff(vbase, vbo[i], lv + (uint32_t)(i * 64 * NW) * 16u);
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < PT; ++i) {
            // rows past the end re-read the last key (masked, never used)
            const int row = slot_row(i);
            const int sh = min(k0 + row, a.Skv - 1) - k0 - row;
            dma16_async(kbase + koff(i) + sh * (int)a.ks2, &dK[i * 64 * NW + wave * 64]);
            dma16_async(vbase + voff(i) + sh * (int)a.vs2, &dV[i * 64 * NW + wave * 64]);
        }
    };

    float m = -INFINITY, lsum = 0.f;
    f32x4 o[NB];
#pragma unroll
    for (int t = 0; t < NB; ++t) o[t] = f32x4{0.f, 0.f, 0.f, 0.f};

    // MODE 2 with the mask's tile classes (a.tcls, from mask_tile_class_kernel):
    // the workgroup lists, in key order, the 64-key blocks some of its rows see
    // and stages only those (a block no row sees would leave p = 0 and alpha = 1:
    // the same bits). Otherwise every block up to nkb is visited.
    __shared__ uint16_t slist[MODE == 2 ? PP_LIST_MAX : 1];
    __shared__ int s_wcnt[NW];
    const bool listed = MODE == 2 && a.tcls != nullptr;
    int nvis = nkb;
    if constexpr (MODE == 2) {
        if (listed) {
            const int rg0 = qb * BQ / 32, rg1 = min(qb * BQ + BQ - 1, a.Sq - 1) / 32;
            int base = 0;
            for (int c0 = 0; c0 < nkb_all; c0 += 64 * NW) {
                const int kb = c0 + tid;
                bool any = false;
                if (kb < nkb_all)
                    for (int rg = rg0; rg <= rg1; ++rg) any = any || (a.tcls[(int64_t)rg * a.nkbt + kb] & 1) != 0;
                const uint64_t bal = __ballot(any);
                if (lane == 0) s_wcnt[wave] = __popcll(bal);
                __syncthreads();
                int before = __popcll(bal & ((1ull << lane) - 1ull)), total = 0;
#pragma unroll
                for (int w = 0; w < NW; ++w) {
                    before += w < wave ? s_wcnt[w] : 0;
                    total += s_wcnt[w];
                }
                if (any) slist[base + before] = (uint16_t)kb;
                base += total;
                __syncthreads();
            }
            nvis = base;
        }
    }
    auto block_at = [&](int j) -> int { return listed ? __builtin_amdgcn_readfirstlane((int)slist[j]) : j; };

    if (nvis > 0) issue(0, block_at(0));
    for (int j = 0; j < nvis; ++j) {
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        const int kb = block_at(j);
        if (j + 1 < nvis) issue(j + 1, block_at(j + 1));
        const int k0 = kb * BKV;
        if (!wave_rows) continue;
        if constexpr (MODE == 1) {
            if (k0 + kofs > q0 + 15 + a.diag_off) continue;  // past every row of this wave
        }
        // per-element inputs of MODE 2, issued before the score MFMAs
        uint8_t mk[NKT][4];
        float bv[NKT][4];
        uint32_t mw[NKT];   // a mask alone with 4-byte aligned rows: the lane's 4 bytes of each 16-key tile
        bool mall = false;  // ... every score of the wave's block visible
        if constexpr (MODE == 2) {
            const int qr = min(qrow, a.Sq - 1);
            if (a.mask_words) {
                // Four word loads instead of sixteen byte loads, and the block's class
                // for the wave's rows: none visible -> skip it (its p would all be 0
                // and alpha 1, the same bits), all visible -> no per-score test.
                const uint8_t* mrow = a.mask + (int64_t)qr * a.mask_ld;
                bool any = false, all = true;
#pragma unroll
                for (int kt = 0; kt < NKT; ++kt) {
                    const int key = k0 + kofs + kt * 16 + 4 * g;
                    uint32_t w = 0;
                    if (key + 3 < a.Skv) {
                        w = *reinterpret_cast<const uint32_t*>(mrow + key);
                    } else {
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            if (key + i < a.Skv) w |= (uint32_t)mrow[key + i] << (8 * i);
                    }
                    mw[kt] = w;
                    any = any || w != 0;
                    all = all && ((w - 0x01010101u) & ~w & 0x80808080u) == 0;  // no zero byte
                }
                if (__ballot(any) == 0) continue;  // no row of this wave sees a key of the block
                mall = __ballot(!all) == 0;
            } else {
#pragma unroll
                for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int key = min(k0 + kofs + kt * 16 + 4 * g + i, a.Skv - 1);
                        mk[kt][i] = a.mask != nullptr ? a.mask[(int64_t)qr * a.mask_ld + key] : (uint8_t)1;
                        bv[kt][i] = a.bias != nullptr ? a.bias[(int64_t)qr * a.brs + (int64_t)key * a.bcs] * LOG2E : 0.f;
                    }
            }
        }
        const u32x4* cK = sK + (j & 1) * STG;
        const float* cV = reinterpret_cast<const float*>(sV + (j & 1) * STG);
        f32x4 s[NKT];
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt) s[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int bb = 0; bb < NB; ++bb) {
            f32x4 kf[NKT];
#pragma unroll
            for (int kt = 0; kt < NKT; ++kt) {
                const int key = kofs + kt * 16 + r;
                kf[kt] = __builtin_bit_cast(f32x4, cK[key * KCH + ((4 * bb + g) ^ (key & 15))]);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int kt = 0; kt < NKT; ++kt)
                    s[kt] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[kt][j], qf[bb][j], s[kt], 0, 0, 0);
        }
        // visibility, the block's row maximum, probabilities
        float mx = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int key = k0 + kofs + kt * 16 + 4 * g + i;
                bool vis = key < a.Skv;
                if constexpr (MODE == 1) vis = vis && key <= qrow + a.diag_off;
                float x = s[kt][i];
                if constexpr (MODE == 2) {
                    if (a.mask_words) {
                        vis = vis && (mall || ((mw[kt] >> (8 * i)) & 0xffu) != 0);
                    } else {
                        vis = vis && mk[kt][i] != 0;
                        x += bv[kt][i];
                    }
                }
                s[kt][i] = vis ? x : -INFINITY;
                mx = fmaxf(mx, s[kt][i]);
            }
        mx = max_across_rows(mx);
        const float m_new = fmaxf(m, mx);
        const float m_use = m_new == -INFINITY ? 0.f : m_new;
        const float alpha = exp2f(m - m_use);  // 0 while no key was visible
        float psum = 0.f;
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float p = exp2f(s[kt][i] - m_use);  // masked: exp2(-inf) = 0
                s[kt][i] = p;
                psum += p;
            }
        lsum = fmaf(lsum, alpha, psum);
        m = m_new;
#pragma unroll
        for (int t = 0; t < NB; ++t) o[t] *= alpha;
        // O^T += V^T . P^T over this wave's keys of the block
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int key = kofs + kt * 16 + 4 * g + j;
                const float* vrow = cV + key * D + r;
#pragma unroll
                for (int t = 0; t < NB; ++t) {
                    const float vf = vrow[((t ^ g) << 4)];
                    o[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf, s[kt][j], o[t], 0, 0, 0);
                }
            }
    }
    if constexpr (KS == 2) {
        // Every wave is past the last barrier's reads: the K stages are free.
        // Group 1 leaves O, m and l of each lane; group 0 merges them.
        __syncthreads();
        float* xo = reinterpret_cast<float*>(sK);
        const int slot = (wl * 64 + lane) * (4 * NB + 2);
        if (wave >= 4) {
#pragma unroll
            for (int t = 0; t < NB; ++t)
#pragma unroll
                for (int i = 0; i < 4; ++i) xo[slot + 4 * t + i] = o[t][i];
            xo[slot + 4 * NB] = m;
            xo[slot + 4 * NB + 1] = lsum;
        }
        __syncthreads();
        if (wave >= 4) return;
        const float m1 = xo[slot + 4 * NB], l1 = xo[slot + 4 * NB + 1];
        // a group that saw no visible key has m = -inf and weight 0
        const float mt = fmaxf(m, m1);
        const float a0 = m == -INFINITY ? 0.f : exp2f(m - mt);
        const float a1 = m1 == -INFINITY ? 0.f : exp2f(m1 - mt);
#pragma unroll
        for (int t = 0; t < NB; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) o[t][i] = o[t][i] * a0 + xo[slot + 4 * t + i] * a1;
        lsum = lsum * a0 + l1 * a1;
    }
    if (!wave_rows || qrow >= a.Sq) return;
    // the query's denominator: the sum of its 4 lanes' partials
    float lt = lsum;
    {
        const uint32_t u = __float_as_uint(lt);
        const auto p16 = __builtin_amdgcn_permlane16_swap(u, u, false, false);
        lt = __uint_as_float(p16[0]) + __uint_as_float(p16[1]);
        const uint32_t w = __float_as_uint(lt);
        const auto p32 = __builtin_amdgcn_permlane32_swap(w, w, false, false);
        lt = __uint_as_float(p32[0]) + __uint_as_float(p32[1]);
    }
    const float inv = lt > 0.f ? 1.0f / lt : 0.f;
    float* orow = Op + (int64_t)qrow * a.os2;
#pragma unroll
    for (int t = 0; t < NB; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) orow[(16 * t + 4 * g + i) * a.os3] = lt > 0.f ? o[t][i] * inv : 0.f;
}

// ---------------------------------------------------------------------------
// Decode
// ---------------------------------------------------------------------------
struct DecodeArgs {
    const void* Q;
    const void* K;
    const void* V;
    void* O;
    int64_t qs0, qs1, os0, os1, ks0, ks1, ks2, vs0, vs1, vs2;
    const int32_t* kv_len;
    // Masked single-query calls routed from ythip_attn_prefill (the q_len == 1
    // branch of flash_attention, src/kernel/avx2/flash_attention.inl:469-499):
    // key j is visible iff mask[j] != 0 (row 0 of a bool mask; NULL = all) and
    // bias[j * bcs] (fp32; NULL = none) is added to its scaled score. Only the
    // MK instantiations read them.
    const uint8_t* mask;
    const float* bias;
    int64_t bcs;
    int B, Hq, Hkv, max_ctx, splits;  // keys per split: decode_chunk(kv_len, splits)
    float scale_log2;
    float* ws;  // [B, Hq, splits, D + 2]
    // fused decode step (ythip_attn_decode_rope): the new token's q/k/v come
    // from its qkv row; q and k get RMSNorm + RoPE at position *dev_pos, and
    // k and v are appended to the cache there before the keys are read.
    const void* qkv;
    int64_t ld_qkv;
    const float* wq;
    const float* wk;
    float eps;
    const float* cos_tab;
    const float* sin_tab;
    int64_t ld_tab;
    int tab_rows;
    int32_t* dev_state;  // decode-state record: RoPE row, cache slot, visible keys
    int fused;
    int direct;  // splits == 1 and O given: the split kernel writes O itself
};

constexpr int DEC_GMAX = 8;

// Rounds 8 values to the storage type T and back (what a store and a reload give).
template <class T>
__device__ __forceinline__ void round8(float (&x)[8]) {
    if constexpr (sizeof(typename T::raw) == 2) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t w = pack2<T>(x[2 * e], x[2 * e + 1]);
            x[2 * e] = lo_as_f32(T{}, w);
            x[2 * e + 1] = hi_as_f32(T{}, w);
        }
    }
}

template <class T>
__device__ __forceinline__ void store8_raw(typename T::raw* p, const float (&x)[8]) {
    if constexpr (sizeof(typename T::raw) == 2) {
        *reinterpret_cast<u32x4*>(p) = u32x4{pack2<T>(x[0], x[1]), pack2<T>(x[2], x[3]), pack2<T>(x[4], x[5]),
                                             pack2<T>(x[6], x[7])};
    } else {
        reinterpret_cast<f32x4*>(p)[0] = f32x4{x[0], x[1], x[2], x[3]};
        reinterpret_cast<f32x4*>(p)[1] = f32x4{x[4], x[5], x[6], x[7]};
    }
}

// D = 8 * LPK (LPK lanes per key, 8 elements each); G query heads per kv head.
// FUSED: see DecodeArgs; the per-head RMSNorm / RoPE arithmetic is that of
// norm_rope_kernel, so the fused step gives the same bits as
// ythip_rmsnorm_rope followed by ythip_attn_decode.
// NTH threads per workgroup: 512 (twice the keys in flight, so a split of up to
// 128 keys is one batch) when the grid is too small to cover the CUs.
// MK: a per-key byte mask and / or bias (DecodeArgs::mask, ::bias) take part.
template <class T, int D, int G, bool FUSED, int NTH, bool MK = false>
__global__ __launch_bounds__(NTH) void attn_decode_split(DecodeArgs a) {
    static_assert(!(FUSED && MK), "the fused decode step takes no mask");
    using raw = typename T::raw;
    constexpr int LPK = D / 8;          // lanes per key
    constexpr int SLOTS = NTH / LPK;    // keys in flight per workgroup
    constexpr int UNR = 4;
    const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x;
    const int slot = tid / LPK, part = tid % LPK;
    // Fused: the new token's q rows (and its k / v rows, used by the workgroup that
    // owns the position) and the norm weights are loaded before anything else,
    // in parallel with the position read; the RoPE rows follow once the position
    // is known, then the first K/V batch. (Vector-memory loads retire in issue
    // order: loading the rows after the batch would make their wait cover it.)
    constexpr int HALF = D / 2, LPR = HALF / 8;
    constexpr int RW = sizeof(raw) == 2 ? 1 : 2;  // u32x4 per 8 elements
    const bool prow = FUSED && tid < (G + 2) * LPR;
    const int pr = tid / LPR, pj = tid % LPR;
    u32x4 r1[RW], r2[RW];
    f32x4 wv[4], cs[4];
    if constexpr (FUSED) {
        if (prow) {
            const int head = pr < G ? kvh * G + pr : (pr == G ? a.Hq + kvh : a.Hq + a.Hkv + kvh);
            const raw* src = static_cast<const raw*>(a.qkv) + (int64_t)b * a.ld_qkv + (int64_t)head * D + 8 * pj;
#pragma unroll
            for (int i = 0; i < RW; ++i) {
                r1[i] = reinterpret_cast<const u32x4*>(src)[i];
                r2[i] = reinterpret_cast<const u32x4*>(src + HALF)[i];
            }
            const float* w = pr < G ? a.wq : (pr == G ? a.wk : nullptr);
            if (pr <= G && w != nullptr) {
                wv[0] = reinterpret_cast<const f32x4*>(w + 8 * pj)[0];
                wv[1] = reinterpret_cast<const f32x4*>(w + 8 * pj)[1];
                wv[2] = reinterpret_cast<const f32x4*>(w + HALF + 8 * pj)[0];
                wv[3] = reinterpret_cast<const f32x4*>(w + HALF + 8 * pj)[1];
            }
        }
    }
    int len, pos = -1, rpos = 0;
    bool owner = false;  // FUSED: this workgroup's chunk holds the new token's cache row
    bool rope_ok = false;
    if constexpr (FUSED) {
        // the new token's cache row (ring slot), RoPE row and visible keys; rows
        // out of range are flagged and never used as addresses
        pos = a.dev_state[YTHIP_ST_SLOT];
        rpos = a.dev_state[YTHIP_ST_ROPE_POS];
        len = max(0, min(a.dev_state[YTHIP_ST_KV_LEN], a.max_ctx));
        const bool slot_ok = pos >= 0 && pos < a.max_ctx;
        rope_ok = rpos >= 0 && rpos < a.tab_rows;
        // the split whose chunk holds the row (the last split for a row past them all)
        owner = slot_ok && min(pos / decode_chunk(len, a.splits), a.splits - 1) == split;
        if (tid == 0 && split == 0 && kvh == 0 && b == 0) {
            if (!slot_ok) atomicOr(&a.dev_state[YTHIP_ST_ERROR], (int)YTHIP_ST_ERR_CACHE);
            if (a.cos_tab != nullptr && !rope_ok) atomicOr(&a.dev_state[YTHIP_ST_ERROR], (int)YTHIP_ST_ERR_ROPE);
        }
    } else {
        len = a.kv_len ? max(0, min(a.kv_len[b], a.max_ctx)) : a.max_ctx;
    }
    // this split's keys [kb0, kend) of the len visible ones (none when kb0 >= len);
    // keys past kend load the row kbeg instead, which stays inside the cache
    const int chunk = decode_chunk(len, a.splits);
    const int kb0 = split * chunk;
    const int kend = min(len, kb0 + chunk);
    const int kbeg = min(kb0, max(a.max_ctx - 1, 0));
    if (kb0 >= len && !owner) {
        // a split past the visible keys (a short context in a large ring): the
        // partials of an empty split, m = -inf, l = 0, o = 0 (zeros when direct),
        // the values the key loop below would leave
        for (int idx = tid; idx < G * D; idx += NTH) {
            const int gi = idx / D, d = idx % D, h = kvh * G + gi;
            if (a.direct) {
                store_from_f32<T>(a.O, b * a.os0 + h * a.os1 + d, 0.f);
                continue;
            }
            float* dst = a.ws + (((int64_t)b * a.Hq + h) * a.splits + split) * (D + 2);
            dst[2 + d] = 0.f;
            if (d == 0) {
                dst[0] = -INFINITY;
                dst[1] = 0.f;
            }
        }
        return;
    }

    float m[G], l[G], o[G][8];
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
        m[gi] = -INFINITY;
        l[gi] = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[gi][e] = 0.f;
    }
    const raw* Kb = static_cast<const raw*>(a.K) + b * a.ks0 + kvh * a.ks1 + part * 8;
    const raw* Vb = static_cast<const raw*>(a.V) + b * a.vs0 + kvh * a.vs1 + part * 8;

    // K/V of keys [k0, k0 + SLOTS * UNR) (this lane's 8 elements), clamped rows for
    // keys past the end (loaded but never used). The batch stays in its raw form
    // until the key loop unpacks it: converting right after the loads would make
    // the kernel wait for the batch there, before the work it is meant to overlap.
    constexpr int KW = sizeof(raw) == 2 ? 1 : 2;  // u32x4 per 8 elements
    u32x4 kr[UNR][KW], vr[UNR][KW];
    float kx[UNR][8], vx[UNR][8];
    bool ok[UNR];
    uint8_t mkb[UNR];  // MK: the keys' mask bytes
    float bsv[UNR];    // MK: the keys' bias values
    auto load_batch = [&](int k0) {
#pragma unroll
        for (int u = 0; u < UNR; ++u) {
            const int key = k0 + u * SLOTS;
            ok[u] = key < kend;
            const int kk = ok[u] ? key : kbeg;
            const raw* kp = Kb + (int64_t)kk * a.ks2;
            const raw* vp = Vb + (int64_t)kk * a.vs2;
            if constexpr (MK) {
                mkb[u] = a.mask != nullptr ? a.mask[kk] : (uint8_t)1;
                bsv[u] = a.bias != nullptr ? a.bias[(int64_t)kk * a.bcs] : 0.f;
            }
#pragma unroll
            for (int i = 0; i < KW; ++i) {
                // streamed once: non-temporal loads (measured ~10% more HBM read rate)
                kr[u][i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(kp) + i);
                vr[u][i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(vp) + i);
            }
        }
    };
    auto unpack_batch = [&]() {
#pragma unroll
        for (int u = 0; u < UNR; ++u) {
            if constexpr (sizeof(raw) == 2) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t kw = kr[u][0][e], vw = vr[u][0][e];
                    kx[u][2 * e] = lo_as_f32(T{}, kw);
                    kx[u][2 * e + 1] = hi_as_f32(T{}, kw);
                    vx[u][2 * e] = lo_as_f32(T{}, vw);
                    vx[u][2 * e + 1] = hi_as_f32(T{}, vw);
                }
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    kx[u][e] = __uint_as_float(kr[u][0][e]);
                    kx[u][e + 4] = __uint_as_float(kr[u][1][e]);
                    vx[u][e] = __uint_as_float(vr[u][0][e]);
                    vx[u][e + 4] = __uint_as_float(vr[u][1][e]);
                }
            }
        }
    };
    // Fused: the RoPE rows of the position, then the first K/V batch.
    if constexpr (FUSED) {
        if (prow && pr <= G && a.cos_tab != nullptr && rope_ok) {
            const int64_t t = (int64_t)rpos * a.ld_tab + 8 * pj;
            cs[0] = *reinterpret_cast<const f32x4*>(a.cos_tab + t);
            cs[1] = *reinterpret_cast<const f32x4*>(a.cos_tab + t + 4);
            cs[2] = *reinterpret_cast<const f32x4*>(a.sin_tab + t);
            cs[3] = *reinterpret_cast<const f32x4*>(a.sin_tab + t + 4);
        }
    }
    // issued unconditionally (rows past the end are clamped and masked): a branch
    // around the loads would make the compiler's wait before the prologue
    // arithmetic cover the batch as well
    int k0 = kb0 + slot;
    load_batch(k0);

    float q[G][8];
    __shared__ float s_new[FUSED ? (G + 2) * D : 1];  // normed + roped q heads, then k, then v
    if constexpr (FUSED) {
        // norm_rope_kernel's arithmetic, one LPR-lane group per row (k / v rows only
        // in the workgroup that owns the position)
        if (prow && (pr < G || owner)) {
            const int r = pr, j = pj;
            float x1[8], x2[8];
            auto unpack8 = [&](const u32x4 (&rw)[RW], float (&x)[8]) {
                if constexpr (sizeof(raw) == 2) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const uint32_t we = rw[0][e];
                        x[2 * e] = lo_as_f32(T{}, we);
                        x[2 * e + 1] = hi_as_f32(T{}, we);
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        x[e] = __uint_as_float(rw[0][e]);
                        x[e + 4] = __uint_as_float(rw[RW - 1][e]);
                    }
                }
            };
            unpack8(r1, x1);
            unpack8(r2, x2);
            const float* w = r < G ? a.wq : (r == G ? a.wk : nullptr);
            if (r <= G && w != nullptr) {
                float ss = 0.f;
#pragma unroll
                for (int e = 0; e < 8; ++e) ss = fmaf(x2[e], x2[e], fmaf(x1[e], x1[e], ss));
#pragma unroll
                for (int off = LPR / 2; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, 64);
                const float den = sqrtf(ss / (float)D + a.eps);
                const f32x4 wa = wv[0], wb = wv[1], wc = wv[2], wd = wv[3];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    x1[e] = (x1[e] / den) * wa[e];
                    x1[e + 4] = (x1[e + 4] / den) * wb[e];
                    x2[e] = (x2[e] / den) * wc[e];
                    x2[e + 4] = (x2[e + 4] / den) * wd[e];
                }
            }
            if (r <= G && a.cos_tab != nullptr && rope_ok) {
                const f32x4 c0 = cs[0], c1 = cs[1], s0 = cs[2], s1 = cs[3];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float c = e < 4 ? c0[e] : c1[e - 4], sn = e < 4 ? s0[e] : s1[e - 4];
                    const float y1 = fmaf(x1[e], c, -(x2[e] * sn));
                    const float y2 = fmaf(x2[e], c, x1[e] * sn);
                    x1[e] = y1;
                    x2[e] = y2;
                }
            }
            round8<T>(x1);
            round8<T>(x2);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                s_new[r * D + 8 * j + e] = x1[e];
                s_new[r * D + HALF + 8 * j + e] = x2[e];
            }
            if (r >= G) {  // append k (r == G) or v to the cache at `pos`
                raw* dst = r == G ? static_cast<raw*>(const_cast<void*>(a.K)) + b * a.ks0 + kvh * a.ks1 +
                                        (int64_t)pos * a.ks2
                                  : static_cast<raw*>(const_cast<void*>(a.V)) + b * a.vs0 + kvh * a.vs1 +
                                        (int64_t)pos * a.vs2;
                store8_raw<T>(dst + 8 * j, x1);
                store8_raw<T>(dst + HALF + 8 * j, x2);
            }
        }
        __syncthreads();
#pragma unroll
        for (int gi = 0; gi < G; ++gi)
#pragma unroll
            for (int e = 0; e < 8; ++e) q[gi][e] = s_new[gi * D + part * 8 + e] * a.scale_log2;
    } else {
#pragma unroll
        for (int gi = 0; gi < G; ++gi) {
            const int h = kvh * G + gi;
            const raw* qp = static_cast<const raw*>(a.Q) + b * a.qs0 + h * a.qs1 + part * 8;
#pragma unroll
            for (int e = 0; e < 8; ++e) q[gi][e] = load_as_f32<T>(qp, e) * a.scale_log2;
        }
    }

    for (; k0 < kend; k0 += SLOTS * UNR) {
        unpack_batch();
        if constexpr (FUSED) {
            if (owner) {  // the token appended above: its k / v from LDS, not the cache row
#pragma unroll
                for (int u = 0; u < UNR; ++u)
                    if (k0 + u * SLOTS == pos) {
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            kx[u][e] = s_new[G * D + part * 8 + e];
                            vx[u][e] = s_new[(G + 1) * D + part * 8 + e];
                        }
                    }
            }
        }
#pragma unroll
        for (int gi = 0; gi < G; ++gi) {
            float sc[UNR];
            float mx = m[gi];
#pragma unroll
            for (int u = 0; u < UNR; ++u) {
                float sv = 0.f;
#pragma unroll
                for (int e = 0; e < 8; ++e) sv = fmaf(q[gi][e], kx[u][e], sv);
                sv = dpp_sum_group<LPK>(sv);
                if constexpr (MK) {
                    // the bias is added after scaling, in the kernel's log2 units
                    sc[u] = ok[u] && mkb[u] != 0 ? fmaf(bsv[u], LOG2E, sv) : -INFINITY;
                } else {
                    sc[u] = ok[u] ? sv : -INFINITY;
                }
                mx = fmaxf(mx, sc[u]);
            }
            // One correction per UNR keys; the running max stays finite once any key was seen.
            const float m_use = (mx == -INFINITY) ? 0.f : mx;
            const float corr = __builtin_amdgcn_exp2f(m[gi] - m_use);
            float psum = 0.f;
            float p[UNR];
#pragma unroll
            for (int u = 0; u < UNR; ++u) {
                p[u] = __builtin_amdgcn_exp2f(sc[u] - m_use);
                psum += p[u];
            }
            l[gi] = fmaf(l[gi], corr, psum);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                float acc = o[gi][e] * corr;
#pragma unroll
                for (int u = 0; u < UNR; ++u) acc = fmaf(p[u], vx[u][e], acc);
                o[gi][e] = acc;
            }
            m[gi] = mx;
        }
        if (k0 + SLOTS * UNR < kend) load_batch(k0 + SLOTS * UNR);
    }

    // Merge the SLOTS key slots of this workgroup: LDS holds per slot (m, l) and o.
    __shared__ float s_ml[SLOTS][G][2];
    __shared__ float s_o[SLOTS][G][D];
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
        if (part == 0) {
            s_ml[slot][gi][0] = m[gi];
            s_ml[slot][gi][1] = l[gi];
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) s_o[slot][gi][part * 8 + e] = o[gi][e];
    }
    __syncthreads();
    // NTH = 512 (32 slots): slot weights once per (head, slot) -- one wave per head,
    // lane = slot, the max and the weighted l as wave reductions (a slot that saw
    // no key has m = -inf and o = 0, so weight 0 drops it) -- so the per-element
    // loop is a plain FMA chain. NTH = 256 (16 slots, long splits) keeps the
    // per-element loop, which measured faster there.
    static_assert(SLOTS <= 64, "one lane per slot");
    __shared__ float s_w[NTH == 512 ? G : 1][SLOTS];
    __shared__ float s_ML[G][2];
    if constexpr (NTH == 512) {
        for (int t = tid; t < G * 64; t += NTH) {
            const int gi = t / 64, sl = t % 64;
            const float ms = sl < SLOTS ? s_ml[sl][gi][0] : -INFINITY;
            const float M = lane63(dpp_max_to_lane63(ms));
            const float w = (M != -INFINITY && ms != -INFINITY) ? __builtin_amdgcn_exp2f(ms - M) : 0.f;
            const float L = lane63(dpp_sum_to_lane63(sl < SLOTS ? s_ml[sl][gi][1] * w : 0.f));
            if (sl < SLOTS) s_w[gi][sl] = w;
            if (sl == 0) {
                s_ML[gi][0] = M;
                s_ML[gi][1] = L;
            }
        }
        __syncthreads();
    }
    float* ws = a.ws;
    for (int idx = tid; idx < G * D; idx += NTH) {
        const int gi = idx / D, d = idx % D;
        float M, L, acc = 0.f;
        if constexpr (NTH == 512) {
            M = s_ML[gi][0];
            L = s_ML[gi][1];
#pragma unroll
            for (int sl = 0; sl < SLOTS; ++sl) acc = fmaf(s_o[sl][gi][d], s_w[gi][sl], acc);
        } else {
            M = -INFINITY;
            L = 0.f;
            for (int sl = 0; sl < SLOTS; ++sl) M = fmaxf(M, s_ml[sl][gi][0]);
            if (M != -INFINITY) {
                for (int sl = 0; sl < SLOTS; ++sl) {
                    const float ms = s_ml[sl][gi][0];
                    if (ms == -INFINITY) continue;
                    const float w = __builtin_amdgcn_exp2f(ms - M);
                    L = fmaf(s_ml[sl][gi][1], w, L);
                    acc = fmaf(s_o[sl][gi][d], w, acc);
                }
            }
        }
        const int h = kvh * G + gi;
        if (a.direct) {
            // one split: attn_decode_merge over a single partial is acc / L
            // (its weight exp2(M - M) is exactly 1), stored straight away
            const float out = L > 0.f ? acc / L : 0.f;
            store_from_f32<T>(a.O, b * a.os0 + h * a.os1 + d, out);
            continue;
        }
        float* dst = ws + (((int64_t)b * a.Hq + h) * a.splits + split) * (D + 2);
        dst[2 + d] = acc;
        if (d == 0) {
            dst[0] = M;
            dst[1] = L;
        }
    }
}

// One workgroup per (head, batch), one thread per d. The splits' m and l go
// through LDS and every o_s[d] is loaded up front (splits <= DEC_MAX_SPLITS),
// so the merge pays one memory round trip; the arithmetic is the sequential
// log-sum-exp combine over s = 0, 1, ... (the order the o projection's merge
// prologue reproduces).
// At most 32 splits: a batch-1, 16-head (8 kv-head) call then fills 256
// workgroups, one per CU, of 512 threads (a 40960-row ring: 1203 -> 1318 tok/s
// for the Qwen3-0.6B decode step, batch 1 ctx 8192 11.95 -> 11.4 us).
constexpr int DEC_MAX_SPLITS = 32;
template <class T, int D, int MAXS>  // MAXS >= splits: 8 or DEC_MAX_SPLITS
__global__ __launch_bounds__(D) void attn_decode_merge(DecodeArgs a) {
    static_assert(MAXS <= D, "one thread stages each split's m and l");
    const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
    const float* src = a.ws + ((int64_t)b * a.Hq + h) * a.splits * (D + 2);
    const int S = a.splits;
    __shared__ float s_m[D], s_l[D];  // every thread stores (no branch to sink loads into)
    // Every load is issued before the first wait, m and l first: indices past
    // the last split re-read it (their values are unused), so no load sits
    // behind a branch and the waits count down split by split.
    const float* ml = src + min(d, S - 1) * (D + 2);
    const float mv = ml[0], lv = ml[1];
    float ov[MAXS];
#pragma unroll
    for (int q = 0; q < MAXS; ++q) ov[q] = src[min(q, S - 1) * (D + 2) + 2 + d];
    s_m[d] = d < S ? mv : -INFINITY;
    s_l[d] = lv;
    __syncthreads();
    float M = -INFINITY;
#pragma unroll
    for (int q = 0; q < MAXS; ++q) M = fmaxf(M, s_m[q]);
    // Empty splits (m = -inf, also the padding) get weight 0: every split
    // writes finite l and o, so their terms add exact zeros and the result
    // has the bits of skipping them in the sequential combine. Thread q
    // computes split q's weight once for the workgroup.
    __shared__ float s_w[MAXS];
    if (d < MAXS) s_w[d] = s_m[d] != -INFINITY ? exp2f(s_m[d] - M) : 0.f;
    __syncthreads();
    float L = 0.f, acc = 0.f;
#pragma unroll
    for (int q = 0; q < MAXS; ++q) {
        const float w = s_w[q];
        L = fmaf(s_l[q], w, L);
        acc = fmaf(ov[q], w, acc);
    }
    const float out = L > 0.f ? acc / L : 0.f;
    store_from_f32<T>(a.O, b * a.os0 + h * a.os1 + d, out);
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
namespace {

bool al(const void* p, int bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }

// Compute units of the current device (queried once per device).
int device_cus() {
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cus[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

template <class T, int D, int GH, int QT, int NKT = 4>
hipError_t launch_prefill_gh(AttnArgs a, int mode, hipStream_t s) {
    constexpr int BQ = 64 * QT;
    a.nqb = (a.Sq + BQ - 1) / BQ;
    dim3 grid(a.nqb * a.B * a.Hq / GH);
    // 4-wave workgroups run two per CU: a grid of at most two per CU is resident at once
    a.balance = (GH == 1 && (int64_t)grid.x <= 2 * (int64_t)device_cus()) ? 1 : 0;
    // paired heads take 128-key blocks, except the staged mask (64-key blocks)
    constexpr bool paired_mask = GH == 2 && NKT == 4;
    if (mode == 3) {
        if constexpr (GH == 1 || paired_mask) attn_fwd_mfma<T, D, 3, GH, QT, NKT><<<grid, 256 * GH, 0, s>>>(a);
        else return hipErrorInvalidValue;
    } else if constexpr (paired_mask) {
        return hipErrorInvalidValue;
    } else {
        if (mode == 0) attn_fwd_mfma<T, D, 0, GH, QT, NKT><<<grid, 256 * GH, 0, s>>>(a);
        else if (mode == 1) attn_fwd_mfma<T, D, 1, GH, QT, NKT><<<grid, 256 * GH, 0, s>>>(a);
        else attn_fwd_mfma<T, D, 2, GH, QT, NKT><<<grid, 256 * GH, 0, s>>>(a);
    }
    return hipGetLastError();
}

// One head per 8-wave workgroup, 64 queries, 128-key stages split between the
// two wave groups (128 KB of LDS: one workgroup per CU, heaviest blocks first,
// each CU's next workgroup taken as the previous one ends).
template <class T, int D>
hipError_t launch_prefill_split(AttnArgs a, int mode, hipStream_t s) {
    a.nqb = (a.Sq + 63) / 64;
    a.balance = 0;
    dim3 grid(a.nqb * a.B * a.Hq);
    if (mode == 0) attn_fwd_mfma<T, D, 0, 1, 1, 4, 2><<<grid, 512, 0, s>>>(a);
    else if (mode == 1) attn_fwd_mfma<T, D, 1, 1, 1, 4, 2><<<grid, 512, 0, s>>>(a);
    else attn_fwd_mfma<T, D, 2, 1, 1, 4, 2><<<grid, 512, 0, s>>>(a);
    return hipGetLastError();
}

template <class T, int D>
hipError_t launch_prefill_mfma(AttnArgs a, int mode, hipStream_t s) {
    // Two query heads per workgroup (K/V staged once for both) when the GQA
    // group size is even and the paired grid still covers the 256 CUs twice;
    // without a byte mask those run the ping-pong kernel (S=8192 causal:
    // 248 us against 265 us for attn_fwd_mfma with 128-key blocks).
    const int64_t paired = (int64_t)((a.Sq + 127) / 128) * a.B * a.Hq / 2;
    // The staged bool mask pairs heads with 64-key blocks (80 KB of LDS): with
    // 128-key blocks K, V and the two mask tiles fill all 160 KB and the kernel
    // spills registers (measured slower).
    if ((a.Hq / a.Hkv) % 2 == 0 && paired >= 512) {
        if (mode == 3 && a.tcls != nullptr && a.Skv % 16 == 0) {
            // the mask's tile classes first, then the ping-pong kernel over the
            // blocks each workgroup's rows see (S=8192 causal bytes: 396 -> 2xx us)
            dim3 cgrid((a.Sq + 31) / 32, (a.nkbt + 15) / 16);
            mask_tile_class_kernel<<<cgrid, 256, 0, s>>>(a.mask, a.mask_ld, a.Sq, a.Skv, a.nkbt, a.tcls);
            a.nqb = (a.Sq + 127) / 128;
            dim3 grid(a.nqb * a.B * a.Hq / 2);
            attn_fwd_pingpong<T, D, 3><<<grid, 512, 0, s>>>(a);
            return hipGetLastError();
        }
        if (mode == 3) return launch_prefill_gh<T, D, 2, 2, 4>(a, mode, s);
        if (mode == 0 || mode == 1) {
            a.nqb = (a.Sq + 127) / 128;
            dim3 grid(a.nqb * a.B * a.Hq / 2);
            if (mode == 1) attn_fwd_pingpong<T, D, 1><<<grid, 512, 0, s>>>(a);
            else attn_fwd_pingpong<T, D, 0><<<grid, 512, 0, s>>>(a);
            return hipGetLastError();
        }
        // Per-element masks and biases (mode 2) run unpaired: the paired form
        // with 128-key blocks spills ~190 VGPRs and measured 1.8-2.1x slower
        // (B=2, S=4096, fp32 bias: 2396 against 1345 us).
    }
    // Short sequences: 16 queries per wave doubles the workgroups (two per CU)
    // and halves the per-block work on the longest causal row's serial chain;
    // without a staged mask the key split halves that chain again (S=2048
    // causal: 40.1 -> 35.5 us; S=512: 13.1 -> 11.9 us).
    const int64_t wgs = (int64_t)((a.Sq + 127) / 128) * a.B * a.Hq;
    if (wgs < 512 && mode != 3) return launch_prefill_split<T, D>(a, mode, s);
    // An additive bias (mode 2) keeps 16 queries per wave at any size: the
    // 32-query form spills 35 VGPRs (B=1, S=8192 bias: 3338 against 2738 us; a
    // byte mask read per element is 4% faster on 32 queries, and the bits agree)
    if (wgs < 512 || (mode == 2 && a.bias != nullptr)) return launch_prefill_gh<T, D, 1, 1>(a, mode, s);
    return launch_prefill_gh<T, D, 1, 2>(a, mode, s);
}

template <int D>
hipError_t launch_prefill_f32(AttnArgs a, int mode, hipStream_t s) {
    // a byte mask alone with 16-byte aligned rows and a workspace: its tile
    // classes first, then each workgroup stages only the blocks its rows see
    if (mode == 2 && a.tcls != nullptr && a.mask_words && al(a.mask, 16) && a.mask_ld % 16 == 0) {
        dim3 cgrid((a.Sq + 31) / 32, (a.nkbt + 15) / 16);
        mask_tile_class_kernel<<<cgrid, 256, 0, s>>>(a.mask, a.mask_ld, a.Sq, a.Skv, a.nkbt, a.tcls);
    } else {
        a.tcls = nullptr;
    }
    const int64_t nqb = (a.Sq + 127) / 128;
    if (nqb * a.B * a.Hq < 2 * (int64_t)device_cus()) {
        // fewer than two 128-query blocks per CU: 64-query blocks with the
        // keys of each staged block split between the two wave groups
        dim3 grid((unsigned)((a.Sq + 63) / 64 * a.B * a.Hq));
        if (mode == 1) attn_fwd_f32<D, 1, 2><<<grid, 512, 0, s>>>(a);
        else if (mode == 0) attn_fwd_f32<D, 0, 2><<<grid, 512, 0, s>>>(a);
        else attn_fwd_f32<D, 2, 2><<<grid, 512, 0, s>>>(a);
        return hipGetLastError();
    }
    dim3 grid((unsigned)(nqb * a.B * a.Hq));
    if (mode == 1) attn_fwd_f32<D, 1><<<grid, 512, 0, s>>>(a);
    else if (mode == 0) attn_fwd_f32<D, 0><<<grid, 512, 0, s>>>(a);
    else attn_fwd_f32<D, 2><<<grid, 512, 0, s>>>(a);
    return hipGetLastError();
}

template <class T>
hipError_t launch_rowwise(const AttnArgs& a, hipStream_t s) {
    dim3 grid(a.Sq, a.Hq, a.B);
    attn_rowwise<T><<<grid, 64, sizeof(float) * a.Skv, s>>>(a);
    return hipGetLastError();
}

template <class T>
int prefill_typed(AttnArgs a, hipStream_t s) {
    constexpr int es = sizeof(typename T::raw);
    const bool simple_mask = a.mask == nullptr && a.bias == nullptr;
    // a byte mask whose rows are 16-byte aligned is staged per key block (MODE 3)
    const bool stage_mask = a.mask != nullptr && a.bias == nullptr && !a.causal && al(a.mask, 16) &&
                            a.mask_ld % 16 == 0;
    const int mode = a.causal ? 1 : (simple_mask ? 0 : (stage_mask ? 3 : 2));
    const bool unit_d = a.qs3 == 1 && a.ks3 == 1 && a.vs3 == 1 && a.os3 == 1;
    const bool mfma_ok = es == 2 && unit_d && (a.D == 64 || a.D == 128) && a.Dv == a.D &&
                         !(a.causal && !simple_mask) &&
                         a.scale_log2 > 0.f &&
                         al(a.Q, 16) && al(a.K, 16) && al(a.V, 16) && al(a.O, 8) &&
                         a.qs0 % 8 == 0 && a.qs1 % 8 == 0 && a.qs2 % 8 == 0 && a.ks0 % 8 == 0 && a.ks1 % 8 == 0 &&
                         a.ks2 % 8 == 0 && a.vs0 % 8 == 0 && a.vs1 % 8 == 0 && a.vs2 % 8 == 0 &&
                         a.os0 % 4 == 0 && a.os1 % 4 == 0 && a.os2 % 4 == 0 &&
                         a.ks2 < (1 << 24) && a.vs2 < (1 << 24) && a.ks2 >= 0 && a.vs2 >= 0;
    if (mfma_ok) {
        if constexpr (es == 2) {
            if (a.D == 128) return status_of(launch_prefill_mfma<T, 128>(a, mode, s));
            return status_of(launch_prefill_mfma<T, 64>(a, mode, s));
        }
    }
    if constexpr (es == 4) {
        // fp32 on v_mfma_f32_16x16x4_f32: 16-byte aligned rows of Q, K and V
        // (K / V reach LDS by 16-byte DMA), 64 K / V rows within 2^31 elements
        const bool f32_ok = unit_d && (a.D == 64 || a.D == 128) && a.Dv == a.D && (int64_t)a.B * a.Hq < (1 << 30) &&
                            al(a.Q, 16) && al(a.K, 16) && al(a.V, 16) && a.qs0 % 4 == 0 && a.qs1 % 4 == 0 &&
                            a.qs2 % 4 == 0 && a.ks0 % 4 == 0 && a.ks1 % 4 == 0 && a.ks2 % 4 == 0 &&
                            a.vs0 % 4 == 0 && a.vs1 % 4 == 0 && a.vs2 % 4 == 0 && a.ks2 >= 0 && a.vs2 >= 0 &&
                            a.ks2 < (1 << 24) && a.vs2 < (1 << 24);
        if (f32_ok) {
            const int fmode = a.causal ? 1 : (simple_mask ? 0 : 2);
            if (a.D == 128) return status_of(launch_prefill_f32<128>(a, fmode, s));
            return status_of(launch_prefill_f32<64>(a, fmode, s));
        }
    }
    if (a.Skv > ROW_MAX)
        return fail(YTHIP_EUNSUPPORTED,
                    "ythip_attn_prefill: this layout/dtype uses the row-wise kernel, limited to kv_len <= %d",
                    ROW_MAX);
    return status_of(launch_rowwise<T>(a, s));
}

int decode_splits(int B, int Hq, int max_ctx) {
    const int bh = B * Hq > 0 ? B * Hq : 1;
    int s = (1024 + bh - 1) / bh;
    const int by_len = (max_ctx + 127) / 128;
    if (s > by_len) s = by_len;
    if (s > DEC_MAX_SPLITS) s = DEC_MAX_SPLITS;  // the merge holds one register per split
    if (s < 1) s = 1;
    return s;
}

// The workgroup size is a function of the launch shape only, so the fused and
// the unfused decode paths produce the same partials. 512 threads (32 keys in
// flight, a 128-key batch per round) while the grid holds at most one workgroup
// per CU; a larger grid keeps 256: the fused and masked kernels fit one
// 512-thread workgroup per CU, so more of them would run in two rounds.
inline bool decode_wide(int B, int Hkv, int splits, int G, int D) {
    return (int64_t)B * Hkv * splits <= 256 && (int64_t)(512 / (D / 8)) * G * D * 4 <= 64 * 1024;
}

template <class T, int D, int G>
hipError_t launch_decode_g(const DecodeArgs& a, hipStream_t s) {
    dim3 grid(a.splits, a.Hkv, a.B);
    const bool wide = decode_wide(a.B, a.Hkv, a.splits, G, D);
    const bool mk = a.mask != nullptr || a.bias != nullptr;
    if constexpr ((512 / (D / 8)) * G * D * 4 <= 64 * 1024) {
        if (wide) {
            if (a.fused) attn_decode_split<T, D, G, true, 512><<<grid, 512, 0, s>>>(a);
            else if (mk) attn_decode_split<T, D, G, false, 512, true><<<grid, 512, 0, s>>>(a);
            else attn_decode_split<T, D, G, false, 512><<<grid, 512, 0, s>>>(a);
        }
    }
    if (!wide) {
        if (a.fused) attn_decode_split<T, D, G, true, 256><<<grid, 256, 0, s>>>(a);
        else if (mk) attn_decode_split<T, D, G, false, 256, true><<<grid, 256, 0, s>>>(a);
        else attn_decode_split<T, D, G, false, 256><<<grid, 256, 0, s>>>(a);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.O == nullptr || a.direct) return e;  // O == NULL: the caller merges the partials
    if (a.splits <= 8) attn_decode_merge<T, D, 8><<<dim3(a.Hq, a.B), D, 0, s>>>(a);
    else attn_decode_merge<T, D, DEC_MAX_SPLITS><<<dim3(a.Hq, a.B), D, 0, s>>>(a);
    return hipGetLastError();
}

template <class T, int D>
hipError_t launch_decode_d(const DecodeArgs& a, int G, hipStream_t s) {
    switch (G) {
        case 1: return launch_decode_g<T, D, 1>(a, s);
        case 2: return launch_decode_g<T, D, 2>(a, s);
        case 4: return launch_decode_g<T, D, 4>(a, s);
        case 5: return launch_decode_g<T, D, 5>(a, s);  // e.g. Qwen3-14B, 40 q / 8 kv heads
        case 8: return launch_decode_g<T, D, 8>(a, s);
        default: return hipErrorInvalidValue;
    }
}

template <class T>
hipError_t launch_decode(const DecodeArgs& a, int D, int G, hipStream_t s) {
    if (D == 128) return launch_decode_d<T, 128>(a, G, s);
    return launch_decode_d<T, 64>(a, G, s);
}

// The q_len == 1 branch of flash_attention (src/kernel/avx2/flash_attention.inl:
// 469-499): every single-query call -- no mask, causal, diagonal predicate,
// bool mask, bias -- goes to the split-K decode kernel when its layout fits it
// (d == dv in {64, 128}, Hq / Hkv in {1, 2, 4, 5, 8}, contiguous head dim,
// 16-byte aligned K / V rows). Split-K partials go to the caller's workspace:
// as many splits as it holds, up to decode_splits (none: one split per
// (kv head, batch), written straight to O). Returns -1 when the call does not
// fit (the caller runs the prefill kernels), else the call's status.
int decode_route(int dtype, const AttnArgs& p, int mask_kind, const uint8_t* mask, int64_t mask_ld,
                 void* workspace, size_t ws_bytes, hipStream_t s) {
    if (p.Sq != 1 || p.Skv <= 0 || p.D != p.Dv || (p.D != 64 && p.D != 128)) return -1;
    const int G = p.Hq / p.Hkv;
    if (G != 1 && G != 2 && G != 4 && G != 5 && G != 8) return -1;
    if (p.qs3 != 1 || p.ks3 != 1 || p.vs3 != 1 || p.os3 != 1) return -1;
    const int es = dtype == YTHIP_F32 ? 4 : 2, ev = 16 / es;
    if (!al(p.K, 16) || !al(p.V, 16) || !al(p.Q, es) || !al(p.O, es)) return -1;
    if (p.ks0 % ev || p.ks1 % ev || p.ks2 % ev || p.vs0 % ev || p.vs1 % ev || p.vs2 % ev) return -1;
    // visible keys [0, n): a causal mask's single row sees every key
    // (offset kv_len - 1); a diagonal predicate j <= off sees off + 1 of them
    int64_t n = p.Skv;
    if (mask_kind == YTHIP_MASK_DIAG) n = std::max<int64_t>(0, std::min<int64_t>(mask_ld + 1, p.Skv));
    if (n == 0) return -1;  // no visible key: the prefill path writes the zero rows
    DecodeArgs a{};
    a.Q = p.Q; a.K = p.K; a.V = p.V; a.O = p.O;
    a.qs0 = p.qs0; a.qs1 = p.qs1; a.os0 = p.os0; a.os1 = p.os1;
    a.ks0 = p.ks0; a.ks1 = p.ks1; a.ks2 = p.ks2;
    a.vs0 = p.vs0; a.vs1 = p.vs1; a.vs2 = p.vs2;
    a.kv_len = nullptr;
    a.B = p.B; a.Hq = p.Hq; a.Hkv = p.Hkv; a.max_ctx = (int)n;
    const size_t per_split = (size_t)p.B * p.Hq * (p.D + 2) * sizeof(float);
    int splits = decode_splits(p.B, p.Hq, (int)n);
    if (workspace == nullptr || !al(workspace, 4)) splits = 1;
    else splits = (int)std::min<size_t>((size_t)splits, ws_bytes / per_split);
    if (splits < 1) splits = 1;
    a.splits = splits;
    a.direct = splits == 1;  // one split: the split kernel stores O, no merge
    a.scale_log2 = p.scale_log2;
    a.ws = splits > 1 ? static_cast<float*>(workspace) : nullptr;
    a.mask = mask_kind == YTHIP_MASK_BOOL ? mask : nullptr;
    a.bias = p.bias;
    a.bcs = p.bcs;
    switch (dtype) {
        case YTHIP_F32: return status_of(launch_decode<F32>(a, p.D, G, s));
        case YTHIP_F16: return status_of(launch_decode<F16>(a, p.D, G, s));
        default: return status_of(launch_decode<BF16>(a, p.D, G, s));
    }
}

}  // namespace

}  // namespace ythip

using namespace ythip;

extern "C" {

__attribute__((visibility("default"))) size_t ythip_attn_prefill_workspace_size(int q_len, int kv_len) {
    if (q_len <= 0 || kv_len <= 0) return 0;
    const size_t bytes = (size_t)((q_len + 31) / 32) * (size_t)((kv_len + 63) / 64);
    return (bytes + 255) / 256 * 256;
}

__attribute__((visibility("default"))) int ythip_attn_prefill_ws(
    int dtype, int B, int Hq, int Hkv, int q_len, int kv_len, int d, int dv, const void* Q, const int64_t q_str[4],
    const void* K, const int64_t k_str[4], const void* V, const int64_t v_str[4], void* O, const int64_t o_str[4],
    float scale, int mask_kind, const uint8_t* mask, int64_t mask_ld, const float* bias, int64_t rs_bias,
    int64_t cs_bias, void* workspace, size_t ws_bytes, void* stream);

__attribute__((visibility("default"))) int ythip_attn_prefill(
    int dtype, int B, int Hq, int Hkv, int q_len, int kv_len, int d, int dv, const void* Q, const int64_t q_str[4],
    const void* K, const int64_t k_str[4], const void* V, const int64_t v_str[4], void* O, const int64_t o_str[4],
    float scale, int mask_kind, const uint8_t* mask, int64_t mask_ld, const float* bias, int64_t rs_bias,
    int64_t cs_bias, void* stream) {
    return ythip_attn_prefill_ws(dtype, B, Hq, Hkv, q_len, kv_len, d, dv, Q, q_str, K, k_str, V, v_str, O, o_str,
                                 scale, mask_kind, mask, mask_ld, bias, rs_bias, cs_bias, nullptr, 0, stream);
}

__attribute__((visibility("default"))) int ythip_attn_prefill_ws(
    int dtype, int B, int Hq, int Hkv, int q_len, int kv_len, int d, int dv, const void* Q, const int64_t q_str[4],
    const void* K, const int64_t k_str[4], const void* V, const int64_t v_str[4], void* O, const int64_t o_str[4],
    float scale, int mask_kind, const uint8_t* mask, int64_t mask_ld, const float* bias, int64_t rs_bias,
    int64_t cs_bias, void* workspace, size_t ws_bytes, void* stream) {
    if (B < 0 || Hq < 0 || Hkv < 0 || q_len < 0 || kv_len < 0 || d < 0 || dv < 0)
        return fail(YTHIP_EINVAL, "ythip_attn_prefill: negative size");
    if ((int64_t)B * Hq * q_len == 0 || dv == 0) return 0;
    if (Hkv == 0 || Hq % Hkv != 0) return fail(YTHIP_EINVAL, "ythip_attn_prefill: Hq=%d not a multiple of Hkv=%d", Hq, Hkv);
    if (d == 0 || d > 256 || dv > 256) return fail(YTHIP_EUNSUPPORTED, "ythip_attn_prefill: head dims %d/%d (1..256)", d, dv);
    if (!Q || !O || !q_str || !k_str || !v_str || !o_str || (kv_len > 0 && (!K || !V)))
        return fail(YTHIP_EINVAL, "ythip_attn_prefill: NULL tensor or stride array");
    if (mask_kind < 0 || mask_kind > YTHIP_MASK_DIAG)
        return fail(YTHIP_EINVAL, "ythip_attn_prefill: mask_kind %d", mask_kind);
    if (mask_kind == YTHIP_MASK_BOOL && (mask == nullptr || mask_ld < kv_len))
        return fail(YTHIP_EINVAL, "ythip_attn_prefill: bool mask needs a pointer and mask_ld >= kv_len");
    if (scale == 0.0f) scale = 1.0f / sqrtf((float)d);  // src/function/ops.inl:378-381
    AttnArgs a{};
    a.Q = Q; a.K = K; a.V = V; a.O = O;
    a.qs0 = q_str[0]; a.qs1 = q_str[1]; a.qs2 = q_str[2];
    a.ks0 = k_str[0]; a.ks1 = k_str[1]; a.ks2 = k_str[2];
    a.vs0 = v_str[0]; a.vs1 = v_str[1]; a.vs2 = v_str[2];
    a.os0 = o_str[0]; a.os1 = o_str[1]; a.os2 = o_str[2];
    a.qs3 = q_str[3]; a.ks3 = k_str[3]; a.vs3 = v_str[3]; a.os3 = o_str[3];
    a.o_line = o_str[3] == 1 && o_str[0] % 8 == 0 && o_str[1] % 8 == 0 && o_str[2] % 8 == 0 && al(O, 16);
    a.mask_words = mask_kind == YTHIP_MASK_BOOL && bias == nullptr && al(mask, 4) && mask_ld % 4 == 0;
    a.B = B; a.Hq = Hq; a.Hkv = Hkv; a.Sq = q_len; a.Skv = kv_len; a.D = d; a.Dv = dv;
    a.scale_log2 = scale * LOG2E;
    a.causal = mask_kind == YTHIP_MASK_CAUSAL || mask_kind == YTHIP_MASK_DIAG;
    {
        // j <= i + off for every (i, j) once off >= kv_len; for none once off < -q_len
        const int64_t off = mask_kind == YTHIP_MASK_DIAG ? mask_ld : (int64_t)kv_len - q_len;
        a.diag_off = (int)std::max<int64_t>(-(int64_t)q_len - 1, std::min<int64_t>(off, kv_len));
    }
    a.mask = mask_kind == YTHIP_MASK_BOOL ? mask : nullptr;
    a.mask_ld = mask_ld;
    a.bias = bias; a.brs = rs_bias; a.bcs = cs_bias;
    if (dtype != YTHIP_F32 && dtype != YTHIP_F16 && dtype != YTHIP_BF16)
        return fail(YTHIP_EINVAL, "ythip_attn_prefill: invalid dtype %d", dtype);
    if (q_len == 1) {
        const int st = decode_route(dtype, a, mask_kind, mask, mask_ld, workspace, ws_bytes,
                                    static_cast<hipStream_t>(stream));
        if (st != -1) return st;
    }
    if (workspace != nullptr && mask_kind == YTHIP_MASK_BOOL && kv_len > 0) {
        // room for the mask's tile classes: the long-sequence paired-head path
        // then runs the ping-pong kernel over listed blocks
        const size_t need = ythip_attn_prefill_workspace_size(q_len, kv_len);
        if (ws_bytes < need)
            return fail(YTHIP_EINVAL, "ythip_attn_prefill_ws: workspace of %zu bytes needed, %zu given", need, ws_bytes);
        if ((kv_len + 63) / 64 <= PP_LIST_MAX) {
            a.tcls = static_cast<uint8_t*>(workspace);
            a.nkbt = (kv_len + 63) / 64;
        }
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (kv_len == 0) {
        // No key at all: every row is fully masked -> zeros (flash_attention.inl:241-244).
        a.Skv = 0;
    }
    switch (dtype) {
        case YTHIP_F32: return prefill_typed<F32>(a, s);
        case YTHIP_F16: return prefill_typed<F16>(a, s);
        case YTHIP_BF16: return prefill_typed<BF16>(a, s);
        default: return fail(YTHIP_EINVAL, "ythip_attn_prefill: invalid dtype %d", dtype);
    }
}

__attribute__((visibility("default"))) size_t ythip_attn_decode_workspace_size(int B, int Hq, int max_ctx, int d) {
    if (B <= 0 || Hq <= 0 || max_ctx <= 0 || d <= 0) return 0;
    return (size_t)B * Hq * decode_splits(B, Hq, max_ctx) * (d + 2) * sizeof(float);
}

__attribute__((visibility("default"))) size_t ythip_attn_sdpa_workspace_size(int B, int Hq, int q_len, int kv_len,
                                                                             int d) {
    const size_t tiles = ythip_attn_prefill_workspace_size(q_len, kv_len);
    const size_t dec = q_len == 1 ? ythip_attn_decode_workspace_size(B, Hq, kv_len, d) : 0;
    return std::max(tiles, dec);
}

__attribute__((visibility("default"))) int ythip_attn_decode(int dtype, int B, int Hq, int Hkv, int d, int max_ctx,
                                                             const void* Q, const int64_t q_str[2], const void* Kc,
                                                             const void* Vc, const int64_t kv_str[3],
                                                             const int32_t* kv_len, void* O, const int64_t o_str[2],
                                                             float scale, void* workspace, size_t ws_bytes,
                                                             void* stream) {
    if (B < 0 || Hq < 0 || Hkv < 0 || max_ctx < 0) return fail(YTHIP_EINVAL, "ythip_attn_decode: negative size");
    if ((int64_t)B * Hq == 0) return 0;
    if (Hkv == 0 || Hq % Hkv != 0) return fail(YTHIP_EINVAL, "ythip_attn_decode: Hq=%d not a multiple of Hkv=%d", Hq, Hkv);
    const int G = Hq / Hkv;
    if (d != 64 && d != 128) return fail(YTHIP_EUNSUPPORTED, "ythip_attn_decode: head dim %d (supported: 64, 128)", d);
    if (G != 1 && G != 2 && G != 4 && G != 5 && G != 8)
        return fail(YTHIP_EUNSUPPORTED, "ythip_attn_decode: group size %d (supported: 1, 2, 4, 5, 8)", G);
    if (!Q || !Kc || !Vc || !O || !q_str || !kv_str || !o_str)
        return fail(YTHIP_EINVAL, "ythip_attn_decode: NULL tensor or stride array");
    const size_t need = ythip_attn_decode_workspace_size(B, Hq, max_ctx > 0 ? max_ctx : 1, d);
    if (workspace == nullptr || ws_bytes < need)
        return fail(YTHIP_EINVAL, "ythip_attn_decode: workspace of %zu bytes needed, %zu given", need, ws_bytes);
    const int es = dtype == YTHIP_F32 ? 4 : 2;
    if (dtype != YTHIP_F32 && dtype != YTHIP_F16 && dtype != YTHIP_BF16)
        return fail(YTHIP_EINVAL, "ythip_attn_decode: invalid dtype %d", dtype);
    if (!al(Q, es) || !al(Kc, 16) || !al(Vc, 16) || kv_str[0] % (16 / es) || kv_str[1] % (16 / es) ||
        kv_str[2] % (16 / es))
        return fail(YTHIP_EUNSUPPORTED, "ythip_attn_decode: K/V cache rows must be 16-byte aligned");
    if (scale == 0.0f) scale = 1.0f / sqrtf((float)d);
    DecodeArgs a{};
    a.Q = Q; a.K = Kc; a.V = Vc; a.O = O;
    a.qs0 = q_str[0]; a.qs1 = q_str[1]; a.os0 = o_str[0]; a.os1 = o_str[1];
    a.ks0 = kv_str[0]; a.ks1 = kv_str[1]; a.ks2 = kv_str[2];
    a.vs0 = kv_str[0]; a.vs1 = kv_str[1]; a.vs2 = kv_str[2];
    a.kv_len = kv_len;
    a.B = B; a.Hq = Hq; a.Hkv = Hkv; a.max_ctx = max_ctx;
    a.splits = decode_splits(B, Hq, max_ctx > 0 ? max_ctx : 1);
    a.scale_log2 = scale * LOG2E;
    a.ws = static_cast<float*>(workspace);
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (dtype) {
        case YTHIP_F32: return status_of(launch_decode<F32>(a, d, G, s));
        case YTHIP_F16: return status_of(launch_decode<F16>(a, d, G, s));
        default: return status_of(launch_decode<BF16>(a, d, G, s));
    }
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Decode attention without a caller workspace: the split-K partials live in a
// fixed device array of this library, so the call allocates nothing. One copy
// of the array per GPU (held until the process ends); every call on a GPU
// shares it, so calls that overlap on one GPU (two streams, two threads) race.
// Every split writes its whole partial before the merge reads it, so the
// array needs no clearing between calls.
// ---------------------------------------------------------------------------
namespace ythip {
namespace {

constexpr size_t DEC_SCRATCH_BYTES = size_t(4) << 20;
static __device__ __align__(256) float dec_scratch[DEC_SCRATCH_BYTES / sizeof(float)];

constexpr int SCRATCH_MAX_DEVICES = 64;
std::mutex scratch_mu;
void* scratch_ptr[SCRATCH_MAX_DEVICES];

// Device address of dec_scratch on the current device, looked up once per
// device (the host-side name dec_scratch is not a device address).
int scratch_for_current_device(void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return status_of(e);
    if (dev < 0 || dev >= SCRATCH_MAX_DEVICES)
        return fail(YTHIP_EUNSUPPORTED, "ythip_attn_decode_noalloc: device %d beyond the %d supported", dev,
                    SCRATCH_MAX_DEVICES);
    std::lock_guard<std::mutex> lk(scratch_mu);
    if (scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(dec_scratch));
        if (e != hipSuccess) return status_of(e);
        if (p == nullptr) return fail(YTHIP_EINVAL, "ythip_attn_decode_noalloc: no device address for the scratch");
        scratch_ptr[dev] = p;
    }
    *out = scratch_ptr[dev];
    return 0;
}

}  // namespace
}  // namespace ythip

extern "C" {

__attribute__((visibility("default"))) size_t ythip_attn_decode_noalloc_max_bytes(void) { return DEC_SCRATCH_BYTES; }

__attribute__((visibility("default"))) int ythip_attn_decode_noalloc(int dtype, int B, int Hq, int Hkv, int d,
                                                                     int max_ctx, const void* Q,
                                                                     const int64_t q_str[2], const void* Kc,
                                                                     const void* Vc, const int64_t kv_str[3],
                                                                     const int32_t* kv_len, void* O,
                                                                     const int64_t o_str[2], float scale,
                                                                     void* stream) {
    if (B < 0 || Hq < 0 || Hkv < 0 || max_ctx < 0)
        return fail(YTHIP_EINVAL, "ythip_attn_decode_noalloc: negative size");
    if ((int64_t)B * Hq == 0) return 0;
    const size_t need = ythip_attn_decode_workspace_size(B, Hq, max_ctx > 0 ? max_ctx : 1, d > 0 ? d : 1);
    if (need > DEC_SCRATCH_BYTES)
        return fail(YTHIP_EINVAL,
                    "ythip_attn_decode_noalloc: B=%d Hq=%d max_ctx=%d d=%d needs %zu bytes of split-K scratch, "
                    "the fixed array holds %zu (use ythip_attn_decode with a workspace)",
                    B, Hq, max_ctx, d, need, DEC_SCRATCH_BYTES);
    void* ws = nullptr;
    const int st = scratch_for_current_device(&ws);
    if (st != 0) return st;
    return ythip_attn_decode(dtype, B, Hq, Hkv, d, max_ctx, Q, q_str, Kc, Vc, kv_str, kv_len, O, o_str, scale, ws,
                             DEC_SCRATCH_BYTES, stream);
}

__attribute__((visibility("default"))) int ythip_attn_decode_splits(int B, int Hq, int max_ctx) {
    if (B <= 0 || Hq <= 0 || max_ctx <= 0) return 0;
    return decode_splits(B, Hq, max_ctx);
}

__attribute__((visibility("default"))) int ythip_attn_decode_rope(
    int dtype, int B, int Hq, int Hkv, int d, int max_ctx, const void* qkv, int64_t ld_qkv, const float* wq,
    const float* wk, float eps, const float* cos_tab, const float* sin_tab, int64_t ld_tab, int tab_rows,
    int32_t* dev_state, void* Kc, void* Vc, const int64_t kv_str[3], void* O, const int64_t o_str[2], float scale,
    void* workspace, size_t ws_bytes, void* stream) {
    const char* who = "ythip_attn_decode_rope";
    if (B < 0 || Hq < 0 || Hkv < 0 || max_ctx <= 0) return fail(YTHIP_EINVAL, "%s: bad size", who);
    if ((int64_t)B * Hq == 0) return 0;
    if (Hkv == 0 || Hq % Hkv != 0) return fail(YTHIP_EINVAL, "%s: Hq=%d not a multiple of Hkv=%d", who, Hq, Hkv);
    const int G = Hq / Hkv;
    if (d != 64 && d != 128) return fail(YTHIP_EUNSUPPORTED, "%s: head dim %d (supported: 64, 128)", who, d);
    if (G != 1 && G != 2 && G != 4 && G != 5 && G != 8)
        return fail(YTHIP_EUNSUPPORTED, "%s: group size %d (supported: 1, 2, 4, 5, 8)", who, G);
    if (!qkv || !dev_state || !Kc || !Vc || !kv_str || (O && !o_str) || (cos_tab == nullptr) != (sin_tab == nullptr))
        return fail(YTHIP_EINVAL, "%s: NULL pointer", who);
    if (cos_tab != nullptr && (tab_rows <= 0 || ld_tab < d)) return fail(YTHIP_EINVAL, "%s: bad table args", who);
    if (dtype != YTHIP_F32 && dtype != YTHIP_F16 && dtype != YTHIP_BF16)
        return fail(YTHIP_EINVAL, "%s: invalid dtype %d", who, dtype);
    const int es = dtype == YTHIP_F32 ? 4 : 2;
    if (!al(Kc, 16) || !al(Vc, 16) || kv_str[0] % (16 / es) || kv_str[1] % (16 / es) || kv_str[2] % (16 / es) ||
        !al(qkv, 16) || ld_qkv % (16 / es) || (wq && !al(wq, 16)) || (wk && !al(wk, 16)) ||
        (cos_tab && (!al(cos_tab, 16) || !al(sin_tab, 16) || (ld_tab & 3))))
        return fail(YTHIP_EUNSUPPORTED, "%s: qkv rows, K/V cache rows, norm weights and tables must be 16-byte aligned",
                    who);
    const size_t need = ythip_attn_decode_workspace_size(B, Hq, max_ctx, d);
    if (workspace == nullptr || ws_bytes < need)
        return fail(YTHIP_EINVAL, "%s: workspace of %zu bytes needed, %zu given", who, need, ws_bytes);
    if (scale == 0.0f) scale = 1.0f / sqrtf((float)d);
    DecodeArgs a{};
    a.K = Kc; a.V = Vc; a.O = O;
    if (O) {
        a.os0 = o_str[0];
        a.os1 = o_str[1];
    }
    a.ks0 = kv_str[0]; a.ks1 = kv_str[1]; a.ks2 = kv_str[2];
    a.vs0 = kv_str[0]; a.vs1 = kv_str[1]; a.vs2 = kv_str[2];
    a.B = B; a.Hq = Hq; a.Hkv = Hkv; a.max_ctx = max_ctx;
    a.splits = decode_splits(B, Hq, max_ctx);
    a.direct = O != nullptr && a.splits == 1;  // one split: no merge launch
    a.scale_log2 = scale * LOG2E;
    a.ws = static_cast<float*>(workspace);
    a.qkv = qkv; a.ld_qkv = ld_qkv; a.wq = wq; a.wk = wk; a.eps = eps;
    a.cos_tab = cos_tab; a.sin_tab = sin_tab; a.ld_tab = ld_tab; a.tab_rows = tab_rows; a.dev_state = dev_state;
    a.fused = 1;
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (dtype) {
        case YTHIP_F32: return status_of(launch_decode<F32>(a, d, G, s));
        case YTHIP_F16: return status_of(launch_decode<F16>(a, d, G, s));
        default: return status_of(launch_decode<BF16>(a, d, G, s));
    }
}

}  // extern "C"
