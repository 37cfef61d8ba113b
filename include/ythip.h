/*
 * ythip.h — C ABI of libythip.so, the MI355X (gfx950) back end for YTensor's
 * two hot operators (SnifferCaptain/ytensor v0.13): the blocked GEMM behind
 * YTensor::matmul / yt::function::linear, and the SDPA / flash-attention
 * forward behind yt::function::scaledDotProductAttention, plus the fused
 * RMSNorm+RoPE that sits between them in the Qwen3 example.
 *
 * Conventions (shared by every entry point):
 *   - All tensor pointers are DEVICE pointers; sizes are int, element strides
 *     int64 (as in the reference's kernel API), in ELEMENTS, not bytes.
 *   - `stream` is a hipStream_t (NULL = the legacy default stream). Calls are
 *     asynchronous on that stream and re-entrant across streams.
 *   - Return value: 0 on success, a negative YTHIP_E* code for argument errors
 *     (nothing was launched), or a positive hipError_t from the launch.
 *     ythip_last_error() returns the calling thread's last message.
 *   - No entry point allocates device memory: scratch space is passed in
 *     (the .yt file calls below own pinned HOST staging buffers), except that
 *     ythip_attn_decode_noalloc uses a fixed array the library holds per GPU.
 *   - No C++ exceptions cross this boundary.
 */
#ifndef YTHIP_H
#define YTHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types: the reference's fp32 / float16 / bfloat16 type set
 * (include/ytensor_types.hpp:137-175; include/types/bfloat16.hpp;
 * include/types/float_spec.hpp:533). */
enum ythip_dtype { YTHIP_F32 = 0, YTHIP_F16 = 1, YTHIP_BF16 = 2 };

enum ythip_status {
    YTHIP_OK = 0,
    YTHIP_EINVAL = -1,       /* bad argument (shape, stride, pointer, dtype) */
    YTHIP_EUNSUPPORTED = -2, /* valid but not implemented combination */
    YTHIP_EIO = -3,          /* file could not be opened, read or written */
    YTHIP_EFORMAT = -4,      /* not a .yt file, or a corrupt / truncated one */
    YTHIP_ENOTFOUND = -5     /* no tensor of that name */
};

/* Attention mask kinds. */
enum ythip_mask_kind {
    YTHIP_MASK_NONE = 0,   /* every key visible */
    YTHIP_MASK_CAUSAL = 1, /* key j visible to query i iff j <= (kv_len - q_len) + i
                              (example/qwen3/src/qwen3.cpp:46-55) */
    YTHIP_MASK_BOOL = 2,   /* byte mask [q_len, mask_ld]; nonzero = visible
                              (include/kernel/avx2/flash_attention.hpp:21-44 `const bool* mask`) */
    YTHIP_MASK_DIAG = 3    /* predicate: key j visible to query i iff j <= i + mask_ld (the offset
                              travels in mask_ld, mask is NULL) -- the predicate-functor masks of
                              scaledDotProductAttention / masked_matmul (src/function/ops.inl:449-503,
                              src/ytensor_math.inl:372-410), e.g. [](int i, int j){ return j <= i; }
                              (doc/en/api/function/fused.mdx:200) with offset 0. Other predicates
                              are evaluated into a bool mask by the caller. */
};

/* ABI version of this header; bumped on any signature change. */
#define YTHIP_ABI_VERSION 3
int ythip_abi_version(void);

/* Thread-local description of the last failure on this thread ("" if none). */
const char* ythip_last_error(void);

/*
 * Batched strided GEMM:  C[b] = alpha * A[b] . B[b] + beta * C[b]
 *   A[b]: m x k at A + b*sa_b, element (i,p) at i*rsa + p*csa
 *   B[b]: k x n at B + b*sb_b, element (p,j) at p*rsb + j*csb   (sb_b = 0: shared weight)
 *   C[b]: m x n at C + b*sc_b, element (i,j) at i*rsc + j*csc
 * Replaces yt::kernel::avx2::sgemm (include/kernel/avx2/sgemm.hpp:51-58) and
 * hgemm (include/kernel/avx2/hgemm.hpp:26-33) for device-resident operands, and
 * the per-matrix loop of YTensor::matmul (src/ytensor_math.inl:954-1051).
 * dtype_in: F32, F16 or BF16 (A and B share it). Accumulation is fp32.
 * dtype_out: same as dtype_in, or F32 (fp32 diagnostics output) for 16-bit input.
 * `linear(x, W)` is B = W^T, i.e. rsb = 1, csb = ldW (src/function/ops.inl:84-91).
 * Semantics at the edges follow sgemm.inl:594-604: m == 0 or n == 0 is a no-op;
 * k == 0 or alpha == 0 scales C by beta (beta == 0 writes zeros).
 */
int ythip_gemm(int dtype_in, int dtype_out, int batch, int m, int n, int k,
               const void* A, int64_t sa_b, int64_t rsa, int64_t csa,
               const void* B, int64_t sb_b, int64_t rsb, int64_t csb,
               void* C, int64_t sc_b, int64_t rsc, int64_t csc,
               float alpha, float beta, void* stream);

/*
 * Attention forward, prefill (any q_len >= 1):
 *   O[b,h] = softmax(scale * Q[b,h] . K[b,h/G]^T + bias, masked) . V[b,h/G],  G = Hq / Hkv
 * Q: [B,Hq,q_len,d], K: [B,Hkv,kv_len,d], V: [B,Hkv,kv_len,dv], O: [B,Hq,q_len,dv];
 * each *_str gives the 4 element strides (batch, head, row, col); col stride must be 1.
 * scale == 0 means 1/sqrt(d) (src/function/ops.inl:378-381).
 * bias (fp32, optional): [q_len, kv_len] at bias + i*rs_bias + j*cs_bias, added after scaling.
 * Rows with no visible key produce zeros (src/kernel/avx2/flash_attention.inl:241-244, 327-331).
 * Replaces the per-(batch, head) loop of _scaledDotProductAttentionFlash
 * (src/function/ops.inl:109-234) over yt::kernel::avx2::flash_attention
 * (include/kernel/avx2/flash_attention.hpp:21-69). Supported: d == dv in {64, 128}.
 * q_len == 1 (the reference's decode branch, src/kernel/avx2/flash_attention.inl:
 * 469-499) runs the split-K decode kernel for every mask kind and bias when
 * d == dv in {64, 128}, Hq / Hkv in {1, 2, 4, 5, 8}, the head dim is contiguous
 * and K / V rows are 16-byte aligned; without a workspace (this call) that is
 * one split per (kv head, batch) -- ythip_attn_prefill_ws with
 * ythip_attn_sdpa_workspace_size bytes runs the full split count.
 */
int ythip_attn_prefill(int dtype, int B, int Hq, int Hkv, int q_len, int kv_len, int d, int dv,
                       const void* Q, const int64_t q_str[4],
                       const void* K, const int64_t k_str[4],
                       const void* V, const int64_t v_str[4],
                       void* O, const int64_t o_str[4],
                       float scale, int mask_kind, const uint8_t* mask, int64_t mask_ld,
                       const float* bias, int64_t rs_bias, int64_t cs_bias, void* stream);

/*
 * ythip_attn_prefill with a device workspace for a bool mask's tile classes
 * (one byte per 32-row x 64-key tile, ythip_attn_prefill_workspace_size(q_len,
 * kv_len) bytes; fewer is YTHIP_EINVAL). Same arguments and results as
 * ythip_attn_prefill, which is this call with no workspace. With one, a bool
 * mask on the long-sequence paired-head path (d in {64, 128}, Hq / Hkv even)
 * is classified tile by tile first, and the attention then stages only the key
 * blocks each 128-row query block sees. Same replaced interface as
 * ythip_attn_prefill (the bool-mask call of flash_attention,
 * include/kernel/avx2/flash_attention.hpp:21-69); the workspace is this
 * library's addition, as for ythip_attn_math.
 */
size_t ythip_attn_prefill_workspace_size(int q_len, int kv_len);
/*
 * Workspace for ythip_attn_prefill_ws that serves every call shape: the bool
 * mask's tile classes, and for q_len == 1 the split-K partials of the decode
 * kernel (ythip_attn_decode_workspace_size(B, Hq, kv_len, d)). A smaller
 * workspace still works (fewer splits). Same replaced interface as
 * ythip_attn_prefill; the workspace is this library's addition.
 */
size_t ythip_attn_sdpa_workspace_size(int B, int Hq, int q_len, int kv_len, int d);
int ythip_attn_prefill_ws(int dtype, int B, int Hq, int Hkv, int q_len, int kv_len, int d, int dv,
                          const void* Q, const int64_t q_str[4],
                          const void* K, const int64_t k_str[4],
                          const void* V, const int64_t v_str[4],
                          void* O, const int64_t o_str[4],
                          float scale, int mask_kind, const uint8_t* mask, int64_t mask_ld,
                          const float* bias, int64_t rs_bias, int64_t cs_bias,
                          void* workspace, size_t ws_bytes, void* stream);

/*
 * Attention forward with the MATH backend (scaledDotProductAttention with
 * sdpaBackend::MATH, src/function/ops.inl:388-418, 474-490): the score matrix is
 * materialised,
 *   S = masked_matmul(Q, K^T, mask, -1e9) * scale + bias,  P = softmax_(S, -1),
 *   O = P . V,  rows with no visible key -> 0 (ops.inl:18-40),
 * with S in fp32 and P in the input type (the reference's score tensor has the
 * input type). Same tensor and mask arguments as ythip_attn_prefill, except that
 * every stride may be any value (transposed K / V included). workspace: device
 * scratch of ythip_attn_math_workspace_size(dtype, B, Hq, q_len, kv_len) bytes.
 */
size_t ythip_attn_math_workspace_size(int dtype, int B, int Hq, int q_len, int kv_len);
int ythip_attn_math(int dtype, int B, int Hq, int Hkv, int q_len, int kv_len, int d, int dv,
                    const void* Q, const int64_t q_str[4],
                    const void* K, const int64_t k_str[4],
                    const void* V, const int64_t v_str[4],
                    void* O, const int64_t o_str[4],
                    float scale, int mask_kind, const uint8_t* mask, int64_t mask_ld,
                    const float* bias, int64_t rs_bias, int64_t cs_bias,
                    void* workspace, size_t ws_bytes, void* stream);

/*
 * Masked GEMM (yt::kernel::avx2::sgemm_masked, src/kernel/avx2/sgemm.inl:342-584;
 * YTensor::masked_matmul, src/ytensor_math.inl:318-410): operands as ythip_gemm;
 * for every batch entry, where the [m, n] mask is set
 *   C = alpha * A.B + beta * C   (k == 0 or alpha == 0: C *= beta, 0 for beta == 0)
 * and elsewhere C is left unchanged, or set to masked_value when fill_masked != 0
 * (masked_matmul's fill). mask_kind / mask / mask_ld as for attention, with the
 * causal offset n - m. workspace: ythip_gemm_masked_workspace_size(batch, m, n)
 * bytes of device scratch (the fp32 product).
 */
size_t ythip_gemm_masked_workspace_size(int batch, int m, int n);
int ythip_gemm_masked(int dtype_in, int dtype_out, int batch, int m, int n, int k,
                      const void* A, int64_t sa_b, int64_t rsa, int64_t csa,
                      const void* B, int64_t sb_b, int64_t rsb, int64_t csb,
                      void* C, int64_t sc_b, int64_t rsc, int64_t csc,
                      float alpha, float beta, int mask_kind, const uint8_t* mask, int64_t mask_ld,
                      int fill_masked, float masked_value, void* workspace, size_t ws_bytes, void* stream);

/*
 * Single-query decode attention over a KV cache (the q_len == 1 path,
 * src/kernel/avx2/flash_attention.inl:202-272), split over the context:
 *   Q: [B,Hq,d] with strides q_str[0..1] (batch, head), contiguous d
 *   Kc/Vc: [B,Hkv,max_ctx,d] with strides kv_str (batch, head, pos); contiguous d
 *   kv_len: device int32[B] (keys [0, kv_len[b]) are visible) or NULL = max_ctx for all
 *   O: [B,Hq,d] with strides o_str[0..1]
 * workspace: device scratch of ythip_attn_decode_workspace_size(B, Hq, max_ctx, d) bytes.
 */
size_t ythip_attn_decode_workspace_size(int B, int Hq, int max_ctx, int d);
int ythip_attn_decode(int dtype, int B, int Hq, int Hkv, int d, int max_ctx,
                      const void* Q, const int64_t q_str[2],
                      const void* Kc, const void* Vc, const int64_t kv_str[3],
                      const int32_t* kv_len, void* O, const int64_t o_str[2],
                      float scale, void* workspace, size_t ws_bytes, void* stream);

/*
 * Device-resident decode state: int32[YTHIP_ST_WORDS] read by the decode-step
 * kernels when they run (so one captured HIP graph serves every step) and
 * advanced by ythip_argmax_step / ythip_argmax_finish. It carries the
 * bookkeeping of the reference's ring KV cache (KVCache, example/qwen3/src/
 * qwen3.cpp:57-126) and its RoPE start rule (Qwen3Model::forward, 365-375),
 * for batch 1:
 *   TOTAL    tokens written to the cache so far (KVCache::total_written)
 *   SLOT     cache row of the next token, TOTAL % RING (KVCache::write_pos)
 *   KV_LEN   keys the next token sees after its append, min(TOTAL + 1, RING)
 *            (KVCache::cur_len); once the ring is full every row is visible,
 *            which is what get_mask gives a single query (104-126)
 *   ROPE_POS RoPE table row of the next token: TOTAL if TOTAL + 1 <= MAX_POS,
 *            else min(TOTAL, RING) if that + 1 <= MAX_POS, else 0 (365-375)
 *   RING     cache rows (KVCache::max_len; the reference sizes it MAX_POS)
 *   MAX_POS  max_position_embeddings (RoPE table rows)
 *   GENERATED / HISTORY  next history index / history capacity
 *   ERROR    bits the kernels set instead of touching memory out of range:
 *            1 = cache row outside the cache, 2 = RoPE row outside the table,
 *            4 = history full (the token is still returned in *token)
 */
enum ythip_decode_state_field {
    YTHIP_ST_GENERATED = 0,
    YTHIP_ST_ROPE_POS = 1,
    YTHIP_ST_KV_LEN = 2,
    YTHIP_ST_SLOT = 3,
    YTHIP_ST_TOTAL = 4,
    YTHIP_ST_RING = 5,
    YTHIP_ST_MAX_POS = 6,
    YTHIP_ST_HISTORY = 7,
    YTHIP_ST_ERROR = 8,
    YTHIP_ST_WORDS = 16
};
enum ythip_decode_error { YTHIP_ST_ERR_CACHE = 1, YTHIP_ST_ERR_ROPE = 2, YTHIP_ST_ERR_HISTORY = 4 };

/*
 * ythip_attn_decode without a workspace argument. No counterpart in the
 * reference: this entry point is for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, hosts that forbid
 * hipMalloc). It calls no allocating routine; the split-K partials go to a
 * fixed array of ythip_attn_decode_noalloc_max_bytes() bytes (4 MiB) that the
 * library holds once per GPU until the process ends. A call whose
 * ythip_attn_decode_workspace_size(B, Hq, max_ctx, d) exceeds that returns
 * YTHIP_EINVAL. All calls on one GPU share the array: calls that overlap on one
 * GPU (other streams, other threads) race. Same kernels, same bits as
 * ythip_attn_decode.
 */
size_t ythip_attn_decode_noalloc_max_bytes(void);
int ythip_attn_decode_noalloc(int dtype, int B, int Hq, int Hkv, int d, int max_ctx,
                              const void* Q, const int64_t q_str[2],
                              const void* Kc, const void* Vc, const int64_t kv_str[3],
                              const int32_t* kv_len, void* O, const int64_t o_str[2],
                              float scale, void* stream);

/*
 * One decode step's attention for the Qwen3 layer with the q/k norm and RoPE
 * fused in: the equivalent of ythip_rmsnorm_rope (S = 1, dev_state) followed by
 * ythip_attn_decode (kv_len = &dev_state[YTHIP_ST_KV_LEN]), with the same bits:
 *   qkv: the new token's projection row per batch entry (row b at qkv + b*ld_qkv),
 *        q heads, then k heads, then v heads (example/qwen3/src/qwen3.cpp:233-248);
 *   q, k <- RMSNorm (wq / wk, may be NULL) + RoPE at table row
 *        dev_state[YTHIP_ST_ROPE_POS] (cos/sin may be NULL; tab_rows rows);
 *        k and v are written to cache row dev_state[YTHIP_ST_SLOT] (kv_str as
 *        for ythip_attn_decode, K and V share it; max_ctx rows);
 *   O[b, h] = softmax(scale * q . K[0..n)^T) . V[0..n), n = dev_state[YTHIP_ST_KV_LEN]
 *        (the q_len == 1 path, src/kernel/avx2/flash_attention.inl:202-272).
 * A slot or RoPE row out of range sets the ERROR bits and is not accessed.
 * workspace: ythip_attn_decode_workspace_size(B, Hq, max_ctx, d) bytes. With
 * O == NULL only the split-K partials are produced, in the workspace as
 * fp32 [B][Hq][S][d + 2] = (running max m in log2 units, sum l, o[d]) per
 * split, S = ythip_attn_decode_splits(B, Hq, max_ctx), for a caller that
 * merges them itself. Split s holds keys [s*c, (s+1)*c) of the n visible
 * ones, c = max(128, ceil(n / S)); splits past them hold m = -inf, l = 0,
 * o = 0.
 * qkv rows, norm weights and cos/sin rows must be 16-byte aligned.
 */
int ythip_attn_decode_splits(int B, int Hq, int max_ctx);
int ythip_attn_decode_rope(int dtype, int B, int Hq, int Hkv, int d, int max_ctx,
                           const void* qkv, int64_t ld_qkv, const float* wq, const float* wk, float eps,
                           const float* cos_tab, const float* sin_tab, int64_t ld_tab, int tab_rows,
                           int32_t* dev_state, void* Kc, void* Vc, const int64_t kv_str[3], void* O,
                           const int64_t o_str[2], float scale, void* workspace, size_t ws_bytes, void* stream);

/*
 * Fused per-head RMSNorm + rotate-half RoPE on the fused qkv projection output,
 * scattering Q to [B,Hq,S,d] and K/V into cache rows (cache_pos + s) % cache_rows
 * (the ring write of KVCache::append, example/qwen3/src/qwen3.cpp:70-88):
 *   qkv: rows of (Hq + 2*Hkv)*d elements, row (b*S + s) at qkv + (b*S+s)*ld_qkv;
 *        q heads, then k heads, then v heads (example/qwen3/src/qwen3.cpp:233-238)
 *   q, k <- rmsNorm_(x, w, -1, eps) (src/function/normalization.inl:256-267)
 *   q, k <- rope with table row (pos0 + s) (example/qwen3/src/qwen3.cpp:522-559)
 *   v    <- copied unchanged
 * wq / wk (fp32 [d]) may be NULL to skip that norm; cos/sin (fp32 [tab_rows,
 * ld_tab], from RoPECache::precompute, qwen3.cpp:161-175) may be NULL to skip RoPE.
 * Output strides are (batch, head, row); d is contiguous. K/V outputs may be NULL;
 * when given, 0 <= cache_pos < cache_rows and S <= cache_rows.
 * All tensors, rows, strides and tables must keep 16-byte alignment
 * (YTHIP_EUNSUPPORTED otherwise).
 * dev_state: optional decode-state record (see ythip_decode_state_field); when
 * given, pos0 = dev_state[YTHIP_ST_ROPE_POS] and cache_pos = dev_state[YTHIP_ST_SLOT]
 * are read when the kernel runs (a decode step captured once in a HIP graph);
 * rows out of range then set its ERROR bits and are not accessed.
 */
int ythip_rmsnorm_rope(int dtype, int B, int S, int Hq, int Hkv, int d,
                       const void* qkv, int64_t ld_qkv,
                       const float* wq, const float* wk, float eps,
                       const float* cos_tab, const float* sin_tab, int64_t ld_tab, int tab_rows, int pos0,
                       void* Qout, const int64_t q_str[3],
                       void* Kout, const int64_t k_str[3],
                       void* Vout, const int64_t v_str[3],
                       int cache_rows, int cache_pos, int32_t* dev_state, void* stream);

/*
 * RMSNorm over the last axis of [rows, n] (the hidden-state norms of the Qwen3
 * layers, src/function/normalization.inl:256-267): y = x / sqrt(mean(x^2)+eps) * w.
 * x/y rows at stride ld_x / ld_y (in place allowed when the dtypes match);
 * w fp32 [n]. dtype_in/dtype_out may differ (fp32 residual -> bf16 GEMM input).
 */
int ythip_rms_norm(int dtype_in, int dtype_out, int rows, int n, const void* x, int64_t ld_x,
                   const float* w, float eps, void* y, int64_t ld_y, void* stream);

/*
 * ythip_rms_norm with element strides: element i of row r at x + r*ld_x +
 * i*cs_x (y likewise), w fp32 [n] contiguous. Normalises over one axis of any
 * stride -- rmsNorm / rmsNorm_ over an axis other than the last, or over
 * several neighbouring axes whose strides nest (include/function/
 * normalization.hpp:59-89, src/function/normalization.inl:33-54, 88-101,
 * 233-277). Same arithmetic and bits as ythip_rms_norm. In place (x == y)
 * needs one dtype and one layout.
 */
int ythip_rms_norm_strided(int dtype_in, int dtype_out, int rows, int n, const void* x, int64_t ld_x,
                           int64_t cs_x, const float* w, float eps, void* y, int64_t ld_y, int64_t cs_y,
                           void* stream);

/*
 * SwiGLU over a fused gate_up projection (Qwen3MLP::forward,
 * example/qwen3/src/qwen3.cpp:193-200): for each row r and j < n,
 *   out[r][j] = swish(gu[r][j]) * gu[r][n + j],  swish(a) = a * sigmoid(a)
 * with the stable sigmoid of src/ytensor_function.inl:43-52.
 */
int ythip_silu_mul(int dtype_in, int dtype_out, int rows, int n, const void* gate_up, int64_t ld_gu,
                   void* out, int64_t ld_out, void* stream);

/*
 * Embedding gather (Qwen3Model::forward, example/qwen3/src/qwen3.cpp:378-385):
 *   out[r][:] = table[ids[r]][:]   (table [vocab, n], ids device int32[rows])
 * An id outside [0, vocab) is never used as an address: its row is written
 * as zeros (the reference indexes unchecked; hosts should reject such ids).
 */
int ythip_embedding(int dtype_table, int dtype_out, int rows, int n, int vocab, const void* table,
                    const int32_t* ids, void* out, int64_t ld_out, void* stream);

/*
 * The bias step of yt::function::linear(x, W, b) (src/function/ops.inl:93-104):
 * the product x . W^T is already in `out` (rows x n, row stride ld_out, stored
 * in dtype); the bias [n] of the same dtype is then added in that type,
 *   out[r][j] = T(out[r][j] + bias[j]).
 */
int ythip_add_bias(int dtype, int rows, int n, void* out, int64_t ld_out, const void* bias, void* stream);

/*
 * Greedy token selection over fp32 logits [n]: *token = first index of the
 * maximum. If state (the decode-state record, see ythip_decode_state_field) is
 * given, the token that was just run is counted as written and the record
 * advances to the next token: history[GENERATED] = token (history may be NULL;
 * past HISTORY entries the ERROR bit 4 is set instead), GENERATED += 1,
 * TOTAL += 1, then SLOT, KV_LEN and ROPE_POS are derived from TOTAL, RING and
 * MAX_POS. Replaces the example's top-20 sampling (qwen3.cpp:465-486) by
 * argmax, as configs[4] specifies.
 */
int ythip_argmax_step(int n, const float* logits, int32_t* token, int32_t* history,
                      int32_t* state, void* stream);

/*
 * Decode-time linear with a fused operand prologue, for M <= 16 rows:
 *   C[m, n] = alpha * A'[m, k] . W[n, k]^T + beta * C
 * (W row-major [n][k] with row stride ldw -- the weight of `linear`,
 * src/function/ops.inl:84-91, which the reference runs as gemv_row_simd for
 * one row, src/kernel/avx2/sgemv.inl:443-717). dtype_in is W's type.
 *   prologue 0: A' = A (dtype_in, [m][k], row stride lda);
 *   prologue 1: A' = bf16/fp16-rounded rmsNorm_(A, norm_w, eps) of fp32 rows A
 *               (src/function/normalization.inl:256-277; the pre-attention,
 *               pre-MLP and final norms of qwen3.cpp:271-283, 365-413), with the
 *               same arithmetic as ythip_rms_norm, so bits match the unfused pair;
 *   prologue 2: A' = rounded swish(gate) * up of dtype_in rows A = [gate | up]
 *               ([m][2k], qwen3.cpp:193-200), arithmetic of ythip_silu_mul.
 * argmax_parts (optional, fp32 device buffer of 2 * ceil(n / 16) values): one
 * (max, index-as-bits) pair of row 0 per 16-column tile, lowest index on ties,
 * for ythip_argmax_finish. Requires 16-byte aligned A/W rows and k a multiple
 * of 8 (16-bit) or 4 (fp32); prologues 1 and 2 need 16-bit W.
 */
int ythip_gemv_fused(int prologue, int dtype_in, int dtype_out, int m, int n, int k,
                     const void* A, int64_t lda, const float* norm_w, float eps,
                     const void* W, int64_t ldw, void* C, int64_t ldc, float alpha,
                     float beta, float* argmax_parts, void* stream);

/*
 * The MLP's first half for M <= 16 rows, Qwen3MLP::forward up to the down
 * projection (qwen3.cpp:193-200): the fused gate_up linear followed by the
 * SwiGLU, C[m, i] = swish(g) * u with g = A'.W[i]^T and u = A'.W[inter + i]^T
 * each rounded to dtype first (W = [gate rows | up rows], [2*inter][k], row
 * stride ldw; C [m][inter], row stride ldc). prologue 0: A' = A (dtype rows);
 * 1: A' = the rounded rmsNorm_ of fp32 rows A as in ythip_gemv_fused. The bits
 * equal ythip_gemv_fused(prologue) into a [m][2*inter] buffer followed by
 * ythip_silu_mul; the [m][2*inter] intermediate is never written. dtype is
 * bf16 or fp16 (W and C); same alignment rules as ythip_gemv_fused.
 */
/*
 * The attention output projection of a decode step with the split-K merge as
 * its operand prologue (Qwen3Attention::forward's linear(attn3, o_proj) after
 * the q_len == 1 attention, qwen3.cpp:254-268; the merge is the combine of
 * src/kernel/avx2/flash_attention.inl:202-272's per-block softmax state):
 *   A'[b, h*hd + d] = sum_s 2^(m_s - M) o_s[d] / sum_s 2^(m_s - M) l_s, rounded
 *   to dtype, over the partials ythip_attn_decode_rope(O = NULL) leaves in its
 *   workspace (fp32 [m][hq][splits][hd + 2], row stride ld_part floats;
 *   splits = ythip_attn_decode_splits), then
 *   C[m, n] = alpha * A' . W[n, hq*hd]^T + beta * C   (dtype W, dtype_out C).
 * Same bits as the merge inside ythip_attn_decode_rope(O given) followed by
 * ythip_gemv_fused(prologue 0). The attention output is never written.
 * dev_state / max_ctx: the decode-state record and ring size the split kernel
 * ran with; the splits are cut by the visible key count min(KV_LEN, max_ctx)
 * at run time, so only the splits holding keys are read. NULL: every split is
 * read (the empty ones add exact zeros; same bits).
 */
int ythip_gemv_attn_merge(int dtype, int dtype_out, int m, int n, int hq, int hd, int splits,
                          const float* partials, int64_t ld_part, const void* W, int64_t ldw,
                          void* C, int64_t ldc, float alpha, float beta,
                          const int32_t* dev_state, int max_ctx, void* stream);

int ythip_gemv_swiglu(int prologue, int dtype, int m, int inter, int k, const void* A,
                      int64_t lda, const float* norm_w, float eps, const void* W, int64_t ldw,
                      void* C, int64_t ldc, void* stream);

/*
 * Greedy selection from ythip_gemv_fused's per-tile pairs (n_parts tiles):
 * same result, tie rule and state update as ythip_argmax_step over the full
 * logits (qwen3.cpp:465-486, argmax as configs[4] specifies).
 */
int ythip_argmax_finish(const float* parts, int n_parts, int32_t* token, int32_t* history,
                        int32_t* state, void* stream);

/*
 * RoPE tables on the HOST, as RoPECache::precompute builds them
 * (example/qwen3/src/qwen3.cpp:161-175): cosv/sinv [max_len][dim] (host memory).
 */
int ythip_rope_tables(int dim, int max_len, float theta, float* cosv, float* sinv);

/* ------------------------------------------------------------------------
 * .yt checkpoint files (yt::io::YTensorIO, include/ytensor_io.hpp:81-180,
 * src/ytensor_io.inl) read straight into device memory and written from it.
 * Host-side calls: paths and the info/tensor descriptors are HOST memory,
 * `dst` / `data` are DEVICE pointers. Loads are queued on `stream` through two
 * pinned staging buffers owned by the handle; the destination is complete once
 * the stream reaches the call's last copy (or after ythip_yt_sync).
 * ---------------------------------------------------------------------- */

/* dtype for ythip_yt_load / ythip_yt_tensor: copy the stored bytes unchanged
 * (any dense element type, e.g. int32 or float64). */
#define YTHIP_YT_RAW (-1)

typedef struct ythip_yt_file ythip_yt_file; /* opaque handle */

/* One tensor record (TensorInfo, include/ytensor_io.hpp:67-78). The strings
 * and the shape array stay valid until ythip_yt_close. */
typedef struct ythip_yt_tensor_info {
    const char* name;
    const char* dtype;       /* typeName, e.g. "bfloat16", "float32" */
    const char* tensor_type; /* "dense" (loadable), "map", ... */
    const char* compress;    /* "" or "zlib" */
    int32_t type_size;       /* bytes per element */
    int32_t ndim;
    const int32_t* shape;    /* ndim dims; ndim == 0 is one element */
    uint64_t data_offset;    /* payload position in the file */
    uint64_t compressed_size;
    uint64_t nbytes;         /* type_size * prod(shape) (uncompressedSize) */
} ythip_yt_tensor_info;

/* YTensorIO::open(path, yt::io::Read) (src/ytensor_io.inl:256-311) with
 * readHeader + readIndex (458-559). */
int ythip_yt_open(const char* path, ythip_yt_file** out);
/* YTensorIO::close for a read handle; waits for queued copies. */
int ythip_yt_close(ythip_yt_file* f);
/* getTensorNames().size() (src/ytensor_io.inl:419-425). */
int ythip_yt_count(const ythip_yt_file* f);
/* The header's metadata string (readHeader, src/ytensor_io.inl:482). */
const char* ythip_yt_metadata(const ythip_yt_file* f);
/* Index of a tensor by name; "" or NULL is the first one, as getTensorInfo("")
 * (src/ytensor_io.inl:427-443). Negative status if absent. */
int ythip_yt_find(const ythip_yt_file* f, const char* name);
/* getTensorInfo for index (0 <= index < count). */
int ythip_yt_info(const ythip_yt_file* f, int index, ythip_yt_tensor_info* info);
/*
 * YTensorIO::load (src/ytensor_io.inl:785-830) of a dense tensor into device
 * memory `dst` (dst_bytes available), as dtype F32 / F16 / BF16 or YTHIP_YT_RAW.
 * A stored float32 / bfloat16 / float16 / float64 / int32 tensor converts with
 * the reference's casts (the static_casts of toFloat, qwen3.cpp:16-45, and
 * yt::bfloat16 / yt::float16's conversions); matching types are copied as is.
 * zlib payloads are inflated on the way. A payload whose size differs from
 * type_size * prod(shape) is rejected (YTHIP_EFORMAT).
 */
int ythip_yt_load(ythip_yt_file* f, int index, void* dst, int dtype, uint64_t dst_bytes, void* stream);
/*
 * The same for n tensors at once (a whole checkpoint): index[i] into dst[i]
 * as dtype[i] with dst_bytes[i] available. Every argument is checked before
 * anything is queued. Tensors copied unchanged are read in file order in
 * spans of many neighbouring payloads per staging buffer.
 */
int ythip_yt_load_many(ythip_yt_file* f, int n, const int* index, void* const* dst, const int* dtype,
                       const uint64_t* dst_bytes, void* stream);
/*
 * HOST-memory element conversion with the reference's casts, as the loads
 * above use them: float -> bfloat16 (include/types/bfloat16.hpp:78-80),
 * float -> float16 (include/types/float_spec.hpp:435-491, subnormals flush to
 * zero), 16-bit -> float (exact; the reference's fp16 subnormal doubling kept).
 * For callers that prepare 16-bit weights on the host (src and dst are host
 * pointers, n elements; dtypes F32 / F16 / BF16).
 */
int ythip_convert_host(int src_dtype, int dst_dtype, const void* src, void* dst, int64_t n);
/* Waits until every copy queued by this handle has completed. */
int ythip_yt_sync(ythip_yt_file* f);

/* A device tensor to save (dense, row-major). */
typedef struct ythip_yt_tensor {
    const char* name;        /* "" = numbered by position, as save() (src/ytensor_io.inl:712) */
    int dtype;               /* F32 / F16 / BF16, or YTHIP_YT_RAW with dtype_name + type_size */
    const char* dtype_name;  /* typeName written for YTHIP_YT_RAW (e.g. "int32") */
    int32_t type_size;       /* bytes per element for YTHIP_YT_RAW */
    int32_t ndim;
    const int32_t* shape;
    const void* data;        /* device pointer */
} ythip_yt_tensor;

/*
 * YTensorIO::open(path, Write or Append) + save(t_i, name_i) for each tensor +
 * close() (src/ytensor_io.inl:256-417, 703-783): byte-for-byte the file the
 * reference writes for the same tensors. compress "zlib" deflates each payload
 * as compressData does (templates.inl:17-46); anything else stores it raw.
 * append = 0 (Write): tensors of an existing file that are not saved again are
 * dropped; append = 1 (Append): they are kept. A name already present is
 * replaced in place. The file is written to a temporary name and renamed.
 */
int ythip_yt_save(const char* path, int n, const ythip_yt_tensor* tensors, const char* compress, int append,
                  void* stream);

#ifdef __cplusplus
}
#endif

#endif /* YTHIP_H */
