// ref_shim.cpp — C-ABI harness around the REFERENCE itself (YTensor v0.13),
// compiled from the reference's own headers and example source where they lie
// under /root/reference. Build: oracle/Makefile target `ref`, output only into
// oracle/_ref/. This file contains no reference code: it only calls the
// reference's public functions so that tests can compare the restatement in
// ytoracle.cpp against the real thing, and so that bench.py can time the real
// CPU path ("kind": "reference").
//
// TEST INFRASTRUCTURE ONLY — never linked into the product.

#include "ytensor.hpp"
#include "qwen3.hpp"

#include <cstdint>
#include <cstring>
#include <vector>

#define REXPORT extern "C" __attribute__((visibility("default")))

REXPORT int ref_abi_version(void) { return 1; }

REXPORT void ref_seed(uint32_t s) { yt::YTensor<float, 1>::seed(s); }

REXPORT void ref_randn(float* out, int64_t n) {
    auto t = yt::YTensor<float, 1>::randn(static_cast<int>(n));
    std::memcpy(out, t.data(), sizeof(float) * static_cast<size_t>(n));
}

REXPORT void ref_bf16_round(const float* x, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        yt::bfloat16 b(x[i]);
        std::memcpy(&out[i], &b, 2);
    }
}

REXPORT void ref_bf16_to_f32(const uint16_t* x, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        yt::bfloat16 b;
        std::memcpy(&b, &x[i], 2);
        out[i] = static_cast<float>(b);
    }
}

REXPORT void ref_f16_round(const float* x, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        yt::float16 h(x[i]);
        std::memcpy(&out[i], &h, 2);
    }
}

REXPORT void ref_f16_to_f32(const uint16_t* x, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        yt::float16 h;
        std::memcpy(&h, &x[i], 2);
        out[i] = static_cast<float>(h);
    }
}

REXPORT void ref_set_num_threads(int t) { yt::kernel::avx2::set_num_threads(t); }

REXPORT void ref_sgemm(const float* A, const float* B, float* C, int m, int n, int k, float alpha, float beta,
                       int64_t rsa, int64_t csa, int64_t rsb, int64_t csb, int64_t rsc, int64_t csc) {
    yt::kernel::avx2::sgemm(A, B, C, m, n, k, alpha, beta, rsa, csa, rsb, csb, rsc, csc);
}

// YTensor<float,2>::matmul through the tensor API (AVX2 backend): A [m,k] row-major;
// B either [k,n] row-major (b_trans=0) or a transposed view of W [n,k] (b_trans=1),
// which is what yt::function::linear passes (src/function/ops.inl:84-91).
REXPORT void ref_matmul(const float* A, const float* B, float* C, int m, int n, int k, int b_trans) {
    yt::YTensor<float, 2> a(m, k);
    std::memcpy(a.data(), A, sizeof(float) * static_cast<size_t>(m) * k);
    yt::YTensor<float, 2> out;
    if (b_trans) {
        yt::YTensor<float, 2> w(n, k);
        std::memcpy(w.data(), B, sizeof(float) * static_cast<size_t>(n) * k);
        out = yt::function::linear(a, w);
    } else {
        yt::YTensor<float, 2> b(k, n);
        std::memcpy(b.data(), B, sizeof(float) * static_cast<size_t>(k) * n);
        out = a.matmul(b);
    }
    auto c = out.contiguous();
    std::memcpy(C, c.data(), sizeof(float) * static_cast<size_t>(m) * n);
}

REXPORT void ref_flash_attention(const float* Q, const float* K, const float* V, float* O, int q_len, int kv_len,
                                 int head_dim, int value_dim, float scale, int64_t rsq, int64_t csq, int64_t rsk,
                                 int64_t csk, int64_t rsv, int64_t csv, int64_t rso, int64_t cso,
                                 const uint8_t* mask, int64_t mask_stride, const float* bias, int64_t rsbias,
                                 int64_t csbias) {
    std::vector<char> mb;
    const bool* mp = nullptr;
    if (mask) {
        size_t cnt = static_cast<size_t>(q_len) * static_cast<size_t>(mask_stride);
        mb.resize(cnt);
        for (size_t i = 0; i < cnt; ++i) mb[i] = mask[i] ? 1 : 0;
        mp = reinterpret_cast<const bool*>(mb.data());
    }
    yt::kernel::avx2::flash_attention(Q, K, V, O, q_len, kv_len, head_dim, value_dim, scale, rsq, csq, rsk, csk,
                                      rsv, csv, rso, cso, mp, mask_stride, bias, rsbias, csbias);
}

// scaledDotProductAttention(FLASH_AVX2) with GQA exactly as the qwen3 example
// builds it (example/qwen3/src/qwen3.cpp:250-264): q [B,Hkv,G,S,D] view,
// k/v unsqueeze(2).repeat(1,1,G,1,1), bool causal mask [S,kv].
REXPORT void ref_sdpa_gqa(const float* Q, const float* K, const float* V, float* O, int B, int Hq, int Hkv,
                          int q_len, int kv_len, int D, float scale, int causal) {
    const int G = Hq / Hkv;
    yt::YTensor<float, 4> q4(B, Hq, q_len, D), k4(B, Hkv, kv_len, D), v4(B, Hkv, kv_len, D);
    std::memcpy(q4.data(), Q, sizeof(float) * q4.size());
    std::memcpy(k4.data(), K, sizeof(float) * k4.size());
    std::memcpy(v4.data(), V, sizeof(float) * v4.size());
    auto q5 = q4.reshape(B, Hkv, G, q_len, D);
    yt::YTensor<float, 5> k5(k4.unsqueeze(2).repeat(1, 1, G, 1, 1));
    yt::YTensor<float, 5> v5(v4.unsqueeze(2).repeat(1, 1, G, 1, 1));
    yt::YTensor<bool, 2> mask(q_len, kv_len);
    const int start = kv_len - q_len;
    for (int i = 0; i < q_len; ++i)
        for (int j = 0; j < kv_len; ++j) mask.at(i, j) = causal ? (j <= start + i) : true;
    auto o5 = yt::function::scaledDotProductAttention(q5, k5, v5, scale, &mask, nullptr,
                                                      yt::function::sdpaBackend::FLASH_AVX2);
    auto oc = o5.contiguous();
    std::memcpy(O, oc.data(), sizeof(float) * static_cast<size_t>(B) * Hq * q_len * D);
}

REXPORT void ref_rms_norm(float* x, const float* w, int64_t rows, int n, float eps) {
    yt::YTensor<float, 2> t(static_cast<int>(rows), n);
    std::memcpy(t.data(), x, sizeof(float) * static_cast<size_t>(rows) * n);
    yt::YTensor<float, 1> wt(n);
    std::memcpy(wt.data(), w, sizeof(float) * n);
    yt::function::rmsNorm_(t, wt, -1, eps);
    std::memcpy(x, t.data(), sizeof(float) * static_cast<size_t>(rows) * n);
}

REXPORT void ref_rope_precompute(int dim, int max_len, float theta, float* cosv, float* sinv) {
    qwen3::RoPECache rc;
    rc.precompute(dim, max_len, theta);
    std::memcpy(cosv, rc.cos.data(), sizeof(float) * static_cast<size_t>(dim) * max_len);
    std::memcpy(sinv, rc.sin.data(), sizeof(float) * static_cast<size_t>(dim) * max_len);
}

REXPORT void ref_rope(float* x, int B, int H, int L, int D, const float* cosv, const float* sinv) {
    yt::YTensor<float, 4> k(B, H, L, D);
    std::memcpy(k.data(), x, sizeof(float) * k.size());
    yt::YTensor<float, 2> c(L, D), s(L, D);
    std::memcpy(c.data(), cosv, sizeof(float) * static_cast<size_t>(L) * D);
    std::memcpy(s.data(), sinv, sizeof(float) * static_cast<size_t>(L) * D);
    qwen3::ops::rope_k(k, c, s);
    std::memcpy(x, k.data(), sizeof(float) * k.size());
}

// The reference's own Qwen3ForCausalLM (example/qwen3/src/qwen3.cpp), weights
// filled from the same flat fp32 buffer the oracle takes (layout documented in
// ytoracle.cpp), driven greedily over n_turns turns with the KV caches kept
// between turns, as repeated Qwen3ForCausalLM::generate calls keep them: per
// turn forward(prompt, chat_only=true), then forward(token, false) per step,
// argmax on the returned logits. Arguments as oracle_qwen3_run.
REXPORT int ref_qwen3_run(const int* cfg_i, const float* cfg_f, const float* W, int n_turns, const int* prompt_lens,
                          const int* prompts, const int* steps, int* out_tokens, float* out_margins,
                          const int* logit_steps, int n_logit_steps, float* out_logits) {
    qwen3::Qwen3Config cfg;
    cfg.hidden_size = cfg_i[0];
    cfg.num_hidden_layers = cfg_i[1];
    cfg.vocab_size = cfg_i[2];
    cfg.intermediate_size = cfg_i[3];
    cfg.num_attention_heads = cfg_i[4];
    cfg.num_key_value_heads = cfg_i[5];
    cfg.head_dim = cfg_i[6];
    cfg.max_position_embeddings = cfg_i[7];
    cfg.rms_norm_eps = cfg_f[0];
    cfg.rope_theta = cfg_f[1];
    auto* lm = new qwen3::Qwen3ForCausalLM();
    lm->init(cfg);
    const int H = cfg.hidden_size, V = cfg.vocab_size, I = cfg.intermediate_size, hd = cfg.head_dim;
    const int nh = cfg.num_attention_heads, nkv = cfg.num_key_value_heads;
    const float* p = W;
    auto take2 = [&](int r, int c) {
        yt::YTensor<float, 2> t(r, c);
        std::memcpy(t.data(), p, sizeof(float) * static_cast<size_t>(r) * c);
        p += static_cast<size_t>(r) * c;
        return t;
    };
    auto take1 = [&](int n) {
        yt::YTensor<float, 1> t(n);
        std::memcpy(t.data(), p, sizeof(float) * n);
        p += n;
        return t;
    };
    lm->model.embed = take2(V, H);
    for (int i = 0; i < cfg.num_hidden_layers; ++i) {
        auto& L = lm->model.layers[i];
        L.attn.qkv_proj = take2((nh + 2 * nkv) * hd, H);
        L.attn.o_proj = take2(H, nh * hd);
        L.attn.q_norm.weight = take1(hd);
        L.attn.k_norm.weight = take1(hd);
        L.mlp.gate_up = take2(2 * I, H);
        L.mlp.down = take2(H, I);
        L.norm1.weight = take1(H);
        L.norm2.weight = take1(H);
    }
    lm->model.norm.weight = take1(H);
    int g = 0;
    const int* pr = prompts;
    for (int t = 0; t < n_turns; ++t) {
        yt::YTensor<int, 2> ids(1, prompt_lens[t]);
        std::memcpy(ids.data(), pr, sizeof(int) * prompt_lens[t]);
        pr += prompt_lens[t];
        auto logits = lm->forward(ids, true);
        for (int step = 0; step < steps[t]; ++step, ++g) {
            auto lc = logits.contiguous();
            const float* lg = lc.data();
            for (int q = 0; q < n_logit_steps; ++q)
                if (out_logits && logit_steps[q] == g) std::memcpy(out_logits + static_cast<size_t>(q) * V, lg, sizeof(float) * V);
            int best = 0;
            for (int j = 1; j < V; ++j) if (lg[j] > lg[best]) best = j;
            float second = -INFINITY;
            for (int j = 0; j < V; ++j) if (j != best && lg[j] > second) second = lg[j];
            out_tokens[g] = best;
            out_margins[g] = lg[best] - second;
            if (step + 1 < steps[t]) {
                yt::YTensor<int, 2> nid(1, 1);
                nid.at(0, 0) = best;
                logits = lm->forward(nid, false);
            }
        }
    }
    delete lm;
    return 0;
}

REXPORT int ref_qwen3_generate(const int* cfg_i, const float* cfg_f, const float* W, const int* prompt,
                               int prompt_len, int n_steps, int* out_tokens, float* out_margins, float* logits0) {
    const int zero = 0;
    return ref_qwen3_run(cfg_i, cfg_f, W, 1, &prompt_len, prompt, &n_steps, out_tokens, out_margins, &zero,
                         logits0 ? 1 : 0, logits0);
}

// ---------------------------------------------------------------------------
// .yt files through the reference's own yt::io::YTensorIO
// (include/ytensor_io.hpp, src/ytensor_io.inl, src/ytensor_io_templates.inl).
// ---------------------------------------------------------------------------

// Writes n dense tensors (YTensorIO::open(path, mode) + save(...) + close()),
// mode 2 = yt::io::Write, 3 = yt::io::Append. shapes holds the dims of every
// tensor back to back (ndims[i] each); compress is "" or "zlib"
// (yt::io::compressMethod).
REXPORT int ref_yt_save(const char* path, int n, const char* const* names, const char* const* dtypes,
                        const int* ndims, const int* shapes, const void* const* data, const char* compress,
                        int mode) {
    yt::io::compressMethod = compress ? compress : "";
    yt::io::YTensorIO io;
    if (!io.open(path, mode == 3 ? yt::io::Append : yt::io::Write)) return 1;
    int so = 0;
    for (int i = 0; i < n; ++i) {
        std::vector<int> shape(shapes + so, shapes + so + ndims[i]);
        so += ndims[i];
        yt::YTensorBase t(shape, dtypes[i]);
        const size_t bytes = t.size() * t.elementSize();
        if (bytes) std::memcpy(t.data(), data[i], bytes);
        if (!io.save(t, names[i])) return 2;
    }
    io.close();
    yt::io::compressMethod = "";
    return 0;
}

// Tensor names of a file, '\n'-separated; returns the count or -1.
REXPORT int ref_yt_names(const char* path, char* buf, int64_t cap) {
    yt::io::YTensorIO io;
    if (!io.open(path, yt::io::Read)) return -1;
    std::string all;
    auto names = io.getTensorNames();
    for (auto& s : names) all += s + "\n";
    if (static_cast<int64_t>(all.size()) + 1 > cap) return -1;
    std::memcpy(buf, all.c_str(), all.size() + 1);
    return static_cast<int>(names.size());
}

// YTensorIO::load of one tensor ("" = the first): dtype name, shape and the
// dense bytes. Returns 0, or 1 (open failed), 2 (load returned false), 3 (cap).
REXPORT int ref_yt_load(const char* path, const char* name, void* out, int64_t cap, int64_t* nbytes,
                        char* dtype, int dtype_cap, int* ndim, int* shape) {
    yt::io::YTensorIO io;
    if (!io.open(path, yt::io::Read)) return 1;
    yt::YTensorBase t;
    if (!io.load(t, name ? name : "")) return 2;
    const int64_t bytes = static_cast<int64_t>(t.size() * t.elementSize());
    *nbytes = bytes;
    if (bytes > cap || static_cast<int>(t.dtype().size()) + 1 > dtype_cap) return 3;
    if (bytes) std::memcpy(out, t.data(), static_cast<size_t>(bytes));
    std::memcpy(dtype, t.dtype().c_str(), t.dtype().size() + 1);
    auto sh = t.shape();
    *ndim = static_cast<int>(sh.size());
    for (size_t i = 0; i < sh.size() && i < 16; ++i) shape[i] = sh[i];
    return 0;
}

// ---------------------------------------------------------------------------
// MATH backend, masked matmul and predicate masks
// ---------------------------------------------------------------------------

// yt::function::scaledDotProductAttention on fp32 [H, Lq, D] / [H, Lkv, D] /
// [H, Lkv, Dv] tensors (src/function/ops.inl:368-503): backend 0 = MATH,
// 1 = FLASH_AVX2; mask = bool bytes [Lq, Lkv] or NULL; diag != 0 passes the
// predicate functor j <= i + diag_off instead (the doc's
// [](int i, int j){ return j <= i; } for diag_off = 0); bias [Lq, Lkv] or NULL.
REXPORT void ref_sdpa_ex(const float* Q, const float* K, const float* V, float* O, int H, int Lq, int Lkv, int D,
                         int Dv, float scale, const uint8_t* mask, const float* bias, int backend, int diag,
                         int diag_off) {
    yt::YTensor<float, 3> q(H, Lq, D), k(H, Lkv, D), v(H, Lkv, Dv);
    std::memcpy(q.data(), Q, sizeof(float) * q.size());
    std::memcpy(k.data(), K, sizeof(float) * k.size());
    std::memcpy(v.data(), V, sizeof(float) * v.size());
    yt::YTensor<float, 2> bt;
    yt::YTensor<float, 2>* bp = nullptr;
    if (bias) {
        bt = yt::YTensor<float, 2>(Lq, Lkv);
        std::memcpy(bt.data(), bias, sizeof(float) * bt.size());
        bp = &bt;
    }
    const auto be = backend == 0 ? yt::function::sdpaBackend::MATH : yt::function::sdpaBackend::FLASH_AVX2;
    yt::YTensor<float, 3> o;
    if (diag) {
        auto pred = [diag_off](int i, int j) { return j <= i + diag_off; };
        o = yt::function::scaledDotProductAttention(q, k, v, scale, pred, bp, be);
    } else if (mask) {
        yt::YTensor<bool, 2> m(Lq, Lkv);
        for (int i = 0; i < Lq; ++i)
            for (int j = 0; j < Lkv; ++j) m.at(i, j) = mask[static_cast<size_t>(i) * Lkv + j] != 0;
        o = yt::function::scaledDotProductAttention(q, k, v, scale, &m, bp, be);
    } else {
        o = yt::function::scaledDotProductAttention(q, k, v, scale, static_cast<yt::YTensor<bool, 2>*>(nullptr),
                                                    bp, be);
    }
    auto oc = o.contiguous();
    std::memcpy(O, oc.data(), sizeof(float) * static_cast<size_t>(H) * Lq * Dv);
}

// yt::kernel::avx2::sgemm_masked with a bool mask [m, n] (src/kernel/avx2/sgemm.inl:342-447).
REXPORT void ref_sgemm_masked(const float* A, const float* B, float* C, int m, int n, int k, float alpha,
                              float beta, int64_t rsa, int64_t csa, int64_t rsb, int64_t csb, int64_t rsc,
                              int64_t csc, const uint8_t* mask) {
    std::vector<char> mb(static_cast<size_t>(m) * n);
    for (size_t i = 0; i < mb.size(); ++i) mb[i] = mask[i] ? 1 : 0;
    yt::kernel::avx2::sgemm_masked(A, B, C, m, n, k, alpha, beta, rsa, csa, rsb, csb, rsc, csc,
                                   reinterpret_cast<const bool*>(mb.data()));
}

// YTensor<float,2>::masked_matmul (src/ytensor_math.inl:318-410): A [m,k] . B [k,n]
// where the bool mask [m,n] (or, diag != 0, the predicate j <= i + diag_off) is
// true, masked_value elsewhere.
REXPORT void ref_masked_matmul(const float* A, const float* B, float* O, int m, int n, int k,
                               const uint8_t* mask, int diag, int diag_off, float masked_value) {
    yt::YTensor<float, 2> a(m, k), b(k, n);
    std::memcpy(a.data(), A, sizeof(float) * a.size());
    std::memcpy(b.data(), B, sizeof(float) * b.size());
    yt::YTensor<float, 2> o;
    if (diag) {
        o = a.masked_matmul(b, [diag_off](int i, int j) { return j <= i + diag_off; }, masked_value);
    } else {
        yt::YTensor<bool, 2> mk(m, n);
        for (int i = 0; i < m; ++i)
            for (int j = 0; j < n; ++j) mk.at(i, j) = mask[static_cast<size_t>(i) * n + j] != 0;
        o = a.masked_matmul(b, mk, masked_value);
    }
    auto oc = o.contiguous();
    std::memcpy(O, oc.data(), sizeof(float) * static_cast<size_t>(m) * n);
}
