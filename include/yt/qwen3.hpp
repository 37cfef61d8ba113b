// yt/qwen3.hpp -- the Qwen3 example's decoder (example/qwen3/include/qwen3.hpp,
// example/qwen3/src/qwen3.cpp) as a C++ host over include/yt/ytensor.hpp whose
// whole forward runs on one MI355X through libythip.so.
//
// The classes keep the example's names and roles: Qwen3Config (qwen3.hpp:46-60,
// init from config.json: qwen3.cpp:128-159), RoPECache (161-175), KVCache with
// the ring bookkeeping of append / get_mask (57-126), the decoder layers
// (193-283), Qwen3Model (285-413) and Qwen3ForCausalLM with forward / generate /
// reset_kv_cache (415-516). Weights are YTensor storage with device mirrors:
// matrices in the model's 16-bit type T (yt::bfloat16 or yt::float16, rounded
// with the reference's casts), norms fp32, q/k/v fused into one [(h + 2 kv_h) hd,
// hidden] matrix and gate/up into [2 inter, hidden] as the example's load() does
// (qwen3.cpp:326-349); the embedding is the LM head unless the checkpoint has
// lm_head.weight (Qwen3ForCausalLM::forward, 446-457).
//
// Execution on the device:
//   * the residual stream is fp32; GEMM inputs, activations and the KV cache are
//     T; the o / down projections add into the residual in their epilogue;
//   * a prompt (forward, the first step of generate) runs per layer RMSNorm ->
//     qkv GEMM -> per-head q/k RMSNorm + RoPE with the K/V ring append ->
//     causal (or get_mask bool) attention -> o GEMM -> RMSNorm -> gate_up GEMM ->
//     SwiGLU -> down GEMM, then the final norm, LM head and greedy pick;
//   * a generated token runs 5 launches per layer (RMSNorm in the qkv / gate_up
//     GEMV prologues, SwiGLU in the gate_up GEMV epilogue, q/k norm + RoPE +
//     cache append inside the split-K attention, the merge of its splits in the o
//     projection's prologue) plus the LM head with the argmax folded in. Its cache
//     row, RoPE row and visible keys come from a device-resident decode-state
//     record that the argmax advances (the KVCache rules as data), so the step is
//     captured once with hipStreamBeginCapture and replayed with hipGraphLaunch;
//     a prompt is captured once per length the same way.
// The kernel sequence is that of ytensor_amd/qwen3.py, so both hosts give the
// same bits.
//
// Token selection is greedy (argmax, lowest index on ties): configs[4]'s
// decoding in place of the example's top-20 sampling (qwen3.cpp:465-486).
#pragma once

#include <cstdio>
#include <fstream>
#include <functional>
#include <map>
#include <sstream>
#include <string>
#include <vector>

#include "ytensor.hpp"

namespace qwen3 {

// example/qwen3/include/qwen3.hpp:46-60.
struct Qwen3Config {
    int hidden_size = 1024;
    int num_hidden_layers = 28;
    int vocab_size = 151936;
    float rms_norm_eps = 1e-6f;
    float rope_theta = 1e6f;
    int intermediate_size = 3072;
    int num_attention_heads = 16;
    int num_key_value_heads = 8;
    int head_dim = 128;
    int max_position_embeddings = 4096;
    std::string model_dir = "model";

    // Qwen3Config::init (qwen3.cpp:128-159): the Hugging Face config.json keys,
    // each keeping its default when absent. Numbers only, as the example reads.
    void init(const std::string& dir) {
        model_dir = dir;
        std::ifstream f(dir + "/config.json");
        if (!f) throw std::runtime_error("qwen3::Qwen3Config::init: cannot open " + dir + "/config.json");
        std::stringstream ss;
        ss << f.rdbuf();
        const std::string j = ss.str();
        auto num = [&](const char* key, auto& dst) {
            const std::string k = std::string("\"") + key + "\"";
            size_t p = j.find(k);
            if (p == std::string::npos) return;
            p = j.find(':', p + k.size());
            if (p == std::string::npos) return;
            dst = static_cast<std::decay_t<decltype(dst)>>(std::strtod(j.c_str() + p + 1, nullptr));
        };
        num("hidden_size", hidden_size);
        num("num_hidden_layers", num_hidden_layers);
        num("vocab_size", vocab_size);
        num("rms_norm_eps", rms_norm_eps);
        num("rope_theta", rope_theta);
        num("intermediate_size", intermediate_size);
        num("num_attention_heads", num_attention_heads);
        num("num_key_value_heads", num_key_value_heads);
        num("head_dim", head_dim);
        num("max_position_embeddings", max_position_embeddings);
    }
};

// RoPECache::precompute (qwen3.cpp:161-175): the float tables built on the host
// (ythip_rope_tables), uploaded once.
struct RoPECache {
    yt::YTensor<float, 2> cos, sin;
    void precompute(int dim, int max_len, float theta) {
        cos = yt::YTensor<float, 2>(std::vector<int>{max_len, dim});
        sin = yt::YTensor<float, 2>(std::vector<int>{max_len, dim});
        yt::hip::check(ythip_rope_tables(dim, max_len, theta, cos.data(), sin.data()), "qwen3::RoPECache");
        cos.toDevice();
        sin.toDevice();
    }
};

// The ring KV cache of one layer (qwen3.cpp:57-126): buffers [b, kv_h, max_len,
// hd] on the device, filled by the attention kernels; the host keeps the
// bookkeeping (append advances it, get_mask reads it).
template <class T>
class KVCache {
public:
    yt::YTensor<T, 4> k_buffer, v_buffer;
    int cur_len = 0;
    int max_len = 0;
    int write_pos = 0;
    int total_written = 0;
    int num_kv_heads = 0;
    int head_dim = 0;

    void init(int batch, int max_length, int kv_heads, int hd) {
        max_len = max_length;
        num_kv_heads = kv_heads;
        head_dim = hd;
        reset();
        k_buffer = yt::YTensor<T, 4>::deviceOutput({batch, kv_heads, max_length, hd});
        v_buffer = yt::YTensor<T, 4>::deviceOutput({batch, kv_heads, max_length, hd});
        const size_t bytes = k_buffer.size() * sizeof(T);
        yt::hip::check(hipMemsetAsync(k_buffer.deviceWrite(), 0, bytes, yt::hip::stream()), "qwen3::KVCache");
        yt::hip::check(hipMemsetAsync(v_buffer.deviceWrite(), 0, bytes, yt::hip::stream()), "qwen3::KVCache");
    }
    void reset() {
        cur_len = 0;
        write_pos = 0;
        total_written = 0;
    }
    // KVCache::append's bookkeeping for n rows (the kernels wrote them at
    // write_pos, write_pos + 1, ... mod max_len).
    void append(int n) {
        for (int t = 0; t < n; ++t) {
            write_pos = (write_pos + 1) % max_len;
            ++total_written;
            if (cur_len < max_len) ++cur_len;
        }
    }
    bool empty() const { return cur_len == 0; }
    bool full() const { return cur_len >= max_len; }
    int remaining() const { return max_len - cur_len; }
    int get_global_position() const { return total_written; }

    // KVCache::get_mask (qwen3.cpp:104-126): [query_len, cur_len], causal over
    // physical rows until the ring is full, then over logical (write) order.
    yt::YTensor<bool, 2> get_mask(int query_len) const {
        const int kv_len = cur_len;
        yt::YTensor<bool, 2> mask(std::vector<int>{query_len, kv_len});
        bool* m = mask.data();
        const int start = kv_len - query_len;
        for (int qi = 0; qi < query_len; ++qi)
            for (int ki = 0; ki < kv_len; ++ki) {
                const int k_logical = full() ? (ki - write_pos + max_len) % max_len : ki;
                m[static_cast<int64_t>(qi) * kv_len + ki] = k_logical <= start + qi;
            }
        return mask;
    }
};

// One decoder layer's weights (Qwen3Attention / Qwen3MLP / the two RMSNorms,
// qwen3.hpp:62-140).
template <class T>
struct Qwen3DecoderLayer {
    yt::YTensor<T, 2> qkv_proj, o_proj, gate_up, down;
    yt::YTensor<float, 1> q_norm, k_norm, norm1, norm2;
};

template <class T>
class Qwen3Model {
public:
    Qwen3Config config;
    yt::YTensor<T, 2> embed;
    yt::YTensor<T, 2> lm_head;  // empty: tied to embed
    std::vector<Qwen3DecoderLayer<T>> layers;
    yt::YTensor<float, 1> norm;
    RoPECache rope;

    // Qwen3Model::init (qwen3.cpp:285-301): shapes, device storage, RoPE tables.
    void init(const Qwen3Config& cfg) {
        config = cfg;
        const int H = cfg.hidden_size, I = cfg.intermediate_size, hd = cfg.head_dim;
        const int nh = cfg.num_attention_heads, nkv = cfg.num_key_value_heads;
        embed = yt::YTensor<T, 2>::deviceOutput({cfg.vocab_size, H});
        layers.assign(cfg.num_hidden_layers, {});
        for (auto& L : layers) {
            L.qkv_proj = yt::YTensor<T, 2>::deviceOutput({(nh + 2 * nkv) * hd, H});
            L.o_proj = yt::YTensor<T, 2>::deviceOutput({H, nh * hd});
            L.gate_up = yt::YTensor<T, 2>::deviceOutput({2 * I, H});
            L.down = yt::YTensor<T, 2>::deviceOutput({H, I});
            L.q_norm = yt::YTensor<float, 1>::deviceOutput({hd});
            L.k_norm = yt::YTensor<float, 1>::deviceOutput({hd});
            L.norm1 = yt::YTensor<float, 1>::deviceOutput({H});
            L.norm2 = yt::YTensor<float, 1>::deviceOutput({H});
        }
        norm = yt::YTensor<float, 1>::deviceOutput({H});
        lm_head = yt::YTensor<T, 2>();
        rope.precompute(hd, cfg.max_position_embeddings, cfg.rope_theta);
    }

    const yt::YTensor<T, 2>& head() const { return lm_head.size() > 0 ? lm_head : embed; }

    // Random init in configs[4]'s recipe: YTensor::seed(seed), then every tensor
    // randn * scale in the order embed, per layer q, k, v, o, q_norm, k_norm, gate,
    // up, down, norm1, norm2, then the final norm (one randn call per tensor), each
    // value rounded to T (matrices) or to bf16 and back to float (norms, which
    // configs[4] draws like the rest). norm_spread > 0: the norms are instead
    // 1 + norm_spread * randn (the discriminating variant of the same stream).
    void init_random(unsigned seed, float scale = 0.02f, float norm_spread = 0.0f) {
        const Qwen3Config& c = config;
        const int H = c.hidden_size, I = c.intermediate_size, hd = c.head_dim;
        const int nh = c.num_attention_heads, nkv = c.num_key_value_heads;
        yt::YTensor<float, 1>::seed(seed);
        // one randn call of n values into rows [row0, row0 + n / cols) of a T matrix
        auto mat = [&](yt::YTensor<T, 2>& dst, int64_t offset, int64_t n) {
            auto x = yt::YTensor<float, 1>::randn(static_cast<int>(n));
            float* p = x.data();
            for (int64_t i = 0; i < n; ++i) p[i] *= scale;
            std::vector<uint16_t> bits(static_cast<size_t>(n));
            yt::hip::check(ythip_convert_host(YTHIP_F32, yt::hip::dtype_code<T>(), p, bits.data(), n),
                           "qwen3: convert");
            yt::hip::check(hipMemcpy(reinterpret_cast<uint16_t*>(dst.deviceWrite()) + offset, bits.data(),
                                     static_cast<size_t>(n) * 2, hipMemcpyHostToDevice),
                           "qwen3: upload");
        };
        auto vec = [&](yt::YTensor<float, 1>& dst) {
            const int n = dst.shape(0);
            auto x = yt::YTensor<float, 1>::randn(n);
            float* p = x.data();
            for (int i = 0; i < n; ++i) {
                const float v = norm_spread > 0.0f ? 1.0f + p[i] * norm_spread : p[i] * scale;
                p[i] = static_cast<float>(yt::bfloat16(v));
            }
            yt::hip::check(hipMemcpy(dst.deviceWrite(), p, static_cast<size_t>(n) * 4, hipMemcpyHostToDevice),
                           "qwen3: upload");
        };
        mat(embed, 0, static_cast<int64_t>(c.vocab_size) * H);
        for (auto& L : layers) {
            mat(L.qkv_proj, 0, static_cast<int64_t>(nh) * hd * H);
            mat(L.qkv_proj, static_cast<int64_t>(nh) * hd * H, static_cast<int64_t>(nkv) * hd * H);
            mat(L.qkv_proj, static_cast<int64_t>(nh + nkv) * hd * H, static_cast<int64_t>(nkv) * hd * H);
            mat(L.o_proj, 0, static_cast<int64_t>(H) * nh * hd);
            vec(L.q_norm);
            vec(L.k_norm);
            mat(L.gate_up, 0, static_cast<int64_t>(I) * H);
            mat(L.gate_up, static_cast<int64_t>(I) * H, static_cast<int64_t>(I) * H);
            mat(L.down, 0, static_cast<int64_t>(H) * I);
            vec(L.norm1);
            vec(L.norm2);
        }
        vec(norm);
    }

    // Qwen3Model::load (qwen3.cpp:304-363) from a .yt checkpoint straight into the
    // device layout: q/k/v land in the row blocks of qkv_proj and gate/up in
    // gate_up; matrices as T, norms as fp32 (converted with the reference's casts
    // when stored otherwise); lm_head.weight when present. Unlike the example, a
    // missing tensor is an error (false) rather than an empty weight.
    bool load(const std::string& path) {
        ythip_yt_file* f = nullptr;
        if (ythip_yt_open(path.c_str(), &f) != 0) return false;
        const Qwen3Config& c = config;
        const int H = c.hidden_size, I = c.intermediate_size, hd = c.head_dim;
        const int nh = c.num_attention_heads, nkv = c.num_key_value_heads;
        std::vector<int> index, dtype;
        std::vector<void*> dst;
        std::vector<uint64_t> bytes;
        bool ok = true;
        const int code = yt::hip::dtype_code<T>();
        auto plan = [&](const std::string& name, void* p, int dt, uint64_t n_elem) {
            const int i = ythip_yt_find(f, name.c_str());
            if (i < 0) {
                std::fprintf(stderr, "qwen3::load: %s has no tensor %s\n", path.c_str(), name.c_str());
                ok = false;
                return;
            }
            index.push_back(i);
            dst.push_back(p);
            dtype.push_back(dt);
            bytes.push_back(n_elem * (dt == YTHIP_F32 ? 4 : 2));
        };
        auto row = [](yt::YTensor<T, 2>& m, int64_t r) {
            return static_cast<void*>(m.deviceWrite() + r * m.shape(1));
        };
        plan("model.embed_tokens.weight", embed.deviceWrite(), code, embed.size());
        for (int i = 0; i < c.num_hidden_layers; ++i) {
            auto& L = layers[i];
            const std::string p = "model.layers." + std::to_string(i) + ".";
            plan(p + "self_attn.q_proj.weight", row(L.qkv_proj, 0), code, uint64_t(nh) * hd * H);
            plan(p + "self_attn.k_proj.weight", row(L.qkv_proj, int64_t(nh) * hd), code, uint64_t(nkv) * hd * H);
            plan(p + "self_attn.v_proj.weight", row(L.qkv_proj, int64_t(nh + nkv) * hd), code,
                 uint64_t(nkv) * hd * H);
            plan(p + "self_attn.o_proj.weight", L.o_proj.deviceWrite(), code, L.o_proj.size());
            plan(p + "self_attn.q_norm.weight", L.q_norm.deviceWrite(), YTHIP_F32, hd);
            plan(p + "self_attn.k_norm.weight", L.k_norm.deviceWrite(), YTHIP_F32, hd);
            plan(p + "mlp.gate_proj.weight", row(L.gate_up, 0), code, uint64_t(I) * H);
            plan(p + "mlp.up_proj.weight", row(L.gate_up, I), code, uint64_t(I) * H);
            plan(p + "mlp.down_proj.weight", L.down.deviceWrite(), code, L.down.size());
            plan(p + "input_layernorm.weight", L.norm1.deviceWrite(), YTHIP_F32, H);
            plan(p + "post_attention_layernorm.weight", L.norm2.deviceWrite(), YTHIP_F32, H);
        }
        plan("model.norm.weight", norm.deviceWrite(), YTHIP_F32, H);
        if (ythip_yt_find(f, "lm_head.weight") >= 0) {
            lm_head = yt::YTensor<T, 2>::deviceOutput({c.vocab_size, H});
            plan("lm_head.weight", lm_head.deviceWrite(), code, lm_head.size());
        }
        int st = 0;
        if (ok) {
            st = ythip_yt_load_many(f, static_cast<int>(index.size()), index.data(), dst.data(), dtype.data(),
                                    bytes.data(), yt::hip::stream());
            if (st != 0) std::fprintf(stderr, "qwen3::load: %s\n", ythip_last_error());
            if (st == 0) st = ythip_yt_sync(f);
        }
        ythip_yt_close(f);
        return ok && st == 0;
    }
};

// Qwen3ForCausalLM (qwen3.hpp:142-170, qwen3.cpp:415-516) for batch 1.
template <class T = yt::bfloat16>
class Qwen3ForCausalLM {
    static_assert(std::is_same_v<T, yt::bfloat16> || std::is_same_v<T, yt::float16>,
                  "the decoder runs its matrices, activations and KV cache in bfloat16 or float16");

public:
    Qwen3Config config;
    Qwen3Model<T> model;
    std::vector<KVCache<T>> kv_caches;  // one per layer (they advance together)

    Qwen3ForCausalLM() = default;
    Qwen3ForCausalLM(const Qwen3ForCausalLM&) = delete;
    Qwen3ForCausalLM& operator=(const Qwen3ForCausalLM&) = delete;
    ~Qwen3ForCausalLM() { release_graphs(); if (stream_) (void)hipStreamDestroy(stream_); }

    // Qwen3ForCausalLM::init (qwen3.cpp:415-421). max_ctx: ring rows (default
    // max_position_embeddings, as the example sizes KVCache); max_prompt: the
    // longest prompt one forward takes; max_tokens: history capacity (the most
    // tokens one generate call returns).
    void init(const Qwen3Config& cfg, int max_prompt = 512, int max_ctx = 0, int max_tokens = 4096) {
        config = cfg;
        if (!stream_) yt::hip::check(hipStreamCreate(&stream_), "qwen3: hipStreamCreate");
        yt::hip::StreamGuard g(stream_);
        max_ctx_ = max_ctx > 0 ? std::min(max_ctx, cfg.max_position_embeddings) : cfg.max_position_embeddings;
        max_prompt_ = max_prompt;
        max_tokens_ = max_tokens;
        model.init(cfg);
        kv_caches.assign(cfg.num_hidden_layers, {});
        for (auto& c : kv_caches) c.init(1, max_ctx_, cfg.num_key_value_heads, cfg.head_dim);
        const int H = cfg.hidden_size, I = cfg.intermediate_size, hd = cfg.head_dim;
        const int nh = cfg.num_attention_heads, nkv = cfg.num_key_value_heads, P = max_prompt;
        x_ = yt::YTensor<float, 2>::deviceOutput({P, H});
        h_ = yt::YTensor<T, 2>::deviceOutput({P, H});
        qkv_ = yt::YTensor<T, 2>::deviceOutput({P, (nh + 2 * nkv) * hd});
        q_ = yt::YTensor<T, 4>::deviceOutput({1, nh, P, hd});
        attn_ = yt::YTensor<T, 2>::deviceOutput({P, nh * hd});
        gu_ = yt::YTensor<T, 2>::deviceOutput({P, 2 * I});
        act_ = yt::YTensor<T, 2>::deviceOutput({P, I});
        hf_ = yt::YTensor<T, 2>::deviceOutput({1, H});
        logits_ = yt::YTensor<float, 2>::deviceOutput({1, cfg.vocab_size});
        ids_ = yt::YTensor<int32_t, 1>::deviceOutput({P});
        token_ = yt::YTensor<int32_t, 1>::deviceOutput({1});
        history_ = yt::YTensor<int32_t, 1>::deviceOutput({max_tokens});
        state_ = yt::YTensor<int32_t, 1>::deviceOutput({YTHIP_ST_WORDS});
        amax_ = yt::YTensor<float, 1>::deviceOutput({2 * ((cfg.vocab_size + 15) / 16)});
        splits_ = ythip_attn_decode_splits(1, nh, max_ctx_);
        ws_bytes_ = std::max(ythip_attn_decode_workspace_size(1, nh, max_ctx_, hd),
                             ythip_attn_sdpa_workspace_size(1, nh, P, max_ctx_, hd));
        ws_ = yt::YTensor<uint8_t, 1>::deviceOutput({static_cast<int>(ws_bytes_)});
        release_graphs();
        yt::hip::check(hipStreamSynchronize(stream_), "qwen3::init");
    }

    // Qwen3ForCausalLM::load (qwen3.cpp:423-431).
    bool load(const std::string& path) {
        yt::hip::StreamGuard g(stream_);
        return model.load(path);
    }
    void init_random(unsigned seed, float scale = 0.02f, float norm_spread = 0.0f) {
        yt::hip::StreamGuard g(stream_);
        model.init_random(seed, scale, norm_spread);
    }

    void reset_kv_cache() {
        for (auto& c : kv_caches) c.reset();
    }
    int get_kv_cache_len() const { return kv_caches.empty() ? 0 : kv_caches[0].cur_len; }
    int get_max_context_len() const { return config.max_position_embeddings; }
    hipStream_t stream() const { return stream_; }

    // Qwen3ForCausalLM::forward (qwen3.cpp:446-457) for a prompt of ids [1, l]:
    // the whole prompt through every layer (its K/V appended to the caches), then
    // the final norm and the LM head on the last row. Returns the logits [1,
    // vocab] (fp32, on the device). The greedy pick of the next token is made on
    // the device as well (next_token()). use_graph: replay the prompt's launches
    // from a graph captured once per prompt length (fresh caches only).
    // chat_only is accepted for the example's signature; every row of the last
    // layer is computed, which leaves the last row's result unchanged.
    yt::YTensor<float, 2> forward(const yt::YTensor<int, 2>& ids, bool chat_only = false, bool use_graph = false) {
        (void)chat_only;
        const int P = ids.shape(1);
        if (ids.shape(0) != 1) throw std::invalid_argument("qwen3::forward: batch 1 only");
        std::vector<int32_t> v(P);
        for (int j = 0; j < P; ++j) v[j] = ids.at(0, j);
        prefill(v, use_graph);
        return logits_;
    }

    // The token the last forward / decode step picked (downloads it).
    int next_token() {
        int32_t t = 0;
        yt::hip::check(hipMemcpyAsync(&t, token_.deviceData(), 4, hipMemcpyDeviceToHost, stream_), "qwen3: token");
        yt::hip::check(hipStreamSynchronize(stream_), "qwen3: token");
        return t;
    }

    // Qwen3ForCausalLM::generate (qwen3.cpp:459-516), greedy: the prompt's forward
    // picks the first token, then each further token is one replay of the
    // captured decode step, until max_tokens tokens or `eos` (eos < 0: never stop;
    // as in the example, eos itself is not returned nor appended to the cache).
    // The caches keep the turn for the next call (reset_kv_cache() clears them).
    // eos >= 0 is checked every `eos_chunk` tokens (one host round trip each); the
    // steps run past an eos are undone in the bookkeeping, their cache rows are
    // overwritten later -- with a ring that has wrapped the chunk drops to 1 so no
    // visible row is ever overwritten.
    std::vector<int> generate(const std::vector<int>& new_ids, int max_tokens, int eos = 2,
                              std::function<void(int)> on_token = nullptr, bool chat_only = true,
                              int eos_chunk = 16) {
        (void)chat_only;
        std::vector<int> out;
        if (max_tokens <= 0) return out;
        if (max_tokens > max_tokens_)
            throw std::invalid_argument("qwen3::generate: max_tokens beyond the history capacity");
        std::vector<int32_t> ids(new_ids.begin(), new_ids.end());
        const int t0 = kv_caches[0].total_written;
        prefill(ids, t0 == 0);
        yt::hip::StreamGuard g(stream_);
        if (!decode_graph_) capture_decode();
        int done = 1;  // history entries written (the prompt's pick is entry 0)
        auto flush = [&](int upto) -> bool {  // reads history[0, upto); true when eos was met
            std::vector<int32_t> hist(upto);
            yt::hip::check(hipMemcpyAsync(hist.data(), history_.deviceData(), upto * 4, hipMemcpyDeviceToHost,
                                          stream_),
                           "qwen3: history");
            yt::hip::check(hipStreamSynchronize(stream_), "qwen3: history");
            for (int i = static_cast<int>(out.size()); i < upto; ++i) {
                if (eos >= 0 && hist[i] == eos) {
                    // undo the steps that ran past eos: tokens 0 .. i-1 were forwarded
                    set_total(t0 + static_cast<int>(ids.size()) + i);
                    return true;
                }
                out.push_back(hist[i]);
                if (on_token) on_token(hist[i]);
            }
            return false;
        };
        const int start_total = t0 + static_cast<int>(ids.size());
        if (eos >= 0 && flush(1)) return out;
        while (done < max_tokens) {
            int n = eos >= 0 ? std::min(eos_chunk, max_tokens - done) : max_tokens - done;
            if (eos >= 0 && start_total + done + n > max_ctx_) n = 1;
            for (int i = 0; i < n; ++i) launch_decode_graph();
            done += n;
            if (eos >= 0 && flush(done)) return out;
        }
        if (eos < 0) flush(done);
        for (auto& c : kv_caches) c.append(done - 1);  // every generated token but the last was forwarded
        check_state();
        return out;
    }

    // One generated token: a replay of the captured decode step (advances the
    // device state; the host bookkeeping follows in generate / sync_steps).
    void launch_decode_graph() {
        if (!decode_graph_) capture_decode();
        yt::hip::check(hipGraphLaunch(decode_graph_, stream_), "qwen3: hipGraphLaunch");
    }
    // The bookkeeping of n decode steps launched with launch_decode_graph.
    void sync_steps(int n) {
        yt::hip::check(hipStreamSynchronize(stream_), "qwen3: sync");
        for (auto& c : kv_caches) c.append(n);
    }

    // history[0, n) (the tokens picked since the last prompt) on the host.
    std::vector<int> history(int n) {
        std::vector<int32_t> h(n);
        yt::hip::check(hipMemcpyAsync(h.data(), history_.deviceData(), n * 4, hipMemcpyDeviceToHost, stream_),
                       "qwen3: history");
        yt::hip::check(hipStreamSynchronize(stream_), "qwen3: history");
        return std::vector<int>(h.begin(), h.end());
    }
    const yt::YTensor<float, 2>& logits() const { return logits_; }

    // Throws if a kernel flagged an out-of-range cache row, RoPE row or history
    // entry (the kernels never access those), or the device's TOTAL disagrees
    // with the host bookkeeping.
    void check_state() {
        int32_t st[YTHIP_ST_WORDS];
        yt::hip::check(hipMemcpyAsync(st, state_.deviceData(), sizeof st, hipMemcpyDeviceToHost, stream_),
                       "qwen3: state");
        yt::hip::check(hipStreamSynchronize(stream_), "qwen3: state");
        if (st[YTHIP_ST_ERROR])
            throw std::runtime_error("qwen3: decode state error bits " + std::to_string(st[YTHIP_ST_ERROR]));
        if (st[YTHIP_ST_TOTAL] != kv_caches[0].total_written)
            throw std::runtime_error("qwen3: decode state TOTAL " + std::to_string(st[YTHIP_ST_TOTAL]) +
                                     " != " + std::to_string(kv_caches[0].total_written));
    }

private:
    hipStream_t stream_ = nullptr;
    int max_ctx_ = 0, max_prompt_ = 0, max_tokens_ = 0, splits_ = 1;
    size_t ws_bytes_ = 0;
    yt::YTensor<float, 2> x_, logits_;
    yt::YTensor<T, 2> h_, qkv_, attn_, gu_, act_, hf_;
    yt::YTensor<T, 4> q_;
    yt::YTensor<int32_t, 1> ids_, token_, history_, state_;
    yt::YTensor<float, 1> amax_;
    yt::YTensor<uint8_t, 1> ws_;
    yt::YTensor<bool, 2> mask_;  // get_mask of a prompt into a full ring
    hipGraphExec_t decode_graph_ = nullptr;
    std::map<int, hipGraphExec_t> prefill_graphs_;

    static constexpr int code = yt::hip::dtype_code<T>();

    void release_graphs() {
        if (decode_graph_) (void)hipGraphExecDestroy(decode_graph_);
        decode_graph_ = nullptr;
        for (auto& kv : prefill_graphs_) (void)hipGraphExecDestroy(kv.second);
        prefill_graphs_.clear();
    }

    template <class F>
    hipGraphExec_t capture(F&& body) {
        yt::hip::StreamGuard g(stream_);
        hipGraph_t graph = nullptr;
        yt::hip::check(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal), "qwen3: capture");
        body();
        yt::hip::check(hipStreamEndCapture(stream_, &graph), "qwen3: capture");
        hipGraphExec_t exec = nullptr;
        yt::hip::check(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0), "qwen3: instantiate");
        yt::hip::check(hipGraphDestroy(graph), "qwen3: graph");
        return exec;
    }
    void capture_decode() { decode_graph_ = capture([&] { decode_body(); }); }

    // The decode-state record for the next token after `total` written ones
    // (KVCache rules, qwen3.cpp:70-126, 365-375), written before a replay.
    void write_state(int total) {
        int32_t st[YTHIP_ST_WORDS] = {0};
        const int ring = max_ctx_, P = config.max_position_embeddings;
        const int cur = std::min(total, ring);
        st[YTHIP_ST_TOTAL] = total;
        st[YTHIP_ST_RING] = ring;
        st[YTHIP_ST_MAX_POS] = P;
        st[YTHIP_ST_HISTORY] = max_tokens_;
        st[YTHIP_ST_SLOT] = total % ring;
        st[YTHIP_ST_KV_LEN] = std::min(total + 1, ring);
        st[YTHIP_ST_ROPE_POS] = total + 1 <= P ? total : (cur + 1 <= P ? cur : 0);
        yt::hip::check(hipMemcpyAsync(state_.deviceWrite(), st, sizeof st, hipMemcpyHostToDevice, stream_),
                       "qwen3: state");
        yt::hip::check(hipStreamSynchronize(stream_), "qwen3: state");
    }
    // Rolls the bookkeeping back (or forward) to `total` written tokens.
    void set_total(int total) {
        for (auto& c : kv_caches) {
            c.reset();
            c.append(total);
        }
        write_state(total);
    }

    // Qwen3Model::forward's prompt pass (qwen3.cpp:365-413) from t0 written
    // tokens: RoPE start rule, first cache row, visible keys, causal or get_mask.
    void prefill(const std::vector<int32_t>& ids, bool use_graph) {
        yt::hip::StreamGuard g(stream_);
        const Qwen3Config& c = config;
        const int P = static_cast<int>(ids.size());
        if (P == 0 || P > max_prompt_ || P > max_ctx_ || P > c.max_position_embeddings)
            throw std::invalid_argument("qwen3::forward: prompt of " + std::to_string(P) +
                                        " tokens (1 .. max_prompt, max_ctx, max_position_embeddings)");
        for (int t : ids)
            if (t < 0 || t >= c.vocab_size) throw std::invalid_argument("qwen3::forward: token id out of range");
        KVCache<T>& kc0 = kv_caches[0];
        const int t0 = kc0.total_written;
        int start = t0 > 0 ? kc0.get_global_position() : 0;
        if (start + P > c.max_position_embeddings) {
            start = kc0.cur_len;
            if (start + P > c.max_position_embeddings) start = 0;
        }
        const int row = kc0.write_pos;
        for (auto& kc : kv_caches) kc.append(P);
        const int kv_len = kc0.cur_len;
        const bool bool_mask = t0 + P > max_ctx_;  // full after the append: logical order
        if (bool_mask) {
            mask_ = kc0.get_mask(P);
            mask_.toDevice();
        }
        yt::hip::check(hipMemcpyAsync(ids_.deviceWrite(), ids.data(), P * 4, hipMemcpyHostToDevice, stream_),
                       "qwen3: ids");
        // the head's argmax counts the last prompt token as written: TOTAL = t0 + P after it
        write_state(t0 + P - 1);
        if (use_graph && t0 == 0 && !bool_mask) {
            auto it = prefill_graphs_.find(P);
            if (it == prefill_graphs_.end())
                it = prefill_graphs_.emplace(P, capture([&] { prefill_body(P, start, row, kv_len, false); })).first;
            yt::hip::check(hipGraphLaunch(it->second, stream_), "qwen3: hipGraphLaunch");
        } else {
            prefill_body(P, start, row, kv_len, bool_mask);
        }
    }

    void prefill_body(int S, int start, int row, int kv_len, bool bool_mask) {
        const Qwen3Config& c = config;
        const int H = c.hidden_size, I = c.intermediate_size, hd = c.head_dim;
        const int nh = c.num_attention_heads, nkv = c.num_key_value_heads, W = (nh + 2 * nkv) * hd;
        const float eps = c.rms_norm_eps;
        hipStream_t s = stream_;
        float* x = x_.deviceWrite();
        void* h = h_.deviceWrite();
        void* qkv = qkv_.deviceWrite();
        void* q = q_.deviceWrite();
        void* attn = attn_.deviceWrite();
        void* gu = gu_.deviceWrite();
        void* act = act_.deviceWrite();
        const float* cs = model.rope.cos.deviceData();
        const float* sn = model.rope.sin.deviceData();
        const int P = max_prompt_;
        auto ck = [](int st, const char* what) { yt::hip::check(st, what); };
        ck(ythip_embedding(code, YTHIP_F32, S, H, c.vocab_size, model.embed.deviceData(), ids_.deviceData(), x, H, s),
           "qwen3: embedding");
        const int64_t q_str[3] = {int64_t(nh) * P * hd, int64_t(P) * hd, hd};
        const int64_t kv_str[3] = {int64_t(nkv) * max_ctx_ * hd, int64_t(max_ctx_) * hd, hd};
        const int64_t q4[4] = {int64_t(nh) * P * hd, int64_t(P) * hd, hd, 1};
        const int64_t kv4[4] = {int64_t(nkv) * max_ctx_ * hd, int64_t(max_ctx_) * hd, hd, 1};
        const int64_t o4[4] = {int64_t(S) * nh * hd, hd, int64_t(nh) * hd, 1};  // attn [S, nh*hd] as [1, nh, S, hd]
        for (int i = 0; i < c.num_hidden_layers; ++i) {
            auto& L = model.layers[i];
            void* kc = kv_caches[i].k_buffer.deviceWrite();
            void* vc = kv_caches[i].v_buffer.deviceWrite();
            ck(ythip_rms_norm(YTHIP_F32, code, S, H, x, H, L.norm1.deviceData(), eps, h, H, s), "qwen3: norm1");
            ck(ythip_gemm(code, code, 1, S, W, H, h, 0, H, 1, L.qkv_proj.deviceData(), 0, 1, H, qkv, 0, W, 1, 1.f,
                          0.f, s),
               "qwen3: qkv");
            ck(ythip_rmsnorm_rope(code, 1, S, nh, nkv, hd, qkv, W, L.q_norm.deviceData(), L.k_norm.deviceData(), eps,
                                  cs, sn, hd, c.max_position_embeddings, start, q, q_str, kc, kv_str, vc, kv_str,
                                  max_ctx_, row, nullptr, s),
               "qwen3: q/k norm + rope");
            const int kind = bool_mask ? YTHIP_MASK_BOOL : YTHIP_MASK_CAUSAL;
            const uint8_t* mp = bool_mask ? reinterpret_cast<const uint8_t*>(mask_.deviceData()) : nullptr;
            const int64_t mld = bool_mask ? kv_len : 0;
            if (bool_mask || S == 1) {
                const size_t need = ythip_attn_sdpa_workspace_size(1, nh, S, kv_len, hd);
                ck(ythip_attn_prefill_ws(code, 1, nh, nkv, S, kv_len, hd, hd, q, q4, kc, kv4, vc, kv4, attn, o4, 0.f,
                                         kind, mp, mld, nullptr, 0, 0, ws_.deviceWrite(), need, s),
                   "qwen3: attention");
            } else {
                ck(ythip_attn_prefill(code, 1, nh, nkv, S, kv_len, hd, hd, q, q4, kc, kv4, vc, kv4, attn, o4, 0.f, kind,
                                      mp, mld, nullptr, 0, 0, s),
                   "qwen3: attention");
            }
            ck(ythip_gemm(code, YTHIP_F32, 1, S, H, nh * hd, attn, 0, nh * hd, 1, L.o_proj.deviceData(), 0, 1,
                          nh * hd, x, 0, H, 1, 1.f, 1.f, s),
               "qwen3: o_proj");
            ck(ythip_rms_norm(YTHIP_F32, code, S, H, x, H, L.norm2.deviceData(), eps, h, H, s), "qwen3: norm2");
            ck(ythip_gemm(code, code, 1, S, 2 * I, H, h, 0, H, 1, L.gate_up.deviceData(), 0, 1, H, gu, 0, 2 * I, 1,
                          1.f, 0.f, s),
               "qwen3: gate_up");
            ck(ythip_silu_mul(code, code, S, I, gu, 2 * I, act, I, s), "qwen3: swiglu");
            ck(ythip_gemm(code, YTHIP_F32, 1, S, H, I, act, 0, I, 1, L.down.deviceData(), 0, 1, I, x, 0, H, 1, 1.f,
                          1.f, s),
               "qwen3: down");
        }
        ck(ythip_rms_norm(YTHIP_F32, code, 1, H, x + int64_t(S - 1) * H, H, model.norm.deviceData(), eps,
                          hf_.deviceWrite(), H, s),
           "qwen3: final norm");
        ck(ythip_gemm(code, YTHIP_F32, 1, 1, c.vocab_size, H, hf_.deviceData(), 0, H, 1, model.head().deviceData(), 0,
                      1, H, logits_.deviceWrite(), 0, c.vocab_size, 1, 1.f, 0.f, s),
           "qwen3: lm_head");
        ck(ythip_argmax_step(c.vocab_size, logits_.deviceData(), token_.deviceWrite(), history_.deviceWrite(),
                             state_.deviceWrite(), s),
           "qwen3: argmax");
    }

    // One generated token (Qwen3Model::forward with l = 1 and the head), every
    // position taken from the decode-state record.
    void decode_body() {
        const Qwen3Config& c = config;
        const int H = c.hidden_size, I = c.intermediate_size, hd = c.head_dim;
        const int nh = c.num_attention_heads, nkv = c.num_key_value_heads, W = (nh + 2 * nkv) * hd;
        const float eps = c.rms_norm_eps;
        hipStream_t s = stream_;
        float* x = x_.deviceWrite();
        void* qkv = qkv_.deviceWrite();
        void* act = act_.deviceWrite();
        int32_t* st = state_.deviceWrite();
        float* ws = reinterpret_cast<float*>(ws_.deviceWrite());
        auto ck = [](int r, const char* what) { yt::hip::check(r, what); };
        ck(ythip_embedding(code, YTHIP_F32, 1, H, c.vocab_size, model.embed.deviceData(), token_.deviceData(), x, H,
                           s),
           "qwen3: embedding");
        const int64_t kv_str[3] = {int64_t(nkv) * max_ctx_ * hd, int64_t(max_ctx_) * hd, hd};
        const int64_t ld_part = int64_t(nh) * splits_ * (hd + 2);
        for (int i = 0; i < c.num_hidden_layers; ++i) {
            auto& L = model.layers[i];
            ck(ythip_gemv_fused(1, code, code, 1, W, H, x, H, L.norm1.deviceData(), eps, L.qkv_proj.deviceData(), H,
                                qkv, W, 1.f, 0.f, nullptr, s),
               "qwen3: norm1 + qkv");
            ck(ythip_attn_decode_rope(code, 1, nh, nkv, hd, max_ctx_, qkv, W, L.q_norm.deviceData(),
                                      L.k_norm.deviceData(), eps, model.rope.cos.deviceData(),
                                      model.rope.sin.deviceData(), hd, c.max_position_embeddings, st,
                                      kv_caches[i].k_buffer.deviceWrite(), kv_caches[i].v_buffer.deviceWrite(), kv_str,
                                      nullptr, nullptr, 0.f, ws, ws_bytes_, s),
               "qwen3: q/k norm + rope + attention");
            ck(ythip_gemv_attn_merge(code, YTHIP_F32, 1, H, nh, hd, splits_, ws, ld_part, L.o_proj.deviceData(),
                                     nh * hd, x, H, 1.f, 1.f, st, max_ctx_, s),
               "qwen3: merge + o_proj");
            ck(ythip_gemv_swiglu(1, code, 1, I, H, x, H, L.norm2.deviceData(), eps, L.gate_up.deviceData(), H, act, I,
                                 s),
               "qwen3: norm2 + gate_up + swiglu");
            ck(ythip_gemv_fused(0, code, YTHIP_F32, 1, H, I, act, I, nullptr, eps, L.down.deviceData(), I, x, H, 1.f,
                                1.f, nullptr, s),
               "qwen3: down");
        }
        ck(ythip_gemv_fused(1, code, YTHIP_F32, 1, c.vocab_size, H, x, H, model.norm.deviceData(), eps,
                            model.head().deviceData(), H, logits_.deviceWrite(), c.vocab_size, 1.f, 0.f,
                            amax_.deviceWrite(), s),
           "qwen3: final norm + lm_head");
        ck(ythip_argmax_finish(amax_.deviceData(), amax_.shape(0) / 2, token_.deviceWrite(), history_.deviceWrite(),
                               st, s),
           "qwen3: argmax");
    }
};

}  // namespace qwen3
