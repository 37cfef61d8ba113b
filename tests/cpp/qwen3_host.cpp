// configs[4] through the C++ host: the Qwen3 decoder of include/yt/qwen3.hpp
// (the example's Qwen3ForCausalLM over include/yt/ytensor.hpp and libythip.so)
// with random-init weights drawn by YTensor::seed / randn in the model's layout
// order, a prompt read from a file of int32 token ids, greedy decoding.
//
//   yt_qwen3 fixture PROMPT OUT_DIR STEPS SEED SCALE NORM_SPREAD
//       prompt, then STEPS tokens one graph replay at a time; writes each step's
//       fp32 logits to OUT_DIR/logits.f32 and the tokens to OUT_DIR/tokens.i32
//       (tests/test_gpu_qwen3_cpp.py checks them against the compiled reference's
//       fixture). Also runs generate() on a fresh cache and writes its tokens to
//       OUT_DIR/generate.i32.
//   yt_qwen3 bench PROMPT N_TOKENS
//       configs[4] (seed 3, randn * 0.02): the prompt's forward as a captured graph,
//       then N_TOKENS - 1 decode graph replays timed with HIP events; prints one
//       JSON line (prefill ms, decode tok/s).
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <string>
#include <vector>

#include "yt/qwen3.hpp"

static std::vector<int> read_ids(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot open " + path);
    std::vector<int32_t> v;
    int32_t x;
    while (f.read(reinterpret_cast<char*>(&x), 4)) v.push_back(x);
    return std::vector<int>(v.begin(), v.end());
}

template <class V>
static void write_raw(const std::string& path, const V& v, std::ios::openmode extra = {}) {
    std::ofstream f(path, std::ios::binary | extra);
    f.write(reinterpret_cast<const char*>(v.data()), static_cast<std::streamsize>(v.size() * sizeof(v[0])));
}

static double seconds_since(std::chrono::steady_clock::time_point t0) {
    return std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
}

int main(int argc, char** argv) {
    if (argc < 3) {
        std::fprintf(stderr, "usage: %s fixture PROMPT OUT_DIR STEPS SEED SCALE NORM_SPREAD | bench PROMPT N\n",
                     argv[0]);
        return 2;
    }
    const std::string mode = argv[1];
    const auto prompt = read_ids(argv[2]);
    qwen3::Qwen3Config cfg;  // the defaults are Qwen3-0.6B's
    using Model = qwen3::Qwen3ForCausalLM<yt::bfloat16>;
    try {
        if (mode == "fixture" && argc >= 8) {
            const std::string out = argv[3];
            const int steps = std::atoi(argv[4]);
            const unsigned seed = static_cast<unsigned>(std::atoi(argv[5]));
            const float scale = std::strtof(argv[6], nullptr), spread = std::strtof(argv[7], nullptr);
            Model m;
            m.init(cfg, 512, 1024, 4096);
            auto t0 = std::chrono::steady_clock::now();
            m.init_random(seed, scale, spread);
            std::printf("weights drawn in %.1f s\n", seconds_since(t0));
            std::fflush(stdout);
            yt::YTensor<int, 2> ids(std::vector<int>{1, static_cast<int>(prompt.size())});
            for (size_t j = 0; j < prompt.size(); ++j) ids.at(0, static_cast<int>(j)) = prompt[j];
            std::ofstream(out + "/logits.f32", std::ios::binary | std::ios::trunc);
            std::vector<float> lg(cfg.vocab_size);
            m.forward(ids, false, true);
            for (int k = 0; k < steps; ++k) {
                if (k > 0) m.launch_decode_graph();
                yt::hip::check(hipMemcpyAsync(lg.data(), m.logits().deviceData(), lg.size() * 4,
                                              hipMemcpyDeviceToHost, m.stream()),
                               "logits");
                yt::hip::check(hipStreamSynchronize(m.stream()), "sync");
                write_raw(out + "/logits.f32", lg, std::ios::app);
            }
            m.sync_steps(steps - 1);
            m.check_state();
            const auto toks = m.history(steps);
            write_raw(out + "/tokens.i32", std::vector<int32_t>(toks.begin(), toks.end()));
            // the example's API on a fresh turn: generate from an empty cache
            m.reset_kv_cache();
            const auto gen = m.generate(prompt, steps, -1);
            write_raw(out + "/generate.i32", std::vector<int32_t>(gen.begin(), gen.end()));
            std::printf("tokens:");
            for (int t : toks) std::printf(" %d", t);
            std::printf("\ndone\n");
            return 0;
        }
        if (mode == "bench" && argc >= 4) {
            const int n = std::atoi(argv[3]);
            const int P = static_cast<int>(prompt.size());
            Model m;
            m.init(cfg, P, P + n + 64, 4096);
            auto t0 = std::chrono::steady_clock::now();
            m.init_random(3, 0.02f, 0.0f);
            const double init_s = seconds_since(t0);
            yt::YTensor<int, 2> ids(std::vector<int>{1, P});
            for (int j = 0; j < P; ++j) ids.at(0, j) = prompt[j];
            hipEvent_t e0, e1;
            yt::hip::check(hipEventCreate(&e0), "event");
            yt::hip::check(hipEventCreate(&e1), "event");
            auto fwd = [&](bool graph) {
                m.reset_kv_cache();
                yt::hip::check(hipEventRecord(e0, m.stream()), "event");
                m.forward(ids, false, graph);
                yt::hip::check(hipEventRecord(e1, m.stream()), "event");
                yt::hip::check(hipEventSynchronize(e1), "event");
                float ms = 0;
                yt::hip::check(hipEventElapsedTime(&ms, e0, e1), "event");
                return ms;
            };
            fwd(false);  // warm-up
            const float eager_ms = fwd(false);
            fwd(true);  // capture + first replay
            const float graph_ms = fwd(true);
            m.launch_decode_graph();  // capture the step + one warm replay
            m.sync_steps(1);
            yt::hip::check(hipEventRecord(e0, m.stream()), "event");
            for (int i = 0; i < n - 2; ++i) m.launch_decode_graph();
            yt::hip::check(hipEventRecord(e1, m.stream()), "event");
            yt::hip::check(hipEventSynchronize(e1), "event");
            float dec_ms = 0;
            yt::hip::check(hipEventElapsedTime(&dec_ms, e0, e1), "event");
            m.sync_steps(n - 2);
            m.check_state();
            const auto toks = m.history(n);
            int distinct = 0;
            {
                std::vector<int> s(toks);
                std::sort(s.begin(), s.end());
                distinct = static_cast<int>(std::unique(s.begin(), s.end()) - s.begin());
            }
            const double per_tok = dec_ms / (n - 2);
            std::printf("{\"host\": \"C++ (include/yt/qwen3.hpp)\", \"decode_tok_s\": %.1f, \"ms_per_token\": %.4f, "
                        "\"prefill_ms_512\": %.3f, \"prefill_ms_512_eager\": %.3f, \"tokens_timed\": %d, "
                        "\"distinct_tokens\": %d, \"weight_init_s\": %.1f}\n",
                        1e3 / per_tok, per_tok, graph_ms, eager_ms, n - 2, distinct, init_s);
            return 0;
        }
    } catch (const std::exception& e) {
        std::fprintf(stderr, "error: %s\n", e.what());
        return 1;
    }
    std::fprintf(stderr, "bad arguments\n");
    return 2;
}
