// Runs the hot path through the reference's own C++ operator signatures on the
// GPU (include/yt/ytensor.hpp over libythip.so) and writes every result as raw
// float32 into the directory given as argv[1], for tests/test_gpu_host_cpp.py to
// compare with the golden fixtures and the oracle. Inputs come from
// YTensor::seed / randn exactly as the configs specify them.
//   randn0_head   seed(0), randn(64)                      (vs fixture randn0_head, bit-exact)
//   c0            configs[0]: seed(0); A, B = randn(1024, 1024); A.matmul(B, MatmulBackend::HIP)
//   c1_nn, c1_nt  configs[1] (128, 3072, 1024) bf16: A ~ N(0,1), B [K,N] ~ N(0,0.02) via
//                 YTensor::matmul; W [N,K] ~ N(0,0.02) via yt::function::linear
//   c1_bias       linear(x, W, b) in fp32 on a small shape
//   prefill       configs[2] at S=256: seed(1) Q, K, V bf16; the qwen3 example's call
//                 (5-D q, repeat_kv'd K/V, bool causal mask, FLASH_AVX2: qwen3.cpp:250-264)
//   prefill_pred  the same with the CausalMask predicate and FLASH_HIP
//   prefill_math  the same through sdpaBackend::MATH
//   decode        configs[3] (B=1, ctx 1024): seed(2) K, V, Q; one query per head
//   dec_B{B}_c{ctx}  configs[3] at all four (B, ctx) in the Qwen3 example's per-token call
//                 form (qwen3.cpp:250-264): 5-D q, repeat_kv'd K/V, KVCache::get_mask's bool
//                 mask of a wrapped ring (qwen3.cpp:104-126), FLASH_AVX2
//   dec_rand      B=1, ctx 1024: a random bool mask and a bias row
//   dec_none      the same inputs with an all-false mask (zeros)
//   dec_pred      the same inputs with the CausalMask{ctx/2} predicate (keys 0..ctx/2)
//   dec_g5        repeat_kv by 5 (40 q heads over 8 kv heads), ctx 512, bool mask
//   concurrent    two std::threads on two streams decoding configs[3]'s B=16 / B=1 ctx 8192
//                 inputs 12 times each at once: mismatches against the serial bits (0)
//   rmsnorm       seed(12) x [2,3,128], w [128]; rmsNorm_(x, w, -1, 1e-6) (vs fixture rmsnorm)
//   rmsnorm_oop   rmsNorm(x, w, -1, 1e-6) out of place (same values)
//   rmsnorm_ax1   seed(13) x [2,64,3]; rmsNorm_(x, w[64], 1, 1e-6) (a strided axis)
//   rmsnorm_ax12  seed(14) x [2,4,32]; rmsNorm(x, w[4,32], {1,2}, 1e-6)
#include <cstdio>
#include <cstring>
#include <fstream>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "yt/ytensor.hpp"

using yt::YTensor;
using yt::bfloat16;
namespace hip = yt::hip;

static std::string g_dir;

template <class T, int d>
static void dump(const char* name, const YTensor<T, d>& t) {
    const auto c = t.contiguous();
    const T* p = c.data();
    std::vector<float> buf(c.size());
    for (size_t i = 0; i < buf.size(); ++i) buf[i] = static_cast<float>(p[i]);
    std::ofstream f(g_dir + "/" + name + ".f32", std::ios::binary);
    f.write(reinterpret_cast<const char*>(buf.data()), static_cast<std::streamsize>(buf.size() * sizeof(float)));
    std::printf("%s:", name);
    for (int s : t.shape()) std::printf(" %d", s);
    std::printf("\n");
}

template <int d>
static YTensor<bfloat16, d> to_bf16(const YTensor<float, d>& x, float scale = 1.0f) {
    YTensor<bfloat16, d> out(x.shape());
    const float* s = x.data();
    bfloat16* o = out.data();
    for (size_t i = 0; i < x.size(); ++i) o[i] = bfloat16(s[i] * scale);
    return out;
}

static YTensor<bool, 2> causal_mask(int q_len, int kv_len) {  // example/qwen3/src/qwen3.cpp:46-55
    YTensor<bool, 2> m(std::vector<int>{q_len, kv_len});
    const int start = kv_len - q_len;
    for (int qi = 0; qi < q_len; ++qi)
        for (int ki = 0; ki < kv_len; ++ki) m.at(qi, ki) = ki <= start + qi;
    return m;
}

static YTensor<bfloat16, 5> repeat_kv(const YTensor<bfloat16, 4>& x, int n) {  // qwen3.cpp:583-589
    return x.unsqueeze(2).repeat(1, 1, n, 1, 1);
}

// KVCache::get_mask(query_len) of a ring of max_len rows that has wrapped, with
// its next write at write_pos (example/qwen3/src/qwen3.cpp:104-126).
static YTensor<bool, 2> ring_mask(int query_len, int max_len, int write_pos) {
    YTensor<bool, 2> m(std::vector<int>{query_len, max_len});
    const int start = max_len - query_len;
    for (int qi = 0; qi < query_len; ++qi)
        for (int ki = 0; ki < max_len; ++ki) m.at(qi, ki) = (ki - write_pos + max_len) % max_len <= start + qi;
    return m;
}

// seed(2); K, V = randn(B, 8, ctx, 128), Q = randn(B, 16, 1, 128), bf16.
struct DecodeCase {
    YTensor<bfloat16, 4> K, V, Q;
};
static DecodeCase decode_case(int B, int ctx) {
    YTensor<float, 4>::seed(2);
    DecodeCase c;
    c.K = to_bf16(YTensor<float, 4>::randn(B, 8, ctx, 128));
    c.V = to_bf16(YTensor<float, 4>::randn(B, 8, ctx, 128));
    c.Q = to_bf16(YTensor<float, 4>::randn(B, 16, 1, 128));
    return c;
}

// The Qwen3 example's per-token attention call (qwen3.cpp:250-264).
static YTensor<bfloat16, 5> qwen3_decode_call(const DecodeCase& c, YTensor<bool, 2>& mask) {
    const int B = c.Q.shape(0);
    auto q5 = c.Q.view(B, 8, 2, 1, 128);
    auto k5 = repeat_kv(c.K, 2);
    auto v5 = repeat_kv(c.V, 2);
    return yt::function::scaledDotProductAttention(q5, k5, v5, bfloat16(0.0f), &mask, nullptr,
                                                   yt::function::sdpaBackend::FLASH_AVX2);
}

static std::vector<uint16_t> bits_of(const YTensor<bfloat16, 5>& t) {
    const auto c = t.contiguous();
    std::vector<uint16_t> b(c.size());
    std::memcpy(b.data(), c.data(), b.size() * sizeof(uint16_t));
    return b;
}

int main(int argc, char** argv) {
    if (argc < 2) {
        std::fprintf(stderr, "usage: %s OUT_DIR\n", argv[0]);
        return 2;
    }
    g_dir = argv[1];
    using yt::infos::MatmulBackend;
    using yt::function::sdpaBackend;

    YTensor<float, 1>::seed(0);
    dump("randn0_head", YTensor<float, 1>::randn(64));

    // configs[0]
    YTensor<float, 2>::seed(0);
    auto A = YTensor<float, 2>::randn(1024, 1024);
    auto B = YTensor<float, 2>::randn(1024, 1024);
    dump("c0", A.matmul(B, MatmulBackend::HIP));

    // configs[1], (M, N, K) = (128, 3072, 1024)
    const int M = 128, N = 3072, K = 1024;
    YTensor<float, 2>::seed(0);
    auto a16 = to_bf16(YTensor<float, 2>::randn(M, K));
    auto b16 = to_bf16(YTensor<float, 2>::randn(K, N), 0.02f);
    dump("c1_nn", a16.matmul(b16));
    YTensor<float, 2>::seed(0);
    auto x16 = to_bf16(YTensor<float, 2>::randn(M, K));
    auto w16 = to_bf16(YTensor<float, 2>::randn(N, K), 0.02f);
    dump("c1_nt", yt::function::linear(x16, w16));

    YTensor<float, 2>::seed(5);
    auto xs = YTensor<float, 2>::randn(33, 64);
    auto ws = YTensor<float, 2>::randn(40, 64);
    auto bs = YTensor<float, 1>::randn(40);
    dump("c1_bias", yt::function::linear(xs, ws, bs));
    bool threw = false;
    try {
        yt::function::linear(xs, YTensor<float, 2>::randn(40, 63));
    } catch (const std::invalid_argument&) {
        threw = true;
    }
    if (!threw) {
        std::fprintf(stderr, "linear with mismatched features did not throw\n");
        return 1;
    }

    // configs[2] layout at S = 256: q [1,16,S,128], k/v [1,8,S,128]
    const int S = 256, D = 128;
    YTensor<float, 4>::seed(1);
    auto Q = to_bf16(YTensor<float, 4>::randn(1, 16, S, D));
    auto Kt = to_bf16(YTensor<float, 4>::randn(1, 8, S, D));
    auto Vt = to_bf16(YTensor<float, 4>::randn(1, 8, S, D));
    auto q5 = Q.view(1, 8, 2, S, D);
    auto k5 = repeat_kv(Kt, 2);
    auto v5 = repeat_kv(Vt, 2);
    auto mask = causal_mask(S, S);
    const bfloat16 rs(0.0f);  // 0: 1/sqrt(d) in float (ops.inl:378-381); a bf16-typed scale would be rounded
    dump("prefill", yt::function::scaledDotProductAttention(q5, k5, v5, rs, &mask, nullptr, sdpaBackend::FLASH_AVX2));
    dump("prefill_pred", yt::function::scaledDotProductAttention(q5, k5, v5, rs, yt::function::CausalMask{0},
                                                                 nullptr, sdpaBackend::FLASH_HIP));
    dump("prefill_math", yt::function::scaledDotProductAttention(q5, k5, v5, rs, &mask, nullptr, sdpaBackend::MATH));

    // configs[3], B = 1, ctx = 1024 (K, V, then Q)
    const int ctx = 1024;
    YTensor<float, 4>::seed(2);
    auto Kc = to_bf16(YTensor<float, 4>::randn(1, 8, ctx, D));
    auto Vc = to_bf16(YTensor<float, 4>::randn(1, 8, ctx, D));
    auto Qd = to_bf16(YTensor<float, 4>::randn(1, 16, 1, D));
    auto qd5 = Qd.view(1, 8, 2, 1, D);
    auto kd5 = repeat_kv(Kc, 2);
    auto vd5 = repeat_kv(Vc, 2);
    dump("decode", yt::function::scaledDotProductAttention(qd5, kd5, vd5, bfloat16(0.0f), nullptr, nullptr,
                                                           sdpaBackend::FLASH_HIP));

    // configs[3] at every (B, ctx) in the example's per-token call form, the
    // bool mask from a wrapped ring (one query row: every key visible)
    const int shapes[4][2] = {{1, 1024}, {1, 8192}, {16, 1024}, {16, 8192}};
    for (const auto& bc : shapes) {
        const auto c = decode_case(bc[0], bc[1]);
        auto m = ring_mask(1, bc[1], bc[1] / 3);
        const std::string name = "dec_B" + std::to_string(bc[0]) + "_c" + std::to_string(bc[1]);
        dump(name.c_str(), qwen3_decode_call(c, m));
    }
    {
        const auto c = decode_case(1, 1024);
        auto q5 = c.Q.view(1, 8, 2, 1, 128);
        auto k5 = repeat_kv(c.K, 2);
        auto v5 = repeat_kv(c.V, 2);
        YTensor<float, 2>::seed(21);
        auto r = YTensor<float, 2>::randn(1, 1024);
        YTensor<bool, 2> m(std::vector<int>{1, 1024});
        for (int j = 0; j < 1024; ++j) m.at(0, j) = r.at(0, j) > -0.5f;  // about 70% visible
        auto bias = to_bf16(YTensor<float, 2>::randn(1, 1024));
        dump("dec_rand", yt::function::scaledDotProductAttention(q5, k5, v5, bfloat16(0.0f), &m, &bias,
                                                                 sdpaBackend::FLASH_AVX2));
        YTensor<bool, 2> none(std::vector<int>{1, 1024});
        dump("dec_none", yt::function::scaledDotProductAttention(q5, k5, v5, bfloat16(0.0f), &none, nullptr,
                                                                 sdpaBackend::FLASH_HIP));
        dump("dec_pred", yt::function::scaledDotProductAttention(q5, k5, v5, bfloat16(0.0f),
                                                                 yt::function::CausalMask{512}, nullptr,
                                                                 sdpaBackend::FLASH_HIP));
    }
    {
        // repeat_kv by 5 (Qwen3-14B's 40 / 8 heads) on the decode kernel
        YTensor<float, 4>::seed(22);
        auto K5 = to_bf16(YTensor<float, 4>::randn(1, 8, 512, 128));
        auto V5 = to_bf16(YTensor<float, 4>::randn(1, 8, 512, 128));
        auto Q5 = to_bf16(YTensor<float, 4>::randn(1, 40, 1, 128));
        auto q5 = Q5.view(1, 8, 5, 1, 128);
        auto k5 = repeat_kv(K5, 5);
        auto v5 = repeat_kv(V5, 5);
        auto m = ring_mask(1, 512, 100);
        dump("dec_g5", yt::function::scaledDotProductAttention(q5, k5, v5, bfloat16(0.0f), &m, nullptr,
                                                               sdpaBackend::FLASH_AVX2));
    }
    {
        // two host threads, each on its own stream, decoding different inputs at
        // the same time: every result must have the serial bits
        const auto ca = decode_case(16, 8192), cb = decode_case(1, 8192);
        auto ma = ring_mask(1, 8192, 5), mb = ring_mask(1, 8192, 7);
        const auto ra = bits_of(qwen3_decode_call(ca, ma)), rb = bits_of(qwen3_decode_call(cb, mb));
        hip::check(hipDeviceSynchronize(), "sync");
        int bad[2] = {0, 0};
        auto worker = [&](int id) {
            hipStream_t st;
            hip::check(hipStreamCreate(&st), "hipStreamCreate");
            {
                yt::hip::StreamGuard g(st);
                std::vector<YTensor<bfloat16, 5>> outs;
                for (int it = 0; it < 12; ++it) {
                    auto mcopy = id == 0 ? ma : mb;
                    outs.push_back(qwen3_decode_call(id == 0 ? ca : cb, mcopy));
                }
                for (auto& o : outs) bad[id] += bits_of(o) != (id == 0 ? ra : rb);
                yt::hip::releaseWorkspace();
            }
            hip::check(hipStreamDestroy(st), "hipStreamDestroy");
        };
        std::thread t0(worker, 0), t1(worker, 1);
        t0.join();
        t1.join();
        YTensor<float, 1> mism(std::vector<int>{1});
        mism.at(0) = static_cast<float>(bad[0] + bad[1]);
        dump("concurrent", mism);
    }

    // rmsNorm_ (the golden fixture's norm case)
    YTensor<float, 3>::seed(12);
    auto xn = YTensor<float, 3>::randn(2, 3, 128);
    auto wn = YTensor<float, 1>::randn(128);
    dump("rmsnorm_oop", yt::function::rmsNorm(xn, wn, -1, 1e-6f));
    yt::function::rmsNorm_(xn, wn, -1, 1e-6f);
    dump("rmsnorm", xn);
    YTensor<float, 3>::seed(13);
    auto xa = YTensor<float, 3>::randn(2, 64, 3);
    auto wa = YTensor<float, 1>::randn(64);
    yt::function::rmsNorm_(xa, wa, 1, 1e-6f);
    dump("rmsnorm_ax1", xa);
    YTensor<float, 3>::seed(14);
    auto xb = YTensor<float, 3>::randn(2, 4, 32);
    auto wb = YTensor<float, 2>::randn(4, 32);
    dump("rmsnorm_ax12", yt::function::rmsNorm(xb, wb, std::vector<int>{1, 2}, 1e-6f));

    std::printf("done\n");
    return 0;
}
