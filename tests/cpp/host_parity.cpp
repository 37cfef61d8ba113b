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
//   rmsnorm       seed(12) x [2,3,128], w [128]; rmsNorm_(x, w, -1, 1e-6) (vs fixture rmsnorm)
#include <cstdio>
#include <fstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "yt/ytensor.hpp"

using yt::YTensor;
using yt::bfloat16;

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

    // rmsNorm_ (the golden fixture's norm case)
    YTensor<float, 3>::seed(12);
    auto xn = YTensor<float, 3>::randn(2, 3, 128);
    auto wn = YTensor<float, 1>::randn(128);
    yt::function::rmsNorm_(xn, wn, -1, 1e-6f);
    dump("rmsnorm", xn);

    std::printf("done\n");
    return 0;
}
