// yt/ytensor.hpp -- a from-scratch, header-only subset of YTensor's C++20 host
// API (SnifferCaptain/ytensor v0.13) whose operators run on one MI355X through
// libythip.so. It keeps the reference's names, signatures and argument
// meanings for the hot path:
//   yt::YTensor<T, dim>               storage = std::shared_ptr<char[]> + element
//                                     offset + int shape / strides
//                                     (include/ytensor_base.hpp:388-393)
//   YTensor::matmul(other, backend)   (include/ytensor_math.hpp:70-73,
//                                     src/ytensor_math.inl:284-316, 954-1051)
//   yt::infos::MatmulBackend          + HIP (include/ytensor_infos.hpp:125-141)
//   yt::function::matmul / linear     (include/function/ops.hpp:10-19, src/function/ops.inl:84-104)
//   yt::function::sdpaBackend         + FLASH_HIP (include/function/ops.hpp:21-24)
//   yt::function::scaledDotProductAttention, all four overloads
//                                     (include/function/ops.hpp:26-70, src/function/ops.inl:368-503)
//   yt::function::rmsNorm / rmsNorm_  (include/function/normalization.hpp:59-89), any neighbouring axes
//   yt::kernel::hip::{sgemm, matmul, hgemm, flash_attention, sdpa_gqa}
//                                     the kernel API (include/kernel/avx2/sgemm.hpp:51-68,
//                                     hgemm.hpp:26-42, flash_attention.hpp:21-69) on device pointers
//   YTensor::seed / randn             (include/ytensor_core.hpp:44-58, 350-361)
//   yt::bfloat16, yt::float16         (include/types/bfloat16.hpp, include/types/float_spec.hpp)
//
// Device memory. Every storage block owns a device mirror (detail::Mirror),
// shared by all views of it exactly as they share _data, and freed with it.
// The mirror tracks which copy is current: an operator uploads an operand whose
// device copy is stale, writes its result on the device only, and host access
// (data(), at()) downloads a stale host copy first -- so results read like the
// reference's while staying in HBM between operators. toDevice() / toHost()
// move a tensor explicitly.
//
// Streams. Every operator launches on yt::hip::stream() (a per-thread
// hipStream_t, NULL by default; set it with yt::hip::StreamGuard), which it
// passes to the C ABI call by call. Device scratch (split-K partials of
// single-query attention, a bool mask's tile classes, MATH scores) comes from
// yt::hip::workspace(): one buffer per host thread and (device, stream), kept
// and grown by the host, so operators on different threads or streams never
// share one and operators on one stream reuse it in launch order.
//
// Errors. Argument problems raise std::invalid_argument, as the reference's
// L3/L4 callers do (src/function/ops.inl:123-128, 382-387); a failing HIP call
// or kernel launch raises std::runtime_error with ythip_last_error().
//
// This build has no CPU kernels: every MatmulBackend / sdpaBackend value that
// names a CPU implementation (Naive, Eigen, AVX2, FLASH_AVX2) runs the HIP
// kernels too -- a call site such as the Qwen3 example's attention, which asks
// for FLASH_AVX2 (example/qwen3/src/qwen3.cpp:256-264), needs no edit. MATH
// runs the materialised-score path (ythip_attn_math).
//
// Compile with a C++20 host compiler, -I<repo>/include -I/opt/rocm/include
// -D__HIP_PLATFORM_AMD__, and link libythip.so and libamdhip64.so.
#pragma once

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <functional>
#include <initializer_list>
#include <map>
#include <memory>
#include <mutex>
#include <numeric>
#include <random>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <utility>
#include <vector>

#include "../ythip.h"

namespace yt {

// ---------------------------------------------------------------------------
// 16-bit storage types. The casts are the reference's (bfloat16.hpp:78-98:
// round half up on an odd last bit, truncate otherwise; float_spec.hpp:435-491:
// round to nearest even, subnormals flushed to zero), taken from libythip's
// host converter so there is one implementation of them.
// ---------------------------------------------------------------------------
struct bfloat16 {
    uint16_t bits = 0;
    bfloat16() = default;
    bfloat16(float f) { ythip_convert_host(YTHIP_F32, YTHIP_BF16, &f, &bits, 1); }
    operator float() const {
        float f;
        ythip_convert_host(YTHIP_BF16, YTHIP_F32, &bits, &f, 1);
        return f;
    }
};

struct float16 {
    uint16_t bits = 0;
    float16() = default;
    float16(float f) { ythip_convert_host(YTHIP_F32, YTHIP_F16, &f, &bits, 1); }
    operator float() const {
        float f;
        ythip_convert_host(YTHIP_F16, YTHIP_F32, &bits, &f, 1);
        return f;
    }
};

namespace infos {
// include/ytensor_infos.hpp:125-141 plus this build's back end.
enum class MatmulBackend { Naive = 0, Eigen = 1, AVX2 = 2, HIP = 3 };
inline constexpr MatmulBackend defaultMatmulBackend = MatmulBackend::HIP;
// The shared generator of YTensor::seed / randn (ytensor_infos.hpp:81-85).
inline std::mt19937 gen = std::mt19937(std::random_device{}());
inline std::mutex rngMutex;
}  // namespace infos

namespace hip {

inline hipStream_t& stream() {
    thread_local hipStream_t s = nullptr;
    return s;
}

// Runs the operators of a scope on stream s (restores the previous stream).
struct StreamGuard {
    hipStream_t prev;
    explicit StreamGuard(hipStream_t s) : prev(stream()) { stream() = s; }
    ~StreamGuard() { stream() = prev; }
    StreamGuard(const StreamGuard&) = delete;
    StreamGuard& operator=(const StreamGuard&) = delete;
};

inline void check(int status, const std::string& what) {
    if (status == 0) return;
    const std::string msg = what + ": " + ythip_last_error();
    if (status == YTHIP_EINVAL || status == YTHIP_EUNSUPPORTED) throw std::invalid_argument(msg);
    throw std::runtime_error(msg);
}

inline void check(hipError_t e, const std::string& what) {
    if (e != hipSuccess) throw std::runtime_error(what + ": " + hipGetErrorString(e));
}

// Device scratch of the calling thread for the current device and stream,
// at least `bytes` long (grown in 1 MiB steps; the old buffer is freed once
// the stream has finished with it). Freed when the thread ends.
struct ThreadWorkspaces {
    struct Buf {
        void* p = nullptr;
        size_t bytes = 0;
    };
    std::map<std::pair<int, hipStream_t>, Buf> bufs;
    ThreadWorkspaces() = default;
    ThreadWorkspaces(const ThreadWorkspaces&) = delete;
    ThreadWorkspaces& operator=(const ThreadWorkspaces&) = delete;
    ~ThreadWorkspaces() {
        for (auto& kv : bufs)
            if (kv.second.p) (void)hipFree(kv.second.p);
    }
};

inline ThreadWorkspaces& thread_workspaces() {
    thread_local ThreadWorkspaces w;
    return w;
}

inline void* workspace(size_t bytes) {
    if (bytes == 0) return nullptr;
    int dev = 0;
    check(hipGetDevice(&dev), "yt: hipGetDevice");
    auto& b = thread_workspaces().bufs[{dev, stream()}];
    if (b.bytes < bytes) {
        if (b.p) {
            check(hipStreamSynchronize(stream()), "yt: workspace");
            check(hipFree(b.p), "yt: hipFree (workspace)");
            b.p = nullptr;
            b.bytes = 0;
        }
        const size_t step = size_t(1) << 20, sz = (bytes + step - 1) / step * step;
        check(hipMalloc(&b.p, sz), "yt: hipMalloc (workspace)");
        b.bytes = sz;
    }
    return b.p;
}

// Frees the calling thread's workspace for the current device and stream
// (for a stream about to be destroyed).
inline void releaseWorkspace() {
    int dev = 0;
    check(hipGetDevice(&dev), "yt: hipGetDevice");
    auto& m = thread_workspaces().bufs;
    auto it = m.find({dev, stream()});
    if (it == m.end()) return;
    if (it->second.p) {
        check(hipStreamSynchronize(stream()), "yt: workspace");
        check(hipFree(it->second.p), "yt: hipFree (workspace)");
    }
    m.erase(it);
}

template <class T> constexpr int dtype_code() {
    if constexpr (std::is_same_v<T, float>) return YTHIP_F32;
    else if constexpr (std::is_same_v<T, float16>) return YTHIP_F16;
    else if constexpr (std::is_same_v<T, bfloat16>) return YTHIP_BF16;
    else return -1;
}
template <class T> constexpr bool kernel_type = dtype_code<T>() >= 0;

}  // namespace hip

namespace detail {

// Device copy of one storage block, shared by every view of it.
struct Mirror {
    size_t bytes = 0;
    void* dev = nullptr;
    bool host_valid = true;  // the host copy holds the current values
    bool dev_valid = false;  // the device copy holds the current values
    Mirror() = default;
    Mirror(const Mirror&) = delete;
    Mirror& operator=(const Mirror&) = delete;
    ~Mirror() {
        if (dev) (void)hipFree(dev);
    }
};

inline void host_to_device(const char* host, Mirror& m) {
    if (m.dev == nullptr && m.bytes > 0) hip::check(hipMalloc(&m.dev, m.bytes), "yt: hipMalloc");
    if (!m.dev_valid && m.bytes > 0)
        hip::check(hipMemcpyAsync(m.dev, host, m.bytes, hipMemcpyHostToDevice, hip::stream()), "yt: upload");
    m.dev_valid = true;
}

inline void device_to_host(char* host, Mirror& m) {
    if (!m.host_valid && m.bytes > 0) {
        hip::check(hipMemcpyAsync(host, m.dev, m.bytes, hipMemcpyDeviceToHost, hip::stream()), "yt: download");
        hip::check(hipStreamSynchronize(hip::stream()), "yt: download");
    }
    m.host_valid = true;
}

inline std::vector<int> broadcast_shape(const std::vector<std::vector<int>>& shapes) {
    size_t n = 0;
    for (auto& s : shapes) n = std::max(n, s.size());
    std::vector<int> out(n, 1);
    for (auto& s : shapes)
        for (size_t i = 0; i < s.size(); ++i) {
            int& o = out[n - s.size() + i];
            if (s[i] == o || s[i] == 1) continue;
            if (o != 1) throw std::invalid_argument("yt: shapes do not broadcast");
            o = s[i];
        }
    return out;
}

// Strides of a tensor's leading dims seen through the broadcast shape `lead`
// (size-1 and missing dims get stride 0).
inline std::vector<int64_t> lead_strides(const std::vector<int>& shape, const std::vector<int>& stride, int nlead,
                                         const std::vector<int>& lead) {
    std::vector<int64_t> out(lead.size(), 0);
    const int own = nlead;
    for (int i = 0; i < own; ++i) {
        const int j = static_cast<int>(lead.size()) - own + i;
        out[j] = shape[i] == 1 ? 0 : stride[i];
    }
    return out;
}

constexpr int max3(int a, int b, int c) { return std::max(a, std::max(b, c)); }

}  // namespace detail

template <class T, int dim>
class YTensor {
    static_assert(dim >= 1, "YTensor needs at least one dimension");

public:
    using value_type = T;

    YTensor() = default;
    YTensor(const std::vector<int> shape) { _allocate(shape); }
    YTensor(std::initializer_list<int> list) : YTensor(std::vector<int>(list)) {}
    template <class... Args>
        requires(sizeof...(Args) == dim && (std::is_integral_v<Args> && ...))
    explicit YTensor(Args... args) : YTensor(std::vector<int>{static_cast<int>(args)...}) {}

    // ---- shape and layout (include/ytensor_base.hpp) ----
    int shape(int i) const { return _shape.at(_axis(i)); }
    std::vector<int> shape() const { return _shape; }
    int stride_(int i) const { return _stride.at(_axis(i)); }
    std::vector<int> stride_() const { return _stride; }
    size_t size() const {
        size_t n = 1;
        for (int s : _shape) n *= static_cast<size_t>(s);
        return _shape.empty() ? 0 : n;
    }
    size_t elementSize() const { return sizeof(T); }
    int offset() const { return _offset; }
    bool isContiguous() const {
        int64_t expect = 1;
        for (int i = dim - 1; i >= 0; --i) {
            if (_shape[i] != 1 && _stride[i] != expect) return false;
            expect *= _shape[i];
        }
        return true;
    }

    // ---- host access (downloads a stale host copy first) ----
    T* data() {
        _host_current();
        _mirror->dev_valid = false;  // the caller may write through the pointer
        return reinterpret_cast<T*>(_data.get()) + _offset;
    }
    const T* data() const {
        _host_current();
        return reinterpret_cast<const T*>(_data.get()) + _offset;
    }
    template <class... I>
        requires(sizeof...(I) == dim && (std::is_integral_v<I> && ...))
    T& at(I... idx) {
        return data()[_lin(std::vector<int>{static_cast<int>(idx)...})];
    }
    template <class... I>
        requires(sizeof...(I) == dim && (std::is_integral_v<I> && ...))
    const T& at(I... idx) const {
        return data()[_lin(std::vector<int>{static_cast<int>(idx)...})];
    }
    // Element `i` in row-major order of the shape (any strides).
    T& atData_(size_t i) { return data()[_lin(_unravel(i))]; }
    const T& atData_(size_t i) const { return data()[_lin(_unravel(i))]; }

    // ---- device mirror ----
    bool onDevice() const { return _mirror && _mirror->dev_valid; }
    YTensor& toDevice() {
        detail::host_to_device(_data.get(), *_mirror);
        return *this;
    }
    YTensor& toHost() {
        _host_current();
        return *this;
    }
    // Device pointer of element 0 (uploads a stale device copy). For writing,
    // deviceWrite() also marks the host copy stale.
    const T* deviceData() const {
        detail::host_to_device(_data.get(), *_mirror);
        return static_cast<const T*>(_mirror->dev) + _offset;
    }
    T* deviceWrite() {
        detail::host_to_device(_data.get(), *_mirror);
        _mirror->host_valid = false;
        return static_cast<T*>(_mirror->dev) + _offset;
    }
    // A fresh tensor whose values will be produced on the device: no upload.
    static YTensor deviceOutput(const std::vector<int>& shape) {
        YTensor t(shape);
        if (t._mirror->bytes > 0) hip::check(hipMalloc(&t._mirror->dev, t._mirror->bytes), "yt: hipMalloc");
        t._mirror->dev_valid = true;
        t._mirror->host_valid = false;
        return t;
    }

    // ---- views (share _data and the mirror) ----
    YTensor transpose(int a = -2, int b = -1) const {
        YTensor v = *this;
        std::swap(v._shape[_axis(a)], v._shape[_axis(b)]);
        std::swap(v._stride[_axis(a)], v._stride[_axis(b)]);
        return v;
    }
    YTensor permute(const std::vector<int>& order) const {
        if (static_cast<int>(order.size()) != dim) throw std::invalid_argument("yt::YTensor::permute: rank");
        YTensor v = *this;
        for (int i = 0; i < dim; ++i) {
            v._shape[i] = _shape[_axis(order[i])];
            v._stride[i] = _stride[_axis(order[i])];
        }
        return v;
    }
    template <class... A>
        requires(sizeof...(A) == dim && (std::is_integral_v<A> && ...))
    YTensor permute(A... a) const {
        return permute(std::vector<int>{static_cast<int>(a)...});
    }
    YTensor slice(int axis, int start, int end) const {
        const int ax = _axis(axis);
        if (start < 0) start += _shape[ax];
        if (end < 0) end += _shape[ax];
        if (start < 0 || end > _shape[ax] || start > end) throw std::invalid_argument("yt::YTensor::slice: range");
        YTensor v = *this;
        v._offset += start * _stride[ax];
        v._shape[ax] = end - start;
        return v;
    }
    // A size-1 dim inserted at `axis`.
    YTensor<T, dim + 1> unsqueeze(int axis) const {
        const int a = axis < 0 ? axis + dim + 1 : axis;
        if (a < 0 || a > dim) throw std::invalid_argument("yt::YTensor::unsqueeze: axis out of range");
        YTensor<T, dim + 1> v;
        v._data = _data;
        v._mirror = _mirror;
        v._offset = _offset;
        v._shape = _shape;
        v._stride = _stride;
        v._shape.insert(v._shape.begin() + a, 1);
        v._stride.insert(v._stride.begin() + a, a < dim ? _stride[a] * _shape[a] : 1);
        return v;
    }
    // Size-1 dims repeated `times[i]` times as a stride-0 view
    // (src/ytensor_base.inl:797-811).
    YTensor repeat(const std::vector<int>& times) const {
        if (static_cast<int>(times.size()) != dim) throw std::invalid_argument("repeat: times size must match ndim");
        YTensor v = *this;
        for (int i = 0; i < dim; ++i) {
            if (times[i] <= 1) continue;
            if (_shape[i] != 1) throw std::runtime_error("Can only repeat on dimensions of size 1.");
            v._shape[i] = times[i];
            v._stride[i] = 0;
        }
        return v;
    }
    template <class... A>
        requires(sizeof...(A) == dim && (std::is_integral_v<A> && ...))
    YTensor repeat(A... times) const {
        return repeat(std::vector<int>{static_cast<int>(times)...});
    }

    // View with a new shape (contiguous tensors; one -1 is inferred).
    template <int nd>
    YTensor<T, nd> view(const std::vector<int>& shape) const {
        if (!isContiguous()) throw std::invalid_argument("yt::YTensor::view: needs a contiguous tensor");
        std::vector<int> s = shape;
        int64_t known = 1, neg = -1;
        for (int i = 0; i < nd; ++i) {
            if (s[i] == -1) neg = i;
            else known *= s[i];
        }
        if (neg >= 0) s[neg] = known ? static_cast<int>(static_cast<int64_t>(size()) / known) : 0;
        int64_t n = 1;
        for (int x : s) n *= x;
        if (n != static_cast<int64_t>(size())) throw std::invalid_argument("yt::YTensor::view: size mismatch");
        YTensor<T, nd> v;
        v._data = _data;
        v._mirror = _mirror;
        v._offset = _offset;
        v._shape = s;
        v._stride.assign(nd, 1);
        for (int i = nd - 2; i >= 0; --i) v._stride[i] = v._stride[i + 1] * v._shape[i + 1];
        return v;
    }
    template <class... A>
        requires(sizeof...(A) >= 1 && (std::is_integral_v<A> && ...))
    YTensor<T, static_cast<int>(sizeof...(A))> view(A... a) const {
        return view<static_cast<int>(sizeof...(A))>(std::vector<int>{static_cast<int>(a)...});
    }
    template <class... A>
        requires(sizeof...(A) >= 1 && (std::is_integral_v<A> && ...))
    YTensor<T, static_cast<int>(sizeof...(A))> reshape(A... a) const {
        return contiguous().template view<static_cast<int>(sizeof...(A))>(std::vector<int>{static_cast<int>(a)...});
    }
    // A contiguous copy (this tensor itself when already contiguous).
    YTensor contiguous() const {
        if (isContiguous()) return *this;
        YTensor out(_shape);
        T* o = out.data();
        const size_t n = size();
        for (size_t i = 0; i < n; ++i) o[i] = atData_(i);
        return out;
    }
    YTensor clone() const {
        YTensor out(_shape);
        T* o = out.data();
        for (size_t i = 0; i < size(); ++i) o[i] = atData_(i);
        return out;
    }

    // ---- RNG (include/ytensor_core.hpp:44-58, src/ytensor_core.inl:728-732):
    // one std::normal_distribution<double>(0, 1) per call, drawn row-major from
    // the shared mt19937, each value cast to T.
    static void seed(unsigned int s = std::random_device{}()) {
        std::lock_guard<std::mutex> lock(infos::rngMutex);
        infos::gen.seed(s);
    }
    template <class... Args>
        requires((std::is_integral_v<Args> && ...))
    static YTensor<T, static_cast<int>(sizeof...(Args))> randn(Args... args) {
        std::normal_distribution<double> dist(0.0, 1.0);
        YTensor<T, static_cast<int>(sizeof...(Args))> op(std::vector<int>{static_cast<int>(args)...});
        T* p = op.data();
        const size_t n = op.size();
        std::lock_guard<std::mutex> lock(infos::rngMutex);
        for (size_t i = 0; i < n; ++i) p[i] = static_cast<T>(static_cast<float>(dist(infos::gen)));
        return op;
    }

    // ---- YTensor::matmul (src/ytensor_math.inl:284-316, 954-1051) ----
    template <int dim1>
    YTensor<T, detail::max3(dim, dim1, 2)> matmul(const YTensor<T, dim1>& other,
                                                  infos::MatmulBackend backend = infos::defaultMatmulBackend) const;

    // internals, shared by the other instantiations and the operators
    template <class, int> friend class YTensor;
    std::shared_ptr<char[]> _data;
    int _offset = 0;
    std::vector<int> _shape;
    std::vector<int> _stride;
    std::shared_ptr<detail::Mirror> _mirror;

    int _axis(int i) const {
        const int a = i < 0 ? i + dim : i;
        if (a < 0 || a >= dim) throw std::invalid_argument("yt::YTensor: axis out of range");
        return a;
    }

private:
    void _allocate(const std::vector<int>& shape) {
        if (static_cast<int>(shape.size()) != dim) throw std::invalid_argument("yt::YTensor: shape rank != dim");
        _shape = shape;
        _stride.assign(dim, 1);
        for (int i = dim - 2; i >= 0; --i) _stride[i] = _stride[i + 1] * _shape[i + 1];
        size_t n = 1;
        for (int s : shape) {
            if (s < 0) throw std::invalid_argument("yt::YTensor: negative dimension");
            n *= static_cast<size_t>(s);
        }
        _data = std::shared_ptr<char[]>(new char[std::max<size_t>(n * sizeof(T), 1)]());
        _mirror = std::make_shared<detail::Mirror>();
        _mirror->bytes = n * sizeof(T);
        _offset = 0;
    }
    void _host_current() const { detail::device_to_host(_data.get(), *_mirror); }
    std::vector<int> _unravel(size_t i) const {
        std::vector<int> idx(dim);
        for (int d = dim - 1; d >= 0; --d) {
            idx[d] = static_cast<int>(i % static_cast<size_t>(_shape[d]));
            i /= static_cast<size_t>(_shape[d]);
        }
        return idx;
    }
    int64_t _lin(const std::vector<int>& idx) const {
        int64_t o = 0;
        for (int d = 0; d < dim; ++d) o += static_cast<int64_t>(idx[d]) * _stride[d];
        return o;
    }
};

namespace detail {

// Every broadcast index of the leading dims except the last one, as element
// offsets into a tensor with the given leading strides.
inline void for_outer(const std::vector<int>& lead, const std::vector<std::vector<int64_t>>& strides,
                      const std::function<void(const std::vector<int64_t>&)>& fn) {
    const int n = static_cast<int>(lead.size()) - 1;
    std::vector<int> idx(std::max(n, 0), 0);
    while (true) {
        std::vector<int64_t> off(strides.size(), 0);
        for (size_t t = 0; t < strides.size(); ++t)
            for (int i = 0; i < n; ++i) off[t] += static_cast<int64_t>(idx[i]) * strides[t][i];
        fn(off);
        int i = n - 1;
        while (i >= 0 && ++idx[i] == lead[i]) idx[i--] = 0;
        if (i < 0) break;
    }
}

}  // namespace detail

template <class T, int dim>
template <int dim1>
YTensor<T, detail::max3(dim, dim1, 2)> YTensor<T, dim>::matmul(const YTensor<T, dim1>& other,
                                                               infos::MatmulBackend backend) const {
    static_assert(hip::kernel_type<T>, "matmul runs float, yt::float16 and yt::bfloat16 on the GPU");
    static_assert(dim >= 2 && dim1 >= 2, "matmul here takes operands of at least 2 dimensions");
    constexpr int R = detail::max3(dim, dim1, 2);
    (void)backend;  // every backend value runs the HIP kernels in this build
    const int M = shape(-2), K = shape(-1), N = other.shape(-1);
    if (other.shape(-2) != K) throw std::invalid_argument("yt::YTensor::matmul: inner dimensions differ");
    const std::vector<int> la(_shape.begin(), _shape.end() - 2), lb(other._shape.begin(), other._shape.end() - 2);
    const std::vector<int> lead = detail::broadcast_shape({la, lb});
    std::vector<int> oshape = lead;
    oshape.push_back(M);
    oshape.push_back(N);
    auto out = YTensor<T, R>::deviceOutput(oshape);
    if (out.size() == 0) return out;
    constexpr int code = hip::dtype_code<T>();
    const auto* A = reinterpret_cast<const char*>(deviceData());
    const auto* B = reinterpret_cast<const char*>(other.deviceData());
    auto* C = reinterpret_cast<char*>(out.deviceWrite());
    const int64_t rsa = stride_(-2), csa = stride_(-1), rsb = other.stride_(-2), csb = other.stride_(-1);
    // Batch-flatten (src/ytensor_math.inl:960-1017): a 2-D right operand and
    // rows of the left that fold into one uniform row stride are one launch.
    bool fold = std::all_of(lb.begin(), lb.end(), [](int s) { return s == 1; }) && la == lead;
    for (int i = 0; fold && i < dim - 2; ++i)
        fold = _shape[i] == 1 || static_cast<int64_t>(_stride[i]) == rsa * std::accumulate(
                                     _shape.begin() + i + 1, _shape.end() - 1, int64_t{1}, std::multiplies<>());
    if (fold) {
        int64_t rows = M;
        for (int s : lead) rows *= s;
        hip::check(ythip_gemm(code, code, 1, static_cast<int>(rows), N, K, A, 0, rsa, csa, B, 0, rsb, csb, C, 0, N, 1,
                              1.0f, 0.0f, hip::stream()),
                   "yt::YTensor::matmul");
        return out;
    }
    if (lead.empty()) {
        hip::check(ythip_gemm(code, code, 1, M, N, K, A, 0, rsa, csa, B, 0, rsb, csb, C, 0, N, 1, 1.0f, 0.0f,
                              hip::stream()),
                   "yt::YTensor::matmul");
        return out;
    }
    const auto sa = detail::lead_strides(_shape, _stride, dim - 2, lead);
    const auto sb = detail::lead_strides(other._shape, other._stride, dim1 - 2, lead);
    const auto sc = detail::lead_strides(out._shape, out._stride, R - 2, lead);
    const size_t es = sizeof(T);
    detail::for_outer(lead, {sa, sb, sc}, [&](const std::vector<int64_t>& off) {
        hip::check(ythip_gemm(code, code, lead.back(), M, N, K, A + off[0] * es, sa.back(), rsa, csa, B + off[1] * es,
                              sb.back(), rsb, csb, C + off[2] * es, sc.back(), N, 1, 1.0f, 0.0f, hip::stream()),
                   "yt::YTensor::matmul");
    });
    return out;
}

// The reference's L2 kernel API (yt::kernel::avx2: include/kernel/avx2/
// sgemm.hpp:51-68, hgemm.hpp:26-42, flash_attention.hpp:21-69) for DEVICE
// pointers: the same names, sizes and element strides, one matrix per call
// (plus the batched GQA form the qwen3 example drives), launched on `stream`
// (nullptr: the thread's yt::hip::stream()). Argument errors raise
// std::invalid_argument, a failing launch std::runtime_error, as the
// reference's L3/L4 callers do.
namespace kernel::hip {

inline hipStream_t pick(void* stream) { return stream ? static_cast<hipStream_t>(stream) : yt::hip::stream(); }

// yt::kernel::avx2::sgemm (sgemm.hpp:51-58): C = alpha*A.B + beta*C, element strides.
inline void sgemm(const float* A, const float* B, float* C, int m, int n, int k, float alpha, float beta,
                  int64_t rsa, int64_t csa, int64_t rsb, int64_t csb, int64_t rsc, int64_t csc,
                  void* stream = nullptr) {
    yt::hip::check(ythip_gemm(YTHIP_F32, YTHIP_F32, 1, m, n, k, A, 0, rsa, csa, B, 0, rsb, csb, C, 0, rsc, csc, alpha,
                              beta, pick(stream)),
                   "yt::kernel::hip::sgemm");
}

// yt::kernel::avx2::matmul (sgemm.hpp:60-68): alpha = 1, beta = 0.
inline void matmul(const float* A, const float* B, float* C, int m, int n, int k, int64_t rsa, int64_t csa,
                   int64_t rsb, int64_t csb, int64_t rsc, int64_t csc, void* stream = nullptr) {
    sgemm(A, B, C, m, n, k, 1.0f, 0.0f, rsa, csa, rsb, csb, rsc, csc, stream);
}

// yt::kernel::avx2::hgemm (hgemm.hpp:26-33) for the 16-bit members of the type
// set: A / B / C hold raw float16 (YTHIP_F16) or bfloat16 (YTHIP_BF16) bits;
// accumulation is fp32 as in the reference's fp32 fast path (hgemm.inl:165-216).
inline void hgemm(int dtype, const void* A, const void* B, void* C, int m, int n, int k, float alpha, float beta,
                  int64_t rsa, int64_t csa, int64_t rsb, int64_t csb, int64_t rsc, int64_t csc,
                  void* stream = nullptr) {
    yt::hip::check(ythip_gemm(dtype, dtype, 1, m, n, k, A, 0, rsa, csa, B, 0, rsb, csb, C, 0, rsc, csc, alpha, beta,
                              pick(stream)),
                   "yt::kernel::hip::hgemm");
}

// yt::kernel::avx2::flash_attention (flash_attention.hpp:21-44): one matrix with
// row / column element strides, an optional bool mask [q_len, mask_stride] and
// an additive bias. Column strides must be 1. q_len == 1 runs the decode path
// (flash_attention.inl:469-499) with one split per call (no workspace here).
inline void flash_attention(int dtype, const void* Q, const void* K, const void* V, void* O, int q_len, int kv_len,
                            int head_dim, int value_dim, float scale, int64_t rsq, int64_t csq, int64_t rsk,
                            int64_t csk, int64_t rsv, int64_t csv, int64_t rso, int64_t cso,
                            const bool* mask = nullptr, int64_t mask_stride = 0, const float* bias = nullptr,
                            int64_t rsbias = 0, int64_t csbias = 0, void* stream = nullptr) {
    if (csq != 1 || csk != 1 || csv != 1 || cso != 1)
        throw std::invalid_argument("yt::kernel::hip::flash_attention: column strides must be 1");
    const int64_t qs[4] = {0, 0, rsq, 1}, ks[4] = {0, 0, rsk, 1}, vs[4] = {0, 0, rsv, 1}, os[4] = {0, 0, rso, 1};
    yt::hip::check(ythip_attn_prefill(dtype, 1, 1, 1, q_len, kv_len, head_dim, value_dim, Q, qs, K, ks, V, vs, O, os,
                                      scale, mask ? YTHIP_MASK_BOOL : YTHIP_MASK_NONE,
                                      reinterpret_cast<const uint8_t*>(mask), mask_stride, bias, rsbias, csbias,
                                      pick(stream)),
                   "yt::kernel::hip::flash_attention");
}

// The batched GQA form the qwen3 example drives through
// scaledDotProductAttention(..., FLASH_AVX2) (example/qwen3/src/qwen3.cpp:250-264):
// Q [B,Hq,q_len,d], K/V [B,Hkv,kv_len,d] with 4 strides each; causal with the
// example's offset (kv_len - q_len).
inline void sdpa_gqa(int dtype, int B, int Hq, int Hkv, int q_len, int kv_len, int d, const void* Q,
                     const int64_t q_str[4], const void* K, const int64_t k_str[4], const void* V,
                     const int64_t v_str[4], void* O, const int64_t o_str[4], float scale, bool causal,
                     void* stream = nullptr) {
    yt::hip::check(ythip_attn_prefill(dtype, B, Hq, Hkv, q_len, kv_len, d, d, Q, q_str, K, k_str, V, v_str, O, o_str,
                                      scale, causal ? YTHIP_MASK_CAUSAL : YTHIP_MASK_NONE, nullptr, 0, nullptr, 0, 0,
                                      pick(stream)),
                   "yt::kernel::hip::sdpa_gqa");
}

}  // namespace kernel::hip

namespace function {

// include/function/ops.hpp:21-24 plus this build's back end.
enum struct sdpaBackend { MATH, FLASH_AVX2, FLASH_HIP };

// A predicate mask the kernels evaluate themselves: key j visible to query i
// iff j <= i + offset (the causal mask of example/qwen3/src/qwen3.cpp:46-55
// is offset = kv_len - q_len). Callable as the reference's MaskFunc.
struct CausalMask {
    int offset = 0;
    bool operator()(int i, int j) const { return j <= i + offset; }
};

template <class T, int dim0, int dim1>
YTensor<T, detail::max3(dim0, dim1, 2)> matmul(const YTensor<T, dim0>& a, const YTensor<T, dim1>& b) {
    return a.matmul(b);
}

// src/function/ops.inl:84-91: x . weight^T, weight [out_features, in_features].
template <class T, int dim>
YTensor<T, dim> linear(const YTensor<T, dim>& x, const YTensor<T, 2>& weight) {
    static_assert(dim >= 2, "linear here takes inputs of at least 2 dimensions");
    if (x.shape(-1) != weight.shape(1))
        throw std::invalid_argument("yt::function::linear: input feature size must match weight.shape(1)");
    return x.matmul(weight.transpose());
}

// src/function/ops.inl:93-104: the product rounded to T, then the bias added in T.
template <class T, int dim>
YTensor<T, dim> linear(const YTensor<T, dim>& x, const YTensor<T, 2>& weight, const YTensor<T, 1>& bias) {
    if (bias.shape(0) != weight.shape(0))
        throw std::invalid_argument("yt::function::linear: bias size must match weight.shape(0)");
    auto out = linear(x, weight);
    const int n = out.shape(-1);
    const int64_t rows = static_cast<int64_t>(out.size()) / std::max(n, 1);
    auto b = bias.contiguous();
    hip::check(ythip_add_bias(hip::dtype_code<T>(), static_cast<int>(rows), n, out.deviceWrite(), n, b.deviceData(),
                              hip::stream()),
               "yt::function::linear");
    return out;
}

namespace detail_norm {

// The reference's _normalizeAxes (src/ytensor_function.inl:60-82): negative
// axes wrap, duplicates and an empty list are errors; the order is kept.
template <int dim>
std::vector<int> normalize_axes(const std::vector<int>& axes) {
    if (axes.empty()) throw std::invalid_argument("yt::function: axes must not be empty");
    std::vector<int> out;
    std::vector<bool> used(dim, false);
    for (int axis : axes) {
        const int a = (axis % dim + dim) % dim;
        if (used[a]) throw std::invalid_argument("yt::function: duplicate axes are not allowed");
        used[a] = true;
        out.push_back(a);
    }
    return out;
}

// Size and element stride of the dims `ax` (ascending) read as one axis, or
// false when their strides do not nest (size-1 dims are ignored).
inline bool fold_axes(const std::vector<int>& shape, const std::vector<int>& stride, const std::vector<int>& ax,
                      int64_t& n, int64_t& cs) {
    n = 1;
    cs = 1;
    int prev = -1;
    for (int i = static_cast<int>(ax.size()) - 1; i >= 0; --i) {
        const int a = ax[i];
        n *= shape[a];
        if (shape[a] == 1) continue;
        if (prev < 0) cs = stride[a];
        else if (static_cast<int64_t>(stride[a]) != static_cast<int64_t>(stride[prev]) * shape[prev]) return false;
        prev = a;
    }
    return true;
}

// y <- x / sqrt(mean(x^2 over axes) + eps) * weight on the device (y may be x).
// The weight's dims match x's along `axes` in the order given, its elements
// read row-major over the axes in ascending order (_makeAffineView,
// src/ytensor_function.inl:136-157). Normalised axes must be neighbouring dims
// whose strides nest (one strided axis for the kernel); the other dims are rows.
template <class T, int dim, int weightDim>
void rms_norm_into(const YTensor<T, dim>& x, const YTensor<T, weightDim>& weight, const std::vector<int>& axes,
                   float eps, YTensor<T, dim>& y, const std::string& name) {
    const auto ax = normalize_axes<dim>(axes);
    if (static_cast<int>(ax.size()) != weightDim)
        throw std::invalid_argument(name + ": gamma dim must match axes size");
    for (int i = 0; i < weightDim; ++i)
        if (weight.shape(i) != x.shape(ax[i])) throw std::invalid_argument(name + ": gamma shape must match affine axes");
    auto sorted = ax;
    std::sort(sorted.begin(), sorted.end());
    for (size_t i = 1; i < sorted.size(); ++i)
        if (sorted[i] != sorted[i - 1] + 1)
            throw std::invalid_argument(name + ": the normalised axes must be neighbouring dims on the GPU");
    int64_t n = 0, csx = 1, csy = 1, ny = 0;
    if (!fold_axes(x._shape, x._stride, sorted, n, csx) || !fold_axes(y._shape, y._stride, sorted, ny, csy))
        throw std::invalid_argument(name + ": the normalised axes' strides must nest on the GPU");
    if (x.size() == 0) return;
    // the other dims are rows: all but the last looped, the last one launched
    std::vector<int> lead;
    std::vector<int64_t> sx, sy;
    for (int d = 0; d < dim; ++d) {
        if (std::binary_search(sorted.begin(), sorted.end(), d)) continue;
        lead.push_back(x._shape[d]);
        sx.push_back(x._stride[d]);
        sy.push_back(y._stride[d]);
    }
    if (lead.empty()) {
        lead = {1};
        sx = {0};
        sy = {0};
    }
    auto w = weight.contiguous();
    const float* wp = reinterpret_cast<const float*>(w.deviceData());
    const auto* xb = reinterpret_cast<const char*>(x.deviceData());
    auto* yb = reinterpret_cast<char*>(y.deviceWrite());
    const int rows = lead.back();
    const int64_t es = static_cast<int64_t>(sizeof(T));
    detail::for_outer(lead, {sx, sy}, [&](const std::vector<int64_t>& off) {
        const void* xp = xb + off[0] * es;
        void* yp = yb + off[1] * es;
        const int64_t ldx = rows == 1 ? n : sx.back(), ldy = rows == 1 ? n : sy.back();
        int st;
        if (csx == 1 && csy == 1 && ldx >= n && ldy >= n)
            st = ythip_rms_norm(YTHIP_F32, YTHIP_F32, rows, static_cast<int>(n), xp, ldx, wp, eps, yp, ldy,
                                hip::stream());
        else
            st = ythip_rms_norm_strided(YTHIP_F32, YTHIP_F32, rows, static_cast<int>(n), xp, sx.back(), csx, wp, eps,
                                        yp, sy.back(), csy, hip::stream());
        hip::check(st, name);
    });
}

}  // namespace detail_norm

// yt::function::rmsNorm_ (include/function/normalization.hpp:76-89,
// src/function/normalization.inl:256-277): x <- x / sqrt(mean(x^2) + eps) *
// weight over `axes`, in place, on the device.
template <class T, int dim, int weightDim>
YTensor<T, dim>& rmsNorm_(YTensor<T, dim>& x, const YTensor<T, weightDim>& weight, const std::vector<int>& axes,
                          T eps = static_cast<T>(1e-5)) {
    static_assert(std::is_floating_point_v<T>, "T must be floating point type in yt::function::rmsNorm_()");
    static_assert(std::is_same_v<T, float>, "yt::function::rmsNorm_ runs float on the GPU (no double kernel)");
    detail_norm::rms_norm_into(x, weight, axes, static_cast<float>(eps), x, "yt::function::rmsNorm_");
    return x;
}

template <class T, int dim, int weightDim>
YTensor<T, dim>& rmsNorm_(YTensor<T, dim>& x, const YTensor<T, weightDim>& weight, int axis = -1,
                          T eps = static_cast<T>(1e-5)) {
    return rmsNorm_(x, weight, std::vector<int>{axis}, eps);
}

// yt::function::rmsNorm (include/function/normalization.hpp:59-73,
// src/function/normalization.inl:233-254): the same into a new tensor.
template <class T, int dim, int weightDim>
YTensor<T, dim> rmsNorm(const YTensor<T, dim>& x, const YTensor<T, weightDim>& weight, const std::vector<int>& axes,
                        T eps = static_cast<T>(1e-5)) {
    static_assert(std::is_floating_point_v<T>, "T must be floating point type in yt::function::rmsNorm_()");
    static_assert(std::is_same_v<T, float>, "yt::function::rmsNorm runs float on the GPU (no double kernel)");
    auto out = YTensor<T, dim>::deviceOutput(x.shape());
    detail_norm::rms_norm_into(x, weight, axes, static_cast<float>(eps), out, "yt::function::rmsNorm_");
    return out;
}

template <class T, int dim, int weightDim>
YTensor<T, dim> rmsNorm(const YTensor<T, dim>& x, const YTensor<T, weightDim>& weight, int axis = -1,
                        T eps = static_cast<T>(1e-5)) {
    return rmsNorm(x, weight, std::vector<int>{axis}, eps);
}

namespace detail_sdpa {

// The leading dims of q / k / v / o folded into the C ABI's (batch, head)
// form: the last lead dim is the head dim; when K and V repeat along it with
// stride 0 (repeat_kv, example/qwen3/src/qwen3.cpp:583-589) the heads are a GQA
// group, and the dim before it folds in as the KV head when Q's strides allow.
// The dims left over are looped, the last of them as the kernel's batch.
struct Fold {
    int heads_q = 1, heads_kv = 1, batch = 1;
    int64_t hq = 0, hk = 0, hv = 0, ho = 0;  // head strides
    int64_t bq = 0, bk = 0, bv = 0, bo = 0;  // batch strides
    std::vector<int> loop;                   // remaining dims (looped)
    std::vector<std::vector<int64_t>> loop_strides;  // q, k, v, o strides of the looped dims
};

inline Fold fold(const std::vector<int>& lead, const std::vector<int64_t>& sq, const std::vector<int64_t>& sk,
                 const std::vector<int64_t>& sv, const std::vector<int64_t>& so) {
    Fold f;
    int n = static_cast<int>(lead.size());
    if (n == 0) return f;
    const int l = lead[n - 1];
    if (l > 1 && sk[n - 1] == 0 && sv[n - 1] == 0 && sq[n - 1] != 0) {
        f.heads_q = l;
        f.hq = sq[n - 1];
        f.ho = so[n - 1];
        --n;
        if (n >= 1 && sq[n - 1] == l * sq[n] && so[n - 1] == l * so[n]) {
            f.heads_q *= lead[n - 1];
            f.heads_kv = lead[n - 1];
            f.hk = sk[n - 1];
            f.hv = sv[n - 1];
            --n;
        }
    } else {
        f.heads_q = f.heads_kv = l;
        f.hq = sq[n - 1];
        f.hk = sk[n - 1];
        f.hv = sv[n - 1];
        f.ho = so[n - 1];
        --n;
    }
    if (n >= 1) {
        f.batch = lead[n - 1];
        f.bq = sq[n - 1];
        f.bk = sk[n - 1];
        f.bv = sv[n - 1];
        f.bo = so[n - 1];
        --n;
    }
    f.loop.assign(lead.begin(), lead.begin() + n);
    f.loop_strides = {std::vector<int64_t>(sq.begin(), sq.begin() + n), std::vector<int64_t>(sk.begin(), sk.begin() + n),
                      std::vector<int64_t>(sv.begin(), sv.begin() + n), std::vector<int64_t>(so.begin(), so.begin() + n)};
    return f;
}

}  // namespace detail_sdpa

// The body of every scaledDotProductAttention overload: mask_kind / mask bytes
// / bias already resolved (src/function/ops.inl:368-425, 449-503).
template <class T, int dim>
YTensor<T, dim> _sdpa_hip(YTensor<T, dim>& query, YTensor<T, dim>& key, YTensor<T, dim>& value, T scale,
                          int mask_kind, const YTensor<bool, 2>* mask, int64_t diag_offset,
                          const YTensor<T, 2>* bias, sdpaBackend backend) {
    static_assert(hip::kernel_type<T>, "attention runs float, yt::float16 and yt::bfloat16 on the GPU");
    static_assert(dim >= 2, "attention tensors are [..., L, D]");
    float sc = static_cast<float>(scale);
    if (sc == 0.0f) sc = 1.0f / std::sqrt(static_cast<float>(query.shape(-1)));  // ops.inl:378-381
    if (query.shape(-1) != key.shape(-1)) throw std::invalid_argument("Query and key head dim must match.");
    if (key.shape(-2) != value.shape(-2)) throw std::invalid_argument("Key/value sequence length must match.");
    const int Lq = query.shape(-2), Lkv = key.shape(-2), D = query.shape(-1), Dv = value.shape(-1);
    if (mask != nullptr && (mask->shape(0) != Lq || mask->shape(1) != Lkv))
        throw std::invalid_argument("Mask shape must match the last two dimensions of the score tensor.");
    if (bias != nullptr && (bias->shape(0) != Lq || bias->shape(1) != Lkv))
        throw std::invalid_argument("Bias shape must match the last two dimensions of the score tensor.");
    const std::vector<int> lq(query._shape.begin(), query._shape.end() - 2);
    const std::vector<int> lk(key._shape.begin(), key._shape.end() - 2);
    const std::vector<int> lv(value._shape.begin(), value._shape.end() - 2);
    const std::vector<int> lead = detail::broadcast_shape({lq, lk, lv});
    std::vector<int> oshape = lead;
    oshape.push_back(Lq);
    oshape.push_back(Dv);
    auto out = YTensor<T, dim>::deviceOutput(oshape);
    if (out.size() == 0) return out;
    const int nl = dim - 2;
    const auto sq = detail::lead_strides(query._shape, query._stride, nl, lead);
    const auto sk = detail::lead_strides(key._shape, key._stride, nl, lead);
    const auto sv = detail::lead_strides(value._shape, value._stride, nl, lead);
    const auto so = detail::lead_strides(out._shape, out._stride, nl, lead);
    const auto f = detail_sdpa::fold(lead, sq, sk, sv, so);
    const char* Q = reinterpret_cast<const char*>(query.deviceData());
    const char* K = reinterpret_cast<const char*>(key.deviceData());
    const char* V = reinterpret_cast<const char*>(value.deviceData());
    char* O = reinterpret_cast<char*>(out.deviceWrite());
    const uint8_t* mp = nullptr;
    int64_t mask_ld = diag_offset;
    YTensor<bool, 2> mc;
    if (mask_kind == YTHIP_MASK_BOOL) {
        mc = mask->stride_(1) == 1 ? *mask : mask->contiguous();
        mp = reinterpret_cast<const uint8_t*>(mc.deviceData());
        mask_ld = mc.stride_(0);
    }
    YTensor<float, 2> bf;
    const float* bp = nullptr;
    int64_t brs = 0, bcs = 0;
    if (bias != nullptr) {
        if constexpr (std::is_same_v<T, float>) {
            bf = *bias;
        } else {
            bf = YTensor<float, 2>(std::vector<int>{Lq, Lkv});
            float* d = bf.data();
            for (int i = 0; i < Lq; ++i)
                for (int j = 0; j < Lkv; ++j) d[static_cast<int64_t>(i) * Lkv + j] = static_cast<float>(bias->at(i, j));
        }
        bp = bf.deviceData();
        brs = bf.stride_(0);
        bcs = bf.stride_(1);
    }
    constexpr int code = hip::dtype_code<T>();
    const size_t es = sizeof(T);
    const int64_t qs2 = query.stride_(-2), ks2 = key.stride_(-2), vs2 = value.stride_(-2), os2 = out.stride_(-2);
    const int64_t qs3 = query.stride_(-1), ks3 = key.stride_(-1), vs3 = value.stride_(-1);
    std::vector<int> loop = f.loop;
    std::vector<std::vector<int64_t>> ls = f.loop_strides;
    loop.push_back(1);  // for_outer loops over all but the last dim
    for (auto& s : ls) s.push_back(0);
    detail::for_outer(loop, ls, [&](const std::vector<int64_t>& off) {
        const void* q = Q + off[0] * es;
        const void* k = K + off[1] * es;
        const void* v = V + off[2] * es;
        void* o = O + off[3] * es;
        const int64_t qstr[4] = {f.bq, f.hq, qs2, qs3}, kstr[4] = {f.bk, f.hk, ks2, ks3},
                      vstr[4] = {f.bv, f.hv, vs2, vs3}, ostr[4] = {f.bo, f.ho, os2, 1};
        if (backend == sdpaBackend::MATH) {
            const size_t need = ythip_attn_math_workspace_size(code, f.batch, f.heads_q, Lq, Lkv);
            hip::check(ythip_attn_math(code, f.batch, f.heads_q, f.heads_kv, Lq, Lkv, D, Dv, q, qstr, k, kstr, v,
                                       vstr, o, ostr, sc, mask_kind, mp, mask_ld, bp, brs, bcs, hip::workspace(need),
                                       need, hip::stream()),
                       "yt::function::scaledDotProductAttention(MATH)");
            return;
        }
        // One query row runs the split-K decode kernel for every mask kind and
        // bias (flash_attention's q_len == 1 branch, src/kernel/avx2/
        // flash_attention.inl:469-499), its partials in this thread's workspace
        // for the stream; a bool mask's tile classes use the same workspace.
        const size_t need = ythip_attn_sdpa_workspace_size(f.batch, f.heads_q, Lq, Lkv, D);
        hip::check(ythip_attn_prefill_ws(code, f.batch, f.heads_q, f.heads_kv, Lq, Lkv, D, Dv, q, qstr, k, kstr, v,
                                         vstr, o, ostr, sc, mask_kind, mp, mask_ld, bp, brs, bcs,
                                         hip::workspace(need), need, hip::stream()),
                   "yt::function::scaledDotProductAttention");
    });
    return out;
}

// include/function/ops.hpp:26-45 (default backend MATH, as in the reference).
template <class T, int dim>
YTensor<T, dim> scaledDotProductAttention(YTensor<T, dim>& query, YTensor<T, dim>& key, YTensor<T, dim>& value,
                                          T scale = static_cast<T>(0.0), YTensor<bool, 2>* mask = nullptr,
                                          YTensor<T, 2>* bias = nullptr, sdpaBackend backend = sdpaBackend::MATH) {
    return _sdpa_hip(query, key, value, scale, mask ? YTHIP_MASK_BOOL : YTHIP_MASK_NONE, mask, 0, bias, backend);
}

template <class T, int dim>
YTensor<T, dim> scaledDotProductAttention(YTensor<T, dim>& query, YTensor<T, dim>& key, YTensor<T, dim>& value,
                                          T scale, YTensor<bool, 2>* mask, std::nullptr_t,
                                          sdpaBackend backend = sdpaBackend::MATH) {
    return _sdpa_hip(query, key, value, scale, mask ? YTHIP_MASK_BOOL : YTHIP_MASK_NONE, mask, 0,
                     static_cast<YTensor<T, 2>*>(nullptr), backend);
}

// include/function/ops.hpp:47-70: a predicate mask(i, j) -> bool. CausalMask
// runs inside the kernels; any other predicate is evaluated into a bool mask
// per element, as the reference calls it (src/kernel/avx2/flash_attention.inl:14-49).
template <class T, int dim, class MaskFunc>
    requires(!std::is_pointer_v<std::decay_t<MaskFunc>> && std::is_invocable_r_v<bool, MaskFunc, int, int>)
YTensor<T, dim> scaledDotProductAttention(YTensor<T, dim>& query, YTensor<T, dim>& key, YTensor<T, dim>& value,
                                          T scale, MaskFunc&& mask, YTensor<T, 2>* bias = nullptr,
                                          sdpaBackend backend = sdpaBackend::MATH) {
    if constexpr (std::is_same_v<std::decay_t<MaskFunc>, CausalMask>) {
        return _sdpa_hip(query, key, value, scale, YTHIP_MASK_DIAG, static_cast<YTensor<bool, 2>*>(nullptr),
                         mask.offset, bias, backend);
    } else {
        const int Lq = query.shape(-2), Lkv = key.shape(-2);
        YTensor<bool, 2> m(std::vector<int>{Lq, Lkv});
        bool* p = m.data();
        for (int i = 0; i < Lq; ++i)
            for (int j = 0; j < Lkv; ++j) p[static_cast<int64_t>(i) * Lkv + j] = mask(i, j);
        return _sdpa_hip(query, key, value, scale, YTHIP_MASK_BOOL, &m, 0, bias, backend);
    }
}

template <class T, int dim, class MaskFunc>
    requires(!std::is_pointer_v<std::decay_t<MaskFunc>> && std::is_invocable_r_v<bool, MaskFunc, int, int>)
YTensor<T, dim> scaledDotProductAttention(YTensor<T, dim>& query, YTensor<T, dim>& key, YTensor<T, dim>& value,
                                          T scale, MaskFunc&& mask, std::nullptr_t,
                                          sdpaBackend backend = sdpaBackend::MATH) {
    return scaledDotProductAttention(query, key, value, scale, std::forward<MaskFunc>(mask),
                                     static_cast<YTensor<T, 2>*>(nullptr), backend);
}

}  // namespace function
}  // namespace yt
