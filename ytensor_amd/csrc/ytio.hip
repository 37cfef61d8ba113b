// ytio.hip — YTensor's .yt checkpoint files read straight into device memory
// and written from it (the checkpoint loader of the Qwen3 example,
// example/qwen3/src/qwen3.cpp:304-363, without its host fp32 up-conversion).
//
// Reference: yt::io::YTensorIO (include/ytensor_io.hpp:81-180,
// src/ytensor_io.inl, src/ytensor_io_templates.inl). On-disk layout, all
// integers little-endian (readHeader/readIndex src/ytensor_io.inl:458-559,
// close() 313-417, writeIndex 561-578):
//   "YTENSORF" | u8 version | str metadata
//   record*:   str name | str typeName | i32 typeSize | str tensorType |
//              u64 byte count + i32 dims[] | str compressMethod |
//              u64 compressedSize | payload (raw row-major bytes, or a zlib stream)
//   index:     u64 record offset[count] | u32 count        (the file's last bytes)
// with str = u32 length + bytes.
//
// MI355X design: the transfer is bound by the host side (page cache / disk
// reads and PCIe), so the device does nothing but receive DMA. Each file handle
// owns two pinned staging buffers; chunk c is read (and inflated or converted)
// on the host into buffer c % 2 while the copy engine moves chunk c - 1, and
// an event per buffer keeps a buffer from being refilled before its copy has
// left. A tensor stored in the requested device type (bf16 checkpoints into
// bf16 weights) is never touched by the CPU beyond the read. Type changes
// happen on the host into the pinned buffer, so an fp32 checkpoint crosses PCIe
// already narrowed to bf16.

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>
#include <zlib.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <condition_variable>
#include <cstring>
#include <functional>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "launch.hpp"

namespace ythip {
namespace {

constexpr char kMagic[8] = {'Y', 'T', 'E', 'N', 'S', 'O', 'R', 'F'};  // include/ytensor_infos.hpp:119
constexpr uint8_t kVersion = 0;                                         // include/ytensor_infos.hpp:122
constexpr size_t kChunk = 64u << 20;                                    // staging buffer bytes
constexpr int kMaxDims = 64;

// ---------------------------------------------------------------- type rules
// Element conversions with the reference's casts, bit for bit:
//   float -> bfloat16: include/types/bfloat16.hpp:78-80 (adds bit 16 >> 1,
//     then truncates; the default RoundMode::nearestEven, ytensor_infos.hpp:91)
//   bfloat16 -> float: bfloat16.hpp:285-291 (shift left by 16)
//   float -> float16:  include/types/float_spec.hpp:435-491 (subnormal inputs
//     and underflow flush to signed zero, overflow to inf, NaN keeps mantissa 1,
//     otherwise round-to-nearest-even on the mantissa)
//   float16 -> float:  float_spec.hpp:299-370 (exact for normal numbers; NaN
//     mantissa becomes 1; subnormals come out doubled, as there)
//   double / int32 -> float: static_cast, as toFloat (qwen3.cpp:16-45).
inline uint32_t f2u(float x) { uint32_t u; std::memcpy(&u, &x, 4); return u; }
inline float u2f(uint32_t u) { float x; std::memcpy(&x, &u, 4); return x; }

inline uint16_t to_bf16(float x) {
    const uint32_t u = f2u(x);
    return static_cast<uint16_t>((u + ((u & 0x00010000u) >> 1)) >> 16);
}
inline float from_bf16(uint16_t h) { return u2f(static_cast<uint32_t>(h) << 16); }

inline uint16_t to_f16(float x) {
    const uint32_t bits = f2u(x);
    const uint32_t s = bits >> 31, e = (bits >> 23) & 0xFFu, m = bits & 0x7FFFFFu;
    uint32_t ne = 0, nm = 0;
    if (e == 0xFF) {
        ne = 31;
        nm = m != 0 ? 1u : 0u;
    } else if (e != 0) {
        const int biased = static_cast<int>(e) - 127 + 15;
        if (biased >= 31) {
            ne = 31;
        } else if (biased > 0) {
            ne = static_cast<uint32_t>(biased);
            nm = m >> 13;
            const uint32_t rest = m & 0x1FFFu;
            if (rest > 0x1000u || (rest == 0x1000u && (nm & 1u))) {
                if (++nm == 0x400u) {
                    nm = 0;
                    if (++ne == 31) nm = 0;
                }
            }
        }
    }
    return static_cast<uint16_t>((s << 15) | (ne << 10) | nm);
}

inline float from_f16(uint16_t h) {
    const uint32_t s = (h >> 15) & 1u, e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu, r;
    if (e == 31) {
        r = (s << 31) | (0xFFu << 23) | (m != 0 ? 1u : 0u);
    } else if (e != 0) {
        r = (s << 31) | ((e + 112u) << 23) | (m << 13);
    } else if (m == 0) {
        r = s << 31;
    } else {
        // subnormal: the reference normalises to bit 9 and then drops the next
        // bit, so its exponent is one above the value's (a subnormal reads
        // back doubled); reproduced as is
        int shift = 0;
        while (!(m & 0x200u) && shift < 10) { m <<= 1; ++shift; }
        m = (m << 1) & 0x3FFu;
        r = (s << 31) | (static_cast<uint32_t>(113 - shift) << 23) | (m << 13);
    }
    return u2f(r);
}

// File element types that convert to a device float type.
enum Src { SRC_F32, SRC_BF16, SRC_F16, SRC_F64, SRC_I32, SRC_OTHER };

Src src_kind(const std::string& t, int32_t size) {
    if (t == "float32" && size == 4) return SRC_F32;
    if (t == "bfloat16" && size == 2) return SRC_BF16;
    if (t == "float16" && size == 2) return SRC_F16;
    if (t == "float64" && size == 8) return SRC_F64;
    if (t == "int32" && size == 4) return SRC_I32;
    return SRC_OTHER;
}

int dst_size(int dtype) { return dtype == YTHIP_F32 ? 4 : 2; }

const char* dtype_name(int dtype) {
    return dtype == YTHIP_F32 ? "float32" : dtype == YTHIP_BF16 ? "bfloat16" : "float16";
}

bool same_type(Src s, int dtype) {
    return (s == SRC_F32 && dtype == YTHIP_F32) || (s == SRC_BF16 && dtype == YTHIP_BF16) ||
           (s == SRC_F16 && dtype == YTHIP_F16);
}

float read_elem(Src s, const unsigned char* p) {
    switch (s) {
        case SRC_F32: { float v; std::memcpy(&v, p, 4); return v; }
        case SRC_BF16: { uint16_t h; std::memcpy(&h, p, 2); return from_bf16(h); }
        case SRC_F16: { uint16_t h; std::memcpy(&h, p, 2); return from_f16(h); }
        case SRC_F64: { double v; std::memcpy(&v, p, 8); return static_cast<float>(v); }
        case SRC_I32: { int32_t v; std::memcpy(&v, p, 4); return static_cast<float>(v); }
        default: return 0.0f;
    }
}

// n elements of type s at src -> device type dtype at dst.
void convert(Src s, int dtype, const unsigned char* src, unsigned char* dst, size_t n) {
    const int ss = s == SRC_F64 ? 8 : (s == SRC_BF16 || s == SRC_F16) ? 2 : 4;
    if (dtype == YTHIP_F32) {
        float* d = reinterpret_cast<float*>(dst);
        for (size_t i = 0; i < n; ++i) d[i] = read_elem(s, src + i * ss);
    } else if (dtype == YTHIP_BF16) {
        uint16_t* d = reinterpret_cast<uint16_t*>(dst);
        if (s == SRC_F32) {
            const float* f = reinterpret_cast<const float*>(src);
            for (size_t i = 0; i < n; ++i) d[i] = to_bf16(f[i]);
        } else {
            for (size_t i = 0; i < n; ++i) d[i] = to_bf16(read_elem(s, src + i * ss));
        }
    } else {
        uint16_t* d = reinterpret_cast<uint16_t*>(dst);
        for (size_t i = 0; i < n; ++i) d[i] = to_f16(read_elem(s, src + i * ss));
    }
}

// A process-wide pool of host workers for the page-cache reads and the type
// conversions (created on first use, never torn down: its threads sleep on a
// condition variable and end with the process). run(n, fn) calls fn(i) exactly
// once for each i in [0, n), on the workers and the calling thread, and
// returns when every call has returned; concurrent callers take turns. Each
// run has its own index counter, so a worker that wakes late only finds that
// run's counter exhausted and never touches a later run.
class Pool {
   public:
    static Pool& get() {
        static Pool* p = new Pool(static_cast<int>(std::min(8u, std::max(1u, std::thread::hardware_concurrency()))));
        return *p;
    }
    int size() const { return nthreads_ + 1; }
    void run(int n, const std::function<void(int)>& fn) {
        std::lock_guard<std::mutex> serial(run_m_);
        auto job = std::make_shared<Job>();
        job->fn = &fn;
        job->n = n;
        job->pending.store(n);
        {
            std::lock_guard<std::mutex> lk(m_);
            job_ = job;
            ++gen_;
        }
        cv_.notify_all();
        work(*job);
        std::unique_lock<std::mutex> lk(m_);
        done_cv_.wait(lk, [&] { return job->pending.load() == 0; });
    }

   private:
    struct Job {
        const std::function<void(int)>* fn = nullptr;
        int n = 0;
        std::atomic<int> next{0}, pending{0};
    };
    explicit Pool(int n) : nthreads_(n) {
        for (int i = 0; i < n; ++i) std::thread([this] { loop(); }).detach();
    }
    void work(Job& j) {
        for (;;) {
            const int i = j.next.fetch_add(1);
            if (i >= j.n) break;
            (*j.fn)(i);
            if (j.pending.fetch_sub(1) == 1) {
                std::lock_guard<std::mutex> lk(m_);
                done_cv_.notify_all();
            }
        }
    }
    void loop() {
        uint64_t seen = 0;
        for (;;) {
            std::shared_ptr<Job> j;
            {
                std::unique_lock<std::mutex> lk(m_);
                cv_.wait(lk, [&] { return gen_ != seen; });
                seen = gen_;
                j = job_;
            }
            work(*j);
        }
    }
    const int nthreads_;
    std::mutex run_m_, m_;
    std::condition_variable cv_, done_cv_;
    uint64_t gen_ = 0;
    std::shared_ptr<Job> job_;
};

// Conversion of a large chunk split over the pool.
void convert_parallel(Src s, int dtype, const unsigned char* src, unsigned char* dst, size_t n) {
    const int ss = s == SRC_F64 ? 8 : (s == SRC_BF16 || s == SRC_F16) ? 2 : 4;
    const int ds = dst_size(dtype);
    const size_t per = 1u << 19;
    const int parts = static_cast<int>(std::min<size_t>(Pool::get().size(), (n + per - 1) / per));
    if (parts <= 1) return convert(s, dtype, src, dst, n);
    const size_t step = (n + parts - 1) / parts;
    Pool::get().run(parts, [&](int t) {
        const size_t b = t * step, e = std::min(n, b + step);
        if (b < e) convert(s, dtype, src + b * ss, dst + b * ds, e - b);
    });
}

// ---------------------------------------------------------------- file I/O
bool pread_all(int fd, void* buf, size_t n, uint64_t off) {
    unsigned char* p = static_cast<unsigned char*>(buf);
    while (n) {
        const ssize_t r = ::pread(fd, p, n, static_cast<off_t>(off));
        if (r <= 0) return false;
        p += r;
        n -= static_cast<size_t>(r);
        off += static_cast<uint64_t>(r);
    }
    return true;
}

// Large reads split over the pool (page-cache copies are per-core bound).
bool pread_parallel(int fd, void* buf, size_t n, uint64_t off) {
    const size_t per = 2u << 20;
    const int parts = static_cast<int>(std::min<size_t>(Pool::get().size(), (n + per - 1) / per));
    if (parts <= 1) return pread_all(fd, buf, n, off);
    const size_t step = ((n + parts - 1) / parts + 4095) & ~size_t(4095);
    std::atomic<int> bad{0};
    Pool::get().run(parts, [&](int t) {
        const size_t b = t * step;
        if (b >= n) return;
        if (!pread_all(fd, static_cast<unsigned char*>(buf) + b, std::min(n - b, step), off + b)) bad.store(1);
    });
    return bad.load() == 0;
}

bool write_all(int fd, const void* buf, size_t n) {
    const unsigned char* p = static_cast<const unsigned char*>(buf);
    while (n) {
        const ssize_t r = ::write(fd, p, n);
        if (r <= 0) return false;
        p += r;
        n -= static_cast<size_t>(r);
    }
    return true;
}

// Sequential little-endian reader over a byte range of the file.
struct Reader {
    int fd;
    uint64_t pos, end;
    bool ok = true;
    bool bytes(void* dst, size_t n) {
        if (!ok || n > end - pos) return ok = false;
        if (n && !pread_all(fd, dst, n, pos)) return ok = false;
        pos += n;
        return true;
    }
    uint32_t u32() { uint32_t v = 0; bytes(&v, 4); return v; }
    uint64_t u64() { uint64_t v = 0; bytes(&v, 8); return v; }
    std::string str() {
        const uint32_t n = u32();
        if (!ok || n > end - pos || n > (1u << 24)) { ok = false; return {}; }
        std::string s(n, '\0');
        bytes(s.data(), n);
        return s;
    }
};

struct Entry {
    std::string name, dtype, ttype, compress;
    int32_t type_size = 0;
    std::vector<int32_t> shape;
    uint64_t record_offset = 0, data_offset = 0, compressed_size = 0, nbytes = 0;
};

}  // namespace
}  // namespace ythip

// The opaque handle of include/ythip.h.
struct ythip_yt_file {
    int fd = -1;
    uint64_t size = 0;
    uint8_t version = 0;
    std::string metadata;
    std::vector<ythip::Entry> entries;
    std::vector<ythip_yt_tensor_info> infos;  // views into entries
    void* pinned[2] = {nullptr, nullptr};
    hipEvent_t ev[2] = {nullptr, nullptr};
    bool pending[2] = {false, false};
    int next_buf = 0;  // staging buffer for the next chunk (alternates across calls)
    std::vector<unsigned char> host;  // conversion source / compressed input
};

namespace ythip {
namespace {

int ensure_staging(ythip_yt_file* f) {
    if (f->pinned[0]) return 0;
    for (int b = 0; b < 2; ++b) {
        hipError_t e = hipHostMalloc(&f->pinned[b], kChunk, hipHostMallocDefault);
        if (e != hipSuccess) return status_of(e);
        e = hipEventCreateWithFlags(&f->ev[b], hipEventDisableTiming);
        if (e != hipSuccess) return status_of(e);
    }
    return 0;
}

// Waits until staging buffer b may be overwritten.
int acquire(ythip_yt_file* f, int b) {
    if (!f->pending[b]) return 0;
    f->pending[b] = false;
    return status_of(hipEventSynchronize(f->ev[b]));
}

int drain(ythip_yt_file* f) {
    int st = 0;
    for (int b = 0; b < 2; ++b)
        if (f->ev[b]) {
            const int s2 = acquire(f, b);
            if (!st) st = s2;
        }
    return st;
}

void release_staging(ythip_yt_file* f) {
    drain(f);
    for (int b = 0; b < 2; ++b) {
        if (f->ev[b]) (void)hipEventDestroy(f->ev[b]);
        if (f->pinned[b]) (void)hipHostFree(f->pinned[b]);
        f->ev[b] = nullptr;
        f->pinned[b] = nullptr;
    }
}

// Parses header and index: YTensorIO::readHeader + readIndex (src/ytensor_io.inl:458-559).
int parse(ythip_yt_file* f, const char* path) {
    Reader rd{f->fd, 0, f->size};
    char magic[8];
    if (!rd.bytes(magic, 8) || std::memcmp(magic, kMagic, 8) != 0)
        return fail(YTHIP_EFORMAT, "ythip_yt_open: %s is not a .yt file (bad magic)", path);
    rd.bytes(&f->version, 1);  // a newer version only warns in the reference (472-480)
    f->metadata = rd.str();
    if (!rd.ok) return fail(YTHIP_EFORMAT, "ythip_yt_open: %s: truncated header", path);
    if (f->size < rd.pos + 4) return fail(YTHIP_EFORMAT, "ythip_yt_open: %s: no index", path);
    uint32_t count = 0;
    pread_all(f->fd, &count, 4, f->size - 4);
    const uint64_t index_bytes = 4 + 8ull * count;
    if (index_bytes > f->size - rd.pos)
        return fail(YTHIP_EFORMAT, "ythip_yt_open: %s: index of %u tensors does not fit the file", path, count);
    std::vector<uint64_t> offsets(count);
    if (count && !pread_all(f->fd, offsets.data(), 8ull * count, f->size - index_bytes))
        return fail(YTHIP_EIO, "ythip_yt_open: %s: cannot read the index", path);
    const uint64_t data_end = f->size - index_bytes;
    f->entries.resize(count);
    for (uint32_t i = 0; i < count; ++i) {
        Entry& e = f->entries[i];
        Reader r{f->fd, offsets[i], data_end};
        if (offsets[i] >= data_end) r.ok = false;
        e.record_offset = offsets[i];
        e.name = r.str();
        e.dtype = r.str();
        r.bytes(&e.type_size, 4);
        e.ttype = r.str();
        const uint64_t shape_bytes = r.u64();
        if (!r.ok || shape_bytes % 4 || shape_bytes > 4ull * kMaxDims)
            return fail(YTHIP_EFORMAT, "ythip_yt_open: %s: tensor %u: bad shape record", path, i);
        e.shape.resize(shape_bytes / 4);
        r.bytes(e.shape.data(), shape_bytes);
        e.compress = r.str();
        e.compressed_size = r.u64();
        e.data_offset = r.pos;
        if (!r.ok || e.compressed_size > data_end - e.data_offset)
            return fail(YTHIP_EFORMAT, "ythip_yt_open: %s: tensor %u: truncated record", path, i);
        if (e.type_size <= 0)
            return fail(YTHIP_EFORMAT, "ythip_yt_open: %s: tensor '%s': type size %d", path, e.name.c_str(),
                        e.type_size);
        // uncompressedSize = typeSize * prod(shape) (src/ytensor_io.inl:551-554)
        unsigned __int128 nb = static_cast<uint32_t>(e.type_size);
        for (int32_t d : e.shape) {
            if (d < 0)
                return fail(YTHIP_EFORMAT, "ythip_yt_open: %s: tensor '%s': negative dimension", path,
                            e.name.c_str());
            nb *= static_cast<uint32_t>(d);
            if (nb >> 62) return fail(YTHIP_EFORMAT, "ythip_yt_open: %s: tensor '%s': size overflow", path,
                                      e.name.c_str());
        }
        e.nbytes = static_cast<uint64_t>(nb);
    }
    f->infos.resize(count);
    for (uint32_t i = 0; i < count; ++i) {
        const Entry& e = f->entries[i];
        ythip_yt_tensor_info& o = f->infos[i];
        o.name = e.name.c_str();
        o.dtype = e.dtype.c_str();
        o.tensor_type = e.ttype.c_str();
        o.compress = e.compress.c_str();
        o.type_size = e.type_size;
        o.ndim = static_cast<int32_t>(e.shape.size());
        o.shape = e.shape.data();
        o.data_offset = e.data_offset;
        o.compressed_size = e.compressed_size;
        o.nbytes = e.nbytes;
    }
    return 0;
}

// Streams `total` payload bytes of entry e through the staging buffers: the
// producer fills a host span with the next bytes (raw or inflated), the chunk
// is converted if needed and queued for the copy engine.
struct Sink {
    ythip_yt_file* f;
    Src src;
    int dtype;  // -1: raw bytes
    unsigned char* dst;
    hipStream_t stream;
    uint64_t done_elems = 0;
    int chunk_idx = 0;
    int src_size() const { return src == SRC_F64 ? 8 : (src == SRC_BF16 || src == SRC_F16) ? 2 : 4; }
};

// Hands `elems` source elements sitting in `buf` (pinned buffer b when no
// conversion, host memory otherwise) to the device.
int push_chunk(Sink& s, int b, const unsigned char* buf, size_t elems, size_t raw_bytes) {
    ythip_yt_file* f = s.f;
    size_t out_bytes;
    uint64_t dst_off;
    if (s.dtype < 0) {
        out_bytes = raw_bytes;
        dst_off = s.done_elems;  // counted in bytes for raw copies
    } else if (same_type(s.src, s.dtype)) {
        out_bytes = elems * dst_size(s.dtype);
        dst_off = s.done_elems * dst_size(s.dtype);
    } else {
        convert_parallel(s.src, s.dtype, buf, static_cast<unsigned char*>(f->pinned[b]), elems);
        out_bytes = elems * dst_size(s.dtype);
        dst_off = s.done_elems * dst_size(s.dtype);
    }
    hipError_t e = hipMemcpyAsync(s.dst + dst_off, f->pinned[b], out_bytes, hipMemcpyHostToDevice, s.stream);
    if (e != hipSuccess) return status_of(e);
    e = hipEventRecord(f->ev[b], s.stream);
    if (e != hipSuccess) return status_of(e);
    f->pending[b] = true;
    s.done_elems += s.dtype < 0 ? raw_bytes : elems;
    return 0;
}

int load_entry(ythip_yt_file* f, const Entry& e, void* dst, int dtype, hipStream_t stream) {
    Sink s{f, src_kind(e.dtype, e.type_size), dtype, static_cast<unsigned char*>(dst), stream};
    const bool direct = dtype < 0 || same_type(s.src, dtype);
    const size_t es = dtype < 0 ? 1 : static_cast<size_t>(e.type_size);
    // source elements per chunk: the converted output must fit one staging buffer
    const size_t out_es = dtype < 0 ? 1 : static_cast<size_t>(dst_size(dtype));
    const size_t per_chunk = kChunk / std::max(es, out_es);
    if (int st = ensure_staging(f)) return st;
    if (!direct && f->host.size() < per_chunk * es) f->host.resize(per_chunk * es);
    const bool zlib = e.compress == "zlib";  // other names read raw (checkCompressMethod, 11-22)
    if (!zlib) {
        if (e.compressed_size != e.nbytes)
            return fail(YTHIP_EFORMAT, "ythip_yt_load: tensor '%s': %llu payload bytes for %llu expected",
                        e.name.c_str(), (unsigned long long)e.compressed_size, (unsigned long long)e.nbytes);
        uint64_t off = 0;
        int& b = f->next_buf;
        while (off < e.nbytes) {
            const size_t bytes = static_cast<size_t>(std::min<uint64_t>(per_chunk * es, e.nbytes - off));
            if (int st = acquire(f, b)) return st;
            unsigned char* buf = direct ? static_cast<unsigned char*>(f->pinned[b]) : f->host.data();
            if (!pread_parallel(f->fd, buf, bytes, e.data_offset + off))
                return fail(YTHIP_EIO, "ythip_yt_load: tensor '%s': read failed", e.name.c_str());
            if (int st = push_chunk(s, b, buf, bytes / es, bytes)) return st;
            off += bytes;
            b ^= 1;
        }
        return 0;
    }
    // zlib stream (decompressData, src/ytensor_io.inl:147-250: inflateInit2(15 + 32))
    z_stream zs;
    std::memset(&zs, 0, sizeof(zs));
    if (inflateInit2(&zs, 15 + 32) != Z_OK) return fail(YTHIP_EIO, "ythip_yt_load: inflateInit2 failed");
    std::vector<unsigned char> in(1u << 20);
    uint64_t in_off = 0, produced = 0;
    int& b = f->next_buf;
    int zr = Z_OK, st = 0;
    while (produced < e.nbytes && st == 0) {
        if ((st = acquire(f, b))) break;
        unsigned char* buf = direct ? static_cast<unsigned char*>(f->pinned[b]) : f->host.data();
        const size_t want = static_cast<size_t>(std::min<uint64_t>(per_chunk * es, e.nbytes - produced));
        zs.next_out = buf;
        zs.avail_out = static_cast<uInt>(want);
        while (zs.avail_out > 0 && zr != Z_STREAM_END) {
            if (zs.avail_in == 0) {
                const size_t n = static_cast<size_t>(std::min<uint64_t>(in.size(), e.compressed_size - in_off));
                if (n == 0) break;
                if (!pread_all(f->fd, in.data(), n, e.data_offset + in_off)) { zr = Z_ERRNO; break; }
                in_off += n;
                zs.next_in = in.data();
                zs.avail_in = static_cast<uInt>(n);
            }
            zr = inflate(&zs, Z_NO_FLUSH);
            if (zr != Z_OK && zr != Z_STREAM_END) break;
        }
        const size_t got = want - zs.avail_out;
        if (zr != Z_OK && zr != Z_STREAM_END) {
            st = fail(YTHIP_EFORMAT, "ythip_yt_load: tensor '%s': corrupt zlib stream (%d)", e.name.c_str(), zr);
            break;
        }
        if (got != want) {
            st = fail(YTHIP_EFORMAT, "ythip_yt_load: tensor '%s': %llu bytes inflated, %llu expected", e.name.c_str(),
                      (unsigned long long)(produced + got), (unsigned long long)e.nbytes);
            break;
        }
        st = push_chunk(s, b, buf, got / es, got);
        produced += got;
        b ^= 1;
    }
    if (st == 0 && zr != Z_STREAM_END && e.nbytes > 0) {
        // all expected bytes arrived; the stream must end here (no trailing data)
        unsigned char extra;
        zs.next_out = &extra;
        zs.avail_out = 1;
        if (zs.avail_in == 0 && in_off < e.compressed_size) {
            const size_t n = static_cast<size_t>(std::min<uint64_t>(in.size(), e.compressed_size - in_off));
            if (pread_all(f->fd, in.data(), n, e.data_offset + in_off)) {
                in_off += n;
                zs.next_in = in.data();
                zs.avail_in = static_cast<uInt>(n);
            }
        }
        zr = inflate(&zs, Z_NO_FLUSH);
        if (zr != Z_STREAM_END || zs.avail_out == 0)
            st = fail(YTHIP_EFORMAT, "ythip_yt_load: tensor '%s': zlib stream longer than the tensor",
                      e.name.c_str());
    }
    inflateEnd(&zs);
    return st;
}

// ---------------------------------------------------------------- writer
void put_u32(std::vector<unsigned char>& o, uint32_t v) {
    const unsigned char* p = reinterpret_cast<const unsigned char*>(&v);
    o.insert(o.end(), p, p + 4);
}
void put_u64(std::vector<unsigned char>& o, uint64_t v) {
    const unsigned char* p = reinterpret_cast<const unsigned char*>(&v);
    o.insert(o.end(), p, p + 8);
}
void put_str(std::vector<unsigned char>& o, const std::string& s) {  // string2data (24-32)
    put_u32(o, static_cast<uint32_t>(s.size()));
    o.insert(o.end(), s.begin(), s.end());
}

// One staged tensor of a save: where its payload comes from.
struct Staged {
    Entry meta;
    const void* device = nullptr;     // dense device bytes, or
    const ythip_yt_file* src = nullptr;  // payload copied verbatim from an existing file (append)
};

int write_file(const char* path, const std::string& metadata, std::vector<Staged>& items, bool zlib_new,
               hipStream_t stream) {
    const std::string tmp = std::string(path) + ".ythip-tmp";
    const int fd = ::open(tmp.c_str(), O_WRONLY | O_CREAT | O_TRUNC, 0644);
    if (fd < 0) return fail(YTHIP_EIO, "ythip_yt_save: cannot create %s", tmp.c_str());
    auto bail = [&](int code) {
        ::close(fd);
        ::unlink(tmp.c_str());
        return code;
    };
    std::vector<unsigned char> hdr(kMagic, kMagic + 8);  // writeHeader (487-506)
    hdr.push_back(kVersion);
    put_str(hdr, metadata);
    if (!write_all(fd, hdr.data(), hdr.size()))
        return bail(fail(YTHIP_EIO, "ythip_yt_save: write failed"));
    uint64_t pos = hdr.size();
    std::vector<uint64_t> offsets;
    void* pinned = nullptr;  // device-to-host staging, allocated on the first device payload
    hipError_t he = hipSuccess;
    for (const Staged& it : items)
        if (it.device && it.meta.nbytes > 0) {
            he = hipHostMalloc(&pinned, kChunk, hipHostMallocDefault);
            if (he != hipSuccess) return bail(status_of(he));
            break;
        }
    std::vector<unsigned char> zout;
    int st = 0;
    for (Staged& it : items) {
        Entry& m = it.meta;
        offsets.push_back(pos);
        // payload first (its size goes in the record); kept in memory like the
        // reference's compressedData when compressed, streamed when not.
        std::vector<unsigned char> payload;
        const bool compress_this = it.device && zlib_new && m.nbytes > 0;
        if (it.src) {
            payload.resize(static_cast<size_t>(m.compressed_size));
            if (m.compressed_size && !pread_all(it.src->fd, payload.data(), payload.size(), m.data_offset)) {
                st = fail(YTHIP_EIO, "ythip_yt_save: cannot read tensor '%s' of the existing file", m.name.c_str());
                break;
            }
        } else if (compress_this) {
            // compressData (src/ytensor_io_templates.inl:17-46): level Z_DEFAULT_COMPRESSION,
            // window 15, memLevel 8, Z_FILTERED, one zlib stream per tensor
            z_stream zs;
            std::memset(&zs, 0, sizeof(zs));
            if (deflateInit2(&zs, Z_DEFAULT_COMPRESSION, Z_DEFLATED, 15, 8, Z_FILTERED) != Z_OK) {
                st = fail(YTHIP_EIO, "ythip_yt_save: deflateInit2 failed");
                break;
            }
            zout.resize(deflateBound(&zs, static_cast<uLong>(m.nbytes)));
            zs.next_out = zout.data();
            zs.avail_out = static_cast<uInt>(zout.size());
            uint64_t off = 0;
            int zr = Z_OK;
            while (off < m.nbytes && st == 0) {
                const size_t n = static_cast<size_t>(std::min<uint64_t>(kChunk, m.nbytes - off));
                he = hipMemcpyAsync(pinned, static_cast<const unsigned char*>(it.device) + off, n,
                                    hipMemcpyDeviceToHost, stream);
                if (he == hipSuccess) he = hipStreamSynchronize(stream);
                if (he != hipSuccess) { st = status_of(he); break; }
                zs.next_in = static_cast<unsigned char*>(pinned);
                zs.avail_in = static_cast<uInt>(n);
                off += n;
                zr = deflate(&zs, off == m.nbytes ? Z_FINISH : Z_NO_FLUSH);
                if (zr == Z_STREAM_ERROR || zs.avail_in != 0) {
                    st = fail(YTHIP_EIO, "ythip_yt_save: deflate failed for '%s'", m.name.c_str());
                }
            }
            if (st == 0 && zr != Z_STREAM_END) st = fail(YTHIP_EIO, "ythip_yt_save: deflate did not finish");
            payload.assign(zout.begin(), zout.begin() + zs.total_out);
            deflateEnd(&zs);
            if (st) break;
            m.compressed_size = payload.size();
            m.compress = "zlib";
        } else {
            m.compressed_size = m.nbytes;
            m.compress = zlib_new && it.device ? "zlib" : m.compress;
        }
        std::vector<unsigned char> rec;  // record header, close() (367-391)
        put_str(rec, m.name);
        put_str(rec, m.dtype);
        put_u32(rec, static_cast<uint32_t>(m.type_size));
        put_str(rec, m.ttype);
        put_u64(rec, 4ull * m.shape.size());  // array2data (templates 5-14)
        for (int32_t d : m.shape) put_u32(rec, static_cast<uint32_t>(d));
        put_str(rec, m.compress);
        put_u64(rec, m.compressed_size);
        if (!write_all(fd, rec.data(), rec.size())) { st = fail(YTHIP_EIO, "ythip_yt_save: write failed"); break; }
        pos += rec.size();
        if (it.src || compress_this) {
            if (!write_all(fd, payload.data(), payload.size())) {
                st = fail(YTHIP_EIO, "ythip_yt_save: write failed");
                break;
            }
            pos += payload.size();
            continue;
        }
        uint64_t off = 0;  // uncompressed device payload, streamed
        while (off < m.nbytes) {
            const size_t n = static_cast<size_t>(std::min<uint64_t>(kChunk, m.nbytes - off));
            he = hipMemcpyAsync(pinned, static_cast<const unsigned char*>(it.device) + off, n, hipMemcpyDeviceToHost,
                                stream);
            if (he == hipSuccess) he = hipStreamSynchronize(stream);
            if (he != hipSuccess) { st = status_of(he); break; }
            if (!write_all(fd, pinned, n)) { st = fail(YTHIP_EIO, "ythip_yt_save: write failed"); break; }
            off += n;
        }
        if (st) break;
        pos += m.nbytes;
    }
    if (pinned) (void)hipHostFree(pinned);
    if (st) return bail(st);
    std::vector<unsigned char> idx;  // writeIndex (561-578)
    for (uint64_t o : offsets) put_u64(idx, o);
    put_u32(idx, static_cast<uint32_t>(offsets.size()));
    if (!write_all(fd, idx.data(), idx.size()))
        return bail(fail(YTHIP_EIO, "ythip_yt_save: write failed"));
    ::close(fd);
    if (::rename(tmp.c_str(), path) != 0) {
        ::unlink(tmp.c_str());
        return fail(YTHIP_EIO, "ythip_yt_save: cannot replace %s", path);
    }
    return 0;
}

}  // namespace
}  // namespace ythip

using namespace ythip;

extern "C" {

__attribute__((visibility("default"))) int ythip_yt_open(const char* path, ythip_yt_file** out) {
    if (!path || !out) return fail(YTHIP_EINVAL, "ythip_yt_open: NULL argument");
    *out = nullptr;
    const int fd = ::open(path, O_RDONLY);
    if (fd < 0) return fail(YTHIP_EIO, "ythip_yt_open: cannot open %s", path);
    struct stat sb;
    if (fstat(fd, &sb) != 0) {
        ::close(fd);
        return fail(YTHIP_EIO, "ythip_yt_open: cannot stat %s", path);
    }
    auto* f = new ythip_yt_file;
    f->fd = fd;
    f->size = static_cast<uint64_t>(sb.st_size);
    if (int st = parse(f, path)) {
        ::close(fd);
        delete f;
        return st;
    }
    *out = f;
    return 0;
}

__attribute__((visibility("default"))) int ythip_yt_close(ythip_yt_file* f) {
    if (!f) return 0;
    release_staging(f);
    if (f->fd >= 0) ::close(f->fd);
    delete f;
    return 0;
}

__attribute__((visibility("default"))) int ythip_yt_count(const ythip_yt_file* f) {
    return f ? static_cast<int>(f->entries.size()) : 0;
}

__attribute__((visibility("default"))) const char* ythip_yt_metadata(const ythip_yt_file* f) {
    return f ? f->metadata.c_str() : "";
}

__attribute__((visibility("default"))) int ythip_yt_find(const ythip_yt_file* f, const char* name) {
    if (!f) return fail(YTHIP_EINVAL, "ythip_yt_find: NULL file");
    if (!name || !*name) {  // getTensorInfo("") is the first tensor (src/ytensor_io.inl:427-434)
        if (f->entries.empty()) return fail(YTHIP_ENOTFOUND, "ythip_yt_find: no tensors available");
        return 0;
    }
    for (size_t i = 0; i < f->entries.size(); ++i)
        if (f->entries[i].name == name) return static_cast<int>(i);
    return fail(YTHIP_ENOTFOUND, "ythip_yt_find: tensor not found: %s", name);
}

__attribute__((visibility("default"))) int ythip_yt_info(const ythip_yt_file* f, int index, ythip_yt_tensor_info* info) {
    if (!f || !info) return fail(YTHIP_EINVAL, "ythip_yt_info: NULL argument");
    if (index < 0 || index >= static_cast<int>(f->infos.size()))
        return fail(YTHIP_EINVAL, "ythip_yt_info: index %d of %zu", index, f->infos.size());
    *info = f->infos[static_cast<size_t>(index)];
    return 0;
}

namespace ythip {
namespace {

// Argument checks shared by the single and the batched load; returns the
// destination byte count in *need.
int check_load(const ythip_yt_file* f, int index, const void* dst, int dtype, uint64_t dst_bytes, uint64_t* need) {
    if (!f) return fail(YTHIP_EINVAL, "ythip_yt_load: NULL file");
    if (index < 0 || index >= static_cast<int>(f->entries.size()))
        return fail(YTHIP_EINVAL, "ythip_yt_load: index %d of %zu", index, f->entries.size());
    const Entry& e = f->entries[static_cast<size_t>(index)];
    if (e.ttype != "dense")
        return fail(YTHIP_EUNSUPPORTED, "ythip_yt_load: tensor '%s' is '%s'; only dense tensors go to the device",
                    e.name.c_str(), e.ttype.c_str());
    if (dtype != YTHIP_YT_RAW && dtype != YTHIP_F32 && dtype != YTHIP_F16 && dtype != YTHIP_BF16)
        return fail(YTHIP_EINVAL, "ythip_yt_load: dtype %d", dtype);
    const Src s = src_kind(e.dtype, e.type_size);
    if (dtype != YTHIP_YT_RAW && s == SRC_OTHER)
        return fail(YTHIP_EUNSUPPORTED, "ythip_yt_load: tensor '%s' of type %s cannot convert to %s", e.name.c_str(),
                    e.dtype.c_str(), dtype_name(dtype));
    *need = dtype == YTHIP_YT_RAW ? e.nbytes : e.nbytes / e.type_size * dst_size(dtype);
    if (dst_bytes < *need)
        return fail(YTHIP_EINVAL, "ythip_yt_load: tensor '%s' needs %llu bytes, destination has %llu", e.name.c_str(),
                    (unsigned long long)*need, (unsigned long long)dst_bytes);
    if (*need && !dst) return fail(YTHIP_EINVAL, "ythip_yt_load: NULL destination");
    return 0;
}

// A tensor whose stored bytes go to the device unchanged and whole.
bool is_verbatim(const Entry& e, int dtype) {
    return e.compress != "zlib" && e.compressed_size == e.nbytes && e.nbytes > 0 && e.nbytes <= kChunk &&
           (dtype == YTHIP_YT_RAW || same_type(src_kind(e.dtype, e.type_size), dtype));
}

}  // namespace
}  // namespace ythip

__attribute__((visibility("default"))) int ythip_yt_load(ythip_yt_file* f, int index, void* dst, int dtype,
                                                         uint64_t dst_bytes, void* stream) {
    uint64_t need = 0;
    if (int st = check_load(f, index, dst, dtype, dst_bytes, &need)) return st;
    if (need == 0) return 0;
    return load_entry(f, f->entries[static_cast<size_t>(index)], dst, dtype == YTHIP_YT_RAW ? -1 : dtype,
                      static_cast<hipStream_t>(stream));
}

__attribute__((visibility("default"))) int ythip_yt_load_many(ythip_yt_file* f, int n, const int* index,
                                                              void* const* dst, const int* dtype,
                                                              const uint64_t* dst_bytes, void* stream) {
    if (!f || n < 0 || (n > 0 && (!index || !dst || !dtype || !dst_bytes)))
        return fail(YTHIP_EINVAL, "ythip_yt_load_many: bad arguments");
    for (int i = 0; i < n; ++i) {  // everything is checked before anything is queued
        uint64_t need = 0;
        if (int st = check_load(f, index[i], dst[i], dtype[i], dst_bytes[i], &need)) return st;
    }
    const hipStream_t hs = static_cast<hipStream_t>(stream);
    // Verbatim tensors in file order are read in spans of up to one staging
    // buffer (one parallel read covers many neighbouring payloads and the
    // small record headers between them) and copied out of the buffer one
    // tensor at a time; the rest go through the per-tensor path.
    std::vector<int> order;
    for (int i = 0; i < n; ++i)
        if (f->entries[static_cast<size_t>(index[i])].nbytes > 0) order.push_back(i);
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) {
        return f->entries[static_cast<size_t>(index[a])].data_offset <
               f->entries[static_cast<size_t>(index[b])].data_offset;
    });
    if (int st = ensure_staging(f)) return st;
    size_t k = 0;
    while (k < order.size()) {
        const Entry& e0 = f->entries[static_cast<size_t>(index[order[k]])];
        if (!is_verbatim(e0, dtype[order[k]])) {
            const int i = order[k++];
            if (int st = load_entry(f, e0, dst[i], dtype[i] == YTHIP_YT_RAW ? -1 : dtype[i], hs)) return st;
            continue;
        }
        const uint64_t begin = e0.data_offset;
        size_t k1 = k + 1;
        uint64_t end = e0.data_offset + e0.nbytes;
        while (k1 < order.size()) {
            const Entry& e = f->entries[static_cast<size_t>(index[order[k1]])];
            if (!is_verbatim(e, dtype[order[k1]]) || e.data_offset < end ||
                e.data_offset + e.nbytes - begin > kChunk)
                break;
            end = e.data_offset + e.nbytes;
            ++k1;
        }
        int& b = f->next_buf;
        if (int st = acquire(f, b)) return st;
        unsigned char* buf = static_cast<unsigned char*>(f->pinned[b]);
        if (!pread_parallel(f->fd, buf, static_cast<size_t>(end - begin), begin))
            return fail(YTHIP_EIO, "ythip_yt_load_many: read failed at offset %llu", (unsigned long long)begin);
        for (size_t j = k; j < k1; ++j) {
            const int i = order[j];
            const Entry& e = f->entries[static_cast<size_t>(index[i])];
            hipError_t he = hipMemcpyAsync(dst[i], buf + (e.data_offset - begin), e.nbytes, hipMemcpyHostToDevice, hs);
            if (he != hipSuccess) return status_of(he);
        }
        hipError_t he = hipEventRecord(f->ev[b], hs);
        if (he != hipSuccess) return status_of(he);
        f->pending[b] = true;
        b ^= 1;
        k = k1;
    }
    return 0;
}

__attribute__((visibility("default"))) int ythip_convert_host(int src_dtype, int dst_dtype, const void* src,
                                                              void* dst, int64_t n) {
    auto kind = [](int d) { return d == YTHIP_F32 ? SRC_F32 : d == YTHIP_BF16 ? SRC_BF16 : SRC_F16; };
    auto ok = [](int d) { return d == YTHIP_F32 || d == YTHIP_F16 || d == YTHIP_BF16; };
    if (!ok(src_dtype) || !ok(dst_dtype) || n < 0 || (n > 0 && (!src || !dst)))
        return fail(YTHIP_EINVAL, "ythip_convert_host: bad arguments");
    if (n == 0) return 0;
    if (src_dtype == dst_dtype) {
        std::memcpy(dst, src, static_cast<size_t>(n) * dst_size(dst_dtype));
        return 0;
    }
    convert_parallel(kind(src_dtype), dst_dtype, static_cast<const unsigned char*>(src),
                     static_cast<unsigned char*>(dst), static_cast<size_t>(n));
    return 0;
}

__attribute__((visibility("default"))) int ythip_yt_sync(ythip_yt_file* f) {
    if (!f) return fail(YTHIP_EINVAL, "ythip_yt_sync: NULL file");
    return drain(f);
}

__attribute__((visibility("default"))) int ythip_yt_save(const char* path, int n, const ythip_yt_tensor* tensors,
                                                         const char* compress, int append, void* stream) {
    if (!path || n < 0 || (n > 0 && !tensors)) return fail(YTHIP_EINVAL, "ythip_yt_save: bad arguments");
    // checkCompressMethod (src/ytensor_io.inl:11-22): unknown names mean no compression
    const bool zlib = compress && std::strcmp(compress, "zlib") == 0;
    std::vector<Staged> items;
    std::string metadata;
    ythip_yt_file* old = nullptr;
    // Write and Append both start from an existing file's tensors (open(),
    // src/ytensor_io.inl:256-290): saving a name they hold replaces it in place
    // (715-724) and an unnamed tensor is numbered after them (712). At close,
    // Write drops the ones not saved again (339-344) and Append keeps them. The metadata string
    // of the existing file survives either way.
    {
        struct stat sb;
        if (::stat(path, &sb) == 0 && ythip_yt_open(path, &old) == 0) {
            metadata = old->metadata;
            for (const Entry& e : old->entries) {
                Staged s;
                s.meta = e;
                s.src = old;
                items.push_back(s);
            }
        } else {
            old = nullptr;
        }
    }
    int st = 0;
    for (int i = 0; i < n && st == 0; ++i) {
        const ythip_yt_tensor& t = tensors[i];
        Staged s;
        Entry& m = s.meta;
        if (t.dtype == YTHIP_YT_RAW) {
            if (!t.dtype_name || !*t.dtype_name || t.type_size <= 0)
                st = fail(YTHIP_EINVAL, "ythip_yt_save: tensor %d: raw tensors need dtype_name and type_size", i);
            m.dtype = t.dtype_name ? t.dtype_name : "";
            m.type_size = t.type_size;
        } else if (t.dtype == YTHIP_F32 || t.dtype == YTHIP_F16 || t.dtype == YTHIP_BF16) {
            m.dtype = dtype_name(t.dtype);
            m.type_size = dst_size(t.dtype);
        } else {
            st = fail(YTHIP_EINVAL, "ythip_yt_save: tensor %d: dtype %d", i, t.dtype);
        }
        if (st) break;
        if (t.ndim < 0 || t.ndim > kMaxDims || (t.ndim > 0 && !t.shape)) {
            st = fail(YTHIP_EINVAL, "ythip_yt_save: tensor %d: ndim %d", i, t.ndim);
            break;
        }
        uint64_t nb = static_cast<uint64_t>(m.type_size);
        for (int d = 0; d < t.ndim; ++d) {
            if (t.shape[d] < 0) st = fail(YTHIP_EINVAL, "ythip_yt_save: tensor %d: negative dimension", i);
            m.shape.push_back(t.shape[d]);
            nb *= static_cast<uint64_t>(std::max(0, t.shape[d]));
        }
        if (st) break;
        if (nb > 0 && !t.data) {
            st = fail(YTHIP_EINVAL, "ythip_yt_save: tensor %d: NULL data", i);
            break;
        }
        m.nbytes = nb;
        m.ttype = "dense";
        m.compress = zlib ? "zlib" : "";
        s.device = t.data;
        // save(): "" is named by its position (712); an existing name is replaced in place (715-724)
        m.name = (t.name && *t.name) ? t.name : std::to_string(items.size());
        auto same = std::find_if(items.begin(), items.end(), [&](const Staged& x) { return x.meta.name == m.name; });
        if (same != items.end())
            *same = s;
        else
            items.push_back(s);
    }
    if (!append)
        items.erase(std::remove_if(items.begin(), items.end(), [](const Staged& x) { return x.src != nullptr; }),
                    items.end());
    if (st == 0) st = write_file(path, metadata, items, zlib, static_cast<hipStream_t>(stream));
    if (old) ythip_yt_close(old);
    return st;
}

}  // extern "C"
