// GGUF reader and device loader: the on-disk format of the model packages whose
// BF16 / F16 / Q8_0 / Q5_K lookup tables feed shp_get_rows and shp_get_rows_sum
// (src/arch/qwen3-tts/catalog.cpp:77-104 resolves them by name, type and shape;
// tools/synthesize-quantize/policy.cpp:49-98 decides their types).
//
// The format (GGUF v2/v3, ggml's published specification), all little-endian:
//   u32 magic "GGUF", u32 version, u64 n_tensors, u64 n_kv,
//   n_kv x { string key, u32 value_type, value },
//   n_tensors x { string name, u32 n_dims, u64 ne[n_dims], u32 ggml_type, u64 offset },
//   zero padding to `general.alignment` (u32, default 32), then the data
//   section; each tensor's bytes sit at data_start + offset, in ggml's layout
//   (ne[0] fastest, block types as consecutive blocks).
// A string is u64 length + bytes (no terminator); an array is u32 element
// type + u64 count + elements.
//
// Opening parses and validates the header in host code only (no HIP call), so
// a package can be inspected on a machine without a GPU. Loading streams a
// tensor's bytes from the file into device memory through two pinned staging
// buffers: the read of chunk i+1 (split over up to 8 threads) overlaps the
// host-to-device copy of chunk i.

#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cerrno>
#include <cstdint>
#include <cstring>
#include <map>
#include <string>
#include <thread>
#include <vector>

#include "shp_internal.hpp"
#include "synth_gguf.h"

namespace {

constexpr uint32_t kGgufMagic       = 0x46554747u;  // "GGUF" read as a little-endian u32
constexpr uint32_t kDefaultAlign    = 32;
constexpr uint64_t kMaxStringBytes  = uint64_t{ 1 } << 30;
constexpr uint64_t kMaxCount        = uint64_t{ 1 } << 40;
constexpr int      kMaxDims         = 4;
constexpr size_t   kStageBytes      = size_t{ 32 } << 20;
constexpr unsigned kReadThreads     = 8;                   // parallel reads per staging chunk
constexpr size_t   kReadSplitMin    = size_t{ 1 } << 20;   // below this a chunk is read by one thread

enum GgufValueType : uint32_t {
    kU8 = 0, kI8 = 1, kU16 = 2, kI16 = 3, kU32 = 4, kI32 = 5, kF32 = 6, kBool = 7,
    kString = 8, kArray = 9, kU64 = 10, kI64 = 11, kF64 = 12,
};

// Bytes per element of a scalar value type (0 for string / array / unknown).
size_t scalar_size(uint32_t t) {
    switch (t) {
        case kU8: case kI8: case kBool: return 1;
        case kU16: case kI16: return 2;
        case kU32: case kI32: case kF32: return 4;
        case kU64: case kI64: case kF64: return 8;
        default: return 0;
    }
}

// ggml block geometry (elements per block, bytes per block) of the tensor types
// the reference's packages hold; 0 for a type this reader does not know.
struct BlockInfo {
    int64_t elems;
    size_t  bytes;
};

BlockInfo block_info(uint32_t type) {
    switch (type) {
        case 0: return { 1, 4 };      // F32
        case 1: return { 1, 2 };      // F16
        case 2: return { 32, 18 };    // Q4_0
        case 3: return { 32, 20 };    // Q4_1
        case 6: return { 32, 22 };    // Q5_0
        case 7: return { 32, 24 };    // Q5_1
        case 8: return { 32, 34 };    // Q8_0
        case 10: return { 256, 84 };  // Q2_K
        case 11: return { 256, 110 }; // Q3_K
        case 12: return { 256, 144 }; // Q4_K
        case 13: return { 256, 176 }; // Q5_K
        case 14: return { 256, 210 }; // Q6_K
        case 24: return { 1, 1 };     // I8
        case 25: return { 1, 2 };     // I16
        case 26: return { 1, 4 };     // I32
        case 27: return { 1, 8 };     // I64
        case 28: return { 1, 8 };     // F64
        case 30: return { 1, 2 };     // BF16
        default: return { 0, 0 };
    }
}

struct KvValue {
    uint32_t    type       = 0;
    uint64_t    u          = 0;  // unsigned / bool / bit pattern of scalars
    int64_t     i          = 0;  // signed scalars
    double      f          = 0;  // float scalars
    std::string s;               // string value
    uint32_t    array_type = 0;
    uint64_t    array_len  = 0;
};

struct TensorInfo {
    std::string name;
    int32_t     n_dims = 0;
    int64_t     ne[kMaxDims] = { 1, 1, 1, 1 };
    uint32_t    type   = 0;
    uint64_t    offset = 0;  // from the start of the data section
    uint64_t    nbytes = 0;
};

// Bounds-checked sequential reader over the file.
class Reader {
  public:
    Reader(int fd, uint64_t size) : fd_(fd), size_(size) {}

    bool bytes(void * dst, uint64_t n) {
        if (n > size_ - pos_) {
            return false;
        }
        uint8_t * out = static_cast<uint8_t *>(dst);
        while (n > 0) {
            if (buf_pos_ == buf_len_ && !refill()) {
                return false;
            }
            const uint64_t take = std::min<uint64_t>(n, buf_len_ - buf_pos_);
            std::memcpy(out, buf_.data() + buf_pos_, take);
            buf_pos_ += take;
            pos_ += take;
            out += take;
            n -= take;
        }
        return true;
    }

    template <class T> bool scalar(T & v) { return bytes(&v, sizeof(T)); }

    bool skip(uint64_t n) {
        if (n > size_ - pos_) {
            return false;
        }
        const uint64_t in_buf = std::min<uint64_t>(n, buf_len_ - buf_pos_);
        buf_pos_ += in_buf;
        pos_ += in_buf;
        n -= in_buf;
        if (n > 0) {  // beyond the buffer: drop it and reposition
            pos_ += n;
            file_pos_ = pos_;
            buf_pos_ = buf_len_ = 0;
        }
        return true;
    }

    bool string(std::string & s) {
        uint64_t len = 0;
        if (!scalar(len) || len > kMaxStringBytes || len > size_ - pos_) {
            return false;
        }
        s.resize(len);
        return len == 0 || bytes(&s[0], len);
    }

    uint64_t pos() const { return pos_; }

    uint64_t left() const { return size_ - pos_; }

  private:
    bool refill() {
        buf_.resize(1 << 16);
        const ssize_t got = pread(fd_, buf_.data(), buf_.size(), static_cast<off_t>(file_pos_));
        if (got <= 0) {
            return false;
        }
        file_pos_ += static_cast<uint64_t>(got);
        buf_pos_ = 0;
        buf_len_ = static_cast<uint64_t>(got);
        return true;
    }

    int                  fd_;
    uint64_t             size_;
    uint64_t             pos_      = 0;  // logical position
    uint64_t             file_pos_ = 0;  // file offset of the end of buf_
    std::vector<uint8_t> buf_;
    uint64_t             buf_pos_ = 0;
    uint64_t             buf_len_ = 0;
};

bool read_value(Reader & r, uint32_t type, KvValue & v) {
    v.type = type;
    switch (type) {
        case kU8: { uint8_t x; if (!r.scalar(x)) return false; v.u = x; v.i = x; return true; }
        case kI8: { int8_t x; if (!r.scalar(x)) return false; v.i = x; v.u = static_cast<uint64_t>(x); return true; }
        case kU16: { uint16_t x; if (!r.scalar(x)) return false; v.u = x; v.i = x; return true; }
        case kI16: { int16_t x; if (!r.scalar(x)) return false; v.i = x; v.u = static_cast<uint64_t>(x); return true; }
        case kU32: { uint32_t x; if (!r.scalar(x)) return false; v.u = x; v.i = x; return true; }
        case kI32: { int32_t x; if (!r.scalar(x)) return false; v.i = x; v.u = static_cast<uint64_t>(x); return true; }
        case kU64: { uint64_t x; if (!r.scalar(x)) return false; v.u = x; v.i = static_cast<int64_t>(x); return true; }
        case kI64: { int64_t x; if (!r.scalar(x)) return false; v.i = x; v.u = static_cast<uint64_t>(x); return true; }
        case kF32: { float x; if (!r.scalar(x)) return false; v.f = x; return true; }
        case kF64: { double x; if (!r.scalar(x)) return false; v.f = x; return true; }
        case kBool: {
            uint8_t x;
            if (!r.scalar(x) || x > 1) return false;
            v.u = x;
            return true;
        }
        case kString: return r.string(v.s);
        case kArray: {
            uint32_t et = 0;
            uint64_t n  = 0;
            if (!r.scalar(et) || !r.scalar(n) || n > kMaxCount) {
                return false;
            }
            v.array_type = et;
            v.array_len  = n;
            if (et == kString) {
                std::string tmp;
                for (uint64_t k = 0; k < n; ++k) {
                    if (!r.string(tmp)) {
                        return false;
                    }
                }
                return true;
            }
            const size_t es = scalar_size(et);
            if (es == 0 || n > UINT64_MAX / es) {
                return false;  // nested arrays and unknown types are not GGUF
            }
            return r.skip(n * es);
        }
        default:
            return false;
    }
}

}  // namespace

struct shp_gguf {
    int                              fd        = -1;
    uint64_t                         file_size = 0;
    uint32_t                         version   = 0;
    uint32_t                         alignment = kDefaultAlign;
    uint64_t                         data_start = 0;
    std::map<std::string, KvValue>   kv;
    std::vector<TensorInfo>          tensors;
    std::map<std::string, size_t>    by_name;
    void *                           stage[2]  = { nullptr, nullptr };
    hipEvent_t                       done[2]   = { nullptr, nullptr };
};

namespace {

shp_status_t parse(shp_gguf & g) {
    Reader   r(g.fd, g.file_size);
    uint32_t magic = 0;
    uint64_t n_tensors = 0, n_kv = 0;
    if (!r.scalar(magic) || magic != kGgufMagic || !r.scalar(g.version) || (g.version != 2 && g.version != 3) ||
        !r.scalar(n_tensors) || !r.scalar(n_kv)) {
        return SHP_ERR_INVALID_ARG;
    }
    // Every key/value takes at least 14 bytes (key length, a 1-byte key, value
    // type, a 1-byte value) and every tensor info at least 33 (name length, a
    // 1-byte name, n_dims, one dimension, type, offset), so counts the rest of
    // the file cannot hold are refused before anything is sized by them.
    if (n_kv > r.left() / 14 || n_tensors > r.left() / 33) {
        return SHP_ERR_INVALID_ARG;
    }
    for (uint64_t k = 0; k < n_kv; ++k) {
        std::string key;
        uint32_t    type = 0;
        KvValue     v;
        if (!r.string(key) || key.empty() || !r.scalar(type) || !read_value(r, type, v)) {
            return SHP_ERR_INVALID_ARG;
        }
        if (!g.kv.emplace(key, std::move(v)).second) {
            return SHP_ERR_INVALID_ARG;  // duplicate key
        }
    }
    const auto al = g.kv.find("general.alignment");
    if (al != g.kv.end()) {
        const uint64_t a = al->second.u;
        if (al->second.type != kU32 || a == 0 || (a & (a - 1)) != 0) {
            return SHP_ERR_INVALID_ARG;
        }
        g.alignment = static_cast<uint32_t>(a);
    }
    g.tensors.reserve(static_cast<size_t>(n_tensors));
    for (uint64_t t = 0; t < n_tensors; ++t) {
        g.tensors.emplace_back();
        TensorInfo & ti = g.tensors.back();
        uint32_t     nd = 0;
        if (!r.string(ti.name) || ti.name.empty() || !r.scalar(nd) || nd < 1 || nd > kMaxDims) {
            return SHP_ERR_INVALID_ARG;
        }
        ti.n_dims = static_cast<int32_t>(nd);
        for (uint32_t d = 0; d < nd; ++d) {
            uint64_t e = 0;
            if (!r.scalar(e) || e == 0 || e > (uint64_t{ 1 } << 62)) {
                return SHP_ERR_INVALID_ARG;
            }
            ti.ne[d] = static_cast<int64_t>(e);
        }
        if (!r.scalar(ti.type) || !r.scalar(ti.offset)) {
            return SHP_ERR_INVALID_ARG;
        }
        const BlockInfo b = block_info(ti.type);
        if (b.elems == 0) {
            return SHP_ERR_UNSUPPORTED;  // a tensor type this reader does not size
        }
        if (ti.ne[0] % b.elems != 0 || ti.offset % g.alignment != 0) {
            return SHP_ERR_INVALID_ARG;
        }
        // bytes = blocks per row * block bytes * ne1 * ne2 * ne3, one factor at a
        // time: each partial product must neither wrap nor pass 2^62, so every
        // stride describe() derives (a partial product) and the element count
        // (at most the byte count) fit an int64 as well.
        constexpr uint64_t kMaxBytes = uint64_t{ 1 } << 62;
        uint64_t           nb        = static_cast<uint64_t>(ti.ne[0] / b.elems);
        const uint64_t     factors[] = { b.bytes, static_cast<uint64_t>(ti.ne[1]), static_cast<uint64_t>(ti.ne[2]),
                                         static_cast<uint64_t>(ti.ne[3]) };
        for (const uint64_t f : factors) {
            if (__builtin_mul_overflow(nb, f, &nb) || nb > kMaxBytes) {
                return SHP_ERR_INVALID_ARG;
            }
        }
        ti.nbytes = nb;
        if (!g.by_name.emplace(ti.name, t).second) {
            return SHP_ERR_INVALID_ARG;  // duplicate tensor name
        }
    }
    g.data_start = (r.pos() + g.alignment - 1) / g.alignment * g.alignment;
    if (g.data_start > g.file_size) {
        return SHP_ERR_INVALID_ARG;
    }
    const uint64_t data_bytes = g.file_size - g.data_start;
    for (const TensorInfo & ti : g.tensors) {
        if (ti.offset > data_bytes || ti.nbytes > data_bytes - ti.offset) {
            return SHP_ERR_INVALID_ARG;  // tensor data past the end of the file
        }
    }
    return SHP_OK;
}

const TensorInfo * find_tensor(const shp_gguf * g, const char * name) {
    if (g == nullptr || name == nullptr) {
        return nullptr;
    }
    try {
        const auto it = g->by_name.find(name);
        return it == g->by_name.end() ? nullptr : &g->tensors[it->second];
    } catch (...) {
        return nullptr;
    }
}

const KvValue * find_kv(const shp_gguf * g, const char * key) {
    try {
        const auto it = g->kv.find(key);
        return it == g->kv.end() ? nullptr : &it->second;
    } catch (...) {
        return nullptr;
    }
}

// The shp_tensor of a tensor info (data left null): ggml's strides, nb[0] the
// element size, or the block size for Q8_0.
void describe(const TensorInfo & ti, shp_tensor * out) {
    const BlockInfo b = block_info(ti.type);
    std::memset(out, 0, sizeof(*out));
    out->type = static_cast<int32_t>(ti.type);
    for (int d = 0; d < kMaxDims; ++d) {
        out->ne[d] = ti.ne[d];
    }
    out->nb[0] = b.bytes;
    out->nb[1] = static_cast<size_t>(ti.ne[0] / b.elems) * b.bytes;
    for (int d = 2; d < kMaxDims; ++d) {
        out->nb[d] = out->nb[d - 1] * static_cast<size_t>(ti.ne[d - 1]);
    }
}

bool loadable_type(uint32_t t) {
    return t == SHP_TYPE_F32 || t == SHP_TYPE_F16 || t == SHP_TYPE_BF16 || t == SHP_TYPE_Q8_0 || t == SHP_TYPE_Q5_K ||
           t == SHP_TYPE_I32;
}

// Reads n bytes at file offset off into dst; false on a short read. Large
// reads are split over up to kReadThreads threads (a single thread copying
// out of the page cache, not PCIe, bounds the load otherwise).
bool pread_all(int fd, char * d, size_t len, uint64_t o) {
    size_t got = 0;
    while (got < len) {
        const ssize_t rd = pread(fd, d + got, len - got, static_cast<off_t>(o + got));
        if (rd < 0 && errno == EINTR) {
            continue;
        }
        if (rd <= 0) {
            return false;
        }
        got += static_cast<size_t>(rd);
    }
    return true;
}

bool read_range(int fd, char * dst, size_t n, uint64_t off) {
    auto one = [fd](char * d, size_t len, uint64_t o) { return pread_all(fd, d, len, o); };
    const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
    const unsigned nt = static_cast<unsigned>(std::min<size_t>({ kReadThreads, hw, n / kReadSplitMin }));
    if (nt <= 1) {
        return one(dst, n, off);
    }
    std::atomic<bool>        ok{ true };
    std::vector<std::thread> th;
    const size_t             part    = (n / nt + 4095) & ~size_t{ 4095 };
    unsigned                 started = 0;
    for (; started < nt; ++started) {
        const size_t b = std::min(n, part * started), e = std::min(n, part * (started + 1));
        if (b >= e) {
            continue;
        }
        try {
            th.emplace_back([&, b, e] {
                if (!one(dst + b, e - b, off + b)) {
                    ok = false;
                }
            });
        } catch (...) {  // no more threads: this thread reads what is left
            break;
        }
    }
    if (started < nt && !one(dst + part * started, n - std::min(n, part * started), off + part * started)) {
        ok = false;
    }
    for (auto & t : th) {
        t.join();
    }
    return ok;
}

void release_staging(shp_gguf * g) {
    for (int k = 0; k < 2; ++k) {
        if (g->done[k] != nullptr) {
            (void) hipEventSynchronize(g->done[k]);
            (void) hipEventDestroy(g->done[k]);
            g->done[k] = nullptr;
        }
        if (g->stage[k] != nullptr) {
            (void) hipHostFree(g->stage[k]);
            g->stage[k] = nullptr;
        }
    }
}

}  // namespace

extern "C" shp_status_t shp_gguf_open(const char * path, shp_gguf ** out) {
    if (path == nullptr || out == nullptr) {
        return SHP_ERR_INVALID_ARG;
    }
    *out    = nullptr;
    auto *g = new (std::nothrow) shp_gguf();
    if (g == nullptr) {
        return SHP_ERR_BACKEND;
    }
    g->fd = open(path, O_RDONLY | O_CLOEXEC);
    struct stat st {};
    if (g->fd < 0 || fstat(g->fd, &st) != 0 || !S_ISREG(st.st_mode)) {
        shp_gguf_close(g);
        return SHP_ERR_INVALID_ARG;
    }
    g->file_size    = static_cast<uint64_t>(st.st_size);
    shp_status_t rc = SHP_ERR_INVALID_ARG;
    try {
        rc = parse(*g);
    } catch (...) {  // allocation failure while sizing a hostile header
        rc = SHP_ERR_INVALID_ARG;
    }
    if (rc != SHP_OK) {
        shp_gguf_close(g);
        return rc;
    }
    *out = g;
    return SHP_OK;
}

extern "C" void shp_gguf_close(shp_gguf * g) {
    if (g == nullptr) {
        return;
    }
    release_staging(g);
    if (g->fd >= 0) {
        close(g->fd);
    }
    delete g;
}

extern "C" uint32_t shp_gguf_version(const shp_gguf * g) {
    return g != nullptr ? g->version : 0;
}

extern "C" int64_t shp_gguf_tensor_count(const shp_gguf * g) {
    return g != nullptr ? static_cast<int64_t>(g->tensors.size()) : -1;
}

extern "C" const char * shp_gguf_tensor_name(const shp_gguf * g, int64_t index) {
    if (g == nullptr || index < 0 || static_cast<uint64_t>(index) >= g->tensors.size()) {
        return nullptr;
    }
    return g->tensors[static_cast<size_t>(index)].name.c_str();
}

extern "C" shp_status_t shp_gguf_tensor_info(const shp_gguf * g,
                                             const char *     name,
                                             shp_tensor *     desc,
                                             uint64_t *       nbytes,
                                             uint64_t *       file_offset) {
    const TensorInfo * ti = find_tensor(g, name);
    if (ti == nullptr || desc == nullptr) {
        return SHP_ERR_INVALID_ARG;
    }
    describe(*ti, desc);
    if (nbytes != nullptr) {
        *nbytes = ti->nbytes;
    }
    if (file_offset != nullptr) {
        *file_offset = g->data_start + ti->offset;
    }
    return SHP_OK;
}

extern "C" shp_status_t shp_gguf_kv_u32(const shp_gguf * g, const char * key, uint32_t * value) {
    if (g == nullptr || key == nullptr || value == nullptr) {
        return SHP_ERR_INVALID_ARG;
    }
    const KvValue * v = find_kv(g, key);
    if (v == nullptr || v->type != kU32) {
        return SHP_ERR_INVALID_ARG;
    }
    *value = static_cast<uint32_t>(v->u);
    return SHP_OK;
}

extern "C" shp_status_t shp_gguf_kv_string(const shp_gguf * g, const char * key, char * buf, size_t capacity) {
    if (g == nullptr || key == nullptr || buf == nullptr || capacity == 0) {
        return SHP_ERR_INVALID_ARG;
    }
    const KvValue * v = find_kv(g, key);
    if (v == nullptr || v->type != kString || v->s.size() + 1 > capacity ||
        std::memchr(v->s.data(), 0, v->s.size()) != nullptr) {
        return SHP_ERR_INVALID_ARG;
    }
    std::memcpy(buf, v->s.data(), v->s.size());
    buf[v->s.size()] = '\0';
    return SHP_OK;
}

extern "C" shp_status_t shp_gguf_load_tensor(shp_gguf *   g,
                                             const char * name,
                                             void *       device_dst,
                                             size_t       capacity,
                                             shp_tensor * desc,
                                             shp_stream_t stream) {
    const TensorInfo * ti = find_tensor(g, name);
    if (ti == nullptr || device_dst == nullptr || desc == nullptr) {
        return SHP_ERR_INVALID_ARG;
    }
    if (!loadable_type(ti->type)) {
        return SHP_ERR_UNSUPPORTED;
    }
    if (ti->nbytes > capacity) {
        return SHP_ERR_INVALID_ARG;
    }
    const hipStream_t s = shp::as_stream(stream);
    for (int k = 0; k < 2; ++k) {
        if (g->stage[k] == nullptr) {
            if (hipHostMalloc(&g->stage[k], kStageBytes, hipHostMallocDefault) != hipSuccess ||
                hipEventCreateWithFlags(&g->done[k], hipEventDisableTiming) != hipSuccess) {
                release_staging(g);
                return SHP_ERR_BACKEND;
            }
        }
    }
    uint64_t done_bytes = 0;
    int      k          = 0;
    while (done_bytes < ti->nbytes) {
        const size_t n = static_cast<size_t>(std::min<uint64_t>(kStageBytes, ti->nbytes - done_bytes));
        // the copy that last used this staging buffer must have finished
        if (hipEventSynchronize(g->done[k]) != hipSuccess) {
            return SHP_ERR_BACKEND;
        }
        if (!read_range(g->fd, static_cast<char *>(g->stage[k]), n, g->data_start + ti->offset + done_bytes)) {
            (void) hipStreamSynchronize(s);
            return SHP_ERR_INVALID_ARG;  // the file shrank under us
        }
        if (hipMemcpyAsync(static_cast<char *>(device_dst) + done_bytes, g->stage[k], n, hipMemcpyHostToDevice, s) !=
                hipSuccess ||
            hipEventRecord(g->done[k], s) != hipSuccess) {
            (void) hipStreamSynchronize(s);
            return SHP_ERR_BACKEND;
        }
        done_bytes += n;
        k ^= 1;
    }
    if (hipStreamSynchronize(s) != hipSuccess) {
        return SHP_ERR_BACKEND;
    }
    describe(*ti, desc);
    desc->data = device_dst;
    return SHP_OK;
}

namespace {

// One piece of a staging chunk: n bytes of the file at file_off, staged at
// stage_off, bound for dst.
struct Piece {
    size_t   stage_off;
    uint64_t file_off;
    size_t   n;
    char *   dst;
};

// Reads a chunk's pieces into the staging buffer: the chunk's filled bytes
// are split into up to kReadThreads equal parts, and each part's thread reads
// the parts of the pieces that fall in it, so a chunk of many small tensors
// is read as much in parallel as one large tensor.
bool read_pieces(int fd, char * stage, const std::vector<Piece> & ps, size_t fill) {
    auto span = [&](size_t b, size_t e) {
        for (const Piece & p : ps) {
            const size_t lo = std::max(b, p.stage_off), hi = std::min(e, p.stage_off + p.n);
            if (lo < hi && !pread_all(fd, stage + lo, hi - lo, p.file_off + (lo - p.stage_off))) {
                return false;
            }
        }
        return true;
    };
    const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
    const unsigned nt = static_cast<unsigned>(std::min<size_t>({ kReadThreads, hw, fill / kReadSplitMin }));
    if (nt <= 1) {
        return span(0, fill);
    }
    std::atomic<bool>        ok{ true };
    std::vector<std::thread> th;
    const size_t             part = (fill / nt + 4095) & ~size_t{ 4095 };
    size_t                   b    = 0;
    for (unsigned t = 0; t < nt && b < fill; ++t, b += part) {
        const size_t e = std::min(fill, b + part);
        try {
            th.emplace_back([&, b, e] {
                if (!span(b, e)) {
                    ok = false;
                }
            });
        } catch (...) {  // no more threads: this thread reads what is left
            break;
        }
    }
    if (b < fill && !span(b, fill)) {
        ok = false;
    }
    for (auto & t : th) {
        t.join();
    }
    return ok;
}

}  // namespace

extern "C" shp_status_t shp_gguf_load_tensors(shp_gguf *          g,
                                              const char * const * names,
                                              int32_t              count,
                                              void * const *       device_dsts,
                                              const size_t *       capacities,
                                              shp_tensor *         descs,
                                              shp_stream_t         stream) {
    if (g == nullptr || count < 0 || (count > 0 && (names == nullptr || device_dsts == nullptr ||
                                                    capacities == nullptr || descs == nullptr))) {
        return SHP_ERR_INVALID_ARG;
    }
    // Every tensor is checked before anything is read.
    std::vector<const TensorInfo *> tis(static_cast<size_t>(count));
    for (int32_t i = 0; i < count; ++i) {
        const TensorInfo * ti = names[i] != nullptr ? find_tensor(g, names[i]) : nullptr;
        if (ti == nullptr || device_dsts[i] == nullptr) {
            return SHP_ERR_INVALID_ARG;
        }
        if (!loadable_type(ti->type)) {
            return SHP_ERR_UNSUPPORTED;
        }
        if (ti->nbytes > capacities[i]) {
            return SHP_ERR_INVALID_ARG;
        }
        tis[static_cast<size_t>(i)] = ti;
    }
    if (count == 0) {
        return SHP_OK;
    }
    const hipStream_t s = shp::as_stream(stream);
    for (int k = 0; k < 2; ++k) {
        if (g->stage[k] == nullptr) {
            if (hipHostMalloc(&g->stage[k], kStageBytes, hipHostMallocDefault) != hipSuccess ||
                hipEventCreateWithFlags(&g->done[k], hipEventDisableTiming) != hipSuccess) {
                release_staging(g);
                return SHP_ERR_BACKEND;
            }
        }
    }
    // The tensors' bytes go through the staging buffers back to back: a chunk
    // holds the ends and starts of as many tensors as fit, its pieces are read
    // in parallel, and each piece is one copy to its destination.
    std::vector<Piece> ps;
    size_t             fill = 0;
    int                k    = 0;
    auto flush = [&]() -> shp_status_t {
        if (fill == 0) {
            return SHP_OK;
        }
        if (hipEventSynchronize(g->done[k]) != hipSuccess) {  // the chunk's previous copies
            return SHP_ERR_BACKEND;
        }
        char * stage = static_cast<char *>(g->stage[k]);
        if (!read_pieces(g->fd, stage, ps, fill)) {
            (void) hipStreamSynchronize(s);
            return SHP_ERR_INVALID_ARG;  // the file shrank under us
        }
        for (const Piece & p : ps) {
            if (hipMemcpyAsync(p.dst, stage + p.stage_off, p.n, hipMemcpyHostToDevice, s) != hipSuccess) {
                (void) hipStreamSynchronize(s);
                return SHP_ERR_BACKEND;
            }
        }
        if (hipEventRecord(g->done[k], s) != hipSuccess) {
            (void) hipStreamSynchronize(s);
            return SHP_ERR_BACKEND;
        }
        ps.clear();
        fill = 0;
        k ^= 1;
        return SHP_OK;
    };
    for (int32_t i = 0; i < count; ++i) {
        const TensorInfo * ti  = tis[static_cast<size_t>(i)];
        uint64_t           off = 0;
        while (off < ti->nbytes) {
            const size_t take = static_cast<size_t>(std::min<uint64_t>(kStageBytes - fill, ti->nbytes - off));
            ps.push_back(Piece{ fill, g->data_start + ti->offset + off, take,
                                static_cast<char *>(device_dsts[i]) + off });
            fill += take;
            off += take;
            if (fill == kStageBytes) {
                const shp_status_t st = flush();
                if (st != SHP_OK) {
                    return st;
                }
            }
        }
    }
    const shp_status_t st = flush();
    if (st != SHP_OK) {
        return st;
    }
    if (hipStreamSynchronize(s) != hipSuccess) {
        return SHP_ERR_BACKEND;
    }
    for (int32_t i = 0; i < count; ++i) {
        describe(*tis[static_cast<size_t>(i)], &descs[i]);
        descs[i].data = device_dsts[i];
    }
    return SHP_OK;
}

extern "C" shp_status_t shp_table_type_for_profile(const char * profile, int32_t * type) {
    if (profile == nullptr || type == nullptr) {
        return SHP_ERR_INVALID_ARG;
    }
    const std::string p(profile);
    // The talker half's Role::Matrix tensors -- the text and codec embedding
    // tables among them -- under each Qwen3-TTS quantization profile
    // (qwen3-tts/catalog.cpp:155-196; the profile table of
    // tools/synthesize-quantize/policy.cpp:49-98).
    if (p == "BF16") {
        *type = SHP_TYPE_BF16;
    } else if (p == "F16") {
        *type = SHP_TYPE_F16;
    } else if (p == "Q8_MIXED") {
        *type = SHP_TYPE_Q8_0;
    } else if (p == "Q5_K_MIXED") {
        *type = SHP_TYPE_Q5_K;
    } else {
        return SHP_ERR_INVALID_ARG;
    }
    return SHP_OK;
}
