// state_dict.hip -- weight files to and from HBM: the reference's GHOSTFLW
// state dict (ghostflow-core/src/serialize.rs:11-186) and GHOSTFLQ, this
// library's file for QuantizedTensor (ghostflow-nn/src/quantization.rs:
// 40-51).  The byte layouts are spelled out in include/ghostflow_hip.h.
//
// Reading maps the file once and validates every size against the mapping
// before anything is copied.  A tensor then streams to the device through
// two pinned staging buffers: while the DMA engine copies chunk i from one,
// host threads (a pool the handle keeps) fill chunk i + 1 into the other, so
// the page-cache copy and the PCIe transfer overlap; the pieces of one read
// call (codes, scales, zero points) share that pipeline.  Writing copies device tensors back through the
// same staging size and writes the reference's byte layout.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdio>
#include <cerrno>
#include <cstring>
#include <memory>
#include <new>
#include <string>
#include <condition_variable>
#include <mutex>
#include <thread>
#include <unordered_map>
#include <vector>

#include "common.hpp"

namespace {

using gfh::set_error;

constexpr char kMagicW[8] = {'G', 'H', 'O', 'S', 'T', 'F', 'L', 'W'};
constexpr char kMagicQ[8] = {'G', 'H', 'O', 'S', 'T', 'F', 'L', 'Q'};
constexpr uint32_t kVersion = 1;
constexpr size_t kChunk = 16u << 20;  // staging buffer size
constexpr uint64_t kAlign = 64;       // GHOSTFLQ payload alignment

struct Entry {
    std::string name;
    int kind = 0;   // 0 f32 tensor, 1 QuantizedTensor
    int dtype = 2;  // dtype byte (kind 0) or scheme (kind 1)
    std::vector<int64_t> dims;
    int64_t numel = 0;
    int64_t nscales = 0;
    uint64_t data_off = 0, scales_off = 0, zps_off = 0;
};

// Rust's String::from_utf8 acceptance: well-formed UTF-8 only (no overlong
// forms, no surrogates, nothing above U+10FFFF).
bool valid_utf8(const uint8_t *s, size_t n) {
    size_t i = 0;
    while (i < n) {
        const uint8_t c = s[i];
        if (c < 0x80) {
            ++i;
            continue;
        }
        int len;
        uint32_t cp;
        if ((c & 0xE0) == 0xC0) {
            len = 2;
            cp = c & 0x1F;
        } else if ((c & 0xF0) == 0xE0) {
            len = 3;
            cp = c & 0x0F;
        } else if ((c & 0xF8) == 0xF0) {
            len = 4;
            cp = c & 0x07;
        } else {
            return false;
        }
        if (i + len > n) return false;
        for (int j = 1; j < len; ++j) {
            if ((s[i + j] & 0xC0) != 0x80) return false;
            cp = (cp << 6) | (s[i + j] & 0x3F);
        }
        if ((len == 2 && cp < 0x80) || (len == 3 && cp < 0x800) || (len == 4 && cp < 0x10000)) return false;
        if (cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF)) return false;
        i += len;
    }
    return true;
}

// Bounds-checked little-endian reader over the mapping.
struct Cursor {
    const uint8_t *base;
    uint64_t size, pos = 0;
    bool take(uint64_t n, const uint8_t **out) {
        if (n > size - pos) return false;
        *out = base + pos;
        pos += n;
        return true;
    }
    template <typename T>
    bool get(T *v) {
        const uint8_t *p;
        if (!take(sizeof(T), &p)) return false;
        std::memcpy(v, p, sizeof(T));  // the file is little-endian, as is the host
        return true;
    }
    bool align(uint64_t a) {
        const uint64_t next = (pos + a - 1) / a * a;
        if (next > size) return false;
        pos = next;
        return true;
    }
};

int read_error(const char *what) { return set_error(GFH_INVALID_DATA, "state dict: Read error: %s", what); }

// Page cache -> pinned memory on up to kCopyThreads threads (one thread
// moves ~10 GB/s, below the host link's rate): the calling thread and
// kCopyThreads - 1 workers that live as long as the handle, so a chunk does
// not pay for starting threads.  The parts of a chunk are taken from a
// shared counter by whichever thread is free, the caller included, so a
// copy completes even if no worker could be started.
constexpr int kCopyThreads = 8;
class CopyPool {
  public:
    ~CopyPool() {
        {
            std::lock_guard<std::mutex> lk(mu_);
            stop_ = true;
        }
        cv_.notify_all();
        for (std::thread &t : th_) t.join();
    }

    void copy(void *dst, const void *src, size_t n) {
        const size_t per = std::max<size_t>((n + kCopyThreads - 1) / kCopyThreads, 512u << 10);
        const int parts = (int)((n + per - 1) / per);
        if (parts <= 1) {
            std::memcpy(dst, src, n);
            return;
        }
        start();
        {
            std::lock_guard<std::mutex> lk(mu_);
            dst_ = static_cast<char *>(dst);
            src_ = static_cast<const char *>(src);
            n_ = n;
            per_ = per;
            parts_ = parts;
            next_ = 0;
            pending_ = parts;
        }
        cv_.notify_all();
        std::unique_lock<std::mutex> lk(mu_);
        take_parts(lk);
        done_.wait(lk, [&] { return pending_ == 0; });
    }

  private:
    void start() {
        if (started_) return;
        started_ = true;
        try {
            for (int t = 1; t < kCopyThreads; ++t) th_.emplace_back([this] { worker(); });
        } catch (...) {  // fewer workers: the callers take the rest of the parts
        }
    }
    // Copy parts while any is left; called and returning with lk held.
    void take_parts(std::unique_lock<std::mutex> &lk) {
        while (next_ < parts_) {
            const int part = next_++;
            const size_t off = (size_t)part * per_, len = std::min(per_, n_ - off);
            lk.unlock();
            std::memcpy(dst_ + off, src_ + off, len);
            lk.lock();
            if (--pending_ == 0) done_.notify_all();
        }
    }
    void worker() {
        std::unique_lock<std::mutex> lk(mu_);
        for (;;) {
            cv_.wait(lk, [&] { return stop_ || next_ < parts_; });
            if (stop_) return;
            take_parts(lk);
        }
    }

    std::mutex mu_;
    std::condition_variable cv_, done_;
    std::vector<std::thread> th_;
    bool started_ = false, stop_ = false;
    char *dst_ = nullptr;
    const char *src_ = nullptr;
    size_t n_ = 0, per_ = 0;
    int parts_ = 0, next_ = 0, pending_ = 0;
};

}  // namespace

struct gfh_state_dict {
    int fd = -1;
    const uint8_t *map = nullptr;
    size_t size = 0;
    std::vector<Entry> entries;
    std::unordered_map<std::string, int64_t> index;
    void *pinned[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    bool used[2] = {false, false};  // a copy from that buffer may still be in flight
    int next_buf = 0;
    CopyPool pool;

    ~gfh_state_dict() {
        (void)finish();  // no pinned buffer is freed under a copy
        for (int i = 0; i < 2; ++i) {
            if (done[i]) (void)hipEventDestroy(done[i]);
            if (pinned[i]) (void)hipHostFree(pinned[i]);
        }
        if (map) munmap(const_cast<uint8_t *>(map), size);
        if (fd >= 0) close(fd);
    }

    int staging() {
        for (int i = 0; i < 2; ++i) {
            if (!pinned[i] && hipHostMalloc(&pinned[i], kChunk, hipHostMallocDefault) != hipSuccess)
                return set_error(GFH_ALLOCATION_FAILED, "state dict: pinned staging allocation failed");
            if (!done[i] && hipEventCreateWithFlags(&done[i], hipEventDisableTiming) != hipSuccess)
                return set_error(GFH_COMPUTATION_FAILED, "state dict: event creation failed");
        }
        return GFH_SUCCESS;
    }

    // Host bytes [off, off + n) of the mapping toward device memory at dst,
    // chunk by chunk through the two staging buffers in turn; the pieces of
    // one read call share the pipeline, and finish() waits for it.
    // Chunks of about a sixth of the piece, 4 to 16 MB: the first chunk's
    // host copy and the last one's transfer do not overlap anything, which
    // favours small chunks for short pieces, while every chunk costs a
    // submission and a wait.  Measured (MB/chunk: ms): three 45 MB int8
    // tensors 16: 3.34-3.49, 8: 3.08-3.11; three 180 MB fp32 tensors 16:
    // 10.81, 8: 10.89-11.25.
    int enqueue(uint64_t off, uint64_t n, void *dst, hipStream_t s) {
        if (n == 0) return GFH_SUCCESS;
        GFH_TRY(staging());
        constexpr uint64_t kMiB = 1u << 20;
        const uint64_t chunk = std::min<uint64_t>(kChunk, std::max<uint64_t>(4 * kMiB, (n / 6 + kMiB - 1) / kMiB * kMiB));
        for (uint64_t done_bytes = 0; done_bytes < n;) {
            const int b = next_buf;
            const uint64_t len = std::min<uint64_t>(chunk, n - done_bytes);
            if (used[b]) {
                if (hipEventSynchronize(done[b]) != hipSuccess)
                    return set_error(GFH_COMPUTATION_FAILED, "state dict: copy failed");
                used[b] = false;
            }
            pool.copy(pinned[b], map + off + done_bytes, len);
            if (hipMemcpyAsync(static_cast<char *>(dst) + done_bytes, pinned[b], len, hipMemcpyHostToDevice, s) !=
                hipSuccess)
                return set_error(GFH_COMPUTATION_FAILED, "state dict: host-to-device copy failed");
            used[b] = true;  // from here on the buffer may be in use, recorded or not
            if (hipEventRecord(done[b], s) != hipSuccess) {
                (void)hipStreamSynchronize(s);
                used[b] = false;
                return set_error(GFH_COMPUTATION_FAILED, "state dict: host-to-device copy failed");
            }
            next_buf = b ^ 1;
            done_bytes += len;
        }
        return GFH_SUCCESS;
    }
    // Waits until no staging buffer is being copied from.
    int finish() {
        int rc = GFH_SUCCESS;
        for (int b = 0; b < 2; ++b) {
            if (used[b] && hipEventSynchronize(done[b]) != hipSuccess)
                rc = set_error(GFH_COMPUTATION_FAILED, "state dict: copy failed");
            used[b] = false;
        }
        return rc;
    }
};

namespace {

// Parse one entry at the cursor (GHOSTFLW: kind 0 without a kind byte).
int parse_entry(Cursor &c, bool quantized, Entry &e) {
    uint32_t name_len;
    const uint8_t *name;
    if (!c.get(&name_len) || !c.take(name_len, &name)) return read_error("truncated name");
    if (!valid_utf8(name, name_len)) return set_error(GFH_INVALID_DATA, "state dict: Invalid UTF-8 in a name");
    e.name.assign(reinterpret_cast<const char *>(name), name_len);
    uint8_t kind = 0, dtype;
    if (quantized && !c.get(&kind)) return read_error("truncated kind");
    if (kind > 1) return set_error(GFH_INVALID_DATA, "state dict: unknown entry kind %u", (unsigned)kind);
    if (!c.get(&dtype)) return read_error("truncated dtype");
    if (kind == 0 && dtype > 9) return set_error(GFH_INVALID_DATA, "state dict: Unknown dtype: %u", (unsigned)dtype);
    if (kind == 1 && dtype > 2)
        return set_error(GFH_INVALID_DATA, "state dict: unknown quantization scheme %u", (unsigned)dtype);
    e.kind = kind;
    e.dtype = dtype;
    uint32_t ndim;
    if (!c.get(&ndim)) return read_error("truncated ndim");
    if ((uint64_t)ndim * 8 > c.size - c.pos) return read_error("truncated dims");
    e.dims.resize(ndim);
    __int128 numel = 1;
    for (uint32_t d = 0; d < ndim; ++d) {
        uint64_t v;
        if (!c.get(&v)) return read_error("truncated dims");
        if (v > (uint64_t)INT64_MAX) return set_error(GFH_INVALID_DATA, "state dict: dimension too large");
        e.dims[d] = (int64_t)v;
        numel *= (__int128)v;
        if (numel > ((__int128)1 << 56)) return set_error(GFH_INVALID_DATA, "state dict: tensor too large");
    }
    e.numel = (int64_t)numel;
    const uint8_t *p;
    if (kind == 0) {
        if (quantized && !c.align(kAlign)) return read_error("truncated padding");
        e.data_off = c.pos;
        if (!c.take((uint64_t)e.numel * 4, &p)) return read_error("truncated tensor data");
        return GFH_SUCCESS;
    }
    uint64_t nscales;
    if (!c.get(&nscales)) return read_error("truncated scale count");
    if (nscales != 1 && (ndim == 0 || nscales != (uint64_t)e.dims[0] || e.numel == 0))
        return set_error(GFH_INVALID_DATA, "state dict: %llu scales for shape of %lld elements",
                         (unsigned long long)nscales, (long long)e.numel);
    e.nscales = (int64_t)nscales;
    if (!c.align(kAlign)) return read_error("truncated padding");
    e.scales_off = c.pos;
    if (!c.take(nscales * 4, &p)) return read_error("truncated scales");
    e.zps_off = c.pos;
    if (!c.take(nscales, &p) || !c.align(kAlign)) return read_error("truncated zero points");
    e.data_off = c.pos;
    if (!c.take((uint64_t)e.numel, &p)) return read_error("truncated codes");
    return GFH_SUCCESS;
}

int open_impl(const char *path, gfh_state_dict **out) {
    if (!path || !out) return set_error(GFH_NULL_POINTER, "state dict: path and out must be non-NULL");
    *out = nullptr;
    std::unique_ptr<gfh_state_dict> sd(new gfh_state_dict());
    sd->fd = ::open(path, O_RDONLY | O_CLOEXEC);
    if (sd->fd < 0) return set_error(GFH_INVALID_DATA, "state dict: Failed to open file: %s", strerror(errno));
    struct stat st;
    if (fstat(sd->fd, &st) != 0) return set_error(GFH_INVALID_DATA, "state dict: stat failed: %s", strerror(errno));
    sd->size = (size_t)st.st_size;
    if (sd->size > 0) {
        void *m = mmap(nullptr, sd->size, PROT_READ, MAP_PRIVATE, sd->fd, 0);
        if (m == MAP_FAILED) return set_error(GFH_INVALID_DATA, "state dict: mmap failed: %s", strerror(errno));
        sd->map = static_cast<const uint8_t *>(m);
        (void)madvise(m, sd->size, MADV_SEQUENTIAL);
    }
    Cursor c{sd->map, sd->size};
    const uint8_t *magic;
    if (!c.take(8, &magic)) return read_error("truncated header");
    const bool quantized = std::memcmp(magic, kMagicQ, 8) == 0;
    if (!quantized && std::memcmp(magic, kMagicW, 8) != 0)
        return set_error(GFH_INVALID_DATA, "state dict: Invalid file format");
    uint32_t version, count;
    if (!c.get(&version)) return read_error("truncated version");
    if (version > kVersion)
        return set_error(GFH_INVALID_DATA, "state dict: Unsupported version: %u (max: %u)", version, kVersion);
    if (!c.get(&count)) return read_error("truncated count");
    for (uint32_t i = 0; i < count; ++i) {
        Entry e;
        GFH_TRY(parse_entry(c, quantized, e));
        auto it = sd->index.find(e.name);
        if (it != sd->index.end()) {
            sd->entries[(size_t)it->second] = std::move(e);  // HashMap insert: the last one wins
        } else {
            sd->index.emplace(e.name, (int64_t)sd->entries.size());
            sd->entries.push_back(std::move(e));
        }
    }
    *out = sd.release();
    return GFH_SUCCESS;
}

int check_entry(const gfh_state_dict *sd, int64_t index) {
    if (!sd) return set_error(GFH_NULL_POINTER, "state dict: NULL handle");
    if (index < 0 || index >= (int64_t)sd->entries.size())
        return set_error(GFH_INVALID_SHAPE, "state dict: index %lld out of range (%zu entries)", (long long)index,
                         sd->entries.size());
    return GFH_SUCCESS;
}

// ---- writing ----------------------------------------------------------------

struct Writer {
    FILE *f = nullptr;
    uint64_t pos = 0;
    void *stage = nullptr;
    ~Writer() {
        if (stage) (void)hipHostFree(stage);
        if (f) fclose(f);
    }
    bool put(const void *p, size_t n) {
        if (n && fwrite(p, 1, n, f) != n) return false;
        pos += n;
        return true;
    }
    template <typename T>
    bool val(T v) {
        return put(&v, sizeof(T));
    }
    bool pad(uint64_t a) {
        static const uint8_t zeros[kAlign] = {};
        const uint64_t n = (a - pos % a) % a;
        return put(zeros, n);
    }
    // Device bytes [src, src + n) appended to the file.
    int device(const void *src, uint64_t n) {
        if (!stage && hipHostMalloc(&stage, kChunk, hipHostMallocDefault) != hipSuccess)
            return set_error(GFH_ALLOCATION_FAILED, "state dict: pinned staging allocation failed");
        for (uint64_t off = 0; off < n; off += kChunk) {
            const uint64_t len = std::min<uint64_t>(kChunk, n - off);
            if (hipMemcpy(stage, static_cast<const char *>(src) + off, len, hipMemcpyDeviceToHost) != hipSuccess)
                return set_error(GFH_COMPUTATION_FAILED, "state dict: device-to-host copy failed");
            if (!put(stage, len)) return set_error(GFH_COMPUTATION_FAILED, "state dict: Write error");
        }
        return GFH_SUCCESS;
    }
};

int save_impl(const char *path, int quantized, const gfh_tensor_entry *entries, int64_t count, hipStream_t s) {
    if (!path || (count > 0 && !entries)) return set_error(GFH_NULL_POINTER, "state dict: path and entries needed");
    if (count < 0 || count > UINT32_MAX) return set_error(GFH_INVALID_SHAPE, "state dict: count out of range");
    // Validate everything before the file is created.
    std::vector<int64_t> numel((size_t)count);
    for (int64_t i = 0; i < count; ++i) {
        const gfh_tensor_entry &e = entries[i];
        if (!e.name) return set_error(GFH_NULL_POINTER, "state dict: entry %lld has no name", (long long)i);
        if (e.kind != 0 && !(quantized && e.kind == 1))
            return set_error(GFH_INVALID_DATA, "state dict: entry '%s' kind %d not allowed in this format", e.name,
                             e.kind);
        if (e.ndim < 0 || (e.ndim > 0 && !e.dims))
            return set_error(GFH_INVALID_SHAPE, "state dict: entry '%s' has bad ndim %d", e.name, e.ndim);
        if ((e.kind == 0 && (e.dtype < 0 || e.dtype > 9)) || (e.kind == 1 && (e.dtype < 0 || e.dtype > 2)))
            return set_error(GFH_INVALID_DATA, "state dict: entry '%s' has bad dtype / scheme %d", e.name, e.dtype);
        __int128 n = 1;
        for (int d = 0; d < e.ndim; ++d) {
            if (e.dims[d] < 0) return set_error(GFH_INVALID_SHAPE, "state dict: entry '%s' negative dim", e.name);
            n *= e.dims[d];
            if (n > ((__int128)1 << 56)) return set_error(GFH_INVALID_SHAPE, "state dict: entry '%s' too large", e.name);
        }
        numel[(size_t)i] = (int64_t)n;
        if (e.kind == 0) {
            GFH_TRY(gfh::require_range(e.data, (size_t)n * 4, "data"));
        } else {
            if (e.nscales != 1 && (e.ndim == 0 || e.nscales != e.dims[0] || n == 0))
                return set_error(GFH_INVALID_SHAPE, "state dict: entry '%s' nscales must be 1 or dims[0]", e.name);
            GFH_TRY(gfh::require_range(e.data, (size_t)n, "codes"));
            GFH_TRY(gfh::require_range(e.scales, (size_t)e.nscales * 4, "scales"));
            GFH_TRY(gfh::require_range(e.zero_points, (size_t)e.nscales, "zero_points"));
        }
        if (!valid_utf8(reinterpret_cast<const uint8_t *>(e.name), strlen(e.name)))
            return set_error(GFH_INVALID_DATA, "state dict: entry name is not UTF-8");
    }
    if (hipStreamSynchronize(s) != hipSuccess)
        return set_error(GFH_COMPUTATION_FAILED, "state dict: stream synchronization failed");
    Writer w;
    w.f = fopen(path, "wb");
    if (!w.f) return set_error(GFH_INVALID_DATA, "state dict: Failed to create file: %s", strerror(errno));
    bool ok = w.put(quantized ? kMagicQ : kMagicW, 8) && w.val<uint32_t>(kVersion) && w.val<uint32_t>((uint32_t)count);
    for (int64_t i = 0; ok && i < count; ++i) {
        const gfh_tensor_entry &e = entries[i];
        const uint32_t name_len = (uint32_t)strlen(e.name);
        ok = w.val(name_len) && w.put(e.name, name_len);
        if (ok && quantized) ok = w.val<uint8_t>((uint8_t)e.kind);
        ok = ok && w.val<uint8_t>((uint8_t)e.dtype) && w.val<uint32_t>((uint32_t)e.ndim);
        for (int d = 0; ok && d < e.ndim; ++d) ok = w.val<uint64_t>((uint64_t)e.dims[d]);
        if (!ok) break;
        if (e.kind == 0) {
            if (quantized && !w.pad(kAlign)) break;
            GFH_TRY(w.device(e.data, (uint64_t)numel[(size_t)i] * 4));
        } else {
            ok = w.val<uint64_t>((uint64_t)e.nscales) && w.pad(kAlign);
            if (!ok) break;
            GFH_TRY(w.device(e.scales, (uint64_t)e.nscales * 4));
            GFH_TRY(w.device(e.zero_points, (uint64_t)e.nscales));
            if (!w.pad(kAlign)) {
                ok = false;
                break;
            }
            GFH_TRY(w.device(e.data, (uint64_t)numel[(size_t)i]));
        }
    }
    if (!ok || fflush(w.f) != 0) return set_error(GFH_COMPUTATION_FAILED, "state dict: Write error");
    return GFH_SUCCESS;
}

template <typename F>
int guarded(F &&f) {
    try {
        return f();
    } catch (const std::bad_alloc &) {
        return set_error(GFH_ALLOCATION_FAILED, "state dict: host allocation failed");
    } catch (...) {
        return set_error(GFH_UNKNOWN, "state dict: unexpected C++ exception");
    }
}

}  // namespace

extern "C" {

GFH_API int gfh_state_dict_open(const char *path, gfh_state_dict **out) {
    return guarded([&] { return open_impl(path, out); });
}

GFH_API void gfh_state_dict_close(gfh_state_dict *sd) { delete sd; }

GFH_API int64_t gfh_state_dict_count(const gfh_state_dict *sd) { return sd ? (int64_t)sd->entries.size() : -1; }

GFH_API int gfh_state_dict_entry(const gfh_state_dict *sd, int64_t index, const char **name, int *kind, int *dtype,
                                 int *ndim, int64_t *dims, int max_dims, int64_t *nscales) {
    GFH_TRY(check_entry(sd, index));
    const Entry &e = sd->entries[(size_t)index];
    if (name) *name = e.name.c_str();
    if (kind) *kind = e.kind;
    if (dtype) *dtype = e.dtype;
    if (ndim) *ndim = (int)e.dims.size();
    if (dims)
        for (int d = 0; d < max_dims && d < (int)e.dims.size(); ++d) dims[d] = e.dims[(size_t)d];
    if (nscales) *nscales = e.nscales;
    return GFH_SUCCESS;
}

GFH_API int64_t gfh_state_dict_find(const gfh_state_dict *sd, const char *name) {
    if (!sd || !name) return -1;
    auto it = sd->index.find(name);
    return it == sd->index.end() ? -1 : it->second;
}

GFH_API int gfh_state_dict_read_f32(gfh_state_dict *sd, int64_t index, float *dst, gfh_stream_t stream) {
    return guarded([&]() -> int {
        GFH_TRY(check_entry(sd, index));
        const Entry &e = sd->entries[(size_t)index];
        if (e.kind != 0)
            return set_error(GFH_INVALID_DATA, "state dict: '%s' is a quantized entry; use read_q8", e.name.c_str());
        if (e.numel == 0) return GFH_SUCCESS;
        GFH_TRY(gfh::require_range(dst, (size_t)e.numel * 4, "dst"));
        GFH_TRY(gfh::ensure_init());
        const int rc = sd->enqueue(e.data_off, (uint64_t)e.numel * 4, dst, gfh::as_stream(stream));
        const int rf = sd->finish();
        return rc != GFH_SUCCESS ? rc : rf;
    });
}

GFH_API int gfh_state_dict_read_q8(gfh_state_dict *sd, int64_t index, int8_t *codes, float *scales,
                                   int8_t *zero_points, gfh_stream_t stream) {
    return guarded([&]() -> int {
        GFH_TRY(check_entry(sd, index));
        const Entry &e = sd->entries[(size_t)index];
        if (e.kind != 1)
            return set_error(GFH_INVALID_DATA, "state dict: '%s' is an f32 entry; use read_f32", e.name.c_str());
        GFH_TRY(gfh::require_range(codes, (size_t)e.numel, "codes"));
        GFH_TRY(gfh::require_range(scales, (size_t)e.nscales * 4, "scales"));
        GFH_TRY(gfh::require_range(zero_points, (size_t)e.nscales, "zero_points"));
        GFH_TRY(gfh::ensure_init());
        hipStream_t s = gfh::as_stream(stream);
        int rc = sd->enqueue(e.scales_off, (uint64_t)e.nscales * 4, scales, s);
        if (rc == GFH_SUCCESS) rc = sd->enqueue(e.zps_off, (uint64_t)e.nscales, zero_points, s);
        if (rc == GFH_SUCCESS) rc = sd->enqueue(e.data_off, (uint64_t)e.numel, codes, s);
        const int rf = sd->finish();  // the call returns once its data is in device memory
        return rc != GFH_SUCCESS ? rc : rf;
    });
}

GFH_API int gfh_state_dict_save(const char *path, int quantized_format, const gfh_tensor_entry *entries, int64_t count,
                                gfh_stream_t stream) {
    return guarded([&] { return save_impl(path, quantized_format != 0, entries, count, gfh::as_stream(stream)); });
}

}  // extern "C"
