// Host runtime: the gfx950 code object, kernel launches, device buffers.
//
// One Device per GPU ordinal and process: it loads hbrocm_gfx950.hsaco
// (found beside libhbrocm.so) with hipModuleLoad, owns one HIP stream at
// the default priority, and launches kernels by name with a single
// by-value argument record (abi.h).
#pragma once
#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <cstring>
#include <functional>
#include <mutex>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

namespace hbr {

// Status codes of the C ABI (include/hessboost_rocm.h).
enum Status : int { kOk = 0, kRefused = 1, kDeviceError = 2, kInvalid = 3 };

struct Error : std::runtime_error {
    int status;
    Error(int s, const std::string &m) : std::runtime_error(m), status(s) {}
};

[[noreturn]] void fail(int status, const std::string &msg);
void check_hip(hipError_t e, const char *what);
#define HBR_HIP(call) ::hbr::check_hip((call), #call)

class Device {
public:
    explicit Device(int ordinal);
    ~Device();
    Device(const Device &) = delete;
    Device &operator=(const Device &) = delete;

    int ordinal() const { return ordinal_; }
    hipStream_t stream() const { return stream_; }
    int cu_count() const { return cu_count_; }
    // Make this device current on the calling thread.
    void activate() const;

    template <typename Args>
    void launch(const char *kernel, dim3 grid, dim3 block, const Args &args, uint32_t lds_bytes = 0) {
        launch_raw(kernel, grid, block, &args, lds_bytes);
    }
    void sync();

    // Kernel timing with HIP events on this device's stream (off by default):
    // only kernels whose name starts with `prefix` (every kernel when empty).
    // every: 0 off; N >= 1 times every N-th launch of the kernels whose name
    // starts with prefix (all of them are counted)
    void set_profiling(uint32_t every, const std::string &prefix = "");
    struct KernelStat {
        double total_ms = 0.0;  // over the timed launches
        uint64_t launches = 0;  // timed
        uint64_t calls = 0;     // every matching launch while profiling
    };
    std::unordered_map<std::string, KernelStat> kernel_stats();
    void reset_stats();

    // Rows in host memory to the device in chunks of at most chunk_rows rows
    // (a multiple of 64): the host's threads copy a chunk from the caller's
    // pageable memory into one of two pinned staging buffers, a copy stream
    // moves it into one of two device buffers, and fn(device rows, first
    // row, rows) queues the chunk's work on stream() while the next chunk is
    // staged; events order each buffer's reuse. Returns once the last chunk
    // is copied (the queued work may still run). The buffers are the
    // device's, kept until the process ends; one caller at a time.
    void host_rows(const float *x, uint64_t n, uint64_t n_cols, uint64_t chunk_rows,
                   const std::function<void(const float *, uint64_t, uint64_t)> &fn);

private:
    void launch_raw(const char *kernel, dim3 grid, dim3 block, const void *args, uint32_t lds_bytes);
    hipFunction_t function(const char *kernel);
    void drain_events();

    int ordinal_;
    int cu_count_ = 0;
    hipStream_t stream_ = nullptr;
    hipModule_t module_ = nullptr;
    std::unordered_map<std::string, hipFunction_t> functions_;
    uint32_t profile_every_ = 0;
    uint64_t profile_seen_ = 0;
    std::string profile_prefix_;
    struct Pending {
        std::string name;
        hipEvent_t start, stop;
    };
    std::vector<Pending> pending_;
    std::vector<hipEvent_t> event_pool_;
    hipEvent_t take_event();
    std::unordered_map<std::string, KernelStat> stats_;
    // host_rows' staging
    std::mutex pipe_mu_;
    hipStream_t pipe_copy_ = nullptr;
    hipEvent_t pipe_copied_[2] = {nullptr, nullptr};  // a chunk's copy has read its staging buffer
    hipEvent_t pipe_used_[2] = {nullptr, nullptr};    // the queued work has read a device buffer
    void *pipe_stage_[2] = {nullptr, nullptr};
    float *pipe_rows_[2] = {nullptr, nullptr};
    bool pipe_used_set_[2] = {false, false};
    uint64_t pipe_bytes_ = 0;
};

// The process's Device for an ordinal (created on first use).
Device &device(int ordinal);
int device_count();

// A typed device allocation.
template <typename T>
class DBuf {
public:
    DBuf() = default;
    explicit DBuf(size_t n) { resize(n); }
    ~DBuf() { release(); }
    DBuf(const DBuf &) = delete;
    DBuf &operator=(const DBuf &) = delete;
    DBuf(DBuf &&o) noexcept : p_(o.p_), n_(o.n_) {
        o.p_ = nullptr;
        o.n_ = 0;
    }
    DBuf &operator=(DBuf &&o) noexcept {
        if (this != &o) {
            release();
            p_ = o.p_;
            n_ = o.n_;
            o.p_ = nullptr;
            o.n_ = 0;
        }
        return *this;
    }
    void resize(size_t n) {
        if (n == n_) return;
        release();
        if (n) HBR_HIP(hipMalloc((void **)&p_, n * sizeof(T)));
        n_ = n;
    }
    // Grow to at least n elements (contents not kept).
    void reserve(size_t n) {
        if (n > n_) resize(n);
    }
    void release() {
        if (p_) (void)hipFree(p_);
        p_ = nullptr;
        n_ = 0;
    }
    T *get() const { return p_; }
    size_t size() const { return n_; }
    void upload(const T *src, size_t n, hipStream_t s, size_t at = 0) {
        if (n) HBR_HIP(hipMemcpyAsync(p_ + at, src, n * sizeof(T), hipMemcpyHostToDevice, s));
    }
    void download(T *dst, size_t n, hipStream_t s, size_t at = 0) const {
        if (n) HBR_HIP(hipMemcpyAsync(dst, p_ + at, n * sizeof(T), hipMemcpyDeviceToHost, s));
    }
    void zero(hipStream_t s) {
        if (n_) HBR_HIP(hipMemsetAsync(p_, 0, n_ * sizeof(T), s));
    }

private:
    T *p_ = nullptr;
    size_t n_ = 0;
};

// Page-locked host staging for the small per-level records, so their copies
// queue without blocking the host. Allocations bump through pinned blocks;
// nothing is reused until reset(), which the owner calls only after the
// stream has drained (every staged copy has completed).
class Stage {
public:
    Stage() = default;
    ~Stage();
    Stage(const Stage &) = delete;
    Stage &operator=(const Stage &) = delete;
    void *alloc(size_t bytes);
    void reset();

private:
    struct Block {
        void *p;
        size_t cap, used;
    };
    std::vector<Block> blocks_;
};

// Pinned host memory that outlives staging resets (a copy into it may still
// be queued when the owner resets its stage).
class PinnedBuf {
public:
    PinnedBuf() = default;
    ~PinnedBuf() {
        if (p_) (void)hipHostFree(p_);
    }
    PinnedBuf(const PinnedBuf &) = delete;
    PinnedBuf &operator=(const PinnedBuf &) = delete;
    // At least `bytes` (contents not kept); only while no copy uses it.
    void *reserve(size_t bytes) {
        if (bytes > n_) {
            if (p_) (void)hipHostFree(p_);
            p_ = nullptr;
            n_ = 0;
            HBR_HIP(hipHostMalloc(&p_, bytes, hipHostMallocDefault));
            n_ = bytes;
        }
        return p_;
    }
    void *get() const { return p_; }

private:
    void *p_ = nullptr;
    size_t n_ = 0;
};

// Grow `buf` (keeping nothing) and copy `v` into it through `stage`.
template <typename T>
void upload_vec(DBuf<T> &buf, const std::vector<T> &v, Stage &stage, hipStream_t s) {
    buf.reserve(v.size() ? v.size() : 1);
    if (v.empty()) return;
    void *p = stage.alloc(v.size() * sizeof(T));
    std::memcpy(p, v.data(), v.size() * sizeof(T));
    buf.upload(static_cast<const T *>(p), v.size(), s);
}

}  // namespace hbr
