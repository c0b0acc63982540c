#include "runtime.h"

// hip_ext.h's launch with timing events (its own templates need a HIP
// compiler; this file is built by the host compiler)
extern "C" hipError_t hipExtModuleLaunchKernel(hipFunction_t f, uint32_t globalWorkSizeX, uint32_t globalWorkSizeY,
                                               uint32_t globalWorkSizeZ, uint32_t localWorkSizeX,
                                               uint32_t localWorkSizeY, uint32_t localWorkSizeZ, size_t sharedMemBytes,
                                               hipStream_t hStream, void **kernelParams, void **extra,
                                               hipEvent_t startEvent, hipEvent_t stopEvent, uint32_t flags);

#include <dlfcn.h>
#include <omp.h>
#include <algorithm>
#include <cstdlib>

#include <memory>

namespace hbr {

void fail(int status, const std::string &msg) { throw Error(status, msg); }

void check_hip(hipError_t e, const char *what) {
    if (e != hipSuccess) fail(kDeviceError, std::string(what) + ": " + hipGetErrorString(e));
}

// The code object sits beside this library: <dir of libhbrocm.so>/hbrocm_gfx950.hsaco.
static std::string code_object_path() {
    Dl_info info;
    if (dladdr((void *)&code_object_path, &info) && info.dli_fname) {
        std::string so = info.dli_fname;
        auto slash = so.rfind('/');
        std::string dir = slash == std::string::npos ? "." : so.substr(0, slash);
        return dir + "/hbrocm_gfx950.hsaco";
    }
    return "hbrocm_gfx950.hsaco";
}

Device::Device(int ordinal) : ordinal_(ordinal) {
    int count = 0;
    HBR_HIP(hipGetDeviceCount(&count));
    if (ordinal < 0 || ordinal >= count)
        fail(kInvalid, "no ROCm device with ordinal " + std::to_string(ordinal));
    HBR_HIP(hipSetDevice(ordinal));
    hipDeviceProp_t prop;
    HBR_HIP(hipGetDeviceProperties(&prop, ordinal));
    if (std::string(prop.gcnArchName).rfind("gfx950", 0) != 0)
        fail(kRefused, std::string("device is ") + prop.gcnArchName + ", the code object is gfx950");
    cu_count_ = prop.multiProcessorCount;
    HBR_HIP(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));
    std::string path = code_object_path();
    hipError_t e = hipModuleLoad(&module_, path.c_str());
    if (e != hipSuccess) fail(kDeviceError, "hipModuleLoad(" + path + "): " + hipGetErrorString(e));
    // the kernels' argument records must be the ones this library fills
    hipDeviceptr_t stamp_ptr = nullptr;
    size_t stamp_size = 0;
    e = hipModuleGetGlobal(&stamp_ptr, &stamp_size, module_, "hbr_abi_stamp");
    if (e != hipSuccess || stamp_size != sizeof(uint32_t))
        fail(kDeviceError, path + " carries no argument-layout stamp: rebuild hessboost_amd/csrc");
    uint32_t stamp = 0;
    HBR_HIP(hipMemcpy(&stamp, stamp_ptr, sizeof(stamp), hipMemcpyDeviceToHost));
    if (stamp != HBR_ABI_STAMP)
        fail(kDeviceError, path + " was built from a different abi.h than libhbrocm.so: rebuild hessboost_amd/csrc");
}

Device::~Device() {
    if (stream_) (void)hipStreamSynchronize(stream_);
    if (pipe_copy_) {
        (void)hipStreamSynchronize(pipe_copy_);
        for (int b = 0; b < 2; b++) {
            (void)hipEventDestroy(pipe_copied_[b]);
            (void)hipEventDestroy(pipe_used_[b]);
            if (pipe_stage_[b]) (void)hipHostFree(pipe_stage_[b]);
            if (pipe_rows_[b]) (void)hipFree(pipe_rows_[b]);
        }
        (void)hipStreamDestroy(pipe_copy_);
    }
    for (auto &p : pending_) {
        (void)hipEventDestroy(p.start);
        (void)hipEventDestroy(p.stop);
    }
    for (auto e : event_pool_) (void)hipEventDestroy(e);
    if (module_) (void)hipModuleUnload(module_);
    if (stream_) (void)hipStreamDestroy(stream_);
}

void Device::activate() const { HBR_HIP(hipSetDevice(ordinal_)); }

hipFunction_t Device::function(const char *kernel) {
    auto it = functions_.find(kernel);
    if (it != functions_.end()) return it->second;
    hipFunction_t f;
    hipError_t e = hipModuleGetFunction(&f, module_, kernel);
    if (e != hipSuccess) fail(kDeviceError, std::string("kernel ") + kernel + " not in the code object");
    functions_.emplace(kernel, f);
    return f;
}

void Device::launch_raw(const char *kernel, dim3 grid, dim3 block, const void *args, uint32_t lds_bytes) {
    if (grid.x == 0 || grid.y == 0 || grid.z == 0) return;
    hipFunction_t f = function(kernel);
    // one by-value struct parameter: its address is the parameter's
    void *params[] = {const_cast<void *>(args)};
    bool timed = false;
    if (profile_every_ && std::strncmp(kernel, profile_prefix_.c_str(), profile_prefix_.size()) == 0) {
        // a sample of the launches: the events' own stalls stay out of the rest
        stats_[kernel].calls++;
        timed = profile_seen_++ % profile_every_ == 0;
    }
    if (!timed) {
        HBR_HIP(hipModuleLaunchKernel(f, grid.x, grid.y, grid.z, block.x, block.y, block.z, lds_bytes, stream_,
                                      params, nullptr));
        return;
    }
    // the runtime records the pair of events with the dispatch's own begin
    // and end timestamps (the kernel's duration, as a kernel trace has it),
    // not as separate queue entries around the dispatch
    Pending ev{};
    ev.start = take_event();
    ev.stop = take_event();
    HBR_HIP(hipExtModuleLaunchKernel(f, grid.x * block.x, grid.y * block.y, grid.z * block.z, block.x, block.y,
                                     block.z, lds_bytes, stream_, params, nullptr, ev.start, ev.stop, 0));
    ev.name = kernel;
    pending_.push_back(ev);
}

hipEvent_t Device::take_event() {
    if (!event_pool_.empty()) {
        hipEvent_t e = event_pool_.back();
        event_pool_.pop_back();
        return e;
    }
    // timing events without the system-scope fence a plain event adds (the
    // fence stalls the stream around every timed kernel)
    static const bool fence = [] {
        const char *v = std::getenv("HBROCM_EVENT_FENCE");
        return v && std::strtol(v, nullptr, 10) != 0;
    }();
    hipEvent_t e;
    HBR_HIP(hipEventCreateWithFlags(&e, fence ? hipEventDefault : hipEventDisableSystemFence));
    return e;
}

void Device::sync() {
    HBR_HIP(hipStreamSynchronize(stream_));
    if (!pending_.empty()) drain_events();
}

void Device::drain_events() {
    for (auto &p : pending_) {
        float ms = 0.0f;
        HBR_HIP(hipEventElapsedTime(&ms, p.start, p.stop));
        auto &s = stats_[p.name];
        s.total_ms += ms;
        s.launches++;
        event_pool_.push_back(p.start);
        event_pool_.push_back(p.stop);
    }
    pending_.clear();
}

void Device::set_profiling(uint32_t every, const std::string &prefix) {
    sync();
    if (every) stats_.clear();
    profile_every_ = every;
    profile_seen_ = 0;
    profile_prefix_ = prefix;
}

std::unordered_map<std::string, Device::KernelStat> Device::kernel_stats() {
    sync();
    return stats_;
}

void Device::reset_stats() {
    sync();
    stats_.clear();
}

// Pageable host bytes into pinned memory with the host's threads (one
// thread's memcpy reaches a fraction of the link's rate). The thread count
// is the processors', whatever the process last set for its own parallel
// regions.
static void copy_threads(void *dst, const void *src, uint64_t bytes) {
    constexpr uint64_t kPiece = 4ull << 20;
    const int64_t pieces = (int64_t)((bytes + kPiece - 1) / kPiece);
    const int threads = std::max(1, std::min(32, omp_get_num_procs()));
#pragma omp parallel for schedule(static) num_threads(threads)
    for (int64_t i = 0; i < pieces; i++) {
        const uint64_t off = (uint64_t)i * kPiece;
        std::memcpy(static_cast<char *>(dst) + off, static_cast<const char *>(src) + off,
                    std::min<uint64_t>(kPiece, bytes - off));
    }
}

void Device::host_rows(const float *x, uint64_t n, uint64_t n_cols, uint64_t chunk_rows,
                       const std::function<void(const float *, uint64_t, uint64_t)> &fn) {
    if (n == 0) return;
    if (chunk_rows == 0 || chunk_rows % 64) fail(kInvalid, "host rows: chunks of a multiple of 64 rows");
    std::lock_guard<std::mutex> lock(pipe_mu_);
    const uint64_t row_bytes = n_cols * sizeof(float);
    const uint64_t bytes = std::min(chunk_rows, n) * row_bytes;
    if (!pipe_copy_) {
        HBR_HIP(hipStreamCreateWithFlags(&pipe_copy_, hipStreamNonBlocking));
        for (int b = 0; b < 2; b++) {
            HBR_HIP(hipEventCreateWithFlags(&pipe_copied_[b], hipEventDisableTiming));
            HBR_HIP(hipEventCreateWithFlags(&pipe_used_[b], hipEventDisableTiming));
        }
    }
    // a call that ended early (its work refused) may have left a copy
    // reading a staging buffer
    HBR_HIP(hipStreamSynchronize(pipe_copy_));
    if (bytes > pipe_bytes_) {  // nothing in flight uses the old buffers (the last call waited for its copies)
        sync();
        for (int b = 0; b < 2; b++) {
            if (pipe_stage_[b]) (void)hipHostFree(pipe_stage_[b]);
            if (pipe_rows_[b]) (void)hipFree(pipe_rows_[b]);
            pipe_stage_[b] = nullptr;
            pipe_rows_[b] = nullptr;
        }
        pipe_bytes_ = 0;
        for (int b = 0; b < 2; b++) {
            HBR_HIP(hipHostMalloc(&pipe_stage_[b], bytes, hipHostMallocDefault));
            HBR_HIP(hipMalloc((void **)&pipe_rows_[b], bytes));
        }
        pipe_bytes_ = bytes;
    }
    const uint64_t chunks = (n + chunk_rows - 1) / chunk_rows;
    for (uint64_t c = 0; c < chunks; c++) {
        const int b = (int)(c & 1u);
        const uint64_t r0 = c * chunk_rows, rows = std::min(chunk_rows, n - r0);
        // the copy two chunks back has read this staging buffer, and the
        // work last queued on this device buffer has read it
        if (c >= 2) HBR_HIP(hipEventSynchronize(pipe_copied_[b]));
        copy_threads(pipe_stage_[b], x + r0 * n_cols, rows * row_bytes);
        // (an earlier call's last chunks count: their work may still run)
        if (pipe_used_set_[b]) HBR_HIP(hipStreamWaitEvent(pipe_copy_, pipe_used_[b], 0));
        HBR_HIP(hipMemcpyAsync(pipe_rows_[b], pipe_stage_[b], rows * row_bytes, hipMemcpyHostToDevice, pipe_copy_));
        HBR_HIP(hipEventRecord(pipe_copied_[b], pipe_copy_));
        HBR_HIP(hipStreamWaitEvent(stream_, pipe_copied_[b], 0));
        fn(pipe_rows_[b], r0, rows);
        HBR_HIP(hipEventRecord(pipe_used_[b], stream_));
        pipe_used_set_[b] = true;
    }
    HBR_HIP(hipStreamSynchronize(pipe_copy_));
}

static std::mutex g_devices_mu;
static std::unordered_map<int, std::unique_ptr<Device>> g_devices;

Device &device(int ordinal) {
    std::lock_guard<std::mutex> lock(g_devices_mu);
    auto it = g_devices.find(ordinal);
    if (it != g_devices.end()) {
        it->second->activate();
        return *it->second;
    }
    auto d = std::make_unique<Device>(ordinal);
    Device &ref = *d;
    g_devices.emplace(ordinal, std::move(d));
    return ref;
}

int device_count() {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

Stage::~Stage() {
    for (auto &b : blocks_) (void)hipHostFree(b.p);
}

void *Stage::alloc(size_t bytes) {
    bytes = (bytes + 255) & ~size_t(255);
    for (auto &b : blocks_) {
        if (b.cap - b.used >= bytes) {
            void *p = static_cast<char *>(b.p) + b.used;
            b.used += bytes;
            return p;
        }
    }
    size_t cap = bytes > (size_t(1) << 20) ? bytes : (size_t(1) << 20);
    void *p = nullptr;
    HBR_HIP(hipHostMalloc(&p, cap, hipHostMallocDefault));
    blocks_.push_back({p, cap, bytes});
    return p;
}

void Stage::reset() {
    for (auto &b : blocks_) b.used = 0;
}

}  // namespace hbr
