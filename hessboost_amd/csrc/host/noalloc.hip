// The library's fixed device scratch for the entry points that allocate
// nothing (hbr_build_device_noalloc). One file-scope device array: each GPU
// the library runs on holds its own copy from the first call on it until
// the process ends. Host code never passes the array's name to a kernel or
// a copy (on the host it is only a stand-in for the symbol); it uses the
// device address hipGetSymbolAddress returns, resolved once per device with
// that device current, and kept per device.
#include <hip/hip_runtime.h>

#include <mutex>

#include "noalloc.h"
#include "runtime.h"

// 128 KiB for the row-check word, the node record and the tile plan, then
// 32 MiB of tile partial sums (one tile of 32 features x 256 bins of int64
// pairs takes 128 KiB: 256 such tiles).
static constexpr size_t kScratchBytes = (32u << 20) + (128u << 10);
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace hbr {

namespace {
constexpr int kMaxOrdinals = 64;
std::mutex g_mu;
void *g_addr[kMaxOrdinals] = {};
std::mutex g_use[kMaxOrdinals];  // one holder of a device's scratch at a time
}  // namespace

std::unique_lock<std::mutex> fixed_scratch_lock(int ordinal) {
    if (ordinal < 0 || ordinal >= kMaxOrdinals) fail(kInvalid, "fixed scratch: device ordinal out of range");
    return std::unique_lock<std::mutex>(g_use[ordinal]);
}

uint8_t *fixed_scratch(int ordinal, uint64_t *bytes) {
    if (ordinal < 0 || ordinal >= kMaxOrdinals) fail(kInvalid, "fixed scratch: device ordinal out of range");
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_addr[ordinal]) {
        int current = -1;
        HBR_HIP(hipGetDevice(&current));
        if (current != ordinal) fail(kInvalid, "fixed scratch: resolve it with its device current");
        void *p = nullptr;
        HBR_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) fail(kDeviceError, "fixed scratch: no device address");
        g_addr[ordinal] = p;
    }
    *bytes = kScratchBytes;
    return static_cast<uint8_t *>(g_addr[ordinal]);
}

}  // namespace hbr
