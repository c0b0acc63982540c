// The fixed per-device scratch of the entry points that allocate nothing.
#pragma once
#include <cstdint>
#include <mutex>

namespace hbr {
// Device address and size of the library's fixed scratch array on device
// `ordinal`, which must be current on the calling thread. The address is
// resolved on the first call for the device and kept; every call on one
// device shares the same memory, which keeps the last call's contents.
uint8_t *fixed_scratch(int ordinal, uint64_t *bytes);
// Held for the whole of a call that uses device `ordinal`'s scratch, so that
// calls from several threads (engines sharing one GPU) take it in turn.
std::unique_lock<std::mutex> fixed_scratch_lock(int ordinal);
}  // namespace hbr
