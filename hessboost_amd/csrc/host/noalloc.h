// The fixed per-device scratch of the entry points that allocate nothing.
#pragma once
#include <cstdint>

namespace hbr {
// Device address and size of the library's fixed scratch array on device
// `ordinal`, which must be current on the calling thread. The address is
// resolved on the first call for the device and kept; every call on one
// device shares the same memory, which keeps the last call's contents.
uint8_t *fixed_scratch(int ordinal, uint64_t *bytes);
}  // namespace hbr
