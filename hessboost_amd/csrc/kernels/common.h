// Device helpers shared by the gfx950 kernels (wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../abi.h"

namespace hbr {

constexpr int kWave = 64;

__device__ __forceinline__ uint32_t lane_id() { return __lane_id(); }

// rint(x * 2^-exp) as an integer; |result| <= 2^62 for every value the
// exponent was chosen for. The power-of-two scaling is exact in f32.
__device__ __forceinline__ int64_t quantize(float x, int32_t exp) {
    float s = __builtin_ldexpf(x, -exp);
    float r = __builtin_rintf(s);
    return (int64_t)r;
}

// Wave-wide inclusive prefix sum of a 64-bit integer.
__device__ __forceinline__ int64_t wave_inclusive_scan(int64_t v) {
    const uint32_t lane = lane_id();
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        int64_t t = __shfl_up(v, d, kWave);
        if (lane >= (uint32_t)d) v += t;
    }
    return v;
}

__device__ __forceinline__ int64_t wave_broadcast(int64_t v, int src) { return __shfl(v, src, kWave); }

// f64 value of a fixed-point sum: k * 2^exp (the int64 -> f64 conversion
// rounds once, to nearest; the scaling is exact).
__device__ __forceinline__ double dequant(int64_t k, int32_t exp) {
    return __builtin_ldexp((double)k, exp);
}

}  // namespace hbr
