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

// Exclusive scan of one value per thread over a workgroup of THREADS
// threads; every thread receives the workgroup total. All threads call it.
template <uint32_t THREADS>
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t *total) {
    __shared__ uint32_t wave_sums[THREADS / kWave];
    const uint32_t lane = lane_id(), wave = threadIdx.x / kWave;
    uint32_t x = v;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        uint32_t t = __shfl_up(x, d, kWave);
        if (lane >= (uint32_t)d) x += t;
    }
    if (lane == kWave - 1) wave_sums[wave] = x;
    __syncthreads();
    uint32_t base = 0, all = 0;
    for (uint32_t w = 0; w < THREADS / kWave; w++) {
        if (w < wave) base += wave_sums[w];
        all += wave_sums[w];
    }
    __syncthreads();
    *total = all;
    return base + x - v;
}

// f64 value of a fixed-point sum: k * 2^exp (the int64 -> f64 conversion
// rounds once, to nearest; the scaling is exact).
__device__ __forceinline__ double dequant(int64_t k, int32_t exp) {
    return __builtin_ldexp((double)k, exp);
}

}  // namespace hbr
