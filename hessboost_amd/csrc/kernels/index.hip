// Re-encoding a dense index on the device (the reference's CUDA backend does
// the same, src/backend/cuda/mod.rs:1687-1739): the caller's global bins
// become feature-local u8 bins in two layouts, row-major for histograms of
// gathered rows and feature-major for routing rows on one feature.
#include "common.h"

using namespace hbr;

extern "C" __global__ __launch_bounds__(256) void hbr_encode_dense(EncodeArgs a) {
    const uint64_t cells = (uint64_t)a.chunk_rows * a.n_cols;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < cells;
         i += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t r = a.row0 + i / a.n_cols;
        const uint32_t f = (uint32_t)(i % a.n_cols);
        const uint32_t gb = a.g16 ? (uint32_t)a.g16[i] : a.g32[i];
        const uint8_t local = (uint8_t)(gb - a.feature_offset[f]);
        a.rows8[r * a.stride + f] = local;
        a.cols8[(uint64_t)f * a.n_rows + r] = local;
    }
}

// Binning a dense f32 matrix on the device. bin = #{cuts <= v} over the
// feature's cuts (an upper bound), clamped to its last bin, as
// HistCuts::bin_of (src/data/quantile.rs:285-296) and the host's
// Cuts::bin_of compute it; a cell equal to the missing marker (any NaN when
// the marker is NaN) is absent: local bin 0 in the columns, its bit set in
// the missing bitmap, not counted. Cut values sit in LDS when they fit.
constexpr uint32_t kBinLdsCuts = 12288;

__device__ __forceinline__ uint32_t local_bin(const float *cuts, uint32_t nb, float v) {
    uint32_t lo = 0, n = nb;  // first index whose cut is > v
    while (n > 0) {
        const uint32_t half = n >> 1;
        if (!(v < cuts[lo + half])) {
            lo += half + 1;
            n -= half + 1;
        } else {
            n = half;
        }
    }
    return lo < nb ? lo : nb - 1;
}

extern "C" __global__ __launch_bounds__(256) void hbr_bin_dense(BinArgs a) {
    __shared__ float s_cuts[kBinLdsCuts];
    const bool in_lds = a.total_bins <= kBinLdsCuts;
    if (in_lds)
        for (uint32_t i = threadIdx.x; i < a.total_bins; i += blockDim.x) s_cuts[i] = a.cut_values[i];
    __syncthreads();
    const float *cuts = in_lds ? s_cuts : a.cut_values;
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;  // row within the chunk
    const bool active = i < a.chunk_rows;
    const uint64_t r = a.row0 + i;
    const float *row = a.x + (uint64_t)i * a.n_cols;
    uint32_t count = 0, mask = 0;
    for (uint32_t f0 = 0; f0 < a.n_cols; f0 += 4) {
        uint32_t word = 0;
#pragma unroll
        for (uint32_t q = 0; q < 4; q++) {
            const uint32_t f = f0 + q;
            if (f >= a.n_cols) break;  // uniform
            const float v = active ? row[f] : 0.0f;
            const bool absent = a.missing_is_nan ? __builtin_isnan(v) : v == a.missing_value;
            const uint32_t fs = a.feature_offset[f], nb = a.feature_offset[f + 1] - fs;
            const uint32_t local = absent || !active ? 0u : local_bin(cuts + fs, nb, v);
            word |= local << (8 * q);
            if (active) a.cols8[(uint64_t)f * a.n_rows + r] = (uint8_t)local;
            // a wave is 64 consecutive rows of one bitmap word
            const uint64_t miss = __ballot(active && absent);
            if (lane_id() == 0 && r < a.n_rows) a.missing[(uint64_t)f * a.words + (r >> 6)] = miss;
            count += active && !absent ? 1u : 0u;
            mask |= absent ? 1u << f : 0u;
        }
        if (active && a.rows8) *reinterpret_cast<uint32_t *>(a.rows8 + r * a.stride + f0) = word;
    }
    if (active && a.rows8 && a.row_mask)  // kept only when some cell is missing (else the word is padding)
        *reinterpret_cast<uint32_t *>(a.rows8 + r * a.stride + 4 * kMaskWord) = mask;
    if (active) a.row_count[r] = count;
}

// Per block of kCountBlock rows: the total of its counts.
extern "C" __global__ __launch_bounds__(1024) void hbr_count_blocks(CountScanArgs a) {
    const uint64_t base = (uint64_t)blockIdx.x * kCountBlock;
    unsigned long long sum = 0;
    for (uint32_t k = threadIdx.x; k < kCountBlock; k += blockDim.x)
        if (base + k < a.n_rows) sum += a.row_count[base + k];
    __shared__ unsigned long long red[1024 / kWave];
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) sum += __shfl_xor(sum, d, kWave);
    if (lane_id() == 0) red[threadIdx.x / kWave] = sum;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long t = 0;
        for (uint32_t w = 0; w < blockDim.x / kWave; w++) t += red[w];
        a.block_total[blockIdx.x] = t;
    }
}

// row_ptr[r + 1] = the block's offset + the inclusive count within the block.
extern "C" __global__ __launch_bounds__(1024) void hbr_count_offsets(CountScanArgs a) {
    const uint64_t base = (uint64_t)blockIdx.x * kCountBlock;
    __shared__ unsigned long long wave_sums[1024 / kWave];
    unsigned long long carry = a.block_offset[blockIdx.x];
    if (blockIdx.x == 0 && threadIdx.x == 0) a.row_ptr[0] = 0;
    for (uint32_t k0 = 0; k0 < kCountBlock; k0 += blockDim.x) {
        const uint64_t r = base + k0 + threadIdx.x;
        unsigned long long v = r < a.n_rows ? a.row_count[r] : 0ull;
        // inclusive wave scan, then across waves
        const uint32_t lane = lane_id(), w = threadIdx.x / kWave;
#pragma unroll
        for (int d = 1; d < kWave; d <<= 1) {
            const unsigned long long t = __shfl_up(v, d, kWave);
            if (lane >= (uint32_t)d) v += t;
        }
        if (lane == kWave - 1) wave_sums[w] = v;
        __syncthreads();
        unsigned long long before = 0, all = 0;
        for (uint32_t q = 0; q < blockDim.x / kWave; q++) {
            if (q < w) before += wave_sums[q];
            all += wave_sums[q];
        }
        __syncthreads();
        if (r < a.n_rows) a.row_ptr[r + 1] = carry + before + v;
        carry += all;
    }
}

extern "C" __global__ __launch_bounds__(256) void hbr_csr_fill(CsrFillArgs a) {
    const uint64_t r = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= a.n_rows) return;
    uint64_t e = a.row_ptr[r];
    for (uint32_t f = 0; f < a.n_cols; f++) {
        const bool absent = (a.missing[(uint64_t)f * a.words + (r >> 6)] >> (r & 63)) & 1ull;
        if (!absent) a.gbins[e++] = a.feature_offset[f] + a.cols8[(uint64_t)f * a.n_rows + r];
    }
}
