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

// Dense indexes with a feature of more than 256 bins: the global bins of
// the index's dense CSR rows (row r's entries at r * n_cols, in feature
// order) to rows of u16 local bins, zero beyond n_cols.
extern "C" __global__ __launch_bounds__(256) void hbr_encode_dense16(Encode16Args a) {
    const uint64_t cells = a.n_rows * a.stride16;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < cells;
         i += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t r = i / a.stride16;
        const uint32_t f = (uint32_t)(i % a.stride16);
        a.rows16[i] = f < a.n_cols ? (uint16_t)(a.gbins[r * a.n_cols + f] - a.feature_offset[f]) : (uint16_t)0;
    }
}

// Binning a dense f32 matrix on the device. bin = #{cuts <= v} over the
// feature's cuts (an upper bound), clamped to its last bin, as
// HistCuts::bin_of (src/data/quantile.rs:285-296) and the host's
// Cuts::bin_of compute it; a cell equal to the missing marker (any NaN when
// the marker is NaN) is absent: local bin 0 in the columns, its bit set in
// the missing bitmap, not counted. Cut values sit in LDS when they fit
// (kBinLdsCuts).

// A cell's local bin: the first index whose cut is > v (a binary search
// whose probes follow the host's Cuts::bin_of exactly: a feature whose
// present values include NaN ends its cuts with NaN, which every probe
// treats as <= v), clamped to the feature's last bin. At most 256 cuts (the
// host refuses more) take at most 9 halvings, so the search is unrolled to
// 9 predicated steps: no loop, and the searches of several features
// interleave.
__device__ __forceinline__ uint32_t local_bin256(const float *cuts, uint32_t nb, float v) {
    uint32_t lo = 0, n = nb;
#pragma unroll
    for (int step = 0; step < 9; step++) {
        const uint32_t half = n >> 1;
        const float c = cuts[min(lo + half, nb - 1)];  // lo + half < nb while n > 0
        const bool right = n > 0 && !(v < c);
        lo = right ? lo + half + 1 : lo;
        n = right ? n - half - 1 : half;
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
            const uint32_t local = absent || !active ? 0u : local_bin256(cuts + fs, nb, v);
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

// hbr_bin_dense for 32 features or fewer and 32-byte rows, writing every
// 32-byte u8 row whole (padding zero, or the missing mask when a.row_mask)
// as two 16-byte stores. STAGED: each wave copies its 64 rows (contiguous
// f32) into LDS with 16-byte loads, so that the reads are coalesced, and
// every lane bins its own row from LDS; otherwise (n_cols a multiple of 4)
// every lane reads its own row with 16-byte loads into registers. Dynamic
// LDS: the cut values (total_bins <= kBinLdsCuts, checked by the host), then
// (STAGED) 4 waves x 64 rows x n_cols floats.
template <bool STAGED>
__device__ __forceinline__ void bin_dense32(const BinArgs &a) {
    extern __shared__ float s_lds[];
    __shared__ uint32_t s_fo[33];
    const uint32_t F = a.n_cols;  // <= 32
    const uint32_t lane = lane_id(), wave = threadIdx.x / kWave;
    float *s_cuts = s_lds;
    for (uint32_t i = threadIdx.x; i < a.total_bins; i += blockDim.x) s_cuts[i] = a.cut_values[i];
    if (threadIdx.x <= F) s_fo[threadIdx.x] = a.feature_offset[threadIdx.x];
    const uint32_t w0 = blockIdx.x * blockDim.x + wave * kWave;  // the wave's first row in the chunk
    const uint32_t rows = w0 < a.chunk_rows ? min(kWave, a.chunk_rows - w0) : 0u;
    const bool active = lane < rows;
    float xv[32];
    const float *row = nullptr;
    if (STAGED) {
        float *s_rows = s_lds + a.total_bins + wave * (kWave * F);
        const float *src = a.x + (uint64_t)w0 * F;  // 256-byte aligned: w0 is a multiple of 64
        const uint32_t total = rows * F;
        for (uint32_t i = 4 * lane; i < total; i += 4 * kWave) {
            if (i + 4 <= total) {
                const float4 v = *reinterpret_cast<const float4 *>(src + i);
                s_rows[i] = v.x;
                s_rows[i + 1] = v.y;
                s_rows[i + 2] = v.z;
                s_rows[i + 3] = v.w;
            } else {
                for (uint32_t k = i; k < total; k++) s_rows[k] = src[k];
            }
        }
        row = s_rows + lane * F;
    } else {
        const float4 *src = reinterpret_cast<const float4 *>(a.x + (uint64_t)(w0 + lane) * F);
#pragma unroll
        for (uint32_t q = 0; q < 8; q++) {
            float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (4 * q < F && active) v = src[q];
            xv[4 * q] = v.x;
            xv[4 * q + 1] = v.y;
            xv[4 * q + 2] = v.z;
            xv[4 * q + 3] = v.w;
        }
    }
    __syncthreads();
    const uint64_t r = a.row0 + w0 + lane;
    uint32_t w[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
    uint32_t count = 0, mask = 0;
#pragma unroll
    for (uint32_t f = 0; f < 32; f++) {
        if (f >= F) continue;  // uniform; the loop unrolls, so w[] stays in registers
        const float v = !active ? 0.0f : STAGED ? row[f] : xv[f];
        const bool absent = a.missing_is_nan ? __builtin_isnan(v) : v == a.missing_value;
        const uint32_t fs = s_fo[f], nb = s_fo[f + 1] - fs;
        const uint32_t local = absent || !active ? 0u : local_bin256(s_cuts + fs, nb, v);
        w[f >> 2] |= local << (8 * (f & 3u));
        if (active) a.cols8[(uint64_t)f * a.n_rows + r] = (uint8_t)local;
        // a wave is 64 consecutive rows of one bitmap word
        const uint64_t miss = __ballot(active && absent);
        if (lane == 0 && rows > 0) a.missing[(uint64_t)f * a.words + (r >> 6)] = miss;
        count += active && !absent ? 1u : 0u;
        mask |= absent ? 1u << f : 0u;
    }
    if (a.row_mask) w[kMaskWord] = mask;  // kept only when some cell is missing (else the word is padding)
    if (active) {
        uint4 *dst = reinterpret_cast<uint4 *>(a.rows8 + r * 32u);
        dst[0] = make_uint4(w[0], w[1], w[2], w[3]);
        dst[1] = make_uint4(w[4], w[5], w[6], w[7]);
        a.row_count[r] = count;
    }
}

extern "C" __global__ __launch_bounds__(256) void hbr_bin_dense32(BinArgs a) { bin_dense32<true>(a); }
extern "C" __global__ __launch_bounds__(256) void hbr_bin_dense32_rows(BinArgs a) { bin_dense32<false>(a); }

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
