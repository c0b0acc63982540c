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
