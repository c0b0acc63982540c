// Stable row partition of a whole level of splits by prefix-sum compaction.
//
// Replaces partition_rows (builder/partition.rs:106-242) for every split of a
// level at once: a present local bin of the split feature below `limit`
// goes left, a missing value follows default_left, and both children keep
// the parent's ascending row order (left child first in the segment).
//
// Three passes over fixed tiles of kPartTile rows: count the left rows of
// each tile, scan the tile counts of each split (which also fixes each
// child's length and which child is the smaller, built one), then scatter
// every row to its stable position in the other row buffer.
#include "common.h"

namespace hbr {

constexpr uint32_t kRowsPerThread = kPartTile / kPartThreads;  // 8

__device__ __forceinline__ bool goes_left(const PartArgs &a, const PartSplit &sp, uint32_t r) {
    if (a.dense) {
        const size_t at = (size_t)sp.feature * a.n_rows + r;
        if (a.missing) {
            const uint64_t word = a.missing[(size_t)sp.feature * a.words + (r >> 6)];
            if ((word >> (r & 63)) & 1ull) return sp.default_left != 0;
        }
        const uint32_t local = a.cols8 ? (uint32_t)a.cols8[at] : (uint32_t)a.cols16[at];
        return local < sp.limit;
    }
    const uint32_t fs = a.feature_offset[sp.feature], fe = a.feature_offset[sp.feature + 1];
    for (uint64_t e = a.row_ptr[r]; e < a.row_ptr[r + 1]; e++) {
        const uint32_t gb = a.gbins[e];
        if (gb >= fs && gb < fe) return gb - fs < sp.limit;
    }
    return sp.default_left != 0;
}

// Exclusive block scan of one value per thread (kPartThreads threads).
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t *total) {
    __shared__ uint32_t wave_sums[kPartThreads / kWave];
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
    for (uint32_t w = 0; w < kPartThreads / kWave; w++) {
        if (w < wave) base += wave_sums[w];
        all += wave_sums[w];
    }
    __syncthreads();
    *total = all;
    return base + x - v;
}

}  // namespace hbr

using namespace hbr;

extern "C" __global__ __launch_bounds__(256) void hbr_part_count(PartArgs a) {
    const uint32_t tile = blockIdx.x;
    if (tile >= a.n_tiles) return;
    const PartSplit sp = a.splits[a.tile_split[tile]];
    const uint32_t base = (tile - sp.tile_begin) * kPartTile;
    const uint32_t *src = a.src_rows[sp.seg.buf] + sp.seg.offset;
    uint32_t cnt = 0;
#pragma unroll
    for (uint32_t k = 0; k < kRowsPerThread; k++) {
        const uint32_t j = base + threadIdx.x * kRowsPerThread + k;
        if (j < sp.seg.len) cnt += goes_left(a, sp, src[j]) ? 1u : 0u;
    }
    uint32_t total;
    block_exclusive_scan(cnt, &total);
    if (threadIdx.x == 0) a.tile_left[tile] = total;
}

// One workgroup per split: exclusive scan of its tiles' left counts.
extern "C" __global__ __launch_bounds__(256) void hbr_part_scan(PartArgs a) {
    const uint32_t s = blockIdx.x;
    if (s >= a.n_splits) return;
    const PartSplit sp = a.splits[s];
    const uint32_t n_tiles = (sp.seg.len + kPartTile - 1) / kPartTile;
    uint32_t carry = 0;
    for (uint32_t t0 = 0; t0 < n_tiles; t0 += kPartThreads) {
        const uint32_t t = t0 + threadIdx.x;
        const uint32_t v = t < n_tiles ? a.tile_left[sp.tile_begin + t] : 0u;
        uint32_t total;
        const uint32_t ex = block_exclusive_scan(v, &total);
        if (t < n_tiles) a.tile_left[sp.tile_begin + t] = carry + ex;
        carry += total;
    }
    if (threadIdx.x == 0) {
        PartOut o;
        o.left_len = carry;
        o.built_left = carry <= sp.seg.len - carry ? 1u : 0u;
        o.pad[0] = o.pad[1] = 0;
        a.out[s] = o;
    }
}

extern "C" __global__ __launch_bounds__(256) void hbr_part_scatter(PartArgs a) {
    const uint32_t tile = blockIdx.x;
    if (tile >= a.n_tiles) return;
    const uint32_t s = a.tile_split[tile];
    const PartSplit sp = a.splits[s];
    const uint32_t left_len = a.out[s].left_len;
    const uint32_t tile_pos = (tile - sp.tile_begin) * kPartTile;
    const uint32_t left_before = a.tile_left[tile];
    const uint32_t right_before = tile_pos - left_before;
    const uint32_t *src = a.src_rows[sp.seg.buf] + sp.seg.offset;
    uint32_t *dst = a.dst_rows[sp.seg.buf ^ 1u] + sp.seg.offset;
    uint32_t row[kRowsPerThread];
    uint32_t flags = 0, nl = 0, nr = 0;
#pragma unroll
    for (uint32_t k = 0; k < kRowsPerThread; k++) {
        const uint32_t j = tile_pos + threadIdx.x * kRowsPerThread + k;
        row[k] = 0;
        if (j < sp.seg.len) {
            row[k] = src[j];
            if (goes_left(a, sp, row[k])) {
                flags |= 1u << k;
                nl++;
            } else {
                nr++;
            }
        }
    }
    uint32_t tl, tr;
    uint32_t lpos = block_exclusive_scan(nl, &tl);
    uint32_t rpos = block_exclusive_scan(nr, &tr);
#pragma unroll
    for (uint32_t k = 0; k < kRowsPerThread; k++) {
        const uint32_t j = tile_pos + threadIdx.x * kRowsPerThread + k;
        if (j >= sp.seg.len) continue;
        if ((flags >> k) & 1u)
            dst[left_before + lpos++] = row[k];
        else
            dst[left_len + right_before + rpos++] = row[k];
    }
}

// Leaf values onto the margins of each leaf's rows (training/margins.rs:247-289,
// one f32 add per row per tree).
extern "C" __global__ __launch_bounds__(256) void hbr_add_leaves(LeafArgs a) {
    const uint32_t tile = blockIdx.x;
    if (tile >= a.n_tiles) return;
    const LeafSeg lf = a.leaves[a.tile_leaf[tile]];
    const uint32_t row0 = a.tile_row0[tile];
    const uint32_t end = min(row0 + a.tile_rows, lf.seg.len);
    const uint32_t *rows = a.rows[lf.seg.buf] + lf.seg.offset;
    for (uint32_t j = row0 + threadIdx.x; j < end; j += blockDim.x) {
        const uint32_t r = rows[j];
        float *m = a.margins + (size_t)r * a.stride + a.output;
        *m = *m + lf.value;
    }
}
