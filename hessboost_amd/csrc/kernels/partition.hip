// Stable row partition of a whole level of splits by prefix-sum compaction.
//
// Replaces partition_rows (builder/partition.rs:106-242) for every split of a
// level at once: a present local bin of the split feature below `limit`
// (for a categorical split: whose bit is set in its table) goes left, a
// missing value follows default_left, and both children keep the parent's
// ascending row order (left child first in the segment).
//
// Three passes over fixed tiles of kPartTile rows: count the left rows of
// each tile (keeping each wave's 64-row ballot of decisions), scan the tile
// counts of each split (which also fixes each child's length and which
// child is the smaller, built one), then scatter every row to its stable
// position in the other row buffer from the ballots, without routing it
// again. Row j of a tile is handled by lane j % 64 of ballot j / 64.
#include "common.h"

namespace hbr {

constexpr uint32_t kRowsPerThread = kPartTile / kPartThreads;  // 8
constexpr uint32_t kBallots = kPartTile / kWave;                // 32 per tile

// A present row's direction from its local bin: below the limit, or, for a
// categorical split (RowRule::Table, src/tree/hist/mod.rs:173-178), the
// bin's bit in the split's table (local bins of a categorical feature are
// below kCatMaxBins).
__device__ __forceinline__ bool present_left(const PartArgs &a, const PartSplit &sp, uint32_t local) {
    if (sp.table) return (a.cat_tables[(size_t)(sp.table - 1u) * kCatWords + (local >> 5)] >> (local & 31u)) & 1u;
    return local < sp.limit;
}

__device__ __forceinline__ bool goes_left(const PartArgs &a, const PartSplit &sp, uint32_t r) {
    if (a.dense) {
        const size_t at = (size_t)sp.feature * a.n_rows + r;
        if (a.missing) {
            const uint64_t word = a.missing[(size_t)sp.feature * a.words + (r >> 6)];
            if ((word >> (r & 63)) & 1ull) return sp.default_left != 0;
        }
        const uint32_t local = a.cols8 ? (uint32_t)a.cols8[at] : (uint32_t)a.cols16[at];
        return present_left(a, sp, local);
    }
    // a row's global bins ascend (its entries are in feature order, and a
    // feature's bins follow the previous feature's): the first bin >= fs,
    // by binary search, is the feature's entry if it lies below fe
    const uint32_t fs = a.feature_offset[sp.feature], fe = a.feature_offset[sp.feature + 1];
    if (!a.csr_ascending) {  // entries in the caller's order: scan them
        for (uint64_t e = a.row_ptr[r]; e < a.row_ptr[r + 1]; e++) {
            const uint32_t gb = a.gbins[e];
            if (gb >= fs && gb < fe) return present_left(a, sp, gb - fs);
        }
        return sp.default_left != 0;
    }
    uint64_t lo = a.row_ptr[r], hi = a.row_ptr[r + 1];
    while (lo < hi) {
        const uint64_t mid = lo + (hi - lo) / 2;
        if (a.gbins[mid] < fs) lo = mid + 1;
        else hi = mid;
    }
    if (lo < a.row_ptr[r + 1]) {
        const uint32_t gb = a.gbins[lo];
        if (gb < fe) return present_left(a, sp, gb - fs);
    }
    return sp.default_left != 0;
}

// The split owning a tile: the last split whose first tile is at or before
// it (a split without rows shares its first tile with the next split).
// `listed`: the tile's entry of a.tile_split, loaded by the caller.
__device__ __forceinline__ uint32_t split_of_tile(const PartArgs &a, uint32_t n_splits, uint32_t tile,
                                                  uint32_t listed) {
    if (a.tile_split) return listed;
    uint32_t lo = 0, hi = n_splits;
    while (hi - lo > 1) {
        const uint32_t mid = (lo + hi) / 2;
        if (a.splits[mid].tile_begin <= tile) lo = mid;
        else hi = mid;
    }
    return lo;
}

// The level's counts: from the device when a grown level set them.
__device__ __forceinline__ uint32_t part_splits(const PartArgs &a) { return a.grow ? a.grow->n_splits : a.n_splits; }
__device__ __forceinline__ uint32_t part_tiles(const PartArgs &a) { return a.grow ? a.grow->n_tiles : a.n_tiles; }

}  // namespace hbr

using namespace hbr;

// The routing bytes of a thread's rows, all loads issued before the first
// is used (a dense index with u8 columns; rows past the segment read
// nothing and route right).
template <bool MISSING>
__device__ __forceinline__ void route_dense8(const PartArgs &a, const PartSplit &sp, const uint32_t (&r)[kRowsPerThread],
                                             bool (&left)[kRowsPerThread]) {
    const uint8_t *col = a.cols8 + (size_t)sp.feature * a.n_rows;
    uint32_t b[kRowsPerThread];
#pragma unroll
    for (uint32_t k = 0; k < kRowsPerThread; k++) b[k] = r[k] != 0xffffffffu ? (uint32_t)col[r[k]] : 0xffffffffu;
    uint64_t w[kRowsPerThread];
    if constexpr (MISSING) {
        const uint64_t *bits = a.missing + (size_t)sp.feature * a.words;
#pragma unroll
        for (uint32_t k = 0; k < kRowsPerThread; k++) w[k] = r[k] != 0xffffffffu ? bits[r[k] >> 6] : 0ull;
    }
#pragma unroll
    for (uint32_t k = 0; k < kRowsPerThread; k++) {
        bool l = r[k] != 0xffffffffu && present_left(a, sp, b[k]);
        if constexpr (MISSING) {
            if ((w[k] >> (r[k] & 63u)) & 1ull) l = sp.default_left != 0;
        }
        left[k] = r[k] != 0xffffffffu && l;
    }
}

// Count pass: each wave's 64-row ballots of "goes left" and the tile's left
// count. The row ids, then the routing bytes, are loaded eight at a time.
extern "C" __global__ __launch_bounds__(256) void hbr_part_count(PartArgs a) {
    __shared__ uint32_t wave_count[kPartThreads / kWave];
    const uint32_t tile = blockIdx.x;
    // the tile's split, loaded with the tile count (the table covers the
    // grid), so that the two loads take one trip to memory
    const uint32_t listed = a.tile_split ? a.tile_split[tile] : 0u;
    if (tile >= part_tiles(a)) return;
    const PartSplit sp = a.splits[split_of_tile(a, part_splits(a), tile, listed)];
    const uint32_t base = (tile - sp.tile_begin) * kPartTile;
    const uint32_t *src = a.src_rows[sp.seg.buf] + sp.seg.offset;
    const uint32_t id0 = sp.identity ? sp.seg.offset % a.n_rows : 0u;  // a root of a batched level
    const uint32_t wave = threadIdx.x / kWave;
    uint32_t r[kRowsPerThread];
#pragma unroll
    for (uint32_t k = 0; k < kRowsPerThread; k++) {
        const uint32_t j = base + (k * (kPartThreads / kWave) + wave) * kWave + lane_id();
        r[k] = j < sp.seg.len ? (sp.identity ? id0 + j : src[j]) : 0xffffffffu;
    }
    bool left[kRowsPerThread];
    if (a.dense && a.cols8) {
        if (a.missing) route_dense8<true>(a, sp, r, left);
        else route_dense8<false>(a, sp, r, left);
    } else {
#pragma unroll
        for (uint32_t k = 0; k < kRowsPerThread; k++) left[k] = r[k] != 0xffffffffu && goes_left(a, sp, r[k]);
    }
    uint64_t m[kRowsPerThread];
#pragma unroll
    for (uint32_t k = 0; k < kRowsPerThread; k++) m[k] = __ballot(left[k]);
    uint64_t *dec = a.decisions + (size_t)tile * kBallots;
    uint32_t cnt = 0;
#pragma unroll
    for (uint32_t k = 0; k < kRowsPerThread; k++) {
        if (lane_id() == 0) dec[k * (kPartThreads / kWave) + wave] = m[k];
        cnt += (uint32_t)__popcll(m[k]);
    }
    if (lane_id() == 0) wave_count[wave] = cnt;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t total = 0;
        for (uint32_t w = 0; w < kPartThreads / kWave; w++) total += wave_count[w];
        a.tile_left[tile] = total;
    }
}

// One workgroup per split: exclusive scan of its tiles' left counts.
constexpr uint32_t kScanThreads = 1024;
extern "C" __global__ __launch_bounds__(1024) void hbr_part_scan(PartArgs a) {
    const uint32_t s = blockIdx.x;
    if (s >= part_splits(a)) return;
    const PartSplit sp = a.splits[s];
    const uint32_t n_tiles = (sp.seg.len + kPartTile - 1) / kPartTile;
    uint32_t carry = 0;
    // the counts of up to kScanAhead blocks of tiles loaded at once (one
    // trip to memory for a split of up to 8,192 tiles), then scanned block
    // by block
    constexpr uint32_t kScanAhead = 8;
    for (uint32_t t0 = 0; t0 < n_tiles; t0 += kScanThreads * kScanAhead) {
        uint32_t v[kScanAhead];
#pragma unroll
        for (uint32_t k = 0; k < kScanAhead; k++) {
            const uint32_t t = t0 + k * kScanThreads + threadIdx.x;
            v[k] = t < n_tiles ? a.tile_left[sp.tile_begin + t] : 0u;
        }
#pragma unroll
        for (uint32_t k = 0; k < kScanAhead; k++) {
            if (t0 + k * kScanThreads >= n_tiles) break;  // uniform
            const uint32_t t = t0 + k * kScanThreads + threadIdx.x;
            uint32_t total;
            const uint32_t ex = block_exclusive_scan<kScanThreads>(v[k], &total);
            if (t < n_tiles) a.tile_left[sp.tile_begin + t] = carry + ex;
            carry += total;
        }
    }
    if (threadIdx.x == 0) {
        PartOut o;
        o.left_len = carry;
        o.built_left = carry <= sp.seg.len - carry ? 1u : 0u;
        o.pad[0] = o.pad[1] = 0;
        a.out[s] = o;
    }
}

// Scatter pass: lanes 0..31 of every wave load the tile's 32 ballots at
// once and scan their left counts; each wave then moves the rows of its own
// eight ballots (row ids loaded together), left rows to the left child's
// run and right rows to the right child's, both in row order.
extern "C" __global__ __launch_bounds__(256) void hbr_part_scatter(PartArgs a) {
    const uint32_t tile = blockIdx.x;
    const uint32_t wave = threadIdx.x / kWave, lane = lane_id();
    // everything indexed by the tile alone is loaded with the tile count
    // (the tables cover the grid): one trip to memory before the split's
    const uint32_t listed = a.tile_split ? a.tile_split[tile] : 0u;
    const uint32_t left_before = a.tile_left[tile];
    const uint64_t *dec = a.decisions + (size_t)tile * kBallots;
    // ballot q sits in lane q
    const uint64_t mine = lane < kBallots ? dec[lane] : 0ull;
    if (tile >= part_tiles(a)) return;
    const uint32_t s = split_of_tile(a, part_splits(a), tile, listed);
    const PartSplit sp = a.splits[s];
    const uint32_t left_len = a.out[s].left_len;
    const uint32_t tile_pos = (tile - sp.tile_begin) * kPartTile;
    const uint32_t right_before = tile_pos - left_before;
    const uint32_t *src = a.src_rows[sp.seg.buf] + sp.seg.offset;
    uint32_t *dst = a.dst_rows[sp.seg.buf ^ 1u] + sp.seg.offset;
    const uint32_t id0 = sp.identity ? sp.seg.offset % a.n_rows : 0u;
    const uint64_t below = (1ull << lane) - 1ull;
    // the ballot's left rows and the left rows before it
    const uint32_t cnt = (uint32_t)__popcll(mine);
    uint32_t incl = cnt;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        const uint32_t t = __shfl_up(incl, d, kWave);
        if (lane >= (uint32_t)d) incl += t;
    }
    const uint32_t excl = incl - cnt;
    uint32_t r[kRowsPerThread];
#pragma unroll
    for (uint32_t k = 0; k < kRowsPerThread; k++) {
        const uint32_t q = k * (kPartThreads / kWave) + wave;
        const uint32_t j = tile_pos + q * kWave + lane;
        r[k] = j < sp.seg.len ? (sp.identity ? id0 + j : src[j]) : 0xffffffffu;
    }
#pragma unroll
    for (uint32_t k = 0; k < kRowsPerThread; k++) {
        const uint32_t q = k * (kPartThreads / kWave) + wave;
        const uint64_t m = (uint64_t)(uint32_t)__shfl((int)(uint32_t)mine, q, kWave) |
                           ((uint64_t)(uint32_t)__shfl((int)(uint32_t)(mine >> 32), q, kWave) << 32);
        const uint32_t run = (uint32_t)__shfl((int)excl, q, kWave);  // left rows of the ballots before q
        if (r[k] == 0xffffffffu) continue;
        if ((m >> lane) & 1ull) {
            dst[left_before + run + (uint32_t)__popcll(m & below)] = r[k];
        } else {
            // every row before this one in the tile exists: q*64 + lane rows
            const uint32_t rights = q * kWave - run + (uint32_t)__popcll(~m & below);
            dst[left_len + right_before + rights] = r[k];
        }
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

// The same margins update for a dense u8 index, in row order: each row is
// routed down the grown tree on its own local bins (the routing of the
// partition: bin < limit goes left), so the last level needs no partition
// and the margins are read and written once, coalesced. A node table that
// does not lead to a leaf within n_nodes steps leaves the row unchanged.
// The node count of the walked tree: given, or from a device-grown tree's
// counts (whose records are then read instead of meta/left/value; a leaf's
// left is -1).
__device__ __forceinline__ uint32_t walk_nodes(const WalkArgs &a) { return a.tree ? a.counts->n_nodes : a.n_nodes; }

__device__ __forceinline__ uint32_t node_meta(const WalkArgs &a, uint32_t i, uint32_t *left) {
    if (!a.tree) {
        *left = a.left[i];
        return a.meta[i];
    }
    const GrowTreeNode t = a.tree[i];
    *left = t.left < 0 ? 0u : (uint32_t)t.left;
    return t.left < 0 ? 1u << 31 : t.feature | (t.default_left ? kMetaDefaultLeft : 0u) | (t.limit << 16);
}

// A guarded walk that must not happen: the tree's gradients (any of its
// guard_n scales) were not finite, or an earlier guarded walk was skipped.
// Every workgroup reads the same words, so the answer is uniform; the first
// thread of the grid records the skip.
__device__ __forceinline__ bool walk_skipped(const WalkArgs &a) {
    if (!a.guard) return false;
    uint32_t bad = *a.poison;
    for (uint32_t i = 0; i < max(a.guard_n, 1u); i++) bad |= a.guard[i].nonfinite;
    if (bad && blockIdx.x == 0 && threadIdx.x == 0) *a.poison = 1u;
    return bad != 0;
}

extern "C" __global__ __launch_bounds__(256) void hbr_walk_leaves(WalkArgs a) {
    if (walk_skipped(a)) return;
    const uint32_t n_nodes = walk_nodes(a);
    for (uint32_t r = blockIdx.x * blockDim.x + threadIdx.x; r < a.n; r += gridDim.x * blockDim.x) {
        const uint8_t *b = a.bins8 + (size_t)r * a.stride;
        uint32_t nid = 0, left;
        uint32_t meta = node_meta(a, 0, &left);
        for (uint32_t step = 0; step < n_nodes && !(meta >> 31); step++) {
            const uint32_t f = meta & (kMetaDefaultLeft - 1u), lim = (meta >> 16) & 0x7fffu;
            // masked rows: feature f's bit of its group's mask word
            const uint32_t mask =
                a.masked ? *reinterpret_cast<const uint32_t *>(b + a.mask_at + 4 * (f >> 5)) >> (f & 31u) : 0u;
            const bool right = (mask & 1u) ? !(meta & kMetaDefaultLeft) : (uint32_t)b[f] >= lim;
            nid = left + (right ? 1u : 0u);
            nid = nid < n_nodes ? nid : 0u;
            meta = node_meta(a, nid, &left);
        }
        if (meta >> 31) {
            float *m = a.margins + (size_t)r * a.m_stride + a.output;
            *m = *m + (a.tree ? a.tree[nid].value : a.value[nid]);
        }
    }
}



// The walks for 32-byte rows and trees of at most kWalkLdsNodes nodes: the
// node table sits in LDS as (meta, left) pairs, and each thread walks
// kWalkRows rows per pass with every memory load of the pass issued before
// the first walk (a row's 32 bins in eight registers, its margin, label and
// weight); the routing byte is picked out of the registers.
constexpr uint32_t kWalkLdsNodes = 1024;
constexpr uint32_t kWalkRows = 8;

__device__ __forceinline__ uint32_t pick_byte(const uint32_t (&w)[8], uint32_t f) {
    // bit blends rather than selects on the array (which the compiler would
    // turn into a dynamically indexed scratch read)
    const uint32_t m4 = (f & 16u) ? ~0u : 0u, m2 = (f & 8u) ? ~0u : 0u, m1 = (f & 4u) ? ~0u : 0u;
    const uint32_t a0 = w[0] ^ ((w[0] ^ w[4]) & m4), a1 = w[1] ^ ((w[1] ^ w[5]) & m4);
    const uint32_t a2 = w[2] ^ ((w[2] ^ w[6]) & m4), a3 = w[3] ^ ((w[3] ^ w[7]) & m4);
    const uint32_t b0 = a0 ^ ((a0 ^ a2) & m2), b1 = a1 ^ ((a1 ^ a3) & m2);
    const uint32_t c = b0 ^ ((b0 ^ b1) & m1);
    return (c >> ((f & 3u) * 8u)) & 0xffu;
}

// Byte f (f < 64) of a 64-byte row held in sixteen registers.
__device__ __forceinline__ uint32_t pick_byte16(const uint32_t (&w)[16], uint32_t f) {
    const uint32_t m8 = (f & 32u) ? ~0u : 0u;
    uint32_t h[8];
#pragma unroll
    for (int i = 0; i < 8; i++) h[i] = w[i] ^ ((w[i] ^ w[i + 8]) & m8);
    return pick_byte(h, f & 31u);
}

// The class trees of a softmax round added to their margins in one pass
// over the rows (32- or 64-byte rows, W words, or the first 64 bytes of a
// masked row of at most 64 features): every tree's node table in
// LDS, each row's bins read once into registers, then walked through tree
// 0, 1, ..., each leaf added to its own margin (output + c) with the same
// single f32 add as hbr_walk_leaves, so the margins are those of one walk
// per tree. The host checks that the tables fit (kBatchWalkNodes nodes,
// kBatchWalkTrees trees).
template <int W>
__device__ __forceinline__ void walk_leaves_batch(const WalkArgs &a) {
    __shared__ uint2 s_node[kBatchWalkNodes];
    __shared__ float s_value[kBatchWalkNodes];
    __shared__ uint32_t s_first[kBatchWalkTrees + 1];
    if (walk_skipped(a)) return;
    const uint32_t K = a.n_trees;
    if (threadIdx.x == 0) {
        uint32_t total = 0;
        for (uint32_t c = 0; c < K; c++) {
            s_first[c] = total;
            const GrowCounts *cc = reinterpret_cast<const GrowCounts *>(
                reinterpret_cast<const char *>(a.counts) + (size_t)c * a.tree_bytes);
            total += min(cc->n_nodes, kBatchWalkNodes - total);
        }
        s_first[K] = total;
    }
    __syncthreads();
    for (uint32_t c = 0; c < K; c++) {
        const GrowTreeNode *tc = reinterpret_cast<const GrowTreeNode *>(
            reinterpret_cast<const char *>(a.tree) + (size_t)c * a.tree_bytes);
        const uint32_t first = s_first[c], n = s_first[c + 1] - first;
        for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
            const GrowTreeNode t = tc[i];
            const uint32_t meta =
                t.left < 0 ? 1u << 31 : t.feature | (t.default_left ? kMetaDefaultLeft : 0u) | (t.limit << 16);
            s_node[first + i] = make_uint2(meta, t.left < 0 ? 0u : (uint32_t)t.left);
            s_value[first + i] = t.value;
        }
    }
    __syncthreads();
    for (uint32_t r = blockIdx.x * blockDim.x + threadIdx.x; r < a.n; r += gridDim.x * blockDim.x) {
        uint32_t w[W];
        const uint4 *src = reinterpret_cast<const uint4 *>(a.bins8 + (size_t)r * a.stride);
#pragma unroll
        for (int q = 0; q < W / 4; q++) {
            const uint4 v = src[q];
            w[4 * q] = v.x;
            w[4 * q + 1] = v.y;
            w[4 * q + 2] = v.z;
            w[4 * q + 3] = v.w;
        }
        // masked rows: the mask word of 32-byte rows; wider rows (at most 64
        // features) keep their first two mask words at mask_at
        uint2 mk = make_uint2(0u, 0u);
        if (a.masked) {
            if constexpr (W == 8)
                mk.x = w[kMaskWord];
            else
                mk = *reinterpret_cast<const uint2 *>(a.bins8 + (size_t)r * a.stride + a.mask_at);
        }
        float *m = a.margins + (size_t)r * a.m_stride + a.output;
        for (uint32_t c = 0; c < K; c++) {
            const uint32_t first = s_first[c], n = s_first[c + 1] - first;
            if (n == 0) continue;
            uint32_t nid = 0;
            uint2 nd = s_node[first];
            for (uint32_t step = 0; step < n && !(nd.x >> 31); step++) {
                const uint32_t f = nd.x & (kMetaDefaultLeft - 1u), lim = (nd.x >> 16) & 0x7fffu;
                uint32_t bin;
                if constexpr (W == 16) {
                    bin = pick_byte16(w, f & 63u);
                } else {
                    uint32_t h[8];
#pragma unroll
                    for (int i = 0; i < 8; i++) h[i] = w[i];
                    bin = pick_byte(h, f & 31u);
                }
                const uint32_t mask = (W == 16 && (f & 32u)) ? mk.y : mk.x;
                const bool right = ((mask >> (f & 31u)) & 1u) ? !(nd.x & kMetaDefaultLeft) : bin >= lim;
                nid = nd.y + (right ? 1u : 0u);
                nid = nid < n ? nid : 0u;
                nd = s_node[first + nid];
            }
            if (nd.x >> 31) m[c] = m[c] + s_value[first + nid];
        }
    }
}

extern "C" __global__ __launch_bounds__(256) void hbr_walk_leaves_batch32(WalkArgs a) { walk_leaves_batch<8>(a); }
extern "C" __global__ __launch_bounds__(256) void hbr_walk_leaves_batch64(WalkArgs a) { walk_leaves_batch<16>(a); }

__device__ __forceinline__ uint32_t load_walk_nodes(const WalkArgs &a, uint2 *s_node, float *s_value) {
    const uint32_t n_nodes = min(walk_nodes(a), kWalkLdsNodes);
    for (uint32_t i = threadIdx.x; i < n_nodes; i += blockDim.x) {
        uint32_t meta, left;
        float value;
        if (a.tree) {
            const GrowTreeNode t = a.tree[i];
            meta = t.left < 0 ? 1u << 31 : t.feature | (t.default_left ? kMetaDefaultLeft : 0u) | (t.limit << 16);
            left = t.left < 0 ? 0u : (uint32_t)t.left;
            value = t.value;
        } else {
            meta = a.meta[i];
            left = a.left[i];
            value = a.value[i];
        }
        s_node[i] = make_uint2(meta, left);
        s_value[i] = value;
    }
    return n_nodes;
}

// The leaf a row reaches (n_nodes steps at most; -1 when no leaf is reached).
// mask: the row's missing features (masked rows), 0 otherwise.
__device__ __forceinline__ int32_t walk_row(const uint2 *s_node, uint32_t n_nodes, const uint32_t (&w)[8],
                                            uint32_t mask = 0u) {
    uint32_t nid = 0;
    uint2 nd = s_node[0];
    for (uint32_t step = 0; step < n_nodes && !(nd.x >> 31); step++) {
        const uint32_t f = nd.x & 31u, lim = (nd.x >> 16) & 0x7fffu;
        const bool right = ((mask >> f) & 1u) ? !(nd.x & kMetaDefaultLeft) : pick_byte(w, f) >= lim;
        nid = nd.y + (right ? 1u : 0u);
        nid = nid < n_nodes ? nid : 0u;
        nd = s_node[nid];
    }
    return (nd.x >> 31) ? (int32_t)nid : -1;
}

__device__ __forceinline__ void load_row_bins(const WalkArgs &a, uint32_t r, uint32_t (&w)[8]) {
    const uint4 *src = reinterpret_cast<const uint4 *>(a.bins8 + (size_t)r * 32u);
    const uint4 x = src[0], y = src[1];
    w[0] = x.x;
    w[1] = x.y;
    w[2] = x.z;
    w[3] = x.w;
    w[4] = y.x;
    w[5] = y.y;
    w[6] = y.z;
    w[7] = y.w;
}

extern "C" __global__ __launch_bounds__(256) void hbr_walk_leaves32(WalkArgs a) {
    __shared__ uint2 s_node[kWalkLdsNodes];
    __shared__ float s_value[kWalkLdsNodes];
    if (walk_skipped(a)) return;
    const uint32_t n_nodes = load_walk_nodes(a, s_node, s_value);
    __syncthreads();
    const uint32_t stride = gridDim.x * blockDim.x;
    for (uint32_t r0 = blockIdx.x * blockDim.x + threadIdx.x; r0 < a.n; r0 += kWalkRows * stride) {
        uint32_t w[kWalkRows][8];
        float m[kWalkRows];
#pragma unroll
        for (uint32_t k = 0; k < kWalkRows; k++) {
            const uint32_t r = r0 + k * stride;
            if (r < a.n) {
                load_row_bins(a, r, w[k]);
                m[k] = a.margins[(size_t)r * a.m_stride + a.output];
            }
        }
#pragma unroll
        for (uint32_t k = 0; k < kWalkRows; k++) {
            const uint32_t r = r0 + k * stride;
            if (r >= a.n) continue;
            const int32_t leaf = walk_row(s_node, n_nodes, w[k], a.masked ? w[k][kMaskWord] : 0u);
            if (leaf >= 0) a.margins[(size_t)r * a.m_stride + a.output] = m[k] + s_value[leaf];
        }
    }
}

// hbr_walk_leaves32 and, for the same rows while their updated margins are
// in registers, the next round's gradient pairs (row_gradient_yw: the
// gradient kernel's arithmetic, its 8-row vector test and its max fold).
// The rows of a wave are 64 consecutive rows (the strides are multiples of
// 64), and whole waves stay in the loop past the last row, as in
// hbr_gradients.
extern "C" __global__ __launch_bounds__(256) void hbr_walk_grad32(WalkGradArgs args) {
    const WalkArgs &a = args.w;
    const GradArgs &ga = args.g;
    __shared__ uint2 s_node[kWalkLdsNodes];
    __shared__ float s_value[kWalkLdsNodes];
    if (walk_skipped(a)) return;
    const uint32_t n_nodes = load_walk_nodes(a, s_node, s_value);
    __syncthreads();
    uint32_t mg = 0, mh = 0, bad = 0;
    const uint32_t end = (a.n + kWave - 1) / kWave * kWave;
    const uint32_t stride = gridDim.x * blockDim.x;
    for (uint32_t r0 = blockIdx.x * blockDim.x + threadIdx.x; r0 < end; r0 += kWalkRows * stride) {
        uint32_t w[kWalkRows][8], orig[kWalkRows];
        float m[kWalkRows], y[kWalkRows], wt[kWalkRows];
#pragma unroll
        for (uint32_t k = 0; k < kWalkRows; k++) {
            const uint32_t r = r0 + k * stride;
            m[k] = 0.0f;
            y[k] = 0.0f;
            wt[k] = 1.0f;
            orig[k] = r;
            if (r < a.n) {
                load_row_bins(a, r, w[k]);
                m[k] = a.margins[(size_t)r * a.m_stride + a.output];
                y[k] = ga.labels[r];
                if (ga.weights) wt[k] = ga.weights[r];
                if (ga.perm) orig[k] = ga.perm[r];
            }
        }
#pragma unroll
        for (uint32_t k = 0; k < kWalkRows; k++) {
            const uint32_t r = r0 + k * stride;
            const bool active = r < a.n;
            if (active) {
                const int32_t leaf = walk_row(s_node, n_nodes, w[k], a.masked ? w[k][kMaskWord] : 0u);
                if (leaf >= 0) {
                    m[k] = m[k] + s_value[leaf];
                    a.margins[(size_t)r * a.m_stride + a.output] = m[k];
                }
            }
            if (r < end) {
                uint32_t word = w[k][7];  // a deferred row's word is written by hbr_finish_scale
                row_gradient_yw<true>(ga, r, orig[k], active, m[k], y[k], wt[k], mg, mh, bad, &word);
                if (ga.pair_rows && active) {  // the whole 32-byte row back, its pair in the last word
                    uint4 *dst = reinterpret_cast<uint4 *>(ga.pair_rows + (size_t)r * 32u);
                    dst[0] = make_uint4(w[k][0], w[k][1], w[k][2], w[k][3]);
                    dst[1] = make_uint4(w[k][4], w[k][5], w[k][6], word);
                }
            }
        }
    }
    fold_block(ga.scale, mg, mh, bad);
}

// hbr_walk_grad32 that also sums the next tree's root histogram: each
// active row's new pair, quantised with the bound exponents hbr_finish_scale
// will set (the unit-weight logistic loss: |g| <= 1, h <= 1/4), goes into a
// bin-major LDS histogram of 32 feature columns, as the dense histogram
// kernel adds it (the lanes' features rotated; columns past the index's
// features take the row's padding and pair bytes and are never written
// out). One workgroup per CU, its sub-histogram written to its own partial
// ([f][256]); rows the walk defers to hbr_finish_scale are summed by
// hbr_root_fixup. The pair's bits equal those the histogram kernel derives
// from the row's word, so the sums are the root histogram's.
constexpr uint32_t kRootWalkRows = 4;

// NF < 32: the row's first NF bytes are its features (25 to 28), and the
// lanes rotate over those alone, so no atomic goes to a padding column.
template <uint32_t NF>
__device__ __forceinline__ void walk_grad_root(const WalkGradArgs &args) {
    const WalkArgs &a = args.w;
    const GradArgs &ga = args.g;
    __shared__ uint2 s_node[kWalkLdsNodes];
    __shared__ float s_value[kWalkLdsNodes];
    // NF < kRootFeatures: h's words start on g's last (bin 255, a padding
    // column no add reaches), so that one address with an LDS offset
    // serves both adds of a cell
    constexpr uint32_t kHAt = NF < kRootFeatures ? kRootTile - 1 : kRootTile;
    __shared__ unsigned long long lgh[kHAt + kRootTile];
    unsigned long long *const lg = lgh, *const lh = lgh + kHAt;
    if (walk_skipped(a)) return;
    for (uint32_t i = threadIdx.x; i < kHAt + kRootTile; i += blockDim.x) lgh[i] = 0ull;
    const uint32_t n_nodes = load_walk_nodes(a, s_node, s_value);
    __syncthreads();
    const uint32_t rot = NF == kRootFeatures ? lane_id() & (kRootFeatures - 1u) : lane_id() % NF;
    uint32_t mg = 0, mh = 0, bad = 0;
    const uint32_t end = (a.n + kWave - 1) / kWave * kWave;
    const uint32_t stride = gridDim.x * blockDim.x;
    for (uint32_t r0 = blockIdx.x * blockDim.x + threadIdx.x; r0 < end; r0 += kRootWalkRows * stride) {
        uint32_t w[kRootWalkRows][8], orig[kRootWalkRows];
        float m[kRootWalkRows], y[kRootWalkRows];
#pragma unroll
        for (uint32_t k = 0; k < kRootWalkRows; k++) {
            const uint32_t r = r0 + k * stride;
            m[k] = 0.0f;
            y[k] = 0.0f;
            orig[k] = r;
            if (r < a.n) {
                load_row_bins(a, r, w[k]);
                m[k] = a.margins[(size_t)r * a.m_stride + a.output];
                y[k] = ga.labels[r];
                if (ga.perm) orig[k] = ga.perm[r];
            }
        }
#pragma unroll
        for (uint32_t k = 0; k < kRootWalkRows; k++) {
            const uint32_t r = r0 + k * stride;
            const bool active = r < a.n;
            if (active) {
                // rows carrying pairs hold no missing mask (word 7 is the pair)
                const int32_t leaf = walk_row(s_node, n_nodes, w[k]);
                if (leaf >= 0) {
                    m[k] = m[k] + s_value[leaf];
                    a.margins[(size_t)r * a.m_stride + a.output] = m[k];
                }
            }
            if (r >= end) continue;
            uint32_t word = w[k][7];
            // p stays NaN unless the row's pair is computed here (a deferred
            // row's is hbr_finish_scale's; a non-finite pair fails the tree)
            GPair p{__builtin_nanf(""), 0.0f};
            row_gradient_yw<true>(ga, r, orig[k], active, m[k], y[k], 1.0f, mg, mh, bad, &word, &p);
            const bool summed = active && p.g == p.g;
            if (active) {  // the whole 32-byte row back, its pair in the last word
                uint4 *dst = reinterpret_cast<uint4 *>(ga.pair_rows + (size_t)r * 32u);
                dst[0] = make_uint4(w[k][0], w[k][1], w[k][2], w[k][3]);
                dst[1] = make_uint4(w[k][4], w[k][5], w[k][6], word);
            }
            if (summed) {
                const unsigned long long qg = (unsigned long long)quantize(p.g, args.root_exp_g);
                const unsigned long long qh = (unsigned long long)quantize(p.h, args.root_exp_h);
                uint32_t v[NF / 4];
#pragma unroll
                for (uint32_t i = 0; i < NF / 4; i++) v[i] = w[k][i];
                rotate_bytes<NF / 4>(v, rot);
#pragma unroll
                for (int f = 0; f < (int)NF; f++) {
                    uint32_t ff = (uint32_t)f + rot;
                    ff = NF == kRootFeatures ? ff & (kRootFeatures - 1u) : (ff >= NF ? ff - NF : ff);
                    const uint32_t bin = (v[f >> 2] >> ((f & 3) * 8)) & 0xffu;
                    atomicAdd(&lg[bin * kRootFeatures + ff], qg);
                    atomicAdd(&lh[bin * kRootFeatures + ff], qh);
                }
            }
        }
    }
    fold_block(ga.scale, mg, mh, bad);
    __syncthreads();
    QBin *dst = args.root_partial + (size_t)blockIdx.x * kRootTile;
    for (uint32_t i = threadIdx.x; i < kRootTile; i += blockDim.x) {
        const uint32_t ff = i % kRootFeatures, bin = i / kRootFeatures;
        if (ff < args.n_cols) dst[ff * 256u + bin] = QBin{(int64_t)lg[i], (int64_t)lh[i]};
    }
}

extern "C" __global__ __launch_bounds__(1024) void hbr_walk_grad_root(WalkGradArgs args) {
    walk_grad_root<kRootFeatures>(args);
}
extern "C" __global__ __launch_bounds__(1024) void hbr_walk_grad_root_nf28(WalkGradArgs args) {
    walk_grad_root<28>(args);
}

// One workgroup after hbr_finish_scale: the rows the fused walk deferred
// (their words now written) into partial n_walk_tiles, as the histogram
// kernel derives their pairs from the words, then the root's node record
// for hbr_hist_reduce: every partial from the first.
extern "C" __global__ __launch_bounds__(1024) void hbr_root_fixup(RootFixupArgs a) {
    __shared__ unsigned long long lg[kRootTile], lh[kRootTile];
    for (uint32_t i = threadIdx.x; i < kRootTile; i += blockDim.x) {
        lg[i] = 0ull;
        lh[i] = 0ull;
    }
    __syncthreads();
    const QScale q = *a.scale;
    for (uint32_t j = threadIdx.x; j < q.deferred; j += blockDim.x) {
        const uint32_t r = a.listed[j];
        const uint4 *src = reinterpret_cast<const uint4 *>(a.bins8 + (size_t)r * 32u);
        const uint4 x = src[0], z = src[1];
        const uint32_t w[8] = {x.x, x.y, x.z, x.w, z.x, z.y, z.z, z.w};
        const float pv = __uint_as_float(w[7] & 0x7fffffffu);
        const float y = (w[7] >> 31) ? 1.0f : 0.0f;
        const float qv = pv * (1.0f - pv);
        const GPair p{(pv - y) * 1.0f, (qv > a.min_hess ? qv : a.min_hess) * 1.0f};
        const unsigned long long qg = (unsigned long long)quantize(p.g, q.exp_g);
        const unsigned long long qh = (unsigned long long)quantize(p.h, q.exp_h);
        for (uint32_t f = 0; f < a.n_cols; f++) {
            const uint32_t bin = (w[f >> 2] >> ((f & 3u) * 8u)) & 0xffu;
            atomicAdd(&lg[bin * kRootFeatures + f], qg);
            atomicAdd(&lh[bin * kRootFeatures + f], qh);
        }
    }
    __syncthreads();
    QBin *dst = a.partial + (size_t)a.n_walk_tiles * kRootTile;
    for (uint32_t i = threadIdx.x; i < kRootTile; i += blockDim.x) {
        const uint32_t ff = i % kRootFeatures, bin = i / kRootFeatures;
        if (ff < a.n_cols) dst[ff * 256u + bin] = QBin{(int64_t)lg[i], (int64_t)lh[i]};
    }
    if (threadIdx.x == 0) {
        a.node->tile_begin = 0;
        a.node->n_tiles = a.n_walk_tiles + 1u + a.regroup_tile;
        a.node->pad[0] = 0;
        a.node->pad[1] = 0;
    }
}

// One workgroup after a fused walk over reordered rows, before
// hbr_finish_scale: each marked original vector's rows that took the vector
// path on their own margins (|m| within the range) join the scalar list,
// and, for hbr_walk_grad_root, their summed vector pairs come back out of
// the root histogram through partial n_walk_tiles + 1 (hbr_root_fixup
// then sums their scalar pairs in).
extern "C" __global__ __launch_bounds__(1024) void hbr_regroup(RegroupArgs a) {
    __shared__ unsigned long long lg[kRootTile], lh[kRootTile];
    const GradArgs &ga = a.g;
    if (a.root_partial) {
        for (uint32_t i = threadIdx.x; i < kRootTile; i += blockDim.x) {
            lg[i] = 0ull;
            lh[i] = 0ull;
        }
        __syncthreads();
    }
    const uint32_t groups = ga.bad_groups[0];
    for (uint32_t j = threadIdx.x; j < 8u * groups; j += blockDim.x) {
        const uint32_t orig = 8u * ga.bad_groups[1u + j / 8u] + (j & 7u);
        const uint32_t r = a.perm_inv[orig];
        const float m = ga.margins[r];
        if (orig >= ga.vec_rows || !(__builtin_fabsf(m) <= ga.max_input)) continue;  // already a scalar row
        ga.scalar_list[atomicAdd(&ga.scale->scalar_rows, 1u)] = r;
        if (!a.root_partial) continue;
        float p;
        const GPair q = logistic_vector_pair(ga, m, ga.labels[r], 1.0f, &p);
        const unsigned long long qg = (unsigned long long)(-quantize(q.g, a.root_exp_g));
        const unsigned long long qh = (unsigned long long)(-quantize(q.h, a.root_exp_h));
        const uint4 *src = reinterpret_cast<const uint4 *>(a.bins8 + (size_t)r * 32u);
        const uint4 x = src[0], z = src[1];
        const uint32_t w[8] = {x.x, x.y, x.z, x.w, z.x, z.y, z.z, z.w};
        for (uint32_t f = 0; f < a.n_cols && f < kMaskedMaxFeatures; f++) {  // word 7 is the pair
            const uint32_t bin = (w[f >> 2] >> ((f & 3u) * 8u)) & 0xffu;
            atomicAdd(&lg[bin * kRootFeatures + f], qg);
            atomicAdd(&lh[bin * kRootFeatures + f], qh);
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) ga.bad_groups[0] = 0u;
    if (!a.root_partial) return;
    QBin *dst = a.root_partial + (size_t)(a.n_walk_tiles + 1u) * kRootTile;
    for (uint32_t i = threadIdx.x; i < kRootTile; i += blockDim.x) {
        const uint32_t ff = i % kRootFeatures, bin = i / kRootFeatures;
        if (ff < a.n_cols) dst[ff * 256u + bin] = QBin{(int64_t)lg[i], (int64_t)lh[i]};
    }
}

// Masked dense rows from an index's local u8 columns and missing bitmap (a
// host-built index of a matrix with missing values, or a wide matrix binned
// on the device): one thread per row writes its whole record, word by word:
// its bins in bytes 0..n_cols-1 (0 beyond), and its mask words from byte
// mask_at (bit f % 32 of word f / 32: feature f missing; 32-byte rows keep
// the one word in kMaskWord).
extern "C" __global__ __launch_bounds__(256) void hbr_rows_from_cols(RowsFromColsArgs a) {
    const uint64_t r = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= a.n_rows) return;
    uint32_t *dst = reinterpret_cast<uint32_t *>(a.rows8 + r * a.stride);
    const uint32_t words = a.stride / 4, mask0 = a.mask_at / 4;
    for (uint32_t w = 0; w < words; w++) {
        uint32_t v = 0;
        if (w >= mask0) {
            const uint32_t f0 = 32 * (w - mask0);
            for (uint32_t j = 0; j < 32 && f0 + j < a.n_cols && a.missing; j++)
                v |= (uint32_t)((a.missing[(uint64_t)(f0 + j) * a.words + (r >> 6)] >> (r & 63u)) & 1ull) << j;
        } else {
            for (uint32_t j = 0; j < 4 && 4 * w + j < a.n_cols; j++)
                v |= (uint32_t)a.cols8[(uint64_t)(4 * w + j) * a.n_rows + r] << (8 * j);
        }
        dst[w] = v;
    }
}

// ---- rows reordered by a tree's leaves ------------------------------------------
//
// The whole-round trainer reorders the rows once, by the leaves of its
// first tree: later trees split on much the same features, so the rows of
// one of their deep nodes then share cache lines, and the gathers of the
// histogram and of the partition's routing bytes fetch far fewer lines.
// Every sum is an integer sum, so the trees do not depend on the order.

// Each row's leaf in the tree (staged walk of its 32-byte row), and each
// leaf's row count: a workgroup's counts in LDS, then one global add per
// leaf it saw. The host checks that the tree's nodes fit kOrderMaxNodes.
extern "C" __global__ __launch_bounds__(256) void hbr_order_leaves(OrderArgs a) {
    __shared__ uint2 s_node[kWalkLdsNodes];
    __shared__ float s_value[kWalkLdsNodes];
    __shared__ uint32_t s_count[kOrderMaxNodes];
    const uint32_t n_nodes = load_walk_nodes(a.w, s_node, s_value);
    for (uint32_t i = threadIdx.x; i < kOrderMaxNodes; i += blockDim.x) s_count[i] = 0u;
    __syncthreads();
    for (uint32_t r = blockIdx.x * blockDim.x + threadIdx.x; r < a.w.n; r += gridDim.x * blockDim.x) {
        uint32_t w[8];
        load_row_bins(a.w, r, w);
        const int32_t leaf = walk_row(s_node, n_nodes, w);
        const uint32_t l = leaf >= 0 && (uint32_t)leaf < kOrderMaxNodes ? (uint32_t)leaf : 0u;
        a.leaf[r] = l;
        atomicAdd(&s_count[l], 1u);
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < kOrderMaxNodes; i += blockDim.x)
        if (s_count[i]) atomicAdd(&a.count[i], s_count[i]);
}

// One workgroup: each leaf's first position (exclusive scan of the counts).
extern "C" __global__ __launch_bounds__(1024) void hbr_order_scan(OrderArgs a) {
    static_assert(kOrderMaxNodes == 1024, "one count per thread");
    uint32_t total;
    const uint32_t v = a.count[threadIdx.x];
    a.cursor[threadIdx.x] = block_exclusive_scan<1024>(v, &total);
}

// Each row's position: a workgroup counts its rows per leaf again (the
// same rows as in hbr_order_leaves' grid-stride loop of the same launch
// shape), takes a run of positions from each leaf's cursor with one
// atomic per leaf, and hands them out to its rows through LDS atomics.
extern "C" __global__ __launch_bounds__(256) void hbr_order_place(OrderArgs a) {
    __shared__ uint32_t s_count[kOrderMaxNodes];
    for (uint32_t i = threadIdx.x; i < kOrderMaxNodes; i += blockDim.x) s_count[i] = 0u;
    __syncthreads();
    for (uint32_t r = blockIdx.x * blockDim.x + threadIdx.x; r < a.w.n; r += gridDim.x * blockDim.x)
        atomicAdd(&s_count[a.leaf[r]], 1u);
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < kOrderMaxNodes; i += blockDim.x)
        s_count[i] = s_count[i] ? atomicAdd(&a.cursor[i], s_count[i]) : 0u;
    __syncthreads();
    for (uint32_t r = blockIdx.x * blockDim.x + threadIdx.x; r < a.w.n; r += gridDim.x * blockDim.x)
        a.perm[atomicAdd(&s_count[a.leaf[r]], 1u)] = r;
}

// inverse[perm[i]] = i
extern "C" __global__ __launch_bounds__(256) void hbr_order_invert(GatherArgs a) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < a.n) reinterpret_cast<uint32_t *>(a.dst8)[a.index[i]] = (uint32_t)i;
}

// dst record i = src record index[i] (row_bytes each, 16 bytes at a time)
extern "C" __global__ __launch_bounds__(256) void hbr_gather_records(GatherArgs a) {
    const uint32_t words = a.row_bytes / 16u;
    const uint64_t total = a.n * words;
    for (uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t i = t / words;
        const uint32_t q = (uint32_t)(t % words);
        reinterpret_cast<uint4 *>(a.dst8)[t] =
            reinterpret_cast<const uint4 *>(a.src8)[(uint64_t)a.index[i] * words + q];
    }
}

// The columns of 32-byte rows (bins in bytes 0..n_cols-1): dst column f,
// row i = byte f of src record i (the rows already in their new order).
extern "C" __global__ __launch_bounds__(256) void hbr_columns_from_rows(GatherArgs a) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.n; i += (uint64_t)gridDim.x * blockDim.x) {
        const uint4 *src = reinterpret_cast<const uint4 *>(a.src8 + i * 32u);
        const uint4 x = src[0], z = src[1];
        const uint32_t w[8] = {x.x, x.y, x.z, x.w, z.x, z.y, z.z, z.w};
        for (uint32_t f = 0; f < a.n_cols && f < 32u; f++)
            a.dst8[(uint64_t)f * a.n + i] = (uint8_t)(w[f >> 2] >> ((f & 3u) * 8u));
    }
}

// dst row i = src row index[i] (k f32 values a row)
extern "C" __global__ __launch_bounds__(256) void hbr_gather_f32(GatherArgs a) {
    const uint64_t total = a.n * a.k;
    for (uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t i = t / a.k;
        const uint32_t c = (uint32_t)(t % a.k);
        a.dst32[t] = a.src32[(uint64_t)a.index[i] * a.k + c];
    }
}
