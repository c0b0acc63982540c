// Gradient histograms in fixed point (the hot kernel of tree growth).
//
// Replaces CpuBackend::build (tree/hist/mod.rs:510-547): every bin of a node
// receives the integer sum of its rows' quantized (g, h). Integer sums are
// exact and order-free, so any launch shape, tile size or workgroup count
// gives the same bins; when the reference's own sums are exact
// (backend/exact_sum.rs:14-37) these equal its f64 bins bit for bit.
//
// A launch covers a batch of nodes. hbr_hist_plan cuts every node's rows
// into tiles sized so that the batch is about one wave of workgroups (the
// nodes of a level are only known on the device, after the partition).
// Dense indexes read row-major local bins (u8 for <= 256 bins per feature):
// a workgroup takes one tile and one group of FG features, accumulates into
// LDS with 64-bit integer atomics, then writes its sub-histogram with plain
// stores: straight into the node's slot when the node is one tile, else to
// a partial that hbr_hist_reduce sums. No device-scope atomics.
// Sparse (CSR) indexes add each stored entry straight to the slot.
#include "common.h"

namespace hbr {

__device__ __forceinline__ Seg resolve_node(const PlanArgs &a, const HistNode &nd) {
    if (!nd.from_split) return nd.seg;
    const PartSplit sp = a.splits[nd.split];
    const PartOut po = a.part_out[nd.split];
    Seg s;
    s.buf = sp.seg.buf ^ 1u;
    s.pad = 0;
    if (po.built_left) {
        s.offset = sp.seg.offset;
        s.len = po.left_len;
    } else {
        s.offset = sp.seg.offset + po.left_len;
        s.len = sp.seg.len - po.left_len;
    }
    return s;
}

// LDS row of one feature: 256 bins plus one pad word, so that the same bin
// of consecutive features falls in different banks.
constexpr uint32_t kLdsFeature = 257;

// Rotate the FG feature bytes held in W words right by `rot` bytes: byte i
// of the result is byte (i + rot) mod 4W of the input.
template <int W>
__device__ __forceinline__ void rotate_bytes(uint32_t (&w)[W], uint32_t rot) {
    const uint32_t wr = rot >> 2;
#pragma unroll
    for (int b = 1; b < W; b <<= 1) {
        // a bit blend rather than a select, which the compiler would turn
        // into a dynamically indexed (scratch) array read
        const uint32_t m = (wr & (uint32_t)b) ? ~0u : 0u;
        uint32_t t[W];
#pragma unroll
        for (int i = 0; i < W; i++) t[i] = w[i] ^ ((w[i] ^ w[(i + b) % W]) & m);
#pragma unroll
        for (int i = 0; i < W; i++) w[i] = t[i];
    }
    const uint32_t sh = (rot & 3u) * 8u;
    uint32_t t[W];
#pragma unroll
    for (int i = 0; i < W; i++) t[i] = __builtin_amdgcn_alignbit(w[(i + 1) % W], w[i], sh);
#pragma unroll
    for (int i = 0; i < W; i++) w[i] = t[i];
}

template <int FG>
__device__ __forceinline__ void load_bins(const uint8_t *p, uint32_t (&w)[FG / 4]) {
    if constexpr (FG == 8) {
        const uint2 v = *reinterpret_cast<const uint2 *>(p);
        w[0] = v.x;
        w[1] = v.y;
    } else {
#pragma unroll
        for (int i = 0; i < FG / 16; i++) {
            const uint4 v = reinterpret_cast<const uint4 *>(p)[i];
            w[4 * i] = v.x;
            w[4 * i + 1] = v.y;
            w[4 * i + 2] = v.z;
            w[4 * i + 3] = v.w;
        }
    }
}

// Row loop of one workgroup. Lane l starts at feature l mod FG (the bytes
// rotated in registers), so that rows piled in one bin of one feature do not
// all hit the same LDS word in one instruction (on data with point masses
// this runs 2.3x faster than feature-in-lockstep, and as fast on smooth
// data).
//
// BIN_MAJOR: the LDS sub-histogram is [bin][feature]. A 64-bit word's bank
// pair then depends on its feature only, and the rotation gives the lanes
// of each 16-lane group 16 different features: their atomics never share a
// bank, whatever the bins. Otherwise [feature][257] (bins padded), where
// the banks follow the data, and features past nf go to per-lane dummies.
//
// NF < FG (bin-major only): the row's first NF bytes are its features and
// the lanes rotate over those alone (lane l starts at feature l mod NF, still
// 16 different features in every 16-lane group), so no atomic goes to a
// padding column: 28 features take 56 atomics a row instead of 64.
template <int FG, bool BIN_MAJOR, bool MASKED = false, int NF = FG>
__device__ __forceinline__ void hist_dense8(const HistArgs &a) {
    static_assert(NF == FG || (BIN_MAJOR && NF % 4 == 0 && NF < FG && NF >= 16), "NF: whole words, bin-major");
    constexpr int W = FG / 4;
    constexpr int NW = NF / 4;
    constexpr uint32_t kWords = BIN_MAJOR ? FG * 256 : FG * kLdsFeature + kWave;
    constexpr uint32_t kDummy = FG * kLdsFeature;
    // NF < FG: g's last word (bin 255, column FG - 1) is a padding column
    // no add reaches, so h's words start on it; a cell's h then sits
    // (kWords - 1) x 8 bytes after its g, within an LDS instruction's
    // 16-bit offset, and one address serves both adds
    constexpr uint32_t kHAt = BIN_MAJOR && NF < FG ? kWords - 1 : kWords;
    __shared__ unsigned long long lgh[kHAt + kWords];
    unsigned long long *const lg = lgh, *const lh = lgh + kHAt;
    const uint32_t entry = blockIdx.x / a.groups, grp = blockIdx.x % a.groups;
    if (entry >= a.counts[0]) return;  // uniform across the workgroup
    const HistTile t = a.tiles[entry];
    const HistNode nd = a.nodes[t.node];
    const uint32_t f0 = grp * FG;
    const uint32_t nf = min((uint32_t)FG, a.n_cols - f0);
    for (uint32_t i = threadIdx.x; i < kHAt + kWords; i += blockDim.x) lgh[i] = 0ull;
    __syncthreads();
    const int eg = a.scale[nd.cls].exp_g, eh = a.scale[nd.cls].exp_h;
    const GPair *gpair = a.gpair + (size_t)nd.cls * a.class_rows;
    const uint32_t *rows = a.rows[nd.seg.buf] + nd.seg.offset;
    const uint32_t lane = lane_id();
    const uint32_t rot = NF == FG ? lane & (FG - 1) : lane % (uint32_t)NF;
    const uint32_t end = t.row0 + t.rows;
    const bool row_pairs = a.row_pairs != 0;  // uniform
    for (uint32_t j = t.row0 + threadIdx.x; j < end; j += blockDim.x) {
        const uint32_t r = nd.contiguous ? nd.seg.offset + j : rows[j];
        uint32_t w[W];
        GPair p;
        if (row_pairs) {  // the logistic pair from the row's last word (one cache line per row)
            load_bins<FG>(a.bins8 + (size_t)r * a.stride + f0, w);
            const float pv = __uint_as_float(w[W - 1] & 0x7fffffffu);
            const float y = (w[W - 1] >> 31) ? 1.0f : 0.0f;
            const float q = pv * (1.0f - pv);
            p = GPair{(pv - y) * 1.0f, (q > a.min_hess ? q : a.min_hess) * 1.0f};
        } else {
            p = gpair[r];
            load_bins<FG>(a.bins8 + (size_t)r * a.stride + f0, w);
        }
        const unsigned long long qg = (unsigned long long)quantize(p.g, eg);
        const unsigned long long qh = (unsigned long long)quantize(p.h, eh);
        // a row's missing cells add nowhere (masked rows: the group's mask
        // word, the row's last word when a row is one group of 32 bytes)
        uint32_t mask = 0u;
        if (MASKED)
            mask = a.mask_at == 4 * kMaskWord
                       ? w[kMaskWord % W]
                       : *reinterpret_cast<const uint32_t *>(a.bins8 + (size_t)r * a.stride + a.mask_at + 4 * grp);
        uint32_t v[NW];
#pragma unroll
        for (int i = 0; i < NW; i++) v[i] = w[i];
        rotate_bytes<NW>(v, rot);
#pragma unroll
        for (int f = 0; f < NF; f++) {
            uint32_t ff = (uint32_t)f + rot;
            ff = NF == FG ? ff & (FG - 1) : (ff >= (uint32_t)NF ? ff - (uint32_t)NF : ff);
            const uint32_t bin = (v[f >> 2] >> ((f & 3) * 8)) & 0xffu;
            // bin-major: a feature past nf adds its (padding) byte into its
            // own column, which is never read back
            const uint32_t at = BIN_MAJOR ? bin * FG + ff : (ff < nf ? ff * kLdsFeature + bin : kDummy + lane);
            if (MASKED && ((mask >> ff) & 1u)) continue;
            atomicAdd(&lg[at], qg);
            atomicAdd(&lh[at], qh);
        }
    }
    __syncthreads();
    const uint32_t *fo = a.feature_offset + f0;
    QBin *dst = nd.n_tiles == 1 ? a.hist + (size_t)nd.slot * a.total_bins
                                : a.partial + ((size_t)(nd.pad[0] + t.k) * a.groups + grp) * (FG * 256u);
    for (uint32_t i = threadIdx.x; i < FG * 256u; i += blockDim.x) {
        // bin-major: consecutive threads read consecutive features (no bank conflicts)
        const uint32_t ff = BIN_MAJOR ? i % FG : i >> 8, bin = BIN_MAJOR ? i / FG : i & 255u;
        if (ff >= nf) continue;
        const uint32_t at = BIN_MAJOR ? i : ff * kLdsFeature + bin;
        const QBin v{(int64_t)lg[at], (int64_t)lh[at]};
        if (nd.n_tiles == 1) {
            const uint32_t lo = fo[ff], nb = fo[ff + 1] - lo;
            if (bin < nb) {
                dst[lo + bin] = v;
                if (nd.pad[1]) {  // this workgroup alone completes these bins: sibling = parent - built
                    QBin *par = a.hist + (size_t)(nd.pad[1] - 1u) * a.total_bins + lo + bin;
                    const QBin pv = *par;
                    *par = QBin{pv.g - v.g, pv.h - v.h};
                }
            }
        } else {
            dst[ff * 256u + bin] = v;
        }
    }
}

// Sparse rows into one range of kCsrGroupBins global bins, privately in
// LDS: the workgroup's 16 waves take the tile's rows, each wave four rows
// at a time (their row pointers, pairs and entries loaded together), its
// lanes 64 entries of a row at a time; an entry in the range adds its
// row's quantised pair with LDS atomics. Then the range goes to the node's
// slot (a node of one tile) or to the tile's partial, summed by
// hbr_hist_reduce_csr. Every range of every tile is written, so slots need
// no zeroing.
constexpr uint32_t kCsrRows = 4;

__device__ __forceinline__ void hist_csr(const HistArgs &a) {
    __shared__ unsigned long long s_g[kCsrGroupBins], s_h[kCsrGroupBins];
    const uint32_t entry = blockIdx.x / a.groups, grp = blockIdx.x % a.groups;
    if (entry >= a.counts[0]) return;  // uniform across the workgroup
    const HistTile t = a.tiles[entry];
    const HistNode nd = a.nodes[t.node];
    const uint32_t lo_bin = grp * kCsrGroupBins;
    const uint32_t nb = min(kCsrGroupBins, a.total_bins - lo_bin);
    for (uint32_t i = threadIdx.x; i < nb; i += blockDim.x) s_g[i] = s_h[i] = 0ull;
    __syncthreads();
    const int eg = a.scale[nd.cls].exp_g, eh = a.scale[nd.cls].exp_h;
    const GPair *gpair = a.gpair + (size_t)nd.cls * a.class_rows;
    const uint32_t *rows = a.rows[nd.seg.buf] + nd.seg.offset;
    const uint32_t end = t.row0 + t.rows;
    const uint32_t wave = threadIdx.x / kWave, waves = blockDim.x / kWave, lane = lane_id();
    for (uint32_t j0 = t.row0 + wave; j0 < end; j0 += kCsrRows * waves) {
        uint64_t b[kCsrRows], e[kCsrRows];
        unsigned long long qg[kCsrRows], qh[kCsrRows];
        uint32_t iters = 0;
#pragma unroll
        for (uint32_t u = 0; u < kCsrRows; u++) {
            const uint32_t j = j0 + u * waves;
            const bool ok = j < end;
            const uint32_t r = ok ? (nd.contiguous ? nd.seg.offset + j : rows[j]) : 0u;
            b[u] = ok ? a.row_ptr[r] : 0ull;
            e[u] = ok ? a.row_ptr[r + 1] : 0ull;
            if (ok && a.csr_ranges) {  // only this range's entries
                const uint32_t *rg = a.csr_ranges + (size_t)r * (a.groups + 1) + grp;
                e[u] = b[u] + rg[1];
                b[u] += rg[0];
            }
            const GPair p = ok ? gpair[r] : GPair{0.0f, 0.0f};
            qg[u] = (unsigned long long)quantize(p.g, eg);
            qh[u] = (unsigned long long)quantize(p.h, eh);
            iters = max(iters, (uint32_t)((e[u] - b[u] + kWave - 1) / kWave));
        }
        for (uint32_t k = 0; k < iters; k++) {
            uint32_t d[kCsrRows];
#pragma unroll
            for (uint32_t u = 0; u < kCsrRows; u++) {
                const uint64_t x = b[u] + (uint64_t)k * kWave + lane;
                d[u] = x < e[u] ? a.gbins[x] - lo_bin : 0xffffffffu;
            }
#pragma unroll
            for (uint32_t u = 0; u < kCsrRows; u++) {
                if (d[u] < nb) {
                    atomicAdd(&s_g[d[u]], qg[u]);
                    atomicAdd(&s_h[d[u]], qh[u]);
                }
            }
        }
    }
    __syncthreads();
    QBin *dst = nd.n_tiles == 1 ? a.hist + (size_t)nd.slot * a.total_bins + lo_bin
                                : a.partial + ((size_t)(nd.pad[0] + t.k) * a.groups + grp) * kCsrGroupBins;
    for (uint32_t i = threadIdx.x; i < nb; i += blockDim.x) dst[i] = QBin{(int64_t)s_g[i], (int64_t)s_h[i]};
}

}  // namespace hbr

using namespace hbr;

// Sum of one value per thread over the (256-thread) workgroup.
__device__ __forceinline__ unsigned long long block_sum(unsigned long long v) {
    __shared__ unsigned long long lds[256 / kWave];
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, kWave);
    __syncthreads();  // earlier readers of lds are done
    if (lane_id() == 0) lds[threadIdx.x / kWave] = v;
    __syncthreads();
    unsigned long long total = 0;
    for (uint32_t w = 0; w < 256 / kWave; w++) total += lds[w];
    return total;
}

// One workgroup: resolve each node's rows, choose the tile size, number the
// tiles (and the partials of nodes cut into several tiles). The tile size is
// the smallest that cuts the nodes into at most target_tiles tiles, so that
// a launch is one wave of workgroups (no lone tail wave); when the nodes
// outnumber the target, every node is one tile.
constexpr uint32_t kPlanLdsNodes = 4096;

extern "C" __global__ __launch_bounds__(256) void hbr_hist_plan(PlanArgs a) {
    __shared__ __align__(16) uint32_t s_len[kPlanLdsNodes];  // node lengths, for the candidate counts
    __shared__ uint32_t s_first[256], s_count[256];
    const uint32_t n_nodes = a.grow ? a.grow->n_splits : a.n_nodes;
    unsigned long long sum = 0, longest = 0;
    for (uint32_t i = threadIdx.x; i < n_nodes; i += blockDim.x) {
        HistNode nd = a.nodes[i];
        const Seg s = resolve_node(a, nd);
        a.nodes[i].seg = s;
        a.nodes[i].pad[1] = nd.from_split && a.fuse_subtract ? a.splits[nd.split].parent_slot + 1u : 0u;
        if (i < kPlanLdsNodes) s_len[i] = s.len;
        sum += s.len;
        longest = max(longest, (unsigned long long)s.len);
    }
    // lengths padded with zeros (no tiles) to whole groups of four
    const uint32_t n_lds = min(n_nodes, kPlanLdsNodes), n_lds4 = (n_lds + 3u) & ~3u;
    if (threadIdx.x < n_lds4 - n_lds) s_len[n_lds + threadIdx.x] = 0u;
    const unsigned long long total = block_sum(sum);
    {
        __shared__ unsigned long long lds_max[256 / kWave];
#pragma unroll
        for (int d = 32; d >= 1; d >>= 1) longest = max(longest, __shfl_xor(longest, d, kWave));
        if (lane_id() == 0) lds_max[threadIdx.x / kWave] = longest;
        __syncthreads();
        for (uint32_t w = 0; w < 256 / kWave; w++) longest = max(longest, lds_max[w]);
    }
    // Candidate sizes spaced geometrically over [lo, hi], one per thread,
    // each counted against every node at once; the smallest that fits wins.
    // hi = the longest node fits whenever the nodes do not outnumber the
    // target (one tile each).
    const unsigned long long lo =
        max((total + a.target_tiles - 1) / a.target_tiles, (unsigned long long)a.min_rows);
    const unsigned long long hi = max(longest, lo);
    const double ratio = (double)hi / (double)lo;
    unsigned long long cand = threadIdx.x == blockDim.x - 1
                                  ? hi
                                  : (unsigned long long)((double)lo * pow(ratio, (double)threadIdx.x /
                                                                                          (double)(blockDim.x - 1)));
    cand = min(max(cand, lo), hi);
    const uint32_t c32 = (uint32_t)min(cand, 0xffffffffull);  // 32-bit divisions
    auto tiles_of = [c32](uint32_t len) { return len / c32 + (len % c32 != 0 ? 1u : 0u); };
    unsigned long long c = 0;
    // four lengths per LDS read, their divisions independent
    for (uint32_t i = 0; i < n_lds4; i += 4) {
        const uint4 l = *reinterpret_cast<const uint4 *>(&s_len[i]);
        c += (unsigned long long)(tiles_of(l.x) + tiles_of(l.y)) + (tiles_of(l.z) + tiles_of(l.w));
    }
    for (uint32_t i = kPlanLdsNodes; i < n_nodes; i++) c += tiles_of(a.nodes[i].seg.len);
    unsigned long long pick = c <= a.target_tiles ? cand : ~0ull;
    {
        __shared__ unsigned long long lds_min[256 / kWave];
#pragma unroll
        for (int d = 32; d >= 1; d >>= 1) pick = min(pick, __shfl_xor(pick, d, kWave));
        __syncthreads();
        if (lane_id() == 0) lds_min[threadIdx.x / kWave] = pick;
        __syncthreads();
        for (uint32_t w = 0; w < 256 / kWave; w++) pick = min(pick, lds_min[w]);
    }
    // More nodes than the target (a batch of class trees' deep levels): no
    // size fits, so the balanced one, lo, cuts the long nodes as it would
    // cut them alone: at most target + n_nodes tiles, and the tiles of
    // nodes of several tiles at most 2 x target (each such node's n tiles
    // hold more than (n - 1) x lo rows), which the launch and the partial
    // buffer reserve.
    const unsigned long long size = pick == ~0ull ? lo : pick;
    const uint32_t tile_rows = (uint32_t)((size + kWave - 1) / kWave * kWave);
    uint32_t carry = 0, part_carry = 0;
    for (uint32_t base = 0; base < n_nodes; base += blockDim.x) {
        const uint32_t i = base + threadIdx.x;
        const uint32_t len = i < n_nodes ? (i < kPlanLdsNodes ? s_len[i] : a.nodes[i].seg.len) : 0u;
        const uint32_t n = (len + tile_rows - 1) / tile_rows;
        uint32_t all, part_all;
        const uint32_t first = block_exclusive_scan<256>(n, &all);
        const uint32_t part_first = block_exclusive_scan<256>(n > 1 ? n : 0u, &part_all);
        if (i < n_nodes) {
            a.nodes[i].tile_begin = carry + first;
            a.nodes[i].n_tiles = n;
            a.nodes[i].pad[0] = part_carry + part_first;
        }
        s_first[threadIdx.x] = carry + first;
        s_count[threadIdx.x] = n;
        __syncthreads();
        // each wave writes the tiles of every fourth node, one tile per lane
        const uint32_t chunk = min(n_nodes - base, (uint32_t)blockDim.x);
        for (uint32_t q = threadIdx.x / kWave; q < chunk; q += blockDim.x / kWave) {
            const uint32_t qn = s_count[q], qf = s_first[q];
            const uint32_t qlen = base + q < kPlanLdsNodes ? s_len[base + q] : a.nodes[base + q].seg.len;
            for (uint32_t k = lane_id(); k < qn; k += kWave) {
                HistTile t;
                t.node = base + q;
                t.row0 = k * tile_rows;
                t.rows = min(tile_rows, qlen - k * tile_rows);
                t.k = k;
                a.tiles[qf + k] = t;
            }
        }
        __syncthreads();
        carry += all;
        part_carry += part_all;
    }
    if (threadIdx.x == 0) {
        a.counts[0] = carry;
        a.counts[1] = tile_rows;
        a.counts[2] = part_carry;
    }
}

// Dense rows of u16 local bins (features of more than 256 bins): a
// workgroup sums one tile's rows for one group of FG features into an LDS
// sub-histogram of FG x B u64 pairs ([feature][bin], B = kWideLdsBins / FG
// bins per feature), each row's FG bins read with one vector load, its pair
// from the pair array; then the node's slot (a node of one tile, its parent
// turned into the sibling as for u8 rows) or the tile's partial, which
// hbr_hist_reduce sums. Rows past a feature group's last feature hold zeros
// and add nowhere.
template <int FG>
__device__ __forceinline__ void load_bins16(const uint16_t *p, uint32_t (&w)[(FG + 1) / 2]) {
    if constexpr (FG == 16) {
        const uint4 x = reinterpret_cast<const uint4 *>(p)[0], y = reinterpret_cast<const uint4 *>(p)[1];
        w[0] = x.x; w[1] = x.y; w[2] = x.z; w[3] = x.w; w[4] = y.x; w[5] = y.y; w[6] = y.z; w[7] = y.w;
    } else if constexpr (FG == 8) {
        const uint4 x = reinterpret_cast<const uint4 *>(p)[0];
        w[0] = x.x; w[1] = x.y; w[2] = x.z; w[3] = x.w;
    } else if constexpr (FG == 4) {
        const uint2 x = reinterpret_cast<const uint2 *>(p)[0];
        w[0] = x.x; w[1] = x.y;
    } else if constexpr (FG == 2) {
        w[0] = reinterpret_cast<const uint32_t *>(p)[0];
    } else {
        w[0] = p[0];
    }
}

template <int FG>
__device__ __forceinline__ void hist_dense16(const HistArgs &a) {
    constexpr uint32_t B = kWideLdsBins / FG;
    constexpr uint32_t kWords = FG * B;
    __shared__ unsigned long long lg[kWords];
    __shared__ unsigned long long lh[kWords];
    const uint32_t entry = blockIdx.x / a.groups, grp = blockIdx.x % a.groups;
    if (entry >= a.counts[0]) return;  // uniform across the workgroup
    const HistTile t = a.tiles[entry];
    const HistNode nd = a.nodes[t.node];
    const uint32_t f0 = grp * FG;
    const uint32_t nf = min((uint32_t)FG, a.n_cols - f0);
    for (uint32_t i = threadIdx.x; i < kWords; i += blockDim.x) {
        lg[i] = 0ull;
        lh[i] = 0ull;
    }
    __syncthreads();
    const int eg = a.scale[nd.cls].exp_g, eh = a.scale[nd.cls].exp_h;
    const GPair *gpair = a.gpair + (size_t)nd.cls * a.class_rows;
    const uint32_t *rows = a.rows[nd.seg.buf] + nd.seg.offset;
    const uint32_t end = t.row0 + t.rows;
    for (uint32_t j = t.row0 + threadIdx.x; j < end; j += blockDim.x) {
        const uint32_t r = nd.contiguous ? nd.seg.offset + j : rows[j];
        uint32_t w[(FG + 1) / 2];
        load_bins16<FG>(a.bins16 + (size_t)r * a.stride16 + f0, w);
        const GPair p = gpair[r];
        const unsigned long long qg = (unsigned long long)quantize(p.g, eg);
        const unsigned long long qh = (unsigned long long)quantize(p.h, eh);
#pragma unroll
        for (int f = 0; f < FG; f++) {
            if ((uint32_t)f >= nf) break;
            const uint32_t bin = FG == 1 ? w[0] & 0xffffu : (w[f >> 1] >> ((f & 1) * 16)) & 0xffffu;
            atomicAdd(&lg[f * B + bin], qg);
            atomicAdd(&lh[f * B + bin], qh);
        }
    }
    __syncthreads();
    const uint32_t *fo = a.feature_offset + f0;
    QBin *dst = nd.n_tiles == 1 ? a.hist + (size_t)nd.slot * a.total_bins
                                : a.partial + ((size_t)(nd.pad[0] + t.k) * a.groups + grp) * kWords;
    for (uint32_t i = threadIdx.x; i < kWords; i += blockDim.x) {
        const uint32_t ff = i / B, bin = i % B;
        if (ff >= nf) continue;
        const QBin v{(int64_t)lg[i], (int64_t)lh[i]};
        if (nd.n_tiles == 1) {
            const uint32_t lo = fo[ff], nb = fo[ff + 1] - lo;
            if (bin < nb) {
                dst[lo + bin] = v;
                if (nd.pad[1]) {  // this workgroup alone completes these bins: sibling = parent - built
                    QBin *par = a.hist + (size_t)(nd.pad[1] - 1u) * a.total_bins + lo + bin;
                    const QBin pv = *par;
                    *par = QBin{pv.g - v.g, pv.h - v.h};
                }
            }
        } else {
            dst[i] = v;
        }
    }
}

// Launched with 512 or 1024 threads.
extern "C" __global__ __launch_bounds__(1024) void hbr_hist_dense8_fg8(HistArgs a) { hist_dense8<8, false>(a); }
extern "C" __global__ __launch_bounds__(1024) void hbr_hist_dense8_fg16(HistArgs a) { hist_dense8<16, false>(a); }
extern "C" __global__ __launch_bounds__(1024) void hbr_hist_dense8_fg32(HistArgs a) { hist_dense8<32, false>(a); }
extern "C" __global__ __launch_bounds__(1024) void hbr_hist_dense8_fg16_bm(HistArgs a) { hist_dense8<16, true>(a); }
extern "C" __global__ __launch_bounds__(1024) void hbr_hist_dense8_fg32_bm(HistArgs a) { hist_dense8<32, true>(a); }
extern "C" __global__ __launch_bounds__(1024) void hbr_hist_dense16_fg16(HistArgs a) { hist_dense16<16>(a); }
extern "C" __global__ __launch_bounds__(1024) void hbr_hist_dense16_fg8(HistArgs a) { hist_dense16<8>(a); }
extern "C" __global__ __launch_bounds__(1024) void hbr_hist_dense16_fg4(HistArgs a) { hist_dense16<4>(a); }
extern "C" __global__ __launch_bounds__(1024) void hbr_hist_dense16_fg2(HistArgs a) { hist_dense16<2>(a); }
extern "C" __global__ __launch_bounds__(1024) void hbr_hist_dense16_fg1(HistArgs a) { hist_dense16<1>(a); }
// Masked rows (a missing mask in word kMaskWord): one group of 32 features.
extern "C" __global__ __launch_bounds__(1024) void hbr_hist_dense8_fg32_bm_masked(HistArgs a) {
    hist_dense8<32, true, true>(a);
}
// Rows of 25 to 28 features (one group): no atomics for the padding columns.
extern "C" __global__ __launch_bounds__(1024) void hbr_hist_dense8_fg32_bm_nf28(HistArgs a) {
    hist_dense8<32, true, false, 28>(a);
}
extern "C" __global__ __launch_bounds__(1024) void hbr_hist_dense8_fg32_bm_masked_nf28(HistArgs a) {
    hist_dense8<32, true, true, 28>(a);
}
extern "C" __global__ __launch_bounds__(1024) void hbr_hist_csr(HistArgs a) { hist_csr(a); }

// Nodes cut into several tiles: the slot is the sum of the tiles' partials.
// A workgroup takes 64 bins of one feature of one node (a.quarters
// workgroups per feature); its 16 waves split the node's tiles, then
// combine in LDS.
extern "C" __global__ __launch_bounds__(1024) void hbr_hist_reduce(ReduceArgs a) {
    __shared__ int64_t acc[2][16][64];
    const uint32_t f = blockIdx.x / a.quarters, quarter = blockIdx.x % a.quarters;
    if (a.grow && blockIdx.y >= a.grow->n_splits) return;
    const HistNode nd = a.nodes[blockIdx.y];
    if (f >= a.n_cols || nd.n_tiles == 1) return;  // uniform across the workgroup
    const uint32_t lo = a.feature_offset[f], nb = a.feature_offset[f + 1] - lo;
    if (quarter * 64u >= nb) return;
    const uint32_t col = threadIdx.x & 63u, ks = threadIdx.x >> 6;
    const uint32_t bin = quarter * 64u + col;
    const uint32_t grp = f / a.fg, local = (f % a.fg) * a.group_bins + bin;
    int64_t g = 0, h = 0;
    if (bin < nb) {
        for (uint32_t k = ks; k < nd.n_tiles; k += 16) {
            const QBin q = a.partial[((size_t)(nd.pad[0] + k) * a.groups + grp) * (a.fg * a.group_bins) + local];
            g += q.g;
            h += q.h;
        }
    }
    acc[0][ks][col] = g;
    acc[1][ks][col] = h;
    __syncthreads();
    if (ks == 0 && bin < nb) {
        for (uint32_t k = 1; k < 16; k++) {
            g += acc[0][k][col];
            h += acc[1][k][col];
        }
        a.hist[(size_t)nd.slot * a.total_bins + lo + bin] = QBin{g, h};
        if (nd.pad[1]) {  // sibling = parent - built
            QBin *par = a.hist + (size_t)(nd.pad[1] - 1u) * a.total_bins + lo + bin;
            const QBin pv = *par;
            *par = QBin{pv.g - g, pv.h - h};
        }
    }
}

// One thread per row: the row's first entry of every bin range (the
// entries' global bins ascend), relative to the row's first entry.
extern "C" __global__ __launch_bounds__(256) void hbr_csr_ranges(CsrRangeArgs a) {
    const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= a.n_rows) return;
    const uint64_t b = a.row_ptr[r], e = a.row_ptr[r + 1];
    uint32_t *out = a.ranges + (size_t)r * (a.groups + 1);
    uint32_t g = 0;
    out[0] = 0;
    for (uint64_t x = b; x < e; x++) {
        const uint32_t gg = min(a.gbins[x] / kCsrGroupBins, a.groups);
        while (g < gg) out[++g] = (uint32_t)(x - b);
    }
    while (g < a.groups) out[++g] = (uint32_t)(e - b);
}

// Nodes of several tiles (CSR): slot bin b = the sum of the tiles' partials.
extern "C" __global__ __launch_bounds__(256) void hbr_hist_reduce_csr(ReduceArgs a) {
    const HistNode nd = a.nodes[blockIdx.y];
    const uint32_t b = blockIdx.x * blockDim.x + threadIdx.x;
    if (nd.n_tiles == 1 || b >= a.total_bins) return;
    const QBin *src = a.partial + (size_t)nd.pad[0] * a.groups * kCsrGroupBins + (size_t)(b / kCsrGroupBins) * kCsrGroupBins +
                      b % kCsrGroupBins;
    int64_t g = 0, h = 0;
    for (uint32_t k = 0; k < nd.n_tiles; k++) {
        const QBin q = src[(size_t)k * a.groups * kCsrGroupBins];
        g += q.g;
        h += q.h;
    }
    a.hist[(size_t)nd.slot * a.total_bins + b] = QBin{g, h};
}

// ---- a histogram of a caller's device row list in a fixed scratch area ----

extern "C" __global__ __launch_bounds__(64) void hbr_fixed_begin(FixedBuildArgs a) {
    if (threadIdx.x == 0) *a.flag = 0u;
}

// Any row id at or beyond the index's rows sets the word.
extern "C" __global__ __launch_bounds__(256) void hbr_fixed_check(FixedBuildArgs a) {
    bool bad = false;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.m; i += (uint64_t)gridDim.x * blockDim.x)
        bad |= a.rows[i] >= a.n_rows;
    if (__ballot(bad) != 0ull && lane_id() == 0) atomicOr(a.flag, 1u);
}

// The node record: every row of the list, or none when an id was out of
// range (the kernels after it then read no row and the bins are zero).
extern "C" __global__ __launch_bounds__(64) void hbr_fixed_node(FixedBuildArgs a) {
    if (threadIdx.x != 0) return;
    HistNode nd{};
    nd.seg = Seg{0u, *a.flag ? 0u : (uint32_t)a.m, 0u, 0u};
    nd.slot = 0u;
    *a.node = nd;
}

// int64 bins to f64 pairs in place, each by its exponent: the host's
// ldexp((double)q, e) on the same bits.
extern "C" __global__ __launch_bounds__(256) void hbr_fixed_finish(FixedBuildArgs a) {
    const uint32_t b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= a.total_bins) return;
    const QBin q = a.bins[b];
    const int eg = a.scale->exp_g, eh = a.scale->exp_h;
    a.out[2 * (size_t)b] = ldexp((double)q.g, eg);
    a.out[2 * (size_t)b + 1] = ldexp((double)q.h, eh);
}

// sibling = parent - built (exact in integers), in the parent's slot.
extern "C" __global__ __launch_bounds__(256) void hbr_subtract(SubArgs a) {
    const uint32_t s = blockIdx.y;
    if (s >= a.n_splits) return;
    const PartSplit sp = a.splits[s];
    QBin *parent = a.hist + (size_t)sp.parent_slot * a.total_bins;
    const QBin *built = a.hist + (size_t)sp.fresh_slot * a.total_bins;
    for (uint32_t b = blockIdx.x * blockDim.x + threadIdx.x; b < a.total_bins; b += gridDim.x * blockDim.x) {
        QBin p = parent[b];
        const QBin c = built[b];
        p.g -= c.g;
        p.h -= c.h;
        parent[b] = p;
    }
}


// ---- the reference's CPU sum order (replays) -----------------------------------
// Each bin is the f64 chain of its rows' f32 values in row order, from +0.0,
// within each block of `grain` rows (builder order of tree/hist/mod.rs:
// accumulate, accumulate_blocks); thread f walks the block's rows and adds
// into feature f's bins only, so no bin has two writers. Rows are fetched
// eight at a time ahead of the adds.
extern "C" __global__ __launch_bounds__(kExactThreads) void hbr_hist_exact(ExactArgs a) {
    __shared__ double s_h[kExactMaxWords];
    const uint32_t words = 2u * a.total_bins;
    for (uint32_t i = threadIdx.x; i < words; i += blockDim.x) s_h[i] = 0.0;
    __syncthreads();
    const uint32_t blk = a.blk0 + blockIdx.x;
    const uint32_t start = blk * a.grain;
    const uint32_t end = min(a.m, start + a.grain);
    const uint32_t f = threadIdx.x;
    if (f < a.n_cols) {
        const uint32_t base = a.feature_offset[f];
        constexpr uint32_t kAhead = 8;
        for (uint32_t j0 = start; j0 < end; j0 += kAhead) {
            uint32_t bin[kAhead], mask[kAhead];
            GPair p[kAhead];
#pragma unroll
            for (uint32_t k = 0; k < kAhead; k++) {
                const uint32_t j = j0 + k;
                bin[k] = 0;
                mask[k] = 1u;
                p[k] = GPair{0.0f, 0.0f};
                if (j >= end) continue;
                const uint32_t r = a.rows ? a.rows[j] : a.first + j;
                const uint8_t *row = a.bins8 + (size_t)r * a.stride;
                bin[k] = row[f];
                const uint32_t word = *reinterpret_cast<const uint32_t *>(row + 4 * kMaskWord);
                mask[k] = a.masked ? (*reinterpret_cast<const uint32_t *>(row + a.mask_at + 4 * (f >> 5)) >> (f & 31u)) &
                                         1u
                                   : 0u;
                if (a.row_pairs) {
                    const float pv = __uint_as_float(word & 0x7fffffffu);
                    const float y = (word >> 31) ? 1.0f : 0.0f;
                    const float q = pv * (1.0f - pv);
                    p[k] = GPair{(pv - y) * 1.0f, (q > a.min_hess ? q : a.min_hess) * 1.0f};
                } else {
                    p[k] = a.gpair[r];
                }
            }
#pragma unroll
            for (uint32_t k = 0; k < kAhead; k++) {
                if (mask[k]) continue;
                const uint32_t at = 2u * (base + bin[k]);
                s_h[at] += (double)p[k].g;
                s_h[at + 1] += (double)p[k].h;
            }
        }
    }
    __syncthreads();
    double *dst = a.partial + (size_t)blockIdx.x * words;
    for (uint32_t i = threadIdx.x; i < words; i += blockDim.x) dst[i] = s_h[i];
}

// out = block 0's partial (first launch) then + each later block's, in order;
// or out -= minus (a sibling's bins from its parent's and the built child's).
extern "C" __global__ __launch_bounds__(256) void hbr_hist_exact_sum(ExactSumArgs a) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= a.n) return;
    if (a.minus) {
        a.out[i] = a.out[i] - a.minus[i];
        return;
    }
    uint32_t k = 0;
    double v;
    if (a.first) {
        v = a.partial[i];
        k = 1;
    } else {
        v = a.out[i];
    }
    for (; k < a.n_blocks; k++) v += a.partial[(size_t)k * a.n + i];
    a.out[i] = v;
}
