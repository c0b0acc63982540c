// Depthwise growth decided on the device: one workgroup per level turns the
// frontier's winners into splits or leaves, so that a whole tree is grown
// from one stream of launches and read back once.
//
// Restates, per frontier node and in frontier order, the host builder's
// level step (builder/hist/mod.rs:458-573 depthwise frontier;
// builder/mod.rs:167-193 SplitPos and BestSplit::valid; builder/shared.rs:
// 89-141 bounded weights and node gains, :174-187 final leaf values;
// tree/constraints.rs child bounds at the f64 midpoint): node ids of the
// children are appended in frontier order (left, right), a split whose
// children sit at the depth limit makes two leaves, and every leaf's value
// is calc_weight clamped to its bounds, rounded to f32, times eta.
//
// Histogram slots: the built child of split i takes the i-th slot (in
// ascending order) that no splitting parent holds; its sibling keeps the
// parent's slot (the histogram kernels turn the parent into the sibling).
//
// A batched level decides the levels of several trees at once (the class
// trees of a softmax round): the frontier holds their nodes in tree order,
// each tree numbers its own nodes (children appended in its frontier order)
// and writes its own records and header; slots, splits and tiles are
// shared.
#include "common.h"

namespace hbr {

// calc_weight (tree/gain.rs:107-116) then Bounds::clamp, in f64.
__device__ __forceinline__ double leaf_weight(double g, double h, const ScanParams &r, double lower, double upper) {
    double w = 0.0;
    if (!(h < r.min_child_weight || h <= 0.0)) {
        w = -threshold_l1(g, r.alpha) / (h + r.lambda);
        if (r.max_delta_step > 0.0)
            w = w < -r.max_delta_step ? -r.max_delta_step : (w > r.max_delta_step ? r.max_delta_step : w);
    }
    if (w < lower) w = lower;
    if (w > upper) w = upper;
    return w;
}

// f64::midpoint.
__device__ __forceinline__ double midpoint(double a, double b) {
    const double hi = 1.7976931348623157e308 / 2.0, lo = 2.2250738585072014e-308 * 2.0;
    if (__builtin_fabs(a) <= hi && __builtin_fabs(b) <= hi) return (a + b) / 2.0;
    if (__builtin_fabs(a) < lo) return a + b / 2.0;
    if (__builtin_fabs(b) < lo) return a / 2.0 + b;
    return a / 2.0 + b / 2.0;
}

constexpr uint32_t kGrowThreads = 512;
constexpr uint32_t kGrowLdsOffsets = 4096;  // feature offsets kept in LDS (more features read them from memory)
constexpr uint32_t kGrowSlotWords = kGrowMaxSlots / 32;

__device__ __forceinline__ GrowTreeNode *tree_of(const GrowArgs &a, uint32_t t) {
    return reinterpret_cast<GrowTreeNode *>(reinterpret_cast<char *>(a.tree) + (size_t)t * a.tree_bytes);
}

__device__ __forceinline__ TreeHeader *header_of(const GrowArgs &a, uint32_t t) {
    return reinterpret_cast<TreeHeader *>(reinterpret_cast<char *>(a.header) + (size_t)t * a.tree_bytes);
}

}  // namespace hbr

using namespace hbr;

template <bool BATCHED>
__device__ __forceinline__ void grow_decide(const GrowArgs &a) {
    __shared__ uint32_t s_used[kGrowSlotWords];   // slots of splitting parents
    __shared__ uint32_t s_free[kGrowMaxSlots];    // the other slots, ascending
    __shared__ uint32_t s_fo[kGrowLdsOffsets + 1];
    __shared__ uint32_t s_tile_begin[kGrowMaxSlots / 2];  // first tile of each split
    // batched: each tree's node count before this level, its first split of
    // the level, its splits and its quantisation exponents
    __shared__ uint32_t s_base[BATCHED ? kGrowMaxTrees : 1];
    __shared__ uint32_t s_first[BATCHED ? kGrowMaxTrees : 1];
    __shared__ uint32_t s_nsplit[BATCHED ? kGrowMaxTrees : 1];
    __shared__ int2 s_exp[BATCHED ? kGrowMaxTrees : 1];
    __shared__ GrowCounts s_final;  // the level's counts as thread 0 writes them
    const uint32_t tid = threadIdx.x;
    const uint32_t n_trees = BATCHED ? a.n_trees : 1u;
    if (BATCHED) {
        // the per-tree loads first: a wait for a load waits for every load
        // issued before it; these are needed before the first barrier, the
        // records read ahead below only in the loop
        for (uint32_t t = tid; t < n_trees; t += kGrowThreads) {
            s_first[t] = 0xffffffffu;
            s_nsplit[t] = 0u;
            s_exp[t] = make_int2(a.scale[t].exp_g, a.scale[t].exp_h);
            s_base[t] = a.level == 0 ? 1u : a.tree_nodes[t];
        }
    }
    const bool fo_lds = a.n_features <= kGrowLdsOffsets;
    if (fo_lds)
        for (uint32_t k = tid; k <= a.n_features; k += kGrowThreads) s_fo[k] = a.feature_offset[k];
    // Every record a thread may need is loaded at once, before the counts
    // say which frontier nodes exist (the arrays hold front_cap records), so
    // that the level costs one round trip to memory.
    const uint32_t j0 = tid;
    const bool cap0 = j0 < a.front_cap;
    GrowNode g0{};
    PartSplit sp0{};
    PartOut po0{};
    ScanBest b0{};
    if (cap0 && a.level > 0) {
        g0 = a.front[j0];
        sp0 = a.prev_splits[j0 >> 1];
        po0 = a.prev_out[j0 >> 1];
    }
    if (cap0) b0 = a.best[j0];
    QBin root_total{0, 0};
    if (a.level == 0 && cap0) root_total = a.root_total[j0];
    GrowCounts c0 = *a.counts;
    if (a.level == 0) {
        c0.n_front = n_trees;
        c0.n_nodes = n_trees;
        c0.hist_nodes = n_trees;
        c0.error = 0;
        c0.hist_rows = 0;
        c0.part_rows = 0;
        c0.near_ties = 0;
    }
    const uint32_t n_front = c0.n_front, node_base = c0.n_nodes;
    const int eg1 = BATCHED ? 0 : a.scale->exp_g, eh1 = BATCHED ? 0 : a.scale->exp_h;
    for (uint32_t w = tid; w < kGrowSlotWords; w += kGrowThreads) s_used[w] = 0u;
    __syncthreads();

    uint32_t split_carry = 0, tile_carry = 0;
    unsigned long long hist_rows = 0, part_rows = 0;
    uint32_t near_ties = 0;
    for (uint32_t base = 0; base < n_front; base += kGrowThreads) {
        const uint32_t j = base + tid;
        const bool active = j < n_front;
        // the node: its rows, slot, statistics and bounds
        Seg seg{0u, 0u, 0u, 0u};
        uint32_t slot = 0, nid = 0, identity = 0, tree = 0;
        QBin total{0, 0};
        double lower = -__builtin_inf(), upper = __builtin_inf();
        ScanBest b{};
        if (active && a.level == 0) {
            tree = j;  // the roots: all rows of each tree, in its own region of the row buffers
            seg = Seg{j * a.n_rows, a.n_rows, 0u, 0u};
            identity = 1;
            slot = a.root_slot + j;
            total = root_total;
            b = b0;
        } else if (active) {
            const bool first = base == 0;
            const GrowNode g = first ? g0 : a.front[j];
            const uint32_t i = j >> 1, c = j & 1u;
            const PartSplit sp = first ? sp0 : a.prev_splits[i];
            const PartOut po = first ? po0 : a.prev_out[i];
            b = first ? b0 : a.best[j];
            const uint32_t nl = po.left_len;
            seg.buf = sp.seg.buf ^ 1u;
            seg.offset = c == 0 ? sp.seg.offset : sp.seg.offset + nl;
            seg.len = c == 0 ? nl : sp.seg.len - nl;
            const bool built = (c == 0) == (po.built_left != 0);
            slot = built ? sp.fresh_slot : sp.parent_slot;
            total = g.total;
            lower = g.lower;
            upper = g.upper;
            nid = g.nid;
            tree = g.tree;
            if (c == 0) {
                part_rows += sp.seg.len;
                hist_rows += po.built_left ? nl : sp.seg.len - nl;
            }
        }
        if (active && (b.flags & kScanNearTie)) near_ties++;
        const int eg = BATCHED ? s_exp[active ? tree : 0u].x : eg1, eh = BATCHED ? s_exp[active ? tree : 0u].y : eh1;
        GrowTreeNode *records = BATCHED ? tree_of(a, tree) : a.tree;
        const double ng = dequant(total.g, eg), nh = dequant(total.h, eh);
        // the winner as a split position (builder/mod.rs:167-193)
        bool valid = false;
        uint32_t f = 0, limit = 0, dl = 0;
        int32_t bin = -1;
        double lg = 0, lh = 0, rg = 0, rh = 0;
        float wl = 0.0f, wr = 0.0f;
        if (active) {
            if (b.index != 0xffffffffu) {
                f = b.feature;
                const uint32_t fs = fo_lds ? s_fo[f] : a.feature_offset[f];
                const uint32_t nb = (fo_lds ? s_fo[f + 1] : a.feature_offset[f + 1]) - fs;
                if (b.index < nb) {
                    bin = (int32_t)(fs + b.index);
                    limit = b.index + 1;
                    dl = 0;
                } else {
                    const uint32_t off = nb - 1 - (b.index - nb);
                    bin = off == 0 ? -1 : (int32_t)(fs + off - 1);
                    limit = off;
                    dl = 1;
                }
                lg = dequant(b.left.g, eg);
                lh = dequant(b.left.h, eh);
                rg = dequant(b.right.g, eg);
                rh = dequant(b.right.h, eh);
                wl = bounded_weight(lg, lh, a.reg, (float)lower, (float)upper);
                wr = bounded_weight(rg, rh, a.reg, (float)lower, (float)upper);
                const double loss = (double)b.loss;
                valid = loss > 1e-6 && loss >= a.gamma && lh > 0.0 && rh > 0.0 && lh >= a.reg.min_child_weight &&
                        rh >= a.reg.min_child_weight;
            }
        }
        const uint32_t tiles = valid && !a.terminal ? (seg.len + kPartTile - 1) / kPartTile : 0u;
        uint32_t n_valid, n_tiles;
        const uint32_t i = split_carry + block_exclusive_scan<kGrowThreads>(valid ? 1u : 0u, &n_valid);
        const uint32_t tile_begin = tile_carry + block_exclusive_scan<kGrowThreads>(tiles, &n_tiles);
        // each tree's first split of the level (the frontier is in tree order)
        if (BATCHED) {
            if (active && valid) {
                atomicMin(&s_first[tree], i);
                atomicAdd(&s_nsplit[tree], 1u);
            }
            __syncthreads();
        }
        if (active && a.level == 0) {
            GrowTreeNode r{};
            r.left = -1;
            r.bin = -2;
            r.default_left = 1;
            r.sum_hess = (float)nh;
            records[0] = r;
        }
        if (active && !valid) {
            // a leaf: builder/shared.rs:174-187 then scale_leaves(eta)
            const float w = (float)leaf_weight(ng, nh, a.reg, lower, upper);
            records[nid].value = w * a.eta;
        } else if (active) {
            const uint32_t left = BATCHED ? s_base[tree] + 2 * (i - s_first[tree]) : node_base + 2 * i;
            GrowTreeNode &r = records[nid];
            r.left = (int32_t)left;
            r.feature = f;
            r.limit = limit;
            r.bin = bin;
            r.default_left = dl;
            r.gain = b.loss;
            // child bounds (tree/constraints.rs) at the midpoint of the f32 weights
            double cb[4] = {lower, upper, lower, upper};
            const int dir = f < a.n_monotone && a.monotone ? (int)a.monotone[f] : 0;
            if (dir != 0) {
                const double mid = midpoint((double)wl, (double)wr);
                if (dir > 0) {
                    cb[1] = mid;
                    cb[2] = mid;
                } else {
                    cb[0] = mid;
                    cb[3] = mid;
                }
            }
            const double cg[2] = {lg, rg}, ch[2] = {lh, rh};
            const float cw[2] = {wl, wr};
            const QBin ct[2] = {b.left, b.right};
#pragma unroll
            for (uint32_t c = 0; c < 2; c++) {
                GrowTreeNode k{};
                k.left = -1;
                k.bin = -2;
                k.default_left = 1;
                k.value = cw[c];
                k.sum_hess = (float)ch[c];
                if (a.terminal) {
                    const float w = (float)leaf_weight(cg[c], ch[c], a.reg, cb[2 * c], cb[2 * c + 1]);
                    k.value = w * a.eta;
                } else {
                    GrowNode g{};
                    g.total = ct[c];
                    g.lower = cb[2 * c];
                    g.upper = cb[2 * c + 1];
                    g.nid = left + c;
                    g.tree = tree;
                    a.next[2 * i + c] = g;
                    ScanNode s{};
                    s.from_split = 1;
                    s.split = i;
                    s.child = c;
                    s.pad = tree << kScanClassShift;
                    s.total = ct[c];
                    s.root_gain = node_gain(cg[c], ch[c], a.reg, (float)cb[2 * c], (float)cb[2 * c + 1]);
                    s.lower = (float)cb[2 * c];
                    s.upper = (float)cb[2 * c + 1];
                    a.snodes[2 * i + c] = s;
                }
                records[left + c] = k;
            }
            if (!a.terminal) {
                PartSplit p{};
                p.seg = seg;
                p.feature = f;
                p.limit = limit;
                p.default_left = dl;
                p.identity = identity;
                p.tile_begin = tile_begin;
                p.parent_slot = slot;
                p.tree = tree;
                a.splits[i] = p;
                s_tile_begin[i] = tile_begin;
                HistNode h{};
                h.from_split = 1;
                h.split = i;
                h.cls = tree;
                a.hnodes[i] = h;
                if (slot < a.slot_cap && slot < kGrowMaxSlots) atomicOr(&s_used[slot >> 5], 1u << (slot & 31));
            }
        }
        split_carry += n_valid;
        tile_carry += n_tiles;
    }
    // the built children's slots: the split_carry lowest slots no splitting parent holds
    __syncthreads();
    const uint32_t n_splits = a.terminal ? 0u : split_carry;
    {
        const uint32_t w = tid;
        const uint32_t cap_words = (min(a.slot_cap, kGrowMaxSlots) + 31) / 32;
        uint32_t free_bits = 0;
        if (w < cap_words) {
            const uint32_t valid_bits = (w + 1) * 32 <= a.slot_cap ? ~0u : (1u << (a.slot_cap - w * 32)) - 1u;
            free_bits = ~s_used[w] & valid_bits;
        }
        uint32_t n_free;
        const uint32_t first = block_exclusive_scan<kGrowThreads>((uint32_t)__popc(free_bits), &n_free);
        uint32_t k = first;
        while (free_bits) {
            const uint32_t bit = (uint32_t)__builtin_ctz(free_bits);
            free_bits &= free_bits - 1u;
            s_free[k++] = w * 32 + bit;
        }
        __syncthreads();
        for (uint32_t i = tid; i < n_splits; i += kGrowThreads) {
            const uint32_t slot = i < n_free ? s_free[i] : 0u;
            a.splits[i].fresh_slot = slot;
            a.hnodes[i].slot = slot;
        }
        // the split of every partition tile: the last split whose first tile
        // is at or before it (a split's tiles are contiguous)
        if (a.tile_split && n_splits > 0) {
            for (uint32_t t = tid; t < tile_carry; t += kGrowThreads) {
                uint32_t lo = 0, hi = n_splits;
                while (hi - lo > 1) {
                    const uint32_t mid = (lo + hi) / 2;
                    if (s_tile_begin[mid] <= t) lo = mid;
                    else hi = mid;
                }
                a.tile_split[t] = lo;
            }
        }
        if (tid == 0) {
            GrowCounts c = c0;
            c.n_front = n_splits * 2;
            c.n_splits = n_splits;
            c.n_tiles = a.terminal ? 0u : tile_carry;
            c.n_nodes = node_base + 2 * split_carry;
            c.hist_nodes += n_splits;
            if (n_splits > n_free) c.error = 1;
            a.counts[0] = c;
            s_final = c;
        }
        if (BATCHED)
            for (uint32_t t = tid; t < n_trees; t += kGrowThreads) a.tree_nodes[t] = s_base[t] + 2 * s_nsplit[t];
    }
    // per-thread row counts of the previous level's splits
    __shared__ unsigned long long s_rows[3][kGrowThreads / kWave];
    unsigned long long nt = near_ties;
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        hist_rows += __shfl_xor(hist_rows, d, kWave);
        part_rows += __shfl_xor(part_rows, d, kWave);
        nt += __shfl_xor(nt, d, kWave);
    }
    if (lane_id() == 0) {
        s_rows[0][tid / kWave] = hist_rows;
        s_rows[1][tid / kWave] = part_rows;
        s_rows[2][tid / kWave] = nt;
    }
    __syncthreads();
    if (tid == 0) {
        unsigned long long hr = 0, pr = 0, ties = 0;
        for (uint32_t w = 0; w < kGrowThreads / kWave; w++) {
            hr += s_rows[0][w];
            pr += s_rows[1][w];
            ties += s_rows[2][w];
        }
        a.counts->hist_rows = c0.hist_rows + hr;
        a.counts->part_rows = c0.part_rows + pr;
        a.counts->near_ties = c0.near_ties + (uint32_t)ties;
        s_final.hist_rows = c0.hist_rows + hr;
        s_final.part_rows = c0.part_rows + pr;
        s_final.near_ties = c0.near_ties + (uint32_t)ties;
    }
    // each tree's header: its scale and node count, and the level counts
    // (a batch's totals)
    if (a.terminal && a.header) {
        __syncthreads();
        for (uint32_t t = tid; t < n_trees; t += kGrowThreads) {
            TreeHeader h;
            h.scale = a.scale[t];
            h.counts = s_final;
            if (BATCHED) h.counts.n_nodes = s_base[t] + 2 * s_nsplit[t];
            *header_of(a, t) = h;
        }
    }
}

extern "C" __global__ __launch_bounds__(512) void hbr_grow_decide(GrowArgs a) { grow_decide<false>(a); }
extern "C" __global__ __launch_bounds__(512) void hbr_grow_decide_batch(GrowArgs a) { grow_decide<true>(a); }
