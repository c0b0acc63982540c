// Batched ensemble prediction: one lane per row, trees in order.
//
// Restates the margin walk (model/predict.rs:60-193, compact/mod.rs:1052-1095):
// out = base_score, then for every tree in ascending order
// out[output(t)] += weight(t) * leaf(t, row) in f32 (a multiply, then an
// add); a present value goes left iff value < threshold, a missing one
// follows default_left (tree/mod.rs:52-58). A categorical split sends a
// present value left iff its category is in the node's set; forests with
// such splits take hbr_predict (the category pool read from global memory).
//
// The walks that keep rows resident: a workgroup is one wave; it stages a
// 64-row block in LDS once, feature-major (row l of feature f at f * 64 + l,
// so that lane l reads bank l whatever the feature), and walks it through
// every tree, 16 trees in flight per lane, reading the trees through the
// caches. A wave-wide node load costs about 4 cycles of the texture path per
// distinct 128-byte line it touches (16 at least, 64 at most) whatever its
// width, so the walks spend their loads where the lanes' nodes diverge:
//  - hbr_predict_pairs (the default where the forest allows): complete trees,
//    one 16-byte record per two levels, the last load only the leaf's value;
//  - hbr_predict_mirror: any numeric forest, one 8-byte node per level, the
//    missing value's child first so that every step is a compare and an add;
//  - hbr_predict_resident: compact records, for thresholds the mirror form
//    cannot take (infinities).
// hbr_predict_chunked keeps chunks of the forest in LDS instead and
// re-stages the rows for every chunk; it serves rows too wide for the
// resident walks' LDS block.
//
// hbr_predict_staged: a workgroup is one wave and 64 rows staged in LDS as
// above; every lane walks its row through all trees, eight at a time, the
// leaf values added one tree after another, in order. Nodes are 16-byte
// records read through the caches. hbr_predict reads features from the
// row-major rows directly (rows too wide for LDS, categorical splits).
#include "common.h"

using namespace hbr;

namespace hbr {

// Rust's saturating `v as u32`: NaN and values below 1 give 0, values at or
// above 2^32 give u32::MAX, the rest truncate (tree/mod.rs:34-36).
__device__ __forceinline__ uint32_t category_of(float v) {
    if (!(v >= 1.0f)) return 0u;
    if (v >= 4294967296.0f) return 0xffffffffu;
    return (uint32_t)v;
}

__device__ __forceinline__ bool in_categories(const PredictArgs &a, uint32_t nid, float v) {
    const uint32_t c = category_of(v);
    const uint32_t end = a.node_cat_end[nid];
    bool hit = false;
    for (uint32_t i = a.node_value[nid]; i < end; i++) hit |= a.categories[i] == c;
    return hit;
}

__device__ __forceinline__ uint32_t walk(const PredictArgs &a, const float *row, uint32_t nid) {
    for (;;) {
        const uint32_t meta = a.node_meta[nid];
        if (meta >> 31) return nid;
        const float v = row[meta & 0xfffffu];
        const bool miss = a.missing_is_nan ? __builtin_isnan(v) : (v == a.missing);
        bool left;
        if (miss)
            left = ((meta >> 30) & 1u) != 0;
        else if (meta & kPredCategorical)
            left = in_categories(a, nid, v);
        else
            left = v < __uint_as_float(a.node_value[nid]);
        nid = a.node_left[nid] + (left ? 0u : 1u);
    }
}

// 1 when a row goes to the right child of a compact node: a present value
// goes right unless value < threshold, a missing one unless default_left
// (meta bit 30). Bit arithmetic rather than a select, which the compiler
// would turn into a branch per chain. MISSING_NAN: the missing value is
// NaN, which compares false and so goes right unless default_left.
template <bool MISSING_NAN>
__device__ __forceinline__ uint32_t goes_right(float v, uint32_t meta, uint32_t thr_bits, float missing) {
    const uint32_t not_lt = v < __uint_as_float(thr_bits) ? 0u : 1u;
    const uint32_t dl = (meta >> 30) & 1u;
    if (MISSING_NAN) {
        const uint32_t nan = v != v ? 1u : 0u;
        return not_lt & ~(nan & dl);
    }
    const uint32_t miss = 0u - (v == missing ? 1u : 0u);
    return (not_lt & ~miss) | ((dl ^ 1u) & miss);
}

constexpr uint32_t kPredLanes = 64;
constexpr int kPredChains = 8;

// Copy a block of `rows` consecutive rows (rows * n_cols floats, contiguous;
// 16-byte aligned when the rows are, blocks starting at multiples of 64 rows) into LDS
// feature-major, s_x[f * kPredPitch + row]. The wave's lanes read 16 bytes
// each, consecutive, several loads in flight.
// MIRROR: feature f goes to slot f + 1 (slot 0 holds NaN for the mirror
// walk's leaves) and, unless MISSING_NAN, the missing value becomes NaN and
// a present NaN +inf (mirror_value).
template <bool MISSING_NAN>
__device__ __forceinline__ float mirror_value(float v, float missing) {
    if (MISSING_NAN) return v;
    return v == missing ? __builtin_nanf("") : (v != v ? __builtin_inff() : v);
}

template <bool NT = false, bool MIRROR = false, bool MISSING_NAN = true>
__device__ __forceinline__ void stage_rows(float *s_x, const float *src, uint32_t rows, uint32_t n_cols,
                                           uint32_t lane, float missing = 0.0f) {
    if (MIRROR) s_x += kPredPitch;
    const uint32_t total = rows * n_cols;
    const uint32_t n4 = ((uintptr_t)src & 15u) == 0 ? total / 4 : 0;  // an unaligned caller pointer: scalar
    const float inv = 1.0f / (float)n_cols;
    const float4 *src4 = reinterpret_cast<const float4 *>(src);
#pragma unroll 5
    for (uint32_t i = lane; i < n4; i += kPredLanes) {
        typedef float f4 __attribute__((ext_vector_type(4)));
        const f4 nv = NT ? __builtin_nontemporal_load(reinterpret_cast<const f4 *>(src4) + i) : f4{};
        const float4 v = NT ? float4{nv.x, nv.y, nv.z, nv.w} : src4[i];
        const uint32_t e = i * 4;
        uint32_t rl = (uint32_t)((float)e * inv);  // e < 2^24: exact, then corrected
        if (rl * n_cols > e) rl--;
        if ((rl + 1) * n_cols <= e) rl++;
        uint32_t f = e - rl * n_cols;
        const float vals[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            s_x[f * kPredPitch + rl] = MIRROR ? mirror_value<MISSING_NAN>(vals[j], missing) : vals[j];
            if (++f == n_cols) {
                f = 0;
                rl++;
            }
        }
    }
    for (uint32_t e = n4 * 4 + lane; e < total; e += kPredLanes) {
        const uint32_t rl = e / n_cols;
        const float v = src[e];
        s_x[(e - rl * n_cols) * kPredPitch + rl] = MIRROR ? mirror_value<MISSING_NAN>(v, missing) : v;
    }
}

// One 8-byte node record in a single load (the records are 8-byte aligned).
template <typename Node>
__device__ __forceinline__ Node load_node(const Node *p, uint32_t i) {
    static_assert(sizeof(Node) == 8, "8-byte node records");
    typedef uint32_t u2 __attribute__((ext_vector_type(2)));
    const u2 v = reinterpret_cast<const u2 *>(p)[i];
    return Node{v.x, v.y};
}

// CH chains of the mirror walk, `depth` steps each (every chain then sits
// on its leaf): per step the value of the node's slot, its sign flipped by
// the node's m bit, compared with t, and the next node.
template <int CH>
__device__ __forceinline__ void mirror_walk(const MirrorNode *nodes, const float *xr, uint32_t (&g)[CH],
                                            MirrorNode (&nd)[CH], uint32_t depth) {
    for (uint32_t s = 0; s < depth; s++) {
        float v[CH];
#pragma unroll
        for (int k = 0; k < CH; k++) v[k] = xr[(nd[k].w & 0xffffu) * kPredPitch];
#pragma unroll
        for (int k = 0; k < CH; k++) {
            const float x = __uint_as_float(__float_as_uint(v[k]) ^ (nd[k].w & 0x80000000u));
            g[k] += ((nd[k].w >> 16) & 0x7fffu) + (x < __uint_as_float(nd[k].t) ? 1u : 0u);
        }
#pragma unroll
        for (int k = 0; k < CH; k++) nd[k] = load_node(nodes, g[k]);
    }
}

// A row's starting margin of output o: the caller's (BoostedModel's
// initial margins, a DMatrix's base_margin) or the base score.
__device__ __forceinline__ float start_margin(const PredictArgs &a, uint32_t r, uint32_t o) {
    return a.init ? a.init[(size_t)r * a.n_outputs + o] : a.base_score[o];
}

}  // namespace hbr

extern "C" __global__ __launch_bounds__(256) void hbr_predict(PredictArgs a) {
    const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= a.n) return;
    const float *row = a.x + (size_t)r * a.n_cols;
    float *out = a.out + (size_t)r * a.n_outputs;
    if (a.n_outputs == 1) {
        float acc = start_margin(a, r, 0);
        for (uint32_t t = 0; t < a.n_trees; t++) {
            const uint32_t leaf = walk(a, row, a.tree_root[t]);
            if (a.leaf_out) a.leaf_out[(size_t)r * a.n_trees + t] = a.node_orig[leaf];
            const float contrib = a.tree_weight[t] * __uint_as_float(a.node_value[leaf]);
            acc = acc + contrib;
        }
        out[0] = acc;
        return;
    }
    for (uint32_t c = 0; c < a.n_outputs; c++) out[c] = start_margin(a, r, c);
    for (uint32_t t = 0; t < a.n_trees; t++) {
        const uint32_t leaf = walk(a, row, a.tree_root[t]);
        if (a.leaf_out) a.leaf_out[(size_t)r * a.n_trees + t] = a.node_orig[leaf];
        const float contrib = a.tree_weight[t] * __uint_as_float(a.node_value[leaf]);
        float *o = out + a.tree_output[t];
        *o = *o + contrib;
    }
}

// Dynamic LDS: n_cols * kPredPitch floats. Grid-stride over 64-row blocks.
extern "C" __global__ __launch_bounds__(64) void hbr_predict_staged(PredictArgs a) {
    extern __shared__ float s_x[];
    const uint32_t lane = threadIdx.x;
    const uint32_t n_blocks = (a.n + kPredLanes - 1) / kPredLanes;
    for (uint32_t blk = blockIdx.x; blk < n_blocks; blk += gridDim.x) {
        const uint32_t r0 = blk * kPredLanes;
        const uint32_t rows = min(kPredLanes, a.n - r0);
        stage_rows(s_x, a.x + (size_t)r0 * a.n_cols, rows, a.n_cols, lane);
        __syncthreads();
        if (lane < rows) {
            const uint32_t r = r0 + lane;
            const float *xr = s_x + lane;
            float *out = a.out + (size_t)r * a.n_outputs;
            float acc = start_margin(a, r, 0);
            if (a.n_outputs != 1)
                for (uint32_t c = 0; c < a.n_outputs; c++) out[c] = start_margin(a, r, c);
            for (uint32_t t0 = 0; t0 < a.n_trees; t0 += kPredChains) {
                uint32_t nid[kPredChains];
                PredNode nd[kPredChains];
#pragma unroll
                for (int k = 0; k < kPredChains; k++) {
                    nid[k] = a.tree_root[min(t0 + (uint32_t)k, a.n_trees - 1)];
                    nd[k] = a.nodes[nid[k]];
                }
                // every chain moves one level per round until all sit at
                // leaves (a chain at its leaf re-reads it; no branches, so
                // the loads of all chains overlap)
                for (;;) {
                    float v[kPredChains];
#pragma unroll
                    for (int k = 0; k < kPredChains; k++) v[k] = xr[(nd[k].meta & 0xfffffu) * kPredPitch];
                    bool open = false;
#pragma unroll
                    for (int k = 0; k < kPredChains; k++) {
                        const bool miss = a.missing_is_nan ? __builtin_isnan(v[k]) : (v[k] == a.missing);
                        const bool left =
                            miss ? ((nd[k].meta >> 30) & 1u) != 0 : (v[k] < __uint_as_float(nd[k].value));
                        nid[k] = (nd[k].meta >> 31) ? nid[k] : nd[k].left + (left ? 0u : 1u);
                    }
#pragma unroll
                    for (int k = 0; k < kPredChains; k++) {
                        nd[k] = a.nodes[nid[k]];
                        open = open || !(nd[k].meta >> 31);
                    }
                    if (!open) break;
                }
#pragma unroll
                for (int k = 0; k < kPredChains; k++) {
                    const uint32_t t = t0 + (uint32_t)k;
                    if (t < a.n_trees) {
                        if (a.leaf_out) a.leaf_out[(size_t)r * a.n_trees + t] = nd[k].orig;
                        const float contrib = a.tree_weight[t] * __uint_as_float(nd[k].value);
                        if (a.n_outputs == 1) {
                            acc = acc + contrib;
                        } else {
                            float *o = out + a.tree_output[t];
                            *o = *o + contrib;
                        }
                    }
                }
            }
            if (a.n_outputs == 1) out[0] = acc;
        }
        __syncthreads();
    }
}

// Trees resident, rows streamed. The forest is cut into chunks of whole
// trees that fit the LDS node table; for each chunk in order, the
// workgroup copies the chunk's compact nodes, roots and weights into LDS,
// then every wave stages its 64-row blocks (feature-major, as above) and
// walks them through the chunk's trees. Each row's margin is carried from
// chunk to chunk in `out` (the same wave owns the same rows in every
// chunk), so the f32 adds keep the tree order. MISSING_NAN: the missing
// value is NaN (the comparison that tests it is specialised). Dynamic LDS:
// chunk_cap compact nodes, kChunkTrees roots and weights, then one
// n_cols * kPredPitch block per wave.
constexpr uint32_t kChunkTrees = 256;

template <bool MISSING_NAN>
__device__ __forceinline__ void predict_chunked(const PredictArgs &a) {
    extern __shared__ uint32_t lds[];
    CompactNode *s_nodes = reinterpret_cast<CompactNode *>(lds);
    uint32_t *s_root = lds + 2 * a.chunk_cap;
    float *s_weight = reinterpret_cast<float *>(s_root + kChunkTrees);
    const uint32_t wave = threadIdx.x / kWave, lane = lane_id();
    const uint32_t waves = blockDim.x / kWave;
    float *s_x = s_weight + kChunkTrees + wave * (a.n_cols * kPredPitch);
    const float *xr = s_x + lane;
    const uint32_t n_blocks = (a.n + kPredLanes - 1) / kPredLanes;
    for (uint32_t c = 0; c < a.n_chunks; c++) {
        const uint32_t nb = a.chunk_node[c], cnt = a.chunk_node[c + 1] - nb;
        const uint32_t t_lo = a.chunk_tree[c], t_hi = a.chunk_tree[c + 1];
        __syncthreads();  // every wave is done with the previous chunk
        for (uint32_t i = threadIdx.x; i < cnt; i += blockDim.x) s_nodes[i] = a.compact[nb + i];
        for (uint32_t i = threadIdx.x; i < t_hi - t_lo; i += blockDim.x) {
            s_root[i] = a.tree_root[t_lo + i] - nb;
            s_weight[i] = a.tree_weight[t_lo + i];
        }
        __syncthreads();
        for (uint32_t blk = blockIdx.x * waves + wave; blk < n_blocks; blk += gridDim.x * waves) {
            const uint32_t r0 = blk * kPredLanes;
            const uint32_t rows = min(kPredLanes, a.n - r0);
            const float *src = a.x + (size_t)r0 * a.n_cols;
            const uint32_t r = r0 + min(lane, rows - 1);
            float *out = a.out + (size_t)r * a.n_outputs;
            float acc = c == 0 ? start_margin(a, r, 0) : out[0];
            // the wave's previous walk has read its block: lanes finish in lockstep
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            stage_rows(s_x, src, rows, a.n_cols, lane);
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            if (c == 0 && lane < rows && a.n_outputs != 1)
                for (uint32_t o = 0; o < a.n_outputs; o++) out[o] = start_margin(a, r, o);
            if (lane >= rows) continue;
            for (uint32_t t0 = t_lo; t0 < t_hi; t0 += kPredChains) {
                uint32_t nid[kPredChains];
                CompactNode nd[kPredChains];
#pragma unroll
                for (int k = 0; k < kPredChains; k++) {
                    nid[k] = s_root[min(t0 + (uint32_t)k, t_hi - 1) - t_lo];
                    nd[k] = load_node(s_nodes, nid[k]);
                }
                // branch-free rounds: a chain at its leaf re-reads it, so
                // the LDS reads of all chains overlap
                for (;;) {
                    float v[kPredChains];
#pragma unroll
                    for (int k = 0; k < kPredChains; k++) v[k] = xr[(nd[k].meta & 0xffffu) * kPredPitch];
                    bool open = false;
#pragma unroll
                    for (int k = 0; k < kPredChains; k++) {
                        const uint32_t meta = nd[k].meta;
                        const uint32_t right = goes_right<MISSING_NAN>(v[k], meta, nd[k].value, a.missing);
                        const uint32_t next = nid[k] + ((meta >> 16) & 0x3fffu) + right;
                        nid[k] = (meta >> 31) ? nid[k] : next;
                    }
#pragma unroll
                    for (int k = 0; k < kPredChains; k++) {
                        nd[k] = load_node(s_nodes, nid[k]);
                        open = open || !(nd[k].meta >> 31);
                    }
                    if (!open) break;
                }
#pragma unroll
                for (int k = 0; k < kPredChains; k++) {
                    const uint32_t t = t0 + (uint32_t)k;
                    if (t < t_hi) {
                        if (a.leaf_out) a.leaf_out[(size_t)r * a.n_trees + t] = a.node_orig[nb + nid[k]];
                        const float contrib = s_weight[t - t_lo] * __uint_as_float(nd[k].value);
                        if (a.n_outputs == 1) {
                            acc = acc + contrib;
                        } else {
                            float *o = out + a.tree_output[t];
                            *o = *o + contrib;
                        }
                    }
                }
            }
            if (a.n_outputs == 1) out[0] = acc;
        }
    }
}

extern "C" __global__ __launch_bounds__(256) void hbr_predict_chunked_nan(PredictArgs a) { predict_chunked<true>(a); }
extern "C" __global__ __launch_bounds__(256) void hbr_predict_chunked(PredictArgs a) { predict_chunked<false>(a); }

// Rows resident, trees streamed through the caches. A workgroup is one wave;
// it stages a 64-row block in LDS once (feature-major, as above) and walks
// it through every tree of the forest, CH trees at a time, reading the
// compact node records from global memory (a wave's lanes walk the same
// trees, so a level's reads share a few cache lines and the forest stays in
// L2/MALL). The rows are read from HBM once, however large the forest.
template <bool MISSING_NAN, int CH, bool NT = false>
__device__ __forceinline__ void predict_resident(const PredictArgs &a) {
    extern __shared__ float s_rows[];
    const uint32_t lane = lane_id();
    const float *xr = s_rows + lane;
    const uint32_t n_blocks = (a.n + kPredLanes - 1) / kPredLanes;
    for (uint32_t blk = blockIdx.x; blk < n_blocks; blk += gridDim.x) {
        const uint32_t r0 = blk * kPredLanes;
        const uint32_t rows = min(kPredLanes, a.n - r0);
        // the previous block's walk has read its rows: lanes finish in lockstep
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        stage_rows<NT>(s_rows, a.x + (size_t)r0 * a.n_cols, rows, a.n_cols, lane);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (lane >= rows) continue;
        const uint32_t r = r0 + lane;
        float *out = a.out + (size_t)r * a.n_outputs;
        if (a.n_outputs != 1)
            for (uint32_t o = 0; o < a.n_outputs; o++) out[o] = start_margin(a, r, o);
        float acc = start_margin(a, r, 0);
        for (uint32_t t0 = 0; t0 < a.n_trees; t0 += CH) {
            uint32_t g[CH];
            CompactNode nd[CH];
#pragma unroll
            for (int k = 0; k < CH; k++) {
                g[k] = a.tree_root[min(t0 + (uint32_t)k, a.n_trees - 1)];
                nd[k] = load_node(a.compact, g[k]);
            }
            // branch-free rounds: a chain at its leaf re-reads it, so the
            // node loads of all chains are in flight together
            for (;;) {
                float v[CH];
#pragma unroll
                for (int k = 0; k < CH; k++) v[k] = xr[(nd[k].meta & 0xffffu) * kPredPitch];
#pragma unroll
                for (int k = 0; k < CH; k++) {
                    const uint32_t meta = nd[k].meta;
                    const uint32_t right = goes_right<MISSING_NAN>(v[k], meta, nd[k].value, a.missing);
                    const uint32_t next = g[k] + ((meta >> 16) & 0x3fffu) + right;
                    g[k] = (meta >> 31) ? g[k] : next;
                }
                bool open = false;
#pragma unroll
                for (int k = 0; k < CH; k++) {
                    nd[k] = load_node(a.compact, g[k]);
                    open = open || !(nd[k].meta >> 31);
                }
                if (!open) break;
            }
#pragma unroll
            for (int k = 0; k < CH; k++) {
                const uint32_t t = t0 + (uint32_t)k;
                if (t < a.n_trees) {
                    if (a.leaf_out) a.leaf_out[(size_t)r * a.n_trees + t] = a.node_orig[g[k]];
                    const float contrib = a.tree_weight[t] * __uint_as_float(nd[k].value);
                    if (a.n_outputs == 1) {
                        acc = acc + contrib;
                    } else {
                        float *o = out + a.tree_output[t];
                        *o = *o + contrib;
                    }
                }
            }
        }
        if (a.n_outputs == 1) out[0] = acc;
    }
}

// 16 trees in flight per lane (8 leave the node loads latency-bound, 32
// gain nothing more); rows staged with non-temporal loads, so that the
// streamed rows do not push the forest out of L2.
extern "C" __global__ __launch_bounds__(64) void hbr_predict_resident_nan(PredictArgs a) {
    predict_resident<true, 16, true>(a);
}
extern "C" __global__ __launch_bounds__(64) void hbr_predict_resident(PredictArgs a) {
    predict_resident<false, 16, true>(a);
}

// The mirror walk with rows resident in LDS and the nodes read through the
// caches: a workgroup is one wave; it stages a 64-row block once (slot 0
// NaN, feature f in slot f + 1) and walks it through every tree, CH trees
// in flight per lane, each group for the largest depth among its trees.
template <bool MISSING_NAN, int CH>
__device__ __forceinline__ void predict_mirror(const PredictArgs &a) {
    extern __shared__ float s_rows[];  // (n_cols + 1) * kPredPitch
    const uint32_t lane = lane_id();
    const float *xr = s_rows + lane;
    s_rows[lane] = __builtin_nanf("");
    const uint32_t n_blocks = (a.n + kPredLanes - 1) / kPredLanes;
    for (uint32_t blk = blockIdx.x; blk < n_blocks; blk += gridDim.x) {
        const uint32_t r0 = blk * kPredLanes;
        const uint32_t rows = min(kPredLanes, a.n - r0);
        // the previous block's walk has read its rows: lanes finish in lockstep
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        stage_rows<true, true, MISSING_NAN>(s_rows, a.x + (size_t)r0 * a.n_cols, rows, a.n_cols, lane, a.missing);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (lane >= rows) continue;
        const uint32_t r = r0 + lane;
        float *out = a.out + (size_t)r * a.n_outputs;
        if (a.n_outputs != 1)
            for (uint32_t o = 0; o < a.n_outputs; o++) out[o] = start_margin(a, r, o);
        float acc = start_margin(a, r, 0);
        for (uint32_t t0 = 0; t0 < a.n_trees; t0 += CH) {
            uint32_t g[CH];
            MirrorNode nd[CH];
            uint32_t depth = 0;
#pragma unroll
            for (int k = 0; k < CH; k++) {
                const uint32_t t = min(t0 + (uint32_t)k, a.n_trees - 1);
                g[k] = a.mirror_root[t];
                nd[k] = load_node(a.mirror, g[k]);
                depth = max(depth, (uint32_t)a.tree_depth[t]);
            }
            mirror_walk<CH>(a.mirror, xr, g, nd, depth);
#pragma unroll
            for (int k = 0; k < CH; k++) {
                const uint32_t t = t0 + (uint32_t)k;
                if (t < a.n_trees) {
                    if (a.leaf_out) a.leaf_out[(size_t)r * a.n_trees + t] = a.mirror_orig[g[k]];
                    const float contrib = a.tree_weight[t] * __uint_as_float(nd[k].t);
                    if (a.n_outputs == 1) {
                        acc = acc + contrib;
                    } else {
                        float *o = out + a.tree_output[t];
                        *o = *o + contrib;
                    }
                }
            }
        }
        if (a.n_outputs == 1) out[0] = acc;
    }
}

extern "C" __global__ __launch_bounds__(64) void hbr_predict_mirror_nan(PredictArgs a) { predict_mirror<true, 16>(a); }
extern "C" __global__ __launch_bounds__(64) void hbr_predict_mirror(PredictArgs a) { predict_mirror<false, 16>(a); }

// A load every lane makes from the same address, through the scalar data
// cache (s_load) instead of the texture path: the pointer is taken into the
// constant address space, whose uniform loads the compiler turns into scalar
// loads. Only for data no kernel writes while the walk runs.
template <typename T>
__device__ __forceinline__ T uniform_load(const T *p, size_t i) {
    typedef const __attribute__((address_space(4))) T constant_t;
    return ((constant_t *)p)[i];
}

// One test of the pair walk. A field w of a record's s word (the node's own,
// or a child's rotated into place) holds its slot at bits 8..14 and its m
// at bit 31: the lane's value of that slot is read from LDS at byte
// (w & 0x7f00) | 4 lane (slot * kPredPitch * 4 + 4 lane), its sign flipped
// when m, and compared with t. 1 when the row goes to the second child.
// The pair kernels declare no static LDS, so their dynamic block (the
// staged rows) starts at LDS byte 0 and the and/or above is the whole
// address.
__device__ __forceinline__ bool pair_go(uint32_t lane4, uint32_t w, uint32_t t) {
    typedef const __attribute__((address_space(3))) float lds_float;
    const float v = *(lds_float *)(size_t)((w & 0x7f00u) | lane4);
    const float x = __uint_as_float(__float_as_uint(v) ^ (w & 0x80000000u));
    return x < __uint_as_float(t);
}

// 2 p + b in one add with carry-in (the compiler otherwise spends a select,
// a shift and an or on it).
__device__ __forceinline__ uint32_t double_add(uint32_t p, bool b) {
    uint32_t r;
    const uint64_t m = __builtin_amdgcn_ballot_w64(b);
    asm("v_addc_co_u32_e64 %0, vcc, %1, %1, %2" : "=v"(r) : "v"(p), "s"(m) : "vcc");
    return r;
}

// One record (t_node, t_first, t_second, s): the node's test, then that of
// the child it chose; the position 0..3 of the grandchild reached. s holds
// the node's slot at bits 8..14 and m at bit 31, the first child's slot at
// bits 16..22 and m at bit 7, the second's slot at bits 0..6 and m at bit
// 23: rotating s right by 8 (first child) or 24 (second) brings the child's
// slot and m to where the node's sit.
// pos becomes 4 pos + that position (each doubling plus a test is one add
// with the test's carry).
__device__ __forceinline__ uint32_t pair_step(uint32_t lane4, uint4 rec, uint32_t pos) {
    const bool go = pair_go(lane4, rec.w, rec.x);
    const uint32_t c = __builtin_amdgcn_alignbit(rec.w, rec.w, go ? 24u : 8u);
    const bool go_c = pair_go(lane4, c, go ? rec.z : rec.y);
    return double_add(double_add(pos, go), go_c);
}

// Complete trees walked two levels per record (PredictArgs::pairs), LEVELS
// records deep: rows resident in LDS as in hbr_predict_mirror (one 64-row
// block per one-wave workgroup, slot 0 NaN), CH trees in flight per lane.
// The root record and the tree's weight are the same for every lane (scalar
// loads); a deeper record is read at the tree's level base, a uniform
// address, plus the lane's 32-bit byte offset, and so is the leaf's value:
// a tree costs the texture path one load per level below the root's two and
// one for the leaf. The levels are unrolled so that a chain's next load can
// issue as soon as its own step is done.
// ONE: one output and no leaf indices (the margins alone, added in
// registers).
template <bool MISSING_NAN, int CH, int LEVELS, bool ONE>
__device__ __forceinline__ void predict_pairs(const PredictArgs &a) {
    extern __shared__ float s_rows[];  // (n_cols + 1) * kPredPitch
    const uint32_t lane = lane_id();
    const uint32_t lane4 = lane * 4u;
    s_rows[lane] = __builtin_nanf("");
    constexpr uint32_t per_tree = ((1u << (2 * LEVELS)) - 1u) / 3u;  // records
    constexpr uint32_t leaves = 1u << (2 * LEVELS);
    const uint32_t n_blocks = (a.n + kPredLanes - 1) / kPredLanes;
    for (uint32_t blk = blockIdx.x; blk < n_blocks; blk += gridDim.x) {
        const uint32_t r0 = blk * kPredLanes;
        const uint32_t rows = min(kPredLanes, a.n - r0);
        // the previous block's walk has read its rows: lanes finish in lockstep
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        stage_rows<true, true, MISSING_NAN>(s_rows, a.x + (size_t)r0 * a.n_cols, rows, a.n_cols, lane, a.missing);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (lane >= rows) continue;
        const uint32_t r = r0 + lane;
        float *out = a.out + (size_t)r * a.n_outputs;
        if (a.n_outputs != 1)
            for (uint32_t o = 0; o < a.n_outputs; o++) out[o] = start_margin(a, r, o);
        float acc = start_margin(a, r, 0);
        for (uint32_t t0 = 0; t0 < a.n_trees; t0 += CH) {
            // the group's trees from one base: tree t0 + k at k' = min(k,
            // last) trees past it (the last group repeats its last tree)
            const uint32_t last = a.n_trees - 1 - t0;
            const char *group = reinterpret_cast<const char *>(a.pairs + (size_t)t0 * per_tree);
            const char *group_vals = reinterpret_cast<const char *>(a.pair_values + (size_t)t0 * leaves);
            uint32_t pos[CH];
#pragma unroll
            for (int k = 0; k < CH; k++) {
                const PairRecord rec = uniform_load(a.pairs, (size_t)(t0 + min((uint32_t)k, last)) * per_tree);
                pos[k] = pair_step(lane4, make_uint4(rec.t_node, rec.t_first, rec.t_second, rec.s), 0u);
            }
#pragma unroll
            for (int l = 1; l < LEVELS; l++) {
                const uint32_t base = ((1u << (2 * l)) - 1u) / 3u;  // first record of the level
                uint4 rec[CH];
#pragma unroll
                for (int k = 0; k < CH; k++) {
                    const uint32_t at = (min((uint32_t)k, last) * per_tree + base) * 16u + (pos[k] << 4);
                    rec[k] = *reinterpret_cast<const uint4 *>(group + at);
                }
#pragma unroll
                for (int k = 0; k < CH; k++) pos[k] = pair_step(lane4, rec[k], pos[k]);
            }
            uint32_t leaf[CH];
#pragma unroll
            for (int k = 0; k < CH; k++)
                leaf[k] = *reinterpret_cast<const uint32_t *>(group_vals + min((uint32_t)k, last) * leaves * 4u +
                                                              (pos[k] << 2));
#pragma unroll
            for (int k = 0; k < CH; k++) {
                const uint32_t t = t0 + (uint32_t)k;
                if (t < a.n_trees) {
                    const float contrib = uniform_load(a.tree_weight, t) * __uint_as_float(leaf[k]);
                    if (ONE) {
                        acc = acc + contrib;
                        continue;
                    }
                    if (a.leaf_out) a.leaf_out[(size_t)r * a.n_trees + t] = a.pair_orig[(size_t)t * leaves + pos[k]];
                    if (a.n_outputs == 1) {
                        acc = acc + contrib;
                    } else {
                        float *o = out + a.tree_output[t];
                        *o = *o + contrib;
                    }
                }
            }
        }
        if (a.n_outputs == 1) out[0] = acc;
    }
}

template <bool MISSING_NAN, bool ONE>
__device__ __forceinline__ void predict_pairs_levels(const PredictArgs &a) {
    switch (a.pair_levels) {
    case 1: predict_pairs<MISSING_NAN, 16, 1, ONE>(a); break;
    case 2: predict_pairs<MISSING_NAN, 16, 2, ONE>(a); break;
    case 3: predict_pairs<MISSING_NAN, 16, 3, ONE>(a); break;
    case 4: predict_pairs<MISSING_NAN, 16, 4, ONE>(a); break;
    case 5: predict_pairs<MISSING_NAN, 16, 5, ONE>(a); break;
    case 6: predict_pairs<MISSING_NAN, 16, 6, ONE>(a); break;
    default: break;  // the host builds pair forests of depth 12 at most
    }
}

template <bool MISSING_NAN>
__device__ __forceinline__ void predict_pairs_dispatch(const PredictArgs &a) {
    if (a.n_outputs == 1 && !a.leaf_out)
        predict_pairs_levels<MISSING_NAN, true>(a);
    else
        predict_pairs_levels<MISSING_NAN, false>(a);
}

// The occupancy is the LDS row blocks' (a few waves per SIMD): the walk may
// keep its sixteen chains' records in registers.
extern "C" __global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(1, 2))) void hbr_predict_pairs_nan(
    PredictArgs a) {
    predict_pairs_dispatch<true>(a);
}
extern "C" __global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(1, 2))) void hbr_predict_pairs(
    PredictArgs a) {
    predict_pairs_dispatch<false>(a);
}

// ---- evaluation sets --------------------------------------------------------
//
// A finished tree added into an evaluation set's margins as the host's
// training loop adds it (training/margins.rs:148-152 via add_tree_margins,
// :186-196): margin[output] += leaf(tree, row), one f32 add, the row routed
// by raw value. A device-grown tree is read from its records where its
// growth wrote them, so the walk queues behind the growth on the stream;
// a split's threshold is the cut value of its bin boundary, as the tree's
// host copy records it (or, for a tree the caller passes, its own
// thresholds; a categorical split sends a present value left iff its
// category is among the node's, as the model's prediction does). Thread per
// row; the tree's nodes sit in LDS (eval_node's records) when they fit.

namespace {

// A node of the evaluation walk: (threshold bits, feature | categorical <<
// 30 | default_left << 31, left child or ~0 for a leaf, value bits).
__device__ __forceinline__ uint4 eval_node(const EvalWalkArgs &a, uint32_t i) {
    const GrowTreeNode t = a.tree[i];
    uint4 w;
    if (t.left < 0) {
        w.x = 0u;
        w.y = 0u;
        w.z = 0xffffffffu;
    } else {
        const float cond = a.cond ? a.cond[i]
                           : t.bin >= 0 && (uint32_t)t.bin < a.total_bins ? a.cut_values[t.bin]
                                                                          : -__FLT_MAX__;
        const bool cat = a.cat_span && (a.cat_span[2 * i + 1] >> 31);
        w.x = __float_as_uint(cond);
        w.y = min(t.feature, a.n_cols - 1u) | (cat ? 1u << 30 : 0u) | (t.default_left ? 1u << 31 : 0u);
        w.z = (uint32_t)t.left;
    }
    w.w = __float_as_uint(t.value);
    return w;
}

// The step of a present value at node `id` (record nd): below the
// threshold, or, for a categorical split, its category among the node's.
__device__ __forceinline__ bool eval_present_left(const EvalWalkArgs &a, uint32_t id, const uint4 &nd, float v) {
    if (!(nd.y & (1u << 30))) return v < __uint_as_float(nd.x);
    const uint32_t c = category_of(v);
    const uint32_t end = a.cat_span[2 * id + 1] & 0x7fffffffu;
    bool hit = false;
    for (uint32_t i = a.cat_span[2 * id]; i < end; i++) hit |= a.categories[i] == c;
    return hit;
}

template <bool kLds>
__device__ __forceinline__ void eval_walk(const EvalWalkArgs &a, const uint4 *s_node, uint32_t n_nodes) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t r = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; r < a.n; r += stride) {
        const float *row = a.x + r * a.n_cols;
        uint4 nd = kLds ? s_node[0] : eval_node(a, 0);
        uint32_t id = 0;
        bool leaf = nd.z == 0xffffffffu;
        for (uint32_t step = 0; step < n_nodes && !leaf; step++) {
            const float v = row[nd.y & 0x3fffffffu];
            const bool absent = a.missing_is_nan ? __builtin_isnan(v) : v == a.missing_value;
            const bool go_left = absent ? (nd.y >> 31) != 0u : eval_present_left(a, id, nd, v);
            const uint32_t nid = nd.z + (go_left ? 0u : 1u);
            if (nid >= n_nodes) break;  // a malformed record: the row gets nothing
            nd = kLds ? s_node[nid] : eval_node(a, nid);
            id = nid;
            leaf = nd.z == 0xffffffffu;
        }
        if (leaf) {
            float *m = a.margins + r * a.m_stride + a.output;
            *m = *m + __uint_as_float(nd.w);
        }
    }
}

}  // namespace

// Rows of at most kEvalStagedCols features: each wave stages a 64-row block
// in LDS feature-major with coalesced non-temporal loads (stage_rows), then
// each lane walks its row from LDS. Dynamic LDS: 4 waves x n_cols x
// kPredPitch floats. Every wave of a workgroup runs the same number of
// passes (a wave past the last block stages and walks nothing), so the
// barriers are uniform.
extern "C" __global__ __launch_bounds__(256) void hbr_eval_walk_staged(EvalWalkArgs a) {
    __shared__ uint4 s_node[kEvalLdsNodes];
    extern __shared__ float s_rows[];
    if (a.poison && *a.poison != 0u) return;  // uniform: the tree was not kept
    const uint32_t n_nodes = a.counts ? a.counts->n_nodes : a.n_nodes;
    if (n_nodes == 0 || a.n_cols == 0 || a.n_cols > kEvalStagedCols) return;
    const bool lds_nodes = n_nodes <= kEvalLdsNodes;
    if (lds_nodes)
        for (uint32_t i = threadIdx.x; i < n_nodes; i += blockDim.x) s_node[i] = eval_node(a, i);
    const uint32_t wave = threadIdx.x / kPredLanes, lane = threadIdx.x % kPredLanes;
    const uint32_t waves = blockDim.x / kPredLanes;
    float *s_x = s_rows + (size_t)wave * a.n_cols * kPredPitch;
    const uint64_t n_blocks = (a.n + kPredLanes - 1) / kPredLanes;
    const uint64_t step = (uint64_t)gridDim.x * waves;
    for (uint64_t base = (uint64_t)blockIdx.x * waves; base < n_blocks; base += step) {
        const uint64_t blk = base + wave;
        const uint64_t r0 = blk * kPredLanes;
        const uint32_t rows = blk >= n_blocks ? 0u : a.n - r0 < kPredLanes ? (uint32_t)(a.n - r0) : kPredLanes;
        __syncthreads();  // the previous pass's reads of s_x are done (and the node table is written)
        if (rows) stage_rows<true>(s_x, a.x + r0 * a.n_cols, rows, a.n_cols, lane);
        __syncthreads();
        if (lane >= rows) continue;
        const float *row = s_x + lane;
        uint4 nd = lds_nodes ? s_node[0] : eval_node(a, 0);
        uint32_t id = 0;
        bool leaf = nd.z == 0xffffffffu;
        for (uint32_t st = 0; st < n_nodes && !leaf; st++) {
            const float v = row[(nd.y & 0x3fffffffu) * kPredPitch];
            const bool absent = a.missing_is_nan ? __builtin_isnan(v) : v == a.missing_value;
            const bool go_left = absent ? (nd.y >> 31) != 0u : eval_present_left(a, id, nd, v);
            const uint32_t nid = nd.z + (go_left ? 0u : 1u);
            if (nid >= n_nodes) break;  // a malformed record: the row gets nothing
            nd = lds_nodes ? s_node[nid] : eval_node(a, nid);
            id = nid;
            leaf = nd.z == 0xffffffffu;
        }
        if (leaf) {
            float *m = a.margins + (r0 + lane) * a.m_stride + a.output;
            *m = *m + __uint_as_float(nd.w);
        }
    }
}

extern "C" __global__ __launch_bounds__(256) void hbr_eval_walk(EvalWalkArgs a) {
    __shared__ uint4 s_node[kEvalLdsNodes];
    if (a.poison && *a.poison != 0u) return;  // uniform: the tree was not kept
    const uint32_t n_nodes = a.counts ? a.counts->n_nodes : a.n_nodes;
    if (n_nodes == 0 || a.n_cols == 0) return;
    if (n_nodes <= kEvalLdsNodes) {
        for (uint32_t i = threadIdx.x; i < n_nodes; i += blockDim.x) s_node[i] = eval_node(a, i);
        __syncthreads();
        eval_walk<true>(a, s_node, n_nodes);
    } else {
        eval_walk<false>(a, nullptr, n_nodes);
    }
}
