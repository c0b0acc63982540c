#include "forest.h"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <string>
#include <tuple>
#include <utility>

namespace hbr {

// Each tree is re-laid out breadth-first so every internal node's children
// sit side by side (right = left + 1), the node records its original id for
// leaf queries, and the walk can never loop: every node is reached exactly
// once from the root, or the upload is refused.
Forest::Forest(int ordinal, const hbr_forest_desc &fd) : dev_(device(ordinal)) {
    n_trees_ = fd.n_trees;
    n_outputs_ = fd.n_outputs ? fd.n_outputs : 1;
    std::vector<uint32_t> value, meta, left, root, output, cat_end;
    std::vector<int32_t> orig;
    std::vector<float> weight(n_trees_), base(n_outputs_);
    for (uint32_t c = 0; c < n_outputs_; c++) base[c] = fd.base_score ? fd.base_score[c] : 0.0f;
    for (uint64_t t = 0; t < n_trees_; t++) {
        const uint64_t lo = fd.tree_offset[t], hi = fd.tree_offset[t + 1];
        const uint64_t count = hi - lo;
        if (count == 0) fail(kInvalid, "forest: a tree without nodes");
        weight[t] = fd.tree_weight ? fd.tree_weight[t] : 1.0f;
        const uint32_t out = fd.tree_output ? fd.tree_output[t] : 0;
        if (out >= n_outputs_) fail(kInvalid, "forest: tree output beyond n_outputs");
        output.push_back(out);
        const uint32_t base_id = (uint32_t)value.size();
        root.push_back(base_id);
        std::vector<int32_t> queue{0};
        std::vector<uint8_t> seen(count, 0);
        seen[0] = 1;
        // new id of queue[i] is base_id + i
        for (size_t i = 0; i < queue.size(); i++) {
            const int32_t id = queue[i];
            const uint64_t at = lo + (uint64_t)id;
            orig.push_back(id);
            const int32_t l = fd.left[at], r = fd.right[at];
            if (l == -1) {
                uint32_t bits;
                std::memcpy(&bits, &fd.leaf_value[at], 4);
                value.push_back(bits);
                meta.push_back(1u << 31);
                left.push_back(0);
                cat_end.push_back(0);
                continue;
            }
            if (l < 0 || r < 0 || (uint64_t)l >= count || (uint64_t)r >= count || seen[l] || seen[r])
                fail(kInvalid, "forest: malformed tree " + std::to_string(t));
            if (fd.split_feature[at] >= (1u << 20)) fail(kInvalid, "forest: split feature beyond 2^20");
            seen[l] = seen[r] = 1;
            uint32_t bits;
            std::memcpy(&bits, &fd.split_cond[at], 4);
            uint32_t m = fd.split_feature[at] | ((fd.default_left[at] ? 1u : 0u) << 30);
            uint32_t end = 0;
            if (fd.is_categorical && fd.is_categorical[at]) {
                // the value slot holds the start of the node's category range
                if (!fd.cat_begin || !fd.cat_end || !fd.categories || fd.cat_begin[at] > fd.cat_end[at] ||
                    fd.cat_end[at] > fd.n_categories)
                    fail(kInvalid, "forest: a categorical split's categories are out of range in tree " +
                                       std::to_string(t));
                bits = fd.cat_begin[at];
                end = fd.cat_end[at];
                m |= kPredCategorical;
                has_categorical_ = true;
            }
            value.push_back(bits);
            meta.push_back(m);
            cat_end.push_back(end);
            left.push_back(base_id + (uint32_t)queue.size());
            queue.push_back(l);
            queue.push_back(r);
            max_feature_ = std::max(max_feature_, fd.split_feature[at]);
        }
    }
    hipStream_t s = dev_.stream();
    auto up = [&](auto &buf, const auto &v) {
        buf.resize(v.size() ? v.size() : 1);
        buf.upload(v.data(), v.size(), s);
    };
    up(value_, value);
    up(meta_, meta);
    up(left_, left);
    up(root_, root);
    up(output_, output);
    up(orig_, orig);
    if (has_categorical_) {
        up(cat_end_, cat_end);
        std::vector<uint32_t> pool(fd.categories, fd.categories + fd.n_categories);
        up(categories_, pool);
    }
    std::vector<PredNode> nodes(value.size());
    for (size_t i = 0; i < value.size(); i++) nodes[i] = PredNode{value[i], meta[i], left[i], orig[i]};
    up(nodes_, nodes);
    // compact records: feature < 2^16, left child within 2^14 - 1 nodes
    compact_ok_ = !has_categorical_;  // the compact walks compare thresholds only
    std::vector<CompactNode> compact(value.size());
    for (size_t i = 0; i < value.size(); i++) {
        if (meta[i] >> 31) {
            compact[i] = CompactNode{value[i], 1u << 31};
            continue;
        }
        const uint32_t f = meta[i] & 0xfffffu, rel = left[i] - (uint32_t)i;
        if (f >= (1u << 16) || rel >= (1u << 14)) compact_ok_ = false;
        compact[i] = CompactNode{value[i], (f & 0xffffu) | ((rel & 0x3fffu) << 16) | (meta[i] & (1u << 30))};
    }
    // one spare node past the end: the LDS walk copies 16-byte node pairs
    compact.push_back(CompactNode{0u, 1u << 31});
    if (compact_ok_) up(compact_, compact);
    tree_nodes_.resize(n_trees_);
    for (uint64_t t = 0; t < n_trees_; t++) {
        const uint32_t end = t + 1 < n_trees_ ? root[t + 1] : (uint32_t)value.size();
        tree_nodes_[t] = end - root[t];
        largest_tree_ = std::max(largest_tree_, tree_nodes_[t]);
    }
    up(weight_, weight);
    up(base_, base);
    build_mirror(fd);
    build_pairs(fd);
    dev_.sync();
}

// Largest finite float below c (c finite): v > next_below(c) is v >= c.
static float next_below(float c) {
    uint32_t b;
    std::memcpy(&b, &c, 4);
    if (c > 0.0f) b -= 1;
    else if (c == 0.0f) b = 0x80000001u;  // -(the smallest subnormal)
    else b += 1;
    float r;
    std::memcpy(&r, &b, 4);
    return r;
}

// The pair layout (PredictArgs::pairs): every tree embedded in the
// complete tree of the forest's largest depth rounded up to even, a split's
// first child being the one its missing values take.
void Forest::build_pairs(const hbr_forest_desc &fd) {
    if (has_categorical_ || n_trees_ == 0 || max_feature_ >= 126) return;
    uint32_t depth = 0;
    // depths, and the checks the walk needs
    std::vector<uint32_t> tree_depth(n_trees_, 0);
    for (uint64_t t = 0; t < n_trees_; t++) {
        const uint64_t lo = fd.tree_offset[t];
        std::vector<std::pair<int32_t, uint32_t>> stack{{0, 0}};
        while (!stack.empty()) {
            const auto [id, lv] = stack.back();
            stack.pop_back();
            const uint64_t at = lo + (uint64_t)id;
            tree_depth[t] = std::max(tree_depth[t], lv);
            if (fd.left[at] == -1) continue;
            if (!std::isfinite(fd.split_cond[at]) || lv >= 12) return;
            stack.push_back({fd.left[at], lv + 1});
            stack.push_back({fd.right[at], lv + 1});
        }
        depth = std::max(depth, tree_depth[t]);
    }
    // at least one record per tree: the walk reads every root record
    depth = std::max(depth + (depth & 1u), 2u);
    const uint32_t levels = depth / 2;
    const uint64_t per_tree = ((1ull << depth) - 1) / 3, leaves = 1ull << depth;
    // the complete trees may not outgrow the trees too far
    const uint64_t bytes = n_trees_ * (per_tree * sizeof(PairRecord) + leaves * 8);
    uint64_t real = 0;
    for (uint64_t t = 0; t < n_trees_; t++) real += tree_nodes_[t];
    if (bytes > (1ull << 30) || bytes > 64 * real * sizeof(MirrorNode)) return;
    std::vector<PairRecord> recs(n_trees_ * per_tree);
    std::vector<uint32_t> values(n_trees_ * leaves);
    std::vector<int32_t> orig(n_trees_ * leaves);
    std::vector<uint32_t> t_at, s_at;  // per complete position of levels < depth
    for (uint64_t t = 0; t < n_trees_; t++) {
        const uint64_t lo = fd.tree_offset[t];
        t_at.assign((1ull << depth) - 1, 0u);
        s_at.assign((1ull << depth) - 1, 0u);  // slot 0, m 0: the first child
        // (node, level, position in its level)
        std::vector<std::tuple<int32_t, uint32_t, uint64_t>> stack{{0, 0u, 0ull}};
        while (!stack.empty()) {
            const auto [id, lv, i] = stack.back();
            stack.pop_back();
            const uint64_t at = lo + (uint64_t)id;
            if (fd.left[at] == -1) {
                uint32_t bits;
                std::memcpy(&bits, &fd.leaf_value[at], 4);
                const uint64_t span = 1ull << (depth - lv);
                for (uint64_t j = i * span; j < (i + 1) * span; j++) {
                    values[t * leaves + j] = bits;
                    orig[t * leaves + j] = id;
                }
                continue;
            }
            const bool dl = fd.default_left[at] != 0;
            const float cond = fd.split_cond[at];
            const float tc = dl ? -next_below(cond) : cond;
            const uint64_t p = ((1ull << lv) - 1) + i;
            std::memcpy(&t_at[p], &tc, 4);
            s_at[p] = (dl ? 0x80u : 0u) | (fd.split_feature[at] + 1u);
            stack.push_back({dl ? fd.left[at] : fd.right[at], lv + 1, 2 * i});
            stack.push_back({dl ? fd.right[at] : fd.left[at], lv + 1, 2 * i + 1});
        }
        // s: the node's slot at bits 8..14 and m at 31, the first child's at
        // 16..22 and 7, the second's at 0..6 and 23 (PredictArgs::pairs)
        auto slot = [](uint32_t f) { return f & 0x7fu; };
        auto m = [](uint32_t f) { return f >> 7; };
        uint64_t r = t * per_tree;
        for (uint32_t l = 0; l < levels; l++) {
            const uint32_t lv = 2 * l;
            for (uint64_t i = 0; i < (1ull << lv); i++) {
                const uint64_t p = ((1ull << lv) - 1) + i;
                const uint64_t c = ((1ull << (lv + 1)) - 1) + 2 * i;
                const uint32_t sw = (slot(s_at[p]) << 8) | (m(s_at[p]) << 31) | (slot(s_at[c]) << 16) |
                                    (m(s_at[c]) << 7) | slot(s_at[c + 1]) | (m(s_at[c + 1]) << 23);
                recs[r++] = PairRecord{t_at[p], t_at[c], t_at[c + 1], sw};
            }
        }
    }
    hipStream_t s = dev_.stream();
    pairs_.resize(recs.size() ? recs.size() : 1);
    if (!recs.empty()) pairs_.upload(recs.data(), recs.size(), s);
    pair_values_.resize(values.size());
    pair_values_.upload(values.data(), values.size(), s);
    pair_orig_.resize(orig.size());
    pair_orig_.upload(orig.data(), orig.size(), s);
    pair_levels_ = levels;
    pairs_ok_ = true;
}

// The mirror arena (PredictArgs::mirror): every tree breadth-first with a
// missing value's child first; the trees were checked by the constructor.
void Forest::build_mirror(const hbr_forest_desc &fd) {
    if (has_categorical_ || n_trees_ == 0) return;
    std::vector<MirrorNode> nodes;
    std::vector<uint32_t> roots;
    std::vector<int32_t> orig;
    std::vector<uint8_t> depth;
    for (uint64_t t = 0; t < n_trees_; t++) {
        const uint64_t lo = fd.tree_offset[t];
        const uint32_t base = (uint32_t)nodes.size();
        roots.push_back(base);
        std::vector<int32_t> queue{0};
        std::vector<uint32_t> level{0};
        uint32_t deepest = 0;
        for (size_t i = 0; i < queue.size(); i++) {
            const uint64_t at = lo + (uint64_t)queue[i];
            orig.push_back(queue[i]);
            deepest = std::max(deepest, level[i]);
            uint32_t bits;
            if (fd.left[at] == -1) {
                std::memcpy(&bits, &fd.leaf_value[at], 4);
                nodes.push_back(MirrorNode{bits, 0u});
                continue;
            }
            const float cond = fd.split_cond[at];
            const uint32_t rel = (uint32_t)(queue.size() - i);
            if (!std::isfinite(cond) || fd.split_feature[at] >= 0xffffu || rel > 0x7fffu) return;
            const bool dl = fd.default_left[at] != 0;
            const float t_cond = dl ? -next_below(cond) : cond;
            std::memcpy(&bits, &t_cond, 4);
            nodes.push_back(MirrorNode{bits, (dl ? 1u << 31 : 0u) | (rel << 16) | (fd.split_feature[at] + 1u)});
            queue.push_back(dl ? fd.left[at] : fd.right[at]);
            queue.push_back(dl ? fd.right[at] : fd.left[at]);
            level.push_back(level[i] + 1);
            level.push_back(level[i] + 1);
        }
        if (deepest > 255) return;
        depth.push_back((uint8_t)deepest);
    }
    nodes.push_back(MirrorNode{0u, 0u});  // a spare node: the LDS walk copies 16-byte pairs
    hipStream_t s = dev_.stream();
    mirror_.resize(nodes.size());
    mirror_.upload(nodes.data(), nodes.size(), s);
    mirror_root_.resize(roots.size());
    mirror_root_.upload(roots.data(), roots.size(), s);
    mirror_orig_.resize(orig.size());
    mirror_orig_.upload(orig.data(), orig.size(), s);
    tree_depth_.resize(depth.size());
    tree_depth_.upload(depth.data(), depth.size(), s);
    mirror_ok_ = true;
}

void Forest::predict_device(const float *x, uint64_t n, uint64_t n_cols, float missing, float *out,
                            int32_t *leaf_out, const float *init) {
    if (n == 0) return;
    if (n_trees_ && n_cols <= max_feature_) fail(kInvalid, "predict: rows have fewer columns than the forest reads");
    if (n >= (uint64_t)UINT32_MAX) fail(kRefused, "predict: more than 2^32 - 1 rows per call");
    PredictArgs a{};
    a.nodes = nodes_.get();
    a.node_value = value_.get();
    a.node_meta = meta_.get();
    a.node_left = left_.get();
    a.node_orig = orig_.get();
    a.tree_root = root_.get();
    a.tree_weight = weight_.get();
    a.tree_output = output_.get();
    a.base_score = base_.get();
    a.init = init;
    a.x = x;
    a.out = out;
    a.leaf_out = leaf_out;
    a.n = (uint32_t)n;
    a.n_cols = (uint32_t)n_cols;
    a.n_trees = (uint32_t)n_trees_;
    a.n_outputs = n_outputs_;
    a.missing = missing;
    a.missing_is_nan = missing != missing ? 1u : 0u;
    if (has_categorical_) {  // the category sets are read by hbr_predict's walk
        a.categories = categories_.get();
        a.node_cat_end = cat_end_.get();
        dev_.launch("hbr_predict", dim3((uint32_t)((n + 255) / 256)), dim3(256), a);
        return;
    }
    const uint64_t row_block = n_cols * (uint64_t)kPredPitch * sizeof(float);
    const uint64_t lds_total = 160ull * 1024;
    // HBROCM_PRED_KERNEL selects a walk (pairs, mirror, resident, chunked,
    // staged, or any other value for the generic walk); by default the first
    // of pairs, mirror, resident, chunked and staged that the forest and the
    // rows allow. Each keeps a 64-row block in LDS per one-wave
    // workgroup (rows read from HBM once, however large the forest) and
    // reads the trees through the caches.
    const char *kind = std::getenv("HBROCM_PRED_KERNEL");
    auto allowed = [&](const char *walk) { return !kind || std::strcmp(kind, walk) == 0; };
    const bool nan = missing != missing;
    const uint64_t mirror_block = (n_cols + 1) * (uint64_t)kPredPitch * sizeof(float);
    const uint64_t blocks = (n + 63) / 64;
    // complete trees, two levels per record
    if (n_trees_ && pairs_ok_ && allowed("pairs") && mirror_block <= lds_total / 4) {
        a.pairs = pairs_.get();
        a.pair_values = pair_values_.get();
        a.pair_orig = pair_orig_.get();
        a.pair_levels = pair_levels_;
        const uint64_t grid = std::min<uint64_t>(blocks, (uint64_t)dev_.cu_count() * (lds_total / mirror_block));
        dev_.launch(nan ? "hbr_predict_pairs_nan" : "hbr_predict_pairs", dim3((uint32_t)grid), dim3(64), a,
                    (uint32_t)mirror_block);
        return;
    }
    // the mirror arena, one level per step
    if (n_trees_ && mirror_ok_ && allowed("mirror") && mirror_block <= lds_total / 4) {
        a.mirror = mirror_.get();
        a.mirror_root = mirror_root_.get();
        a.mirror_orig = mirror_orig_.get();
        a.tree_depth = tree_depth_.get();
        const uint64_t grid = std::min<uint64_t>(blocks, (uint64_t)dev_.cu_count() * (lds_total / mirror_block));
        dev_.launch(nan ? "hbr_predict_mirror_nan" : "hbr_predict_mirror", dim3((uint32_t)grid), dim3(64), a,
                    (uint32_t)mirror_block);
        return;
    }
    // compact records, one level per step (any threshold)
    if (n_trees_ && compact_ok_ && allowed("resident") && row_block <= lds_total / 4) {
        a.compact = compact_.get();
        const uint64_t grid = std::min<uint64_t>(blocks, (uint64_t)dev_.cu_count() * (lds_total / row_block));
        dev_.launch(missing != missing ? "hbr_predict_resident_nan" : "hbr_predict_resident", dim3((uint32_t)grid),
                    dim3(64), a, (uint32_t)row_block);
        return;
    }
    // trees resident in LDS, rows streamed (rows too wide for the walks
    // above): row blocks of `waves` waves plus a node table holding at least
    // the largest tree
    const uint64_t tree_tables = 2ull * 256 * sizeof(uint32_t);  // roots and weights of a chunk
    uint32_t waves = 4;
    if (const char *v = std::getenv("HBROCM_PRED_WAVES")) waves = (uint32_t)std::max(1L, std::min(4L, std::strtol(v, nullptr, 10)));
    while (waves > 1 && waves * row_block > lds_total / 2) waves--;
    if (n_trees_ && compact_ok_ && allowed("chunked") &&
        waves * row_block + tree_tables + 8ull * largest_tree_ <= lds_total) {
        const uint32_t cap = (uint32_t)((lds_total - waves * row_block - tree_tables) / 8);
        plan_chunks(cap);
        a.compact = compact_.get();
        a.chunk_tree = chunk_tree_.get();
        a.chunk_node = chunk_node_.get();
        a.n_chunks = n_chunks_;
        a.chunk_cap = cap;
        const uint64_t blocks = (n + 63) / 64;
        const uint64_t grid = std::min<uint64_t>((blocks + waves - 1) / waves, (uint64_t)dev_.cu_count());
        const char *k = missing != missing ? "hbr_predict_chunked_nan" : "hbr_predict_chunked";
        dev_.launch(k, dim3((uint32_t)grid), dim3(64 * waves), a,
                    (uint32_t)(8ull * cap + tree_tables + waves * row_block));
        return;
    }
    // rows staged in LDS when 64 of them fit in a quarter of a CU's LDS
    const uint64_t lds = n_cols * (uint64_t)kPredPitch * sizeof(float);
    if (n_trees_ && allowed("staged") && lds <= 40ull * 1024) {
        const uint64_t blocks = (n + 63) / 64;
        const uint64_t grid = std::min<uint64_t>(blocks, (uint64_t)dev_.cu_count() * 64);
        dev_.launch("hbr_predict_staged", dim3((uint32_t)grid), dim3(64), a, (uint32_t)lds);
        return;
    }
    dev_.launch("hbr_predict", dim3((uint32_t)((n + 255) / 256)), dim3(256), a);
}

void Forest::predict_host(const float *x, uint64_t n, uint64_t n_cols, float missing, float *out,
                          const float *init) {
    if (n == 0) return;
    const uint64_t k = n_outputs_;
    const uint64_t row_bytes = n_cols * sizeof(float);
    hipStream_t s = dev_.stream();
    DBuf<float> dout(n * k), dinit(init ? n * k : 0);
    if (init) dinit.upload(init, n * k, s);
    // below a few chunks' worth the plain copy is as fast
    constexpr uint64_t kChunkBytes = 128ull << 20;
    if (row_bytes == 0 || n * row_bytes < 2 * kChunkBytes) {
        DBuf<float> dx(n * n_cols);
        dx.upload(x, n * n_cols, s);
        predict_device(dx.get(), n, n_cols, missing, dout.get(), nullptr, init ? dinit.get() : nullptr);
        dout.download(out, n * k, s);
        dev_.sync();
        return;
    }
    const uint64_t chunk_rows = std::max<uint64_t>(64, kChunkBytes / row_bytes / 64 * 64);
    dev_.host_rows(x, n, n_cols, chunk_rows, [&](const float *rows_dev, uint64_t r0, uint64_t rows) {
        predict_device(rows_dev, rows, n_cols, missing, dout.get() + r0 * k, nullptr,
                       init ? dinit.get() + r0 * k : nullptr);
    });
    dout.download(out, n * k, s);
    dev_.sync();
}

// Consecutive whole trees per chunk, as many as `cap` nodes hold (at most
// 256 trees, the kernel's root and weight tables).
void Forest::plan_chunks(uint32_t cap) {
    if (cap == chunk_cap_ && n_chunks_) return;
    std::vector<uint32_t> tree{0}, node{0};
    uint32_t used = 0, at = 0;
    for (uint64_t t = 0; t < n_trees_; t++) {
        if (used + tree_nodes_[t] > cap || (uint32_t)t - tree.back() >= 256) {
            tree.push_back((uint32_t)t);
            node.push_back(at);
            used = 0;
        }
        used += tree_nodes_[t];
        at += tree_nodes_[t];
    }
    tree.push_back((uint32_t)n_trees_);
    node.push_back(at);
    n_chunks_ = (uint32_t)tree.size() - 1;
    chunk_cap_ = cap;
    chunk_tree_.resize(tree.size());
    chunk_node_.resize(node.size());
    chunk_tree_.upload(tree.data(), tree.size(), dev_.stream());
    chunk_node_.upload(node.data(), node.size(), dev_.stream());
    dev_.sync();
}

}  // namespace hbr
