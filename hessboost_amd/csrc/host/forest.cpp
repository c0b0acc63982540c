#include "forest.h"

#include <cstring>

namespace hbr {

// Each tree is re-laid out breadth-first so every internal node's children
// sit side by side (right = left + 1), the node records its original id for
// leaf queries, and the walk can never loop: every node is reached exactly
// once from the root, or the upload is refused.
Forest::Forest(int ordinal, const hbr_forest_desc &fd) : dev_(device(ordinal)) {
    n_trees_ = fd.n_trees;
    n_outputs_ = fd.n_outputs ? fd.n_outputs : 1;
    std::vector<uint32_t> value, meta, left, root, output;
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
                continue;
            }
            if (l < 0 || r < 0 || (uint64_t)l >= count || (uint64_t)r >= count || seen[l] || seen[r])
                fail(kInvalid, "forest: malformed tree " + std::to_string(t));
            if (fd.split_feature[at] >= (1u << 20)) fail(kInvalid, "forest: split feature beyond 2^20");
            seen[l] = seen[r] = 1;
            uint32_t bits;
            std::memcpy(&bits, &fd.split_cond[at], 4);
            value.push_back(bits);
            meta.push_back(fd.split_feature[at] | ((fd.default_left[at] ? 1u : 0u) << 30));
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
    up(weight_, weight);
    up(base_, base);
    dev_.sync();
}

void Forest::predict_device(const float *x, uint64_t n, uint64_t n_cols, float missing, float *out,
                            int32_t *leaf_out) {
    if (n == 0) return;
    if (n_trees_ && n_cols <= max_feature_) fail(kInvalid, "predict: rows have fewer columns than the forest reads");
    if (n >= (uint64_t)UINT32_MAX) fail(kRefused, "predict: more than 2^32 - 1 rows per call");
    PredictArgs a{};
    a.node_value = value_.get();
    a.node_meta = meta_.get();
    a.node_left = left_.get();
    a.node_orig = orig_.get();
    a.tree_root = root_.get();
    a.tree_weight = weight_.get();
    a.tree_output = output_.get();
    a.base_score = base_.get();
    a.x = x;
    a.out = out;
    a.leaf_out = leaf_out;
    a.n = (uint32_t)n;
    a.n_cols = (uint32_t)n_cols;
    a.n_trees = (uint32_t)n_trees_;
    a.n_outputs = n_outputs_;
    a.missing = missing;
    a.missing_is_nan = missing != missing ? 1u : 0u;
    dev_.launch("hbr_predict", dim3((uint32_t)((n + 255) / 256)), dim3(256), a);
}

}  // namespace hbr
