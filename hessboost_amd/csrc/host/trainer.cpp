#include "trainer.h"

#include <algorithm>
#include <cfloat>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <limits>
#include <memory>

namespace hbr {

static std::unique_ptr<Engine::EvalCats> eval_cats_of(const Tree &t);

namespace {

// total order of f64 (f64::total_cmp) as a signed key
int64_t total_key(double x) {
    int64_t b;
    std::memcpy(&b, &x, 8);
    return b ^ (int64_t)(((uint64_t)(b >> 63)) >> 1);
}

}  // namespace

TreeBuilder::TreeBuilder(Engine &e, const GrowParams &p) : e_(e), p_(p) {}

double TreeBuilder::deq_g(int64_t k) const { return std::ldexp((double)k, e_.scale().exp_g); }
double TreeBuilder::deq_h(int64_t k) const { return std::ldexp((double)k, e_.scale().exp_h); }

// The winner as the reference records it: SplitPos from the candidate's
// place in its feature's order (forward bins, then the backward pass), the
// children's statistics, bounded f32 weights, and BestSplit::valid
// (builder/mod.rs:167-193).
TreeBuilder::Decision TreeBuilder::decide(const Open &o) const {
    Decision d;
    if (!o.searched || o.best.index == 0xffffffffu) return d;
    const ScanBest &b = o.best;
    const auto &fo = e_.feature_offset();
    const uint32_t f = b.feature, fs = fo[f], nb = fo[f + 1] - fs;
    d.feature = f;
    d.loss = (double)b.loss;
    if (b.flags & kScanCategorical) {
        // the set's child on the left, missing values as flags bit 0 says
        // (BestSplit::categorical with the children swapped, builder/categorical.rs:83-96)
        d.categorical = true;
        d.set = &o.best_set;
        d.bin = -1;
        d.limit = 0;
        d.default_left = b.flags & 1u;
    } else if (b.index < nb) {
        d.bin = (int64_t)fs + b.index;
        d.limit = b.index + 1;
        d.default_left = 0;
    } else {
        const uint32_t off = nb - 1 - (b.index - nb);
        d.bin = off == 0 ? -1 : (int64_t)fs + off - 1;
        d.limit = off;
        d.default_left = 1;
    }
    d.left = b.left;
    d.right = b.right;
    d.lg = deq_g(b.left.g);
    d.lh = deq_h(b.left.h);
    d.rg = deq_g(b.right.g);
    d.rh = deq_h(b.right.h);
    d.wl = xgb_weight(d.lg, d.lh, p_.reg, o.lower, o.upper);
    d.wr = xgb_weight(d.rg, d.rh, p_.reg, o.lower, o.upper);
    d.valid = d.loss > 1e-6 && d.loss >= p_.gamma && children_valid(d.lh, d.rh, p_.reg.min_child_weight);
    return d;
}

LevelSplit TreeBuilder::expand(Tree &t, const Open &o, const Decision &d, double cb[4]) {
    const int dir = d.feature < p_.monotone.size() ? p_.monotone[d.feature] : 0;
    if (d.categorical) {
        // bounds in the orientation the split was scored in (builder/mod.rs:175-182)
        double sw[4];
        child_bounds(o.lower, o.upper, dir, (double)d.wr, (double)d.wl, sw);
        cb[0] = sw[2];
        cb[1] = sw[3];
        cb[2] = sw[0];
        cb[3] = sw[1];
    } else {
        child_bounds(o.lower, o.upper, dir, (double)d.wl, (double)d.wr, cb);
    }
    TreeNode &n = t.nodes[o.nid];
    n.split_feature = d.feature;
    n.split_cond = d.categorical ? 0.0f : (d.bin >= 0 ? e_.cut_values()[d.bin] : -FLT_MAX);
    n.default_left = (uint8_t)d.default_left;
    n.split_bin = d.bin;
    n.split_limit = d.limit;
    n.split_gain = (float)d.loss;
    std::array<uint32_t, kCatWords> table{};
    if (d.categorical) {
        // the set's codes, sorted (BestSplit's set.sort_unstable()), into the
        // tree's pool; rows go left by their bin's code (categories_left,
        // quantile.rs:316-333)
        const auto &fo = e_.feature_offset();
        const uint32_t fs = fo[d.feature], nb = fo[d.feature + 1] - fs;
        std::vector<uint32_t> codes;
        for (uint32_t i = 0; i < nb; i++)
            if ((*d.set)[i / 32] >> (i % 32) & 1u) codes.push_back(category_code(e_.cut_values()[fs + i]));
        std::sort(codes.begin(), codes.end());
        n.is_categorical = 1;
        n.cat_begin = (uint32_t)t.categories.size();
        t.categories.insert(t.categories.end(), codes.begin(), codes.end());
        n.cat_end = (uint32_t)t.categories.size();
        for (uint32_t i = 0; i < nb; i++)
            if (std::binary_search(codes.begin(), codes.end(), category_code(e_.cut_values()[fs + i])))
                table[i / 32] |= 1u << (i % 32);
    }
    const int32_t left = (int32_t)t.nodes.size();
    n.left = left;
    n.right = left + 1;
    TreeNode ln, rn;
    ln.leaf_value = d.wl;
    ln.sum_hess = (float)d.lh;
    rn.leaf_value = d.wr;
    rn.sum_hess = (float)d.rh;
    t.nodes.push_back(ln);
    t.nodes.push_back(rn);
    g_.push_back(d.lg);
    h_.push_back(d.lh);
    lower_.push_back(cb[0]);
    upper_.push_back(cb[1]);
    g_.push_back(d.rg);
    h_.push_back(d.rh);
    lower_.push_back(cb[2]);
    upper_.push_back(cb[3]);
    LevelSplit s;
    s.seg = o.seg;
    s.parent_slot = o.slot;
    s.feature = d.feature;
    s.limit = d.limit;
    s.default_left = d.default_left;
    s.categorical = d.categorical;
    s.table = table;
    s.child_total[0] = d.left;
    s.child_total[1] = d.right;
    s.child_root_gain[0] = xgb_node_gain(d.lg, d.lh, p_.reg, cb[0], cb[1]);
    s.child_root_gain[1] = xgb_node_gain(d.rg, d.rh, p_.reg, cb[2], cb[3]);
    s.child_lower[0] = (float)cb[0];
    s.child_upper[0] = (float)cb[1];
    s.child_lower[1] = (float)cb[2];
    s.child_upper[1] = (float)cb[3];
    return s;
}

void TreeBuilder::leaf(const Open &o) {
    leaves_.push_back({o.nid, o.seg});
    if (o.has_slot) e_.free_slot(o.slot);
}

Engine::TreeTicket TreeBuilder::queue_device() {
    e_.set_scan_params(ScanParams{p_.reg.lambda, p_.reg.alpha, p_.reg.max_delta_step, p_.reg.min_child_weight},
                       p_.monotone);
    e_.begin_tree();
    return e_.queue_device_tree(p_.max_depth, p_.gamma, p_.eta);
}

Engine::TreeTicket TreeBuilder::queue_classes() {
    e_.set_scan_params(ScanParams{p_.reg.lambda, p_.reg.alpha, p_.reg.max_delta_step, p_.reg.min_child_weight},
                       p_.monotone);
    e_.begin_tree();
    return e_.queue_class_trees(p_.max_depth, p_.gamma, p_.eta);
}

// A device-grown tree's records as the model's nodes (split thresholds from
// the cuts on the host).
Tree TreeBuilder::tree_from(const std::vector<GrowTreeNode> &dn) const {
    Tree t;
    const auto &cuts = e_.cut_values();
    t.nodes.resize(dn.size());
    for (size_t i = 0; i < dn.size(); i++) {
        const GrowTreeNode &d = dn[i];
        TreeNode &n = t.nodes[i];
        n.leaf_value = d.value;
        n.sum_hess = d.sum_hess;
        if (d.left < 0) continue;  // a leaf keeps the defaults (split_bin -2)
        if (d.left + 1 >= (int32_t)dn.size() || (d.bin >= 0 && (size_t)d.bin >= cuts.size()))
            fail(kInvalid, "device growth: malformed node");
        n.split_feature = d.feature;
        n.split_cond = d.bin >= 0 ? cuts[d.bin] : -FLT_MAX;
        n.default_left = (uint8_t)d.default_left;
        n.left = d.left;
        n.right = d.left + 1;
        n.split_gain = d.gain;
        n.split_bin = d.bin;
        n.split_limit = d.limit;
    }
    return t;
}

Tree TreeBuilder::grow(std::vector<std::pair<Segment, float>> *leaves_out, bool walk) {
    Tree t;
    g_.clear();
    h_.clear();
    lower_.clear();
    upper_.clear();
    leaves_.clear();
    const uint64_t limit = p_.max_depth;
    e_.set_scan_params(ScanParams{p_.reg.lambda, p_.reg.alpha, p_.reg.max_delta_step, p_.reg.min_child_weight},
                       p_.monotone);

    // a depthwise tree whose depth limit's rows the walk routes: decided on
    // the device level by level, read back once
    if (walk && p_.policy == HBR_GROW_DEPTHWISE && e_.can_grow_device(limit)) {
        e_.begin_tree();
        std::vector<GrowTreeNode> dn;
        if (!e_.grow_device(limit, p_.gamma, p_.eta, dn))
            fail(kRefused, "a gradient is not finite: the round runs on the host");
        return tree_from(dn);
    }

    // root (builder/hist/mod.rs:345-456): statistics, histogram, search
    e_.begin_tree();
    Open root{};
    root.nid = 0;
    root.depth = 0;
    root.seg = Segment{0, (uint32_t)e_.n_rows(), 0};
    root.lower = -std::numeric_limits<double>::infinity();
    root.upper = std::numeric_limits<double>::infinity();
    if (limit > 0) {
        // total, histogram and search in one round trip (the root gain is
        // computed on the device from the device total)
        root.slot = e_.alloc_slot();
        root.has_slot = true;
        if (!e_.grow_root(root.seg, root.slot, (float)root.lower, (float)root.upper, &root.total, &root.best,
                          root.best_set.data()))
            fail(kRefused, "a gradient is not finite: the round runs on the host");
        root.searched = true;
    } else {
        root.total = e_.root_total(root.seg);
    }
    const double rg = deq_g(root.total.g), rh = deq_h(root.total.h);
    TreeNode rn;
    rn.sum_hess = (float)rh;
    t.nodes.push_back(rn);
    g_.push_back(rg);
    h_.push_back(rh);
    lower_.push_back(root.lower);
    upper_.push_back(root.upper);

    if (p_.policy == HBR_GROW_DEPTHWISE) {
        std::vector<Open> frontier{root};
        uint64_t depth = 0;
        while (depth < limit && !frontier.empty()) {
            std::vector<LevelSplit> splits;
            std::vector<std::pair<int32_t, int32_t>> ids;  // children's node ids
            std::vector<Open> parents;
            for (const Open &o : frontier) {
                const Decision d = decide(o);
                if (!d.valid) {
                    leaf(o);
                    continue;
                }
                double cb[4];
                const int32_t left = (int32_t)t.nodes.size();
                splits.push_back(expand(t, o, d, cb));
                ids.push_back({left, left + 1});
                parents.push_back(o);
            }
            const bool terminal = depth + 1 >= limit;
            // the depth limit's children are only needed for their rows'
            // margins, which the walk finds without a partition
            std::vector<LevelChild> kids =
                terminal && walk ? std::vector<LevelChild>(2 * splits.size()) : e_.level(splits, terminal);
            std::vector<Open> next;
            for (size_t i = 0; i < splits.size(); i++) {
                for (int c = 0; c < 2; c++) {
                    Open ch{};
                    ch.nid = c == 0 ? ids[i].first : ids[i].second;
                    ch.depth = depth + 1;
                    ch.seg = kids[2 * i + c].seg;
                    ch.total = splits[i].child_total[c];
                    ch.lower = lower_[ch.nid];
                    ch.upper = upper_[ch.nid];
                    if (terminal) {
                        leaves_.push_back({ch.nid, ch.seg});
                    } else {
                        ch.slot = kids[2 * i + c].slot;
                        ch.has_slot = true;
                        ch.best = kids[2 * i + c].best;
                        ch.best_set = kids[2 * i + c].best_set;
                        ch.searched = true;
                        next.push_back(ch);
                    }
                }
                if (terminal && parents[i].has_slot) e_.free_slot(parents[i].slot);
            }
            frontier.swap(next);
            depth++;
        }
        for (const Open &o : frontier) leaf(o);
    } else {
        // std::collections::BinaryHeap by best.loss_chg (total_cmp): push =
        // sift_up; pop = swap-remove the root, sift_down_to_bottom, sift_up.
        std::vector<Open> heap;
        // a node without a candidate holds BestSplit::none, whose loss is 0
        auto key = [&](const Open &o) -> int64_t {
            return total_key(o.searched && o.best.index != 0xffffffffu ? (double)o.best.loss : 0.0);
        };
        auto sift_up = [&](size_t start, size_t pos) {
            Open elem = heap[pos];
            const int64_t k = key(elem);
            while (pos > start) {
                size_t parent = (pos - 1) / 2;
                if (k <= key(heap[parent])) break;
                heap[pos] = heap[parent];
                pos = parent;
            }
            heap[pos] = elem;
        };
        auto push = [&](const Open &o) {
            heap.push_back(o);
            sift_up(0, heap.size() - 1);
        };
        auto pop = [&](Open *out) -> bool {
            if (heap.empty()) return false;
            Open item = heap.back();
            heap.pop_back();
            if (!heap.empty()) {
                std::swap(item, heap[0]);
                size_t end = heap.size(), pos = 0;
                Open elem = heap[0];
                size_t child = 1;
                while (child + 2 <= end) {
                    if (key(heap[child]) <= key(heap[child + 1])) child++;
                    heap[pos] = heap[child];
                    pos = child;
                    child = 2 * pos + 1;
                }
                if (child == end - 1) {
                    heap[pos] = heap[child];
                    pos = child;
                }
                heap[pos] = elem;
                sift_up(0, pos);
            }
            *out = item;
            return true;
        };
        push(root);
        uint64_t n_leaves = 1;
        Open o;
        while (pop(&o)) {
            if (n_leaves >= p_.max_leaves) {
                leaf(o);
                break;
            }
            const Decision d = decide(o);
            if (!(o.depth < limit && d.valid)) {
                leaf(o);
                continue;
            }
            double cb[4];
            const int32_t left = (int32_t)t.nodes.size();
            std::vector<LevelSplit> one{expand(t, o, d, cb)};
            std::vector<LevelChild> kids = e_.level(one, false);
            n_leaves++;
            for (int c = 0; c < 2; c++) {
                Open ch{};
                ch.nid = left + c;
                ch.depth = o.depth + 1;
                ch.seg = kids[c].seg;
                ch.slot = kids[c].slot;
                ch.has_slot = true;
                ch.total = one[0].child_total[c];
                ch.lower = lower_[ch.nid];
                ch.upper = upper_[ch.nid];
                ch.best = kids[c].best;
                ch.best_set = kids[c].best_set;
                ch.searched = true;
                push(ch);
            }
        }
        for (const Open &rest : heap) leaf(rest);
    }

    // finalize_leaf_values (builder/shared.rs:174-187), then scale_leaves(eta)
    for (auto &lf : leaves_) {
        TreeNode &n = t.nodes[lf.first];
        const double w = calc_weight_bounded(g_[lf.first], h_[lf.first], p_.reg, lower_[lf.first], upper_[lf.first]);
        n.leaf_value = (float)w * p_.eta;
        n.left = n.right = -1;
        n.split_bin = -2;
        if (leaves_out) leaves_out->push_back({lf.second, n.leaf_value});
    }
    return t;
}

// ---- the boosting loop ----------------------------------------------------------

// the Hessian floor of the logistic and softmax losses (objective/mod.rs:150)
constexpr float kMinHess = 1e-16f;

static float weighted_label_mean(const float *labels, const float *weights, uint64_t n) {
    double mean = 0.0;
    if (weights) {
        double sum_w = 0.0;
        for (uint64_t i = 0; i < n; i++) sum_w += (double)weights[i];
        if (sum_w > 0.0)
            for (uint64_t i = 0; i < n; i++) mean += (double)labels[i] / sum_w * (double)weights[i];
    } else if (n > 0) {
        const double dn = (double)n;
        for (uint64_t i = 0; i < n; i++) mean += (double)labels[i] / dn;
    }
    return (float)mean;
}

static float logit(float p) {
    const float eps = 1e-6f;
    p = p < eps ? eps : (p > 1.0f - eps ? 1.0f - eps : p);
    return -std::log(1.0f / p - 1.0f);
}

// newton_intercepts (objective/mod.rs:528-547): one Newton step from
// all-zero margins, fit_stump (:552-566: -G / max(H, 1e-6) with G, H summed
// in f64 in row order, rounded once to f32); the caller applies
// pred_transform and the link. The pairs at a zero margin in closed form,
// with w' = w scaled by scale_pos_weight for a label of exactly 1:
//   squared error (regression.rs:42-58): g = (0 - y) w', h = w';
//   logistic (simd/scalar.rs:8-29): both of the reference's paths give
//   p = 1 / (1 + 1) = 0.5 exactly (the AVX2 exp polynomial and libm expf
//   both return 1 at 0), so g = (0.5 - y) w', h = max(0.25, 1e-16) w'.
static float newton_step(bool logistic, const float *labels, const float *weights, uint64_t n, float spw) {
    double g = 0.0, h = 0.0;
    for (uint64_t i = 0; i < n; i++) {
        const float y = labels[i];
        float w = weights ? weights[i] : 1.0f;
        if (y == 1.0f) w *= spw;
        const float gi = logistic ? (0.5f - y) * w : (0.0f - y) * w;
        const float hi = logistic ? std::fmax(0.25f, kMinHess) * w : w;
        g += (double)gi;
        h += (double)hi;
    }
    return (float)(-g / std::fmax(h, 1e-6));
}

std::vector<float> base_margins(const TrainParams &p, const float *labels, const float *weights, uint64_t n) {
    if (p.objective == HBR_OBJ_SOFTMAX) {
        const uint32_t k = p.num_class;
        std::vector<float> m(k, 0.0f);
        if (p.has_base_score) {
            for (auto &v : m) v = p.base_score;
            return m;
        }
        for (uint64_t i = 0; i < n; i++) {
            if (labels[i] >= 0.0f && (uint32_t)labels[i] < k) m[(uint32_t)labels[i]] += weights ? weights[i] : 1.0f;
        }
        double sum_w = 0.0;
        if (weights)
            for (uint64_t i = 0; i < n; i++) sum_w += (double)weights[i];
        else
            sum_w = (double)(float)n;
        const double inv = 1.0 / sum_w;
        for (auto &v : m) v = std::log((float)((double)v * inv) + 1e-6f);
        const float kf = (float)k;
        float mean = -0.0f;
        for (float v : m) mean += v / kf;
        for (auto &v : m) v -= mean;
        return m;
    }
    if (p.objective == HBR_OBJ_LOGISTIC || p.objective == HBR_OBJ_LOGITRAW) {
        // classification.rs:67-72: binary:logitraw's link is the identity;
        // :132-141: a scale_pos_weight away from 1 takes the Newton step
        const bool raw = p.objective == HBR_OBJ_LOGITRAW;
        if (p.has_base_score) return {raw ? p.base_score : logit(p.base_score)};
        if (std::fabs(p.scale_pos_weight - 1.0f) > 1e-6f) {
            const float step = newton_step(true, labels, weights, n, p.scale_pos_weight);
            if (raw) return {step};
            return {logit(1.0f / (std::exp(std::fmin(-step, 88.7f)) + 1.0f))};  // sigmoid_scalar, simd/mod.rs:425-427
        }
        const float mean = weighted_label_mean(labels, weights, n);
        return {raw ? mean : logit(mean)};
    }
    // regression.rs:66-74: the Newton step when scale_pos_weight != 1
    if (p.has_base_score) return {p.base_score};
    if (std::fabs(p.scale_pos_weight - 1.0f) > 1e-6f)
        return {newton_step(false, labels, weights, n, p.scale_pos_weight)};
    return {weighted_label_mean(labels, weights, n)};
}

Trainer::Trainer(Engine &e, const TrainParams &p, const float *labels, const float *weights, uint64_t n)
    : e_(e), p_(p), n_(n) {
    if (n != e.n_rows()) fail(kInvalid, "trainer: one label per index row");
    eval_owner_ = e.clear_eval_sets();  // an earlier trainer's sets would take this one's trees
    k_ = p.objective == HBR_OBJ_SOFTMAX ? p.num_class : 1;
    if (k_ == 0) fail(kInvalid, "softmax needs num_class");
    if (p.objective == HBR_OBJ_SOFTMAX) {
        if (k_ > kSoftmaxMaxClasses) fail(kRefused, "softmax: at most 1024 classes");
        // multiclass.rs:96-100: class indices, non-negative integers below num_class
        for (uint64_t i = 0; i < n; i++) {
            const float y = labels[i];
            if (!(y >= 0.0f && y < (float)k_) || y != std::floor(y))
                fail(kInvalid, "softmax labels must be class indices below num_class");
        }
    }
    labels_.assign(labels, labels + n);
    if (weights) weights_.assign(weights, weights + n);
    if (const char *v = std::getenv("HBROCM_SOFTMAX_BATCH")) softmax_batches = std::strtol(v, nullptr, 10) != 0;
    base_ = base_margins(p, labels, weights, n);
    // training/train.rs:425-433: a non-finite intercept is an error
    for (float b : base_)
        if (!std::isfinite(b)) fail(kInvalid, "estimated intercept is not finite; check the labels");
    std::vector<float> m((size_t)n * k_);
    for (uint64_t r = 0; r < n; r++)
        for (uint32_t c = 0; c < k_; c++) m[r * k_ + c] = base_[c];
    e_.load_margins(m.data(), m.size(), k_);
    e_.set_labels(labels, weights, n);
}

// Leaf values onto the margins (training/margins.rs:247-289): by routing
// every row through the tree on its bins when the index allows it, else
// over each leaf's row segment.
void Trainer::grow_and_add(TreeBuilder &b, uint32_t output, const hbr_device_loss *next_loss) {
    const bool walk = e_.can_walk();
    std::vector<std::pair<Segment, float>> leaves;
    trees_.push_back(b.grow(&leaves, walk));
    const Tree &t = trees_.back();
    grads_ready_ = false;
    if (e_.n_eval_sets()) e_.walk_evals(records_of(t), output, nullptr, eval_cats_of(t).get());
    if (walk) {
        const size_t n = t.nodes.size();
        std::vector<uint32_t> meta(n), left(n, 0);
        std::vector<float> value(n, 0.0f);
        for (size_t i = 0; i < n; i++) {
            const TreeNode &nd = t.nodes[i];
            if (nd.left < 0) {
                meta[i] = 1u << 31;
                value[i] = nd.leaf_value;
            } else {
                meta[i] = nd.split_feature | (nd.default_left ? kMetaDefaultLeft : 0u) | (nd.split_limit << 16);
                left[i] = (uint32_t)nd.left;
            }
        }
        if (next_loss && e_.can_walk_gradients(n)) {
            e_.walk_add(meta, left, value, output, next_loss);
            grads_ready_ = true;
        } else {
            e_.walk_add(meta, left, value, output);
        }
        return;
    }
    std::vector<Segment> segs;
    std::vector<float> vals;
    for (auto &l : leaves) {
        segs.push_back(l.first);
        vals.push_back(l.second);
    }
    e_.add_leaves(segs, vals, output);
}

// Rounds with the device a tree ahead of the host: tree t+1 and its
// margin walk are queued before tree t is read back, so the device never
// waits for the host. A tree whose gradients turn out not to be finite had
// its walk skipped on the device, and so had every tree queued after it:
// the margins hold the trees before it, and training stops there.
void Trainer::boost_pipelined(uint64_t rounds, const hbr_device_loss &loss, bool fused) {
    TreeBuilder b(e_, p_.grow);
    std::deque<Engine::TreeTicket> inflight;
    uint64_t queued = 0, done = 0;
    while (done < rounds) {
        while (queued < rounds && inflight.size() < 3) {
            if (!grads_ready_) e_.compute_gradients_async(loss, 0);
            inflight.push_back(b.queue_device());
            // before the first tree's walk (and every row_order_every trees
            // after): the rows by that tree's leaves, so that later trees'
            // deep nodes sit together in memory
            if (fused && e_.row_order &&
                (!e_.rows_permuted() || (e_.row_order_every && since_order_ >= e_.row_order_every))) {
                e_.order_rows_by_tree();
                since_order_ = 0;
            }
            since_order_++;
            if (fused)
                e_.walk_device_tree(0, &loss);
            else
                e_.walk_device_tree_then_gradients(loss);
            e_.walk_evals_device(0, 0, true);
            grads_ready_ = true;
            queued++;
        }
        std::vector<GrowTreeNode> nodes;
        const Engine::TreeState st = e_.finish_device_tree(inflight.front(), nodes, nullptr);
        inflight.pop_front();
        if (st != Engine::kTreeOk) {
            e_.drain();
            fail(kRefused, "a gradient is not finite");
        }
        trees_.push_back(b.tree_from(nodes));
        done++;
    }
}

// Softmax rounds with the device ahead of the host: every class's
// gradients at the start of a round (one kernel, from the margins every
// earlier tree has been walked into), then the round's trees, class by
// class, each grown from its class's pairs and walked into its class's
// margins on the device; up to three trees in flight before the host reads
// the oldest back. A tree whose class's gradients are not finite had its
// walks skipped on the device, and so had every tree queued after it: the
// margins and eval sets hold the trees before it, and training stops there.
void Trainer::boost_softmax_pipelined(uint64_t rounds) {
    TreeBuilder b(e_, p_.grow);
    std::deque<Engine::TreeTicket> inflight;
    const uint64_t total = rounds * k_;
    uint64_t queued = 0, done = 0;
    while (done < total) {
        while (queued < total && inflight.size() < 3) {
            const uint32_t c = (uint32_t)(queued % k_);
            if (c == 0) e_.softmax_gradients_async(kMinHess);
            e_.select_class(c);
            inflight.push_back(b.queue_device());
            // guarded by the class's scale: a tree grown from gradients that
            // are not finite, and every tree queued after it, reach no margins
            e_.walk_device_tree(c, nullptr, 0, c, 1);
            e_.walk_evals_device(c, 0, true);
            queued++;
        }
        std::vector<GrowTreeNode> nodes;
        const Engine::TreeState st = e_.finish_device_tree(inflight.front(), nodes, nullptr);
        inflight.pop_front();
        if (st != Engine::kTreeOk) {
            e_.drain();
            fail(kRefused, "a gradient is not finite");
        }
        trees_.push_back(b.tree_from(nodes));
        done++;
    }
}

// Softmax rounds as batches: every class's gradients, then the round's K
// class trees grown together level by level (one launch of each kernel per
// level for all of them), then each walked into its class's margins; up
// to three rounds in flight before the host reads the oldest back.
void Trainer::boost_softmax_batched(uint64_t rounds) {
    TreeBuilder b(e_, p_.grow);
    std::deque<Engine::TreeTicket> inflight;
    uint64_t queued = 0, done = 0;
    while (done < rounds) {
        while (queued < rounds && inflight.size() < 3) {
            e_.softmax_gradients_async(kMinHess);
            inflight.push_back(b.queue_classes());
            // guarded by every class's scale: the host keeps or drops a round whole
            const bool batched_walk = e_.walk_device_trees(0, k_, 0, k_);
            for (uint32_t c = 0; c < k_; c++) {
                if (!batched_walk) e_.walk_device_tree(c, nullptr, c, 0, k_);
                e_.walk_evals_device(c, c, true);
            }
            queued++;
        }
        std::vector<std::vector<GrowTreeNode>> trees;
        const Engine::TreeState st = e_.finish_device_forest(inflight.front(), trees);
        inflight.pop_front();
        if (st != Engine::kTreeOk) {
            e_.drain();
            fail(kRefused, "a gradient is not finite");
        }
        for (const auto &t : trees) trees_.push_back(b.tree_from(t));
        done++;
    }
}

void Trainer::boost(uint64_t rounds) {
    // every sum of the whole-round trainer is fixed point: its scans bound
    // their candidates and count the nodes they cannot certify
    e_.guard_active = e_.guard_on();
    e_.guard_gamma = (float)p_.grow.gamma;
    if (p_.objective == HBR_OBJ_SOFTMAX && p_.grow.policy == HBR_GROW_DEPTHWISE && softmax_batches &&
        e_.can_grow_device(p_.grow.max_depth, k_)) {
        boost_softmax_batched(rounds);
        return;
    }
    if (p_.objective == HBR_OBJ_SOFTMAX && p_.grow.policy == HBR_GROW_DEPTHWISE &&
        e_.can_route_device_tree(p_.grow.max_depth)) {
        boost_softmax_pipelined(rounds);
        return;
    }
    if (p_.objective != HBR_OBJ_SOFTMAX && p_.grow.policy == HBR_GROW_DEPTHWISE &&
        e_.can_walk_device_tree(p_.grow.max_depth)) {
        boost_pipelined(rounds, device_loss(), true);
        return;
    }
    // wider or masked rows, deeper trees: the same rounds with the walk and
    // the next gradients as two passes
    if (p_.objective != HBR_OBJ_SOFTMAX && p_.grow.policy == HBR_GROW_DEPTHWISE &&
        e_.can_walk_then_gradients(p_.grow.max_depth)) {
        boost_pipelined(rounds, device_loss(), false);
        return;
    }
    TreeBuilder b(e_, p_.grow);
    for (uint64_t it = 0; it < rounds; it++) {
        if (p_.objective == HBR_OBJ_SOFTMAX) {
            // every class's gradients from the round's starting margins
            e_.softmax_gradients_async(kMinHess);
            for (uint32_t c = 0; c < k_; c++) {
                e_.select_class(c);
                grow_and_add(b, c);
            }
            continue;
        }
        const hbr_device_loss loss = device_loss();
        // after the first round, the previous tree's margin update computed
        // this round's gradients; either way the root checks them
        if (!grads_ready_) e_.compute_gradients_async(loss, 0);
        grow_and_add(b, 0, &loss);
    }
}

hbr_device_loss Trainer::device_loss() const {
    hbr_device_loss loss{};
    loss.kind = p_.objective == HBR_OBJ_LOGISTIC || p_.objective == HBR_OBJ_LOGITRAW ? HBR_LOSS_LOGISTIC
                                                                                     : HBR_LOSS_SQUARED_ERROR;
    loss.scale_pos_weight = p_.scale_pos_weight;
    loss.min_hess = kMinHess;
    loss.max_input = 80.0f;
    loss.vector_rows = n_ >= 16 ? n_ - n_ % 8 : 0;
    return loss;
}

void Trainer::margins(float *out) { e_.read_margins(out, n_ * k_); }

// A tree's categorical splits as the evaluation walk reads them (null when
// it has none).
static std::unique_ptr<Engine::EvalCats> eval_cats_of(const Tree &t) {
    bool any = false;
    for (const TreeNode &n : t.nodes) any |= n.left >= 0 && n.is_categorical;
    if (!any) return nullptr;
    auto c = std::make_unique<Engine::EvalCats>();
    c->span.assign(2 * t.nodes.size(), 0u);
    for (size_t i = 0; i < t.nodes.size(); i++) {
        const TreeNode &n = t.nodes[i];
        if (n.left < 0 || !n.is_categorical) continue;
        c->span[2 * i] = n.cat_begin;
        c->span[2 * i + 1] = n.cat_end | (1u << 31);
    }
    c->categories = &t.categories;
    return c;
}

// A tree's nodes as the device walks read them: split bin (the threshold is
// its cut value), feature, default direction, children, leaf value.
std::vector<GrowTreeNode> records_of(const Tree &t) {
    std::vector<GrowTreeNode> r(t.nodes.size());
    for (size_t i = 0; i < t.nodes.size(); i++) {
        const TreeNode &n = t.nodes[i];
        GrowTreeNode &g = r[i];
        g = GrowTreeNode{};
        g.left = n.left;
        g.value = n.leaf_value;
        if (n.left < 0) continue;
        g.feature = n.split_feature;
        g.bin = (int32_t)n.split_bin;
        g.default_left = n.default_left;
    }
    return r;
}

// An evaluation set (training/margins.rs:148-152): its margins start from
// `base_margin` ([n][outputs]) or the base score, then take every tree
// grown so far, and every later tree as it is grown.
uint32_t Trainer::add_eval(const float *x, uint64_t n, uint64_t n_cols, float missing, const float *base_margin) {
    check_eval_owner();
    std::vector<float> init(n * k_);
    for (uint64_t r = 0; r < n; r++)
        for (uint32_t c = 0; c < k_; c++) init[r * k_ + c] = base_margin ? base_margin[r * k_ + c] : base_[c];
    const uint32_t set = e_.add_eval_set(x, n, n_cols, missing, init.data(), k_);
    for (size_t t = 0; t < trees_.size(); t++)
        e_.walk_evals_one(set, records_of(trees_[t]), (uint32_t)(t % k_), eval_cats_of(trees_[t]).get());
    return set;
}

void Trainer::eval_margins(uint32_t set, float *out) {
    check_eval_owner();
    e_.read_eval_margins(set, out);
}

void Trainer::check_eval_owner() const {
    if (e_.eval_owner() != eval_owner_)
        fail(kInvalid, "evaluation sets: a newer trainer on this engine owns them");
}

}  // namespace hbr
