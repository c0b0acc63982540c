// Tree growth and the boosting loop over the device engine.
//
// TreeBuilder restates the hist builder's orchestration
// (builder/hist/mod.rs:261-573 host growth, hist/device.rs:147-696 device
// growth): node ids in expansion order, the depthwise frontier and the
// loss-guided heap, child bounds and statistics, terminal children at the
// depth limit, and the final leaf values (builder/shared.rs:174-187). The
// engine partitions, builds and searches whole levels; the host keeps the
// tree and decides each expansion from the winners the device returns.
//
// Trainer restates a plain gbtree run (training/round.rs:105-148,
// :214-424; training/train.rs:406-436): intercepts, then per iteration the
// gradients of the device margins, one tree per output, and each leaf's
// value added to its rows' margins.
#pragma once
#include <cstdint>
#include <vector>

#include "engine.h"
#include "split_math.h"

namespace hbr {

struct TreeNode {
    uint32_t split_feature = 0;
    float split_cond = 0.0f;
    uint8_t default_left = 1;
    int32_t left = -1, right = -1;
    float leaf_value = 0.0f, sum_hess = 0.0f, split_gain = 0.0f;
    int64_t split_bin = -2;
    uint32_t split_limit = 0;  // present local bins below go left
    // a categorical split (regtree.rs:59-66): its categories, which go left,
    // are the tree's categories[cat_begin, cat_end)
    uint8_t is_categorical = 0;
    uint32_t cat_begin = 0, cat_end = 0;
};

struct Tree {
    std::vector<TreeNode> nodes;
    std::vector<uint32_t> categories;
};

struct GrowParams {
    Reg reg{1.0, 0.0, 0.0, 1.0};
    double gamma = 0.0;
    uint64_t max_depth = 6;    // UINT64_MAX: unbounded
    uint64_t max_leaves = UINT64_MAX;
    int policy = HBR_GROW_DEPTHWISE;
    float eta = 0.3f;
    std::vector<int8_t> monotone;
};

class TreeBuilder {
public:
    TreeBuilder(Engine &e, const GrowParams &p);
    // Grow one tree from the staged gradients over every row; each leaf's
    // segment and (eta-scaled) value go to `leaves`. With `walk`, the rows
    // of the depth limit's children are not partitioned (their segments are
    // empty): the caller routes rows through the tree instead.
    Tree grow(std::vector<std::pair<Segment, float>> *leaves, bool walk = false);
    // A depthwise tree queued on the device (Engine::queue_device_tree),
    // and a finished one's records as a Tree.
    Engine::TreeTicket queue_device();
    // every softmax class's tree at once (Engine::queue_class_trees)
    Engine::TreeTicket queue_classes();
    Tree tree_from(const std::vector<GrowTreeNode> &nodes) const;

private:
    struct Open {
        int32_t nid;
        uint64_t depth;
        Segment seg;
        uint32_t slot;
        bool has_slot;
        QBin total;
        double lower, upper;
        ScanBest best;
        std::array<uint32_t, kCatWords> best_set;  // a categorical winner's local bins
        bool searched;
    };
    struct Decision {
        bool valid = false;
        uint32_t feature = 0;
        int64_t bin = -1;
        uint32_t limit = 0;
        uint32_t default_left = 0;
        QBin left{}, right{};
        double lg = 0, lh = 0, rg = 0, rh = 0;
        float wl = 0, wr = 0;
        double loss = 0.0;
        bool categorical = false;
        const std::array<uint32_t, kCatWords> *set = nullptr;
    };
    Decision decide(const Open &o) const;
    // Expand node o by d: children appended to the tree; returns the level split.
    LevelSplit expand(Tree &t, const Open &o, const Decision &d, double cb[4]);
    void leaf(const Open &o);
    double deq_g(int64_t k) const;
    double deq_h(int64_t k) const;

    Engine &e_;
    GrowParams p_;
    // per node id
    std::vector<double> g_, h_, lower_, upper_;
    std::vector<std::pair<int32_t, Segment>> leaves_;
};

struct TrainParams {
    GrowParams grow;
    int objective = HBR_OBJ_SQUARED_ERROR;
    uint32_t num_class = 0;
    float scale_pos_weight = 1.0f;
    bool has_base_score = false;
    float base_score = 0.5f;
};

class Trainer {
public:
    Trainer(Engine &e, const TrainParams &p, const float *labels, const float *weights, uint64_t n);
    void boost(uint64_t rounds);
    uint32_t outputs() const { return k_; }
    const std::vector<float> &base_score() const { return base_; }
    const std::vector<Tree> &trees() const { return trees_; }
    void margins(float *out);
    // Evaluation sets: a dense f32 matrix of the training features whose
    // margins follow the trees on the device (base_margin: [n][outputs] or
    // null for the base score).
    uint32_t add_eval(const float *x, uint64_t n, uint64_t n_cols, float missing, const float *base_margin);
    void eval_margins(uint32_t set, float *out);
    uint64_t eval_rows(uint32_t set) const { return e_.eval_rows(set); }
    void check_eval_owner() const;
    // softmax depthwise rounds grow their class trees as one batch (else one
    // class tree after another); HBROCM_SOFTMAX_BATCH=0 turns it off
    bool softmax_batches = true;

private:
    void boost_softmax_pipelined(uint64_t rounds);
    void boost_softmax_batched(uint64_t rounds);
    void boost_pipelined(uint64_t rounds, const hbr_device_loss &loss, bool fused);
    hbr_device_loss device_loss() const;
    // one grown tree onto the margins of output `output` (and, given
    // next_loss, the next round's gradients in the same pass)
    void grow_and_add(TreeBuilder &b, uint32_t output, const hbr_device_loss *next_loss = nullptr);
    bool grads_ready_ = false;  // the device holds the next round's gradients
    uint64_t since_order_ = 0;  // trees since the engine last reordered the rows

    Engine &e_;
    TrainParams p_;
    uint32_t k_ = 1;
    uint64_t n_;
    std::vector<float> labels_, weights_;
    std::vector<float> base_;
    std::vector<Tree> trees_;
    uint64_t eval_owner_ = 0;  // the engine's eval-set owner number at construction
};

std::vector<GrowTreeNode> records_of(const Tree &t);

// The loss's intercepts (objective base margins, train.rs:406-436).
std::vector<float> base_margins(const TrainParams &p, const float *labels, const float *weights, uint64_t n);

}  // namespace hbr
