// The device engine: one binned index resident on one GPU, its gradients,
// margins, row buffers and histogram slots, and the level-batched growth
// steps the tree builder drives (the reference's HistogramBackend and
// RowEngine, src/tree/hist/mod.rs:73-295).
#pragma once
#include <array>
#include <algorithm>
#include <memory>
#include <cstdint>
#include <mutex>
#include <string>
#include <vector>

#include "../abi.h"
#include "runtime.h"

#include "hessboost_rocm.h"

namespace hbr {

// A node's rows on the device: `len` ids at `offset` of row buffer `buf`.
struct Segment {
    uint32_t offset = 0, len = 0, buf = 0;
};

// A category code: the saturating `value as u32` of the category's cut
// (in_category_set, tree/mod.rs:34-58).
inline uint32_t category_code(float v) {
    if (!(v >= 0.0f)) return 0;
    if (v >= 4294967296.0f) return 0xffffffffu;
    return (uint32_t)v;
}

// One split of a level: the parent's rows, slot and routing.
struct LevelSplit {
    Segment seg;
    uint32_t parent_slot = 0;  // parent's histogram (becomes the sibling's); unused when terminal
    uint32_t feature = 0;
    uint32_t limit = 0;        // present local bins below go left
    uint32_t default_left = 0;
    // a categorical split: the local bins that go left (RowRule::Table)
    bool categorical = false;
    std::array<uint32_t, kCatWords> table{};
    // child scan inputs (non-terminal levels)
    QBin child_total[2];
    float child_root_gain[2];
    float child_lower[2], child_upper[2];
};

struct LevelChild {
    Segment seg;
    uint32_t slot = 0;
    ScanBest best;  // valid when the level was not terminal
    std::array<uint32_t, kCatWords> best_set{};  // the local bins of a categorical winner's set
};

struct ScanInput {
    uint32_t slot;
    QBin total;
    float root_gain, lower, upper;
    uint32_t rows = 0;  // the node's row count (0: from the slot's segment, else every row)
};

class Engine {
public:
    Engine(int ordinal, const hbr_index_desc &desc);
    // A dense f32 matrix (row-major n_rows x n_cols, host or device memory)
    // binned on the device against host cuts (HistCuts::bin_of,
    // src/data/quantile.rs:285-296) into the layouts GHistIndex::from_dmatrix
    // would give (src/data/ghist.rs:213-257). Features of at most 256 bins.
    struct DenseSource {
        const float *x = nullptr;
        bool on_device = false;
        uint64_t n_rows = 0, n_cols = 0;
        float missing = 0.0f;
        const uint32_t *feature_offset = nullptr;  // n_cols + 1
        const float *cut_values = nullptr;
    };
    Engine(int ordinal, const DenseSource &src);
    // The engine's index as it sits on the device (for checking): whether it
    // is dense, its row-major stride (dense u8), stored entries, and whether
    // it keeps local columns and a missing bitmap.
    struct IndexInfo {
        bool dense, dense_u8, has_cols, has_missing;
        uint32_t stride;
        uint64_t entries;
    };
    IndexInfo index_info() const;
    // Copies of the layouts (null pointers skip one): rows8 n_rows x stride,
    // cols8 n_cols x n_rows, missing n_cols x words, row_ptr n_rows + 1,
    // gbins entries.
    void read_index(uint8_t *rows8, uint8_t *cols8, uint64_t *missing, uint64_t *row_ptr, uint32_t *gbins);
    ~Engine();

    std::mutex mu;
    bool failed = false;

    Device &dev() { return dev_; }
    uint64_t n_rows() const { return n_rows_; }
    uint32_t n_cols() const { return n_cols_; }
    uint32_t total_bins() const { return total_bins_; }
    bool dense() const { return dense_; }
    const std::vector<uint32_t> &feature_offset() const { return fo_; }
    const std::vector<float> &cut_values() const { return cuts_; }

    // ---- gradients -----------------------------------------------------------
    // Stage host gradient pairs for the next tree (HistogramBackend::prepare).
    void prepare(const float *gpair, uint64_t n);
    // Device margins and labels (RowEngine::load_margins / gradients).
    void load_margins(const float *m, uint64_t n, uint32_t outputs);
    void set_labels(const float *labels, const float *weights, uint64_t n);
    bool labels_loaded() const { return labels_loaded_; }
    // Gradients of output `output` from the device margins; false when some
    // gradient is not finite.
    bool compute_gradients(const hbr_device_loss &loss, uint32_t output);
    // The same without a host synchronisation: the exponents are computed on
    // the device and checked by the next tree's root or finish.
    void compute_gradients_async(const hbr_device_loss &loss, uint32_t output);
    // The root's total, histogram (into `slot`) and split search with one
    // host synchronisation; false when a gradient is not finite.
    // best_set (kCatWords words, may be null) receives a categorical
    // winner's set.
    bool grow_root(const Segment &seg, uint32_t slot, float lower, float upper, QBin *total, ScanBest *best,
                   uint32_t *best_set = nullptr);
    // Categorical features (HistCuts::is_categorical): at most kCatMaxBins
    // bins each. Their trees are grown by host-decided levels: the device
    // sweeps them (hbr_scan_categorical) and routes by table.
    bool has_categorical() const { return n_cat_ > 0; }
    bool is_categorical(uint32_t f) const { return n_cat_ > 0 && cat_rank_[f] != 0xffffffffu; }
    // Softmax gradients of every class (the margins' outputs, at most
    // kSoftmaxMaxClasses) from the device margins, with the host's bits,
    // class-major on the device, each class's scale folded; no
    // synchronisation. select_class(c) then stages class c's pairs and scale
    // for the next tree (checked by its root or its finish, like
    // compute_gradients_async).
    void softmax_gradients_async(float min_hess);
    void select_class(uint32_t c);
    bool softmax_staged() const { return class_pairs_.size() > 0 && class_outputs_ == outputs_; }
    // compute_gradients' check for the softmax: false when a class has a
    // gradient that is not finite
    bool softmax_all_finite();
    void read_margins(float *out, uint64_t n);
    // Rows reordered by the leaves of the last queued device tree (32-byte
    // rows of a dense index, trees of at most kOrderMaxNodes nodes): the
    // rows, columns, margins, labels and weights move to their new
    // positions; read_margins still returns the original order. The
    // whole-round trainer reorders once; every other caller restores the
    // original order first (restore_row_order, a no-op when nothing moved).
    void order_rows_by_tree();
    void restore_row_order();
    bool rows_permuted() const { return permuted_; }
    void read_gradients(float *out, uint64_t n);
    const QScale &scale() const { return scale_host_; }
    // Whether every sum of at most m staged pairs, in any order, is the
    // reference's f64 sum bit for bit (backend/exact_sum.rs:14-37): every
    // value finite, n x max <= 2^53 grains of each component, and the
    // fixed-point unit at or below the grain (the quantisation is then
    // lossless). False when the staged pairs' grains are not known (the
    // trainer's fused rounds, softmax classes).
    bool sums_exact(uint64_t m) const;
    uint32_t slot_capacity() const { return slot_cap_; }
    // The trait's contract for build / histograms / root_total / the
    // resident scan: when set, they refuse outside the exact domain.
    bool exact_sums_only = true;
    double unit_g() const;
    double unit_h() const;

    // ---- tree growth ------------------------------------------------------------
    uint64_t begin_tree();  // every row in buffer 0; returns the tree stamp
    uint64_t tree() const { return tree_; }
    QBin root_total(const Segment &s);
    // Build node histograms into their (zeroed) slots, then parent -= built.
    void build_nodes(const std::vector<Segment> &segs, const std::vector<uint32_t> &slots);
    void subtract(const std::vector<uint32_t> &parents, const std::vector<uint32_t> &built);
    // The split search of nodes given on the host (numeric and categorical
    // features); sets (may be null) receives kCatWords words per node, a
    // categorical winner's set of local bins.
    std::vector<ScanBest> scan(const std::vector<ScanInput> &nodes, std::vector<uint32_t> *sets = nullptr);
    // Partition + (non-terminal) smaller-child histograms, sibling subtraction
    // and the children's split search, with one host synchronisation.
    std::vector<LevelChild> level(const std::vector<LevelSplit> &splits, bool terminal);
    void add_leaves(const std::vector<Segment> &segs, const std::vector<float> &values, uint32_t output);
    // Dense u8 index: margins of output `output` += the leaf each row reaches
    // through the tree (meta/left/value as WalkArgs lays them out); needs no
    // row segments, so the depth limit's level can skip its partition.
    bool can_walk() const { return dense_u8_ && n_cat_ == 0; }
    // With next_loss, the same pass also computes the next round's gradients
    // of the updated margins (like compute_gradients_async; can_walk_gradients).
    void walk_add(const std::vector<uint32_t> &meta, const std::vector<uint32_t> &left,
                  const std::vector<float> &value, uint32_t output, const hbr_device_loss *next_loss = nullptr);
    bool can_walk_gradients(size_t n_nodes) const;
    // ---- depthwise growth on the device ----------------------------------------
    // A whole depthwise tree decided level by level on the device from the
    // staged gradients and read back with one synchronisation: the nodes in
    // tree order. Needs a dense u8 index (the depth limit's rows are routed
    // by the walk, not partitioned) and max_depth in [1, kMaxDeviceDepth].
    static constexpr uint32_t kMaxDeviceDepth = 13;
    bool can_grow_device(uint64_t max_depth, uint32_t n_trees = 1) const;
    // false when a gradient is not finite
    bool grow_device(uint64_t max_depth, double gamma, float eta, std::vector<GrowTreeNode> &nodes);
    // The same in two halves, so that a tree can be queued before the
    // previous one is read back: queue (no synchronisation), then finish
    // (waits for that tree's readback only). kTreeNotFinite: the gradients
    // it was grown from were not all finite; its guarded walk and every
    // later one were skipped, so the margins hold the trees before it
    // (drain() then waits for the queued work and clears the skip flag).
    struct TreeTicket {
        uint32_t slot = 0;
        bool check = false;  // the gradients' scale is checked at finish
        uint32_t n_trees = 1;
        size_t stride = 0;   // bytes between the trees of the ring slot
    };
    enum TreeState { kTreeOk = 0, kTreeNotFinite = 1 };
    TreeTicket queue_device_tree(uint64_t max_depth, double gamma, float eta);
    TreeState finish_device_tree(const TreeTicket &t, std::vector<GrowTreeNode> &nodes, QScale *scale);
    // The trees of every softmax class at once (the staged softmax pairs,
    // each class with its own scale), level by level: one launch of each
    // kernel per level for all of them. finish_device_forest reads the
    // batch back, tree c for class c; walk_device_tree(c, nullptr, c) adds
    // tree c to the margins of class c.
    TreeTicket queue_class_trees(uint64_t max_depth, double gamma, float eta);
    TreeState finish_device_forest(const TreeTicket &t, std::vector<std::vector<GrowTreeNode>> &trees);
    void drain();
    // The last queued device tree's leaves onto the margins of `output`,
    // routed on the device from its records (no readback); with next_loss
    // also the next round's gradients, guarded: skipped (and every later
    // guarded walk with it, until drain) when the tree's own gradients were
    // not finite. Without next_loss, guard_n > 0 guards the walk the same
    // way by the softmax class scales [guard_first, guard_first + guard_n)
    // (the tree's class, or every class of a batched round).
    bool can_walk_device_tree(uint64_t max_depth) const {
        return can_grow_device(max_depth) && stride_ == 32 && max_depth <= 9 && outputs_ == 1 && labels_loaded_;
    }
    // The walk alone (no gradients): any dense u8 index, any output.
    bool can_route_device_tree(uint64_t max_depth) const { return can_grow_device(max_depth); }
    // The last queued device tree's leaves onto the margins of one output by
    // the walk of any row layout (wider rows, masked rows, deeper trees),
    // guarded by the tree's own scale as walk_device_tree guards it, then
    // the next round's gradients from the updated margins: the two passes
    // the fused walk makes one.
    bool can_walk_then_gradients(uint64_t max_depth) const {
        return can_grow_device(max_depth) && outputs_ == 1 && labels_loaded_;
    }
    void walk_device_tree_then_gradients(const hbr_device_loss &next_loss);
    // The trees of the last queued batch (its trees 0..n_trees-1) added to
    // margins outputs first_output.. in one pass over the rows, guarded as
    // walk_device_tree; false (nothing queued) when the batch does not fit
    // the kernel, for the caller to walk the trees one at a time.
    bool walk_device_trees(uint32_t first_output, uint32_t n_trees, uint32_t guard_first, uint32_t guard_n);
    void walk_device_tree(uint32_t output, const hbr_device_loss *next_loss, uint32_t tree = 0,
                          uint32_t guard_first = 0, uint32_t guard_n = 0);

    // ---- evaluation sets ----------------------------------------------------------
    // A dense f32 matrix (row-major, the index's features, `missing` marks
    // an absent value; NaN: any NaN) kept on the device with its margins
    // ([n][outputs], from `init`), into which finished trees are walked by
    // raw value. Returns the set's number.
    uint32_t add_eval_set(const float *x, uint64_t n_rows, uint64_t n_cols, float missing, const float *init,
                          uint32_t outputs);
    // The last queued device tree (as walk_device_tree names it) into every
    // set's margins of `output`; `guarded`: not when the guarded training
    // walk before it skipped the tree.
    void walk_evals_device(uint32_t output, uint32_t tree, bool guarded);
    // A tree given as records (a host-grown tree) into every set's margins;
    // `cond`: per node thresholds instead of the split bins' cut values;
    // `cats`: its categorical splits (EvalWalkArgs::cat_span, categories).
    struct EvalCats {
        std::vector<uint32_t> span;
        const std::vector<uint32_t> *categories = nullptr;
    };
    void walk_evals(const std::vector<GrowTreeNode> &nodes, uint32_t output,
                    const std::vector<float> *cond = nullptr, const EvalCats *cats = nullptr);
    // ... into one set's margins only (a set added after trees were grown).
    void walk_evals_one(uint32_t set, const std::vector<GrowTreeNode> &nodes, uint32_t output,
                        const EvalCats *cats = nullptr);
    uint32_t n_eval_sets() const { return (uint32_t)evals_.size(); }
    // Drops every set; returns the new owner's number (eval_owner()).
    uint64_t clear_eval_sets() {
        evals_.clear();
        return ++eval_owner_;
    }
    uint64_t eval_owner() const { return eval_owner_; }
    uint64_t eval_rows(uint32_t set) const;
    void read_eval_margins(uint32_t set, float *out);
    // HistogramBackend::build of a host row list (per-node host growth).
    std::vector<QBin> build_rows(const uint32_t *rows, uint64_t m);
    // The same over a device row list into a device output (2 x total_bins
    // f64, g and h interleaved), with every intermediate buffer (the tile
    // plan, tile partials, the node record, a row-check word) inside
    // `scratch` (`bytes` of device memory the caller keeps): nothing is
    // allocated. Refuses an index whose tile partials cannot fit; returns
    // false when a row id is beyond the index (the output then holds zeros).
    bool build_rows_fixed(const uint32_t *rows, uint64_t m, double *out, uint8_t *scratch, uint64_t bytes);
    std::vector<uint32_t> rows_of(const Segment &s);
    std::vector<QBin> read_slot(uint32_t slot);

    // ---- histogram slots ------------------------------------------------------
    uint32_t alloc_slot();
    void free_slot(uint32_t s);
    bool reserve_slots(uint64_t n);

    // scan regularization and monotone directions for the next scans
    void set_scan_params(const ScanParams &p, const std::vector<int8_t> &monotone);

    hbr_engine_counters counters{};
    // ---- the fixed-point guard and exact-order replays ---------------------------
    // The guard bounds every candidate's score error and flags the nodes it
    // cannot certify (kScanNearTie); gamma is the caller's split threshold.
    enum GuardMode { kGuardOff = 0, kGuardReplay = 1, kGuardResolve = 2 };
    int guard_mode = kGuardResolve;  // near ties: reported for a host replay, or resolved on the device
    bool guard_on() const { return guard_mode != kGuardOff; }
    float guard_gamma = 0.0f;
    bool guard_active = false;  // the next scans bound their candidates
    // How each histogram slot of the current tree came about through the row
    // engine's calls: built from a segment's rows, then (a sibling kept in
    // its parent's slot) minus the built children's sums, in order.
    void note_built(const std::vector<Segment> &segs, const std::vector<uint32_t> &slots);
    void note_siblings(const std::vector<uint32_t> &parents, const std::vector<uint32_t> &built);
    uint32_t slot_rows(uint32_t slot) const;  // the node's row count (0: unknown)
    // The histogram of `slot` as the reference's CPU builder has it: each
    // built node's bins summed in the CPU build's own f64 order (each bin's
    // rows in row order from +0.0, in the blocks of sum_order;
    // tree/hist/mod.rs:399-607) and a sibling's as its parent's minus the
    // built child's (with_sibling, builder/partition.rs:244-256), computed
    // on the device from the staged pairs; false when the slot's history is
    // unknown or the index is not row-major u8 (out: 2 x total_bins, g and
    // h interleaved).
    bool exact_hist(uint32_t slot, double *out);
    // A near tie's node searched on those sums on the device (hbr_scan_exact):
    // the CPU builder's winner, with its children in f64 and in fixed point;
    // false when the slot's sums are not available (see exact_hist).
    bool resolve_exact(uint32_t slot, double total_g, double total_h, QBin total_fixed, float lower, float upper,
                       ExactBest *out);
    // algorithmic bytes of summing `rows` rows into a histogram
    uint64_t hist_bytes(uint64_t rows, bool gathered) const;

private:
    void upload_index(const hbr_index_desc &desc);
    void bin_dense(const DenseSource &src);
    void read_tunables();
    const char *dense8_kernel(uint32_t fg) const;
    uint64_t entries_ = 0;
    bool csr_ascending_ = true;  // every CSR row's global bins ascend (device binning writes them so)
    void build_csr_ranges();
    DBuf<uint32_t> csr_ranges_;  // each CSR row's first entry of every histogram bin range
    void ensure_rows();
    bool contiguous(const Segment &sg) const;
    struct SlotHistory {
        bool known = false;
        Segment built;               // the segment first summed into the slot
        std::vector<Segment> minus;  // then subtracted from it, in order
        uint32_t rows = 0;
    };
    std::vector<SlotHistory> slot_history_;
    void exact_segment(const Segment &sg, double *out_dev);  // one node's CPU-order sums into out_dev
    bool exact_hist_dev(uint32_t slot);                       // the slot's CPU-order sums into d_exact_out_
    DBuf<ExactBest> d_exact_best_;
    DBuf<double> d_exact_;
    DBuf<double> d_exact_out_;
    DBuf<double> d_exact_minus_;
    bool identity_rows0_ = false;
    bool rows0_written_ = false;
    void write_identity_rows();  // buffer 0 := 0..n-1, once per tree, when a row list is read
    // `n` nodes (the most a device-grown level can hold, with `grow`);
    // host_nodes: their slots are zeroed first (CSR)
    void launch_hist(const HistNode *nodes_dev, uint32_t n, const std::vector<HistNode> *host_nodes,
                     const PartSplit *splits_dev, const PartOut *part_out_dev, const uint32_t *rows0 = nullptr,
                     const GrowCounts *grow = nullptr);
    void launch_scan(const ScanNode *nodes_dev, uint32_t n, const PartSplit *splits_dev, const PartOut *part_out_dev,
                     ScanBest *best_dev, const GrowCounts *grow = nullptr, uint32_t *best_sets_dev = nullptr);
    // the root's total, histogram and split search, queued (no synchronisation)
    void launch_root(const Segment &seg, uint32_t slot, float lower, float upper);
    // the roots of a device-grown batch (root t in slot t, of class t,
    // unbounded) from records uploaded once per batch size
    void launch_device_roots(uint32_t n_trees);
    TreeTicket queue_device_forest(uint32_t n_trees, uint64_t max_depth, double gamma, float eta);
    DBuf<uint8_t> d_root_in_;
    uint32_t root_in_trees_ = 0;
    // a batched level's pairs (class-major), scales and root totals; null:
    // the staged pairs, the live scale, the root block's total
    const GPair *level_pairs_ = nullptr;
    QScale *level_scale_ = nullptr;
    QBin *level_totals_ = nullptr;
    DBuf<QBin> d_root_totals_;
    DBuf<uint32_t> d_tree_nodes_;
    // Device-grown trees in flight: each is written into a ring slot in
    // device memory and read back on a copy stream (the growth stream never
    // waits for a readback); pinned readbacks and their events. The guarded
    // walk's saved scale and skip flag.
    static constexpr uint32_t kTreeRing = 3;
    size_t ring_slot_bytes_ = 0;  // a ring slot holds a batch: its trees `stride` bytes apart
    size_t last_stride_ = 0;
    DBuf<uint8_t> d_tree_ring_;
    PinnedBuf tree_stage_[kTreeRing];
    hipEvent_t tree_ready_[kTreeRing] = {};
    hipEvent_t tree_copied_[kTreeRing] = {};
    bool ring_used_[kTreeRing] = {};
    hipStream_t copy_stream_ = nullptr;
    uint32_t tree_seq_ = 0, last_ring_ = 0;
    TreeHeader *ring_header(uint32_t r, uint32_t tree, size_t stride) const {
        return reinterpret_cast<TreeHeader *>(d_tree_ring_.get() + r * ring_slot_bytes_ + tree * stride);
    }
    GrowTreeNode *ring_nodes(uint32_t r, uint32_t tree, size_t stride) const {
        return reinterpret_cast<GrowTreeNode *>(d_tree_ring_.get() + r * ring_slot_bytes_ + tree * stride +
                                                kTreeHeaderBytes);
    }
    uint32_t last_depth_ = 0;  // max_depth of the last queued device tree
    DBuf<QScale> guard_scale_;
    DBuf<uint32_t> poison_;
    std::vector<int8_t> monotone_host_;
    PartArgs part_args() const;
    void scan_host_nodes(const std::vector<ScanNode> &nodes, ScanBest *out, uint32_t *sets = nullptr);
    void launch_gradients(const hbr_device_loss &loss, uint32_t output);
    GradArgs grad_args(const hbr_device_loss &loss);
    // bounds: the pair bounds' f32 bits (0: none), whose exponents replace
    // smaller maxima'
    bool check_scale(QScale folded, uint32_t bound_g_bits = 0, uint32_t bound_h_bits = 0);
    const uint64_t *expf_table_dev();  // the expf restatement's table, uploaded once
    bool scale_checked_ = true;  // the host has seen the scale of the staged gradients

    Device &dev_;
    uint64_t n_rows_ = 0;
    uint32_t n_cols_ = 0, total_bins_ = 0;
    bool dense_ = false;      // reference's is_dense: complete rows
    bool have_cols_ = false;  // feature-major local columns for routing
    bool dense_u8_ = false;   // row-major u8 local bins for the dense histogram
    uint32_t stride_ = 0;     // row-major stride in bytes
    uint32_t words_ = 0;      // bitmap words per feature
    std::vector<uint32_t> fo_;
    std::vector<float> cuts_;
    DBuf<uint32_t> d_fo_;
    DBuf<uint8_t> rows8_, cols8_;
    DBuf<uint16_t> cols16_;
    DBuf<uint64_t> missing_, row_ptr_;
    DBuf<uint32_t> gbins_;

    // training state
    DBuf<GPair> gpair_;
    // softmax: every class's pairs ([class][row]) and scales; the selected
    // class's pairs stand in for gpair_ while active_pairs_ is set
    DBuf<GPair> class_pairs_;
    DBuf<QScale> class_scales_;
    DBuf<uint64_t> exp_table_;
    uint32_t class_outputs_ = 0;
    GPair *active_pairs_ = nullptr;
    GPair *pairs() const { return active_pairs_ ? active_pairs_ : gpair_.get(); }
    bool pairs_staged() const { return active_pairs_ || (gpair_.size() >= n_rows_ && gpair_.get()); }
    DBuf<float> margins_, labels_, weights_;
    // the reorder: position -> original row, and its inverse; the marks of
    // the original 8-row vectors a fused walk found outside the vector
    // range (GradArgs::perm)
    bool permuted_ = false;
    DBuf<uint32_t> perm_, perm_inv_, group_stamp_, bad_groups_;
    uint32_t regroup_stamp_ = 0;
    uint32_t root_regroup_tile_ = 0;  // the fused root's partials include hbr_regroup's
    // what a reorder gathers into, swapped with the live arrays (nothing is
    // freed while kernels may still read it), and the reorder's scratch
    struct Spare {
        DBuf<uint8_t> rows, cols;
        DBuf<float> margins, labels, weights;
        DBuf<GPair> pairs;
        DBuf<uint32_t> leaf, order, count, cursor;
    };
    Spare spare_;
    void gather_rows(const uint32_t *index);
    struct EvalSet {
        DBuf<float> x, margins;
        uint64_t n_rows = 0;
        uint32_t outputs = 1;
        float missing = 0.0f;
    };
    std::vector<std::unique_ptr<EvalSet>> evals_;
    uint64_t eval_owner_ = 0;  // bumped whenever the sets are dropped
    DBuf<float> d_cuts_;             // cut values for the evaluation walks
    DBuf<GrowTreeNode> d_eval_tree_; // a host-grown tree's records
    DBuf<float> d_eval_cond_;
    DBuf<uint32_t> d_eval_span_, d_eval_categories_;  // a walked tree's categorical splits
    void upload_eval_cats(const EvalCats &cats, size_t n_nodes);
    void launch_eval_walk(const EvalSet &set, const GrowTreeNode *tree, const GrowCounts *counts, uint32_t n_nodes,
                          uint32_t output, const uint32_t *poison, const float *cond = nullptr,
                          const EvalCats *cats = nullptr);
    uint32_t outputs_ = 1;
    bool labels_loaded_ = false, has_weights_ = false;
    bool labels_binary_ = false;  // every label 0 or 1
    // the staged pairs are the logistic pairs the rows carry (GradArgs::pair_rows)
    bool row_pairs_live_ = false;
    float row_pairs_min_hess_ = 0.0f;
    bool row_pairs_ok(const hbr_device_loss &loss) const;
    // The unit-weight logistic loss (no weights, scale_pos_weight 1, labels
    // 0 or 1) bounds its pairs, |g| <= 1 and h <= 1/4: the exponents are the
    // bounds', known before the pairs are (FinishArgs::bound_*).
    bool bounded_logistic(const hbr_device_loss &loss) const;
    void set_bounds(const hbr_device_loss &loss, FinishArgs &f) const;
    // Dense u8 rows with a missing mask (kMaskWord) of a matrix with missing
    // values (dense_ false, dense_u8_ true).
    bool masked_ = false;
    uint32_t mask_at_ = 0;  // masked rows: the byte of a row's first mask word
    // A dense index with a feature of more than 256 bins (at most
    // kWideBinsMax): rows of u16 local bins for the histograms (the CSR
    // rows and columns serve the rest), fg16_ features per workgroup.
    bool dense16_ = false;
    DBuf<uint16_t> rows16_;
    uint32_t stride16_ = 0, fg16_ = 0;
    void make_rows16(uint32_t widest);
    void make_masked_rows();
    // Partials of the next root's histogram the fused walk left (0: none);
    // the next device tree's root sums them instead of building its own.
    uint32_t root_partials_ = 0;
    // The fused walk wrote its pairs into the rows only (the pair array is
    // stale until the next gradients are staged some other way).
    bool pair_array_stale_ = false;
    // the per-tree scale, the root total and the root's winner, adjacent so
    // that the root's synchronisation reads them back with one copy
    struct RootBlock {
        QScale scale;
        QBin total;
        ScanBest best;
    };
    // followed by the level counts of the device-grown tree being grown
    DBuf<uint8_t> block_;
    static constexpr size_t kCountsAt = (sizeof(RootBlock) + 63) / 64 * 64;
    static constexpr size_t kBlockBytes = kCountsAt + (sizeof(GrowCounts) + 63) / 64 * 64;
    static constexpr size_t kMaxDeviceNodes = (size_t(2) << kMaxDeviceDepth) - 1;
    RootBlock *root_block() const { return reinterpret_cast<RootBlock *>(block_.get()); }
    QScale *scale_dev() const { return &root_block()->scale; }
    QBin *total_dev() const { return &root_block()->total; }
    ScanBest *root_best_dev() const { return &root_block()->best; }
    GrowCounts *grow_counts_dev() const { return reinterpret_cast<GrowCounts *>(block_.get() + kCountsAt); }
    // device-grown levels: frontiers, splits and partition results, two of each
    DBuf<GrowNode> g_front_[2];
    DBuf<PartSplit> g_splits_[2];
    DBuf<PartOut> g_pout_[2];
    QScale scale_host_{};
    bool grains_known_ = false;  // scale_host_.pad holds the staged pairs' grain codes
    DBuf<uint32_t> scalar_list_;  // rows the fused walk defers to hbr_finish_scale
    DBuf<uint32_t> rows_[2];
    DBuf<uint32_t> host_rows_;
    uint64_t tree_ = 0;

    // histogram slots
    DBuf<QBin> hist_;
    uint32_t slot_cap_ = 0;
    std::vector<uint32_t> free_slots_;

    // scan configuration
    ScanParams scan_params_{1.0, 0.0, 0.0, 1.0};
    DBuf<int8_t> monotone_;
    bool has_monotone_ = false;

    // per-call scratch
    Stage stage_;
    DBuf<PartSplit> d_splits_;
    DBuf<uint32_t> d_tile_left_, d_tile_split_;
    DBuf<uint8_t> d_level_in_, d_level_out_;  // one level's records (bytes)
    DBuf<HistNode> d_hnodes_;
    DBuf<HistTile> d_htiles_;
    DBuf<uint32_t> d_hcounts_;
    DBuf<QBin> d_partial_;
    DBuf<uint64_t> d_decisions_;
    DBuf<uint8_t> d_walk_;  // a tree's meta, left and value tables, one after another
    DBuf<ScanNode> d_snodes_;
    DBuf<ScanBest> d_per_feature_, d_best_;
    // categorical features: rank per feature, feature per rank, their
    // per-(node, feature) sets and the root's winning set
    uint32_t n_cat_ = 0;
    std::vector<uint32_t> cat_rank_, cat_feature_;
    DBuf<uint32_t> d_cat_rank_, d_cat_feature_, d_cat_sets_, d_root_set_, d_scan_sets_;
    DBuf<LeafSeg> d_leaves_;
    DBuf<uint32_t> d_tile_leaf_, d_tile_row0_;

public:
    // histogram launch shape: features per workgroup (8, 16 or 32), threads
    // per dense workgroup (512 or 1024) and resident waves of workgroups the
    // plan sizes a launch for
    uint32_t hist_features_per_group = 32;
    uint32_t hist_threads = 1024;
    uint32_t hist_waves = 1;
    bool hist_bin_major = true;  // [bin][feature] LDS layout (16 and 32 feature groups)
    bool hist_nf28 = true;       // 25-28 features: the lanes rotate over the features alone (no padding atomics)
    bool row_pairs = true;       // unit-weight logistic pairs carried in the rows' padding
    bool fused_root = true;      // the margin walk also sums the next root's histogram (row pairs)
    bool masked_rows = true;     // dense u8 rows with a missing mask for matrices with missing values
    bool wide_rows = true;       // dense u16 rows for the histograms of features of more than 256 bins
    bool row_order = true;       // the whole-round trainer reorders 32-byte rows by its first tree's leaves
    uint64_t row_order_min_rows = 1u << 20;  // ... of at least this many rows (smaller ones stay in the caches)
    uint64_t row_order_every = 0;            // ... and again every this many rounds (0: once)
    bool batch_walk = true;  // a softmax round's class trees added to the margins in one walk
    bool bin_rows_in_registers = true;  // device binning of <= 32 features: rows into registers, else staged in LDS
    bool device_grow = true;     // depthwise trees decided on the device where eligible
    bool csr_range_table = true; // CSR histograms read each bin range's entries from a per-row table
    uint32_t walk_blocks_per_cu = 4;  // workgroups per CU of the device-tree margin walk (one resident wave)
};

}  // namespace hbr
