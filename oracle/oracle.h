/*
 * CPU oracle for the hessboost hist path — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of hessboost v0.4.9's CPU `tree_method=hist`
 * training and batch prediction, used as the checker for the MI355X
 * backend. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product never does.
 *
 * What each part restates (reference file:line):
 *   sketch.c    data/sketch.rs:59-680 (WQSketch), data/quantile.rs:65-296
 *   index.c     data/ghist.rs:213-257, :930-1032 (GHistIndex)
 *   hist.c      tree/hist/mod.rs:399-607 (sum_order, CpuBackend::build),
 *               tree/builder/shared.rs:164-170 (sum_rows)
 *   split.c     tree/builder/split.rs:37-141, :391-419; builder/mod.rs:167-342;
 *               builder/shared.rs:89-141; tree/gain.rs:82-116;
 *               tree/constraints.rs
 *   grow.c      tree/builder/hist/mod.rs:261-737 (depthwise, lossguide),
 *               builder/partition.rs:106-313, shared.rs:174-187
 *   objective.c objective/regression.rs:42-58, simd/x86_64.rs:22-160,
 *               simd/scalar.rs:8-29, simd/mod.rs:425-600,
 *               objective/classification.rs:66-141, objective/mod.rs:645-666
 *   predict.c   model/predict.rs:60-193, tree/regtree.rs:38-66, tree/mod.rs:52-58
 *   train.c     training/round.rs:214-424, training/margins.rs:129-289,
 *               training/train.rs:406-436
 *
 * Pins (tests/test_oracle.py): the reference's saved early-stopping model is
 * retrained bit for bit (sketch, index, hist, split, depthwise grow,
 * squared error, train, predict); nine saved models' margins are reproduced
 * bit for bit (predict); the reference's KATs pin the gains, the separating
 * split and the blocked-sum order; closed forms pin cuts of few distinct
 * values, bin assignment, partition routing, both logistic paths, softmax
 * (to 1e-6) and the intercepts; the reference's own softmax tests
 * (simd/tests.rs:133-285) pin the 2- and 4-class vector batches to the
 * scalar rows (1e-6, and bit for bit on underflowing rows).
 *
 * The sketch's prune/merge on data with more distinct values than max_bin
 * is pinned by brute-force rank bounds on every summary it forms, by
 * XGBoost's per-query SetPrune and three-case SetCombine as other
 * formulations, and by the summary budget's definition
 * (tests/test_sketch.py, through the or_summary_* and or_sketch_trace
 * hooks below). The lossguide order under equal gains is pinned by a brute
 * force over its queue events and by Rust's BinaryHeap algorithm
 * (tests/test_oracle.py, through or_lossguide_trace).
 *
 * Parity unpinned (nothing the reference holds reaches them):
 *   - softmax gradients bit for bit: the scalar rows call the host libm
 *     expf, as the reference's f32::exp does, so bits match only for the
 *     same libm; the 2- and 4-class vector batches follow the reference's
 *     intrinsic sequence, pinned to 1e-6 only;
 *   - the sketch's queue order with fractional weights (the reference's
 *     unstable sort; whole-number weights sum exactly in any order).
 */
#ifndef HB_ORACLE_H
#define HB_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- cuts (HistCuts) ---------------------------------------------------- */
typedef struct or_cuts {
    size_t n_features;
    uint32_t *feature_offset; /* n_features + 1 */
    float *cut_values;        /* feature_offset[n_features] values */
    uint8_t *is_categorical;  /* per feature, or NULL (every feature numeric) */
} or_cuts;

/* The most bins (distinct categories) of a categorical feature. */
#define OR_MAX_CAT_BINS 1024

/* Dense f32 matrix (row-major, n x f) with `missing` marking absent cells
 * (NaN matches any NaN). weights may be NULL (unit weights). */
or_cuts *or_cuts_from_dense(const float *x, size_t n, size_t f, size_t max_bin,
                            const float *weights, float missing);
/* CSR matrix: row_ptr[n+1], col[nnz], val[nnz]; every stored entry present. */
or_cuts *or_cuts_from_csr(const size_t *row_ptr, const uint32_t *col,
                          const float *val, size_t n, size_t f, size_t max_bin,
                          const float *weights);
/* The same with per-feature types (categorical != 0: one bin per distinct
 * present value, quantile.rs:524-672; NULL: every feature numeric). */
or_cuts *or_cuts_from_dense_typed(const float *x, size_t n, size_t f, size_t max_bin,
                                  const float *weights, float missing, const uint8_t *categorical);
or_cuts *or_cuts_from_csr_typed(const size_t *row_ptr, const uint32_t *col,
                                const float *val, size_t n, size_t f, size_t max_bin,
                                const float *weights, const uint8_t *categorical);
void or_cuts_free(or_cuts *c);
size_t or_cuts_total_bins(const or_cuts *c);
/* Global bin of value v (present) for feature f: #{cuts <= v}, clamped; a
 * categorical feature's bin holding v exactly, else its first bin
 * (quantile.rs:285-296). */
uint32_t or_bin_of(const or_cuts *c, size_t f, float v);

/* Test hooks of the sketch: summaries as 4 floats per entry (rmin, rmax,
 * wmin, value). */
size_t or_summary_budget(size_t max_bin, size_t n);
size_t or_summary_from_sorted(const float *v, const float *w, size_t n, float *out);
size_t or_summary_prune(float *entries, size_t n, size_t maxsize);
size_t or_summary_combine(const float *a, size_t na, const float *b, size_t nb, float *out);
size_t or_summary_query(const float *entries, size_t n, size_t max_bin, float *out);
/* Test hook: record the loss-guided queue's events of the next trees grown
 * on this thread into buf (4 u64 per event: kind 0 push / 1 pop, node id,
 * loss_chg bits, expandable), at most cap events; buf NULL stops. */
void or_lossguide_trace(uint64_t *buf, size_t cap);
size_t or_lossguide_trace_len(void);
long or_sketch_trace(const float *values, const float *weights, size_t n, size_t max_bin, float *buf,
                     size_t buf_entries, uint64_t *recs, size_t rec_cap, size_t *n_recs, float *cuts);

/* ---- binned index (GHistIndex) ------------------------------------------ */
typedef struct or_index {
    size_t n_rows, n_cols;
    size_t *row_ptr;       /* n_rows + 1 */
    int row_width;         /* 2: u16 global bins, 4: u32 */
    void *rows;            /* CSR global bins */
    int col_width;         /* 0: no columns, else 1/2/4 bytes local bins */
    void *cols;            /* feature-major local bins [f][r] */
    uint64_t *missing;     /* per-feature bitmap (words per feature = ceil(n/64)) or NULL */
    int dense;             /* every row holds every feature in feature order */
    or_cuts *cuts;         /* borrowed */
} or_index;

or_index *or_index_from_dense(const float *x, size_t n, size_t f, float missing,
                              or_cuts *cuts);
or_index *or_index_from_csr(const size_t *row_ptr, const uint32_t *col,
                            const float *val, size_t n, size_t f, or_cuts *cuts);
void or_index_free(or_index *ix);
/* The global bin of (r, f), or -1 when missing. */
int64_t or_index_feature_bin(const or_index *ix, size_t r, size_t f);

/* ---- histograms ---------------------------------------------------------- */
/* gpair: interleaved (g, h) f32 per row of the index. out: 2*total_bins f64
 * (g, h interleaved), overwritten. */
void or_build_hist(const or_index *ix, const uint32_t *rows, size_t m,
                   const float *gpair, double *out);
/* sum_rows: one row-order f64 chain. out[2]. */
void or_sum_rows(const float *gpair, const uint32_t *rows, size_t m, double *out);
/* Rows per block of the Blocked order for a node of `len` rows on the index
 * (0 when the node sums as one Chain). */
size_t or_sum_order_grain(int dense, size_t index_rows, size_t len, int contiguous);

/* ---- training parameters ------------------------------------------------ */
/* OR_OBJ_LOGITRAW: binary:logitraw, the logistic loss with the identity link
   (src/objective/classification.rs:55-72). */
enum { OR_OBJ_SQUARED_ERROR = 0, OR_OBJ_LOGISTIC = 1, OR_OBJ_SOFTMAX = 2, OR_OBJ_LOGITRAW = 3 };
enum { OR_GROW_DEPTHWISE = 0, OR_GROW_LOSSGUIDE = 1 };

typedef struct or_params {
    double eta, gamma, lambda, alpha, min_child_weight, max_delta_step;
    int64_t max_depth;    /* <= 0: unbounded */
    int64_t max_leaves;   /* <= 0: unbounded */
    int grow_policy;
    int objective;
    int num_class;        /* softmax only */
    float scale_pos_weight;
    const int8_t *monotone; /* per feature, or NULL */
    size_t n_monotone;
    int64_t max_bin;
    float base_score;     /* used when has_base_score */
    int has_base_score;
} or_params;

/* ---- split search -------------------------------------------------------- */
typedef struct or_split {
    double loss_chg;      /* an f32 value widened */
    uint32_t feature;
    int64_t bin;          /* global bin boundary (bins <= bin go left), -1: BelowBins */
    int default_left;
    double left_g, left_h, right_g, right_h;
    double w_left, w_right;
    /* a categorical split (builder/categorical.rs:48-170): the local bins
     * whose categories go left (the set XGBoost routes to its right child,
     * recorded as the tree's left child); bin is then -1 */
    int categorical;
    uint32_t cat_left[OR_MAX_CAT_BINS / 32];
} or_split;

/* Sequential hist split search over every feature of the node. */
void or_evaluate(const or_index *ix, const double *hist, double total_g,
                 double total_h, double lower, double upper,
                 const or_params *p, or_split *out);
int or_split_valid(const or_split *s, const or_params *p);
float or_node_gain(double g, double h, double lower, double upper, const or_params *p);
/* tree/gain.rs:107-116 calc_weight (0 below min_child_weight). */
double or_calc_weight(double g, double h, const or_params *p);
/* sweep_categorical (builder/categorical.rs:48-170) of one feature's n
 * categories (ascending codes, stats[2i], stats[2i+1] = G, H, zero for a
 * category the node lacks) against the node total, merged into *best with
 * the tie rule; a winning set lands in best->cat_left by position. */
void or_sweep_categorical(const double *stats, size_t n, double total_g, double total_h, double lower,
                          double upper, int dir, const or_params *p, uint32_t feature, or_split *best);

/* ---- partition ------------------------------------------------------------ */
/* Stable partition of rows[m] on (feature, bin, default_left). Returns the
 * left count; left rows first in `out_left`, right rows in `out_right`. */
size_t or_partition(const or_index *ix, const uint32_t *rows, size_t m,
                    uint32_t feature, int64_t bin, int default_left,
                    uint32_t *out_left, uint32_t *out_right);
/* The same for a categorical split (partition.rs:146-160): a present row
 * goes left when its local bin's bit is set in cat_left. */
size_t or_partition_categorical(const or_index *ix, const uint32_t *rows, size_t m, uint32_t feature,
                                const uint32_t *cat_left, int default_left, uint32_t *out_left,
                                uint32_t *out_right);

/* ---- trees ------------------------------------------------------------------ */
typedef struct or_node {
    uint32_t split_feature;
    float split_cond;
    int32_t default_left;
    int32_t left, right;
    float leaf_value, sum_hess, split_gain;
    /* diagnostics (not part of the model format) */
    int64_t split_bin;     /* global bin, -1 BelowBins, -2 leaf */
    double stat_g, stat_h; /* node statistics the builder stored */
    /* categorical splits: the node's categories (going left) are
     * categories[cat_begin, cat_end) of its tree (regtree.rs:59-66) */
    int32_t is_categorical;
    uint32_t cat_begin, cat_end;
} or_node;

typedef struct or_tree {
    or_node *nodes;
    size_t n_nodes, cap;
    uint32_t *categories;
    size_t n_categories, cat_cap;
} or_tree;

/* Grow one tree over all rows of the index from gpair; leaves scaled by
 * eta (training's tree_eta). leaf_of_row (n_rows, may be NULL) receives each
 * row's leaf node id. */
or_tree *or_grow_tree(const or_index *ix, const float *gpair, const or_params *p,
                      int32_t *leaf_of_row);
void or_tree_free(or_tree *t);
size_t or_tree_n_nodes(const or_tree *t);
size_t or_tree_n_categories(const or_tree *t);
const uint32_t *or_tree_categories(const or_tree *t);
const or_node *or_tree_nodes(const or_tree *t);

/* ---- objectives ------------------------------------------------------------- */
/* preds/labels/weights (weights may be NULL) of n rows; out: 2n floats. */
void or_gradient_squared_error(const float *preds, const float *labels,
                               const float *weights, size_t n, float spw, float *out);
void or_gradient_logistic(const float *preds, const float *labels,
                          const float *weights, size_t n, float spw, float *out);
/* preds n*k row-major; out n*k pairs row-major [row][class]. */
void or_gradient_softmax(const float *preds, const float *labels,
                         const float *weights, size_t n, size_t k, float *out);
/* The same with every row on the scalar path (simd/mod.rs:536-555). */
void or_gradient_softmax_scalar(const float *preds, const float *labels,
                                const float *weights, size_t n, size_t k, float *out);
float or_sigmoid(float x);
/* Per-output intercepts (base margins). out[k]. */
void or_base_margins(const float *labels, const float *weights, size_t n,
                     const or_params *p, float *out);

/* ---- prediction ----------------------------------------------------------- */
typedef struct or_forest_desc {
    size_t n_trees;
    const uint32_t *tree_offset;   /* n_trees + 1 node offsets into the arrays */
    const uint32_t *split_feature;
    const float *split_cond;
    const uint8_t *default_left;
    const int32_t *left, *right;
    const float *leaf_value;
    const float *tree_weight;      /* n_trees */
    const uint32_t *tree_output;   /* n_trees */
    size_t n_outputs;
    const float *base_score;       /* n_outputs */
    /* categorical splits (NULL: every split numeric): node i's categories
     * routed left are categories[cat_begin[i], cat_end[i]) */
    const uint8_t *is_categorical;
    const uint32_t *cat_begin, *cat_end;
    const uint32_t *categories;
} or_forest_desc;

/* margins out[n * n_outputs]; leaf ids (per tree, may be NULL) out_leaf[n * n_trees]. */
void or_predict_margin(const or_forest_desc *fd, const float *x, size_t n,
                       size_t n_cols, float missing, float *out, int32_t *out_leaf);
/* The same margins (NaN missing, numeric splits) by the reference's 16-row
 * lock-step walk over a breadth-first key-compare arena; -1 for a forest it
 * does not take (categorical or non-finite splits, a feature >= n_cols). */
int or_predict_margin_lockstep(const or_forest_desc *fd, const float *x, size_t n,
                               size_t n_cols, float *out);

/* ---- training -------------------------------------------------------------- */
typedef struct or_model or_model;
or_model *or_train(const or_index *ix, const float *labels, const float *weights,
                   const or_params *p, size_t rounds);
/* Continue an existing run by `rounds` more boosting iterations. */
void or_train_more(or_model *m, const float *labels, const float *weights,
                   const or_params *p, size_t rounds);
size_t or_model_n_trees(const or_model *m);
const or_tree *or_model_tree(const or_model *m, size_t i);
const float *or_model_margins(const or_model *m);
const float *or_model_base_score(const or_model *m);
size_t or_model_n_outputs(const or_model *m);
/* The gradients the last round grew its trees from (n * k pairs). */
const float *or_model_last_gpair(const or_model *m);
void or_model_free(or_model *m);

/* Worker threads for the parallel parts (0: OpenMP default). */
void or_set_threads(int n);

#ifdef __cplusplus
}
#endif
#endif
