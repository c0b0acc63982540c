/*
 * hessboost-rocm: the MI355X (gfx950) hist backend's C ABI.
 *
 * The drop-in boundary for hessboost's `tree_method=hist` path. A Rust
 * shim implements the reference's two backend traits over these calls:
 *
 *   HistogramBackend   src/tree/hist/mod.rs:73-105
 *   RowEngine          src/tree/hist/mod.rs:213-295
 *   GpuModel           src/backend/cuda/predict.rs:401-520 (BoostedModel::to_cuda)
 *
 * plus the index and cut construction the trainer runs once per dataset
 * (src/data/quantile.rs:65-78, src/data/ghist.rs:213-257) and a whole
 * device-resident boosting loop (src/training/round.rs:105-148).
 *
 * Conventions. Every call returns an int status:
 *   HBR_OK           the call ran;
 *   HBR_REFUSED      the device does not run this call for these inputs and
 *                    changed nothing: the caller does the work itself (the
 *                    traits' `None`);
 *   HBR_DEVICE_ERROR a HIP error: the handle is poisoned and refuses every
 *                    later call (the CUDA backend's sticky `failed` flag,
 *                    src/backend/cuda/mod.rs:1806-1826);
 *   HBR_INVALID      malformed arguments.
 * hbr_last_error() returns the calling thread's last message. All pointers
 * are host pointers unless a parameter says "device". Handles are safe to
 * use from several threads: each serializes behind its own mutex. No call
 * invokes the caller back.
 */
#ifndef HESSBOOST_ROCM_H
#define HESSBOOST_ROCM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HBR_OK 0
#define HBR_REFUSED 1
#define HBR_DEVICE_ERROR 2
#define HBR_INVALID 3

/* The calling thread's last error message (empty after success). Writes at
 * most len bytes including the terminator; returns the full length. */
size_t hbr_last_error(char *buf, size_t len);

/* Number of ROCm devices visible to the process. */
int hbr_device_count(int *count);

/* The name and architecture of device `ordinal` (for diagnostics, as the
 * Python GpuModel.device_name reports it, python/src/gpu.rs:196-203),
 * NUL-terminated and cut to len bytes. */
int hbr_device_name(int ordinal, char *buf, size_t len);

/* ------------------------------------------------------------------------- */
/* Cuts and binned index (host; once per dataset).                            */
/* ------------------------------------------------------------------------- */

typedef struct hbr_cuts hbr_cuts;
typedef struct hbr_index hbr_index;

/* HistCuts::from_dmatrix (src/data/quantile.rs:65-78): per-feature cuts from
 * XGBoost's weighted quantile sketch (src/data/sketch.rs:480-708) over a
 * dense row-major f32 matrix; cells equal to `missing` (any NaN when missing
 * is NaN) are absent. weights may be NULL. */
int hbr_cuts_from_dense(const float *x, uint64_t n_rows, uint64_t n_cols, uint32_t max_bin,
                        const float *weights, float missing, hbr_cuts **out);
/* The same over CSR storage (row_ptr[n_rows+1], col, val); every stored
 * entry is present. */
int hbr_cuts_from_csr(const uint64_t *row_ptr, const uint32_t *col, const float *val,
                      uint64_t n_rows, uint64_t n_cols, uint32_t max_bin, const float *weights,
                      hbr_cuts **out);
/* The same with feature types (the DMatrix's feature_types,
 * src/data/quantile.rs:120-131): categorical[f] != 0 makes feature f
 * categorical, one bin per distinct present value, ascending
 * (quantile.rs:524-689; bin_of: the bin holding the value exactly, else the
 * feature's first bin, :285-296). categorical may be NULL. */
int hbr_cuts_from_dense_typed(const float *x, uint64_t n_rows, uint64_t n_cols, uint32_t max_bin,
                              const float *weights, float missing, const uint8_t *categorical, hbr_cuts **out);
int hbr_cuts_from_csr_typed(const uint64_t *row_ptr, const uint32_t *col, const float *val, uint64_t n_rows,
                            uint64_t n_cols, uint32_t max_bin, const float *weights, const uint8_t *categorical,
                            hbr_cuts **out);
/* Per feature 1 when categorical (n_cols bytes). */
int hbr_cuts_categorical(const hbr_cuts *c, uint8_t *out);
/* Cuts given by the caller (feature_offset[n_cols+1], cut_values). */
int hbr_cuts_from_values(const uint32_t *feature_offset, const float *cut_values, uint64_t n_cols,
                         hbr_cuts **out);
int hbr_cuts_info(const hbr_cuts *c, uint64_t *n_cols, uint64_t *total_bins);
int hbr_cuts_copy(const hbr_cuts *c, uint32_t *feature_offset, float *cut_values);
void hbr_cuts_free(hbr_cuts *c);

/* GHistIndex::from_dmatrix (src/data/ghist.rs:213-257): global row bins
 * (u16 up to 65,536 bins, else u32), feature-major local columns when at
 * least half full (u8/u16/u32 by the widest feature) with a missing bitmap
 * when any cell is missing, and the `dense` flag. The index keeps its own
 * copy of the cuts. */
int hbr_index_from_dense(const float *x, uint64_t n_rows, uint64_t n_cols, float missing,
                         const hbr_cuts *cuts, hbr_index **out);
int hbr_index_from_csr(const uint64_t *row_ptr, const uint32_t *col, const float *val,
                       uint64_t n_rows, uint64_t n_cols, const hbr_cuts *cuts, hbr_index **out);
void hbr_index_free(hbr_index *ix);

/* A binned index as the reference's GHistIndex lays it out
 * (src/data/ghist.rs:195-209, :315-360). */
typedef struct hbr_index_desc {
    uint64_t n_rows;
    uint64_t n_cols;
    const uint32_t *feature_offset; /* n_cols + 1: feature f owns global bins [fo[f], fo[f+1]) */
    const float *cut_values;        /* fo[n_cols] cut values */
    const uint64_t *row_ptr;        /* n_rows + 1 */
    const void *row_bins;           /* row_ptr[n_rows] global bins */
    uint32_t row_bin_width;         /* 2 (u16) or 4 (u32) */
    uint32_t dense;                 /* every row holds every feature in feature order */
    const void *col_bins;           /* feature-major local bins [f][r], or NULL */
    uint32_t col_bin_width;         /* 1, 2 or 4 */
    uint32_t pad;
    const uint64_t *missing;        /* ceil(n_rows/64) words per feature, bit set = missing; or NULL */
    const uint8_t *is_categorical;  /* per feature (HistCuts::is_categorical), or NULL: every feature numeric */
} hbr_index_desc;

/* A read-only view of an index built by hbr_index_from_* (valid while it lives). */
int hbr_index_describe(const hbr_index *ix, hbr_index_desc *out);

/* ------------------------------------------------------------------------- */
/* The engine: HistogramBackend + RowEngine over one index on one device.    */
/* ------------------------------------------------------------------------- */

typedef struct hbr_engine hbr_engine;

/* CudaHistBackend::new(index, ordinal) (src/backend/cuda/mod.rs:1626-1671):
 * upload the index and re-encode it on the device. */
int hbr_engine_open(int ordinal, const hbr_index_desc *index, hbr_engine **out);
void hbr_engine_close(hbr_engine *e);

/* The engine over a dense f32 matrix binned on the device: the index
 * GHistIndex::from_dmatrix (src/data/ghist.rs:213-257) builds on the host,
 * with bins from HistCuts::bin_of (src/data/quantile.rs:285-296) against
 * `cuts`, computed by the GPU. x is row-major n_rows x n_cols, in host memory
 * or (x_on_device) in this ordinal's device memory; cells equal to `missing`
 * (any NaN when it is NaN) are absent. Refused when a feature has more than
 * 256 bins. The layouts equal hbr_index_from_dense's byte for byte. */
int hbr_engine_open_dense(int ordinal, const float *x, uint64_t n_rows, uint64_t n_cols, float missing,
                          const hbr_cuts *cuts, int x_on_device, hbr_engine **out);

/* The engine's index as it sits on the device, for checking a build
 * (no reference counterpart: the reference reads GHistIndex fields).
 * dense: every row holds every feature; dense_u8: row-major u8 rows of
 * `stride` bytes are kept; has_cols/has_missing: local columns and the
 * missing bitmap are kept; entries: stored cells. */
typedef struct hbr_index_info {
    uint32_t dense, dense_u8, has_cols, has_missing;
    uint32_t stride, pad;
    uint64_t entries;
} hbr_index_info;
int hbr_engine_index_info(hbr_engine *e, hbr_index_info *out);
/* Copies of the layouts (NULL skips one): rows8 n_rows x stride (dense u8),
 * cols8 n_cols x n_rows (u8 columns), missing n_cols x ceil(n_rows/64),
 * row_ptr n_rows + 1 and gbins (u32 global bins, entries) of a CSR index. */
int hbr_engine_index_read(hbr_engine *e, uint8_t *rows8, uint8_t *cols8, uint64_t *missing, uint64_t *row_ptr,
                          uint32_t *gbins);

/* The sums hbr_build, hbr_build_device_noalloc, hbr_histograms,
 * hbr_root_total[_fixed], hbr_scan_resident and hbr_read_hist return.
 * The trait promises the CPU's f64 bits (src/tree/hist/mod.rs:205-207,
 * :220-224). The engine sums the staged pairs in fixed point: integers in a
 * per-tree unit of 2^e, exact and order-free. Inside the reference's exact
 * domain (src/backend/exact_sum.rs:14-37: every pair finite, n x max <=
 * 2^53 grains of its component, with the unit at or below the grain) those
 * sums are the CPU's f64 sums bit for bit, in any order. Outside it they
 * differ from the CPU's row-order f64 chain by that chain's own rounding
 * (relative error about n x 2^-53).
 *   HBR_SUMS_EXACT (the default): those calls return HBR_REFUSED outside
 *     the exact domain, as the CUDA backend refuses or falls back there
 *     (src/backend/cuda/mod.rs:2758-2776); the caller sums on the host.
 *   HBR_SUMS_FIXED_POINT: they return the fixed-point sums everywhere (a
 *     tolerance of the chain's rounding; split choices can differ from the
 *     CPU's on near-ties).
 * The exact domain is known for pairs staged by hbr_prepare and by
 * hbr_gradients; after other staging (softmax classes, the trainer's
 * rounds) it is treated as not exact. */
#define HBR_SUMS_EXACT 0
#define HBR_SUMS_FIXED_POINT 1
int hbr_engine_set_sums(hbr_engine *e, int mode);

/* HistogramBackend::prepare (src/tree/hist/mod.rs:96): stage a tree's
 * gradient pairs (interleaved g, h f32; one per index row). */
int hbr_prepare(hbr_engine *e, const float *gpair, uint64_t n);

/* HistogramBackend::build (src/tree/hist/mod.rs:76): the histogram of
 * `rows` (ascending, distinct) from the staged gradients; out holds
 * 2 * total_bins f64 (g, h interleaved), overwritten. Each bin is the exact
 * sum of its rows' fixed-point gradients, converted to f64. */
int hbr_build(hbr_engine *e, const uint32_t *rows, uint64_t m, double *out);

/* No counterpart in the reference: hbr_build for callers that cannot
 * allocate device memory (tight serving loops, harnesses that forbid
 * hipMalloc). It synchronises the engine's stream before it returns, so it
 * is not for code under HIP graph capture. rows (m ids, device memory) and
 * out (2 * total_bins f64, device memory) are the caller's; the tile plan,
 * the tiles' partial sums, the node record and a row-check word live in one
 * fixed scratch array of the library per device (32 MiB + 128 KiB, held
 * from the first call on a device until the process ends), so the call
 * allocates nothing and returns with out complete. Bins equal hbr_build's
 * for the same rows bit for bit. HBR_INVALID when a row id is at or beyond
 * the index's rows (out then holds zeros), when m >= 2^32 - 1, or when one
 * row tile's partial sums exceed the scratch (more than 8,192 features of a
 * dense u8 index, or more than 2,097,152 bins of a CSR index). Every call
 * on one GPU shares that GPU's scratch and holds a per-GPU lock for its
 * whole duration, so calls from several threads (two engines on one GPU)
 * run one after another. HBR_REFUSED when the last gradient pass left the
 * pairs in the rows only and the index's kernel cannot read them there, and
 * while a trainer holds the engine's rows in a tree's leaf order (any other
 * engine call puts them back, which may allocate). */
int hbr_build_device_noalloc(hbr_engine *e, const uint32_t *rows, uint64_t m, double *out);

/* A node's rows on the device (the reference's Segment, src/tree/hist/mod.rs:107-164):
 * issued by the engine, stamped with its tree. */
typedef struct hbr_segment {
    uint64_t offset;
    uint64_t len;
    uint32_t buffer;
    uint32_t contiguous;
    uint64_t tree;
} hbr_segment;

/* RowEngine::begin_tree: every index row (in order) as the root segment.
 * The reference's `rows` argument is the full ascending row list of an
 * unsampled tree; other row lists are refused. */
int hbr_begin_tree(hbr_engine *e, uint64_t n_rows, hbr_segment *root);

/* RowEngine::root_total: the segment's statistics (f64 of the exact
 * fixed-point sums). */
int hbr_root_total(hbr_engine *e, const hbr_segment *seg, double out[2]);

/* One split to partition (RowRule, RowSplit: src/tree/hist/mod.rs:166-192): a
 * present value goes left by its feature-local bin, as RowRule::Below
 * (table NULL: bins below `below` go left) or RowRule::Table (table[bin] !=
 * 0 goes left; n_table = the feature's bin count, at most 1,024, and the
 * feature categorical in the index); missing values follow default_left. */
typedef struct hbr_row_split {
    hbr_segment seg;
    uint32_t feature;
    uint32_t below;
    uint32_t default_left;
    uint32_t n_table;
    const uint8_t *table;
} hbr_row_split;

typedef struct hbr_partitioned {
    hbr_segment left;
    hbr_segment right;
} hbr_partitioned;

/* RowEngine::partition: stable, in one batch; the children replace the
 * consumed segments. */
int hbr_partition(hbr_engine *e, const hbr_row_split *splits, uint64_t n, hbr_partitioned *out);

/* RowEngine::histograms: out holds n * 2 * total_bins f64. */
int hbr_histograms(hbr_engine *e, const hbr_segment *segs, uint64_t n, double *out);

/* RowEngine::rows: the row ids of one segment (len entries). */
int hbr_rows(hbr_engine *e, const hbr_segment *seg, uint32_t *out);

/* RowEngine::load_margins: start a margin run (n_rows * n_outputs f32). */
int hbr_load_margins(hbr_engine *e, const float *margins, uint64_t n, uint32_t n_outputs);

/* The device loss (DeviceLoss, src/tree/hist/mod.rs:355-365). */
#define HBR_LOSS_SQUARED_ERROR 0
#define HBR_LOSS_LOGISTIC 1
/* Every class of a softmax (the margins' k outputs, k <= 1024; labels are
 * class indices): no counterpart among the reference's DeviceLoss kinds
 * (src/tree/hist/mod.rs:355-370), whose softmax gradients stay on the host
 * (objective/multiclass.rs:43-55, simd/mod.rs:502-600); the same bits. */
#define HBR_LOSS_SOFTMAX 2
typedef struct hbr_device_loss {
    uint32_t kind;
    float scale_pos_weight;
    float min_hess;         /* logistic: 1e-16 */
    float max_input;        /* logistic: the vector kernel's range, 80 */
    uint64_t vector_rows;   /* logistic: rows the host runs 8-wide (VectorSplit.rows) */
} hbr_device_loss;

/* RowEngine::gradients: the loss's gradients of the device margins, with the
 * host's bits; labels (and weights, may be NULL) are copied on the first
 * call after hbr_load_margins. all_finite = 0 when a gradient is not finite. */
int hbr_gradients(hbr_engine *e, const hbr_device_loss *loss, const float *labels,
                  const float *weights, uint64_t n, int *all_finite);

/* The staged gradient pairs (interleaved g, h; n = n_rows), for checking a
 * device loss against the host's bits; after softmax gradients n = n_rows *
 * k gives every class's, class-major ([class][row]). No counterpart in the
 * reference: a diagnostic read of what hbr_gradients / hbr_prepare staged. */
int hbr_read_gradients(hbr_engine *e, float *out, uint64_t n);

/* RowEngine::add_leaf_values: margins[row] += value for each leaf's rows. */
int hbr_add_leaf_values(hbr_engine *e, const hbr_segment *segs, const float *values, uint64_t n);

/* RowEngine::read_margins. */
int hbr_read_margins(hbr_engine *e, float *out, uint64_t n);

/* Evaluation sets at the engine level, for a caller that drives its own
 * rounds (src/training/round.rs:141-143, where the host then adds each
 * finished tree to every eval set: margins.rs:148-152 add_tree_to_evals ->
 * :186-196 add_tree_margins). hbr_engine_add_eval copies a dense row-major
 * f32 matrix of the index's n_cols features (`missing` marks an absent
 * value, NaN: any NaN) and its starting margins (n_rows * n_outputs) to the
 * device; *index receives the set's number. hbr_engine_eval_add_tree adds
 * one tree (the reference's Node fields, src/tree/regtree.rs:38-66, one
 * array per field; children in pairs, right = left + 1; left < 0 marks a
 * leaf) to every set's margins of `output`, each row routed by raw value (a
 * present value goes left iff value < split_cond, a missing one follows
 * default_left), queued on the engine's stream with no synchronisation. */
int hbr_engine_add_eval(hbr_engine *e, const float *x, uint64_t n_rows, uint64_t n_cols, float missing,
                        const float *init_margins, uint32_t n_outputs, uint32_t *index);
int hbr_engine_eval_add_tree(hbr_engine *e, const uint32_t *split_feature, const float *split_cond,
                             const uint8_t *default_left, const int32_t *left, const int32_t *right,
                             const float *leaf_value, uint64_t n_nodes, uint32_t output);
/* hbr_engine_eval_add_tree for a tree with categorical splits (RegTree's
 * categorical nodes, src/tree/regtree.rs:59-66): node i with
 * is_categorical[i] sends a present value left iff its category (the
 * saturating cast of the value, tree/mod.rs:34-36) is among
 * categories[cat_begin[i], cat_end[i]) (the tree's pool, n_categories codes);
 * a missing value follows default_left; other nodes compare split_cond. */
int hbr_engine_eval_add_tree_categorical(hbr_engine *e, const uint32_t *split_feature, const float *split_cond,
                                         const uint8_t *default_left, const int32_t *left, const int32_t *right,
                                         const float *leaf_value, const uint8_t *is_categorical,
                                         const uint32_t *cat_begin, const uint32_t *cat_end,
                                         const uint32_t *categories, uint64_t n_categories, uint64_t n_nodes,
                                         uint32_t output);
/* Eval set `index`'s margins (n_rows * n_outputs, row-major). */
int hbr_engine_eval_margins(hbr_engine *e, uint32_t index, float *out);

/* RowEngine::reserve_hists: fits = 0 (nothing reserved) when `slots`
 * histograms do not fit. */
int hbr_reserve_hists(hbr_engine *e, uint64_t slots, int *fits);

/* RowEngine::build_resident: build each node's histogram into its slot,
 * then turn each (parent, built) pair's parent slot into parent - built.
 * Returns once the work is queued (nothing comes back): the engine's later
 * calls run after it on the same stream, and a device error surfaces at the
 * next call that waits for the device. */
int hbr_build_resident(hbr_engine *e, const hbr_segment *segs, const uint32_t *slots, uint64_t n,
                       const uint32_t *sibling_parent, const uint32_t *sibling_built, uint64_t n_siblings);

/* The split-search regularization (RegParams, src/tree/gain.rs:63-89; values
 * already rounded to f32 and widened). */
typedef struct hbr_reg_params {
    double lambda;
    double alpha;
    double max_delta_step;
    double min_child_weight;
} hbr_reg_params;

/* ScanRequest (src/tree/hist/mod.rs:304-311). `directions` may be NULL
 * (no monotone constraints); features must list every feature 0..n_cols-1.
 * The engine sums in fixed point: when has_fixed is set, fixed_g/fixed_h
 * are the node's exact sums as an earlier call returned them (preferred);
 * otherwise the f64 totals are converted, which is exact while they hold
 * at most 53 significant bits of the tree's fixed-point unit. */
typedef struct hbr_scan_request {
    uint32_t slot;
    uint32_t has_fixed;
    double total_g;
    double total_h;
    int64_t fixed_g;
    int64_t fixed_h;
    float root_gain;
    float lower;
    float upper;
    uint32_t n_features;
    const uint32_t *features;
    const int8_t *directions;
} hbr_scan_request;

/* NodeScan (src/tree/hist/mod.rs:327-350), kinds in its order. */
#define HBR_SCAN_EMPTY 0
#define HBR_SCAN_REPLAY 1
#define HBR_SCAN_NUMERIC 2
#define HBR_SCAN_CATEGORICAL 3
/* ScanFallback (src/tree/hist/mod.rs:313-324): why a node is replayed. */
#define HBR_FALLBACK_NUMERIC_SCORE 1
#define HBR_FALLBACK_CATEGORICAL_ORDER 2
#define HBR_FALLBACK_CATEGORICAL_SCORE 3
/* No counterpart in the reference's ScanFallback: in HBR_SUMS_FIXED_POINT
 * mode, a rival candidate scores within the error bound of the fixed-point
 * sums of the winner, or the winner's loss is within it of the validity
 * threshold; hbr_read_hist then returns the node's histogram in the
 * reference's own f64 summation order for the host's replay. */
#define HBR_FALLBACK_NEAR_TIE 4
typedef struct hbr_node_scan {
    uint32_t kind;
    uint32_t feature;
    float loss_chg;
    uint32_t backward;      /* numeric: the winner came from the missing-left pass */
    uint32_t offset;        /* numeric forward: last local bin going left; backward: first local bin going right */
    float loss_err;         /* numeric, fixed-point guard on: a bound on |loss_chg - the CPU's loss_chg| */
    double acc_g, acc_h;    /* numeric: the pass's accumulated statistics (left forward, right backward) */
    double left_g, left_h, right_g, right_h;
    int64_t fixed_left_g, fixed_left_h, fixed_right_g, fixed_right_h; /* exact sums */
    /* categorical: missing values go left; the winner's categories
     * (ascending codes) are [cat_begin, cat_end) of the scan's pool
     * (hbr_scan_categories). left is the set's child: the orientation the
     * tree records (XGBoost's children swapped). */
    uint32_t default_left;
    uint32_t fallback;      /* HBR_SCAN_REPLAY: an HBR_FALLBACK_* reason */
    uint32_t cat_begin, cat_end;
} hbr_node_scan;

/* RowEngine::root_total with the exact fixed-point sums as well. */
int hbr_root_total_fixed(hbr_engine *e, const hbr_segment *seg, double out[2], int64_t fixed[2]);

/* RowEngine::scan_resident: numeric and categorical features (the
 * reference's sweep, src/tree/builder/categorical.rs:48-170: one-hot below 4
 * categories, else the weight-sorted partition scans). In
 * HBR_SUMS_FIXED_POINT mode beyond the exact domain each numeric winner is
 * certified against its rivals: a node whose winner a rival partition could
 * beat within the error bound of the fixed-point sums (or whose loss is
 * within it of the validity threshold) is HBR_SCAN_REPLAY with
 * HBR_FALLBACK_NEAR_TIE, for the host's replay from hbr_read_hist. */
int hbr_scan_resident(hbr_engine *e, const hbr_reg_params *reg, const hbr_scan_request *requests,
                      uint64_t n, hbr_node_scan *out);
/* The last hbr_scan_resident call's category pool: n entries (the largest
 * cat_end of its categorical winners, 0 when it had none). */
int hbr_scan_categories(hbr_engine *e, uint32_t *out, uint64_t n);

/* RowEngine::read_hist (src/tree/hist/mod.rs:282-295, called for a
 * NodeScan::Replay, src/tree/builder/hist/device.rs:633-646): 2 * total_bins
 * f64. In the exact domain, the slot's fixed-point bins (equal to the CPU's
 * sums). Beyond it, the slot's rows are summed on the device in the CPU
 * build's own f64 order (each bin's rows in row order from +0.0, in the
 * blocks of sum_order, tree/hist/mod.rs:399-607), so the host replays the
 * node on the sums its CPU path would have: for row-major u8 indexes of at
 * most 256 features and 9,216 bins whose slot the row-engine calls of this
 * tree built (hbr_build_resident, siblings included). Otherwise the
 * fixed-point bins (HBR_SUMS_FIXED_POINT) or HBR_REFUSED (HBR_SUMS_EXACT). */
int hbr_read_hist(hbr_engine *e, uint32_t slot, double *out);

/* No counterpart in the reference: the fixed-point guard of
 * hbr_scan_resident and of the whole-round trainer. Beyond the exact domain
 * each numeric winner's score is bounded (the quantisation of every row's
 * pair, the f64 rounding of the CPU's sums, the f32 roundings of the score)
 * against every other partition of the node's rows and against the
 * validity threshold. A node it cannot certify is:
 *   HBR_GUARD_RESOLVE (the default): searched again on the device over its
 *     histogram in the CPU builder's own f64 sums (hbr_read_hist's), and
 *     returned as that search's winner (HBR_SCAN_NUMERIC or _EMPTY), with
 *     the CPU's f64 child statistics and their fixed-point sums;
 *   HBR_GUARD_REPLAY: returned as HBR_SCAN_REPLAY, HBR_FALLBACK_NEAR_TIE,
 *     for the host's own replay from hbr_read_hist;
 *   HBR_GUARD_OFF: returned as the fixed-point winner.
 * gamma: the caller's min_split_loss, checked beside kRtEps (1e-6). The
 * whole-round trainer counts the nodes its device decisions could not
 * certify (hbr_engine_counters.near_ties). */
/* No counterpart in the reference's interface (its builder computes them
 * itself between row-engine calls): the host arithmetic a caller of the row
 * engine needs, as the reference's CPU builder performs it with its
 * RegParams rounded to f32 (tree/gain.rs:82-116): a node's gain at its
 * bounded weight (xgb_node_gain, builder/shared.rs:131-141: the root_gain
 * of a ScanRequest) and a leaf's bounded weight before eta
 * (calc_weight_bounded, tree/constraints.rs; finish_leaf_values,
 * builder/shared.rs:174-187). Host only: no device is touched. */
int hbr_node_gain(const hbr_reg_params *reg, double g, double h, double lower, double upper, float *out);
int hbr_leaf_weight(const hbr_reg_params *reg, double g, double h, double lower, double upper, float *out);

#define HBR_GUARD_OFF 0
#define HBR_GUARD_REPLAY 1
#define HBR_GUARD_RESOLVE 2
int hbr_engine_set_guard(hbr_engine *e, int mode, double gamma);

/* Work counters since the engine opened (no counterpart in the reference;
 * they give the algorithmic bytes the roofline figures divide by). */
typedef struct hbr_engine_counters {
    uint64_t hist_nodes;       /* node histograms built (siblings excluded) */
    uint64_t hist_rows;        /* rows summed into them */
    uint64_t hist_bytes;       /* algorithmic bytes: rows * (bin bytes + 8 (+ 4 gathered)) */
    uint64_t partition_rows;   /* rows routed */
    uint64_t trees;
    uint64_t near_ties;        /* decided nodes whose winner the fixed-point guard could not
                                  certify (see hbr_engine_set_guard) */
    uint64_t near_ties_resolved; /* of those, searched again on the CPU builder's sums on the device */
    uint64_t row_orders;       /* times the whole-round trainer put the rows in a tree's leaf order */
} hbr_engine_counters;
int hbr_engine_counters_read(hbr_engine *e, hbr_engine_counters *out);

/* Per-kernel device time (HIP events on the engine's stream) of the kernels
 * whose name starts with kernel_prefix; profiling is off until enabled, and
 * enabling it clears the previous statistics. on = N >= 1 times every N-th
 * matching launch (each timed launch stalls the stream for its events;
 * N = 1 times them all) and counts them all; on = 0 turns it off.
 * buf receives "name=ms,timed,launches;..." (ms over the timed launches). */
int hbr_set_profiling(hbr_engine *e, int on, const char *kernel_prefix);
int hbr_kernel_stats(hbr_engine *e, char *buf, size_t len);

/* ------------------------------------------------------------------------- */
/* Device-resident training (src/training/round.rs:105-148, grow_round).     */
/* ------------------------------------------------------------------------- */

#define HBR_OBJ_SQUARED_ERROR 0
#define HBR_OBJ_LOGISTIC 1
#define HBR_OBJ_SOFTMAX 2
/* binary:logitraw: the logistic loss with the identity link (raw margins
 * and a raw intercept, src/objective/classification.rs:55-72). */
#define HBR_OBJ_LOGITRAW 3
#define HBR_GROW_DEPTHWISE 0
#define HBR_GROW_LOSSGUIDE 1

/* TrainingParams fields of the path (src/config/params.rs:415-674). */
typedef struct hbr_train_params {
    double eta, gamma, lambda, alpha, min_child_weight, max_delta_step;
    int64_t max_depth;       /* <= 0: unbounded */
    int64_t max_leaves;      /* <= 0: unbounded */
    int32_t grow_policy;
    int32_t objective;
    int32_t num_class;
    float scale_pos_weight;
    const int8_t *monotone;  /* per feature or NULL */
    uint64_t n_monotone;
    float base_score;
    int32_t has_base_score;
} hbr_train_params;

typedef struct hbr_trainer hbr_trainer;

int hbr_trainer_create(hbr_engine *e, const hbr_train_params *p, const float *labels,
                       const float *weights, uint64_t n_rows, hbr_trainer **out);
/* Run `rounds` boosting iterations. */
int hbr_trainer_boost(hbr_trainer *t, uint64_t rounds);
int hbr_trainer_num_trees(hbr_trainer *t, uint64_t *n);
int hbr_trainer_num_outputs(hbr_trainer *t, uint32_t *k);
int hbr_trainer_base_score(hbr_trainer *t, float *out);
/* Tree t's node count. */
int hbr_trainer_tree_size(hbr_trainer *t, uint64_t tree, uint64_t *n_nodes);
/* A tree in the reference's Node layout (src/tree/regtree.rs:38-66), one
 * array per field (n_nodes each). split_bin receives each split's global bin
 * (-1 below every bin, -2 for leaves). */
int hbr_trainer_tree(hbr_trainer *t, uint64_t tree, uint32_t *split_feature, float *split_cond,
                     uint8_t *default_left, int32_t *left, int32_t *right, float *leaf_value,
                     float *sum_hess, float *split_gain, int64_t *split_bin);
/* A tree's categorical splits (src/tree/regtree.rs:59-66): per node
 * is_categorical, and the range [cat_begin, cat_end) of the tree's pool of
 * categories that go left; the pool's length in *n_categories (call first
 * with categories NULL to size it). Trees grown on an index with
 * categorical features (hbr_cuts_from_*_typed) hold them. */
int hbr_trainer_tree_categories(hbr_trainer *t, uint64_t tree, uint8_t *is_categorical, uint32_t *cat_begin,
                                uint32_t *cat_end, uint32_t *categories, uint64_t *n_categories);
/* The training margins (n_rows * n_outputs). */
int hbr_trainer_margins(hbr_trainer *t, float *out);
/* An evaluation set (the `evals` of training, src/training/margins.rs:148-152
 * and src/training/round.rs:141-143, where the host adds each tree to every
 * eval set's margins): a dense row-major f32 matrix with the training
 * matrix's n_cols features (`missing` marks an absent value, NaN: any NaN),
 * copied to the device. Its margins start from base_margin (n_rows *
 * n_outputs, or NULL for the base score), take every tree grown so far and
 * then every later tree on the device as it is grown, routed by raw value.
 * *index receives the set's number. The sets belong to the engine's latest
 * trainer: creating a trainer on the engine drops every set added before. */
int hbr_trainer_add_eval(hbr_trainer *t, const float *x, uint64_t n_rows, uint64_t n_cols, float missing,
                         const float *base_margin, uint32_t *index);
/* Eval set `index`'s margins (n_rows * n_outputs, row-major). */
int hbr_trainer_eval_margins(hbr_trainer *t, uint32_t index, float *out);
void hbr_trainer_free(hbr_trainer *t);

/* ------------------------------------------------------------------------- */
/* Batch prediction (GpuModel, src/backend/cuda/predict.rs:401-520).          */
/* ------------------------------------------------------------------------- */

typedef struct hbr_forest hbr_forest;

/* A scalar-leaf forest: per tree its nodes in the reference's layout; tree
 * t adds tree_weight[t] * leaf to output tree_output[t]. Categorical splits
 * (src/tree/regtree.rs:59-66, tree/mod.rs:34-58): node i with
 * is_categorical[i] sends a present value left iff its saturating u32 cast
 * is one of categories[cat_begin[i], cat_end[i]) (ranges into the forest's
 * one pool of n_categories entries); is_categorical NULL: every split
 * numeric. */
typedef struct hbr_forest_desc {
    uint64_t n_trees;
    const uint64_t *tree_offset;    /* n_trees + 1 */
    const uint32_t *split_feature;
    const float *split_cond;
    const uint8_t *default_left;
    const int32_t *left;
    const int32_t *right;
    const float *leaf_value;
    const float *tree_weight;       /* n_trees */
    const uint32_t *tree_output;    /* n_trees */
    uint32_t n_outputs;
    uint32_t pad;
    const float *base_score;        /* n_outputs */
    const uint8_t *is_categorical;  /* per node, or NULL */
    const uint32_t *cat_begin;      /* per node (categorical nodes) */
    const uint32_t *cat_end;
    const uint32_t *categories;     /* n_categories */
    uint64_t n_categories;
} hbr_forest_desc;

/* BoostedModel::to_cuda: upload the forest once. */
int hbr_forest_upload(int ordinal, const hbr_forest_desc *fd, hbr_forest **out);
void hbr_forest_free(hbr_forest *f);

/* GpuModel::predict_margin over host rows (n_rows x n_cols f32, row-major;
 * `missing` as for the matrix): out[n_rows * n_outputs]. */
int hbr_predict_margin(hbr_forest *f, const float *x, uint64_t n_rows, uint64_t n_cols,
                       float missing, float *out);
/* The same from each row's starting margins (n_rows * n_outputs, row-major;
 * NULL: the base scores): the reference's initial margins, a DMatrix's
 * base_margin (src/backend/shared.rs:218-239, plan_margins), to which the
 * trees' leaf values are added in tree order. */
int hbr_predict_margin_from(hbr_forest *f, const float *x, uint64_t n_rows, uint64_t n_cols, float missing,
                            const float *init_margins, float *out);
/* The same over device memory (x, out and optional leaf ids [n_rows * n_trees]
 * all device pointers): inputs already resident, nothing copied. The
 * outputs are complete when the call returns. */
int hbr_predict_margin_device(hbr_forest *f, const float *x, uint64_t n_rows, uint64_t n_cols,
                              float missing, float *out, int32_t *leaf_out);
/* BoostedModel::predict_leaf: each row's leaf node id per tree (host). */
int hbr_predict_leaf(hbr_forest *f, const float *x, uint64_t n_rows, uint64_t n_cols, float missing,
                     int32_t *out);
int hbr_forest_set_profiling(hbr_forest *f, int on, const char *kernel_prefix);
int hbr_forest_kernel_stats(hbr_forest *f, char *buf, size_t len);

/* The objective's prediction transform, on the host, in place: the
 * reference's Transform::apply (src/model/transform.rs:74-104), which runs
 * on the CPU after GpuModel::predict_margin (src/backend/cuda/predict.rs:
 * 466-474). expf is the host C library's, as the reference's f32::exp.
 *   HBR_TRANSFORM_SIGMOID      XGBoost's common::Sigmoid of each value,
 *                              1 / (expf(min(-x, 88.7)) + 1) (simd/mod.rs:422-427);
 *   HBR_TRANSFORM_SOFTMAX      common::Softmax of each row of n_outputs:
 *                              shift by the row's maximum, expf, sum in f64,
 *                              divide by the sum rounded to f32 (simd/mod.rs:557-573);
 *   HBR_TRANSFORM_CLASS_INDEX  multi:softmax: row r's first largest margin's
 *                              index, as f32, into values[r] (simd/mod.rs:750-758). */
#define HBR_TRANSFORM_SIGMOID 1
#define HBR_TRANSFORM_SOFTMAX 2
#define HBR_TRANSFORM_CLASS_INDEX 3
int hbr_pred_transform(int kind, float *values, uint64_t n_rows, uint32_t n_outputs);

/* Device memory for callers that keep inputs resident (bytes on device
 * `ordinal`). */
int hbr_device_alloc(int ordinal, uint64_t bytes, void **out);
int hbr_device_free(int ordinal, void *p);
int hbr_device_upload(int ordinal, void *dst, const void *src, uint64_t bytes);
int hbr_device_download(int ordinal, void *dst, const void *src, uint64_t bytes);
/* Device-to-device copy (completes before the call returns). No counterpart
 * in the reference: a plain copy of known size, which profiles use to scale
 * hardware byte counters. */
int hbr_device_copy(int ordinal, void *dst, const void *src, uint64_t bytes);

#ifdef __cplusplus
}
#endif
#endif
