// Kernel argument records shared by the HIP kernels and the host runtime.
//
// Every kernel takes exactly one of these structs by value; the host launches
// it through hipModuleLaunchKernel with a single kernel parameter. Plain C
// layout, fixed-width fields, device pointers as typed pointers (64-bit on
// both sides).
#pragma once
#include <stdint.h>

namespace hbr {

// Rows per partition tile (one workgroup).
constexpr uint32_t kPartTile = 2048;
constexpr uint32_t kPartThreads = 256;
// Histogram workgroups: threads, and the fewest rows a tile is cut to (tiles
// are sized per launch so that about one wave of workgroups covers it).
constexpr uint32_t kHistThreads = 512;
constexpr uint32_t kHistMinRows = 4096;
// Bins of one feature the split scan processes per pass (4 per lane).
constexpr uint32_t kScanChunk = 256;
// Threads of the elementwise kernels.
constexpr uint32_t kThreads = 256;

// One row's gradient and Hessian (GradPair, objective/mod.rs:92-97).
struct GPair {
    float g;
    float h;
};

// Fixed-point histogram bin: the exact integer sums of the quantized
// gradients and Hessians of the rows in the bin.
struct QBin {
    int64_t g;
    int64_t h;
};

// Per-tree quantization: x is stored as rint(x * 2^-exp), exp chosen so that
// no sum over the tree's rows can exceed 2^62 in magnitude.
struct QScale {
    int32_t exp_g;
    int32_t exp_h;
    uint32_t max_g_bits;  // |g| maximum as f32 bits (non-negative floats order as ints)
    uint32_t max_h_bits;
    uint32_t nonfinite;   // count of rows with a non-finite g or h
    uint32_t scalar_rows; // rows listed for the scalar sigmoid (until hbr_finish_scale)
    uint32_t pad[2];      // hbr_grain_fold: 1024 - (grain + 150) of g and of h (0: all zero)
    uint32_t deferred;    // rows hbr_finish_scale took from the list (their pairs are its own)
    uint32_t pad2;
};

// A node's rows: `len` row ids at `offset` of row buffer `buf` (0 or 1).
struct Seg {
    uint32_t offset;
    uint32_t len;
    uint32_t buf;
    uint32_t pad;
};

// ---- index ---------------------------------------------------------------------
// Dense re-encode: a chunk of rows' global bins (row-major, n_cols per row)
// to feature-local u8 bins, row-major (stride bytes per row) and feature-major.
struct EncodeArgs {
    const uint16_t *g16;      // chunk's global bins (u16), or null
    const uint32_t *g32;      // or u32
    const uint32_t *feature_offset;
    uint8_t *rows8;
    uint8_t *cols8;
    uint64_t n_rows;          // whole index
    uint64_t row0;            // first row of the chunk
    uint32_t chunk_rows;
    uint32_t n_cols;
    uint32_t stride;
    uint32_t pad;
};

// Binning on the device (HistCuts::bin_of, src/data/quantile.rs:285-296,
// and the GHistIndex layouts, src/data/ghist.rs:213-257): a chunk of a
// dense f32 matrix to feature-local u8 bins (features of at most 256 bins),
// the missing bitmap and each row's count of present values. One thread per
// row; a chunk starts at a multiple of 64 rows.
// Cut values the binning kernels hold in LDS (more: read from memory by
// hbr_bin_dense; hbr_bin_dense32 needs them in LDS).
constexpr uint32_t kBinLdsCuts = 12288;

struct BinArgs {
    const float *x;                 // the chunk's rows, row-major [chunk_rows][n_cols]
    const float *cut_values;        // total_bins
    const uint32_t *feature_offset; // n_cols + 1
    uint8_t *rows8;                 // [n_rows][stride] local bins, or null
    uint8_t *cols8;                 // [n_cols][n_rows] local bins (0 where missing)
    uint64_t *missing;              // [n_cols][words], bit set = missing
    uint32_t *row_count;            // per row: present values
    uint64_t n_rows;
    uint64_t row0;
    uint32_t chunk_rows;
    uint32_t n_cols;
    uint32_t stride;
    uint32_t words;
    uint32_t total_bins;
    float missing_value;            // the absent marker (NaN: any NaN)
    uint32_t missing_is_nan;
    uint32_t row_mask;              // n_cols <= kMaskedMaxFeatures: the row's missing mask in its last word
};

// Dense u8 rows of a matrix with missing values: a missing cell's byte is 0
// and a mask bit marks it. At most kMaskedMaxFeatures features: rows of 32
// bytes, bit f of the row's last word (kMaskWord) for feature f. Wider (at
// most kMaskedWideMaxFeatures): the bins of G = ceil(F / 32) groups of 32
// features, then a 32-byte chunk of mask words, word g (at byte 32 G + 4 g)
// for group g's features. A row's mask words start at its `mask_at` byte
// (28, or 32 G). The histogram kernel skips masked cells; the margin walks
// send them the split's default way.
constexpr uint32_t kMaskedMaxFeatures = 28;
constexpr uint32_t kMaskedWideMaxFeatures = 256;
constexpr uint32_t kMaskWord = 7;
struct RowsFromColsArgs {
    const uint8_t *cols8;       // [n_cols][n_rows]
    const uint64_t *missing;    // [n_cols][words] or null
    uint8_t *rows8;             // [n_rows][stride]
    uint64_t n_rows;
    uint32_t n_cols;
    uint32_t words;
    uint32_t stride;            // 32, or 32 G + 32
    uint32_t mask_at;           // byte of the first mask word: 28, or 32 G
};

// Exclusive scan of the rows' present counts into row_ptr (n_rows + 1):
// per block of kCountBlock rows its total, then (with the blocks' offsets,
// scanned on the host) every row's offset.
constexpr uint32_t kCountBlock = 8192;
struct CountScanArgs {
    const uint32_t *row_count;
    uint64_t *block_total;          // per block (first pass)
    const uint64_t *block_offset;   // per block (second pass)
    uint64_t *row_ptr;              // n_rows + 1 (second pass)
    uint64_t n_rows;
};

// CSR global bins of the present cells, in feature order per row, from the
// local columns and the missing bitmap.
struct CsrFillArgs {
    const uint8_t *cols8;
    const uint64_t *missing;
    const uint32_t *feature_offset;
    const uint64_t *row_ptr;
    uint32_t *gbins;
    uint64_t n_rows;
    uint32_t n_cols;
    uint32_t words;
};

// ---- gradients ---------------------------------------------------------------
enum LossKind : uint32_t { kSquaredError = 0, kLogistic = 1 };

struct GradArgs {
    const float *margins;   // n (one output)
    const float *labels;    // n
    const float *weights;   // n or null
    GPair *gpair;           // n (null: not written, the rows carry the pairs)
    QScale *scale;          // max folds (atomics) land here
    const uint64_t *exp_table;  // the expf restatement's 32 entries (scalar rows)
    uint32_t *scalar_list;  // where kernels that defer the scalar rows list them
    uint32_t n;
    uint32_t vec_rows;      // logistic: rows covered by 8-row vectors
    uint32_t loss;
    float scale_pos_weight;
    float min_hess;
    float max_input;        // logistic vector range (80)
    // Logistic pairs carried by the rows (set only for unit weights, a
    // scale_pos_weight of 1 and labels 0 or 1, which make (g, h) a function
    // of p and y alone): row i's word at pair_rows + i * pair_stride +
    // pair_byte (padding bytes of the index) gets bits(p) | y << 31.
    uint8_t *pair_rows;
    uint32_t pair_stride;
    uint32_t pair_byte;
    // Rows held in another order than the original one (a reorder by a
    // tree's leaves; the fused walks only): position i holds original row
    // perm[i], and the 8-row vectors are those of the original rows. A row
    // then takes the vector path on its own margin's test; a row of the
    // vector range that fails it marks its original vector g
    // (group_stamp[g] = stamp; g listed once in bad_groups[1..], counted in
    // bad_groups[0]), whose other rows hbr_regroup moves to the scalar path.
    const uint32_t *perm;
    uint32_t *group_stamp;  // [vec_rows / 8]
    uint32_t *bad_groups;   // [1 + vec_rows / 8]
    uint32_t stamp;         // this pass's mark (non-zero, new each pass)
    uint32_t pad_perm;
};

// Softmax gradients of every class of every row (simd/mod.rs:502-600),
// class-major: row r's pair for class c at gpair[c * n + r]. Class c's
// magnitude maxima and non-finite count fold into scales[c]. Rows below
// `batched` (2 or 4 classes) take the vector batches of 8 / k rows.
constexpr uint32_t kSoftmaxMaxClasses = 1024;
struct SoftmaxArgs {
    const float *margins;       // [n][k]
    const float *labels;        // n
    const float *weights;       // n or null
    GPair *gpair;               // [k][n]
    QScale *scales;             // k
    const uint64_t *exp_table;  // 32 entries: bits(2^(i/32)) - (i << 47)
    uint32_t n;
    uint32_t k;
    uint32_t batched;
    float min_hess;
};

// ---- row buffers -------------------------------------------------------------
struct IotaArgs {
    uint32_t *rows;
    uint32_t first;
    uint32_t n;
};

// ---- root totals -------------------------------------------------------------
// One sum per blockIdx.y (a tree of a level of trees): its pairs from
// gpair + y tree_pairs, its scale at scale + y, its sums into out + y.
struct TotalArgs {
    const uint32_t *rows;   // null: contiguous from `first`
    uint32_t first;
    uint32_t n;
    const GPair *gpair;
    const QScale *scale;
    QBin *out;              // accumulated with 64-bit atomics (zeroed before)
    uint64_t tree_pairs;
};
// Workgroups per sum: few enough that their atomics on the one total do
// not queue for longer than the rows take to read.
constexpr uint32_t kTotalBlocks = 256;

// ---- level counts on the device ---------------------------------------------------
// A depthwise tree grown on the device: each level's decision kernel writes
// how many splits and partition tiles the level has, and the kernels of the
// level read their work counts from here (their grids are launched for the
// most the level can hold, and the surplus workgroups exit).
struct GrowCounts {
    uint32_t n_front;       // frontier nodes of the level being decided
    uint32_t n_splits;      // splits of the last decided level (0 at the depth limit)
    uint32_t n_tiles;       // their partition tiles
    uint32_t n_nodes;       // tree nodes so far
    uint32_t hist_nodes;    // histograms built this tree (root included)
    uint32_t error;         // nonzero: a level needed more slots than reserved
    uint64_t hist_rows;     // rows summed into built children this tree (root excluded)
    uint64_t part_rows;     // rows partitioned this tree
    uint32_t near_ties;     // nodes decided this tree whose winner carried kScanNearTie
    uint32_t pad;
};

// ---- partition -----------------------------------------------------------------
// One node to partition: its segment, the split's routing and where its
// children's statistics go.
struct PartSplit {
    Seg seg;                // parent rows (source buffer seg.buf)
    uint32_t feature;
    uint32_t limit;         // present local bins < limit go left
    uint32_t default_left;
    uint32_t tile_begin;    // first partition tile of this split
    uint32_t fresh_slot;    // histogram slot for the built child
    uint32_t parent_slot;   // parent's slot, becomes the sibling's
    uint32_t identity;      // the parent's rows are j (seg.offset % n_rows + j; no row list is read)
    uint32_t tree;          // tree of a batched level (the class of a softmax round)
    uint32_t table;         // categorical split: 1 + its row in PartArgs::cat_tables (present local
                            // bins whose bit is set go left; limit is unused); 0: numeric
    uint32_t pad[3];
};

// Device decision per split after the scan of tile counts.
struct PartOut {
    uint32_t left_len;
    uint32_t built_left;    // 1: the left child is the smaller (built) one
    uint32_t pad[2];
};

struct PartArgs {
    const PartSplit *splits;
    uint32_t n_splits;
    uint32_t n_tiles;            // tiles of split s: [tile_begin, next split's tile_begin)
    uint32_t *tile_left;         // per tile left count (count pass) / left offset (after scan)
    uint64_t *decisions;         // per tile kPartTile / 64 ballots of "goes left" (count pass)
    PartOut *out;
    const uint32_t *src_rows[2];
    uint32_t *dst_rows[2];
    // routing data
    uint32_t dense;              // dense columns present
    const uint8_t *cols8;        // feature-major local bins [f][n] (u8)
    const uint16_t *cols16;      // or u16
    const uint64_t *missing;     // feature-major bitmap (ceil(n/64) words per feature) or null
    const uint64_t *row_ptr;     // CSR (no columns)
    const uint32_t *gbins;       // CSR global bins
    const uint32_t *feature_offset;
    uint32_t n_rows;
    uint32_t words;              // bitmap words per feature
    const GrowCounts *grow;      // non-null: n_splits and n_tiles are read from here
    const uint32_t *tile_split;  // non-null: the split of every tile (else found by binary search)
    uint32_t csr_ascending;      // every CSR row's global bins ascend: routing binary-searches them
    uint32_t pad;
    const uint32_t *cat_tables;  // kCatWords words per categorical split: its left local bins
};

// ---- histograms ----------------------------------------------------------------
// A row tile of one node: rows [row0, row0 + rows) of node `node`, the k-th
// of that node's tiles. Every feature group of the launch takes the tile.
struct HistTile {
    uint32_t node;      // index into the node table
    uint32_t row0;
    uint32_t rows;
    uint32_t k;
};

// One node whose histogram is built into `slot`. When `from_split` is set,
// the node is the smaller child of split `split` and its segment comes from
// the partition's device output (the plan kernel resolves it in place).
struct HistNode {
    Seg seg;
    uint32_t slot;
    uint32_t from_split;
    uint32_t split;
    uint32_t contiguous; // rows are seg.offset .. seg.offset+len (no row buffer)
    uint32_t tile_begin; // first row tile (written by the plan kernel)
    uint32_t n_tiles;    // row tiles of the node (written by the plan kernel)
    uint32_t pad[2];     // [0]: first partial of a multi-tile node; [1]: parent slot + 1 of a
                         // split's built child, whose sibling = parent - built as bins complete
                         // (dense kernels; both written by the plan kernel)
    uint32_t cls;        // class (tree) of a batched level: pairs at gpair + cls * class_rows,
                         // quantised with scale[cls]
    uint32_t pad2[3];
};

// Device tiling of a histogram launch: each node's rows cut into tiles of
// `tile_rows` rows (a multiple of 64, at least min_rows), the smallest size
// that gives at most target_tiles tiles (one tile per node when the nodes
// outnumber it); never more than target_tiles + n_nodes tiles.
struct PlanArgs {
    HistNode *nodes;
    uint32_t n_nodes;
    uint32_t target_tiles;
    const PartSplit *splits;
    const PartOut *part_out;
    HistTile *tiles;
    uint32_t *counts;           // [0] tiles, [1] tile_rows
    uint32_t min_rows;
    uint32_t fuse_subtract;     // built children of splits also update their siblings (dense kernels)
    const GrowCounts *grow;     // non-null: one node per split of the level, n_splits read from here
};

// The reference's CPU histogram in its own f64 order (replays): one
// workgroup per block of `grain` rows, thread f owning feature f's bins in
// LDS (each bin one thread's chain in row order from +0.0); every block's
// partial then added to the output in block order.
constexpr uint32_t kExactThreads = 256;     // features per index, at most
constexpr uint32_t kExactMaxWords = 18432;  // f64 words of LDS: 2 x total_bins
struct ExactArgs {
    const uint32_t *rows;    // the node's row ids; null: rows first .. first + m - 1
    uint32_t first;
    uint32_t m;
    uint32_t grain;          // rows per block (the last shorter)
    uint32_t blk0;           // the launch's first block
    const uint8_t *bins8;    // row-major u8 local bins
    uint32_t stride;
    uint32_t n_cols;
    const uint32_t *feature_offset;
    const GPair *gpair;      // or null with row_pairs
    uint32_t row_pairs;      // the logistic pair from each row's last word
    float min_hess;
    uint32_t masked;         // the row's missing cells (mask words from byte mask_at) add nowhere
    uint32_t mask_at;
    uint32_t total_bins;
    double *partial;         // per block of the launch: total_bins x (g, h)
};

struct ExactSumArgs {
    const double *partial;
    uint32_t n_blocks;
    uint32_t first;          // 1: the output starts as block 0's partial
    double *out;
    uint32_t n;              // words (2 x total_bins)
    const double *minus;     // non-null: out -= minus instead (a sibling from its parent)
};

struct HistArgs {
    const HistNode *nodes;
    const HistTile *tiles;
    const uint32_t *counts;     // plan output: [0] tiles
    const uint32_t *rows[2];
    const GPair *gpair;
    const QScale *scale;
    const uint8_t *bins8;       // dense row-major local bins [n][stride]
    uint32_t stride;            // bytes per row
    uint32_t n_cols;
    const uint64_t *row_ptr;    // CSR
    const uint32_t *gbins;
    const uint32_t *feature_offset;
    QBin *hist;                 // slots * total_bins
    QBin *partial;              // per (tile, feature group): fg * 256 bins
    uint32_t total_bins;
    uint32_t groups;            // feature groups (dense) or bin ranges (CSR) per tile
    uint32_t class_rows;        // batched levels: the pairs of class c start at gpair + c * class_rows
    uint32_t pad;
    // CSR rows whose global bins ascend: row r's entries of bin range g are
    // row_ptr[r] + [csr_ranges[r * (groups + 1) + g], ... + g + 1]) (null: scan the row)
    const uint32_t *csr_ranges;
    // Nonzero: the pairs are the logistic pairs the rows carry in the last
    // word of their (single) 32-feature group (GradArgs::pair_rows), g = p - y
    // and h = max(p * (1 - p), min_hess), instead of gpair.
    uint32_t row_pairs;
    float min_hess;
    uint32_t masked;            // rows carry missing masks (fg32 groups; the mask words at mask_at)
    uint32_t mask_at;           // masked: the byte of a row's first mask word (28: 32-byte rows)
    // Dense rows of u16 local bins (hbr_hist_dense16_*): row r's bin of
    // feature f at bins16[r * stride16 + f]; partials of fg x (kWideLdsBins /
    // fg) bins per (tile, feature group)
    const uint16_t *bins16;
    uint32_t stride16;          // elements per row (a multiple of 16)
    uint32_t pad4;
};

// Dense indexes with a feature of more than 256 bins (at most kWideBinsMax):
// rows of u16 local bins. A histogram workgroup holds fg features of
// kWideLdsBins / fg bins each in LDS (fg = 16, 8, 4, 2 or 1: the widest
// feature's bins rounded up to a power of two, times fg, is kWideLdsBins).
constexpr uint32_t kWideBinsMax = 8192;
constexpr uint32_t kWideLdsBins = 8192;
struct Encode16Args {
    const uint32_t *gbins;      // the dense index's global bins, row-major [n_rows][n_cols]
    const uint32_t *feature_offset;
    uint16_t *rows16;           // [n_rows][stride16], zero beyond n_cols
    uint64_t n_rows;
    uint32_t n_cols;
    uint32_t stride16;
};

// Each CSR row's first entry of every kCsrGroupBins range (rows' global bins ascend).
struct CsrRangeArgs {
    const uint64_t *row_ptr;
    const uint32_t *gbins;
    uint32_t *ranges;            // n_rows x (groups + 1), relative to row_ptr[r]
    uint32_t n_rows;
    uint32_t groups;
};

// CSR histograms: a workgroup sums one tile's rows into one range of
// kCsrGroupBins global bins in LDS.
constexpr uint32_t kCsrGroupBins = 8192;
constexpr uint32_t kCsrThreads = 1024;

// A histogram of a caller's device row list built in a fixed scratch area
// (no allocation): the row ids are checked against the index, the one node
// record is written on the device, and the int64 bins of the output are
// turned into f64 in place at the end.
struct FixedBuildArgs {
    const uint32_t *rows;       // caller's device row ids
    uint64_t m;
    uint32_t n_rows;            // index rows: ids at or beyond are refused
    uint32_t total_bins;
    uint32_t *flag;             // scratch word: nonzero when some id is out of range
    HistNode *node;             // scratch node record
    QBin *bins;                 // the caller's output, first as int64 bins
    double *out;                // the same memory as f64 (g, h) pairs
    const QScale *scale;        // the staged tree's exponents
};

// Sum of a node's tile partials into its slot (nodes of one tile are
// written by the histogram kernel directly).
struct ReduceArgs {
    const HistNode *nodes;
    const QBin *partial;
    QBin *hist;
    const uint32_t *feature_offset;
    uint32_t n_cols;
    uint32_t total_bins;
    uint32_t groups;
    uint32_t fg;
    const GrowCounts *grow;     // non-null: nodes = its n_splits (the grid covers the most)
    uint32_t group_bins;        // bins per feature in a partial: 256 (u8 rows) or kWideLdsBins / fg
    uint32_t quarters;          // workgroups per feature: group_bins / 64
};

// sibling = parent - built, in place in the parent's slot, for each split.
struct SubArgs {
    const PartSplit *splits;
    uint32_t n_splits;
    QBin *hist;
    uint32_t total_bins;
};

// ---- split scan ------------------------------------------------------------------
struct ScanNode {
    uint32_t slot;           // histogram slot (ignored when from_split)
    uint32_t from_split;     // slot decided by the partition: child `child` of split `split`
    uint32_t split;
    uint32_t child;          // 0 left, 1 right
    QBin total;              // node statistics (fixed point)
    float root_gain;
    float lower, upper;
    uint32_t pad;            // flags (kScanDeviceRoot) | class << kScanClassShift
    uint32_t rows;           // the node's row count (from_split: read from the partition)
    uint32_t pad2;
};

struct ScanParams {
    double lambda, alpha, max_delta_step, min_child_weight;
};

// Categorical features (builder/categorical.rs): at most kCatMaxBins
// categories (bins) each; a split's set is a bitmask of kCatWords words over
// the feature's local bins.
constexpr uint32_t kCatMaxBins = 1024;
constexpr uint32_t kCatWords = kCatMaxBins / 32;
constexpr uint32_t kScanCategorical = 4u;
// ScanBest::flags bits asking for a host replay of the node (the trait's
// NodeScan::Replay reasons, src/tree/hist/mod.rs:313-331): a numeric
// candidate's score is NaN; a categorical weight is not finite (the sort's
// order is then not total); a categorical candidate's score is NaN.
constexpr uint32_t kScanNumericNaN = 2u;
constexpr uint32_t kScanCatOrder = 8u;
constexpr uint32_t kScanCatNaN = 16u;
constexpr uint32_t kScanReplay = kScanNumericNaN | kScanCatOrder | kScanCatNaN;
// ScanBest::flags of a node's winner that the fixed-point sums cannot
// certify: a rival candidate (another partition of the node's rows) scores
// within the error bound of the winner, or the winner's loss is within the
// bound of a validity threshold (0, kRtEps, gamma). The bound covers the
// quantisation of every row's pair, the reference's f64 chain rounding and
// the f32 roundings of the score; nodes whose sums are exact never carry it.
constexpr uint32_t kScanNearTie = 32u;

// Best candidate of one feature (or of one node after the merge).
struct ScanBest {
    float loss;              // -inf: none
    uint32_t feature;
    uint32_t index;          // candidate order within the feature
    uint32_t flags;          // bit0 backward (categorical: missing values go left), bit2
                             // (kScanCategorical) a categorical split: `left` is its set's child;
                             // kScanReplay bits
    QBin left;
    QBin right;
    float err;               // the candidate's score error bound (0 without the guard)
    float rival;             // feature records: the highest score + error bound of the feature's
                             // other partitions (-inf: none); node records: of the node's rivals
};

// A near tie resolved on the device: the node's split search over its
// histogram in the CPU builder's f64 sums (hbr_hist_exact), candidate for
// candidate as the reference's host search scans (forward prefix in bin
// order, the backward pass when the bins miss some of the node's total),
// keeping the first best per feature and the lowest feature among equals.
struct ExactBest {
    float loss;              // 0 with no candidate (index 0xffffffff)
    uint32_t feature;
    uint32_t index;          // the fixed-point scan's candidate order (forward, then backward)
    uint32_t flags;          // bit0 backward; kScanNumericNaN
    double lg, lh, rg, rh;   // the winner's children (f64, the CPU's sums)
    QBin left, right;        // the same partition's fixed-point sums
};

struct ExactScanArgs {
    const double *hist;      // 2 x total_bins, g and h interleaved
    const QBin *fixed;       // the node's fixed-point bins (its slot)
    const uint32_t *feature_offset;
    uint32_t n_cols;
    uint32_t dense;          // forward pass only
    double total_g, total_h; // the node's statistics as the caller holds them
    QBin total_fixed;
    float lower, upper;
    ScanParams reg;
    const int8_t *monotone;  // per feature or null
    ExactBest *per_feature;  // n_cols records
    ExactBest *best;         // one record
};

struct ScanArgs {
    const ScanNode *nodes;
    uint32_t n_nodes;
    uint32_t n_features;
    const PartSplit *splits;
    const PartOut *part_out;
    const QBin *hist;
    uint32_t total_bins;
    const uint32_t *feature_offset;
    const int8_t *monotone;  // per feature or null
    const QScale *scale;
    ScanParams reg;
    uint32_t dense;          // index without missing values: forward pass only
    float gamma;             // the split validity threshold (with kRtEps) the guard checks against
    ScanBest *per_feature;   // n_nodes * n_features
    ScanBest *best;          // n_nodes
    QBin *root_total;        // nodes flagged kScanDeviceRoot: their total (read, or written when dense)
    const GrowCounts *grow;  // non-null: nodes = 2 x its n_splits (the grid covers the most)
    // categorical features: per feature its rank among them (0xffffffff:
    // numeric), their count, each (node, categorical feature)'s best set and
    // each node's winning set (kCatWords words each), or null without any
    const uint32_t *cat_rank;
    const uint32_t *cat_feature;  // the feature of each rank
    uint32_t n_cat;
    uint32_t guard;          // 1: bound each candidate's error and flag near ties (kScanNearTie)
    uint32_t *cat_sets;
    uint32_t *best_sets;
};

// ScanNode.pad flag: the node's total is on the device and its root gain is
// computed there from it (the unconstrained root). On a dense index every
// row has one bin per feature, so each feature's bins sum to the total: the
// scan sums them itself and the feature-0 wave stores the sum in
// *root_total; otherwise *root_total holds the total already.
constexpr uint32_t kScanDeviceRoot = 1;
constexpr uint32_t kScanClassShift = 8;

// Per-tree quantisation exponents from the folded maxima, on the device,
// after the rows a deferring kernel listed (grad.scalar_list, when not
// null) have their scalar-sigmoid pairs and are folded in.
struct FinishArgs {
    QScale *scale;
    uint64_t n_rows;
    GradArgs grad;
    // Non-zero: the exponents come from these magnitudes (f32 bits), bounds
    // the pairs cannot exceed (the unit-weight logistic loss: |g| <= 1,
    // h <= 1/4), rather than from the folded maxima, so that a kernel can
    // quantise the pairs as it computes them. The larger of the two is taken
    // should a maximum ever exceed its bound.
    uint32_t bound_g_bits;
    uint32_t bound_h_bits;
};

// Every class's exponents from its folded maxima, in place (one thread per class).
struct ScalesArgs {
    QScale *scales;
    uint32_t k;
    uint64_t n_rows;
};

// to = from with the exponents of n_rows rows (one thread): one class's
// folded softmax maxima become the live scale.
struct SelectArgs {
    const QScale *from;
    QScale *to;
    uint64_t n_rows;
};

// saved = live, then live cleared for the next fold (one thread).
struct RotateArgs {
    QScale *live;
    QScale *saved;
};

// ---- depthwise growth on the device -------------------------------------------------
// A frontier node: statistics, monotone bounds and tree node id. Its rows
// and slot come from the split that made it (child j & 1 of split j >> 1 of
// the previous level; the root's are the identity run and root_slot).
struct GrowNode {
    QBin total;
    double lower, upper;
    uint32_t nid;           // id within its tree
    uint32_t tree;          // tree of a batched level
    uint32_t pad[2];
};

// One node of the device-grown tree; the right child is left + 1.
struct GrowTreeNode {
    int32_t left;           // -1: leaf
    uint32_t feature;
    uint32_t limit;         // present local bins below go left
    int32_t bin;            // global bin boundary (bins <= bin go left), -1 below every bin, -2 leaf
    uint32_t default_left;
    float value;            // leaf: final (eta-scaled) value; else the node's bounded weight
    float sum_hess;
    float gain;
};

// A finished device tree as it is read back: the scale its gradients were
// quantized with and its counts (written by the last level's decision),
// followed by its nodes.
struct TreeHeader {
    QScale scale;
    GrowCounts counts;
};
constexpr uint32_t kTreeHeaderBytes = 128;
static_assert(sizeof(TreeHeader) <= kTreeHeaderBytes, "tree header");

// The decision of one level: every frontier node's winner becomes a split
// (children appended to the tree, partition/histogram/scan records of the
// level written) or a leaf (final value written).
struct GrowArgs {
    GrowCounts *counts;
    const GrowNode *front;        // this level's frontier (level > 0)
    GrowNode *next;               // the children (non-terminal levels)
    const PartSplit *prev_splits; // the previous level's splits and their partition results
    const PartOut *prev_out;
    const ScanBest *best;         // the frontier's winners
    const QBin *root_total;       // level 0
    const QScale *scale;
    PartSplit *splits;            // this level's splits, built children and children's scan nodes
    HistNode *hnodes;
    ScanNode *snodes;
    uint32_t *tile_split;         // the split owning each of the level's partition tiles
    GrowTreeNode *tree;
    TreeHeader *header;           // written by the last level (terminal) with the final counts
    const uint32_t *feature_offset;
    const int8_t *monotone;       // per feature, or null
    uint32_t n_monotone;
    uint32_t level;
    uint32_t terminal;            // the children are at the depth limit (leaves)
    uint32_t n_rows;
    uint32_t root_slot;
    uint32_t slot_cap;            // histogram slots the tree may use: [0, slot_cap)
    ScanParams reg;
    double gamma;
    float eta;
    uint32_t front_cap;           // the most frontier nodes this level can have (records read ahead)
    uint32_t n_features;
    // A batched level grows n_trees trees at once (level 0: their roots, root
    // t in slot root_slot + t with root_total[t], best[t], scale[t]); tree t's
    // header and nodes sit tree_bytes after tree t - 1's, and tree_nodes[t]
    // counts its nodes. The frontier is in tree order.
    uint32_t n_trees;
    uint32_t tree_bytes;
    uint32_t *tree_nodes;
};

// Most slots a device-grown tree may hold (the LDS free-slot table).
constexpr uint32_t kGrowMaxSlots = 4096;
// Most trees a batched level may hold.
constexpr uint32_t kGrowMaxTrees = 256;

// ---- leaves -----------------------------------------------------------------------
struct LeafSeg {
    Seg seg;
    float value;
    uint32_t pad[3];
};

struct LeafArgs {
    const LeafSeg *leaves;
    const uint32_t *tile_leaf;   // tile -> leaf
    const uint32_t *tile_row0;
    const uint32_t *rows[2];
    float *margins;
    uint32_t stride;             // outputs per row
    uint32_t output;
    uint32_t tile_rows;
    uint32_t n_tiles;
};

// A grown tree routed over the binned rows: node meta is feature (bits
// 0-14) | default_left << 15 | limit << 16 | leaf << 31 (present local bins
// below `limit` go left, a missing value the default way), left child
// absolute with the right child at left + 1, leaf values as f32.
constexpr uint32_t kMetaDefaultLeft = 1u << 15;
struct WalkArgs {
    const uint32_t *meta;
    const uint32_t *left;
    const float *value;
    const uint8_t *bins8;        // dense row-major local bins [n][stride]
    float *margins;
    uint32_t stride;
    uint32_t n;
    uint32_t m_stride;           // outputs per row
    uint32_t output;
    uint32_t n_nodes;
    uint32_t guard_n;            // QScale records the guard checks (0 counts as 1)
    // A device-grown tree is read from its records (n_nodes from counts)
    // instead of meta/left/value.
    const GrowTreeNode *tree;
    const GrowCounts *counts;
    // Non-null: the walk (and the gradients) happen only when the gradients
    // the tree was grown from were final (no rows left to the host, none
    // non-finite in any of the guard_n scales: a softmax round's classes)
    // and no earlier guarded walk was skipped; a skip sets *poison, which
    // stays set until the host clears it.
    const QScale *guard;
    uint32_t *poison;
    // Rows carry missing masks (their words from byte mask_at): a masked
    // feature sends the row the way of the node's default (meta bit 15 set:
    // left).
    uint32_t masked;
    uint32_t mask_at;
    // hbr_walk_leaves_batch: trees walked in one pass over the rows; tree c's
    // records and counts sit c * tree_bytes after tree 0's, and its leaves
    // go to output + c.
    uint32_t n_trees;
    uint32_t tree_bytes;
};
// Node tables of all the trees of one batched walk, in LDS.
constexpr uint32_t kBatchWalkNodes = 2048;
constexpr uint32_t kBatchWalkTrees = 64;

// A finished tree added to the margins of an evaluation set by raw value:
// a present value goes left iff value < cut_values[bin] (-FLT_MAX for bin
// -1), a missing one follows default_left.
constexpr uint32_t kEvalLdsNodes = 2048;
constexpr uint32_t kEvalStagedCols = 64;  // hbr_eval_walk_staged: rows of at most this many features
struct EvalWalkArgs {
    const float *x;              // [n][n_cols] row-major
    const GrowTreeNode *tree;    // the tree's records
    const GrowCounts *counts;    // a device-grown tree's node count, or null (n_nodes)
    const float *cut_values;     // global bin -> threshold
    const float *cond;           // per node thresholds (a caller's tree), or null: from the bins
    float *margins;              // [n][m_stride]
    const uint32_t *poison;      // non-null: nothing is added while *poison is set
    uint64_t n;
    uint32_t n_cols;
    uint32_t m_stride;
    uint32_t output;
    uint32_t n_nodes;
    float missing_value;         // the absent marker (NaN: any NaN)
    uint32_t missing_is_nan;
    uint32_t total_bins;         // cut_values' length
    uint32_t pad;
    // Categorical splits (a tree grown on an index with categorical
    // features), or null: node i's categories, which go left, are
    // categories[cat_span[2 i], cat_span[2 i + 1] & 0x7fffffff), bit 31 of
    // cat_span[2 i + 1] marking the split categorical; a present value goes
    // left iff its category (the saturating cast) is among them.
    const uint32_t *cat_span;
    const uint32_t *categories;
};

// Rows reordered by a device-grown tree's leaves (the whole-round trainer
// on 32-byte rows, so that the rows of later trees' nodes, which follow
// much the same splits, sit together in memory): each row's leaf and the
// leaves' row counts, their starts, then each row's new position
// (perm[position] = the original row); the row-indexed arrays are then
// gathered through perm (and back through its inverse).
constexpr uint32_t kOrderMaxNodes = 1024;
struct OrderArgs {
    WalkArgs w;                 // the tree (its records and counts) and the 32-byte rows
    uint32_t *leaf;             // [n] each row's leaf
    uint32_t *count;            // [kOrderMaxNodes] rows per leaf
    uint32_t *cursor;           // [kOrderMaxNodes] the scan: each leaf's next free position
    uint32_t *perm;             // [n] position -> original row
};
struct GatherArgs {
    const uint32_t *index;      // [n] position -> source row
    const uint8_t *src8;        // records (row_bytes each) or columns ([n_cols][n] bytes)
    uint8_t *dst8;
    const float *src32;         // k values per row
    float *dst32;
    uint64_t n;
    uint32_t row_bytes;         // a multiple of 16
    uint32_t n_cols;
    uint32_t k;
    uint32_t pad;
};

// The margin walk of a finished tree followed, row by row, by the next
// round's gradients of the updated margin (the gradient kernel's arithmetic
// and max fold; w.margins and g.margins are the same array).
struct WalkGradArgs {
    WalkArgs w;
    GradArgs g;
    // hbr_walk_grad_root: the next tree's root histogram from the pairs the
    // walk computes, quantised with these exponents (the bounds' exponents
    // hbr_finish_scale will set), one partial of kRootTile bins per
    // workgroup (feature-major: [f][256]); rows the walk defers are left to
    // hbr_root_fixup.
    QBin *root_partial;
    int32_t root_exp_g;
    int32_t root_exp_h;
    uint32_t n_cols;
    uint32_t pad;
};

// The bins of one root partial: 32 features of 256 bins (the dense
// histogram kernel's fg32 layout, one feature group).
constexpr uint32_t kRootFeatures = 32;
constexpr uint32_t kRootTile = kRootFeatures * 256;

// The root after hbr_walk_grad_root: the deferred rows' histogram into one
// more partial (after the walk's n_walk_tiles), and the root's node record
// for hbr_hist_reduce (n_tiles = n_walk_tiles + 1 from partial 0).
struct RootFixupArgs {
    const QScale *scale;        // the finished scale: deferred rows and exponents
    const uint32_t *listed;     // the deferred rows (GradArgs::scalar_list)
    const uint8_t *bins8;       // rows of 32 bytes: 28 bins (or fewer) and the pair word
    QBin *partial;
    HistNode *node;
    uint32_t n_walk_tiles;
    uint32_t n_cols;
    float min_hess;
    uint32_t regroup_tile;  // 1: hbr_regroup wrote partial n_walk_tiles + 1 (rows held reordered)
};

// After a fused walk over reordered rows (GradArgs::perm): every row of a
// marked original vector that took the vector path goes to the scalar list
// for hbr_finish_scale; with root_partial, its vector pair (unit weight, as
// hbr_walk_grad_root summed it) is subtracted into partial n_walk_tiles + 1
// (written whole every time). One workgroup; clears bad_groups[0].
struct RegroupArgs {
    GradArgs g;
    const uint32_t *perm_inv;   // [n] original row -> position
    const uint8_t *bins8;       // rows of 32 bytes (root_partial only)
    QBin *root_partial;         // null: no root histogram to correct
    int32_t root_exp_g;
    int32_t root_exp_h;
    uint32_t n_walk_tiles;
    uint32_t n_cols;
};

// ---- prediction ---------------------------------------------------------------------
// Forest nodes are structure-of-arrays: value (threshold or leaf value bits),
// meta (feature | default_left << 30 | leaf << 31), left child (absolute
// index; the right child is left + 1, as the reference's trees allocate them).
// One forest node as the staged prediction kernel reads it (one 16-byte load).
struct PredNode {
    uint32_t value;               // threshold or leaf value (f32 bits)
    uint32_t meta;                // feature | default_left << 30 | leaf << 31
    uint32_t left;                // left child (absolute), right = left + 1
    int32_t orig;                 // the node's id in its tree as the caller numbered it
};

// A compact forest node: value bits, then feature (16 bits), the left
// child's offset from this node (14 bits; right = left + 1), default_left,
// leaf.
struct alignas(8) CompactNode {
    uint32_t value;
    uint32_t meta;
};

// LDS words per feature of a staged 64-row block (feature-major): lane l
// reads row l of every feature from bank l, whatever the feature.
constexpr uint32_t kPredPitch = 64;

// Two levels of a complete tree (PredictArgs::pairs).
struct alignas(16) PairRecord {
    uint32_t t_node, t_first, t_second;
    uint32_t s;  // slots and m bits of the node and its children (PredictArgs::pairs)
};

// A node of the mirror walk (PredictArgs::mirror).
struct alignas(8) MirrorNode {
    uint32_t t;  // threshold bits (a leaf: its value's)
    uint32_t w;  // m << 31 | rel << 16 | slot
};

struct PredictArgs {
    const PredNode *nodes;
    const uint32_t *node_value;   // f32 bits
    const uint32_t *node_meta;    // feature | categorical<<29 | default_left<<30 | leaf<<31
    const uint32_t *node_left;    // left child (absolute), right = left + 1
    const int32_t *node_orig;     // the node's id in its tree as the caller numbered it
    const uint32_t *tree_root;    // n_trees
    const float *tree_weight;
    const uint32_t *tree_output;
    const float *base_score;
    const float *init;            // n x n_outputs starting margins, or null: base_score
    const float *x;               // n x n_cols row-major
    float *out;                   // n x n_outputs
    int32_t *leaf_out;            // n x n_trees or null
    uint32_t n;
    uint32_t n_cols;
    uint32_t n_trees;
    uint32_t n_outputs;
    float missing;
    uint32_t missing_is_nan;
    uint32_t trees_per_chunk;
    uint32_t pad;
    // tree chunks for hbr_predict_chunked: chunk c holds trees
    // [chunk_tree[c], chunk_tree[c + 1]) whose nodes are the compact records
    // [chunk_node[c], chunk_node[c + 1]) of `compact`
    const CompactNode *compact;      // (value bits, feature | rel_left << 16 | dl << 30 | leaf << 31)
    const uint32_t *chunk_tree;   // n_chunks + 1
    const uint32_t *chunk_node;   // n_chunks + 1
    uint32_t n_chunks;
    uint32_t chunk_cap;           // LDS node capacity
    // categorical splits (hbr_predict only): a node with kPredCategorical in
    // its meta holds cat_begin as its value; its set is
    // categories[value, node_cat_end[node])
    const uint32_t *categories;
    const uint32_t *node_cat_end;
    // The forest as branch-free steps (hbr_predict_mirror*): each tree
    // breadth-first with the child a missing value takes first and its
    // sibling next to it. A node is (bits of t, m << 31 | rel << 16 | slot):
    // a row steps to first + 1 when (value, its sign flipped when m) < t,
    // else to first = this node + rel; slot is the feature + 1. A split
    // whose missing values go right has m = 0 and t its threshold (first =
    // the right child: NaN compares false); one whose missing values go left
    // has m = 1 and t = -next_below(threshold) (first = the left child: -v <
    // t is v >= threshold). A leaf is (bits of its value, 0): it steps to
    // itself, reading slot 0, where every row holds NaN. Rows are staged
    // with feature f in slot f + 1 and, when the missing value is not NaN,
    // missing values as NaN and present NaNs as +inf (which go right, as a
    // NaN compared with a threshold does).
    const MirrorNode *mirror;
    const uint32_t *mirror_root;   // n_trees
    const int32_t *mirror_orig;    // per node: its id in its tree as the caller numbered it
    const uint8_t *tree_depth;     // n_trees
    uint32_t pair_levels;          // hbr_predict_pairs: D / 2 (every tree a complete tree of depth D)
    uint32_t pad2;
    // The forest as complete trees of even depth D, two levels per record
    // (hbr_predict_pairs): a tree's records level by level (1, 4, 16, ...
    // records: (4^(D/2) - 1) / 3 per tree), the record of the node at
    // position i of level 2l followed by the value of each of its 2^D level-D
    // positions. A record is (t of the node, t of its first child, t of its
    // second child, s) with t as in the mirror walk; s holds each of the
    // three nodes' slot and m (the node's slot at bits 8..14 and m at bit 31,
    // the first child's at bits 16..22 and 7, the second's at bits 0..6 and
    // 23): a row steps to the second child when (value of slot, its sign
    // flipped when m) < t.
    // The first child is where a missing value goes. A leaf above level D
    // is continued by nodes that read slot 0 (NaN) and so always take their
    // first child, down to its position at level D, which holds its value.
    const PairRecord *pairs;
    const uint32_t *pair_values;   // n_trees x 2^D leaf values (bits)
    const int32_t *pair_orig;      // n_trees x 2^D: the caller's id of the leaf each position holds
};
constexpr uint32_t kPredCategorical = 1u << 29;

}  // namespace hbr
