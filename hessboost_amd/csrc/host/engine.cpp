#include "engine.h"

#include "split_math.h"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <limits>

namespace hbr {

namespace {

constexpr uint32_t kLeafTile = 4096;

uint32_t ceil_div(uint64_t a, uint64_t b) { return (uint32_t)((a + b - 1) / b); }

// Quantization exponent for a maximum magnitude (f32 bits) over `rows` rows:
// with M = m 2^e (m in [0.5, 1)), exp = e + ceil(log2 rows) - 62 keeps every
// sum of the tree's quantized values within 2^62.
int32_t exp_for(uint32_t bits, uint64_t rows) {
    if (bits == 0 || bits >= 0x7f800000u) return 0;
    float m;
    std::memcpy(&m, &bits, 4);
    int e = 0;
    std::frexp(m, &e);
    int log_n = rows > 1 ? 64 - __builtin_clzll(rows - 1) : 0;
    return e + log_n - 62;
}

uint32_t abs_bits(float x) {
    uint32_t b;
    std::memcpy(&b, &x, 4);
    return b & 0x7fffffffu;
}

// The reference's scalar logistic gradient (simd/scalar.rs:8-29 with
// simd/mod.rs:425-427), for the rows its vector kernel leaves to libm.

}  // namespace

Engine::Engine(int ordinal, const hbr_index_desc &desc) : dev_(device(ordinal)) {
    read_tunables();
    upload_index(desc);
    block_.resize(kBlockBytes);
    build_csr_ranges();
}

Engine::Engine(int ordinal, const DenseSource &src) : dev_(device(ordinal)) {
    read_tunables();
    bin_dense(src);
    block_.resize(kBlockBytes);
    build_csr_ranges();
}

// Launch-shape overrides for tuning sweeps (results do not depend on them).
void Engine::read_tunables() {
    if (const char *v = std::getenv("HBROCM_HIST_FG")) {
        const long fg = std::strtol(v, nullptr, 10);
        if (fg == 8 || fg == 16 || fg == 32) hist_features_per_group = (uint32_t)fg;
    }
    if (const char *v = std::getenv("HBROCM_HIST_THREADS")) {
        const long t = std::strtol(v, nullptr, 10);
        if (t == 512 || t == 1024) hist_threads = (uint32_t)t;
    }
    if (const char *v = std::getenv("HBROCM_HIST_BIN_MAJOR")) hist_bin_major = std::strtol(v, nullptr, 10) != 0;
    if (const char *v = std::getenv("HBROCM_HIST_NF28")) hist_nf28 = std::strtol(v, nullptr, 10) != 0;
    if (const char *v = std::getenv("HBROCM_ROW_PAIRS")) row_pairs = std::strtol(v, nullptr, 10) != 0;
    if (const char *v = std::getenv("HBROCM_FUSED_ROOT")) fused_root = std::strtol(v, nullptr, 10) != 0;
    if (const char *v = std::getenv("HBROCM_MASKED_ROWS")) masked_rows = std::strtol(v, nullptr, 10) != 0;
    if (const char *v = std::getenv("HBROCM_WIDE_ROWS")) wide_rows = std::strtol(v, nullptr, 10) != 0;
    if (const char *v = std::getenv("HBROCM_ROW_ORDER")) row_order = std::strtol(v, nullptr, 10) != 0;
    if (const char *v = std::getenv("HBROCM_ROW_ORDER_MIN_ROWS")) row_order_min_rows = std::strtoull(v, nullptr, 10);
    if (const char *v = std::getenv("HBROCM_ROW_ORDER_EVERY")) row_order_every = std::strtoull(v, nullptr, 10);
    if (const char *v = std::getenv("HBROCM_BATCH_WALK")) batch_walk = std::strtol(v, nullptr, 10) != 0;
    if (const char *v = std::getenv("HBROCM_BIN_ROWS_IN_REGISTERS")) bin_rows_in_registers = std::strtol(v, nullptr, 10) != 0;
    if (const char *v = std::getenv("HBROCM_DEVICE_GROW")) device_grow = std::strtol(v, nullptr, 10) != 0;
    if (const char *v = std::getenv("HBROCM_CSR_RANGES")) csr_range_table = std::strtol(v, nullptr, 10) != 0;
    if (const char *v = std::getenv("HBROCM_WALK_BLOCKS")) {
        const long b = std::strtol(v, nullptr, 10);
        if (b >= 1 && b <= 64) walk_blocks_per_cu = (uint32_t)b;
    }
    if (const char *v = std::getenv("HBROCM_HIST_WAVES")) {
        const long w = std::strtol(v, nullptr, 10);
        if (w >= 1 && w <= 64) hist_waves = (uint32_t)w;
    }
}

Engine::~Engine() {
    try {
        dev_.activate();
        dev_.sync();
        if (copy_stream_) {
            (void)hipStreamSynchronize(copy_stream_);
            for (uint32_t r = 0; r < kTreeRing; r++) {
                (void)hipEventDestroy(tree_ready_[r]);
                (void)hipEventDestroy(tree_copied_[r]);
            }
            (void)hipStreamDestroy(copy_stream_);
        }
    } catch (...) {
    }
}

void Engine::upload_index(const hbr_index_desc &d) {
    if (!d.feature_offset || !d.row_ptr || (!d.row_bins && d.row_ptr[d.n_rows] > 0))
        fail(kInvalid, "index: feature_offset, row_ptr and row_bins are required");
    if (d.n_rows >= (uint64_t)UINT32_MAX) fail(kRefused, "index: more than 2^32 - 1 rows");
    if (d.row_bin_width != 2 && d.row_bin_width != 4) fail(kInvalid, "index: row_bin_width must be 2 or 4");
    n_rows_ = d.n_rows;
    n_cols_ = (uint32_t)d.n_cols;
    fo_.assign(d.feature_offset, d.feature_offset + n_cols_ + 1);
    total_bins_ = fo_[n_cols_];
    if (d.cut_values) cuts_.assign(d.cut_values, d.cut_values + total_bins_);
    dense_ = d.dense != 0;
    entries_ = d.row_ptr[n_rows_];
    uint32_t widest = 0;
    for (uint32_t f = 0; f < n_cols_; f++) widest = std::max(widest, fo_[f + 1] - fo_[f]);
    hipStream_t s = dev_.stream();
    d_fo_.resize(n_cols_ + 1);
    d_fo_.upload(fo_.data(), n_cols_ + 1, s);
    words_ = (uint32_t)((n_rows_ + 63) / 64);
    if (d.is_categorical) {
        cat_rank_.assign(n_cols_, 0xffffffffu);
        for (uint32_t f = 0; f < n_cols_; f++) {
            if (!d.is_categorical[f]) continue;
            if (fo_[f + 1] - fo_[f] > kCatMaxBins) fail(kRefused, "index: a categorical feature beyond 1,024 categories");
            cat_rank_[f] = (uint32_t)cat_feature_.size();
            cat_feature_.push_back(f);
        }
        n_cat_ = (uint32_t)cat_feature_.size();
        if (n_cat_) {
            d_cat_rank_.resize(n_cols_);
            d_cat_rank_.upload(cat_rank_.data(), n_cols_, s);
            d_cat_feature_.resize(n_cat_);
            d_cat_feature_.upload(cat_feature_.data(), n_cat_, s);
            d_root_set_.resize(kCatWords);
        } else {
            cat_rank_.clear();
        }
    }

    if (dense_ && widest <= 256 && n_cols_ > 0) {
        dense_u8_ = true;
        have_cols_ = true;
        // a whole number of the widest feature group (32 bytes), so that a
        // group's load never crosses past the row's end
        stride_ = (n_cols_ + 31) / 32 * 32;
        rows8_.resize(n_rows_ * stride_);
        rows8_.zero(s);
        cols8_.resize(n_rows_ * n_cols_);
        // re-encode in chunks of rows, each chunk's global bins staged once
        const uint64_t chunk = std::max<uint64_t>(1, (64ull << 20) / (n_cols_ * (uint64_t)d.row_bin_width));
        DBuf<uint8_t> staging(chunk * n_cols_ * d.row_bin_width);
        for (uint64_t r0 = 0; r0 < n_rows_; r0 += chunk) {
            const uint64_t rows = std::min<uint64_t>(chunk, n_rows_ - r0);
            const size_t bytes = rows * n_cols_ * d.row_bin_width;
            const char *src = static_cast<const char *>(d.row_bins) + r0 * n_cols_ * d.row_bin_width;
            HBR_HIP(hipMemcpyAsync(staging.get(), src, bytes, hipMemcpyHostToDevice, s));
            EncodeArgs a{};
            a.g16 = d.row_bin_width == 2 ? (const uint16_t *)staging.get() : nullptr;
            a.g32 = d.row_bin_width == 4 ? (const uint32_t *)staging.get() : nullptr;
            a.feature_offset = d_fo_.get();
            a.rows8 = rows8_.get();
            a.cols8 = cols8_.get();
            a.n_rows = n_rows_;
            a.row0 = r0;
            a.chunk_rows = (uint32_t)rows;
            a.n_cols = n_cols_;
            a.stride = stride_;
            const uint64_t cells = rows * n_cols_;
            dev_.launch("hbr_encode_dense", dim3(std::min<uint64_t>(ceil_div(cells, 256), 65535)), dim3(256), a);
            dev_.sync();
        }
        return;
    }
    // CSR rows for histograms (global bins widened to u32).
    const uint64_t nnz = d.row_ptr[n_rows_];
    row_ptr_.resize(n_rows_ + 1);
    row_ptr_.upload(d.row_ptr, n_rows_ + 1, s);
    gbins_.resize(nnz ? nnz : 1);
    // whether every row's global bins ascend (entries in feature order)
    csr_ascending_ = true;
    for (uint64_t r = 0; r < n_rows_ && csr_ascending_; r++)
        for (uint64_t e = d.row_ptr[r] + 1; e < d.row_ptr[r + 1]; e++) {
            const uint32_t prev = d.row_bin_width == 4 ? static_cast<const uint32_t *>(d.row_bins)[e - 1]
                                                        : static_cast<const uint16_t *>(d.row_bins)[e - 1];
            const uint32_t cur = d.row_bin_width == 4 ? static_cast<const uint32_t *>(d.row_bins)[e]
                                                       : static_cast<const uint16_t *>(d.row_bins)[e];
            if (cur <= prev) {
                csr_ascending_ = false;
                break;
            }
        }
    if (d.row_bin_width == 4) {
        gbins_.upload(static_cast<const uint32_t *>(d.row_bins), nnz, s);
    } else {
        const uint16_t *g16 = static_cast<const uint16_t *>(d.row_bins);
        const uint64_t chunk = 1ull << 24;
        std::vector<uint32_t> wide;
        for (uint64_t e0 = 0; e0 < nnz; e0 += chunk) {
            const uint64_t m = std::min(chunk, nnz - e0);
            wide.assign(g16 + e0, g16 + e0 + m);
            gbins_.upload(wide.data(), m, s, e0);
            dev_.sync();
        }
    }
    // feature-major columns route rows when the index keeps them
    if (d.col_bins && (d.col_bin_width == 1 || d.col_bin_width == 2)) {
        have_cols_ = true;
        const uint64_t cells = n_rows_ * n_cols_;
        if (d.col_bin_width == 1) {
            cols8_.resize(cells ? cells : 1);
            cols8_.upload(static_cast<const uint8_t *>(d.col_bins), cells, s);
        } else {
            cols16_.resize(cells ? cells : 1);
            cols16_.upload(static_cast<const uint16_t *>(d.col_bins), cells, s);
        }
        if (d.missing) {
            missing_.resize((uint64_t)words_ * n_cols_);
            missing_.upload(d.missing, (uint64_t)words_ * n_cols_, s);
        }
        make_masked_rows();
    }
    // (every row holds n_cols entries in feature order)
    if (wide_rows && dense_ && !dense_u8_ && widest <= kWideBinsMax && n_cols_ > 0 && csr_ascending_ &&
        entries_ == n_rows_ * n_cols_)
        make_rows16(widest);
    dev_.sync();
}

// A dense index whose widest feature has more than 256 bins: its global
// bins (the dense CSR rows, n_cols entries a row in feature order) to rows
// of u16 local bins, 16 elements (32 bytes) a row at least; a histogram
// workgroup then holds fg16_ features of kWideLdsBins / fg16_ bins each.
void Engine::make_rows16(uint32_t widest) {
    uint32_t bins = 512;
    while (bins < widest) bins *= 2;
    fg16_ = std::min<uint32_t>(16, kWideLdsBins / bins);
    stride16_ = (n_cols_ + 15) / 16 * 16;
    rows16_.resize(n_rows_ * stride16_);
    Encode16Args a{gbins_.get(), d_fo_.get(), rows16_.get(), n_rows_, n_cols_, stride16_};
    const uint64_t cells = n_rows_ * stride16_;
    dev_.launch("hbr_encode_dense16", dim3((uint32_t)std::min<uint64_t>(ceil_div(cells, 256), 65535)), dim3(256), a);
    dense16_ = true;
}

// A matrix with missing values and at most kMaskedWideMaxFeatures features
// keeps dense u8 rows with missing masks beside its CSR rows: the histogram
// kernel and the margin walks take them, the partition its columns and
// bitmap. Up to kMaskedMaxFeatures features a row is 32 bytes with its mask
// in the last word; wider, the bins of G groups of 32 features and then a
// 32-byte chunk of G mask words (32 G + 32 bytes).
void Engine::make_masked_rows() {
    if (dense_ || !masked_rows || !cols8_.size() || n_cols_ == 0 || n_cols_ > kMaskedWideMaxFeatures) return;
    for (uint32_t f = 0; f < n_cols_; f++)
        if (fo_[f + 1] - fo_[f] > 256) return;
    const uint32_t groups = ceil_div(n_cols_, 32u);
    const bool compact = n_cols_ <= kMaskedMaxFeatures;
    stride_ = compact ? 32 : 32 * groups + 32;
    mask_at_ = compact ? 4 * kMaskWord : 32 * groups;
    rows8_.release();
    rows8_.resize(n_rows_ * stride_);
    RowsFromColsArgs a{cols8_.get(), missing_.size() ? missing_.get() : nullptr, rows8_.get(), n_rows_, n_cols_,
                       words_, stride_, mask_at_};
    dev_.launch("hbr_rows_from_cols", dim3(ceil_div(n_rows_, 256)), dim3(256), a);
    dense_u8_ = true;
    masked_ = true;
}

// The index binned on the device: one pass over the matrix writes the local
// columns, the missing bitmap, each row's present count and (speculatively)
// the row-major u8 rows. A matrix without absent cells is then the dense u8
// index; otherwise the counts are scanned into row_ptr and the CSR global
// bins are filled from the columns, and the columns and bitmap are kept when
// cells <= 2 x entries (src/data/ghist.rs:235), as on the host.
// Sparse rows in feature order: each row's first entry of every bin range
// of the CSR histogram, so that a range's workgroups read only its entries
// (when the table takes at most 1 GiB).
void Engine::build_csr_ranges() {
    csr_ranges_.release();
    if (!csr_range_table || dense_u8_ || dense16_ || !csr_ascending_ || n_rows_ == 0) return;
    const uint32_t groups = ceil_div(total_bins_, kCsrGroupBins);
    const uint64_t words = n_rows_ * (uint64_t)(groups + 1);
    if (groups < 2 || words * sizeof(uint32_t) > (uint64_t(1) << 30)) return;
    csr_ranges_.resize(words);
    CsrRangeArgs a{row_ptr_.get(), gbins_.get(), csr_ranges_.get(), (uint32_t)n_rows_, groups};
    dev_.launch("hbr_csr_ranges", dim3(ceil_div(n_rows_, 256)), dim3(256), a);
    dev_.sync();
}

void Engine::bin_dense(const DenseSource &src) {
    if (!src.x || !src.feature_offset || (!src.cut_values && src.feature_offset[src.n_cols] > 0))
        fail(kInvalid, "binning: x, feature_offset and cut_values are required");
    if (src.n_rows == 0 || src.n_cols == 0) fail(kInvalid, "binning: an empty matrix");
    if (src.n_rows >= (uint64_t)UINT32_MAX) fail(kRefused, "binning: more than 2^32 - 1 rows");
    n_rows_ = src.n_rows;
    n_cols_ = (uint32_t)src.n_cols;
    fo_.assign(src.feature_offset, src.feature_offset + n_cols_ + 1);
    total_bins_ = fo_[n_cols_];
    cuts_.assign(src.cut_values, src.cut_values + total_bins_);
    for (uint32_t f = 0; f < n_cols_; f++) {
        const uint32_t nb = fo_[f + 1] - fo_[f];
        if (fo_[f + 1] < fo_[f]) fail(kInvalid, "binning: feature_offset must not decrease");
        if (nb == 0) fail(kInvalid, "binning: a feature without bins");
        if (nb > 256) fail(kRefused, "binning on the device: a feature with more than 256 bins");
    }
    hipStream_t s = dev_.stream();
    d_fo_.resize(n_cols_ + 1);
    d_fo_.upload(fo_.data(), n_cols_ + 1, s);
    DBuf<float> d_cuts(total_bins_);
    d_cuts.upload(cuts_.data(), total_bins_, s);
    words_ = (uint32_t)((n_rows_ + 63) / 64);
    stride_ = (n_cols_ + 31) / 32 * 32;
    rows8_.resize(n_rows_ * stride_);
    // up to 32 features: rows read with 16-byte loads (into registers, or
    // staged through LDS when n_cols is not a multiple of 4), every 32-byte
    // row written whole
    const bool wide32 = stride_ == 32 && total_bins_ <= kBinLdsCuts &&
                        (!src.on_device || reinterpret_cast<uintptr_t>(src.x) % 16 == 0);
    const bool in_regs = wide32 && n_cols_ % 4 == 0 && bin_rows_in_registers;
    if (!wide32) rows8_.zero(s);
    cols8_.resize(n_rows_ * n_cols_);
    missing_.resize((uint64_t)words_ * n_cols_);
    DBuf<uint32_t> count(n_rows_);
    // chunks of whole 64-row groups; host rows beyond two chunks go through
    // the device's pinned staging (Device::host_rows: the binning of a chunk
    // runs while the next is staged and copied), fewer through one copy
    const uint64_t row_bytes = n_cols_ * sizeof(float);
    constexpr uint64_t kChunkBytes = 128ull << 20;
    uint64_t chunk = std::max<uint64_t>(64, (kChunkBytes / row_bytes) / 64 * 64);
    if (src.on_device) chunk = std::min<uint64_t>(n_rows_, (uint64_t)UINT32_MAX / 2) / 64 * 64 + 64;
    auto bin_chunk = [&](const float *xs, uint64_t r0, uint64_t rows) {
        BinArgs a{};
        a.x = xs;
        a.cut_values = d_cuts.get();
        a.feature_offset = d_fo_.get();
        a.rows8 = rows8_.get();
        a.cols8 = cols8_.get();
        a.missing = missing_.get();
        a.row_count = count.get();
        a.n_rows = n_rows_;
        a.row0 = r0;
        a.chunk_rows = (uint32_t)rows;
        a.n_cols = n_cols_;
        a.stride = stride_;
        a.words = words_;
        a.total_bins = total_bins_;
        a.missing_value = src.missing;
        a.missing_is_nan = std::isnan(src.missing) ? 1u : 0u;
        a.row_mask = masked_rows && n_cols_ <= kMaskedMaxFeatures && stride_ == 32 ? 1u : 0u;
        if (in_regs)
            dev_.launch("hbr_bin_dense32_rows", dim3(ceil_div(rows, 256)), dim3(256), a,
                        (uint32_t)(total_bins_ * sizeof(float)));
        else if (wide32)
            dev_.launch("hbr_bin_dense32", dim3(ceil_div(rows, 256)), dim3(256), a,
                        (uint32_t)((4 * 64 * n_cols_ + total_bins_) * sizeof(float)));
        else
            dev_.launch("hbr_bin_dense", dim3(ceil_div(rows, 256)), dim3(256), a);
    };
    if (!src.on_device && n_rows_ * row_bytes >= 2 * kChunkBytes) {
        dev_.host_rows(src.x, n_rows_, n_cols_, chunk, bin_chunk);
    } else if (!src.on_device) {
        DBuf<float> staging(n_rows_ * n_cols_);
        staging.upload(src.x, n_rows_ * n_cols_, s);
        bin_chunk(staging.get(), 0, n_rows_);
        dev_.sync();
    } else {
        for (uint64_t r0 = 0; r0 < n_rows_; r0 += chunk)
            bin_chunk(src.x + r0 * n_cols_, r0, std::min<uint64_t>(chunk, n_rows_ - r0));
    }
    // the present counts: totals per block, their offsets on the host, row_ptr
    const uint32_t blocks = ceil_div(n_rows_, kCountBlock);
    DBuf<uint64_t> block_total(blocks), block_offset(blocks);
    CountScanArgs c{};
    c.row_count = count.get();
    c.block_total = block_total.get();
    c.n_rows = n_rows_;
    dev_.launch("hbr_count_blocks", dim3(blocks), dim3(1024), c);
    std::vector<uint64_t> totals(blocks), offsets(blocks);
    block_total.download(totals.data(), blocks, s);
    dev_.sync();
    uint64_t entries = 0;
    for (uint32_t b = 0; b < blocks; b++) {
        offsets[b] = entries;
        entries += totals[b];
    }
    entries_ = entries;
    const uint64_t cells = n_rows_ * n_cols_;
    dense_ = entries == cells;
    if (dense_) {
        // the dense u8 index: row-major rows for histograms, columns for routing
        dense_u8_ = true;
        have_cols_ = true;
        missing_.release();
        dev_.sync();
        return;
    }
    // missing values: CSR rows and, up to kMaskedWideMaxFeatures features,
    // masked dense rows (those of 32 bytes written by the binning pass, wider
    // ones from the columns once they are complete)
    masked_ = masked_rows && n_cols_ <= kMaskedMaxFeatures && stride_ == 32;
    if (masked_) mask_at_ = 4 * kMaskWord;
    if (!masked_) {
        rows8_.release();
        stride_ = 0;
    }
    block_offset.upload(offsets.data(), blocks, s);
    row_ptr_.resize(n_rows_ + 1);
    c.block_offset = block_offset.get();
    c.row_ptr = row_ptr_.get();
    dev_.launch("hbr_count_offsets", dim3(blocks), dim3(1024), c);
    gbins_.resize(entries ? entries : 1);
    CsrFillArgs g{};
    g.cols8 = cols8_.get();
    g.missing = missing_.get();
    g.feature_offset = d_fo_.get();
    g.row_ptr = row_ptr_.get();
    g.gbins = gbins_.get();
    g.n_rows = n_rows_;
    g.n_cols = n_cols_;
    g.words = words_;
    dev_.launch("hbr_csr_fill", dim3(ceil_div(n_rows_, 256)), dim3(256), g);
    if (!masked_) make_masked_rows();
    dev_.sync();
    if (masked_) {  // the masked rows route by the columns and bitmap
        dense_u8_ = true;
        have_cols_ = true;
    } else if (cells <= 2 * entries) {
        have_cols_ = true;
    } else {
        cols8_.release();
        missing_.release();
    }
}

Engine::IndexInfo Engine::index_info() const {
    IndexInfo i{};
    i.dense = dense_;
    i.dense_u8 = dense_u8_;
    i.has_cols = have_cols_;
    i.has_missing = missing_.size() > 0;
    i.stride = stride_;
    i.entries = dense_ ? n_rows_ * n_cols_ : entries_;
    return i;
}

void Engine::read_index(uint8_t *rows8, uint8_t *cols8, uint64_t *missing, uint64_t *row_ptr, uint32_t *gbins) {
    hipStream_t s = dev_.stream();
    if (rows8 && rows8_.size()) rows8_.download(rows8, rows8_.size(), s);
    if (cols8 && cols8_.size()) cols8_.download(cols8, n_rows_ * n_cols_, s);
    if (missing && missing_.size()) missing_.download(missing, (uint64_t)words_ * n_cols_, s);
    if (row_ptr && row_ptr_.size()) row_ptr_.download(row_ptr, n_rows_ + 1, s);
    if (gbins && !dense_ && gbins_.size()) gbins_.download(gbins, entries_, s);
    dev_.sync();
    // a row's padding bytes read as zero (they may carry logistic pairs);
    // masked rows keep their missing mask
    const uint32_t pad_end = masked_ ? mask_at_ : stride_;
    if (rows8 && rows8_.size() && pad_end > n_cols_)
        for (uint64_t r = 0; r < n_rows_; r++) std::memset(rows8 + r * stride_ + n_cols_, 0, pad_end - n_cols_);
}

// ---- gradients -----------------------------------------------------------------

void Engine::load_margins(const float *m, uint64_t n, uint32_t outputs) {
    if (n != n_rows_ * outputs) fail(kInvalid, "load_margins: length is not n_rows * n_outputs");
    outputs_ = outputs;
    active_pairs_ = nullptr;
    row_pairs_live_ = false;
    root_partials_ = 0;  // the staged pairs are no longer the walk's
    pair_array_stale_ = false;
    class_outputs_ = 0;
    margins_.resize(n);
    margins_.upload(m, n, dev_.stream());
    if (poison_.size()) HBR_HIP(hipMemsetAsync(poison_.get(), 0, sizeof(uint32_t), dev_.stream()));
    labels_loaded_ = false;
    dev_.sync();
}

void Engine::set_labels(const float *labels, const float *weights, uint64_t n) {
    if (n != n_rows_) fail(kInvalid, "labels: one per row");
    labels_.resize(n);
    labels_.upload(labels, n, dev_.stream());
    has_weights_ = weights != nullptr;
    if (weights) {
        weights_.resize(n);
        weights_.upload(weights, n, dev_.stream());
    }
    labels_binary_ = true;
    for (uint64_t i = 0; i < n && labels_binary_; i++) labels_binary_ = labels[i] == 0.0f || labels[i] == 1.0f;
    labels_loaded_ = true;
    dev_.sync();
}

void Engine::read_margins(float *out, uint64_t n) {
    if (n > margins_.size()) fail(kInvalid, "read_margins: longer than the margins");
    if (permuted_ && n) {  // back to the original order on the way out
        DBuf<float> tmp(margins_.size());
        GatherArgs g{};
        g.index = perm_inv_.get();
        g.src32 = margins_.get();
        g.dst32 = tmp.get();
        g.n = n_rows_;
        g.k = outputs_ ? outputs_ : 1u;
        dev_.launch("hbr_gather_f32", dim3((uint32_t)std::min<uint64_t>(ceil_div(n_rows_ * g.k, 256), 65535)),
                    dim3(256), g);
        tmp.download(out, n, dev_.stream());
        dev_.sync();
        return;
    }
    margins_.download(out, n, dev_.stream());
    dev_.sync();
}

// Every row-indexed array to the order `index` gives (position i takes
// row index[i]): gathered into the spare buffers, which then swap with the
// live ones, so that nothing is freed and nothing waits.
void Engine::gather_rows(const uint32_t *index) {
    const uint32_t grid = (uint32_t)std::min<uint64_t>(ceil_div(n_rows_, 256), 65535);
    GatherArgs g{};
    g.index = index;
    g.n = n_rows_;
    Spare &sp = spare_;
    sp.rows.resize(rows8_.size());
    g.src8 = rows8_.get();
    g.dst8 = sp.rows.get();
    g.row_bytes = stride_;
    dev_.launch("hbr_gather_records", dim3(grid), dim3(256), g);
    if (cols8_.size()) {  // rebuilt from the gathered rows, which hold every bin
        sp.cols.resize(cols8_.size());
        GatherArgs c = g;
        c.src8 = sp.rows.get();
        c.dst8 = sp.cols.get();
        c.n_cols = n_cols_;
        dev_.launch("hbr_columns_from_rows", dim3(grid), dim3(256), c);
    }
    auto f32 = [&](const float *src, float *dst, uint32_t k) {
        GatherArgs h = g;
        h.src32 = src;
        h.dst32 = dst;
        h.k = k;
        dev_.launch("hbr_gather_f32", dim3((uint32_t)std::min<uint64_t>(ceil_div(n_rows_ * k, 256), 65535)),
                    dim3(256), h);
    };
    // the staged pair array, when it holds the live pairs (two f32 a row)
    const bool pairs_live = !active_pairs_ && !class_outputs_ && !pair_array_stale_ && gpair_.size() >= n_rows_;
    if (pairs_live) {
        sp.pairs.resize(gpair_.size());
        f32(reinterpret_cast<const float *>(gpair_.get()), reinterpret_cast<float *>(sp.pairs.get()), 2u);
        std::swap(gpair_, sp.pairs);
    }
    auto move = [&](DBuf<float> &live, DBuf<float> &spare, uint32_t k) {
        if (!live.size()) return;
        spare.resize(live.size());
        f32(live.get(), spare.get(), k);
        std::swap(live, spare);
    };
    move(margins_, sp.margins, outputs_ ? outputs_ : 1u);
    move(labels_, sp.labels, 1u);
    if (has_weights_) move(weights_, sp.weights, 1u);
    std::swap(rows8_, sp.rows);
    if (cols8_.size()) std::swap(cols8_, sp.cols);
    // the rows carry their pair words with them; the rows a walk deferred
    // are listed by their old positions, so the next root sums every row
    root_partials_ = 0;
    grains_known_ = false;
}

// The rows by the leaves of the last queued device tree (rows of one leaf
// keep no particular order). Rows already reordered are reordered again
// from where they are, the two orders composed.
void Engine::order_rows_by_tree() {
    if (!dense_ || !dense_u8_ || masked_ || stride_ != 32 || n_cols_ == 0 || n_cols_ > 32 || missing_.size() ||
        cols16_.size() || rows16_.size() || class_outputs_ || n_rows_ < row_order_min_rows ||
        n_rows_ >= (1ull << 32) || last_depth_ > 9 || (2ull << last_depth_) - 1 > kOrderMaxNodes || outputs_ != 1)
        return;
    hipStream_t s = dev_.stream();
    Spare &sp = spare_;
    sp.leaf.resize(n_rows_);
    sp.order.resize(n_rows_);
    sp.count.resize(kOrderMaxNodes);
    sp.cursor.resize(kOrderMaxNodes);
    if (!permuted_) {
        perm_inv_.resize(n_rows_);
        group_stamp_.resize(n_rows_ / 8 + 1);
        bad_groups_.resize(n_rows_ / 8 + 2);
        group_stamp_.zero(s);
        bad_groups_.zero(s);
        regroup_stamp_ = 0;
    }
    sp.count.zero(s);
    OrderArgs o{};
    o.w.tree = ring_nodes(last_ring_, 0, last_stride_);
    o.w.counts = &ring_header(last_ring_, 0, last_stride_)->counts;
    o.w.bins8 = rows8_.get();
    o.w.stride = stride_;
    o.w.n = (uint32_t)n_rows_;
    o.leaf = sp.leaf.get();
    o.count = sp.count.get();
    o.cursor = sp.cursor.get();
    o.perm = sp.order.get();  // new position -> present position
    const uint32_t grid = std::min<uint32_t>(ceil_div(n_rows_, 256), (uint32_t)dev_.cu_count() * 8);
    dev_.launch("hbr_order_leaves", dim3(grid), dim3(256), o);
    dev_.launch("hbr_order_scan", dim3(1), dim3(1024), o);
    dev_.launch("hbr_order_place", dim3(grid), dim3(256), o);
    gather_rows(sp.order.get());
    if (permuted_) {  // new position -> original row: perm_[order[i]]
        GatherArgs c{};
        c.index = sp.order.get();
        c.n = n_rows_;
        c.src32 = reinterpret_cast<const float *>(perm_.get());
        c.dst32 = reinterpret_cast<float *>(sp.leaf.get());  // the leaves are spent
        c.k = 1;
        dev_.launch("hbr_gather_f32", dim3((uint32_t)std::min<uint64_t>(ceil_div(n_rows_, 256), 65535)), dim3(256), c);
        std::swap(perm_, sp.leaf);
    } else {
        std::swap(perm_, sp.order);
    }
    GatherArgs inv{};
    inv.index = perm_.get();
    inv.dst8 = reinterpret_cast<uint8_t *>(perm_inv_.get());
    inv.n = n_rows_;
    dev_.launch("hbr_order_invert", dim3(ceil_div(n_rows_, 256)), dim3(256), inv);
    permuted_ = true;
    counters.row_orders++;
}

void Engine::restore_row_order() {
    if (!permuted_) return;
    gather_rows(perm_inv_.get());
    dev_.sync();
    permuted_ = false;
    perm_.release();
    perm_inv_.release();
    group_stamp_.release();
    bad_groups_.release();
    spare_ = Spare{};
}

void Engine::read_gradients(float *out, uint64_t n) {
    if (pair_array_stale_ && !softmax_staged())
        fail(kRefused, "read_gradients: the last margin walk left its pairs in the rows only");
    if (softmax_staged() && n == n_rows_ * outputs_) {
        class_pairs_.download(reinterpret_cast<GPair *>(out), n, dev_.stream());
    } else {
        if (n != n_rows_ || !pairs_staged()) fail(kInvalid, "read_gradients: nothing staged for every row");
        HBR_HIP(hipMemcpyAsync(out, pairs(), n * sizeof(GPair), hipMemcpyDeviceToHost, dev_.stream()));
    }
    dev_.sync();
}

double Engine::unit_g() const { return std::ldexp(1.0, scale_host_.exp_g); }
double Engine::unit_h() const { return std::ldexp(1.0, scale_host_.exp_h); }

// backend/exact_sum.rs:244-254: the exponent of v's lowest set bit, as
// the code hbr_grain_fold folds (1024 - (grain + 150); 0 for zero).
static uint32_t grain_code(float v) {
    uint32_t bits;
    std::memcpy(&bits, &v, 4);
    const uint32_t biased = (bits >> 23) & 0xffu, mant = bits & 0x7fffffu;
    if (biased == 0xffu || (biased == 0u && mant == 0u)) return 0u;
    const uint32_t sig = biased == 0u ? mant : (mant | 0x800000u);
    const int32_t grain = (biased == 0u ? -149 : (int32_t)biased - 150) + __builtin_ctz(sig);
    return (uint32_t)(1024 - (grain + 150));
}

bool Engine::sums_exact(uint64_t m) const {
    if (!grains_known_ || scale_host_.nonfinite) return false;
    auto one = [&](uint32_t max_bits, uint32_t code, int32_t exp) {
        if (code == 0) return true;  // every value zero
        const int32_t grain = (int32_t)(1024 - code) - 150;
        if (grain < exp) return false;  // values below the fixed-point unit
        float mx;
        std::memcpy(&mx, &max_bits, 4);
        const double units = std::ldexp((double)mx, -grain);  // an exact integer
        const double limit = 9007199254740992.0;             // 2^53
        return units <= limit && (unsigned __int128)m * (unsigned __int128)(uint64_t)units <= (unsigned __int128)(1ull << 53);
    };
    return one(scale_host_.max_g_bits, scale_host_.pad[0], scale_host_.exp_g) &&
           one(scale_host_.max_h_bits, scale_host_.pad[1], scale_host_.exp_h);
}

void Engine::prepare(const float *gpair, uint64_t n) {
    if (n != n_rows_) fail(kInvalid, "prepare: one gradient pair per row");
    row_pairs_live_ = false;
    root_partials_ = 0;  // the staged pairs are no longer the walk's
    pair_array_stale_ = false;
    active_pairs_ = nullptr;
    class_outputs_ = 0;  // the softmax pairs are no longer the staged gradients
    gpair_.resize(n_rows_ ? n_rows_ : 1);
    gpair_.upload(reinterpret_cast<const GPair *>(gpair), n, dev_.stream());
    QScale q{};
    for (uint64_t i = 0; i < n; i++) {
        const float g = gpair[2 * i], h = gpair[2 * i + 1];
        if (!std::isfinite(g) || !std::isfinite(h)) {
            q.nonfinite++;
            continue;
        }
        q.max_g_bits = std::max(q.max_g_bits, abs_bits(g));
        q.max_h_bits = std::max(q.max_h_bits, abs_bits(h));
        q.pad[0] = std::max(q.pad[0], grain_code(g));
        q.pad[1] = std::max(q.pad[1], grain_code(h));
    }
    q.exp_g = exp_for(q.max_g_bits, n_rows_);
    q.exp_h = exp_for(q.max_h_bits, n_rows_);
    scale_host_ = q;
    grains_known_ = true;
    scale_checked_ = true;
    HBR_HIP(hipMemcpyAsync(scale_dev(), &scale_host_, sizeof(QScale), hipMemcpyHostToDevice, dev_.stream()));
    dev_.sync();
    if (q.nonfinite) fail(kRefused, "a staged gradient is not finite");
}

// The table of the expf restatement: bits(2^(i/32)) - (i << 47), from the
// host's exp2 (exact: 2^(i/32) correctly rounded).
static std::vector<uint64_t> expf_table() {
    std::vector<uint64_t> t(32);
    for (uint32_t i = 0; i < 32; i++) {
        const double v = std::exp2((double)i / 32.0);
        uint64_t b;
        std::memcpy(&b, &v, sizeof b);
        t[i] = b - ((uint64_t)i << 47);
    }
    return t;
}

// Logistic pairs a row can carry: with unit weights, a scale_pos_weight of
// 1 and labels 0 or 1, (g, h) = (p - y, max(p (1 - p), min_hess)) follow
// from p and y, which fit one word of the padding of a 32-byte row of at
// most 28 features (the dense kernels' one 32-feature group).
bool Engine::row_pairs_ok(const hbr_device_loss &loss) const {
    return row_pairs && !masked_ && loss.kind == HBR_LOSS_LOGISTIC && loss.scale_pos_weight == 1.0f && !has_weights_ &&
           labels_binary_ && dense_u8_ && stride_ == 32 && n_cols_ <= 28 && hist_features_per_group == 32 &&
           outputs_ == 1;
}

bool Engine::bounded_logistic(const hbr_device_loss &loss) const {
    return loss.kind == HBR_LOSS_LOGISTIC && loss.scale_pos_weight == 1.0f && !has_weights_ && labels_binary_ &&
           loss.min_hess <= 0.25f && outputs_ == 1;
}

void Engine::set_bounds(const hbr_device_loss &loss, FinishArgs &f) const {
    const bool b = bounded_logistic(loss);
    const float g = 1.0f, h = 0.25f;
    f.bound_g_bits = b ? abs_bits(g) : 0u;
    f.bound_h_bits = b ? abs_bits(h) : 0u;
}

GradArgs Engine::grad_args(const hbr_device_loss &loss) {
    GradArgs a{};
    if (row_pairs_ok(loss)) {
        a.pair_rows = rows8_.get();
        a.pair_stride = stride_;
        a.pair_byte = 28;
    }
    a.margins = margins_.get();
    a.labels = labels_.get();
    a.weights = has_weights_ ? weights_.get() : nullptr;
    a.gpair = gpair_.get();
    a.scale = scale_dev();
    a.exp_table = expf_table_dev();
    scalar_list_.reserve(n_rows_ ? n_rows_ : 1);
    a.scalar_list = scalar_list_.get();
    a.n = (uint32_t)n_rows_;
    a.vec_rows = (uint32_t)std::min<uint64_t>(loss.vector_rows, n_rows_);
    a.loss = loss.kind == HBR_LOSS_LOGISTIC ? kLogistic : kSquaredError;
    a.scale_pos_weight = loss.scale_pos_weight;
    a.min_hess = loss.min_hess;
    a.max_input = loss.max_input;
    return a;
}

void Engine::launch_gradients(const hbr_device_loss &loss, uint32_t output) {
    if (!labels_loaded_) fail(kInvalid, "gradients: no labels since load_margins");
    restore_row_order();  // the gradient kernel's 8-row vectors are consecutive rows
    if (outputs_ != 1 || output != 0) fail(kRefused, "device gradients run for one output");
    hipStream_t s = dev_.stream();
    grains_known_ = false;
    active_pairs_ = nullptr;
    class_outputs_ = 0;  // the softmax pairs are no longer the staged gradients
    gpair_.resize(n_rows_ ? n_rows_ : 1);
    HBR_HIP(hipMemsetAsync(scale_dev(), 0, sizeof(QScale), s));
    const GradArgs a = grad_args(loss);
    row_pairs_live_ = a.pair_rows != nullptr;
    root_partials_ = 0;  // the staged pairs are no longer the walk's
    pair_array_stale_ = false;
    row_pairs_min_hess_ = loss.min_hess;
    // grid-stride: a few workgroups per CU, one max fold each
    const uint32_t grad_blocks = std::min<uint32_t>(std::max<uint32_t>(1, ceil_div(n_rows_, kThreads)),
                                                    (uint32_t)dev_.cu_count() * 8);
    dev_.launch("hbr_gradients", dim3(grad_blocks), dim3(kThreads), a);
}

// The exponents of the folded maxima, on the host (the device's rule), and
// the scale back to the device; false when a gradient is not finite.
bool Engine::check_scale(QScale host, uint32_t bound_g_bits, uint32_t bound_h_bits) {
    host.exp_g = exp_for(std::max(host.max_g_bits, bound_g_bits), n_rows_);
    host.exp_h = exp_for(std::max(host.max_h_bits, bound_h_bits), n_rows_);
    scale_host_ = host;
    HBR_HIP(hipMemcpyAsync(scale_dev(), &scale_host_, sizeof(QScale), hipMemcpyHostToDevice, dev_.stream()));
    dev_.sync();
    return host.nonfinite == 0;
}

bool Engine::compute_gradients(const hbr_device_loss &loss, uint32_t output) {
    launch_gradients(loss, output);
    {  // the grains of the pairs, for the exact-domain check of later sums
        const uint32_t blocks = std::min<uint32_t>(std::max<uint32_t>(1, ceil_div(n_rows_, kThreads)),
                                                   (uint32_t)dev_.cu_count() * 8);
        dev_.launch("hbr_grain_fold", dim3(blocks), dim3(kThreads), grad_args(loss));
    }
    QScale *q = static_cast<QScale *>(stage_.alloc(sizeof(QScale)));
    HBR_HIP(hipMemcpyAsync(q, scale_dev(), sizeof(QScale), hipMemcpyDeviceToHost, dev_.stream()));
    dev_.sync();
    const QScale host = *q;
    stage_.reset();
    scale_checked_ = true;
    FinishArgs bounds{};
    set_bounds(loss, bounds);
    const bool ok = check_scale(host, bounds.bound_g_bits, bounds.bound_h_bits);
    grains_known_ = true;
    return ok;
}

void Engine::compute_gradients_async(const hbr_device_loss &loss, uint32_t output) {
    launch_gradients(loss, output);
    FinishArgs f{scale_dev(), n_rows_, grad_args(loss), 0u, 0u};
    set_bounds(loss, f);
    f.grad.scalar_list = nullptr;  // the gradient kernel lists no rows
    dev_.launch("hbr_finish_scale", dim3(1), dim3(kThreads), f);
    scale_checked_ = false;  // grow_root reads the scale back and checks it
}

const uint64_t *Engine::expf_table_dev() {
    if (!exp_table_.size()) {
        const std::vector<uint64_t> t = expf_table();
        exp_table_.resize(t.size());
        exp_table_.upload(t.data(), t.size(), dev_.stream());
        dev_.sync();
    }
    return exp_table_.get();
}

void Engine::softmax_gradients_async(float min_hess) {
    if (!labels_loaded_) fail(kInvalid, "softmax gradients: no labels since load_margins");
    const uint32_t k = outputs_;
    if (k < 1 || k > kSoftmaxMaxClasses) fail(kRefused, "softmax gradients: 1 to 1024 classes");
    if (n_rows_ == 0) fail(kInvalid, "softmax gradients: no rows");
    restore_row_order();  // the vector batches are consecutive rows
    hipStream_t s = dev_.stream();
    row_pairs_live_ = false;
    root_partials_ = 0;  // the staged pairs are no longer the walk's
    pair_array_stale_ = false;
    active_pairs_ = nullptr;
    grains_known_ = false;
    class_pairs_.reserve((size_t)k * n_rows_);
    class_scales_.reserve(k);
    class_outputs_ = k;
    HBR_HIP(hipMemsetAsync(class_scales_.get(), 0, k * sizeof(QScale), s));
    SoftmaxArgs a{};
    a.margins = margins_.get();
    a.labels = labels_.get();
    a.weights = has_weights_ ? weights_.get() : nullptr;
    a.gpair = class_pairs_.get();
    a.scales = class_scales_.get();
    a.exp_table = expf_table_dev();
    a.n = (uint32_t)n_rows_;
    a.k = k;
    // simd/mod.rs:515-519: the 2- and 4-class vector batches need 16 margins
    a.batched = (k == 2 || k == 4) && n_rows_ * k >= 16 ? (uint32_t)(n_rows_ - n_rows_ % (8 / k)) : 0u;
    a.min_hess = min_hess;
    const uint32_t blocks = std::min<uint32_t>(std::max<uint32_t>(1, ceil_div(n_rows_, kThreads)),
                                               (uint32_t)dev_.cu_count() * 8);
    dev_.launch("hbr_softmax_grad", dim3(blocks), dim3(kThreads), a);
}

void Engine::select_class(uint32_t c) {
    if (!softmax_staged() || c >= class_outputs_) fail(kInvalid, "select_class: no softmax gradients of that class");
    SelectArgs a{class_scales_.get() + c, scale_dev(), n_rows_};
    dev_.launch("hbr_scale_select", dim3(1), dim3(64), a);
    active_pairs_ = class_pairs_.get() + (size_t)c * n_rows_;
    grains_known_ = false;
    scale_checked_ = false;  // the tree's root or finish reads the class's scale back
}

bool Engine::softmax_all_finite() {
    if (!softmax_staged()) fail(kInvalid, "softmax: no gradients staged");
    std::vector<QScale> q(class_outputs_);
    class_scales_.download(q.data(), q.size(), dev_.stream());
    dev_.sync();
    for (const QScale &c : q)
        if (c.nonfinite) return false;
    return true;
}

// ---- tree growth -------------------------------------------------------------------

void Engine::ensure_rows() {
    for (auto &r : rows_) r.reserve(n_rows_ ? n_rows_ : 1);
}

uint64_t Engine::begin_tree() {
    ensure_rows();
    // the root's rows are the identity run: kernels that take the root read
    // no row list, and the list itself is written only if something asks
    identity_rows0_ = true;
    rows0_written_ = false;
    counters.trees++;
    for (auto &h : slot_history_) h.known = false;
    return ++tree_;
}

// ---- slot histories (exact-order replays) ---------------------------------------

void Engine::note_built(const std::vector<Segment> &segs, const std::vector<uint32_t> &slots) {
    for (size_t i = 0; i < segs.size() && i < slots.size(); i++) {
        if (slots[i] >= slot_history_.size()) slot_history_.resize(slots[i] + 1);
        SlotHistory &h = slot_history_[slots[i]];
        h.known = true;
        h.built = segs[i];
        h.minus.clear();
        h.rows = segs[i].len;
    }
}

void Engine::note_siblings(const std::vector<uint32_t> &parents, const std::vector<uint32_t> &built) {
    for (size_t i = 0; i < parents.size() && i < built.size(); i++) {
        const uint32_t p = parents[i], b = built[i];
        if (p >= slot_history_.size()) slot_history_.resize(p + 1);
        SlotHistory &h = slot_history_[p];
        const bool ok = h.known && b < slot_history_.size() && slot_history_[b].known &&
                        slot_history_[b].minus.empty() && slot_history_[b].rows <= h.rows;
        if (!ok) {
            h.known = false;
            continue;
        }
        h.minus.push_back(slot_history_[b].built);
        h.rows -= slot_history_[b].rows;
    }
}

uint32_t Engine::slot_rows(uint32_t slot) const {
    return slot < slot_history_.size() && slot_history_[slot].known ? slot_history_[slot].rows : 0u;
}

void Engine::exact_segment(const Segment &sg, double *out_dev) {
    hipStream_t s = dev_.stream();
    const uint64_t m = sg.len;
    ExactArgs a{};
    bool contig = contiguous(sg);
    if (!contig) {
        write_identity_rows();
        a.rows = rows_[sg.buf].get() + sg.offset;
        if (m > 1) {
            // the CPU sweeps a node whose rows are one ascending range by
            // feature (contiguous_range, tree/hist/mod.rs:420-428)
            uint32_t ends[2];
            HBR_HIP(hipMemcpyAsync(&ends[0], a.rows, 4, hipMemcpyDeviceToHost, s));
            HBR_HIP(hipMemcpyAsync(&ends[1], a.rows + m - 1, 4, hipMemcpyDeviceToHost, s));
            dev_.sync();
            contig = ends[1] - ends[0] == m - 1;
        }
    }
    // sum_order (tree/hist/mod.rs:411-419): one chain, or len / 4096 blocks
    constexpr uint64_t kParallelThreshold = 8192, kRowsPerTask = 4096, kGatherMaxRows = 1u << 18;
    uint64_t grain = m ? m : 1;
    if (!(m < kParallelThreshold || (dense_ && (contig || n_rows_ <= kGatherMaxRows)))) {
        const uint64_t blocks = m / kRowsPerTask;
        grain = (m + blocks - 1) / blocks;
    }
    const uint64_t blocks = m ? (m + grain - 1) / grain : 0;
    const uint64_t wave = std::max<uint64_t>(1, std::min<uint64_t>(blocks, (uint64_t)dev_.cu_count()));
    const uint64_t words = 2ull * total_bins_;
    d_exact_.reserve(wave * words);
    a.first = sg.offset;  // an identity run: rows offset .. offset + m - 1
    a.m = (uint32_t)m;
    a.grain = (uint32_t)grain;
    a.bins8 = rows8_.get();
    a.stride = stride_;
    a.n_cols = n_cols_;
    a.feature_offset = d_fo_.get();
    a.row_pairs = row_pairs_live_ && stride_ == 32 ? 1u : 0u;
    a.gpair = a.row_pairs ? nullptr : pairs();
    a.min_hess = row_pairs_min_hess_;
    a.masked = masked_ ? 1u : 0u;
    a.mask_at = mask_at_;
    a.total_bins = total_bins_;
    a.partial = d_exact_.get();
    if (blocks == 0) HBR_HIP(hipMemsetAsync(out_dev, 0, words * sizeof(double), s));
    for (uint64_t b0 = 0; b0 < blocks; b0 += wave) {
        const uint32_t nb = (uint32_t)std::min<uint64_t>(wave, blocks - b0);
        a.blk0 = (uint32_t)b0;
        dev_.launch("hbr_hist_exact", dim3(nb), dim3(kExactThreads), a);
        ExactSumArgs c{d_exact_.get(), nb, b0 == 0 ? 1u : 0u, out_dev, (uint32_t)words, nullptr};
        dev_.launch("hbr_hist_exact_sum", dim3(ceil_div(words, 256)), dim3(256), c);
    }
}

bool Engine::exact_hist(uint32_t slot, double *out) {
    if (!exact_hist_dev(slot)) return false;
    d_exact_out_.download(out, 2ull * total_bins_, dev_.stream());
    dev_.sync();
    return true;
}

bool Engine::resolve_exact(uint32_t slot, double total_g, double total_h, QBin total_fixed, float lower, float upper,
                           ExactBest *out) {
    if (!exact_hist_dev(slot)) return false;
    d_exact_best_.reserve(n_cols_ + 1);
    ExactScanArgs a{};
    a.hist = d_exact_out_.get();
    a.fixed = hist_.get() + (size_t)slot * total_bins_;
    a.feature_offset = d_fo_.get();
    a.n_cols = n_cols_;
    a.dense = dense_ ? 1u : 0u;
    a.total_g = total_g;
    a.total_h = total_h;
    a.total_fixed = total_fixed;
    a.lower = lower;
    a.upper = upper;
    a.reg = scan_params_;
    a.monotone = has_monotone_ ? monotone_.get() : nullptr;
    a.per_feature = d_exact_best_.get() + 1;
    a.best = d_exact_best_.get();
    dev_.launch("hbr_scan_exact", dim3(1), dim3(256), a);
    d_exact_best_.download(out, 1, dev_.stream());
    dev_.sync();
    return true;
}

bool Engine::exact_hist_dev(uint32_t slot) {
    if (slot >= slot_history_.size() || !slot_history_[slot].known) return false;
    if (!dense_u8_ || n_cols_ == 0 || n_cols_ > kExactThreads || 2ull * total_bins_ > kExactMaxWords) return false;
    if (level_pairs_ || softmax_staged()) return false;  // per-class pairs: one tree's pairs only
    if (!(row_pairs_live_ && stride_ == 32) && (pair_array_stale_ || !pairs_staged())) return false;
    const SlotHistory h = slot_history_[slot];
    const uint64_t words = 2ull * total_bins_;
    d_exact_out_.reserve(words);
    exact_segment(h.built, d_exact_out_.get());
    if (!h.minus.empty()) d_exact_minus_.reserve(words);
    for (const Segment &sg : h.minus) {
        // the sibling: parent - built, bin by bin in f64
        exact_segment(sg, d_exact_minus_.get());
        ExactSumArgs c{nullptr, 0, 0, d_exact_out_.get(), (uint32_t)words, d_exact_minus_.get()};
        dev_.launch("hbr_hist_exact_sum", dim3(ceil_div(words, 256)), dim3(256), c);
    }
    return true;
}

void Engine::write_identity_rows() {
    if (!identity_rows0_ || rows0_written_) return;
    IotaArgs a{rows_[0].get(), 0, (uint32_t)n_rows_};
    dev_.launch("hbr_iota", dim3(ceil_div(n_rows_, kThreads)), dim3(kThreads), a);
    rows0_written_ = true;
}

// A segment whose rows are the identity run 0..n-1 (the root of an
// unsampled tree) is summed without reading its row list.
bool Engine::contiguous(const Segment &sg) const {
    return identity_rows0_ && sg.buf == 0 && sg.offset == 0 && sg.len == n_rows_;
}

QBin Engine::root_total(const Segment &sg) {
    hipStream_t s = dev_.stream();
    HBR_HIP(hipMemsetAsync(total_dev(), 0, sizeof(QBin), s));
    TotalArgs a{};
    const bool ident = contiguous(sg);
    a.rows = ident ? nullptr : rows_[sg.buf].get() + sg.offset;
    a.first = ident ? sg.offset : 0;
    a.n = sg.len;
    a.gpair = pairs();
    a.scale = scale_dev();
    a.out = total_dev();
    const uint32_t blocks = std::min<uint32_t>(std::max<uint32_t>(1, ceil_div(sg.len, kThreads)), kTotalBlocks);
    dev_.launch("hbr_total", dim3(blocks), dim3(kThreads), a);
    QBin *out = static_cast<QBin *>(stage_.alloc(sizeof(QBin)));
    HBR_HIP(hipMemcpyAsync(out, total_dev(), sizeof(QBin), hipMemcpyDeviceToHost, s));
    dev_.sync();
    QBin t = *out;
    stage_.reset();
    return t;
}

// The root without a host synchronisation before its split search: the
// total sums on the device, the histogram builds, and the scan takes the
// total and the root gain from the device. One synchronisation then brings
// back the winner, the total and the scale.
void Engine::launch_root(const Segment &seg, uint32_t slot, float lower, float upper) {
    hipStream_t s = dev_.stream();
    // a dense index's root total is the sum of any feature's bins: the scan
    // takes it from feature 0's (which must have bins); else it is summed here
    if (!(dense_ && n_cols_ > 0 && fo_[1] > fo_[0])) {
        HBR_HIP(hipMemsetAsync(total_dev(), 0, sizeof(QBin), s));
        TotalArgs t{};
        const bool ident = contiguous(seg);
        t.rows = ident ? nullptr : rows_[seg.buf].get() + seg.offset;
        t.first = ident ? seg.offset : 0;
        t.n = seg.len;
        t.gpair = pairs();
        t.scale = scale_dev();
        t.out = total_dev();
        dev_.launch("hbr_total",
                    dim3(std::min<uint32_t>(std::max<uint32_t>(1, ceil_div(seg.len, kThreads)), kTotalBlocks)),
                    dim3(kThreads), t);
    }
    // the root's histogram node and scan node in one upload; the winner, the
    // total and the scale back in one copy
    HistNode hn{};
    hn.seg = Seg{seg.offset, seg.len, seg.buf, 0};
    hn.slot = slot;
    hn.contiguous = contiguous(seg) ? 1u : 0u;
    counters.hist_nodes++;
    counters.hist_rows += seg.len;
    counters.hist_bytes += hist_bytes(seg.len, !hn.contiguous);
    ScanNode n{};
    n.slot = slot;
    n.lower = lower;
    n.upper = upper;
    n.pad = kScanDeviceRoot;
    n.rows = seg.len;
    struct RootIn {
        HistNode h;
        ScanNode s;
    };
    RootIn *rin = static_cast<RootIn *>(stage_.alloc(sizeof(RootIn)));
    rin->h = hn;
    rin->s = n;
    d_level_in_.reserve(sizeof(RootIn));
    RootIn *rdev = reinterpret_cast<RootIn *>(d_level_in_.get());
    HBR_HIP(hipMemcpyAsync(rdev, rin, sizeof(RootIn), hipMemcpyHostToDevice, s));
    const std::vector<HistNode> one{hn};
    launch_hist(&rdev->h, 1, &one, nullptr, nullptr);
    launch_scan(&rdev->s, 1, nullptr, nullptr, root_best_dev(), nullptr, n_cat_ ? d_root_set_.get() : nullptr);
}

bool Engine::grow_root(const Segment &seg, uint32_t slot, float lower, float upper, QBin *total, ScanBest *best,
                       uint32_t *best_set) {
    hipStream_t s = dev_.stream();
    launch_root(seg, slot, lower, upper);
    RootBlock *rb = static_cast<RootBlock *>(stage_.alloc(sizeof(RootBlock)));
    HBR_HIP(hipMemcpyAsync(rb, root_block(), sizeof(RootBlock), hipMemcpyDeviceToHost, s));
    uint32_t *set = nullptr;
    if (n_cat_) {
        set = static_cast<uint32_t *>(stage_.alloc(kCatWords * sizeof(uint32_t)));
        HBR_HIP(hipMemcpyAsync(set, d_root_set_.get(), kCatWords * sizeof(uint32_t), hipMemcpyDeviceToHost, s));
    }
    dev_.sync();
    *best = rb->best;
    *total = rb->total;
    if (best->flags & kScanNearTie) counters.near_ties++;
    if (best_set && set) std::memcpy(best_set, set, kCatWords * sizeof(uint32_t));
    const QScale host = rb->scale;
    stage_.reset();
    if (scale_checked_) return true;
    scale_checked_ = true;
    scale_host_ = host;
    return host.nonfinite == 0;
}

uint32_t Engine::alloc_slot() {
    if (free_slots_.empty()) {
        const uint32_t cap = std::max<uint32_t>(8, slot_cap_ * 2);
        if (!reserve_slots(cap)) fail(kRefused, "histogram slots do not fit in device memory");
    }
    const uint32_t s = free_slots_.back();
    free_slots_.pop_back();
    return s;
}

void Engine::free_slot(uint32_t s) { free_slots_.push_back(s); }

bool Engine::reserve_slots(uint64_t n) {
    if (n <= slot_cap_) return true;
    size_t free_b = 0, total_b = 0;
    HBR_HIP(hipMemGetInfo(&free_b, &total_b));
    const uint64_t bytes = n * (uint64_t)total_bins_ * sizeof(QBin);
    if (bytes > free_b / 2) return false;
    DBuf<QBin> grown(n * (uint64_t)total_bins_ + 1);
    if (slot_cap_)
        HBR_HIP(hipMemcpyAsync(grown.get(), hist_.get(), (uint64_t)slot_cap_ * total_bins_ * sizeof(QBin),
                               hipMemcpyDeviceToDevice, dev_.stream()));
    dev_.sync();
    hist_ = std::move(grown);
    for (uint32_t s = (uint32_t)n; s-- > slot_cap_;) free_slots_.push_back(s);
    slot_cap_ = (uint32_t)n;
    return true;
}

// Per row: its bins (one byte per feature for a dense u8 index, else four
// per stored entry), its gradient pair (8 bytes, or the 4-byte word of a
// pair the row carries), and its id when the node's rows are gathered
// through a row list.
uint64_t Engine::hist_bytes(uint64_t rows, bool gathered) const {
    const uint64_t bins = dense_u8_ ? n_cols_ : dense16_ ? 2ull * n_cols_ : 4ull * (n_rows_ ? gbins_.size() / n_rows_ : 0);
    // a pair carried by the row is its one word in the row's padding
    const uint64_t pair = row_pairs_live_ && !level_pairs_ && dense_u8_ && stride_ == 32 ? 4 : 8;
    return rows * (bins + pair + (gathered ? 4 : 0));
}

// The dense u8 histogram kernel for groups of fg features: one group of 25
// to 28 features (compact masked rows included) takes the instance whose
// lanes rotate over those features alone.
const char *Engine::dense8_kernel(uint32_t fg) const {
    const bool bm = hist_bin_major && fg >= 16;
    const bool nf28 = hist_nf28 && bm && fg == 32 && n_cols_ > 24 && n_cols_ <= 28 && (!masked_ || mask_at_ == 28);
    if (masked_) return nf28 ? "hbr_hist_dense8_fg32_bm_masked_nf28" : "hbr_hist_dense8_fg32_bm_masked";
    if (fg <= 8) return "hbr_hist_dense8_fg8";
    if (fg <= 16) return bm ? "hbr_hist_dense8_fg16_bm" : "hbr_hist_dense8_fg16";
    if (!bm) return "hbr_hist_dense8_fg32";
    return nf28 ? "hbr_hist_dense8_fg32_bm_nf28" : "hbr_hist_dense8_fg32_bm";
}

void Engine::set_scan_params(const ScanParams &p, const std::vector<int8_t> &monotone) {
    scan_params_ = p;
    const bool same = has_monotone_ && monotone == monotone_host_;
    has_monotone_ = false;
    for (int8_t d : monotone) has_monotone_ |= d != 0;
    if (has_monotone_ && !same) {
        monotone_host_ = monotone;
        std::vector<int8_t> dirs(n_cols_, 0);
        for (size_t f = 0; f < monotone.size() && f < n_cols_; f++) dirs[f] = monotone[f];
        monotone_.resize(n_cols_);
        monotone_.upload(dirs.data(), n_cols_, dev_.stream());
        dev_.sync();
    }
}

// Histograms of a batch of nodes into their slots: the plan kernel cuts the
// nodes' rows into tiles (about `per_cu` resident workgroups per CU over the
// launch), then one workgroup per (tile, feature group). Dense u8 tiles
// write their sums with plain stores (the reduce kernel adds up nodes of
// several tiles); CSR tiles add into slots zeroed first.
void Engine::launch_hist(const HistNode *nodes_dev, uint32_t n, const std::vector<HistNode> *host_nodes,
                         const PartSplit *splits_dev, const PartOut *part_out_dev, const uint32_t *rows0,
                         const GrowCounts *grow) {
    if (n == 0) return;
    root_partials_ = 0;  // the partials are reused below
    if (!level_pairs_ && !pairs_staged()) fail(kInvalid, "histograms: no gradients staged");
    if (!dense_u8_ && grow) fail(kInvalid, "histograms: device-counted levels need the dense kernels");
    const bool wide = dense16_;  // u16 rows
    const uint32_t fg = wide ? fg16_ : masked_ ? 32u : hist_features_per_group;  // masked rows: fg32 groups
    const uint32_t group_bins = wide ? kWideLdsBins / fg16_ : 256u;
    const bool dense = dense_u8_ || wide;
    // dense: feature groups of fg features; CSR: ranges of kCsrGroupBins
    // global bins (every range of every tile is written: no slot zeroing)
    const uint32_t groups = dense ? ceil_div(n_cols_, fg) : ceil_div(total_bins_, kCsrGroupBins);
    // LDS per workgroup: fg features x 257 words x 16 bytes, or 128 KiB, of 160 KiB
    const uint32_t per_cu = !dense_u8_ ? 1 : fg <= 8 ? 4 : fg <= 16 ? 2 : 1;
    const uint32_t target = std::max<uint32_t>(1, (uint32_t)dev_.cu_count() * per_cu * hist_waves / groups);
    (void)host_nodes;
    d_htiles_.reserve(target + n);
    d_hcounts_.reserve(4);
    d_partial_.reserve((size_t)(dense ? 2 * target : target + n) * groups * (dense ? fg * group_bins : kCsrGroupBins));

    HistNode *nodes_rw = const_cast<HistNode *>(nodes_dev);  // the plan kernel resolves them in place
    PlanArgs p{};
    p.nodes = nodes_rw;
    p.n_nodes = n;
    p.target_tiles = target;
    p.splits = splits_dev;
    p.part_out = part_out_dev;
    p.tiles = d_htiles_.get();
    p.counts = d_hcounts_.get();
    p.min_rows = kHistMinRows;
    p.fuse_subtract = dense ? 1u : 0u;
    p.grow = grow;
    dev_.launch("hbr_hist_plan", dim3(1), dim3(256), p);

    HistArgs a{};
    a.nodes = nodes_dev;
    a.tiles = d_htiles_.get();
    a.counts = d_hcounts_.get();
    a.rows[0] = rows0 ? rows0 : rows_[0].get();
    a.rows[1] = rows_[1].get();
    a.gpair = level_pairs_ ? level_pairs_ : pairs();
    a.scale = level_scale_ ? level_scale_ : scale_dev();
    a.class_rows = level_pairs_ ? (uint32_t)n_rows_ : 0u;
    a.csr_ranges = !dense_u8_ && csr_ranges_.size() ? csr_ranges_.get() : nullptr;
    a.bins8 = rows8_.get();
    a.stride = stride_;
    a.n_cols = n_cols_;
    a.row_ptr = row_ptr_.get();
    a.gbins = gbins_.get();
    a.feature_offset = d_fo_.get();
    a.hist = hist_.get();
    a.partial = d_partial_.get();
    a.total_bins = total_bins_;
    a.groups = groups;
    a.row_pairs = row_pairs_live_ && !level_pairs_ && dense_u8_ && stride_ == 32 && fg == 32 ? 1u : 0u;
    if (pair_array_stale_ && !a.row_pairs && !level_pairs_)
        fail(kRefused, "histograms: the staged pairs are carried in the rows, which this kernel does not read");
    a.masked = masked_ ? 1u : 0u;
    a.mask_at = mask_at_;
    a.min_hess = row_pairs_min_hess_;
    a.bins16 = rows16_.get();
    a.stride16 = stride16_;
    static const char *const wide_kernels[] = {"hbr_hist_dense16_fg1", "hbr_hist_dense16_fg2", "hbr_hist_dense16_fg4",
                                               "hbr_hist_dense16_fg8", "hbr_hist_dense16_fg16"};
    const char *k = wide ? wide_kernels[__builtin_ctz(fg)] : !dense_u8_ ? "hbr_hist_csr" : dense8_kernel(fg);
    dev_.launch(k, dim3((target + n) * groups), dim3(dense ? hist_threads : kCsrThreads), a);
    if (!dense) {
        ReduceArgs r{};
        r.nodes = nodes_dev;
        r.partial = d_partial_.get();
        r.hist = hist_.get();
        r.total_bins = total_bins_;
        r.groups = groups;
        dev_.launch("hbr_hist_reduce_csr", dim3(ceil_div(total_bins_, 256), n), dim3(256), r);
    }
    if (dense) {
        ReduceArgs r{};
        r.nodes = nodes_dev;
        r.partial = d_partial_.get();
        r.hist = hist_.get();
        r.feature_offset = d_fo_.get();
        r.n_cols = n_cols_;
        r.total_bins = total_bins_;
        r.groups = groups;
        r.fg = fg;
        r.grow = grow;
        r.group_bins = group_bins;
        r.quarters = group_bins / 64u;
        dev_.launch("hbr_hist_reduce", dim3(n_cols_ * r.quarters, n), dim3(1024), r);
    }
}

void Engine::build_nodes(const std::vector<Segment> &segs, const std::vector<uint32_t> &slots) {
    if (segs.empty()) return;
    std::vector<HistNode> nodes;
    for (size_t i = 0; i < segs.size(); i++) {
        HistNode n{};
        n.seg = Seg{segs[i].offset, segs[i].len, segs[i].buf, 0};
        n.slot = slots[i];
        n.contiguous = contiguous(segs[i]) ? 1u : 0u;
        nodes.push_back(n);
        counters.hist_nodes++;
        counters.hist_rows += segs[i].len;
        counters.hist_bytes += hist_bytes(segs[i].len, !n.contiguous);
    }
    upload_vec(d_hnodes_, nodes, stage_, dev_.stream());
    launch_hist(d_hnodes_.get(), (uint32_t)nodes.size(), &nodes, nullptr, nullptr);
}

void Engine::subtract(const std::vector<uint32_t> &parents, const std::vector<uint32_t> &built) {
    if (parents.empty()) return;
    std::vector<PartSplit> sp(parents.size());
    for (size_t i = 0; i < parents.size(); i++) {
        sp[i] = PartSplit{};
        sp[i].parent_slot = parents[i];
        sp[i].fresh_slot = built[i];
    }
    upload_vec(d_splits_, sp, stage_, dev_.stream());
    SubArgs a{d_splits_.get(), (uint32_t)sp.size(), hist_.get(), total_bins_};
    dev_.launch("hbr_subtract", dim3(std::min<uint32_t>(ceil_div(total_bins_, 256), 64), (uint32_t)sp.size()),
                dim3(256), a);
}

void Engine::launch_scan(const ScanNode *nodes_dev, uint32_t n, const PartSplit *splits_dev,
                         const PartOut *part_out_dev, ScanBest *best_dev, const GrowCounts *grow,
                         uint32_t *best_sets_dev) {
    const uint64_t pairs = (uint64_t)n * n_cols_;
    d_per_feature_.reserve(pairs ? pairs : 1);
    ScanArgs a{};
    a.nodes = nodes_dev;
    a.n_nodes = n;
    a.n_features = n_cols_;
    a.splits = splits_dev;
    a.part_out = part_out_dev;
    a.hist = hist_.get();
    a.total_bins = total_bins_;
    a.feature_offset = d_fo_.get();
    a.monotone = has_monotone_ ? monotone_.get() : nullptr;
    a.scale = level_scale_ ? level_scale_ : scale_dev();
    a.reg = scan_params_;
    a.dense = dense_ ? 1u : 0u;
    a.guard = guard_active ? 1u : 0u;
    a.gamma = guard_gamma;
    a.per_feature = d_per_feature_.get();
    a.best = best_dev;
    a.root_total = level_totals_ ? level_totals_ : total_dev();
    a.grow = grow;
    if (n_cat_) {
        if (grow) fail(kInvalid, "scan: device-counted levels have no categorical sweep");
        d_cat_sets_.reserve((size_t)n * n_cat_ * kCatWords);
        a.cat_rank = d_cat_rank_.get();
        a.cat_feature = d_cat_feature_.get();
        a.n_cat = n_cat_;
        a.cat_sets = d_cat_sets_.get();
        a.best_sets = best_sets_dev;
    }
    dev_.launch("hbr_scan_features", dim3(ceil_div(pairs, 4)), dim3(256), a);
    if (n_cat_) dev_.launch("hbr_scan_categorical", dim3(n * n_cat_), dim3(64), a);
    dev_.launch("hbr_scan_merge", dim3(n), dim3(256), a);
}

// Scan nodes given on the host: upload, scan, copy the winners into `out`
// and, with categorical features, their sets into `sets` (both pinned; valid
// after the next synchronisation).
void Engine::scan_host_nodes(const std::vector<ScanNode> &nodes, ScanBest *out, uint32_t *sets) {
    hipStream_t s = dev_.stream();
    upload_vec(d_snodes_, nodes, stage_, s);
    d_best_.reserve(nodes.size());
    uint32_t *sets_dev = nullptr;
    if (n_cat_) {
        d_scan_sets_.reserve(nodes.size() * kCatWords);
        sets_dev = d_scan_sets_.get();
    }
    launch_scan(d_snodes_.get(), (uint32_t)nodes.size(), nullptr, nullptr, d_best_.get(), nullptr, sets_dev);
    d_best_.download(out, nodes.size(), s);
    if (sets && sets_dev) d_scan_sets_.download(sets, nodes.size() * kCatWords, s);
}

std::vector<ScanBest> Engine::scan(const std::vector<ScanInput> &in, std::vector<uint32_t> *sets) {
    std::vector<ScanBest> out(in.size());
    if (sets) sets->assign(in.size() * kCatWords, 0u);
    if (in.empty()) return out;
    std::vector<ScanNode> nodes(in.size());
    for (size_t i = 0; i < in.size(); i++) {
        ScanNode n{};
        n.slot = in[i].slot;
        n.total = in[i].total;
        n.root_gain = in[i].root_gain;
        n.lower = in[i].lower;
        n.upper = in[i].upper;
        const uint32_t known = slot_rows(in[i].slot);
        n.rows = in[i].rows ? in[i].rows : known ? known : (uint32_t)n_rows_;
        nodes[i] = n;
    }
    ScanBest *staged = static_cast<ScanBest *>(stage_.alloc(in.size() * sizeof(ScanBest)));
    uint32_t *staged_sets =
        n_cat_ ? static_cast<uint32_t *>(stage_.alloc(in.size() * kCatWords * sizeof(uint32_t))) : nullptr;
    scan_host_nodes(nodes, staged, staged_sets);
    dev_.sync();
    std::memcpy(out.data(), staged, in.size() * sizeof(ScanBest));
    if (sets && staged_sets) std::memcpy(sets->data(), staged_sets, in.size() * kCatWords * sizeof(uint32_t));
    stage_.reset();
    return out;
}

// Bump layout of one level's records in one host block and one device block.
namespace {
struct Layout {
    size_t bytes = 0;
    size_t add(size_t n) {
        const size_t at = bytes;
        bytes += (n + 255) & ~size_t(255);
        return at;
    }
};
}  // namespace

// Routing data and row buffers of the partition kernels (splits, counts and
// outputs are the caller's).
PartArgs Engine::part_args() const {
    PartArgs a{};
    a.tile_left = d_tile_left_.get();
    a.decisions = d_decisions_.get();
    a.src_rows[0] = rows_[0].get();
    a.src_rows[1] = rows_[1].get();
    a.dst_rows[0] = rows_[0].get();
    a.dst_rows[1] = rows_[1].get();
    a.dense = have_cols_ ? 1u : 0u;
    a.cols8 = cols8_.size() ? cols8_.get() : nullptr;
    a.cols16 = cols16_.size() ? cols16_.get() : nullptr;
    a.missing = missing_.size() ? missing_.get() : nullptr;
    a.row_ptr = row_ptr_.get();
    a.gbins = gbins_.get();
    a.csr_ascending = csr_ascending_ ? 1u : 0u;
    a.feature_offset = d_fo_.get();
    a.n_rows = (uint32_t)n_rows_;
    a.words = words_;
    return a;
}

std::vector<LevelChild> Engine::level(const std::vector<LevelSplit> &splits, bool terminal) {
    const uint32_t P = (uint32_t)splits.size();
    std::vector<LevelChild> children(2 * P);
    if (P == 0) return children;
    hipStream_t s = dev_.stream();
    // inputs: splits, built-child histogram nodes, children's scan nodes;
    // outputs: partition results and the children's winners. One copy each way.
    Layout in, out;
    const size_t o_splits = in.add(P * sizeof(PartSplit));
    const size_t o_hnodes = terminal ? 0 : in.add(P * sizeof(HistNode));
    const size_t o_snodes = terminal ? 0 : in.add(2 * P * sizeof(ScanNode));
    uint32_t n_tables = 0;
    for (const LevelSplit &l : splits) n_tables += l.categorical ? 1u : 0u;
    const size_t o_tables = n_tables ? in.add((size_t)n_tables * kCatWords * sizeof(uint32_t)) : 0;
    const size_t o_pout = out.add(P * sizeof(PartOut));
    const size_t o_best = terminal ? 0 : out.add(2 * P * sizeof(ScanBest));
    const size_t o_sets = terminal || !n_cat_ ? 0 : out.add(2 * P * kCatWords * sizeof(uint32_t));
    char *host_in = static_cast<char *>(stage_.alloc(in.bytes));
    char *host_out = static_cast<char *>(stage_.alloc(out.bytes));
    d_level_in_.reserve(in.bytes);
    d_level_out_.reserve(out.bytes);
    char *dev_in = reinterpret_cast<char *>(d_level_in_.get());
    char *dev_out = reinterpret_cast<char *>(d_level_out_.get());

    PartSplit *ps = reinterpret_cast<PartSplit *>(host_in + o_splits);
    uint32_t *tables = n_tables ? reinterpret_cast<uint32_t *>(host_in + o_tables) : nullptr;
    std::vector<uint32_t> fresh(P, 0);
    uint32_t tiles = 0, table = 0;
    for (uint32_t i = 0; i < P; i++) {
        const LevelSplit &l = splits[i];
        PartSplit p{};
        p.seg = Seg{l.seg.offset, l.seg.len, l.seg.buf, 0};
        p.feature = l.feature;
        p.limit = l.limit;
        p.default_left = l.default_left;
        if (l.categorical) {
            if (!is_categorical(l.feature)) fail(kInvalid, "level: a categorical split on a numeric feature");
            std::memcpy(tables + (size_t)table * kCatWords, l.table.data(), kCatWords * sizeof(uint32_t));
            p.table = ++table;
        }
        p.identity = contiguous(l.seg) ? 1u : 0u;
        p.tile_begin = tiles;
        if (!terminal) {
            fresh[i] = alloc_slot();
            p.fresh_slot = fresh[i];
            p.parent_slot = l.parent_slot;
        }
        tiles += ceil_div(l.seg.len, kPartTile);
        ps[i] = p;
    }
    std::vector<HistNode> hn;
    if (!terminal) {
        hn.resize(P);
        ScanNode *sn = reinterpret_cast<ScanNode *>(host_in + o_snodes);
        for (uint32_t i = 0; i < P; i++) {
            HistNode n{};
            n.slot = fresh[i];
            n.from_split = 1;
            n.split = i;
            hn[i] = n;
            for (uint32_t c = 0; c < 2; c++) {
                ScanNode m{};
                m.from_split = 1;
                m.split = i;
                m.child = c;
                m.total = splits[i].child_total[c];
                m.root_gain = splits[i].child_root_gain[c];
                m.lower = splits[i].child_lower[c];
                m.upper = splits[i].child_upper[c];
                sn[2 * i + c] = m;
            }
        }
        std::memcpy(host_in + o_hnodes, hn.data(), P * sizeof(HistNode));
    }
    HBR_HIP(hipMemcpyAsync(dev_in, host_in, in.bytes, hipMemcpyHostToDevice, s));
    const PartSplit *splits_dev = reinterpret_cast<const PartSplit *>(dev_in + o_splits);
    PartOut *pout_dev = reinterpret_cast<PartOut *>(dev_out + o_pout);

    d_tile_left_.reserve(tiles ? tiles : 1);
    d_decisions_.reserve((size_t)(tiles ? tiles : 1) * (kPartTile / 64));
    PartArgs a = part_args();
    a.splits = splits_dev;
    a.n_splits = P;
    a.n_tiles = tiles;
    a.out = pout_dev;
    a.cat_tables = n_tables ? reinterpret_cast<const uint32_t *>(dev_in + o_tables) : nullptr;
    dev_.launch("hbr_part_count", dim3(tiles), dim3(kPartThreads), a);
    dev_.launch("hbr_part_scan", dim3(P), dim3(1024), a);
    dev_.launch("hbr_part_scatter", dim3(tiles), dim3(kPartThreads), a);

    if (!terminal) {
        launch_hist(reinterpret_cast<const HistNode *>(dev_in + o_hnodes), P, &hn, splits_dev, pout_dev);
        if (!dense_u8_ && !dense16_) {  // the dense kernels turn each parent into the sibling as they finish
            SubArgs sub{splits_dev, P, hist_.get(), total_bins_};
            dev_.launch("hbr_subtract", dim3(std::min<uint32_t>(ceil_div(total_bins_, 256), 64), P), dim3(256), sub);
        }
        launch_scan(reinterpret_cast<const ScanNode *>(dev_in + o_snodes), 2 * P, splits_dev, pout_dev,
                    reinterpret_cast<ScanBest *>(dev_out + o_best), nullptr,
                    n_cat_ ? reinterpret_cast<uint32_t *>(dev_out + o_sets) : nullptr);
    }
    HBR_HIP(hipMemcpyAsync(host_out, dev_out, out.bytes, hipMemcpyDeviceToHost, s));
    dev_.sync();
    const PartOut *po = reinterpret_cast<const PartOut *>(host_out + o_pout);
    const ScanBest *best_staged = terminal ? nullptr : reinterpret_cast<const ScanBest *>(host_out + o_best);
    for (uint32_t i = 0; i < P; i++) {
        const Segment &pseg = splits[i].seg;
        const uint32_t nl = po[i].left_len;
        LevelChild &L = children[2 * i];
        LevelChild &R = children[2 * i + 1];
        L.seg = Segment{pseg.offset, nl, pseg.buf ^ 1u};
        R.seg = Segment{pseg.offset + nl, pseg.len - nl, pseg.buf ^ 1u};
        counters.partition_rows += pseg.len;
        if (!terminal) {
            const bool built_left = po[i].built_left != 0;
            L.slot = built_left ? fresh[i] : splits[i].parent_slot;
            R.slot = built_left ? splits[i].parent_slot : fresh[i];
            L.best = best_staged[2 * i];
            R.best = best_staged[2 * i + 1];
            counters.near_ties += ((L.best.flags & kScanNearTie) ? 1u : 0u) + ((R.best.flags & kScanNearTie) ? 1u : 0u);
            if (n_cat_) {
                const uint32_t *sets = reinterpret_cast<const uint32_t *>(host_out + o_sets);
                std::memcpy(L.best_set.data(), sets + (size_t)(2 * i) * kCatWords, kCatWords * sizeof(uint32_t));
                std::memcpy(R.best_set.data(), sets + (size_t)(2 * i + 1) * kCatWords, kCatWords * sizeof(uint32_t));
            }
            const uint32_t built = built_left ? nl : pseg.len - nl;
            counters.hist_nodes++;
            counters.hist_rows += built;
            counters.hist_bytes += hist_bytes(built, true);
        }
    }
    // the scatter wrote every split's rows into the other buffer
    identity_rows0_ = false;
    stage_.reset();
    return children;
}

// Depthwise growth on the device. Per level: the decision kernel (splits,
// leaves, the level's partition/histogram/scan records, tree nodes), then
// the partition, the built children's histograms (siblings by subtraction)
// and the children's search. Grids are launched for the most the level can
// hold (2^level splits, every row in a split); the kernels read the real
// counts from the device. The tree, its counts and the scale come back with
// one copy after the last level.
bool Engine::can_grow_device(uint64_t max_depth, uint32_t n_trees) const {
    if (!device_grow || !dense_u8_ || max_depth < 1 || max_depth > kMaxDeviceDepth || n_rows_ == 0) return false;
    if (n_cat_) return false;  // categorical splits are decided by the host
    if (n_trees < 1 || n_trees > kGrowMaxTrees || (uint64_t)n_trees * n_rows_ > UINT32_MAX) return false;
    const uint64_t slots = (uint64_t)n_trees << (max_depth - 1);
    if (slots > kGrowMaxSlots) return false;
    // the decision kernel's table of each split's first tile
    if ((uint64_t)n_trees * (max_depth >= 2 ? uint64_t(1) << (max_depth - 2) : 1) > kGrowMaxSlots / 2) return false;
    // surplus scan workgroups stay few: both children of every possible split
    const uint64_t pmax = (uint64_t)n_trees * (max_depth >= 2 ? uint64_t(1) << (max_depth - 2) : 1);
    if (2 * pmax * n_cols_ > (uint64_t(1) << 22)) return false;
    size_t free_b = 0, total_b = 0;
    if (hipMemGetInfo(&free_b, &total_b) != hipSuccess) return false;
    return std::max<uint64_t>(slots, slot_cap_) * (uint64_t)total_bins_ * sizeof(QBin) <= free_b / 2;
}

// The roots of a device-grown batch of n_trees trees: their histogram and
// scan records (all rows as the identity run, root t in slot t, of class t,
// unbounded) never change, so they are uploaded once per batch size.
void Engine::launch_device_roots(uint32_t n_trees) {
    const size_t bytes = n_trees * (sizeof(HistNode) + sizeof(ScanNode));
    if (root_in_trees_ != n_trees) {
        std::vector<uint8_t> host(bytes);
        HistNode *hn = reinterpret_cast<HistNode *>(host.data());
        ScanNode *sn = reinterpret_cast<ScanNode *>(host.data() + n_trees * sizeof(HistNode));
        for (uint32_t t = 0; t < n_trees; t++) {
            HistNode h{};
            h.seg = Seg{0, (uint32_t)n_rows_, 0, 0};
            h.slot = t;
            h.contiguous = 1;
            h.cls = t;
            hn[t] = h;
            ScanNode r{};
            r.slot = t;
            r.lower = -std::numeric_limits<float>::infinity();
            r.upper = std::numeric_limits<float>::infinity();
            r.pad = kScanDeviceRoot | (t << kScanClassShift);
            r.rows = (uint32_t)n_rows_;
            sn[t] = r;
        }
        d_root_in_.resize(bytes);
        HBR_HIP(hipMemcpy(d_root_in_.get(), host.data(), bytes, hipMemcpyHostToDevice));
        root_in_trees_ = n_trees;
    }
    hipStream_t s = dev_.stream();
    QBin *totals = level_totals_ ? level_totals_ : total_dev();
    if (!(dense_ && n_cols_ > 0 && fo_[1] > fo_[0])) {
        HBR_HIP(hipMemsetAsync(totals, 0, n_trees * sizeof(QBin), s));
        // every tree's total in one launch (blockIdx.y: the tree)
        TotalArgs a{};
        a.rows = nullptr;
        a.first = 0;
        a.n = (uint32_t)n_rows_;
        a.gpair = level_pairs_ ? level_pairs_ : pairs();
        a.tree_pairs = level_pairs_ ? n_rows_ : 0;
        a.scale = level_scale_ ? level_scale_ : scale_dev();
        a.out = totals;
        dev_.launch("hbr_total",
                    dim3(std::min<uint32_t>(std::max<uint32_t>(1, ceil_div(n_rows_, kThreads)), kTotalBlocks), n_trees),
                    dim3(kThreads), a);
    }
    HistNode *hn = reinterpret_cast<HistNode *>(d_root_in_.get());
    const ScanNode *sn = reinterpret_cast<const ScanNode *>(d_root_in_.get() + n_trees * sizeof(HistNode));
    const uint32_t fused = n_trees == 1 && !level_pairs_ && row_pairs_live_ ? root_partials_ : 0u;
    root_partials_ = 0;
    if (fused) {
        // the margin walk summed the root's rows into `fused` partials; the
        // rows it deferred go into one more, then the reduce makes the slot
        RootFixupArgs f{};
        f.scale = scale_dev();
        f.listed = scalar_list_.get();
        f.bins8 = rows8_.get();
        f.partial = d_partial_.get();
        f.node = hn;
        f.n_walk_tiles = fused;
        f.n_cols = n_cols_;
        f.min_hess = row_pairs_min_hess_;
        f.regroup_tile = root_regroup_tile_;
        dev_.launch("hbr_root_fixup", dim3(1), dim3(1024), f);
        ReduceArgs r{};
        r.nodes = hn;
        r.partial = d_partial_.get();
        r.hist = hist_.get();
        r.feature_offset = d_fo_.get();
        r.n_cols = n_cols_;
        r.total_bins = total_bins_;
        r.groups = 1;
        r.fg = kRootFeatures;
        r.group_bins = 256;
        r.quarters = 4;
        r.grow = nullptr;
        dev_.launch("hbr_hist_reduce", dim3(n_cols_ * 4, 1), dim3(1024), r);
    } else {
        counters.hist_nodes += n_trees;
        counters.hist_rows += n_trees * n_rows_;
        counters.hist_bytes += n_trees * hist_bytes(n_rows_, false);
        launch_hist(hn, n_trees, nullptr, nullptr, nullptr);
    }
    launch_scan(sn, n_trees, nullptr, nullptr, n_trees == 1 ? root_best_dev() : d_best_.get());
}

Engine::TreeTicket Engine::queue_device_tree(uint64_t max_depth, double gamma, float eta) {
    if (!pairs_staged()) fail(kInvalid, "device growth: no gradients staged");
    return queue_device_forest(1, max_depth, gamma, eta);
}

Engine::TreeTicket Engine::queue_class_trees(uint64_t max_depth, double gamma, float eta) {
    if (!softmax_staged()) fail(kInvalid, "device growth: no softmax gradients staged");
    const uint32_t k = class_outputs_;
    if (k > kGrowMaxTrees) fail(kRefused, "device growth: at most 256 class trees per batch");
    // every class's exponents from its folded maxima
    ScalesArgs f{class_scales_.get(), k, n_rows_};
    dev_.launch("hbr_class_scales_finish", dim3(ceil_div(k, 64)), dim3(64), f);
    d_root_totals_.reserve(k);
    counters.trees += k - 1;  // begin_tree counted one
    scale_checked_ = false;   // each class's scale is checked at finish
    level_pairs_ = class_pairs_.get();
    level_scale_ = class_scales_.get();
    level_totals_ = d_root_totals_.get();
    try {
        const TreeTicket t = queue_device_forest(k, max_depth, gamma, eta);
        level_pairs_ = nullptr;
        level_scale_ = nullptr;
        level_totals_ = nullptr;
        return t;
    } catch (...) {
        level_pairs_ = nullptr;
        level_scale_ = nullptr;
        level_totals_ = nullptr;
        throw;
    }
}

Engine::TreeTicket Engine::queue_device_forest(uint32_t n_trees, uint64_t max_depth, double gamma, float eta) {
    if (!can_grow_device(max_depth, n_trees)) fail(kInvalid, "device growth: index or depth not supported");
    hipStream_t s = dev_.stream();
    const uint32_t depth = (uint32_t)max_depth;
    const uint32_t slot_cap = n_trees << (depth - 1);
    if (!reserve_slots(slot_cap)) fail(kRefused, "histogram slots do not fit in device memory");
    const uint32_t pmax_all = n_trees * (depth >= 2 ? 1u << (depth - 2) : 1u);
    // every level partitions at most n_trees x n_rows rows, each tree's in its own region
    const uint32_t row_tiles = (uint32_t)ceil_div((uint64_t)n_trees * n_rows_, kPartTile);
    for (int b = 0; b < 2; b++) {
        g_front_[b].reserve(std::max<uint32_t>(slot_cap, n_trees));
        g_splits_[b].reserve(pmax_all);
        g_pout_[b].reserve(pmax_all);
    }
    for (auto &r : rows_) r.reserve((size_t)n_trees * (n_rows_ ? n_rows_ : 1));
    d_hnodes_.reserve(pmax_all);
    d_snodes_.reserve(2 * pmax_all);
    d_best_.reserve(std::max<uint32_t>(2 * pmax_all, n_trees));
    d_tile_left_.reserve(row_tiles + pmax_all);
    d_decisions_.reserve((size_t)(row_tiles + pmax_all) * (kPartTile / 64));
    d_tile_split_.reserve(row_tiles + pmax_all);
    d_tree_nodes_.reserve(n_trees);
    GrowCounts *counts = grow_counts_dev();

    // tree t of a ring slot: its header, then its nodes, at t * stride
    const size_t n_max = (size_t(2) << depth) - 1;
    const size_t stride = (kTreeHeaderBytes + n_max * sizeof(GrowTreeNode) + 255) / 256 * 256;
    const size_t slot_bytes = n_trees * stride;
    if (!copy_stream_) {
        HBR_HIP(hipStreamCreate(&copy_stream_));
        for (uint32_t r = 0; r < kTreeRing; r++) {
            HBR_HIP(hipEventCreateWithFlags(&tree_ready_[r], hipEventDisableTiming));
            HBR_HIP(hipEventCreateWithFlags(&tree_copied_[r], hipEventDisableTiming));
        }
    }
    if (slot_bytes > ring_slot_bytes_) {
        // nothing may still read or copy the old ring
        dev_.sync();
        HBR_HIP(hipStreamSynchronize(copy_stream_));
        d_tree_ring_.resize(kTreeRing * slot_bytes);
        ring_slot_bytes_ = slot_bytes;
    }
    TreeTicket t;
    t.slot = tree_seq_++ % kTreeRing;
    t.check = !scale_checked_;
    t.n_trees = n_trees;
    t.stride = stride;
    scale_checked_ = true;
    last_ring_ = t.slot;
    last_stride_ = stride;
    last_depth_ = depth;
    // the slot's previous batch must have been read back before it is overwritten
    if (ring_used_[t.slot]) HBR_HIP(hipStreamWaitEvent(s, tree_copied_[t.slot], 0));
    ring_used_[t.slot] = true;
    launch_device_roots(n_trees);
    for (uint32_t lv = 0; lv < depth; lv++) {
        const bool terminal = lv + 1 >= depth;
        const uint32_t pmax = (uint32_t)std::min<uint64_t>((uint64_t)n_trees << lv, (uint64_t)n_trees * n_rows_);
        GrowArgs g{};
        g.counts = counts;
        g.front = g_front_[lv & 1].get();
        g.next = g_front_[(lv + 1) & 1].get();
        g.prev_splits = g_splits_[(lv + 1) & 1].get();
        g.prev_out = g_pout_[(lv + 1) & 1].get();
        g.best = lv == 0 && n_trees == 1 ? root_best_dev() : d_best_.get();
        g.root_total = level_totals_ ? level_totals_ : total_dev();
        g.scale = level_scale_ ? level_scale_ : scale_dev();
        g.splits = g_splits_[lv & 1].get();
        g.hnodes = d_hnodes_.get();
        g.snodes = d_snodes_.get();
        g.tile_split = d_tile_split_.get();
        g.tree = ring_nodes(t.slot, 0, stride);
        g.header = ring_header(t.slot, 0, stride);
        g.feature_offset = d_fo_.get();
        g.monotone = has_monotone_ ? monotone_.get() : nullptr;
        g.n_monotone = has_monotone_ ? n_cols_ : 0u;
        g.level = lv;
        g.terminal = terminal ? 1u : 0u;
        g.n_rows = (uint32_t)n_rows_;
        g.root_slot = 0;
        g.slot_cap = slot_cap;
        g.reg = scan_params_;
        g.gamma = gamma;
        g.eta = eta;
        g.front_cap = lv == 0 ? n_trees : std::min<uint32_t>(n_trees << lv, slot_cap);
        g.n_features = n_cols_;
        g.n_trees = n_trees;
        g.tree_bytes = (uint32_t)stride;
        g.tree_nodes = d_tree_nodes_.get();
        dev_.launch(n_trees == 1 ? "hbr_grow_decide" : "hbr_grow_decide_batch", dim3(1), dim3(512), g);
        if (terminal) break;
        PartArgs a = part_args();
        a.splits = g_splits_[lv & 1].get();
        a.n_splits = pmax;
        a.n_tiles = row_tiles + pmax;
        a.out = g_pout_[lv & 1].get();
        a.grow = counts;
        a.tile_split = d_tile_split_.get();
        dev_.launch("hbr_part_count", dim3(a.n_tiles), dim3(kPartThreads), a);
        dev_.launch("hbr_part_scan", dim3(pmax), dim3(1024), a);
        dev_.launch("hbr_part_scatter", dim3(a.n_tiles), dim3(kPartThreads), a);
        launch_hist(d_hnodes_.get(), pmax, nullptr, a.splits, a.out, nullptr, counts);
        launch_scan(d_snodes_.get(), 2 * pmax, a.splits, a.out, d_best_.get(), counts);
    }
    // every level's scatter wrote into the other buffer
    identity_rows0_ = false;
    // the batch's headers and nodes back in one copy, on the copy stream
    void *host = tree_stage_[t.slot].reserve(slot_bytes);
    HBR_HIP(hipEventRecord(tree_ready_[t.slot], s));
    HBR_HIP(hipStreamWaitEvent(copy_stream_, tree_ready_[t.slot], 0));
    HBR_HIP(hipMemcpyAsync(host, ring_header(t.slot, 0, stride), slot_bytes, hipMemcpyDeviceToHost, copy_stream_));
    HBR_HIP(hipEventRecord(tree_copied_[t.slot], copy_stream_));
    return t;
}

Engine::TreeState Engine::finish_device_forest(const TreeTicket &t, std::vector<std::vector<GrowTreeNode>> &trees) {
    HBR_HIP(hipEventSynchronize(tree_copied_[t.slot]));
    const uint8_t *host = static_cast<const uint8_t *>(tree_stage_[t.slot].get());
    trees.resize(t.n_trees);
    TreeState st = kTreeOk;
    const size_t n_max = (t.stride - kTreeHeaderBytes) / sizeof(GrowTreeNode);
    for (uint32_t k = 0; k < t.n_trees; k++) {
        TreeHeader th;
        std::memcpy(&th, host + k * t.stride, sizeof(th));
        const GrowCounts &gc = th.counts;
        if (gc.error) fail(kInvalid, "device growth: a level needed more histogram slots than reserved");
        if (gc.n_nodes == 0 || gc.n_nodes > n_max) fail(kInvalid, "device growth: node count out of range");
        trees[k].resize(gc.n_nodes);
        std::memcpy(trees[k].data(), host + k * t.stride + kTreeHeaderBytes, gc.n_nodes * sizeof(GrowTreeNode));
        if (k == 0) {  // the level counts are the batch's totals (the roots were counted when queued)
            counters.hist_nodes += gc.hist_nodes - t.n_trees;
            counters.hist_rows += gc.hist_rows;
            counters.hist_bytes += hist_bytes(gc.hist_rows, true);
            counters.partition_rows += gc.part_rows;
            counters.near_ties += gc.near_ties;
        }
        if (t.check && th.scale.nonfinite != 0) st = kTreeNotFinite;
        if (t.check && k == 0 && t.n_trees == 1 && st == kTreeOk) scale_host_ = th.scale;
    }
    return st;
}

Engine::TreeState Engine::finish_device_tree(const TreeTicket &t, std::vector<GrowTreeNode> &nodes, QScale *scale) {
    std::vector<std::vector<GrowTreeNode>> trees;
    const TreeState st = finish_device_forest(t, trees);
    nodes = std::move(trees[0]);
    if (scale) {
        TreeHeader th;
        std::memcpy(&th, tree_stage_[t.slot].get(), sizeof(th));
        *scale = th.scale;
    }
    return st;
}

void Engine::drain() {
    dev_.sync();
    if (copy_stream_) HBR_HIP(hipStreamSynchronize(copy_stream_));
    stage_.reset();
    scale_checked_ = true;
    if (poison_.size()) {
        HBR_HIP(hipMemsetAsync(poison_.get(), 0, sizeof(uint32_t), dev_.stream()));
        dev_.sync();
    }
}

bool Engine::grow_device(uint64_t max_depth, double gamma, float eta, std::vector<GrowTreeNode> &nodes) {
    const TreeTicket t = queue_device_tree(max_depth, gamma, eta);
    if (finish_device_tree(t, nodes, nullptr) == kTreeOk) return true;
    drain();
    return false;
}

bool Engine::walk_device_trees(uint32_t first_output, uint32_t n_trees, uint32_t guard_first, uint32_t guard_n) {
    // the batch's node tables must fit the kernel's LDS whatever the trees
    const uint64_t most = (2ull << std::min<uint32_t>(last_depth_, 20u)) - 1;
    // rows of 32 or 64 bytes, or masked rows of at most 64 features (96 bytes)
    const bool rows_ok = stride_ == 32 || stride_ == 64 || (masked_ && stride_ == 96);
    if (!batch_walk || !dense_u8_ || !rows_ok || n_trees < 2 ||
        n_trees > kBatchWalkTrees || n_trees * most > kBatchWalkNodes || first_output + n_trees > outputs_)
        return false;
    if (guard_n && (!softmax_staged() || guard_first + guard_n > class_outputs_))
        fail(kInvalid, "walk: no softmax class scales to guard by");
    hipStream_t s = dev_.stream();
    if (!poison_.size() && guard_n) {
        poison_.resize(1);
        guard_scale_.resize(1);
        HBR_HIP(hipMemsetAsync(poison_.get(), 0, sizeof(uint32_t), s));
    }
    WalkArgs a{};
    a.masked = masked_ ? 1u : 0u;
    a.mask_at = mask_at_;
    a.tree = ring_nodes(last_ring_, 0, last_stride_);
    a.counts = &ring_header(last_ring_, 0, last_stride_)->counts;
    a.tree_bytes = (uint32_t)last_stride_;
    a.n_trees = n_trees;
    a.bins8 = rows8_.get();
    a.margins = margins_.get();
    a.stride = stride_;
    a.n = (uint32_t)n_rows_;
    a.m_stride = outputs_;
    a.output = first_output;
    if (guard_n) {
        a.guard = class_scales_.get() + guard_first;
        a.guard_n = guard_n;
        a.poison = poison_.get();
    }
    const uint32_t blocks =
        std::min<uint32_t>(std::max<uint32_t>(1, ceil_div(n_rows_, 256)), (uint32_t)dev_.cu_count() * walk_blocks_per_cu);
    dev_.launch(stride_ == 32 ? "hbr_walk_leaves_batch32" : "hbr_walk_leaves_batch64", dim3(blocks), dim3(256), a);
    return true;
}

void Engine::walk_device_tree(uint32_t output, const hbr_device_loss *next_loss, uint32_t tree, uint32_t guard_first,
                              uint32_t guard_n) {
    if (!dense_u8_) fail(kRefused, "walk: the index has no row-major u8 bins");
    if (output >= outputs_) fail(kInvalid, "walk: no such output");
    // the staged walk: 32-byte rows and trees whose nodes fit its LDS table
    const bool staged = stride_ == 32 && last_depth_ <= 9;
    if (next_loss && !staged) fail(kRefused, "walk: gradients need 32-byte rows and depth <= 9");
    hipStream_t s = dev_.stream();
    WalkArgs a{};
    a.masked = masked_ ? 1u : 0u;
    a.mask_at = mask_at_;
    a.tree = ring_nodes(last_ring_, tree, last_stride_);
    a.counts = &ring_header(last_ring_, tree, last_stride_)->counts;
    a.bins8 = rows8_.get();
    a.margins = margins_.get();
    a.stride = stride_;
    a.n = (uint32_t)n_rows_;
    a.m_stride = outputs_;
    a.output = output;
    const uint32_t blocks =
        std::min<uint32_t>(std::max<uint32_t>(1, ceil_div(n_rows_, 256)), (uint32_t)dev_.cu_count() * walk_blocks_per_cu);
    if (!poison_.size() && (next_loss || guard_n)) {
        poison_.resize(1);
        guard_scale_.resize(1);
        HBR_HIP(hipMemsetAsync(poison_.get(), 0, sizeof(uint32_t), s));
    }
    if (!next_loss) {
        if (guard_n) {
            if (!softmax_staged() || guard_first + guard_n > class_outputs_)
                fail(kInvalid, "walk: no softmax class scales to guard by");
            a.guard = class_scales_.get() + guard_first;
            a.guard_n = guard_n;
            a.poison = poison_.get();
        }
        dev_.launch(staged ? "hbr_walk_leaves32" : "hbr_walk_leaves", dim3(blocks), dim3(256), a);
        return;
    }
    if (outputs_ != 1 || !labels_loaded_) fail(kInvalid, "walk: gradients need one output and labels");
    active_pairs_ = nullptr;
    grains_known_ = false;
    class_outputs_ = 0;  // the softmax pairs are no longer the staged gradients
    gpair_.resize(n_rows_ ? n_rows_ : 1);
    // the tree's scale aside (the walk's guard), the live one cleared for the fold
    RotateArgs r{scale_dev(), guard_scale_.get()};
    dev_.launch("hbr_scale_rotate", dim3(1), dim3(64), r);
    a.guard = guard_scale_.get();
    a.poison = poison_.get();
    WalkGradArgs wg{};
    wg.w = a;
    wg.g = grad_args(*next_loss);
    row_pairs_live_ = wg.g.pair_rows != nullptr;
    row_pairs_min_hess_ = next_loss->min_hess;
    FinishArgs f{scale_dev(), n_rows_, wg.g, 0u, 0u};
    set_bounds(*next_loss, f);
    // the next root's histogram in the same pass: row-carried pairs, whose
    // bounds fix the exponents, and one 1024-thread workgroup per CU
    const uint32_t root_tiles = std::min<uint32_t>((uint32_t)dev_.cu_count(), ceil_div(n_rows_, 1024));
    root_partials_ = 0;
    root_regroup_tile_ = 0;
    pair_array_stale_ = false;
    if (permuted_) {  // the original 8-row vectors through the marks and hbr_regroup
        wg.g.perm = perm_.get();
        wg.g.group_stamp = group_stamp_.get();
        wg.g.bad_groups = bad_groups_.get();
        if (++regroup_stamp_ == 0) {  // every mark of 2^32 passes ago cleared
            group_stamp_.zero(s);
            regroup_stamp_ = 1;
        }
        wg.g.stamp = regroup_stamp_;
    }
    RegroupArgs rg{};
    if (fused_root && row_pairs_live_ && f.bound_g_bits && n_cols_ <= kRootFeatures && root_tiles >= 2) {
        d_partial_.reserve((size_t)(root_tiles + 2) * kRootTile);
        wg.root_partial = d_partial_.get();
        wg.root_exp_g = exp_for(f.bound_g_bits, n_rows_);
        wg.root_exp_h = exp_for(f.bound_h_bits, n_rows_);
        wg.n_cols = n_cols_;
        wg.g.gpair = nullptr;  // the rows carry every pair; the finish writes its deferred rows' both ways
        // rows of 25 to 28 features: no atomics for the padding columns
        const bool nf28 = hist_nf28 && n_cols_ > 24 && n_cols_ <= 28;
        dev_.launch(nf28 ? "hbr_walk_grad_root_nf28" : "hbr_walk_grad_root", dim3(root_tiles), dim3(1024), wg);
        root_partials_ = root_tiles;
        pair_array_stale_ = true;
        rg.root_partial = wg.root_partial;
        rg.root_exp_g = wg.root_exp_g;
        rg.root_exp_h = wg.root_exp_h;
        rg.n_walk_tiles = root_tiles;
        rg.n_cols = n_cols_;
        rg.bins8 = rows8_.get();
        root_regroup_tile_ = permuted_ ? 1u : 0u;
    } else {
        dev_.launch("hbr_walk_grad32", dim3(blocks), dim3(256), wg);
    }
    if (permuted_ && wg.g.loss == kLogistic) {  // only the logistic loss has 8-row vectors
        rg.g = wg.g;
        rg.perm_inv = perm_inv_.get();
        dev_.launch("hbr_regroup", dim3(1), dim3(1024), rg);
    } else {
        root_regroup_tile_ = 0;
    }
    dev_.launch("hbr_finish_scale", dim3(1), dim3(kThreads), f);
    scale_checked_ = false;  // the next tree's finish checks the scale
}

void Engine::walk_device_tree_then_gradients(const hbr_device_loss &next_loss) {
    if (!dense_u8_) fail(kRefused, "walk: the index has no row-major u8 bins");
    if (outputs_ != 1 || !labels_loaded_) fail(kInvalid, "walk: gradients need one output and labels");
    hipStream_t s = dev_.stream();
    if (!poison_.size()) {
        poison_.resize(1);
        guard_scale_.resize(1);
        HBR_HIP(hipMemsetAsync(poison_.get(), 0, sizeof(uint32_t), s));
    }
    // the tree's scale aside (the walk's guard); the gradients clear the live one
    RotateArgs r{scale_dev(), guard_scale_.get()};
    dev_.launch("hbr_scale_rotate", dim3(1), dim3(64), r);
    WalkArgs a{};
    a.masked = masked_ ? 1u : 0u;
    a.mask_at = mask_at_;
    a.tree = ring_nodes(last_ring_, 0, last_stride_);
    a.counts = &ring_header(last_ring_, 0, last_stride_)->counts;
    a.bins8 = rows8_.get();
    a.margins = margins_.get();
    a.stride = stride_;
    a.n = (uint32_t)n_rows_;
    a.m_stride = outputs_;
    a.output = 0;
    a.guard = guard_scale_.get();
    a.guard_n = 1;
    a.poison = poison_.get();
    const uint32_t blocks =
        std::min<uint32_t>(std::max<uint32_t>(1, ceil_div(n_rows_, 256)), (uint32_t)dev_.cu_count() * walk_blocks_per_cu);
    dev_.launch("hbr_walk_leaves", dim3(blocks), dim3(256), a);
    compute_gradients_async(next_loss, 0);
}

uint32_t Engine::add_eval_set(const float *x, uint64_t n_rows, uint64_t n_cols, float missing, const float *init,
                              uint32_t outputs) {
    if (!x || !init) fail(kInvalid, "evaluation set: null argument");
    if (n_cols != n_cols_) fail(kInvalid, "evaluation set: not the training matrix's features");
    if (n_rows == 0) fail(kInvalid, "evaluation set: no rows");
    if (outputs == 0) fail(kInvalid, "evaluation set: no outputs");
    hipStream_t s = dev_.stream();
    if (d_cuts_.size() != total_bins_ && total_bins_ > 0) {
        d_cuts_.resize(total_bins_);
        d_cuts_.upload(cuts_.data(), total_bins_, s);
    }
    auto set = std::make_unique<EvalSet>();
    set->n_rows = n_rows;
    set->outputs = outputs;
    set->missing = missing;
    set->x.resize(n_rows * n_cols);
    set->x.upload(x, n_rows * n_cols, s);
    set->margins.resize(n_rows * outputs);
    set->margins.upload(init, n_rows * outputs, s);
    dev_.sync();
    evals_.push_back(std::move(set));
    return (uint32_t)evals_.size() - 1;
}

uint64_t Engine::eval_rows(uint32_t set) const {
    if (set >= evals_.size()) fail(kInvalid, "evaluation set: no such set");
    return evals_[set]->n_rows;
}

void Engine::read_eval_margins(uint32_t set, float *out) {
    if (set >= evals_.size()) fail(kInvalid, "evaluation set: no such set");
    const EvalSet &e = *evals_[set];
    e.margins.download(out, e.n_rows * e.outputs, dev_.stream());
    dev_.sync();
}

void Engine::launch_eval_walk(const EvalSet &set, const GrowTreeNode *tree, const GrowCounts *counts,
                              uint32_t n_nodes, uint32_t output, const uint32_t *poison, const float *cond,
                              const EvalCats *cats) {
    if (output >= set.outputs) fail(kInvalid, "evaluation walk: no such output");
    EvalWalkArgs a{};
    if (cats) {  // uploaded by the caller of this walk
        a.cat_span = d_eval_span_.get();
        a.categories = d_eval_categories_.get();
    }
    a.x = set.x.get();
    a.tree = tree;
    a.counts = counts;
    a.cut_values = d_cuts_.get();
    a.cond = cond;
    a.margins = set.margins.get();
    a.poison = poison;
    a.n = set.n_rows;
    a.n_cols = n_cols_;
    a.m_stride = set.outputs;
    a.output = output;
    a.n_nodes = n_nodes;
    a.missing_value = set.missing;
    a.missing_is_nan = std::isnan(set.missing) ? 1u : 0u;
    a.total_bins = (uint32_t)total_bins_;
    if (n_cols_ <= kEvalStagedCols && !std::getenv("HBROCM_EVAL_IN_PLACE")) {
        // 64-row blocks staged in LDS, one per wave, four waves per workgroup
        const uint32_t lds = 4u * n_cols_ * kPredPitch * (uint32_t)sizeof(float);
        const uint64_t blocks64 = (set.n_rows + 63) / 64;
        const uint32_t grid = (uint32_t)std::min<uint64_t>((blocks64 + 3) / 4, (uint64_t)dev_.cu_count() * 2);
        dev_.launch("hbr_eval_walk_staged", dim3(grid), dim3(256), a, lds);
        return;
    }
    const uint64_t want = (set.n_rows + 255) / 256;
    const uint32_t blocks = (uint32_t)std::min<uint64_t>(want, (uint64_t)dev_.cu_count() * 8);
    dev_.launch("hbr_eval_walk", dim3(blocks), dim3(256), a);
}

void Engine::walk_evals_device(uint32_t output, uint32_t tree, bool guarded) {
    if (evals_.empty()) return;
    if (n_cat_) fail(kInvalid, "evaluation walk: device-grown trees have no categorical splits to route");
    if (guarded && !poison_.size()) fail(kInvalid, "evaluation walk: no guarded walk before it");
    for (const auto &set : evals_)
        launch_eval_walk(*set, ring_nodes(last_ring_, tree, last_stride_),
                         &ring_header(last_ring_, tree, last_stride_)->counts, 0, output,
                         guarded ? poison_.get() : nullptr);
}

// A tree's categorical splits for the next evaluation walks: spans checked
// against the node count and the category pool.
void Engine::upload_eval_cats(const EvalCats &cats, size_t n_nodes) {
    const std::vector<uint32_t> empty;
    const std::vector<uint32_t> &pool = cats.categories ? *cats.categories : empty;
    if (cats.span.size() != 2 * n_nodes) fail(kInvalid, "evaluation walk: two category bounds per node");
    for (size_t i = 0; i < n_nodes; i++) {
        const uint32_t b = cats.span[2 * i], e = cats.span[2 * i + 1] & 0x7fffffffu;
        if ((cats.span[2 * i + 1] >> 31) && (b > e || e > pool.size()))
            fail(kInvalid, "evaluation walk: a categorical split's categories are out of range");
    }
    upload_vec(d_eval_span_, cats.span, stage_, dev_.stream());
    if (!pool.empty()) upload_vec(d_eval_categories_, pool, stage_, dev_.stream());
    else d_eval_categories_.reserve(1);
}

void Engine::walk_evals(const std::vector<GrowTreeNode> &nodes, uint32_t output, const std::vector<float> *cond,
                        const EvalCats *cats) {
    if (evals_.empty() || nodes.empty()) return;
    if (nodes.size() > UINT32_MAX) fail(kRefused, "evaluation walk: a tree of more than 2^32 - 1 nodes");
    for (const auto &set : evals_)
        if (output >= set->outputs) fail(kInvalid, "evaluation walk: no such output");
    upload_vec(d_eval_tree_, nodes, stage_, dev_.stream());
    if (cond) {
        if (cond->size() != nodes.size()) fail(kInvalid, "evaluation walk: one threshold per node");
        upload_vec(d_eval_cond_, *cond, stage_, dev_.stream());
    }
    if (cats) upload_eval_cats(*cats, nodes.size());
    for (const auto &set : evals_)
        launch_eval_walk(*set, d_eval_tree_.get(), nullptr, (uint32_t)nodes.size(), output, nullptr,
                         cond ? d_eval_cond_.get() : nullptr, cats);
}

void Engine::walk_evals_one(uint32_t set, const std::vector<GrowTreeNode> &nodes, uint32_t output,
                            const EvalCats *cats) {
    if (set >= evals_.size()) fail(kInvalid, "evaluation set: no such set");
    if (nodes.empty()) return;
    upload_vec(d_eval_tree_, nodes, stage_, dev_.stream());
    if (cats) upload_eval_cats(*cats, nodes.size());
    launch_eval_walk(*evals_[set], d_eval_tree_.get(), nullptr, (uint32_t)nodes.size(), output, nullptr, nullptr,
                     cats);
}

void Engine::add_leaves(const std::vector<Segment> &segs, const std::vector<float> &values, uint32_t output) {
    if (segs.empty()) return;
    std::vector<LeafSeg> leaves(segs.size());
    std::vector<uint32_t> tile_leaf, tile_row0;
    for (uint32_t i = 0; i < segs.size(); i++) {
        LeafSeg l{};
        l.seg = Seg{segs[i].offset, segs[i].len, segs[i].buf, 0};
        l.value = values[i];
        leaves[i] = l;
        for (uint32_t r0 = 0; r0 < segs[i].len; r0 += kLeafTile) {
            tile_leaf.push_back(i);
            tile_row0.push_back(r0);
        }
    }
    if (tile_leaf.empty()) return;
    write_identity_rows();
    hipStream_t s = dev_.stream();
    upload_vec(d_leaves_, leaves, stage_, s);
    upload_vec(d_tile_leaf_, tile_leaf, stage_, s);
    upload_vec(d_tile_row0_, tile_row0, stage_, s);
    LeafArgs a{};
    a.leaves = d_leaves_.get();
    a.tile_leaf = d_tile_leaf_.get();
    a.tile_row0 = d_tile_row0_.get();
    a.rows[0] = rows_[0].get();
    a.rows[1] = rows_[1].get();
    a.margins = margins_.get();
    a.stride = outputs_;
    a.output = output;
    a.tile_rows = kLeafTile;
    a.n_tiles = (uint32_t)tile_leaf.size();
    dev_.launch("hbr_add_leaves", dim3(a.n_tiles), dim3(256), a);
    dev_.sync();
    stage_.reset();
}

bool Engine::can_walk_gradients(size_t n_nodes) const {
    return dense_u8_ && stride_ == 32 && n_nodes <= 1024 && outputs_ == 1 && labels_loaded_;
}

void Engine::walk_add(const std::vector<uint32_t> &meta, const std::vector<uint32_t> &left,
                      const std::vector<float> &value, uint32_t output, const hbr_device_loss *next_loss) {
    if (!dense_u8_) fail(kRefused, "walk_add: the index has no row-major u8 bins");
    const size_t n = meta.size();
    if (n == 0 || left.size() != n || value.size() != n) fail(kInvalid, "walk_add: one meta, left, value per node");
    for (size_t i = 0; i < n; i++) {
        if (meta[i] >> 31) continue;
        if ((meta[i] & (kMetaDefaultLeft - 1u)) >= n_cols_ || (uint64_t)left[i] + 1 >= n)
            fail(kInvalid, "walk_add: a split names a missing feature or child");
    }
    if (output >= outputs_) fail(kInvalid, "walk_add: no such output");
    hipStream_t s = dev_.stream();
    // the three node tables in one upload
    const size_t bytes = 3 * n * sizeof(uint32_t);
    char *host = static_cast<char *>(stage_.alloc(bytes));
    std::memcpy(host, meta.data(), n * 4);
    std::memcpy(host + n * 4, left.data(), n * 4);
    std::memcpy(host + 2 * n * 4, value.data(), n * 4);
    d_walk_.reserve(bytes);
    char *dev = reinterpret_cast<char *>(d_walk_.get());
    HBR_HIP(hipMemcpyAsync(dev, host, bytes, hipMemcpyHostToDevice, s));
    WalkArgs a{};
    a.masked = masked_ ? 1u : 0u;
    a.mask_at = mask_at_;
    a.meta = reinterpret_cast<const uint32_t *>(dev);
    a.left = reinterpret_cast<const uint32_t *>(dev + n * 4);
    a.value = reinterpret_cast<const float *>(dev + 2 * n * 4);
    a.bins8 = rows8_.get();
    a.margins = margins_.get();
    a.stride = stride_;
    a.n = (uint32_t)n_rows_;
    a.m_stride = outputs_;
    a.output = output;
    a.n_nodes = (uint32_t)n;
    // 32-byte rows and trees that fit the LDS table take the staged walk
    const bool staged = stride_ == 32 && n <= 1024;
    const uint32_t blocks = std::min<uint32_t>(std::max<uint32_t>(1, ceil_div(n_rows_, 256)),
                                               (uint32_t)dev_.cu_count() * (staged ? 8 : 16));
    if (next_loss) {
        // the next round's gradients from the updated margins, in the same pass
        if (!can_walk_gradients(n)) fail(kInvalid, "walk_add: gradients need the staged walk of one output");
        active_pairs_ = nullptr;
        class_outputs_ = 0;
        grains_known_ = false;
        gpair_.resize(n_rows_ ? n_rows_ : 1);
        HBR_HIP(hipMemsetAsync(scale_dev(), 0, sizeof(QScale), s));
        WalkGradArgs wg{};
        wg.w = a;
        wg.g = grad_args(*next_loss);
        row_pairs_live_ = wg.g.pair_rows != nullptr;
        root_partials_ = 0;  // the staged pairs are no longer the walk's
        pair_array_stale_ = false;
        row_pairs_min_hess_ = next_loss->min_hess;
        dev_.launch("hbr_walk_grad32", dim3(blocks), dim3(256), wg);
        FinishArgs f{scale_dev(), n_rows_, wg.g, 0u, 0u};
        set_bounds(*next_loss, f);
        dev_.launch("hbr_finish_scale", dim3(1), dim3(kThreads), f);
        scale_checked_ = false;  // grow_root reads the scale back and checks it
        return;
    }
    dev_.launch(staged ? "hbr_walk_leaves32" : "hbr_walk_leaves", dim3(blocks), dim3(256), a);
    // the staged node tables are released at the next synchronisation
}

std::vector<QBin> Engine::build_rows(const uint32_t *rows, uint64_t m) {
    for (uint64_t i = 0; i < m; i++)
        if (rows[i] >= n_rows_) fail(kRefused, "build: a row beyond the index");
    hipStream_t s = dev_.stream();
    host_rows_.reserve(m ? m : 1);
    host_rows_.upload(rows, m, s);
    const uint32_t slot = alloc_slot();
    HistNode n{};
    n.seg = Seg{0, (uint32_t)m, 0, 0};
    n.slot = slot;
    const std::vector<HistNode> one{n};
    upload_vec(d_hnodes_, one, stage_, s);
    launch_hist(d_hnodes_.get(), (uint32_t)one.size(), &one, nullptr, nullptr, host_rows_.get());
    std::vector<QBin> out(total_bins_);
    hist_.download(out.data(), total_bins_, s, (size_t)slot * total_bins_);
    dev_.sync();
    stage_.reset();
    free_slot(slot);
    return out;
}

// Scratch layout of build_rows_fixed: the row-check word and the plan's
// counts, the node record, the tile plan (at most kFixedMaxTiles tiles),
// then the tile partials.
constexpr uint64_t kFixedNodeAt = 256, kFixedTilesAt = 4096, kFixedMaxTiles = 4096, kFixedPartialAt = 128 * 1024;
static_assert(kFixedTilesAt + (kFixedMaxTiles + 1) * sizeof(HistTile) <= kFixedPartialAt, "tile plan overlaps");

bool Engine::build_rows_fixed(const uint32_t *rows, uint64_t m, double *out, uint8_t *scratch, uint64_t bytes) {
    if (!level_pairs_ && !pairs_staged()) fail(kInvalid, "build: no gradients staged");
    if (m >= (uint64_t)UINT32_MAX) fail(kInvalid, "build: more than 2^32 - 2 rows in one call");
    if (!scratch || bytes <= kFixedPartialAt) fail(kInvalid, "build: no scratch");
    const uint32_t fg = masked_ ? 32u : hist_features_per_group;  // masked rows: one group, the mask word
    const uint32_t groups = dense_u8_ ? ceil_div(n_cols_, fg) : ceil_div(total_bins_, kCsrGroupBins);
    const uint64_t per_tile = (uint64_t)groups * (dense_u8_ ? fg * 256ull : (uint64_t)kCsrGroupBins) * sizeof(QBin);
    const uint64_t budget = bytes - kFixedPartialAt;
    if (per_tile > budget)
        fail(kInvalid, "build (fixed scratch): one row tile's partial sums take " + std::to_string(per_tile) +
                           " bytes, beyond the " + std::to_string(budget) + " bytes the scratch holds for them");
    const uint32_t per_cu = !dense_u8_ ? 1 : fg <= 8 ? 4 : fg <= 16 ? 2 : 1;
    uint64_t target = std::max<uint64_t>(1, (uint64_t)dev_.cu_count() * per_cu * hist_waves / groups);
    target = std::min<uint64_t>({target, budget / per_tile, kFixedMaxTiles - 1});

    hipStream_t s = dev_.stream();
    uint32_t *flag = reinterpret_cast<uint32_t *>(scratch);
    uint32_t *counts = flag + 4;
    HistNode *node = reinterpret_cast<HistNode *>(scratch + kFixedNodeAt);
    HistTile *tiles = reinterpret_cast<HistTile *>(scratch + kFixedTilesAt);
    QBin *partial = reinterpret_cast<QBin *>(scratch + kFixedPartialAt);

    FixedBuildArgs f{};
    f.rows = rows;
    f.m = m;
    f.n_rows = (uint32_t)n_rows_;
    f.total_bins = total_bins_;
    f.flag = flag;
    f.node = node;
    f.bins = reinterpret_cast<QBin *>(out);
    f.out = out;
    f.scale = level_scale_ ? level_scale_ : scale_dev();
    // the word starts at zero on every call (a kernel, not a memset)
    dev_.launch("hbr_fixed_begin", dim3(1), dim3(64), f);
    if (m) {
        const uint64_t blocks = std::min<uint64_t>((m + 255) / 256, (uint64_t)dev_.cu_count() * 8);
        dev_.launch("hbr_fixed_check", dim3((uint32_t)blocks), dim3(256), f);
    }
    dev_.launch("hbr_fixed_node", dim3(1), dim3(64), f);

    PlanArgs p{};
    p.nodes = node;
    p.n_nodes = 1;
    p.target_tiles = (uint32_t)target;
    p.tiles = tiles;
    p.counts = counts;
    p.min_rows = kHistMinRows;
    dev_.launch("hbr_hist_plan", dim3(1), dim3(256), p);

    HistArgs a{};
    a.nodes = node;
    a.tiles = tiles;
    a.counts = counts;
    a.rows[0] = a.rows[1] = rows;
    a.gpair = level_pairs_ ? level_pairs_ : pairs();
    a.scale = f.scale;
    a.class_rows = level_pairs_ ? (uint32_t)n_rows_ : 0u;
    a.csr_ranges = !dense_u8_ && csr_ranges_.size() ? csr_ranges_.get() : nullptr;
    a.bins8 = rows8_.get();
    a.stride = stride_;
    a.n_cols = n_cols_;
    a.row_ptr = row_ptr_.get();
    a.gbins = gbins_.get();
    a.feature_offset = d_fo_.get();
    a.hist = f.bins;
    a.partial = partial;
    a.total_bins = total_bins_;
    a.groups = groups;
    // the pairs live where the last gradient pass wrote them: in the rows'
    // last word after a fused logistic walk (the pair array then holds an
    // earlier round's), else in the pair array
    a.row_pairs = row_pairs_live_ && !level_pairs_ && dense_u8_ && stride_ == 32 && fg == 32 ? 1u : 0u;
    if (pair_array_stale_ && !a.row_pairs && !level_pairs_)
        fail(kRefused, "build: the staged pairs are carried in the rows, which this index's kernel does not read");
    a.masked = masked_ ? 1u : 0u;
    a.mask_at = mask_at_;
    a.min_hess = row_pairs_min_hess_;
    const char *k = !dense_u8_ ? "hbr_hist_csr" : dense8_kernel(fg);
    dev_.launch(k, dim3((uint32_t)(target + 1) * groups), dim3(dense_u8_ ? hist_threads : kCsrThreads), a);
    ReduceArgs r{};
    r.nodes = node;
    r.partial = partial;
    r.hist = f.bins;
    r.feature_offset = d_fo_.get();
    r.n_cols = n_cols_;
    r.total_bins = total_bins_;
    r.groups = groups;
    r.fg = fg;
    r.group_bins = 256;
    r.quarters = 4;
    if (dense_u8_)
        dev_.launch("hbr_hist_reduce", dim3(n_cols_ * 4, 1), dim3(1024), r);
    else
        dev_.launch("hbr_hist_reduce_csr", dim3(ceil_div(total_bins_, 256), 1), dim3(256), r);
    dev_.launch("hbr_fixed_finish", dim3(ceil_div(total_bins_, 256)), dim3(256), f);
    uint32_t bad = 0;
    HBR_HIP(hipMemcpyAsync(&bad, flag, sizeof bad, hipMemcpyDeviceToHost, s));
    dev_.sync();
    return bad == 0;
}

std::vector<uint32_t> Engine::rows_of(const Segment &sg) {
    std::vector<uint32_t> out(sg.len);
    write_identity_rows();
    rows_[sg.buf].download(out.data(), sg.len, dev_.stream(), sg.offset);
    dev_.sync();
    return out;
}

std::vector<QBin> Engine::read_slot(uint32_t slot) {
    if (slot >= slot_cap_) fail(kInvalid, "read_hist: no such slot");
    std::vector<QBin> out(total_bins_);
    hist_.download(out.data(), total_bins_, dev_.stream(), (size_t)slot * total_bins_);
    dev_.sync();
    return out;
}

}  // namespace hbr
