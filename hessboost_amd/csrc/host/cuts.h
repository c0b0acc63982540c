// Cuts and the binned index on the host, once per dataset.
//
// HistCuts (src/data/quantile.rs:28-296) from XGBoost's weighted quantile
// sketch as hessboost reproduces it (src/data/sketch.rs:59-708), one bin
// per distinct value of a categorical feature (quantile.rs:524-672), and the
// GHistIndex layouts (src/data/ghist.rs:195-257).
#pragma once
#include <cstdint>
#include <vector>

namespace hbr {

struct Cuts {
    std::vector<uint32_t> feature_offset;  // n_cols + 1
    std::vector<float> values;
    // per feature: 1 when its bins are categories (one per distinct value);
    // empty when every feature is numeric
    std::vector<uint8_t> categorical;
    uint32_t n_cols() const { return (uint32_t)feature_offset.size() - 1; }
    uint32_t total_bins() const { return feature_offset.back(); }
    bool is_categorical(uint32_t f) const { return !categorical.empty() && categorical[f] != 0; }
    bool any_categorical() const {
        for (uint8_t c : categorical)
            if (c) return true;
        return false;
    }
    // bin = #{cuts <= v}, clamped to the feature's last bin (global index);
    // a categorical feature's bin holding v exactly, else its first
    uint32_t bin_of(uint32_t f, float v) const;
};

// Dense row-major matrix; `missing` cells (any NaN when missing is NaN)
// absent. categorical: per feature, or null for every feature numeric.
Cuts cuts_from_dense(const float *x, uint64_t n, uint64_t f, uint32_t max_bin, const float *weights, float missing,
                     const uint8_t *categorical = nullptr);
Cuts cuts_from_csr(const uint64_t *row_ptr, const uint32_t *col, const float *val, uint64_t n, uint64_t f,
                   uint32_t max_bin, const float *weights, const uint8_t *categorical = nullptr);

struct Index {
    Cuts cuts;
    uint64_t n_rows = 0, n_cols = 0;
    std::vector<uint64_t> row_ptr;
    uint32_t row_width = 2;           // u16 / u32 global bins
    std::vector<uint16_t> rows16;
    std::vector<uint32_t> rows32;
    uint32_t col_width = 0;           // 0: no columns
    std::vector<uint8_t> cols8;
    std::vector<uint16_t> cols16;
    std::vector<uint32_t> cols32;
    std::vector<uint64_t> missing;    // per feature ceil(n/64) words, or empty
    bool dense = false;
};

Index index_from_dense(const float *x, uint64_t n, uint64_t f, float missing, const Cuts &cuts);
Index index_from_csr(const uint64_t *row_ptr, const uint32_t *col, const float *val, uint64_t n, uint64_t f,
                     const Cuts &cuts);

}  // namespace hbr
