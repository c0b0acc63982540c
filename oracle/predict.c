/*
 * Oracle (test infrastructure): batch prediction.
 *
 * model/predict.rs:60-97 (margin_from_trees: per-output intercepts, then
 * accumulate_forest), :107-193 (trees summed in ascending order per
 * (row, output): out += weight * leaf, f32), tree/regtree.rs:38-66 and
 * tree/mod.rs:52-58 (a present value goes left iff value < split_cond; a
 * missing one follows default_left; a categorical split sends a present
 * value left iff its saturated u32 cast is in the node's category set,
 * tree/mod.rs:34-36), compact/mod.rs:1052-1095.
 */
#include "oracle.h"

#include <math.h>

/* Rust's `v as u32` (saturating: NaN and values below 1 give 0, values at
 * or above 2^32 give u32::MAX, the rest truncate), as tree/mod.rs:34-36
 * applies it before looking the category up. */
static uint32_t category_of(float v) {
    if (!(v >= 1.0f)) return 0;
    if (v >= 4294967296.0f) return UINT32_MAX;
    return (uint32_t)v;
}

/* tree/mod.rs:34-36 and :52-58: a present value of a categorical split goes
 * left iff its category is in the node's set. */
static int in_categories(const or_forest_desc *fd, uint32_t at, float v) {
    const uint32_t c = category_of(v);
    for (uint32_t i = fd->cat_begin[at]; i < fd->cat_end[at]; i++)
        if (fd->categories[i] == c) return 1;
    return 0;
}

static int is_missing(float v, float missing) {
    if (isnan(missing)) return isnan(v);
    return v == missing;
}

void or_predict_margin(const or_forest_desc *fd, const float *x, size_t n, size_t n_cols,
                       float missing, float *out, int32_t *out_leaf) {
    size_t k = fd->n_outputs;
#pragma omp parallel for schedule(static)
    for (size_t r = 0; r < n; r++) {
        const float *row = x + r * n_cols;
        float *o = out + r * k;
        for (size_t c = 0; c < k; c++) o[c] = fd->base_score[c];
        for (size_t t = 0; t < fd->n_trees; t++) {
            uint32_t base = fd->tree_offset[t];
            int32_t nid = 0;
            while (fd->left[base + nid] != -1) {
                const uint32_t at = base + (uint32_t)nid;
                float v = row[fd->split_feature[at]];
                int go_left;
                if (is_missing(v, missing))
                    go_left = fd->default_left[at];
                else if (fd->is_categorical && fd->is_categorical[at])
                    go_left = in_categories(fd, at, v);
                else
                    go_left = v < fd->split_cond[at];
                nid = go_left ? fd->left[at] : fd->right[at];
            }
            if (out_leaf) out_leaf[r * fd->n_trees + t] = nid;
            o[fd->tree_output[t]] += fd->tree_weight[t] * fd->leaf_value[base + (uint32_t)nid];
        }
    }
}
