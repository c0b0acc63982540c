/*
 * Oracle (test infrastructure): the binned index (GHistIndex).
 *
 * Follows data/ghist.rs:213-257 (layout rules: u16/u32 global row bins,
 * columns kept iff cells <= 2 * entries, a missing bitmap iff some cell is
 * missing, u8/u16/u32 local column bins by the widest feature, `dense` for
 * complete rows in feature order) and ghist.rs:163-176 (Column::get,
 * missing_bit).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static int is_missing(float v, float missing) {
    if (isnan(missing)) return isnan(v);
    return v == missing;
}

static void set_row_bin(or_index *ix, size_t e, uint32_t bin) {
    if (ix->row_width == 2)
        ((uint16_t *)ix->rows)[e] = (uint16_t)bin;
    else
        ((uint32_t *)ix->rows)[e] = bin;
}

static uint32_t get_row_bin(const or_index *ix, size_t e) {
    return ix->row_width == 2 ? ((const uint16_t *)ix->rows)[e] : ((const uint32_t *)ix->rows)[e];
}

static void set_col_bin(or_index *ix, size_t f, size_t r, uint32_t local) {
    size_t at = f * ix->n_rows + r;
    if (ix->col_width == 1)
        ((uint8_t *)ix->cols)[at] = (uint8_t)local;
    else if (ix->col_width == 2)
        ((uint16_t *)ix->cols)[at] = (uint16_t)local;
    else
        ((uint32_t *)ix->cols)[at] = local;
}

static void layout(or_index *ix) {
    const or_cuts *c = ix->cuts;
    size_t cells = ix->n_rows * ix->n_cols;
    size_t entries = ix->row_ptr[ix->n_rows];
    size_t total = or_cuts_total_bins(c);
    ix->row_width = total <= 65536 ? 2 : 4;
    ix->rows = malloc((entries ? entries : 1) * (size_t)ix->row_width);
    size_t widest = 0;
    for (size_t f = 0; f < ix->n_cols; f++) {
        size_t nb = c->feature_offset[f + 1] - c->feature_offset[f];
        if (nb > widest) widest = nb;
    }
    ix->col_width = 0;
    ix->cols = NULL;
    ix->missing = NULL;
    if (cells <= 2 * entries) {
        ix->col_width = widest <= 256 ? 1 : (widest <= 65536 ? 2 : 4);
        ix->cols = calloc(cells ? cells : 1, (size_t)ix->col_width);
        if (entries < cells) {
            size_t words = (ix->n_rows + 63) / 64;
            ix->missing = (uint64_t *)calloc(words * ix->n_cols ? words * ix->n_cols : 1, 8);
            for (size_t f = 0; f < ix->n_cols; f++)
                for (size_t w = 0; w < words; w++) {
                    size_t valid = ix->n_rows - w * 64;
                    if (valid > 64) valid = 64;
                    ix->missing[f * words + w] = valid == 64 ? ~(uint64_t)0 : (((uint64_t)1 << valid) - 1);
                }
        }
    }
}

static void store(or_index *ix, size_t r, size_t e, size_t f, uint32_t global) {
    set_row_bin(ix, e, global);
    if (ix->cols) {
        set_col_bin(ix, f, r, global - ix->cuts->feature_offset[f]);
        if (ix->missing) {
            size_t words = (ix->n_rows + 63) / 64;
            ix->missing[f * words + (r >> 6)] &= ~((uint64_t)1 << (r & 63));
        }
    }
}

or_index *or_index_from_dense(const float *x, size_t n, size_t f, float missing,
                              or_cuts *cuts) {
    or_index *ix = (or_index *)calloc(1, sizeof(or_index));
    ix->n_rows = n;
    ix->n_cols = f;
    ix->cuts = cuts;
    ix->row_ptr = (size_t *)malloc((n + 1) * sizeof(size_t));
    ix->row_ptr[0] = 0;
    for (size_t r = 0; r < n; r++) {
        size_t cnt = 0;
        for (size_t j = 0; j < f; j++) cnt += !is_missing(x[r * f + j], missing);
        ix->row_ptr[r + 1] = ix->row_ptr[r] + cnt;
    }
    layout(ix);
    ix->dense = ix->row_ptr[n] == n * f;
    /* Blocks of 64 rows own whole words of every feature's missing bitmap. */
    size_t blocks = (n + 63) / 64;
#pragma omp parallel for schedule(static)
    for (size_t blk = 0; blk < blocks; blk++) {
        size_t hi = (blk + 1) * 64 < n ? (blk + 1) * 64 : n;
        for (size_t r = blk * 64; r < hi; r++) {
            size_t e = ix->row_ptr[r];
            for (size_t j = 0; j < f; j++) {
                float v = x[r * f + j];
                if (is_missing(v, missing)) continue;
                store(ix, r, e++, j, or_bin_of(cuts, j, v));
            }
        }
    }
    return ix;
}

or_index *or_index_from_csr(const size_t *row_ptr, const uint32_t *col,
                            const float *val, size_t n, size_t f, or_cuts *cuts) {
    or_index *ix = (or_index *)calloc(1, sizeof(or_index));
    ix->n_rows = n;
    ix->n_cols = f;
    ix->cuts = cuts;
    ix->row_ptr = (size_t *)malloc((n + 1) * sizeof(size_t));
    memcpy(ix->row_ptr, row_ptr, (n + 1) * sizeof(size_t));
    layout(ix);
    int dense = 1;
    for (size_t r = 0; r < n && dense; r++) {
        if (row_ptr[r + 1] - row_ptr[r] != f) dense = 0;
        for (size_t e = row_ptr[r]; e < row_ptr[r + 1] && dense; e++)
            if (col[e] != e - row_ptr[r]) dense = 0;
    }
    ix->dense = dense;
    size_t blocks = (n + 63) / 64;
#pragma omp parallel for schedule(static)
    for (size_t blk = 0; blk < blocks; blk++) {
        size_t hi = (blk + 1) * 64 < n ? (blk + 1) * 64 : n;
        for (size_t r = blk * 64; r < hi; r++)
            for (size_t e = row_ptr[r]; e < row_ptr[r + 1]; e++)
                store(ix, r, e, col[e], or_bin_of(cuts, col[e], val[e]));
    }
    return ix;
}

void or_index_free(or_index *ix) {
    if (!ix) return;
    free(ix->row_ptr);
    free(ix->rows);
    free(ix->cols);
    free(ix->missing);
    free(ix);
}

/* ghist.rs:341-360 (feature_bin): a column read when columns are kept, else
 * the row's stored entries. */
int64_t or_index_feature_bin(const or_index *ix, size_t r, size_t f) {
    uint32_t fs = ix->cuts->feature_offset[f], fe = ix->cuts->feature_offset[f + 1];
    if (ix->cols) {
        size_t words = (ix->n_rows + 63) / 64;
        if (ix->missing && ((ix->missing[f * words + (r >> 6)] >> (r & 63)) & 1)) return -1;
        size_t at = f * ix->n_rows + r;
        uint32_t local = ix->col_width == 1 ? ((uint8_t *)ix->cols)[at]
                         : ix->col_width == 2 ? ((uint16_t *)ix->cols)[at]
                                              : ((uint32_t *)ix->cols)[at];
        return (int64_t)fs + local;
    }
    for (size_t e = ix->row_ptr[r]; e < ix->row_ptr[r + 1]; e++) {
        uint32_t b = get_row_bin(ix, e);
        if (b >= fs && b < fe) return b;
    }
    return -1;
}
