/*
 * Oracle (test infrastructure): CpuBackend::build and sum_rows.
 *
 * tree/hist/mod.rs:399-428 (SumOrder, sum_order), :510-547 (build: Chain
 * for nodes below 8,192 rows or dense indexes swept by feature, otherwise
 * Blocked), :556-607 (accumulate_blocks: first block's partial, then each
 * later block added in block order), walk.rs:50-173 (accumulate: each bin
 * receives its rows in ascending row order from +0.0);
 * builder/shared.rs:164-170 (sum_rows: one row-order chain).
 */
#include "oracle.h"

#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ROWS_PER_TASK 4096
#define PARALLEL_THRESHOLD (2 * ROWS_PER_TASK)
#define GATHER_MAX_ROWS ((size_t)1 << 18)

size_t or_sum_order_grain(int dense, size_t index_rows, size_t len, int contiguous) {
    if (len < PARALLEL_THRESHOLD || (dense && (contiguous || index_rows <= GATHER_MAX_ROWS)))
        return 0;
    size_t blocks = len / ROWS_PER_TASK;
    return (len + blocks - 1) / blocks;
}

static inline uint32_t row_bin(const or_index *ix, size_t e) {
    return ix->row_width == 2 ? ((const uint16_t *)ix->rows)[e] : ((const uint32_t *)ix->rows)[e];
}

/* One chain over rows[0..m) into out (zeroed by the caller). */
static void chain(const or_index *ix, const uint32_t *rows, size_t m, const float *gpair,
                  double *out) {
    for (size_t i = 0; i < m; i++) {
        size_t r = rows[i];
        double g = (double)gpair[2 * r], h = (double)gpair[2 * r + 1];
        for (size_t e = ix->row_ptr[r]; e < ix->row_ptr[r + 1]; e++) {
            uint32_t b = row_bin(ix, e);
            out[2 * b] += g;
            out[2 * b + 1] += h;
        }
    }
}

/* A dense index's chain swept feature by feature: each bin still receives its
 * rows in ascending order (walk.rs:266-283), so the bits equal `chain`. */
static void chain_by_feature(const or_index *ix, const uint32_t *rows, size_t m,
                             const float *gpair, double *out) {
    size_t f_n = ix->n_cols;
#pragma omp parallel for schedule(dynamic, 1)
    for (size_t f = 0; f < f_n; f++) {
        for (size_t i = 0; i < m; i++) {
            size_t r = rows[i];
            uint32_t b = row_bin(ix, r * f_n + f);
            out[2 * b] += (double)gpair[2 * r];
            out[2 * b + 1] += (double)gpair[2 * r + 1];
        }
    }
}

static int is_contiguous(const uint32_t *rows, size_t m) {
    if (m == 0) return 0;
    for (size_t i = 0; i < m; i++)
        if (rows[i] != rows[0] + i) return 0;
    return 1;
}

void or_build_hist(const or_index *ix, const uint32_t *rows, size_t m, const float *gpair,
                   double *out) {
    size_t total = or_cuts_total_bins(ix->cuts);
    memset(out, 0, 2 * total * sizeof(double));
    if (m < PARALLEL_THRESHOLD) {
        chain(ix, rows, m, gpair, out);
        return;
    }
    int dense_cols = ix->dense && ix->cols;
    int contiguous = dense_cols && is_contiguous(rows, m);
    size_t grain = or_sum_order_grain(ix->dense, ix->n_rows, m, contiguous);
    if (grain == 0) {
        if (dense_cols)
            chain_by_feature(ix, rows, m, gpair, out);
        else
            chain(ix, rows, m, gpair, out);
        return;
    }
    size_t blocks = (m + grain - 1) / grain;
    int threads = 1;
#ifdef _OPENMP
    threads = omp_get_max_threads();
#endif
    size_t wave = (size_t)threads;
    if (wave > blocks) wave = blocks;
    if (wave < 1) wave = 1;
    double *partials = (double *)malloc(wave * 2 * total * sizeof(double));
    for (size_t first = 0; first < blocks; first += wave) {
        size_t built = blocks - first < wave ? blocks - first : wave;
#pragma omp parallel for schedule(static, 1)
        for (size_t w = 0; w < built; w++) {
            size_t b = first + w;
            size_t lo = b * grain, hi = lo + grain < m ? lo + grain : m;
            double *p = partials + w * 2 * total;
            memset(p, 0, 2 * total * sizeof(double));
            chain(ix, rows + lo, hi - lo, gpair, p);
        }
        size_t start = 0;
        if (first == 0) {
            memcpy(out, partials, 2 * total * sizeof(double));
            start = 1;
        }
#pragma omp parallel for schedule(static)
        for (size_t i = 0; i < 2 * total; i++)
            for (size_t w = start; w < built; w++) out[i] += partials[w * 2 * total + i];
    }
    free(partials);
}

void or_sum_rows(const float *gpair, const uint32_t *rows, size_t m, double *out) {
    double g = 0.0, h = 0.0;
    for (size_t i = 0; i < m; i++) {
        g += (double)gpair[2 * (size_t)rows[i]];
        h += (double)gpair[2 * (size_t)rows[i] + 1];
    }
    out[0] = g;
    out[1] = h;
}
