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

/* ---- the reference's batch walk, as its CPU baseline -------------------------
 *
 * tree/compact/mod.rs:1-45 (layout), :73-90 (key), :255-300 (next_below and
 * the numeric test), :701-800 (breadth-first arena), :963-1095 (walk_block:
 * 16 rows in lock-step for the tree's depth, then the tail row by row), with
 * model/predict.rs:203-236 and :1040 (blocks of 256 rows in parallel, every
 * tree walked over a block while its keys stay in cache). Numeric splits and
 * NaN as the missing value only: that is the forest the batch-prediction
 * workload holds. The margins equal or_predict_margin's bit for bit (same
 * leaves, same f32 sums in the same tree order), which is how this walk is
 * checked. */

#include <stdlib.h>
#include <string.h>

#define LS_LANES 16
#define LS_SLOTS (2 * LS_LANES)     /* keys of v, then of -v, per feature */
#define LS_BLOCK 256
#define LS_MAX_DEPTH 16
#define LS_LEAF_KEY 0xffffffffu     /* no key compares greater */

typedef struct { uint32_t slot, key, left, leaf_bits; } ls_node;

/* Monotone u32 key of an f32 (-0 and +0 share one); NaN keys to 0, below
 * every other key, so a missing value never compares greater. */
static inline uint32_t ls_key(float v) {
    if (isnan(v)) return 0;
    float z = v + 0.0f;
    uint32_t b;
    memcpy(&b, &z, 4);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

static float ls_next_below(float c) {
    uint32_t b;
    memcpy(&b, &c, 4);
    if (c > 0.0f) b -= 1;
    else if (c == 0.0f) b = 0x80000001u;   /* -(smallest subnormal) */
    else b += 1;
    float r;
    memcpy(&r, &b, 4);
    return r;
}

typedef struct {
    ls_node *nodes;
    uint32_t *root, *depth;
    size_t n_nodes;
} ls_forest;

/* Breadth-first arena: the child a false compare (and a missing value)
 * selects first, its sibling next to it. */
static int ls_build(const or_forest_desc *fd, ls_forest *lf) {
    size_t total = fd->tree_offset[fd->n_trees];
    lf->nodes = malloc((total ? total : 1) * sizeof(ls_node));
    lf->root = malloc((fd->n_trees ? fd->n_trees : 1) * sizeof(uint32_t));
    lf->depth = malloc((fd->n_trees ? fd->n_trees : 1) * sizeof(uint32_t));
    uint32_t *queue = malloc((total ? total : 1) * sizeof(uint32_t));
    uint32_t *new_id = malloc((total ? total : 1) * sizeof(uint32_t));
    uint32_t *lvl = malloc((total ? total : 1) * sizeof(uint32_t));
    int ok = lf->nodes && lf->root && lf->depth && queue && new_id && lvl;
    size_t out = 0;
    for (size_t t = 0; ok && t < fd->n_trees; t++) {
        const uint32_t base = fd->tree_offset[t];
        size_t head = 0, tail = 0;
        queue[tail++] = 0;
        new_id[base] = (uint32_t)out;
        lvl[base] = 0;
        lf->root[t] = (uint32_t)out;
        lf->depth[t] = 0;
        while (head < tail) {
            const uint32_t old = queue[head++];
            const uint32_t at = base + old;
            const uint32_t id = new_id[at];
            ls_node *nd = &lf->nodes[id];
            if (lvl[at] > lf->depth[t]) lf->depth[t] = lvl[at];
            if (fd->left[at] == -1) {
                nd->slot = 0;
                nd->key = LS_LEAF_KEY;
                nd->left = id;
                memcpy(&nd->leaf_bits, &fd->leaf_value[at], 4);
                out++;
                continue;
            }
            if ((fd->is_categorical && fd->is_categorical[at]) || !isfinite(fd->split_cond[at])) {
                ok = 0;
                break;
            }
            const int mirrored = !fd->default_left[at];
            const int32_t first = mirrored ? fd->right[at] : fd->left[at];
            const int32_t second = mirrored ? fd->left[at] : fd->right[at];
            nd->slot = fd->split_feature[at] * LS_SLOTS + (mirrored ? LS_LANES : 0);
            nd->key = mirrored ? ls_key(-fd->split_cond[at]) : ls_key(ls_next_below(fd->split_cond[at]));
            nd->leaf_bits = 0;
            /* children take the next two arena ids, in queue order */
            const uint32_t child = (uint32_t)(lf->root[t] + tail);
            nd->left = child;
            new_id[base + (uint32_t)first] = child;
            new_id[base + (uint32_t)second] = child + 1;
            lvl[base + (uint32_t)first] = lvl[base + (uint32_t)second] = lvl[at] + 1;
            queue[tail++] = (uint32_t)first;
            queue[tail++] = (uint32_t)second;
            out++;
        }
    }
    lf->n_nodes = out;
    free(queue);
    free(new_id);
    free(lvl);
    return ok ? 0 : -1;
}

static void ls_free(ls_forest *lf) {
    free(lf->nodes);
    free(lf->root);
    free(lf->depth);
}

/* One row through one tree until it reaches a leaf (the tail rows, and
 * trees deeper than the fixed-depth kernel runs). */
static uint32_t ls_leaf_of(const ls_forest *lf, size_t t, const float *row) {
    uint32_t id = lf->root[t];
    for (;;) {
        const ls_node *nd = &lf->nodes[id];
        if (nd->left == id) return id;
        const float v = row[nd->slot / LS_SLOTS];
        const uint32_t k = ls_key((nd->slot & LS_LANES) ? -v : v);
        id = nd->left + (k > nd->key);
    }
}

int or_predict_margin_lockstep(const or_forest_desc *fd, const float *x, size_t n, size_t n_cols,
                               float *out) {
    ls_forest lf;
    if (ls_build(fd, &lf) != 0) {
        ls_free(&lf);
        return -1;
    }
    for (size_t t = 0; t < fd->n_trees; t++)
        for (uint32_t i = fd->tree_offset[t]; i < fd->tree_offset[t + 1]; i++)
            if (fd->left[i] != -1 && fd->split_feature[i] >= n_cols) {
                ls_free(&lf);
                return -1;
            }
    const size_t k = fd->n_outputs;
    const size_t n_blocks = (n + LS_BLOCK - 1) / LS_BLOCK;
    const size_t group_len = LS_SLOTS * n_cols;
#pragma omp parallel
    {
        uint32_t *lanes = malloc((LS_BLOCK / LS_LANES) * group_len * sizeof(uint32_t));
#pragma omp for schedule(static)
        for (size_t b = 0; b < n_blocks; b++) {
            const size_t start = b * LS_BLOCK;
            const size_t rows = (n - start < LS_BLOCK) ? n - start : LS_BLOCK;
            const size_t groups = rows / LS_LANES;
            const float *bx = x + start * n_cols;
            float *bo = out + start * k;
            /* [group][feature][keys of v (16), keys of -v (16)] */
            for (size_t g = 0; g < groups; g++)
                for (size_t j = 0; j < LS_LANES; j++) {
                    const float *row = bx + (g * LS_LANES + j) * n_cols;
                    uint32_t *dst = lanes + g * group_len;
                    for (size_t f = 0; f < n_cols; f++) {
                        dst[f * LS_SLOTS + j] = ls_key(row[f]);
                        dst[f * LS_SLOTS + LS_LANES + j] = ls_key(-row[f]);
                    }
                }
            for (size_t r = 0; r < rows; r++)
                for (size_t c = 0; c < k; c++) bo[r * k + c] = fd->base_score[c];
            for (size_t t = 0; t < fd->n_trees; t++) {
                const float w = fd->tree_weight[t];
                const size_t o = fd->tree_output[t];
                const ls_node *nodes = lf.nodes;
                if (lf.depth[t] <= LS_MAX_DEPTH) {
                    for (size_t g = 0; g < groups; g++) {
                        const uint32_t *grp = lanes + g * group_len;
                        uint32_t nid[LS_LANES];
                        for (int j = 0; j < LS_LANES; j++) nid[j] = lf.root[t];
                        for (uint32_t s = 0; s < lf.depth[t]; s++) {
#pragma GCC unroll 16
                            for (int j = 0; j < LS_LANES; j++) {
                                const ls_node *nd = &nodes[nid[j]];
                                nid[j] = nd->left + (grp[nd->slot + j] > nd->key);
                            }
                        }
                        for (int j = 0; j < LS_LANES; j++) {
                            float leaf;
                            memcpy(&leaf, &nodes[nid[j]].leaf_bits, 4);
                            bo[(g * LS_LANES + j) * k + o] += w * leaf;
                        }
                    }
                } else {
                    for (size_t r = 0; r < groups * LS_LANES; r++) {
                        float leaf;
                        memcpy(&leaf, &nodes[ls_leaf_of(&lf, t, bx + r * n_cols)].leaf_bits, 4);
                        bo[r * k + o] += w * leaf;
                    }
                }
                for (size_t r = groups * LS_LANES; r < rows; r++) {
                    float leaf;
                    memcpy(&leaf, &nodes[ls_leaf_of(&lf, t, bx + r * n_cols)].leaf_bits, 4);
                    bo[r * k + o] += w * leaf;
                }
            }
        }
        free(lanes);
    }
    ls_free(&lf);
    return 0;
}
