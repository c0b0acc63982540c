/*
 * Oracle (test infrastructure): growing one hist tree.
 *
 * builder/hist/mod.rs:261-343 (build_inner: root statistics by sum_rows,
 * root histogram, finish_tree), :459-503 (grow_depthwise: frontier order,
 * terminal children at the depth limit), :505-573 (grow_lossguide: a
 * std BinaryHeap ordered by loss_chg.total_cmp), :639-690 (prepare_split:
 * expand, store child stats and bounds), :692-737 (build_children: stable
 * partition, smaller child built, sibling = parent - built);
 * builder/partition.rs:106-242 (routing), :244-313 (with_sibling);
 * builder/mod.rs:143-193 (expand with f32 child weights and covers,
 * split_gain, child_bounds); builder/shared.rs:174-187 (finalize_leaf_values
 * with calc_weight_bounded); tree/regtree.rs:599-601 (scale_leaves);
 * training/round.rs:422-424 (tree_eta = eta as f32); categorical splits
 * (builder/mod.rs:105-120, :175-182: the set recorded as the left child,
 * its codes sorted into the tree's category pool; quantile.rs:316-333 and
 * partition.rs:146-160: rows routed by their bin's code).
 */
#include "oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

typedef struct entry_t {
    int64_t nid;
    size_t depth;
    uint32_t *rows;
    size_t n_rows;
    double *hist; /* NULL for terminal nodes */
    or_split best;
    double lower, upper;
} entry_t;

typedef struct store_t {
    double *g, *h, *lower, *upper;
    size_t len, cap;
} store_t;

static void store_push(store_t *s, double g, double h, double lo, double up) {
    if (s->len == s->cap) {
        s->cap = s->cap ? 2 * s->cap : 64;
        s->g = (double *)realloc(s->g, s->cap * sizeof(double));
        s->h = (double *)realloc(s->h, s->cap * sizeof(double));
        s->lower = (double *)realloc(s->lower, s->cap * sizeof(double));
        s->upper = (double *)realloc(s->upper, s->cap * sizeof(double));
    }
    s->g[s->len] = g;
    s->h[s->len] = h;
    s->lower[s->len] = lo;
    s->upper[s->len] = up;
    s->len++;
}

static or_node leaf_node(float value, float sum_hess) {
    or_node n;
    memset(&n, 0, sizeof(n));
    n.default_left = 1;
    n.left = -1;
    n.right = -1;
    n.leaf_value = value;
    n.sum_hess = sum_hess;
    n.split_bin = -2;
    return n;
}

static void tree_push(or_tree *t, or_node n) {
    if (t->n_nodes == t->cap) {
        t->cap = t->cap ? 2 * t->cap : 64;
        t->nodes = (or_node *)realloc(t->nodes, t->cap * sizeof(or_node));
    }
    t->nodes[t->n_nodes++] = n;
}

typedef struct ctx_t {
    const or_index *ix;
    const float *gpair;
    const or_params *p;
    or_tree *tree;
    store_t store;
    int32_t *leaf_of_row;
    size_t total_bins;
    size_t limit;
} ctx_t;

static int dir_of(const or_params *p, uint32_t f) {
    return (p->monotone && f < p->n_monotone) ? p->monotone[f] : 0;
}

static void record_leaf(ctx_t *c, entry_t *e) {
    if (c->leaf_of_row)
        for (size_t i = 0; i < e->n_rows; i++) c->leaf_of_row[e->rows[i]] = (int32_t)e->nid;
    free(e->rows);
    free(e->hist);
    e->rows = NULL;
    e->hist = NULL;
}

/* constraints.rs child_bounds: the midpoint of the bounded child weights. */
static void child_bounds(double lo, double up, int dir, double wl, double wr, double *l_lo,
                         double *l_up, double *r_lo, double *r_up) {
    *l_lo = lo;
    *l_up = up;
    *r_lo = lo;
    *r_up = up;
    if (dir == 0) return;
    /* f64::midpoint: halves first only where the sum could overflow. */
    const double HI = DBL_MAX / 2.0, LO = DBL_MIN * 2.0;
    double mid;
    if (fabs(wl) <= HI && fabs(wr) <= HI)
        mid = (wl + wr) / 2.0;
    else if (fabs(wl) < LO)
        mid = wl + wr / 2.0;
    else if (fabs(wr) < LO)
        mid = wl / 2.0 + wr;
    else
        mid = wl / 2.0 + wr / 2.0;
    if (dir > 0) {
        *l_up = mid;
        *r_lo = mid;
    } else {
        *l_lo = mid;
        *r_up = mid;
    }
}

typedef struct pending_t {
    entry_t entry;
    int64_t left_id, right_id;
    double l_lo, l_up, r_lo, r_up;
    int terminal;
} pending_t;

/* A category code: the saturating `cut as u32` (in_category_set). */
static uint32_t category_code(float v) {
    if (!(v >= 0.0f)) return 0;
    if (v >= 4294967296.0f) return 0xffffffffu;
    return (uint32_t)v;
}

static int cmp_u32(const void *a, const void *b) {
    uint32_t x = *(const uint32_t *)a, y = *(const uint32_t *)b;
    return (x > y) - (x < y);
}

/* The categories of a categorical split's set (its local bins' codes,
 * sorted: BestSplit's `set.sort_unstable()`), appended to the tree's pool. */
static void record_categories(ctx_t *c, or_node *n, const or_split *b) {
    const uint32_t fs = c->ix->cuts->feature_offset[b->feature];
    const uint32_t nb = c->ix->cuts->feature_offset[b->feature + 1] - fs;
    or_tree *t = c->tree;
    n->is_categorical = 1;
    n->cat_begin = (uint32_t)t->n_categories;
    for (uint32_t i = 0; i < nb; i++) {
        if (!(b->cat_left[i / 32] >> (i % 32) & 1u)) continue;
        if (t->n_categories == t->cat_cap) {
            t->cat_cap = t->cat_cap ? 2 * t->cat_cap : 64;
            t->categories = (uint32_t *)realloc(t->categories, t->cat_cap * sizeof(uint32_t));
        }
        t->categories[t->n_categories++] = category_code(c->ix->cuts->cut_values[fs + i]);
    }
    n->cat_end = (uint32_t)t->n_categories;
    qsort(t->categories + n->cat_begin, n->cat_end - n->cat_begin, sizeof(uint32_t), cmp_u32);
}

static pending_t prepare_split(ctx_t *c, entry_t *e) {
    pending_t s;
    const or_split *b = &e->best;
    int dir = dir_of(c->p, b->feature);
    if (b->categorical) /* bounds in the orientation the split was scored in (builder/mod.rs:175-182) */
        child_bounds(e->lower, e->upper, dir, b->w_right, b->w_left, &s.r_lo, &s.r_up, &s.l_lo, &s.l_up);
    else
        child_bounds(e->lower, e->upper, dir, b->w_left, b->w_right, &s.l_lo, &s.l_up, &s.r_lo, &s.r_up);
    or_node *n = &c->tree->nodes[e->nid];
    n->split_cond = b->categorical ? 0.0f : (b->bin >= 0 ? c->ix->cuts->cut_values[b->bin] : -FLT_MAX);
    n->split_feature = b->feature;
    n->default_left = b->default_left;
    n->split_bin = b->bin;
    if (b->categorical) record_categories(c, n, b);
    int64_t left_id = (int64_t)c->tree->n_nodes;
    n->left = (int32_t)left_id;
    n->right = (int32_t)(left_id + 1);
    n->split_gain = (float)b->loss_chg;
    or_node ln = leaf_node((float)b->w_left, (float)b->left_h);
    or_node rn = leaf_node((float)b->w_right, (float)b->right_h);
    ln.stat_g = b->left_g;
    ln.stat_h = b->left_h;
    rn.stat_g = b->right_g;
    rn.stat_h = b->right_h;
    tree_push(c->tree, ln);
    tree_push(c->tree, rn);
    store_push(&c->store, b->left_g, b->left_h, s.l_lo, s.l_up);
    store_push(&c->store, b->right_g, b->right_h, s.r_lo, s.r_up);
    s.left_id = left_id;
    s.right_id = left_id + 1;
    s.terminal = c->p->grow_policy == OR_GROW_DEPTHWISE && e->depth + 1 >= c->limit;
    s.entry = *e;
    return s;
}

size_t or_partition(const or_index *ix, const uint32_t *rows, size_t m, uint32_t feature,
                    int64_t bin, int default_left, uint32_t *out_left, uint32_t *out_right) {
    size_t nl = 0, nr = 0;
    uint32_t fs = ix->cuts->feature_offset[feature];
    for (size_t i = 0; i < m; i++) {
        uint32_t r = rows[i];
        int64_t gb = or_index_feature_bin(ix, r, feature);
        int left;
        if (gb < 0)
            left = default_left;
        else if (ix->cols) {
            int64_t limit = bin >= 0 ? bin + 1 - (int64_t)fs : 0;
            left = (gb - (int64_t)fs) < limit;
        } else
            left = bin >= 0 && gb <= bin;
        if (left)
            out_left[nl++] = r;
        else
            out_right[nr++] = r;
    }
    return nl;
}

size_t or_partition_categorical(const or_index *ix, const uint32_t *rows, size_t m, uint32_t feature,
                                const uint32_t *cat_left, int default_left, uint32_t *out_left,
                                uint32_t *out_right) {
    /* categories_left (quantile.rs:316-333): a bin goes left when its code
     * is one of the set's codes */
    const uint32_t fs = ix->cuts->feature_offset[feature];
    const uint32_t nb = ix->cuts->feature_offset[feature + 1] - fs;
    uint8_t *left_bin = (uint8_t *)calloc(nb ? nb : 1, 1);
    for (uint32_t i = 0; i < nb; i++) {
        if (!(cat_left[i / 32] >> (i % 32) & 1u)) continue;
        const uint32_t code = category_code(ix->cuts->cut_values[fs + i]);
        for (uint32_t k = 0; k < nb; k++)
            if (category_code(ix->cuts->cut_values[fs + k]) == code) left_bin[k] = 1;
    }
    size_t nl = 0, nr = 0;
    for (size_t i = 0; i < m; i++) {
        uint32_t r = rows[i];
        int64_t gb = or_index_feature_bin(ix, r, feature);
        int left = gb < 0 ? default_left : left_bin[gb - (int64_t)fs];
        if (left)
            out_left[nl++] = r;
        else
            out_right[nr++] = r;
    }
    free(left_bin);
    return nl;
}

static void build_children(ctx_t *c, pending_t *s, entry_t *out_l, entry_t *out_r) {
    entry_t *e = &s->entry;
    const or_split *b = &e->best;
    uint32_t *lrows = (uint32_t *)malloc((e->n_rows ? e->n_rows : 1) * sizeof(uint32_t));
    uint32_t *rrows = (uint32_t *)malloc((e->n_rows ? e->n_rows : 1) * sizeof(uint32_t));
    size_t nl = b->categorical ? or_partition_categorical(c->ix, e->rows, e->n_rows, b->feature, b->cat_left,
                                                          b->default_left, lrows, rrows)
                               : or_partition(c->ix, e->rows, e->n_rows, b->feature, b->bin, b->default_left,
                                              lrows, rrows);
    size_t nr = e->n_rows - nl;
    free(e->rows);
    e->rows = NULL;
    memset(out_l, 0, sizeof(*out_l));
    memset(out_r, 0, sizeof(*out_r));
    out_l->nid = s->left_id;
    out_r->nid = s->right_id;
    out_l->depth = out_r->depth = e->depth + 1;
    out_l->rows = lrows;
    out_l->n_rows = nl;
    out_r->rows = rrows;
    out_r->n_rows = nr;
    out_l->lower = s->l_lo;
    out_l->upper = s->l_up;
    out_r->lower = s->r_lo;
    out_r->upper = s->r_up;
    out_l->best.bin = -1;
    out_l->best.default_left = 1;
    out_r->best.bin = -1;
    out_r->best.default_left = 1;
    if (s->terminal) {
        free(e->hist);
        e->hist = NULL;
        return;
    }
    int left_smaller = nl <= nr;
    double *small = (double *)malloc(2 * c->total_bins * sizeof(double));
    or_build_hist(c->ix, left_smaller ? lrows : rrows, left_smaller ? nl : nr, c->gpair, small);
    double *parent = e->hist;
    for (size_t i = 0; i < 2 * c->total_bins; i++) parent[i] = parent[i] - small[i];
    e->hist = NULL;
    out_l->hist = left_smaller ? small : parent;
    out_r->hist = left_smaller ? parent : small;
    or_evaluate(c->ix, out_l->hist, b->left_g, b->left_h, s->l_lo, s->l_up, c->p, &out_l->best);
    or_evaluate(c->ix, out_r->hist, b->right_g, b->right_h, s->r_lo, s->r_up, c->p, &out_r->best);
}

/* std::collections::BinaryHeap (max-heap) with sift_up / sift_down_to_bottom,
 * ordered by best.loss_chg under f64::total_cmp. */
static int64_t total_cmp_key(double x) {
    int64_t b;
    memcpy(&b, &x, 8);
    return b ^ (int64_t)(((uint64_t)(b >> 63)) >> 1);
}

static int le(const entry_t *a, const entry_t *b) {
    return total_cmp_key(a->best.loss_chg) <= total_cmp_key(b->best.loss_chg);
}

typedef struct heap_t {
    entry_t *d;
    size_t len, cap;
} heap_t;

static size_t sift_up(heap_t *h, size_t start, size_t pos) {
    entry_t elem = h->d[pos];
    while (pos > start) {
        size_t parent = (pos - 1) / 2;
        if (le(&elem, &h->d[parent])) break;
        h->d[pos] = h->d[parent];
        pos = parent;
    }
    h->d[pos] = elem;
    return pos;
}

static void heap_push(heap_t *h, entry_t e) {
    if (h->len == h->cap) {
        h->cap = h->cap ? 2 * h->cap : 64;
        h->d = (entry_t *)realloc(h->d, h->cap * sizeof(entry_t));
    }
    h->d[h->len++] = e;
    sift_up(h, 0, h->len - 1);
}

static void sift_down_to_bottom(heap_t *h, size_t pos) {
    size_t end = h->len, start = pos;
    entry_t elem = h->d[pos];
    size_t child = 2 * pos + 1;
    while (child + 2 <= end) { /* child <= end.saturating_sub(2) */
        if (le(&h->d[child], &h->d[child + 1])) child += 1;
        h->d[pos] = h->d[child];
        pos = child;
        child = 2 * pos + 1;
    }
    if (end > 0 && child == end - 1) {
        h->d[pos] = h->d[child];
        pos = child;
    }
    h->d[pos] = elem;
    sift_up(h, start, pos);
}

static int heap_pop(heap_t *h, entry_t *out) {
    if (h->len == 0) return 0;
    entry_t item = h->d[--h->len];
    if (h->len > 0) {
        entry_t top = h->d[0];
        h->d[0] = item;
        item = top;
        sift_down_to_bottom(h, 0);
    }
    *out = item;
    return 1;
}

/* Test hook: a record of the loss-guided queue's pushes and pops, for
 * tests/test_oracle.py (best-first order under equal gains). One record per
 * event: kind (0 push, 1 pop), node id, loss_chg bits, expandable. */
static uint64_t *g_lg_trace;
static size_t g_lg_cap, g_lg_len;

void or_lossguide_trace(uint64_t *buf, size_t cap) {
    g_lg_trace = buf;
    g_lg_cap = cap;
    g_lg_len = 0;
}

size_t or_lossguide_trace_len(void) { return g_lg_len; }

static void lg_event(int kind, const entry_t *e, int expandable) {
    if (!g_lg_trace || g_lg_len >= g_lg_cap) return;
    uint64_t *r = g_lg_trace + 4 * g_lg_len++;
    uint64_t bits;
    memcpy(&bits, &e->best.loss_chg, 8);
    r[0] = (uint64_t)kind;
    r[1] = (uint64_t)e->nid;
    r[2] = bits;
    r[3] = (uint64_t)expandable;
}

static void finish_tree(ctx_t *c) {
    double lambda = (double)(float)c->p->lambda, alpha = (double)(float)c->p->alpha;
    double mds = (double)(float)c->p->max_delta_step;
    double mcw = (double)(float)c->p->min_child_weight;
    float eta = (float)c->p->eta;
    for (size_t id = 0; id < c->tree->n_nodes; id++) {
        or_node *n = &c->tree->nodes[id];
        if (n->left != -1) continue;
        double g = c->store.g[id], h = c->store.h[id];
        double w;
        if (h < mcw || h <= 0.0)
            w = 0.0;
        else {
            double t = g > alpha ? g - alpha : (g < -alpha ? g + alpha : 0.0);
            w = -t / (h + lambda);
            if (mds > 0.0) w = w < -mds ? -mds : (w > mds ? mds : w);
        }
        double lo = c->store.lower[id], up = c->store.upper[id];
        if (w < lo) w = lo;
        if (w > up) w = up;
        n->leaf_value = (float)w * eta;
    }
}

or_tree *or_grow_tree(const or_index *ix, const float *gpair, const or_params *p,
                      int32_t *leaf_of_row) {
    ctx_t c;
    memset(&c, 0, sizeof(c));
    c.ix = ix;
    c.gpair = gpair;
    c.p = p;
    c.tree = (or_tree *)calloc(1, sizeof(or_tree));
    c.leaf_of_row = leaf_of_row;
    c.total_bins = or_cuts_total_bins(ix->cuts);
    c.limit = p->max_depth > 0 ? (size_t)p->max_depth : SIZE_MAX;

    entry_t root;
    memset(&root, 0, sizeof(root));
    root.n_rows = ix->n_rows;
    root.rows = (uint32_t *)malloc((ix->n_rows ? ix->n_rows : 1) * sizeof(uint32_t));
    for (size_t r = 0; r < ix->n_rows; r++) root.rows[r] = (uint32_t)r;
    double stats[2];
    or_sum_rows(gpair, root.rows, root.n_rows, stats);
    root.hist = (double *)malloc(2 * c.total_bins * sizeof(double));
    or_build_hist(ix, root.rows, root.n_rows, gpair, root.hist);
    root.lower = -INFINITY;
    root.upper = INFINITY;
    or_node rn = leaf_node(0.0f, (float)stats[1]);
    rn.stat_g = stats[0];
    rn.stat_h = stats[1];
    tree_push(c.tree, rn);
    store_push(&c.store, stats[0], stats[1], -INFINITY, INFINITY);
    or_evaluate(ix, root.hist, stats[0], stats[1], root.lower, root.upper, p, &root.best);

    if (p->grow_policy == OR_GROW_DEPTHWISE) {
        entry_t *frontier = (entry_t *)malloc(sizeof(entry_t));
        size_t nf = 1;
        frontier[0] = root;
        size_t depth = 0;
        while (depth < c.limit && nf > 0) {
            pending_t *pend = (pending_t *)malloc(nf * sizeof(pending_t));
            size_t np = 0;
            for (size_t i = 0; i < nf; i++) {
                if (or_split_valid(&frontier[i].best, p))
                    pend[np++] = prepare_split(&c, &frontier[i]);
                else
                    record_leaf(&c, &frontier[i]);
            }
            free(frontier);
            frontier = (entry_t *)malloc((2 * np ? 2 * np : 1) * sizeof(entry_t));
            for (size_t i = 0; i < np; i++) build_children(&c, &pend[i], &frontier[2 * i], &frontier[2 * i + 1]);
            nf = 2 * np;
            free(pend);
            depth++;
        }
        for (size_t i = 0; i < nf; i++) record_leaf(&c, &frontier[i]);
        free(frontier);
    } else {
        size_t max_leaves = p->max_leaves > 0 ? (size_t)p->max_leaves : SIZE_MAX;
        heap_t h = {0};
        heap_push(&h, root);
        lg_event(0, &root, root.depth < c.limit && or_split_valid(&root.best, p));
        size_t n_leaves = 1;
        entry_t e;
        while (heap_pop(&h, &e)) {
            lg_event(1, &e, e.depth < c.limit && or_split_valid(&e.best, p));
            if (n_leaves >= max_leaves) {
                record_leaf(&c, &e);
                break;
            }
            if (!(e.depth < c.limit && or_split_valid(&e.best, p))) {
                record_leaf(&c, &e);
                continue;
            }
            pending_t s = prepare_split(&c, &e);
            entry_t l, r;
            build_children(&c, &s, &l, &r);
            n_leaves++;
            heap_push(&h, l);
            lg_event(0, &l, l.depth < c.limit && or_split_valid(&l.best, p));
            heap_push(&h, r);
            lg_event(0, &r, r.depth < c.limit && or_split_valid(&r.best, p));
        }
        for (size_t i = 0; i < h.len; i++) record_leaf(&c, &h.d[i]);
        free(h.d);
    }
    finish_tree(&c);
    free(c.store.g);
    free(c.store.h);
    free(c.store.lower);
    free(c.store.upper);
    return c.tree;
}

void or_tree_free(or_tree *t) {
    if (!t) return;
    free(t->nodes);
    free(t->categories);
    free(t);
}

size_t or_tree_n_nodes(const or_tree *t) { return t->n_nodes; }
size_t or_tree_n_categories(const or_tree *t) { return t->n_categories; }
const uint32_t *or_tree_categories(const or_tree *t) { return t->categories; }
const or_node *or_tree_nodes(const or_tree *t) { return t->nodes; }
