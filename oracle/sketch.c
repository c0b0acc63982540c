/*
 * Oracle (test infrastructure): XGBoost's weighted quantile sketch as
 * hessboost restates it, and the cut table built from it.
 *
 * Follows data/sketch.rs:59-680 (WQSketch: summary budget, queue, level-wise
 * prune/merge, query) and data/quantile.rs:65-296 (HistCuts::from_dmatrix,
 * bin_of). Every rank quantity is f32 where the reference keeps f32, f64
 * where it widens.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

typedef struct entry {
    float rmin, rmax, wmin, value;
} entry;

typedef struct vec_e {
    entry *d;
    size_t len, cap;
} vec_e;

static void ve_reserve(vec_e *v, size_t cap) {
    if (cap <= v->cap) return;
    size_t nc = v->cap ? v->cap : 16;
    while (nc < cap) nc *= 2;
    v->d = (entry *)realloc(v->d, nc * sizeof(entry));
    v->cap = nc;
}

static void ve_push(vec_e *v, entry e) {
    ve_reserve(v, v->len + 1);
    v->d[v->len++] = e;
}

static void ve_copy(vec_e *dst, const vec_e *src) {
    ve_reserve(dst, src->len);
    if (src->len) memcpy(dst->d, src->d, src->len * sizeof(entry));
    dst->len = src->len;
}

static void ve_swap(vec_e *a, vec_e *b) {
    vec_e t = *a;
    *a = *b;
    *b = t;
}

static entry mk(float rmin, float rmax, float wmin, float value) {
    entry e = {rmin, rmax, wmin, value};
    return e;
}

/* sketch.rs:59-62 */
static double sketch_epsilon(size_t max_bin, size_t n_samples) {
    size_t n = n_samples > 1 ? n_samples : 1;
    return 1.0 / (double)(max_bin < n ? max_bin : n);
}

/* sketch.rs:66-80 */
static size_t limit_size_level(size_t maxn, double eps) {
    if (maxn == 0) return 1;
    double internal_eps = eps / 2.0;
    for (unsigned nlevel = 1;; nlevel++) {
        size_t limit = (size_t)ceil((double)nlevel / internal_eps) + 1;
        if (limit > maxn) limit = maxn;
        if (((size_t)1 << nlevel) * limit >= maxn) return limit;
    }
}

/* sketch.rs:83-85 */
static size_t summary_budget(size_t max_bin, size_t n) {
    return limit_size_level(n, sketch_epsilon(max_bin, n));
}

/* sketch.rs:89-106 (SetFromSorted): equal values merged, f32 rank sums. */
static void set_from_sorted(const float *v, const float *w, size_t n, vec_e *out) {
    out->len = 0;
    float wsum = 0.0f;
    size_t i = 0;
    while (i < n) {
        float value = v[i];
        float wi = w[i];
        size_t j = i + 1;
        while (j < n && v[j] == value) {
            wi += w[j];
            j++;
        }
        ve_push(out, mk(wsum, wsum + wi, wi, value));
        wsum += wi;
        i = j;
    }
}

/* sketch.rs:131-181 (SetPrune). */
static void set_prune(vec_e *data, size_t maxsize) {
    if (maxsize == 0) {
        data->len = 0;
        return;
    }
    size_t src_size = data->len;
    if (src_size <= maxsize) return;
    if (maxsize == 1) {
        data->len = 1;
        return;
    }
    entry *d = data->d;
    float begin = d[0].rmax;
    float range = d[src_size - 1].rmin - d[0].rmax;
    size_t n = maxsize - 1;
    entry tail = d[src_size - 1];
    entry left = d[1];
    entry right = d[2];
    size_t len = 1, i = 1, lastidx = 0;
    for (size_t k = 1; k < n; k++) {
        float dx2 = 2.0f * (((float)k * range) / (float)n + begin);
        while (i < src_size - 1 && dx2 >= right.rmax + right.rmin) {
            i++;
            left = right;
            if (i < src_size - 1) right = d[i + 1];
        }
        if (i == src_size - 1) break;
        float bound = (left.rmin + left.wmin) + (right.rmax - right.wmin);
        if (dx2 < bound) {
            if (i != lastidx) {
                d[len++] = left;
                lastidx = i;
            }
        } else if (i + 1 != lastidx) {
            d[len++] = right;
            lastidx = i + 1;
        }
    }
    if (lastidx != src_size - 1) d[len++] = tail;
    data->len = len;
}

/* sketch.rs:184-201 (FixError). */
static void fix_error(entry *d, size_t n) {
    float prev_rmin = 0.0f, prev_rmax = 0.0f;
    for (size_t i = 0; i < n; i++) {
        entry *e = &d[i];
        if (e->rmin < prev_rmin)
            e->rmin = prev_rmin;
        else
            prev_rmin = e->rmin;
        if (e->rmax < prev_rmax) e->rmax = prev_rmax;
        float rmin_next = e->rmin + e->wmin;
        if (e->rmax < rmin_next) e->rmax = rmin_next;
        prev_rmax = e->rmax;
    }
}

/* sketch.rs:218-345 (SetCombine): one merge pass (the reference's split
 * merge produces the same entries, sketch.rs:209-217). `this` becomes the
 * merge of this and other. */
static void set_combine(vec_e *this_, const vec_e *other, vec_e *ws) {
    if (other->len == 0) return;
    if (this_->len == 0) {
        ve_copy(this_, other);
        return;
    }
    const entry *a = this_->d, *b = other->d;
    size_t na = this_->len, nb = other->len;
    ws->len = 0;
    ve_reserve(ws, na + nb);
    entry *out = ws->d;
    size_t o = 0, ia = 0, ib = 0;
    float aprev = 0.0f, bprev = 0.0f;
    while (ia < na && ib < nb) {
        entry ea = a[ia], eb = b[ib];
        int eq = ea.value == eb.value;
        int lt = ea.value < eb.value;
        int take_a = eq | lt;
        int take_b = !lt;
        float rmin = (take_a ? ea.rmin : aprev) + (take_b ? eb.rmin : bprev);
        float rmax = (take_a ? ea.rmax : (ea.rmax - ea.wmin)) +
                     (take_b ? eb.rmax : (eb.rmax - eb.wmin));
        float wmin = eq ? ea.wmin + eb.wmin : (lt ? ea.wmin : eb.wmin);
        out[o++] = mk(rmin, rmax, wmin, take_a ? ea.value : eb.value);
        if (take_a) aprev = ea.rmin + ea.wmin;
        if (take_b) bprev = eb.rmin + eb.wmin;
        ia += (size_t)take_a;
        ib += (size_t)take_b;
    }
    for (; ia < na; ia++) {
        entry ea = a[ia];
        float next = ib < nb ? (b[ib].rmax - b[ib].wmin) : b[nb - 1].rmax;
        out[o++] = mk(ea.rmin + bprev, ea.rmax + next, ea.wmin, ea.value);
        aprev = ea.rmin + ea.wmin;
    }
    for (; ib < nb; ib++) {
        entry eb = b[ib];
        float next = ia < na ? (a[ia].rmax - a[ia].wmin) : a[na - 1].rmax;
        out[o++] = mk(eb.rmin + aprev, eb.rmax + next, eb.wmin, eb.value);
        bprev = eb.rmin + eb.wmin;
    }
    ws->len = o;
    fix_error(ws->d, o);
    ve_swap(this_, ws);
}

/* sketch.rs:458-509 (QueryCutValues). */
static void query_cut_values(const entry *data, size_t n, size_t max_bin,
                             float **out, size_t *out_len, size_t *out_cap) {
#define PUSH(val)                                                              \
    do {                                                                       \
        if (*out_len == *out_cap) {                                            \
            *out_cap = *out_cap ? *out_cap * 2 : 16;                           \
            *out = (float *)realloc(*out, *out_cap * sizeof(float));           \
        }                                                                      \
        (*out)[(*out_len)++] = (val);                                          \
    } while (0)
    if (n == 0) {
        PUSH(1e-5f);
        return;
    }
    float last_cut = data[0].value;
    size_t next_value = 1;
    while (next_value < n && data[next_value].value <= last_cut) next_value++;
    if (n <= max_bin) {
        while (next_value < n) {
            float cpt = data[next_value].value;
            PUSH(cpt);
            last_cut = cpt;
            next_value++;
            while (next_value < n && data[next_value].value <= last_cut) next_value++;
        }
    } else {
        double total = (double)data[n - 1].rmax;
        size_t q = 0;
        for (size_t i = 1; i < max_bin; i++) {
            double rank2 = 2.0 * ((double)i * total / (double)max_bin);
            while (q < n - 2 && rank2 >= (double)(data[q + 1].rmin + data[q + 1].rmax)) q++;
            float lhs = (data[q].rmin + data[q].wmin) + (data[q + 1].rmax - data[q + 1].wmin);
            entry queried = rank2 < (double)lhs ? data[q] : data[q + 1];
            float cpt = queried.value;
            if (cpt <= last_cut) {
                while (next_value < n && data[next_value].value <= last_cut) next_value++;
                if (next_value == n) break;
                cpt = data[next_value].value;
            } else if (next_value < n && data[next_value].value <= cpt) {
                next_value++;
                while (next_value < n && data[next_value].value <= cpt) next_value++;
            }
            PUSH(cpt);
            last_cut = cpt;
        }
    }
    float cpt = data[n - 1].value;
    PUSH(cpt + (fabsf(cpt) + 1e-5f));
#undef PUSH
}

/* A record of every summary a traced sketch forms (or_sketch_trace): the
 * entries, and the range [lo, hi) of the caller's value indices it covers. */
typedef struct sk_trace {
    float *buf;          /* 4 floats per entry */
    size_t cap, len;     /* in entries */
    uint64_t *recs;      /* 6 per record: offset, count, lo, hi, kind, prune size (0: none) */
    size_t rec_cap, n_recs;
    int overflow;
} sk_trace;

/* The sketch of one feature (sketch.rs:512-680). */
typedef struct sketch {
    size_t max_bin, limit_size;
    float *qv, *qw;
    size_t qlen;
    vec_e *levels;
    size_t nlevels;
    vec_e temp, ws;
    size_t num_elements;
    /* tracing only: the caller's index of the value being pushed, the
     * first index of the queued batch, each level's and temp's coverage */
    sk_trace *tr;
    size_t pos, batch_lo, t_lo, t_hi;
    size_t *lv_lo, *lv_hi;
} sketch;

enum { TR_FROM_SORTED = 0, TR_PRUNE = 1, TR_COMBINE = 2, TR_SUMMARY = 3, TR_FINAL = 4 };

static void tr_record(sketch *s, const vec_e *v, size_t lo, size_t hi, int kind, size_t pruned_to) {
    sk_trace *t = s->tr;
    if (!t) return;
    if (t->len + v->len > t->cap || t->n_recs >= t->rec_cap) {
        t->overflow = 1;
        return;
    }
    memcpy(t->buf + 4 * t->len, v->d, v->len * sizeof(entry));
    uint64_t *r = t->recs + 6 * t->n_recs++;
    r[0] = t->len;
    r[1] = v->len;
    r[2] = lo;
    r[3] = hi;
    r[4] = (uint64_t)kind;
    r[5] = pruned_to;
    t->len += v->len;
}

static void tr_levels(sketch *s, size_t nlevels) {
    if (!s->tr) return;
    s->lv_lo = (size_t *)realloc(s->lv_lo, nlevels * sizeof(size_t));
    s->lv_hi = (size_t *)realloc(s->lv_hi, nlevels * sizeof(size_t));
    s->lv_lo[nlevels - 1] = s->lv_hi[nlevels - 1] = 0;
}

static void sk_init(sketch *s, size_t n_values, size_t max_bin) {
    memset(s, 0, sizeof(*s));
    s->max_bin = max_bin;
    s->limit_size = summary_budget(max_bin, n_values);
    s->qv = (float *)malloc(2 * s->limit_size * sizeof(float));
    s->qw = (float *)malloc(2 * s->limit_size * sizeof(float));
}

static void sk_free(sketch *s) {
    free(s->qv);
    free(s->qw);
    for (size_t l = 0; l < s->nlevels; l++) free(s->levels[l].d);
    free(s->levels);
    free(s->temp.d);
    free(s->ws.d);
    free(s->lv_lo);
    free(s->lv_hi);
}

/* Total order of f32 values (f32::total_cmp) as an unsigned key. */
static uint32_t total_key(float v) {
    uint32_t b;
    memcpy(&b, &v, 4);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

typedef struct keyed {
    uint32_t key;
    uint32_t idx;
} keyed;

static int cmp_keyed(const void *x, const void *y) {
    const keyed *a = (const keyed *)x, *b = (const keyed *)y;
    if (a->key != b->key) return a->key < b->key ? -1 : 1;
    return a->idx < b->idx ? -1 : (a->idx > b->idx);
}

/* sketch.rs:660-674 (PushSummary): level-wise merge with carry. */
static void sk_push_summary(sketch *s) {
    size_t l = 0;
    for (;;) {
        if (s->nlevels <= l) {
            s->levels = (vec_e *)realloc(s->levels, (l + 1) * sizeof(vec_e));
            memset(&s->levels[l], 0, sizeof(vec_e));
            s->nlevels = l + 1;
            tr_levels(s, s->nlevels);
        }
        const size_t keep = s->limit_size;
        set_prune(&s->temp, keep);
        tr_record(s, &s->temp, s->t_lo, s->t_hi, TR_PRUNE, keep);
        if (s->tr && s->levels[l].len) s->t_lo = s->lv_lo[l];  /* the level holds the batches just before */
        set_combine(&s->temp, &s->levels[l], &s->ws);
        tr_record(s, &s->temp, s->t_lo, s->t_hi, TR_COMBINE, 0);
        s->levels[l].len = 0;
        if (s->temp.len <= s->limit_size) break;
        l++;
    }
    ve_swap(&s->levels[l], &s->temp);
    if (s->tr) {
        s->lv_lo[l] = s->t_lo;
        s->lv_hi[l] = s->t_hi;
    }
}

/* sketch.rs:619-656 (Queue::PopSummary + PushSummary). The queue is sorted
 * by f32 total order; equal keys are identical values, so any order among
 * them gives the same summary for whole-number weights. */
static void sk_flush(sketch *s) {
    size_t n = s->qlen;
    keyed *k = (keyed *)malloc((n ? n : 1) * sizeof(keyed));
    for (size_t i = 0; i < n; i++) {
        k[i].key = total_key(s->qv[i]);
        k[i].idx = (uint32_t)i;
    }
    qsort(k, n, sizeof(keyed), cmp_keyed);
    float *v = (float *)malloc((n ? n : 1) * sizeof(float));
    float *w = (float *)malloc((n ? n : 1) * sizeof(float));
    for (size_t i = 0; i < n; i++) {
        v[i] = s->qv[k[i].idx];
        w[i] = s->qw[k[i].idx];
    }
    set_from_sorted(v, w, n, &s->temp);
    free(k);
    free(v);
    free(w);
    s->qlen = 0;
    s->t_lo = s->batch_lo;
    s->t_hi = s->pos;
    s->batch_lo = s->pos;
    tr_record(s, &s->temp, s->t_lo, s->t_hi, TR_FROM_SORTED, 0);
    sk_push_summary(s);
}

/* sketch.rs:584-617 (Push / Queue::Push). */
static void sk_push(sketch *s, float value, float weight) {
    if (weight == 0.0f) return;
    s->num_elements++;
    if (s->qlen > 0 && s->qv[s->qlen - 1] == value) {
        s->qw[s->qlen - 1] += weight;
        return;
    }
    if (s->qlen == 2 * s->limit_size) sk_flush(s);
    s->qv[s->qlen] = value;
    s->qw[s->qlen] = weight;
    s->qlen++;
}

/* sketch.rs:687-697 (GetSummary) and :703-708 (cut_values). */
static void sk_cut_values(sketch *s, float **out, size_t *out_len, size_t *out_cap) {
    size_t budget = summary_budget(s->max_bin, s->num_elements);
    sk_flush(s);
    size_t prune_size = budget > s->limit_size ? budget : s->limit_size;
    vec_e sum = {0};
    size_t lo = s->pos, hi = s->pos;
    for (size_t l = 0; l < s->nlevels; l++) {
        if (s->tr && s->levels[l].len) {
            lo = s->lv_lo[l];  /* levels run from the newest batches to the oldest */
            if (sum.len == 0) hi = s->lv_hi[l];
        }
        set_combine(&sum, &s->levels[l], &s->ws);
        set_prune(&sum, prune_size);
        tr_record(s, &sum, lo, hi, TR_SUMMARY, prune_size);
    }
    set_prune(&sum, budget);
    tr_record(s, &sum, lo, hi, TR_FINAL, budget);
    size_t mb = sum.len < s->max_bin ? sum.len : s->max_bin;
    query_cut_values(sum.d, sum.len, mb, out, out_len, out_cap);
    free(sum.d);
}

static int is_missing(float v, float missing) {
    if (isnan(missing)) return isnan(v);
    return v == missing;
}

static or_cuts *assemble(float **per, size_t *per_len, size_t f) {
    or_cuts *c = (or_cuts *)calloc(1, sizeof(or_cuts));
    c->n_features = f;
    c->feature_offset = (uint32_t *)malloc((f + 1) * sizeof(uint32_t));
    size_t total = 0;
    for (size_t j = 0; j < f; j++) total += per_len[j];
    c->cut_values = (float *)malloc((total ? total : 1) * sizeof(float));
    size_t o = 0;
    c->feature_offset[0] = 0;
    for (size_t j = 0; j < f; j++) {
        memcpy(c->cut_values + o, per[j], per_len[j] * sizeof(float));
        o += per_len[j];
        c->feature_offset[j + 1] = (uint32_t)o;
        free(per[j]);
    }
    return c;
}

/* quantile.rs:65-78, :122-238: every feature's present values, in row order,
 * into its own sketch. */
/* f32::total_cmp as an integer key */
static int32_t total_key32(float v) {
    int32_t b;
    memcpy(&b, &v, 4);
    return b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
}

static int cmp_total(const void *a, const void *b) {
    int32_t ka = total_key32(*(const float *)a), kb = total_key32(*(const float *)b);
    return (ka > kb) - (ka < kb);
}

/* A categorical feature's cuts (quantile.rs:524-672): its present values
 * sorted by total_cmp and deduplicated by bit pattern, then one bin per
 * distinct value by `!=` (build_categorical_cuts); a feature with no
 * present value keeps one degenerate bin at 0. `vals` is consumed. */
static void categorical_cuts(float *vals, size_t m, float **out, size_t *out_len) {
    qsort(vals, m, sizeof(float), cmp_total);
    size_t k = 0;
    for (size_t i = 0; i < m; i++) {
        uint32_t a, b;
        memcpy(&a, &vals[i], 4);
        if (k) memcpy(&b, &vals[k - 1], 4);
        if (k == 0 || a != b) vals[k++] = vals[i];
    }
    float *cuts = (float *)malloc((k ? k : 1) * sizeof(float));
    size_t n = 0;
    if (k == 0)
        cuts[n++] = 0.0f;
    else {
        cuts[n++] = vals[0];
        for (size_t i = 1; i < k; i++)
            if (vals[i - 1] != vals[i]) cuts[n++] = vals[i];
    }
    *out = cuts;
    *out_len = n;
}

or_cuts *or_cuts_from_dense(const float *x, size_t n, size_t f, size_t max_bin,
                            const float *weights, float missing) {
    return or_cuts_from_dense_typed(x, n, f, max_bin, weights, missing, NULL);
}

or_cuts *or_cuts_from_dense_typed(const float *x, size_t n, size_t f, size_t max_bin,
                                  const float *weights, float missing, const uint8_t *categorical) {
    float **per = (float **)calloc(f, sizeof(float *));
    size_t *per_len = (size_t *)calloc(f, sizeof(size_t));
#pragma omp parallel for schedule(dynamic, 1)
    for (size_t j = 0; j < f; j++) {
        size_t present = 0;
        for (size_t r = 0; r < n; r++) present += !is_missing(x[r * f + j], missing);
        if (categorical && categorical[j]) {
            float *vals = (float *)malloc((present ? present : 1) * sizeof(float));
            size_t m = 0;
            for (size_t r = 0; r < n; r++)
                if (!is_missing(x[r * f + j], missing)) vals[m++] = x[r * f + j];
            categorical_cuts(vals, m, &per[j], &per_len[j]);
            free(vals);
            continue;
        }
        sketch s;
        sk_init(&s, present, max_bin);
        for (size_t r = 0; r < n; r++) {
            float v = x[r * f + j];
            if (is_missing(v, missing)) continue;
            sk_push(&s, v, weights ? weights[r] : 1.0f);
        }
        size_t cap = 0;
        sk_cut_values(&s, &per[j], &per_len[j], &cap);
        sk_free(&s);
    }
    or_cuts *c = assemble(per, per_len, f);
    free(per);
    free(per_len);
    if (categorical) {
        c->is_categorical = (uint8_t *)malloc(f ? f : 1);
        for (size_t j = 0; j < f; j++) c->is_categorical[j] = categorical[j] ? 1 : 0;
    }
    return c;
}

or_cuts *or_cuts_from_csr(const size_t *row_ptr, const uint32_t *col,
                          const float *val, size_t n, size_t f, size_t max_bin,
                          const float *weights) {
    return or_cuts_from_csr_typed(row_ptr, col, val, n, f, max_bin, weights, NULL);
}

or_cuts *or_cuts_from_csr_typed(const size_t *row_ptr, const uint32_t *col,
                                const float *val, size_t n, size_t f, size_t max_bin,
                                const float *weights, const uint8_t *categorical) {
    /* CSC view: each feature's stored entries in row order (quantile.rs:219-232). */
    size_t *count = (size_t *)calloc(f + 1, sizeof(size_t));
    size_t nnz = row_ptr[n];
    for (size_t e = 0; e < nnz; e++) count[col[e] + 1]++;
    for (size_t j = 0; j < f; j++) count[j + 1] += count[j];
    uint32_t *crow = (uint32_t *)malloc((nnz ? nnz : 1) * sizeof(uint32_t));
    float *cval = (float *)malloc((nnz ? nnz : 1) * sizeof(float));
    size_t *fill = (size_t *)malloc((f + 1) * sizeof(size_t));
    memcpy(fill, count, (f + 1) * sizeof(size_t));
    for (size_t r = 0; r < n; r++)
        for (size_t e = row_ptr[r]; e < row_ptr[r + 1]; e++) {
            size_t p = fill[col[e]]++;
            crow[p] = (uint32_t)r;
            cval[p] = val[e];
        }
    float **per = (float **)calloc(f, sizeof(float *));
    size_t *per_len = (size_t *)calloc(f, sizeof(size_t));
#pragma omp parallel for schedule(dynamic, 1)
    for (size_t j = 0; j < f; j++) {
        size_t lo = count[j], hi = count[j + 1];
        if (categorical && categorical[j]) {
            float *vals = (float *)malloc((hi - lo ? hi - lo : 1) * sizeof(float));
            memcpy(vals, cval + lo, (hi - lo) * sizeof(float));
            categorical_cuts(vals, hi - lo, &per[j], &per_len[j]);
            free(vals);
            continue;
        }
        sketch s;
        sk_init(&s, hi - lo, max_bin);
        for (size_t p = lo; p < hi; p++) sk_push(&s, cval[p], weights ? weights[crow[p]] : 1.0f);
        size_t cap = 0;
        sk_cut_values(&s, &per[j], &per_len[j], &cap);
        sk_free(&s);
    }
    or_cuts *c = assemble(per, per_len, f);
    if (categorical) {
        c->is_categorical = (uint8_t *)malloc(f ? f : 1);
        for (size_t j = 0; j < f; j++) c->is_categorical[j] = categorical[j] ? 1 : 0;
    }
    free(per);
    free(per_len);
    free(count);
    free(crow);
    free(cval);
    free(fill);
    return c;
}

void or_cuts_free(or_cuts *c) {
    if (!c) return;
    free(c->feature_offset);
    free(c->cut_values);
    free(c->is_categorical);
    free(c);
}

size_t or_cuts_total_bins(const or_cuts *c) { return c->feature_offset[c->n_features]; }

/* quantile.rs:285-296: upper_bound count of cuts <= v, clamped to the last bin. */
uint32_t or_bin_of(const or_cuts *c, size_t f, float v) {
    size_t start = c->feature_offset[f], end = c->feature_offset[f + 1];
    if (c->is_categorical && c->is_categorical[f]) {
        /* the bin whose category equals v (binary search by partial_cmp), else bin 0 */
        size_t lo = 0, hi = end - start;
        while (lo < hi) {
            size_t mid = (lo + hi) / 2;
            float cv = c->cut_values[start + mid];
            if (cv == v) return (uint32_t)(start + mid);
            if (cv < v)
                lo = mid + 1;
            else
                hi = mid;
        }
        return (uint32_t)start;
    }
    size_t lo = 0, hi = end - start;
    const float *cuts = c->cut_values + start;
    while (lo < hi) {
        size_t mid = (lo + hi) / 2;
        if (cuts[mid] <= v)
            lo = mid + 1;
        else
            hi = mid;
    }
    size_t n_cuts = end - start;
    size_t local = lo < (n_cuts ? n_cuts - 1 : 0) ? lo : (n_cuts ? n_cuts - 1 : 0);
    return (uint32_t)(start + local);
}

/* ---- test hooks: the summary operations on caller arrays -----------------
 * An entry is 4 floats (rmin, rmax, wmin, value). Used by tests/test_oracle.py
 * to check the summaries against brute-force ranks and against plain
 * restatements of XGBoost's SetPrune / SetCombine. */

static vec_e wrap(const float *e, size_t n) {
    vec_e v = {0};
    ve_reserve(&v, n ? n : 1);
    if (n) memcpy(v.d, e, n * sizeof(entry));
    v.len = n;
    return v;
}

size_t or_summary_budget(size_t max_bin, size_t n) { return summary_budget(max_bin, n); }

size_t or_summary_from_sorted(const float *v, const float *w, size_t n, float *out) {
    vec_e o = {0};
    set_from_sorted(v, w, n, &o);
    if (o.len) memcpy(out, o.d, o.len * sizeof(entry));
    size_t len = o.len;
    free(o.d);
    return len;
}

size_t or_summary_prune(float *entries, size_t n, size_t maxsize) {
    vec_e v = wrap(entries, n);
    set_prune(&v, maxsize);
    if (v.len) memcpy(entries, v.d, v.len * sizeof(entry));
    size_t len = v.len;
    free(v.d);
    return len;
}

size_t or_summary_combine(const float *a, size_t na, const float *b, size_t nb, float *out) {
    vec_e va = wrap(a, na), vb = wrap(b, nb), ws = {0};
    set_combine(&va, &vb, &ws);
    if (va.len) memcpy(out, va.d, va.len * sizeof(entry));
    size_t len = va.len;
    free(va.d);
    free(vb.d);
    free(ws.d);
    return len;
}

size_t or_summary_query(const float *entries, size_t n, size_t max_bin, float *out) {
    float *cuts = NULL;
    size_t len = 0, cap = 0;
    query_cut_values((const entry *)entries, n, max_bin, &cuts, &len, &cap);
    if (len) memcpy(out, cuts, len * sizeof(float));
    free(cuts);
    return len;
}

/* One feature's streaming sketch over values[0..n) with weights (NULL: 1),
 * recording every summary it forms: after each queue flush (from sorted),
 * each prune and each merge of the level-wise carry, each merge of the
 * final summary, and the final summary. Returns the number of cut values
 * written to `cuts` (at most max_bin + 1); -1 when the buffers overflow. */
long or_sketch_trace(const float *values, const float *weights, size_t n, size_t max_bin, float *buf,
                     size_t buf_entries, uint64_t *recs, size_t rec_cap, size_t *n_recs, float *cuts) {
    sk_trace t = {buf, buf_entries, 0, recs, rec_cap, 0, 0};
    size_t present = 0;
    for (size_t i = 0; i < n; i++) present += (weights ? weights[i] : 1.0f) != 0.0f;
    sketch s;
    sk_init(&s, present, max_bin);
    s.tr = &t;
    for (size_t i = 0; i < n; i++) {
        s.pos = i;
        sk_push(&s, values[i], weights ? weights[i] : 1.0f);
    }
    s.pos = n;
    float *out = NULL;
    size_t len = 0, cap = 0;
    sk_cut_values(&s, &out, &len, &cap);
    sk_free(&s);
    if (len) memcpy(cuts, out, len * sizeof(float));
    free(out);
    *n_recs = t.n_recs;
    return t.overflow ? -1 : (long)len;
}
