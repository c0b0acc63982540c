/*
 * Oracle (test infrastructure): hist split search, sequential semantics.
 *
 * tree/gain.rs:82-116 (RegParams rounded to f32, threshold_l1, calc_weight),
 * tree/constraints.rs (child_bounds midpoint, satisfies, bounded weight),
 * builder/shared.rs:89-141 (xgb_calc_weight, apply_bounds, xgb_weight: f64
 * weight rounded to f32 then bounded; xgb_gain_given_weight with w*w in f32;
 * xgb_node_gain rounded to f32), builder/split.rs:37-56 (loss_chg: each
 * child's gain rounded to f32, added in f32, minus root_gain in f32),
 * :391-419 (for_each_numeric_split: forward pass, then a backward pass only
 * on a non-dense index whose forward total differs from the node total),
 * builder/mod.rs:313-342 (need_replace, xgb_update), :167-193 (found,
 * valid), hist/search.rs:171-259 (feature-order merge; a feature with at
 * most one bin has no candidate); builder/categorical.rs:48-170 (a
 * categorical feature's one-hot or weight-sorted partition sweep).
 */
#include "oracle.h"

#include <math.h>
#include <string.h>

typedef struct reg {
    double lambda, alpha, max_delta_step, min_child_weight;
} reg;

static reg reg_of(const or_params *p) {
    reg r;
    r.lambda = (double)(float)p->lambda;
    r.alpha = (double)(float)p->alpha;
    r.max_delta_step = (double)(float)p->max_delta_step;
    r.min_child_weight = (double)(float)p->min_child_weight;
    return r;
}

static double threshold_l1(double g, double alpha) {
    if (g > alpha) return g - alpha;
    if (g < -alpha) return g + alpha;
    return 0.0;
}

static double xgb_calc_weight(double g, double h, const reg *r) {
    if (h <= 0.0) return 0.0;
    double w = -threshold_l1(g, r->alpha) / (h + r->lambda);
    if (r->max_delta_step != 0.0 && fabs(w) > r->max_delta_step) w = copysign(r->max_delta_step, w);
    return w;
}

static float apply_bounds(float w, float lower, float upper) {
    if (w < lower) return lower;
    if (w > upper) return upper;
    return w;
}

static float xgb_weight(double g, double h, const reg *r, double lower, double upper) {
    float w = (float)xgb_calc_weight(g, h, r);
    return apply_bounds(w, (float)lower, (float)upper);
}

static double gain_given_weight(double g, double h, const reg *r, float w) {
    float w2 = w * w;
    return -(2.0 * g * (double)w + (h + r->lambda) * (double)w2 + 2.0 * r->alpha * (double)fabsf(w));
}

float or_node_gain(double g, double h, double lower, double upper, const or_params *p) {
    reg r = reg_of(p);
    if (h <= 0.0) return 0.0f;
    return (float)gain_given_weight(g, h, &r, xgb_weight(g, h, &r, lower, upper));
}

double or_calc_weight(double g, double h, const or_params *p) {
    reg r = reg_of(p);
    if (h < r.min_child_weight || h <= 0.0) return 0.0;
    double w = -threshold_l1(g, r.alpha) / (h + r.lambda);
    if (r.max_delta_step > 0.0) w = w < -r.max_delta_step ? -r.max_delta_step : (w > r.max_delta_step ? r.max_delta_step : w);
    return w;
}

static int satisfies(int dir, double wl, double wr) {
    if (dir > 0) return wl <= wr;
    if (dir < 0) return wl >= wr;
    return 1;
}

static int children_valid(double lh, double rh, double mcw) {
    return lh > 0.0 && rh > 0.0 && lh >= mcw && rh >= mcw;
}

static int need_replace(float incumbent, uint32_t inc_feature, float loss, uint32_t feature) {
    if (isinf(loss)) return 0;
    if (inc_feature <= feature) return loss > incumbent;
    return !(incumbent > loss);
}

typedef struct scan_ctx {
    reg r;
    double lower, upper;
    float root_gain;
    or_split *best;
} scan_ctx;

static void offer(scan_ctx *c, uint32_t f, int dir, int64_t bin, int default_left, double lg,
                  double lh, double rg, double rh) {
    if (!children_valid(lh, rh, c->r.min_child_weight)) return;
    float wl = xgb_weight(lg, lh, &c->r, c->lower, c->upper);
    float wr = xgb_weight(rg, rh, &c->r, c->lower, c->upper);
    if (!satisfies(dir, (double)wl, (double)wr)) return;
    float gain = (float)gain_given_weight(lg, lh, &c->r, wl) + (float)gain_given_weight(rg, rh, &c->r, wr);
    float loss = gain - c->root_gain;
    or_split *b = c->best;
    if (!need_replace((float)b->loss_chg, b->feature, loss, f)) return;
    b->loss_chg = (double)loss;
    b->feature = f;
    b->bin = bin;
    b->default_left = default_left;
    b->left_g = lg;
    b->left_h = lh;
    b->right_g = rg;
    b->right_h = rh;
    b->w_left = (double)wl;
    b->w_right = (double)wr;
    b->categorical = 0;
}

/* ---- categorical features (builder/categorical.rs:48-170) ---------------- */

#define MAX_CAT_TO_ONEHOT 4
#define MAX_CAT_THRESHOLD 64

/* A feature's best categorical candidate in XGBoost's orientation: the set
 * is its right child, default_left routes missing values. */
typedef struct cat_local {
    int has;
    float loss, wl, wr;
    int default_left;
    double lg, lh, rg, rh;
} cat_local;

/* SplitScorer::loss_chg (builder/split.rs:37-56); 0 when not offered. */
static int score_children(const scan_ctx *c, int dir, double lg, double lh, double rg, double rh, float *loss,
                          float *wl, float *wr) {
    if (!children_valid(lh, rh, c->r.min_child_weight)) return 0;
    *wl = xgb_weight(lg, lh, &c->r, c->lower, c->upper);
    *wr = xgb_weight(rg, rh, &c->r, c->lower, c->upper);
    if (!satisfies(dir, (double)*wl, (double)*wr)) return 0;
    float gain = (float)gain_given_weight(lg, lh, &c->r, *wl) + (float)gain_given_weight(rg, rh, &c->r, *wr);
    *loss = gain - c->root_gain;
    return 1;
}

/* SplitEntry::Update on the feature's own entry, which starts at loss 0. */
static int cat_offer(const scan_ctx *c, int dir, uint32_t f, cat_local *local, int default_left, double lg,
                     double lh, double rg, double rh) {
    float loss, wl, wr;
    if (!score_children(c, dir, lg, lh, rg, rh, &loss, &wl, &wr)) return 0;
    if (!need_replace(local->has ? local->loss : 0.0f, f, loss, f)) return 0;
    local->has = 1;
    local->loss = loss;
    local->wl = wl;
    local->wr = wr;
    local->default_left = default_left;
    local->lg = lg;
    local->lh = lh;
    local->rg = rg;
    local->rh = rh;
    return 1;
}

/* p_best->Update: the feature's candidate against the node's best; the
 * recorded split puts the set on the left (children and missing direction
 * swapped, Children::swapped / Score::swapped). `set` lists local bins. */
static void cat_merge(or_split *best, const cat_local *local, uint32_t f, const size_t *set, size_t n_set) {
    if (!local->has) return;
    if (!need_replace((float)best->loss_chg, best->feature, local->loss, f)) return;
    best->loss_chg = (double)local->loss;
    best->feature = f;
    best->bin = -1;
    best->default_left = !local->default_left;
    best->left_g = local->rg;
    best->left_h = local->rh;
    best->right_g = local->lg;
    best->right_h = local->lh;
    best->w_left = (double)local->wr;
    best->w_right = (double)local->wl;
    best->categorical = 1;
    memset(best->cat_left, 0, sizeof(best->cat_left));
    for (size_t i = 0; i < n_set; i++) best->cat_left[set[i] / 32] |= 1u << (set[i] % 32);
}

static void sweep(const scan_ctx *c, const double *st, size_t n, double tg, double th, int dir, uint32_t f,
                  or_split *best) {
    if (n > OR_MAX_CAT_BINS) return;
    if (n < MAX_CAT_TO_ONEHOT) {
        /* EnumerateOneHot: each category alone, missing values on either side */
        double pg = 0.0, ph = 0.0;
        for (size_t i = 0; i < n; i++) {
            pg += st[2 * i];
            ph += st[2 * i + 1];
        }
        double mg = tg - pg, mh = th - ph;
        cat_local local = {0};
        size_t chosen = 0;
        for (size_t i = 0; i < n; i++) {
            double rg = st[2 * i], rh = st[2 * i + 1];
            if (cat_offer(c, dir, f, &local, 1, tg - rg, th - rh, rg, rh)) chosen = i;
            rg += mg;
            rh += mh;
            if (cat_offer(c, dir, f, &local, 0, tg - rg, th - rh, rg, rh)) chosen = i;
        }
        cat_merge(best, &local, f, &chosen, 1);
        return;
    }
    /* EnumeratePart: categories stably sorted by weight (CalcWeightCat) */
    float keys[OR_MAX_CAT_BINS];
    size_t sorted[OR_MAX_CAT_BINS];
    for (size_t i = 0; i < n; i++) {
        double g = st[2 * i], h = st[2 * i + 1];
        keys[i] = h < c->r.min_child_weight ? 0.0f : (float)xgb_calc_weight(g, h, &c->r);
        sorted[i] = i;
    }
    for (size_t i = 1; i < n; i++) { /* stable insertion sort */
        size_t v = sorted[i], j = i;
        while (j > 0 && keys[v] < keys[sorted[j - 1]]) {
            sorted[j] = sorted[j - 1];
            j--;
        }
        sorted[j] = v;
    }
    size_t depth = n < MAX_CAT_THRESHOLD ? n : MAX_CAT_THRESHOLD;
    for (int forward = 1; forward >= 0; forward--) {
        double ag = 0.0, ah = 0.0;
        cat_local local = {0};
        size_t best_partition = 0;
        for (size_t step = 0; step + 1 < depth; step++) {
            size_t j = forward ? step : n - 1 - step;
            ag += st[2 * sorted[j]];
            ah += st[2 * sorted[j] + 1];
            size_t partition = forward ? step + 1 : j;
            int offered = forward ? cat_offer(c, dir, f, &local, 1, tg - ag, th - ah, ag, ah)
                                  : cat_offer(c, dir, f, &local, 0, ag, ah, tg - ag, th - ah);
            if (offered) best_partition = partition;
        }
        cat_merge(best, &local, f, sorted, best_partition);
    }
}

void or_sweep_categorical(const double *stats, size_t n, double total_g, double total_h, double lower,
                          double upper, int dir, const or_params *p, uint32_t feature, or_split *best) {
    scan_ctx c;
    c.r = reg_of(p);
    c.lower = lower;
    c.upper = upper;
    c.root_gain = or_node_gain(total_g, total_h, lower, upper, p);
    c.best = best;
    sweep(&c, stats, n, total_g, total_h, dir, feature, best);
}

void or_evaluate(const or_index *ix, const double *hist, double total_g, double total_h,
                 double lower, double upper, const or_params *p, or_split *out) {
    memset(out, 0, sizeof(*out));
    out->loss_chg = 0.0;
    out->feature = 0;
    out->bin = -1;
    out->default_left = 1;
    scan_ctx c;
    c.r = reg_of(p);
    c.lower = lower;
    c.upper = upper;
    c.root_gain = or_node_gain(total_g, total_h, lower, upper, p);
    c.best = out;
    const uint32_t *off = ix->cuts->feature_offset;
    for (size_t f = 0; f < ix->n_cols; f++) {
        size_t fs = off[f], fe = off[f + 1];
        int dir = (p->monotone && f < p->n_monotone) ? p->monotone[f] : 0;
        if (ix->cuts->is_categorical && ix->cuts->is_categorical[f]) {
            /* category_stats (hist/search.rs:402-407): every category's bin */
            sweep(&c, hist + 2 * fs, fe - fs, total_g, total_h, dir, (uint32_t)f, out);
            continue;
        }
        if (fe <= fs + 1) continue;
        double ag = 0.0, ah = 0.0;
        for (size_t b = fs; b < fe; b++) {
            ag += hist[2 * b];
            ah += hist[2 * b + 1];
            offer(&c, (uint32_t)f, dir, (int64_t)b, 0, ag, ah, total_g - ag, total_h - ah);
        }
        if (ix->dense || (ag == total_g && ah == total_h)) continue;
        double sg = 0.0, sh = 0.0;
        for (size_t o = fe - fs; o-- > 0;) {
            sg += hist[2 * (fs + o)];
            sh += hist[2 * (fs + o) + 1];
            int64_t pos = o == 0 ? -1 : (int64_t)(fs + o - 1);
            offer(&c, (uint32_t)f, dir, pos, 1, total_g - sg, total_h - sh, sg, sh);
        }
    }
}

int or_split_valid(const or_split *s, const or_params *p) {
    reg r = reg_of(p);
    return s->loss_chg > 1e-6 && s->loss_chg >= p->gamma &&
           children_valid(s->left_h, s->right_h, r.min_child_weight);
}
