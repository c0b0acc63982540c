/*
 * Oracle (test infrastructure): the boosting loop of a plain gbtree run.
 *
 * training/train.rs:406-436 (intercepts: the loss's estimate, or a given
 * base_score through its link), training/round.rs:214-400 (per iteration:
 * gradients of every output from the current margins, then one tree per
 * output from that output's gradient column, leaves scaled by tree_eta),
 * training/margins.rs:247-289 (each training row's margin += its leaf's
 * value, one f32 add per tree).
 */
#include "oracle.h"

#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

struct or_model {
    const or_index *ix;
    size_t n, k;
    float base[64];
    float *margins; /* n * k */
    float *gpair;   /* n * k pairs, [row][output] */
    float *gk;      /* n pairs, one output's column */
    int32_t *leaf;
    or_tree **trees;
    size_t n_trees, cap;
};

void or_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

static void gradients(or_model *m, const float *labels, const float *weights, const or_params *p) {
    if (p->objective == OR_OBJ_SQUARED_ERROR)
        or_gradient_squared_error(m->margins, labels, weights, m->n, p->scale_pos_weight, m->gpair);
    else if (p->objective == OR_OBJ_LOGISTIC || p->objective == OR_OBJ_LOGITRAW)
        or_gradient_logistic(m->margins, labels, weights, m->n, p->scale_pos_weight, m->gpair);
    else
        or_gradient_softmax(m->margins, labels, weights, m->n, m->k, m->gpair);
}

void or_train_more(or_model *m, const float *labels, const float *weights, const or_params *p,
                   size_t rounds) {
    for (size_t it = 0; it < rounds; it++) {
        gradients(m, labels, weights, p);
        for (size_t c = 0; c < m->k; c++) {
            const float *g = m->gpair;
            if (m->k > 1) {
                for (size_t r = 0; r < m->n; r++) {
                    m->gk[2 * r] = m->gpair[2 * (r * m->k + c)];
                    m->gk[2 * r + 1] = m->gpair[2 * (r * m->k + c) + 1];
                }
                g = m->gk;
            }
            or_tree *t = or_grow_tree(m->ix, g, p, m->leaf);
            for (size_t r = 0; r < m->n; r++) m->margins[r * m->k + c] += t->nodes[m->leaf[r]].leaf_value;
            if (m->n_trees == m->cap) {
                m->cap = m->cap ? 2 * m->cap : 64;
                m->trees = (or_tree **)realloc(m->trees, m->cap * sizeof(or_tree *));
            }
            m->trees[m->n_trees++] = t;
        }
    }
}

or_model *or_train(const or_index *ix, const float *labels, const float *weights,
                   const or_params *p, size_t rounds) {
    or_model *m = (or_model *)calloc(1, sizeof(or_model));
    m->ix = ix;
    m->n = ix->n_rows;
    m->k = p->objective == OR_OBJ_SOFTMAX ? (size_t)p->num_class : 1;
    or_base_margins(labels, weights, m->n, p, m->base);
    m->margins = (float *)malloc((m->n * m->k ? m->n * m->k : 1) * sizeof(float));
    for (size_t r = 0; r < m->n; r++)
        for (size_t c = 0; c < m->k; c++) m->margins[r * m->k + c] = m->base[c];
    m->gpair = (float *)malloc((2 * m->n * m->k ? 2 * m->n * m->k : 1) * sizeof(float));
    m->gk = (float *)malloc((2 * m->n ? 2 * m->n : 1) * sizeof(float));
    m->leaf = (int32_t *)malloc((m->n ? m->n : 1) * sizeof(int32_t));
    or_train_more(m, labels, weights, p, rounds);
    return m;
}

size_t or_model_n_trees(const or_model *m) { return m->n_trees; }
const or_tree *or_model_tree(const or_model *m, size_t i) { return m->trees[i]; }
const float *or_model_margins(const or_model *m) { return m->margins; }
const float *or_model_base_score(const or_model *m) { return m->base; }
size_t or_model_n_outputs(const or_model *m) { return m->k; }
const float *or_model_last_gpair(const or_model *m) { return m->gpair; }

void or_model_free(or_model *m) {
    if (!m) return;
    for (size_t i = 0; i < m->n_trees; i++) or_tree_free(m->trees[i]);
    free(m->trees);
    free(m->margins);
    free(m->gpair);
    free(m->gk);
    free(m->leaf);
    free(m);
}
