/*
 * Oracle (test infrastructure): gradients and intercepts.
 *
 * objective/regression.rs:42-58 (squared error: ((p - y) w, w), w scaled by
 * scale_pos_weight for a label of exactly 1), simd/x86_64.rs:22-160 (the
 * AVX2/FMA logistic kernel: 8-row vectors whose margins are all finite with
 * magnitude <= 80; split-ln2 range reduction, Estrin degree-7 polynomial),
 * simd/mod.rs:28-66 (vector rows = n - n % 8 once n >= 16), simd/scalar.rs:8-29
 * and simd/mod.rs:425-427 (the scalar tail: 1 / (expf(min(-x, 88.7)) + 1)),
 * simd/mod.rs:580-600 (softmax row: shift by max(f32::MIN_POSITIVE, preds),
 * f64 sum of expf, p = expf(x - wmax) / (f32)sum, h = max(2p(1-p)w, 1e-16)),
 * objective/mod.rs:645-666 (weighted label mean), classification.rs:66-77
 * (logit link; the identity for binary:logitraw), classification.rs:132-141
 * and regression.rs:66-74 with objective/mod.rs:528-566 (one Newton step
 * from zero margins when scale_pos_weight != 1), multiclass.rs:68-94 (centered log class
 * frequencies).
 *
 * The vector kernel is written with the same AVX2 intrinsics, in the same
 * order, so the oracle reproduces the reference's host bits on any x86-64
 * CPU with AVX2 and FMA.
 */
#include "oracle.h"

#include <float.h>
#include <immintrin.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#define MIN_HESS 1e-16f
#define MAX_FAST_EXP_INPUT 80.0f
#define WIDTH 8
#define MIN_SIMD_LEN 16

void or_gradient_squared_error(const float *preds, const float *labels, const float *weights,
                               size_t n, float spw, float *out) {
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; i++) {
        float w = weights ? weights[i] : 1.0f;
        float y = labels[i];
        if (y == 1.0f) w *= spw;
        out[2 * i] = (preds[i] - y) * w;
        out[2 * i + 1] = w;
    }
}

float or_sigmoid(float x) {
    float t = fminf(-x, 88.7f);
    return 1.0f / (expf(t) + 1.0f);
}

static void logistic_scalar(const float *preds, const float *labels, const float *weights,
                            float spw, float *out, size_t i) {
    float label = labels[i];
    float p = or_sigmoid(preds[i]);
    float w = weights ? weights[i] : 1.0f;
    if (label == 1.0f) w *= spw;
    out[2 * i] = (p - label) * w;
    out[2 * i + 1] = fmaxf(p * (1.0f - p), MIN_HESS) * w;
}

__attribute__((target("avx2,fma"))) static __m256 exp_f32(__m256 value) {
    __m256i exponent = _mm256_cvtps_epi32(_mm256_mul_ps(value, _mm256_set1_ps(1.44269504088896341f)));
    __m256 exponent_f32 = _mm256_cvtepi32_ps(exponent);
    __m256 reduced = _mm256_fnmadd_ps(exponent_f32, _mm256_set1_ps(0.6933594f), value);
    reduced = _mm256_fmadd_ps(exponent_f32, _mm256_set1_ps(2.1219444e-4f), reduced);
    __m256 squared = _mm256_mul_ps(reduced, reduced);
    __m256 fourth = _mm256_mul_ps(squared, squared);
    __m256 pair_0 = _mm256_add_ps(_mm256_set1_ps(1.0f), reduced);
    __m256 pair_1 = _mm256_fmadd_ps(_mm256_set1_ps(1.0f / 6.0f), reduced, _mm256_set1_ps(0.5f));
    __m256 pair_2 = _mm256_fmadd_ps(_mm256_set1_ps(1.0f / 120.0f), reduced, _mm256_set1_ps(1.0f / 24.0f));
    __m256 pair_3 = _mm256_fmadd_ps(_mm256_set1_ps(1.0f / 5040.0f), reduced, _mm256_set1_ps(1.0f / 720.0f));
    __m256 low = _mm256_fmadd_ps(pair_1, squared, pair_0);
    __m256 high = _mm256_fmadd_ps(pair_3, squared, pair_2);
    __m256 poly = _mm256_fmadd_ps(high, fourth, low);
    __m256i bits = _mm256_slli_epi32(_mm256_add_epi32(exponent, _mm256_set1_epi32(127)), 23);
    return _mm256_mul_ps(poly, _mm256_castsi256_ps(bits));
}

__attribute__((target("avx2,fma"))) static void logistic_vector(const float *preds,
                                                                 const float *labels,
                                                                 const float *weights, float spw,
                                                                 float *out, size_t i) {
    __m256 pred = _mm256_loadu_ps(preds + i);
    __m256 absv = _mm256_andnot_ps(_mm256_set1_ps(-0.0f), pred);
    __m256 in_range = _mm256_cmp_ps(absv, _mm256_set1_ps(MAX_FAST_EXP_INPUT), _CMP_LE_OQ);
    if (_mm256_movemask_ps(in_range) != 0xFF) {
        for (size_t j = i; j < i + WIDTH; j++) logistic_scalar(preds, labels, weights, spw, out, j);
        return;
    }
    __m256 one = _mm256_set1_ps(1.0f);
    __m256 label = _mm256_loadu_ps(labels + i);
    __m256 e = exp_f32(_mm256_sub_ps(_mm256_setzero_ps(), absv));
    __m256 den = _mm256_add_ps(one, e);
    __m256 positive = _mm256_div_ps(one, den);
    __m256 negative = _mm256_div_ps(e, den);
    __m256 nonneg = _mm256_cmp_ps(pred, _mm256_setzero_ps(), _CMP_GE_OQ);
    __m256 p = _mm256_blendv_ps(negative, positive, nonneg);
    __m256 weight = weights ? _mm256_loadu_ps(weights + i) : one;
    __m256 pos = _mm256_cmp_ps(label, one, _CMP_EQ_OQ);
    weight = _mm256_mul_ps(weight, _mm256_blendv_ps(one, _mm256_set1_ps(spw), pos));
    __m256 grad = _mm256_mul_ps(_mm256_sub_ps(p, label), weight);
    __m256 hess = _mm256_mul_ps(_mm256_max_ps(_mm256_mul_ps(p, _mm256_sub_ps(one, p)), _mm256_set1_ps(MIN_HESS)), weight);
    float g[8], h[8];
    _mm256_storeu_ps(g, grad);
    _mm256_storeu_ps(h, hess);
    for (int j = 0; j < WIDTH; j++) {
        out[2 * (i + j)] = g[j];
        out[2 * (i + j) + 1] = h[j];
    }
}

void or_gradient_logistic(const float *preds, const float *labels, const float *weights,
                          size_t n, float spw, float *out) {
    size_t vec_rows = n >= MIN_SIMD_LEN ? n - n % WIDTH : 0;
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < vec_rows; i += WIDTH) logistic_vector(preds, labels, weights, spw, out, i);
    for (size_t i = vec_rows; i < n; i++) logistic_scalar(preds, labels, weights, spw, out, i);
}

/* simd/mod.rs:502-528 with simd/x86_64.rs:160-335: with 2 or 4 classes and
 * at least 16 margins, the reference's x86-64 build takes an AVX2 path over
 * batches of 8 / K whole rows (one vector): the row maximum and minimum by
 * the in-lane permutes of row_reduce, shifted by max(f32::MIN_POSITIVE, row
 * max); when every row of the batch is finite and spans at most 80, the
 * vector exp of x - max, the row sum in f32 by the same permutes ((e0 + e1)
 * + (e2 + e3) for four classes) and p = e * (1 / sum); a batch with a row
 * outside that range, and the rows after the last whole batch, take the
 * scalar row (simd/mod.rs:580-600). The trainer accepts only class indices
 * as labels (multiclass.rs:96-100); other labels follow the reference's
 * casts. */
/* Rust's saturating `label as usize` (simd/mod.rs:549): NaN and values
 * below 1 give class 0; k stands for every index past the last class. */
static size_t label_class(float y, size_t k) {
    if (!(y >= 1.0f)) return 0;
    return y < (float)k ? (size_t)y : k;
}

static void softmax_row_scalar(const float *p, float label_f, float weight, size_t k, float *o) {
    float wmax = FLT_MIN;
    for (size_t c = 0; c < k; c++) wmax = fmaxf(p[c], wmax);
    double wsum = 0.0;
    for (size_t c = 0; c < k; c++) wsum += (double)expf(p[c] - wmax);
    float ws = (float)wsum;
    size_t label = label_class(label_f, k);
    for (size_t c = 0; c < k; c++) {
        float pc = expf(p[c] - wmax) / ws;
        float h = fmaxf(2.0f * pc * (1.0f - pc) * weight, MIN_HESS);
        float g = c == label ? pc - 1.0f : pc;
        o[2 * c] = g * weight;
        o[2 * c + 1] = h;
    }
}

#define ROW_REDUCE(name, op)                                                          \
    __attribute__((target("avx2,fma"))) static __m256 name(__m256 v, size_t k) {     \
        __m256 r = op(v, _mm256_permute_ps(v, 0xB1)); /* swap adjacent lanes */       \
        return k == 2 ? r : op(r, _mm256_permute_ps(r, 0x4E)); /* swap lane pairs */ \
    }
ROW_REDUCE(row_max, _mm256_max_ps)
ROW_REDUCE(row_min, _mm256_min_ps)
ROW_REDUCE(row_sum, _mm256_add_ps)

/* 0 when a row of the batch is out of the vector path's range */
__attribute__((target("avx2,fma"))) static int softmax_batch(const float *preds, const float *labels,
                                                            const float *weights, size_t k, size_t row,
                                                            float *out) {
    __m256 v = _mm256_loadu_ps(preds + row * k);
    __m256 maximum = _mm256_max_ps(_mm256_set1_ps(FLT_MIN), row_max(v, k));
    __m256 minimum = row_min(v, k);
    __m256 regular = _mm256_cmp_ps(_mm256_sub_ps(maximum, minimum), _mm256_set1_ps(MAX_FAST_EXP_INPUT), _CMP_LE_OQ);
    if (_mm256_movemask_ps(regular) != 0xFF) return 0;
    __m256 one = _mm256_set1_ps(1.0f);
    __m256 e = exp_f32(_mm256_sub_ps(v, maximum));
    __m256 p = _mm256_mul_ps(e, _mm256_div_ps(one, row_sum(e, k)));
    float ind[8], wt[8];
    for (size_t j = 0; j < WIDTH; j++) {
        ind[j] = label_class(labels[row + j / k], k) == j % k ? 1.0f : 0.0f;
        wt[j] = weights ? weights[row + j / k] : 1.0f;
    }
    __m256 weight = _mm256_loadu_ps(wt);
    __m256 grad = _mm256_mul_ps(_mm256_sub_ps(p, _mm256_loadu_ps(ind)), weight);
    __m256 hess = _mm256_max_ps(_mm256_mul_ps(_mm256_mul_ps(_mm256_mul_ps(p, _mm256_set1_ps(2.0f)),
                                                            _mm256_sub_ps(one, p)), weight),
                                _mm256_set1_ps(MIN_HESS));
    float g[8], h[8];
    _mm256_storeu_ps(g, grad);
    _mm256_storeu_ps(h, hess);
    float *o = out + 2 * row * k;
    for (size_t j = 0; j < WIDTH; j++) {
        o[2 * j] = g[j];
        o[2 * j + 1] = h[j];
    }
    return 1;
}

void or_gradient_softmax_scalar(const float *preds, const float *labels, const float *weights,
                                size_t n, size_t k, float *out) {
#pragma omp parallel for schedule(static)
    for (size_t r = 0; r < n; r++)
        softmax_row_scalar(preds + r * k, labels[r], weights ? weights[r] : 1.0f, k, out + 2 * r * k);
}

void or_gradient_softmax(const float *preds, const float *labels, const float *weights,
                         size_t n, size_t k, float *out) {
    size_t batched = 0;
    if ((k == 2 || k == 4) && n * k >= MIN_SIMD_LEN) {
        const size_t per = WIDTH / k;
        batched = n - n % per;
#pragma omp parallel for schedule(static)
        for (size_t r = 0; r < batched; r += per) {
            if (softmax_batch(preds, labels, weights, k, r, out)) continue;
            for (size_t q = r; q < r + per; q++)
                softmax_row_scalar(preds + q * k, labels[q], weights ? weights[q] : 1.0f, k, out + 2 * q * k);
        }
    }
#pragma omp parallel for schedule(static)
    for (size_t r = batched; r < n; r++)
        softmax_row_scalar(preds + r * k, labels[r], weights ? weights[r] : 1.0f, k, out + 2 * r * k);
}

static float weighted_label_mean(const float *labels, const float *weights, size_t n) {
    double mean = 0.0;
    if (weights) {
        double sum_w = 0.0;
        for (size_t i = 0; i < n; i++) sum_w += (double)weights[i];
        if (sum_w > 0.0)
            for (size_t i = 0; i < n; i++) mean += (double)labels[i] / sum_w * (double)weights[i];
    } else if (n > 0) {
        double dn = (double)n;
        for (size_t i = 0; i < n; i++) mean += (double)labels[i] / dn;
    }
    return (float)mean;
}

static float logit_link(float p) {
    const float eps = 1e-6f;
    if (p < eps) p = eps;
    if (p > 1.0f - eps) p = 1.0f - eps;
    return -logf(1.0f / p - 1.0f);
}

/* newton_intercepts (src/objective/mod.rs:528-547): the loss's own
   gradient at all-zero margins, then fit_stump (:552-566: f64 sums of g and
   h in row order, -G / max(H, 1e-6) rounded once to f32). The caller applies
   pred_transform and the link. */
static float newton_step(int objective, const float *labels, const float *weights, size_t n, float spw) {
    float *zeros = (float *)calloc(n ? n : 1, sizeof(float));
    float *gp = (float *)malloc(2 * (n ? n : 1) * sizeof(float));
    if (objective == OR_OBJ_SQUARED_ERROR)
        or_gradient_squared_error(zeros, labels, weights, n, spw, gp);
    else
        or_gradient_logistic(zeros, labels, weights, n, spw, gp);
    double g = 0.0, h = 0.0;
    for (size_t i = 0; i < n; i++) {
        g += (double)gp[2 * i];
        h += (double)gp[2 * i + 1];
    }
    free(zeros);
    free(gp);
    return (float)(-g / fmax(h, 1e-6));
}

void or_base_margins(const float *labels, const float *weights, size_t n, const or_params *p,
                     float *out) {
    if (p->objective == OR_OBJ_SOFTMAX) {
        size_t k = (size_t)p->num_class;
        if (p->has_base_score) {
            /* A user base_score broadcast through the identity-free softmax link
               is out of this path's scope; margins start at the score. */
            for (size_t c = 0; c < k; c++) out[c] = p->base_score;
            return;
        }
        for (size_t c = 0; c < k; c++) out[c] = 0.0f;
        for (size_t i = 0; i < n; i++) {
            size_t y = (size_t)labels[i];
            if (labels[i] >= 0.0f && y < k) out[y] += weights ? weights[i] : 1.0f;
        }
        double sum_w = 0.0;
        if (weights)
            for (size_t i = 0; i < n; i++) sum_w += (double)weights[i];
        else
            sum_w = (double)(float)n;
        double inv = 1.0 / sum_w;
        for (size_t c = 0; c < k; c++) out[c] = logf((float)((double)out[c] * inv) + 1e-6f);
        float kf = (float)k, mean = -0.0f;
        for (size_t c = 0; c < k; c++) mean += out[c] / kf;
        for (size_t c = 0; c < k; c++) out[c] -= mean;
        return;
    }
    if (p->objective == OR_OBJ_LOGISTIC || p->objective == OR_OBJ_LOGITRAW) {
        /* classification.rs:67-72: binary:logitraw's link is the identity */
        const int raw = p->objective == OR_OBJ_LOGITRAW;
        if (p->has_base_score)
            out[0] = raw ? p->base_score : logit_link(p->base_score);
        else if (fabsf(p->scale_pos_weight - 1.0f) > 1e-6f) /* classification.rs:132-141 */
        {
            const float w = newton_step(p->objective, labels, weights, n, p->scale_pos_weight);
            out[0] = raw ? w : logit_link(or_sigmoid(w)); /* sigmoid_scalar, then the logit */
        }
        else
            out[0] = raw ? weighted_label_mean(labels, weights, n)
                         : logit_link(weighted_label_mean(labels, weights, n));
        return;
    }
    /* regression.rs:66-74: the Newton step when scale_pos_weight != 1 */
    if (p->has_base_score)
        out[0] = p->base_score;
    else if (fabsf(p->scale_pos_weight - 1.0f) > 1e-6f)
        out[0] = newton_step(p->objective, labels, weights, n, p->scale_pos_weight);
    else
        out[0] = weighted_label_mean(labels, weights, n);
}
