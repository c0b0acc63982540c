// Host side of the split arithmetic: leaf weights, node gains and monotone
// bounds, operation for operation as the reference computes them.
//
// tree/gain.rs:82-116 (RegParams rounded to f32, threshold_l1, calc_weight),
// builder/shared.rs:89-141 (xgb_calc_weight, apply_bounds, xgb_weight,
// xgb_gain_given_weight, xgb_node_gain), tree/constraints.rs (child_bounds
// at the f64 midpoint, calc_weight_bounded), builder/mod.rs:167-193
// (found, valid).
#pragma once
#include <cfloat>
#include <cmath>

namespace hbr {

struct Reg {
    double lambda, alpha, max_delta_step, min_child_weight;
};

inline Reg reg_from(double lambda, double alpha, double max_delta_step, double mcw) {
    return Reg{(double)(float)lambda, (double)(float)alpha, (double)(float)max_delta_step, (double)(float)mcw};
}

inline double threshold_l1(double g, double alpha) {
    if (g > alpha) return g - alpha;
    if (g < -alpha) return g + alpha;
    return 0.0;
}

inline double xgb_calc_weight(double g, double h, const Reg &r) {
    if (h <= 0.0) return 0.0;
    double w = -threshold_l1(g, r.alpha) / (h + r.lambda);
    if (r.max_delta_step != 0.0 && std::fabs(w) > r.max_delta_step) w = std::copysign(r.max_delta_step, w);
    return w;
}

inline float apply_bounds(float w, float lower, float upper) {
    if (w < lower) return lower;
    if (w > upper) return upper;
    return w;
}

inline float xgb_weight(double g, double h, const Reg &r, double lower, double upper) {
    return apply_bounds((float)xgb_calc_weight(g, h, r), (float)lower, (float)upper);
}

inline double xgb_gain_given_weight(double g, double h, const Reg &r, float w) {
    const float w2 = w * w;
    return -(2.0 * g * (double)w + (h + r.lambda) * (double)w2 + 2.0 * r.alpha * (double)std::fabs(w));
}

inline float xgb_node_gain(double g, double h, const Reg &r, double lower, double upper) {
    if (h <= 0.0) return 0.0f;
    return (float)xgb_gain_given_weight(g, h, r, xgb_weight(g, h, r, lower, upper));
}

// calc_weight (gain.rs:107-116) then Bounds::clamp: a leaf's final value.
inline double calc_weight_bounded(double g, double h, const Reg &r, double lower, double upper) {
    double w = 0.0;
    if (!(h < r.min_child_weight || h <= 0.0)) {
        w = -threshold_l1(g, r.alpha) / (h + r.lambda);
        if (r.max_delta_step > 0.0) w = w < -r.max_delta_step ? -r.max_delta_step : (w > r.max_delta_step ? r.max_delta_step : w);
    }
    if (w < lower) w = lower;
    if (w > upper) w = upper;
    return w;
}

inline bool children_valid(double lh, double rh, double mcw) {
    return lh > 0.0 && rh > 0.0 && lh >= mcw && rh >= mcw;
}

// f64::midpoint.
inline double midpoint(double a, double b) {
    const double hi = DBL_MAX / 2.0, lo = DBL_MIN * 2.0;
    if (std::fabs(a) <= hi && std::fabs(b) <= hi) return (a + b) / 2.0;
    if (std::fabs(a) < lo) return a + b / 2.0;
    if (std::fabs(b) < lo) return a / 2.0 + b;
    return a / 2.0 + b / 2.0;
}

// child_bounds: (left lower, left upper, right lower, right upper).
inline void child_bounds(double lo, double up, int dir, double wl, double wr, double out[4]) {
    out[0] = lo;
    out[1] = up;
    out[2] = lo;
    out[3] = up;
    if (dir == 0) return;
    const double mid = midpoint(wl, wr);
    if (dir > 0) {
        out[1] = mid;
        out[2] = mid;
    } else {
        out[0] = mid;
        out[3] = mid;
    }
}

}  // namespace hbr
