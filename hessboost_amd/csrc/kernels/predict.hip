// Batched ensemble prediction: one thread per row, trees in order.
//
// Restates the margin walk (model/predict.rs:60-193, compact/mod.rs:1052-1095):
// out = base_score, then for every tree in ascending order
// out[output(t)] += weight(t) * leaf(t, row) in f32 (a multiply, then an
// add); a present value goes left iff value < threshold, a missing one
// follows default_left (tree/mod.rs:52-58).
#include "common.h"

using namespace hbr;

namespace hbr {

__device__ __forceinline__ uint32_t walk(const PredictArgs &a, const float *row, uint32_t nid) {
    for (;;) {
        const uint32_t meta = a.node_meta[nid];
        if (meta >> 31) return nid;
        const float v = row[meta & 0xfffffu];
        const bool miss = a.missing_is_nan ? __builtin_isnan(v) : (v == a.missing);
        const bool left = miss ? ((meta >> 30) & 1u) != 0 : (v < __uint_as_float(a.node_value[nid]));
        nid = a.node_left[nid] + (left ? 0u : 1u);
    }
}

}  // namespace hbr

extern "C" __global__ __launch_bounds__(256) void hbr_predict(PredictArgs a) {
    const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= a.n) return;
    const float *row = a.x + (size_t)r * a.n_cols;
    float *out = a.out + (size_t)r * a.n_outputs;
    if (a.n_outputs == 1) {
        float acc = a.base_score[0];
        for (uint32_t t = 0; t < a.n_trees; t++) {
            const uint32_t leaf = walk(a, row, a.tree_root[t]);
            if (a.leaf_out) a.leaf_out[(size_t)r * a.n_trees + t] = a.node_orig[leaf];
            const float contrib = a.tree_weight[t] * __uint_as_float(a.node_value[leaf]);
            acc = acc + contrib;
        }
        out[0] = acc;
        return;
    }
    for (uint32_t c = 0; c < a.n_outputs; c++) out[c] = a.base_score[c];
    for (uint32_t t = 0; t < a.n_trees; t++) {
        const uint32_t leaf = walk(a, row, a.tree_root[t]);
        if (a.leaf_out) a.leaf_out[(size_t)r * a.n_trees + t] = a.node_orig[leaf];
        const float contrib = a.tree_weight[t] * __uint_as_float(a.node_value[leaf]);
        float *o = out + a.tree_output[t];
        *o = *o + contrib;
    }
}
