// Split-gain search: one wave per (node, feature), then one wave per node.
//
// Restates the hist split search (builder/split.rs:37-56 loss_chg,
// :391-419 for_each_numeric_split; builder/shared.rs:89-141 weights and
// gains; builder/mod.rs:313-342 need_replace) on fixed-point histograms:
// the prefix over a feature's bins is an exact 64-bit wave scan, each
// candidate's children are converted to f64 once, and the score is the
// reference's arithmetic operation for operation (f64 weights rounded to
// f32 then bounded, each child's gain rounded to f32, added in f32, minus
// the node's f32 root_gain). A feature keeps its first best candidate in
// the reference's order (forward bins ascending, then the backward pass
// from the last bin down); the node merge keeps the lowest feature among
// equal losses, and only a loss above the empty split's 0 wins.
//
// The backward pass (missing values to the left) runs for a feature whose
// bins do not sum to the node's statistics, on indexes with missing values.
#include "common.h"

namespace hbr {

__device__ __forceinline__ double threshold_l1(double g, double alpha) {
    if (g > alpha) return g - alpha;
    if (g < -alpha) return g + alpha;
    return 0.0;
}

__device__ __forceinline__ float bounded_weight(double g, double h, const ScanParams &r, float lower,
                                                float upper) {
    double w = 0.0;
    if (h > 0.0) {
        w = -threshold_l1(g, r.alpha) / (h + r.lambda);
        if (r.max_delta_step != 0.0 && __builtin_fabs(w) > r.max_delta_step)
            w = __builtin_copysign(r.max_delta_step, w);
    }
    float wf = (float)w;
    if (wf < lower) return lower;
    if (wf > upper) return upper;
    return wf;
}

__device__ __forceinline__ double gain_at(double g, double h, const ScanParams &r, float w) {
    const float w2 = w * w;
    return -(2.0 * g * (double)w + (h + r.lambda) * (double)w2 + 2.0 * r.alpha * (double)__builtin_fabsf(w));
}

// xgb_node_gain (builder/shared.rs:131-141): the node's own gain at its
// bounded weight, rounded to f32; 0 for a non-positive Hessian.
__device__ __forceinline__ float node_gain(double g, double h, const ScanParams &r, float lower, float upper) {
    if (h <= 0.0) return 0.0f;
    return (float)gain_at(g, h, r, bounded_weight(g, h, r, lower, upper));
}

// loss_chg of one candidate; false when the candidate is not offered.
__device__ __forceinline__ bool score(double lg, double lh, double rg, double rh, const ScanParams &r,
                                      float lower, float upper, int dir, float root_gain, float *loss) {
    if (!(lh > 0.0 && rh > 0.0 && lh >= r.min_child_weight && rh >= r.min_child_weight)) return false;
    const float wl = bounded_weight(lg, lh, r, lower, upper);
    const float wr = bounded_weight(rg, rh, r, lower, upper);
    if (dir > 0 && !((double)wl <= (double)wr)) return false;
    if (dir < 0 && !((double)wl >= (double)wr)) return false;
    const float gain = (float)gain_at(lg, lh, r, wl) + (float)gain_at(rg, rh, r, wr);
    *loss = gain - root_gain;
    return true;
}

struct Cand {
    float loss;
    uint32_t idx;
    int64_t lg, lh, rg, rh;
    uint32_t backward;
};

__device__ __forceinline__ bool better(float la, uint32_t ia, float lb, uint32_t ib) {
    return la > lb || (la == lb && ia < ib);
}

__device__ __forceinline__ void offer(Cand &best, bool &nan_seen, float loss, uint32_t idx, int64_t lg,
                                      int64_t lh, int64_t rg, int64_t rh, uint32_t backward) {
    if (__builtin_isnan(loss)) {
        nan_seen = true;
        return;
    }
    if (__builtin_isinf(loss)) return;
    if (better(loss, idx, best.loss, best.idx)) {
        best.loss = loss;
        best.idx = idx;
        best.lg = lg;
        best.lh = lh;
        best.rg = rg;
        best.rh = rh;
        best.backward = backward;
    }
}

// Nodes of the launch: both children of every split of a device-grown level.
__device__ __forceinline__ uint32_t scan_nodes(const ScanArgs &a) { return a.grow ? 2u * a.grow->n_splits : a.n_nodes; }

__device__ __forceinline__ uint32_t node_slot(const ScanArgs &a, const ScanNode &nd) {
    if (!nd.from_split) return nd.slot;
    const PartSplit sp = a.splits[nd.split];
    const uint32_t built_left = a.part_out[nd.split].built_left;
    const bool built = nd.child == 0 ? built_left != 0 : built_left == 0;
    return built ? sp.fresh_slot : sp.parent_slot;
}

}  // namespace hbr

using namespace hbr;

extern "C" __global__ __launch_bounds__(256) void hbr_scan_features(ScanArgs a) {
    const uint32_t wave = threadIdx.x / kWave, lane = lane_id();
    const uint32_t pair = blockIdx.x * (blockDim.x / kWave) + wave;
    if (pair >= scan_nodes(a) * a.n_features) return;  // uniform per wave
    const uint32_t node = pair / a.n_features, f = pair % a.n_features;
    const ScanNode nd = a.nodes[node];
    const uint32_t fs = a.feature_offset[f], nb = a.feature_offset[f + 1] - fs;
    Cand best;
    best.loss = -__builtin_inff();
    best.idx = 0xffffffffu;
    best.lg = best.lh = best.rg = best.rh = 0;
    best.backward = 0;
    bool nan_seen = false;
    const QBin *h = a.hist + (size_t)node_slot(a, nd) * a.total_bins + fs;
    const bool dev_root = (nd.pad & kScanDeviceRoot) != 0;
    const uint32_t cls = nd.pad >> kScanClassShift;
    QBin *root_total = a.root_total + cls;
    int64_t tg = nd.total.g, th = nd.total.h;
    if (dev_root && a.dense) {
        // the host routes a dense root here only when feature 0 has bins
        int64_t sg = 0, sh = 0;
        for (uint32_t b = lane; b < nb; b += kWave) {
            sg += h[b].g;
            sh += h[b].h;
        }
#pragma unroll
        for (int d = 32; d >= 1; d >>= 1) {
            sg += __shfl_xor(sg, d, kWave);
            sh += __shfl_xor(sh, d, kWave);
        }
        tg = sg;
        th = sh;
        if (f == 0 && lane == 0) *root_total = QBin{tg, th};
    } else if (dev_root) {
        tg = root_total->g;
        th = root_total->h;
    }
    if (nb > 1) {
        const int eg = a.scale[cls].exp_g, eh = a.scale[cls].exp_h;
        const int dir = a.monotone ? (int)a.monotone[f] : 0;
        const float root_gain = dev_root ? node_gain(dequant(tg, eg), dequant(th, eh), a.reg, nd.lower, nd.upper)
                                         : nd.root_gain;
        int64_t carry_g = 0, carry_h = 0;
        // forward pass: bins <= b left, missing right
        for (uint32_t c0 = 0; c0 < nb; c0 += kScanChunk) {
            const uint32_t b0 = c0 + 4 * lane;
            int64_t sg[4], sh[4];
            int64_t rg = 0, rh = 0;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                QBin v = (b0 + k < nb) ? h[b0 + k] : QBin{0, 0};
                rg += v.g;
                rh += v.h;
                sg[k] = rg;
                sh[k] = rh;
            }
            const int64_t ig = wave_inclusive_scan(rg), ih = wave_inclusive_scan(rh);
            const int64_t xg = carry_g + ig - rg, xh = carry_h + ih - rh;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                if (b0 + k >= nb) break;
                const int64_t ag = xg + sg[k], ah = xh + sh[k];
                float loss;
                if (score(dequant(ag, eg), dequant(ah, eh), dequant(tg - ag, eg), dequant(th - ah, eh),
                          a.reg, nd.lower, nd.upper, dir, root_gain, &loss))
                    offer(best, nan_seen, loss, b0 + k, ag, ah, tg - ag, th - ah, 0);
            }
            carry_g += wave_broadcast(ig, kWave - 1);
            carry_h += wave_broadcast(ih, kWave - 1);
        }
        // backward pass: bins >= b right, missing left; ends below every bin
        if (!a.dense && (carry_g != tg || carry_h != th)) {
            const int64_t fg = carry_g, fh = carry_h;
            carry_g = carry_h = 0;
            for (uint32_t c0 = 0; c0 < nb; c0 += kScanChunk) {
                const uint32_t b0 = c0 + 4 * lane;
                int64_t eg_[4], eh_[4];  // exclusive prefix of each bin
                int64_t rg = 0, rh = 0;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    QBin v = (b0 + k < nb) ? h[b0 + k] : QBin{0, 0};
                    eg_[k] = rg;
                    eh_[k] = rh;
                    rg += v.g;
                    rh += v.h;
                }
                const int64_t ig = wave_inclusive_scan(rg), ih = wave_inclusive_scan(rh);
                const int64_t xg = carry_g + ig - rg, xh = carry_h + ih - rh;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const uint32_t o = b0 + k;
                    if (o >= nb) break;
                    const int64_t sgv = fg - (xg + eg_[k]), shv = fh - (xh + eh_[k]);  // suffix from bin o
                    float loss;
                    if (score(dequant(tg - sgv, eg), dequant(th - shv, eh), dequant(sgv, eg), dequant(shv, eh),
                              a.reg, nd.lower, nd.upper, dir, root_gain, &loss))
                        offer(best, nan_seen, loss, nb + (nb - 1 - o), tg - sgv, th - shv, sgv, shv, 1);
                }
                carry_g += wave_broadcast(ig, kWave - 1);
                carry_h += wave_broadcast(ih, kWave - 1);
            }
        }
    }
    // wave arg-best: highest loss, then lowest candidate index
    float bl = best.loss;
    uint32_t bi = best.idx;
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        const float ol = __shfl_xor(bl, d, kWave);
        const uint32_t oi = (uint32_t)__shfl_xor((int)bi, d, kWave);
        if (better(ol, oi, bl, bi)) {
            bl = ol;
            bi = oi;
        }
    }
    const uint64_t any_nan = __ballot(nan_seen);
    const uint64_t mine = __ballot(best.idx == bi && best.loss == bl && bi != 0xffffffffu);
    ScanBest *out = a.per_feature + pair;
    if (mine == 0) {
        if (lane == 0) {
            ScanBest o;
            o.loss = -__builtin_inff();
            o.feature = f;
            o.index = 0xffffffffu;
            o.flags = any_nan ? 2u : 0u;
            o.left = QBin{0, 0};
            o.right = QBin{0, 0};
            *out = o;
        }
    } else if (lane == (uint32_t)(__ffsll((unsigned long long)mine) - 1)) {
        ScanBest o;
        o.loss = bl;
        o.feature = f;
        o.index = bi;
        o.flags = best.backward | (any_nan ? 2u : 0u);
        o.left = QBin{best.lg, best.lh};
        o.right = QBin{best.rg, best.rh};
        *out = o;
    }
}

// Per node: the feature-order merge. A candidate must beat the empty split
// (loss 0); equal losses keep the lower feature.
extern "C" __global__ __launch_bounds__(64) void hbr_scan_merge(ScanArgs a) {
    const uint32_t node = blockIdx.x;
    if (node >= scan_nodes(a)) return;
    const uint32_t lane = lane_id();
    float bl = 0.0f;
    uint32_t bf = 0xffffffffu;
    uint32_t nan_flag = 0;
    for (uint32_t f = lane; f < a.n_features; f += kWave) {
        const ScanBest c = a.per_feature[(size_t)node * a.n_features + f];
        nan_flag |= c.flags & 2u;
        if (c.index == 0xffffffffu) continue;
        // features ascend within a lane: only a strictly larger loss replaces
        if (c.loss > 0.0f && (bf == 0xffffffffu || c.loss > bl)) {
            bl = c.loss;
            bf = f;
        }
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        const float ol = __shfl_xor(bl, d, kWave);
        const uint32_t of = (uint32_t)__shfl_xor((int)bf, d, kWave);
        nan_flag |= (uint32_t)__shfl_xor((int)nan_flag, d, kWave);
        if (of != 0xffffffffu && (bf == 0xffffffffu || ol > bl || (ol == bl && of < bf))) {
            bl = ol;
            bf = of;
        }
    }
    if (lane == 0) {
        ScanBest o;
        if (bf == 0xffffffffu) {
            o.loss = 0.0f;
            o.feature = 0;
            o.index = 0xffffffffu;
            o.flags = nan_flag;
            o.left = QBin{0, 0};
            o.right = QBin{0, 0};
        } else {
            o = a.per_feature[(size_t)node * a.n_features + bf];
            o.flags |= nan_flag;
        }
        a.best[node] = o;
    }
}
