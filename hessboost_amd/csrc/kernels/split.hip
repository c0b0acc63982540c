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

// ---- the near-tie guard -------------------------------------------------------
// A candidate's children are fixed-point sums; the reference scores the same
// candidate from f64 chain sums of the same rows. Their difference per child
// is bounded by the quantisation of each row (half a unit) plus the chain's
// rounding (Higham: k u / (1 - k u) times the sum of |x| for k additions; a
// child's sum is its bins' chains added bin by bin, k <= m + 512; the sum
// of |x| is at most m max|x|), twice over for the right child (total minus
// left). Candidates with equal fixed-point sums are one partition: they can
// differ only by rows whose pairs quantise to zero (below half a unit,
// 2^-62 / n of the largest pair), which moves a score by less than one f32
// rounding in all but a vanishing share of cases. From those
// bounds the error of each child's gain follows through the weight (itself
// rounded to f32, clamped by max_delta_step and the monotone bounds, both
// 1-Lipschitz) and the gain; each f32 rounding of the score adds one spacing.
struct Bound {
    double dg, dh;  // sums of one node's rows
};

// An upper bound on one f32 rounding step at |x|.
__device__ __forceinline__ double ulp32(double x) { return __builtin_fabs(x) * 0x1p-23 + 0x1p-149; }

__device__ __forceinline__ Bound node_bound(uint32_t m, int eg, int eh, float max_g, float max_h) {
    const double md = (double)m;
    // a child's sum is its bins' chains added bin by bin: at most m + 512 additions
    const double chain = (md + 512.0) * 0x1p-53;
    const double gamma_m = chain < 0.5 ? chain / (1.0 - chain) : 1e300;
    return Bound{md * __builtin_ldexp(1.0, eg - 1) + gamma_m * md * (double)max_g,
                 md * __builtin_ldexp(1.0, eh - 1) + gamma_m * md * (double)max_h};
}

// Error bound of one child's gain at weight w (before the gain's f32 rounding),
// and the weight's own error through *dw. Evaluated in f32 with the
// hardware reciprocal: each step's relative error (<= 2^-22) is covered by
// the 2^-12 the caller adds to the total.
__device__ __forceinline__ float gain_err(double g, double h, float w, float dg, float dh, const ScanParams &r,
                                          float *dw_out) {
    const float hl = (float)(h + r.lambda);
    const float den = hl - dh;
    const float aw = __builtin_fabsf(w);
    const float dw = (den > 0.0f ? (dg + aw * dh) * __builtin_amdgcn_rcpf(den) : __builtin_inff()) +
                     2.0f * (float)ulp32(aw);
    const float slope = 2.0f * __builtin_fabsf((float)(g + (h + r.lambda) * (double)w)) + 2.0f * (float)r.alpha;
    *dw_out = dw;
    return 2.0f * aw * dg + aw * aw * dh + (slope + hl * dw) * dw;
}

// The guarded score of one candidate: `ok` as score() decides it; `rival`
// when the reference might offer it (ok, or within the error of the
// min_child_weight and monotone tests); `fragile` when ok but within that
// error of failing them; the score and its error bound.
struct Scored {
    bool ok, rival, fragile;
    float loss;
    float err;
};

__device__ __forceinline__ Scored score_guarded(double lg, double lh, double rg, double rh, const ScanParams &r,
                                                float lower, float upper, int dir, float root_gain, const Bound &b) {
    Scored o{false, false, false, 0.0f, 0.0f};
    if (!(lh > 0.0 && rh > 0.0)) return o;
    const float dgl = (float)b.dg, dhl = (float)b.dh;
    const float dgr = 2.0f * dgl + (float)(__builtin_fabs(rg) * 0x1p-52), dhr = 2.0f * dhl + (float)(rh * 0x1p-52);
    const bool mcw_ok = lh >= r.min_child_weight && rh >= r.min_child_weight;
    const bool mcw_near = lh + dhl >= r.min_child_weight && rh + dhr >= r.min_child_weight;
    const bool mcw_edge = lh - dhl < r.min_child_weight || rh - dhr < r.min_child_weight;
    if (!mcw_near) return o;
    const float wl = bounded_weight(lg, lh, r, lower, upper);
    const float wr = bounded_weight(rg, rh, r, lower, upper);
    float dwl, dwr;
    const float el = gain_err(lg, lh, wl, dgl, dhl, r, &dwl);
    const float er = gain_err(rg, rh, wr, dgr, dhr, r, &dwr);
    const float slack = dwl + dwr;
    bool mono_ok = true, mono_near = true, mono_edge = false;
    if (dir > 0) {
        mono_ok = wl <= wr;
        mono_near = wl <= wr + slack;
        mono_edge = wr - wl <= slack;
    } else if (dir < 0) {
        mono_ok = wl >= wr;
        mono_near = wl + slack >= wr;
        mono_edge = wl - wr <= slack;
    }
    if (!mono_near) return o;
    const float gl = (float)gain_at(lg, lh, r, wl), gr = (float)gain_at(rg, rh, r, wr);
    const float gain = gl + gr;
    o.loss = gain - root_gain;
    o.ok = mcw_ok && mono_ok;
    o.rival = true;
    o.fragile = o.ok && (mcw_edge || (dir != 0 && mono_edge));
    const float e = el + er + 1.2e-7f * (__builtin_fabsf(gl) + __builtin_fabsf(gr) + __builtin_fabsf(gain) +
                                         __builtin_fabsf(o.loss)) + 0x1p-126f;
    o.err = e * (1.0f + 0x1p-12f);
    return o;
}

// The two highest (score + error) of a lane's rival candidates whose left
// sums differ: `top` with its sums, `second` the best of any other sums.
struct Rivals {
    float top, second;
    int64_t tg, th;
    __device__ __forceinline__ void init() {
        top = second = -__builtin_inff();
        tg = th = INT64_MIN;
    }
    __device__ __forceinline__ void offer(float v, int64_t g, int64_t h) {
        if (!(v > -__builtin_inff()) || __builtin_isnan(v)) return;
        if (g == tg && h == th) {
            if (v > top) top = v;
        } else if (v > top) {
            second = top;
            top = v;
            tg = g;
            th = h;
        } else if (v > second) {
            second = v;
        }
    }
    // the best of the candidates whose sums differ from (g, h)
    __device__ __forceinline__ float excluding(int64_t g, int64_t h) const {
        return (g == tg && h == th) ? second : top;
    }
};

struct Cand {
    float loss;
    uint32_t idx;
    int64_t lg, lh, rg, rh;
    uint32_t backward;
    float err;
    uint32_t fragile;
};

__device__ __forceinline__ bool better(float la, uint32_t ia, float lb, uint32_t ib) {
    return la > lb || (la == lb && ia < ib);
}

__device__ __forceinline__ void offer(Cand &best, bool &nan_seen, float loss, uint32_t idx, int64_t lg,
                                      int64_t lh, int64_t rg, int64_t rh, uint32_t backward, float err = 0.0f,
                                      uint32_t fragile = 0u) {
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
        best.err = err;
        best.fragile = fragile;
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

// One wave: feature f of node `node`, its best candidate written to *out
// by one lane. BPL bins per lane and pass: 4 (chunks of 256 bins), or 1 for
// a feature of at most 64 bins, whose lanes would otherwise idle; the
// candidates, and the (highest loss, lowest index) winner, are the same.
// A node's row count: its record's, or the partition's for a child of a split.
__device__ __forceinline__ uint32_t node_rows(const ScanArgs &a, const ScanNode &nd) {
    if (!nd.from_split) return nd.rows;
    const uint32_t left = a.part_out[nd.split].left_len;
    return nd.child == 0 ? left : a.splits[nd.split].seg.len - left;
}

// x rounded up to f32.
__device__ __forceinline__ float up32(double x) {
    float f = (float)x;
    if ((double)f < x) {  // the next f32 above
        uint32_t b = __float_as_uint(f);
        b = f == 0.0f ? 1u : (f > 0.0f ? b + 1u : b - 1u);
        f = __uint_as_float(b);
    }
    return f;
}

template <uint32_t BPL, bool GUARD>
__device__ __forceinline__ void scan_feature(const ScanArgs &a, uint32_t node, uint32_t f, ScanBest *out) {
    const uint32_t lane = lane_id();
    const ScanNode nd = a.nodes[node];
    const uint32_t fs = a.feature_offset[f], nb = a.feature_offset[f + 1] - fs;
    Cand best;
    best.loss = -__builtin_inff();
    best.idx = 0xffffffffu;
    best.lg = best.lh = best.rg = best.rh = 0;
    best.backward = 0;
    best.err = 0.0f;
    best.fragile = 0;
    bool nan_seen = false;
    Rivals riv;
    riv.init();
    Bound bound{0.0, 0.0};
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
    // a categorical feature's record comes from hbr_scan_categorical
    const bool categorical = a.cat_rank && a.cat_rank[f] != 0xffffffffu;
    if (nb > 1 && !categorical) {
        const int eg = a.scale[cls].exp_g, eh = a.scale[cls].exp_h;
        const int dir = a.monotone ? (int)a.monotone[f] : 0;
        const float root_gain = dev_root ? node_gain(dequant(tg, eg), dequant(th, eh), a.reg, nd.lower, nd.upper)
                                         : nd.root_gain;
        if (GUARD)
            bound = node_bound(node_rows(a, nd), eg, eh, __uint_as_float(a.scale[cls].max_g_bits),
                               __uint_as_float(a.scale[cls].max_h_bits));
        int64_t carry_g = 0, carry_h = 0;
        // forward pass: bins <= b left, missing right
        for (uint32_t c0 = 0; c0 < nb; c0 += kWave * BPL) {
            const uint32_t b0 = c0 + BPL * lane;
            int64_t sg[BPL], sh[BPL];
            int64_t rg = 0, rh = 0;
#pragma unroll
            for (int k = 0; k < (int)BPL; k++) {
                QBin v = (b0 + k < nb) ? h[b0 + k] : QBin{0, 0};
                rg += v.g;
                rh += v.h;
                sg[k] = rg;
                sh[k] = rh;
            }
            const int64_t ig = wave_inclusive_scan(rg), ih = wave_inclusive_scan(rh);
            const int64_t xg = carry_g + ig - rg, xh = carry_h + ih - rh;
#pragma unroll
            for (int k = 0; k < (int)BPL; k++) {
                if (b0 + k >= nb) break;
                const int64_t ag = xg + sg[k], ah = xh + sh[k];
                float loss;
                if (GUARD) {
                    const Scored sc = score_guarded(dequant(ag, eg), dequant(ah, eh), dequant(tg - ag, eg),
                                                    dequant(th - ah, eh), a.reg, nd.lower, nd.upper, dir, root_gain,
                                                    bound);
                    if (sc.ok) offer(best, nan_seen, sc.loss, b0 + k, ag, ah, tg - ag, th - ah, 0, sc.err, sc.fragile);
                    if (sc.rival) riv.offer(up32((double)sc.loss + (double)sc.err), ag, ah);
                } else if (score(dequant(ag, eg), dequant(ah, eh), dequant(tg - ag, eg), dequant(th - ah, eh), a.reg,
                                 nd.lower, nd.upper, dir, root_gain, &loss)) {
                    offer(best, nan_seen, loss, b0 + k, ag, ah, tg - ag, th - ah, 0);
                }
            }
            carry_g += wave_broadcast(ig, kWave - 1);
            carry_h += wave_broadcast(ih, kWave - 1);
        }
        // backward pass: bins >= b right, missing left; ends below every bin
        if (!a.dense && (carry_g != tg || carry_h != th)) {
            const int64_t fg = carry_g, fh = carry_h;
            carry_g = carry_h = 0;
            for (uint32_t c0 = 0; c0 < nb; c0 += kWave * BPL) {
                const uint32_t b0 = c0 + BPL * lane;
                int64_t eg_[BPL], eh_[BPL];  // exclusive prefix of each bin
                int64_t rg = 0, rh = 0;
#pragma unroll
                for (int k = 0; k < (int)BPL; k++) {
                    QBin v = (b0 + k < nb) ? h[b0 + k] : QBin{0, 0};
                    eg_[k] = rg;
                    eh_[k] = rh;
                    rg += v.g;
                    rh += v.h;
                }
                const int64_t ig = wave_inclusive_scan(rg), ih = wave_inclusive_scan(rh);
                const int64_t xg = carry_g + ig - rg, xh = carry_h + ih - rh;
#pragma unroll
                for (int k = 0; k < (int)BPL; k++) {
                    const uint32_t o = b0 + k;
                    if (o >= nb) break;
                    const int64_t sgv = fg - (xg + eg_[k]), shv = fh - (xh + eh_[k]);  // suffix from bin o
                    float loss;
                    if (GUARD) {
                        const Scored sc = score_guarded(dequant(tg - sgv, eg), dequant(th - shv, eh), dequant(sgv, eg),
                                                        dequant(shv, eh), a.reg, nd.lower, nd.upper, dir, root_gain,
                                                        bound);
                        if (sc.ok)
                            offer(best, nan_seen, sc.loss, nb + (nb - 1 - o), tg - sgv, th - shv, sgv, shv, 1, sc.err,
                                  sc.fragile);
                        if (sc.rival) riv.offer(up32((double)sc.loss + (double)sc.err), tg - sgv, th - shv);
                    } else if (score(dequant(tg - sgv, eg), dequant(th - shv, eh), dequant(sgv, eg),
                                     dequant(shv, eh), a.reg, nd.lower, nd.upper, dir, root_gain, &loss)) {
                        offer(best, nan_seen, loss, nb + (nb - 1 - o), tg - sgv, th - shv, sgv, shv, 1);
                    }
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
    // the feature's rivals: every other partition of the node's rows it offers
    float rival = -__builtin_inff();
    if (GUARD) {
        const int owner = mine ? __ffsll((unsigned long long)mine) - 1 : 0;
        const int64_t wg = __shfl(best.lg, owner, kWave), wh = __shfl(best.lh, owner, kWave);
        rival = mine ? riv.excluding(wg, wh) : riv.top;
#pragma unroll
        for (int d = 32; d >= 1; d >>= 1) rival = fmaxf(rival, __shfl_xor(rival, d, kWave));
    }
    if (mine == 0) {
        if (lane == 0) {
            ScanBest o;
            o.loss = -__builtin_inff();
            o.feature = f;
            o.index = 0xffffffffu;
            o.flags = any_nan ? kScanNumericNaN : 0u;
            o.left = QBin{0, 0};
            o.right = QBin{0, 0};
            o.err = 0.0f;
            o.rival = rival;
            *out = o;
        }
    } else if (lane == (uint32_t)(__ffsll((unsigned long long)mine) - 1)) {
        ScanBest o;
        o.loss = bl;
        o.feature = f;
        o.index = bi;
        o.flags = best.backward | (any_nan ? kScanNumericNaN : 0u) | (best.fragile ? kScanNearTie : 0u);
        o.left = QBin{best.lg, best.lh};
        o.right = QBin{best.rg, best.rh};
        o.err = best.err;
        o.rival = rival;
        *out = o;
    }
}

extern "C" __global__ __launch_bounds__(256) void hbr_scan_features(ScanArgs a) {
    const uint32_t wave = threadIdx.x / kWave;
    const uint32_t pair = blockIdx.x * (blockDim.x / kWave) + wave;
    if (pair >= scan_nodes(a) * a.n_features) return;  // uniform per wave
    const uint32_t f = pair % a.n_features;
    const bool narrow = a.feature_offset[f + 1] - a.feature_offset[f] <= kWave;  // uniform per wave
    if (a.guard) {
        if (narrow)
            scan_feature<1, true>(a, pair / a.n_features, f, a.per_feature + pair);
        else
            scan_feature<4, true>(a, pair / a.n_features, f, a.per_feature + pair);
    } else if (narrow) {
        scan_feature<1, false>(a, pair / a.n_features, f, a.per_feature + pair);
    } else {
        scan_feature<4, false>(a, pair / a.n_features, f, a.per_feature + pair);
    }
}

// The feature-order merge of a node's per-feature winners (`per_node`,
// n_features records), by one workgroup of kMergeThreads: thread t takes
// features t, t + kMergeThreads, ... (ascending, so within a thread only a
// strictly larger loss replaces), then the threads' bests are reduced, higher
// loss first, the lower feature on equal losses. A candidate must beat the
// empty split (loss 0). Wide indexes (thousands of features) need the
// threads; a node of 28 features leaves most of them idle.
constexpr uint32_t kMergeThreads = 256;

__device__ __forceinline__ bool merge_better(float ol, uint32_t of, float bl, uint32_t bf) {
    return of != 0xffffffffu && (bf == 0xffffffffu || ol > bl || (ol == bl && of < bf));
}

__device__ __forceinline__ void merge_node(const ScanArgs &a, uint32_t node, const ScanBest *per_node) {
    __shared__ float s_loss[kMergeThreads / kWave], s_rival[kMergeThreads / kWave];
    __shared__ uint32_t s_feat[kMergeThreads / kWave], s_nan[kMergeThreads / kWave];
    const uint32_t lane = lane_id(), wave = threadIdx.x / kWave;
    float bl = 0.0f;
    uint32_t bf = 0xffffffffu;
    uint32_t nan_flag = 0;
    for (uint32_t f = threadIdx.x; f < a.n_features; f += kMergeThreads) {
        const ScanBest c = per_node[f];
        nan_flag |= c.flags & kScanReplay;
        if (c.index == 0xffffffffu) continue;
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
        if (merge_better(ol, of, bl, bf)) {
            bl = ol;
            bf = of;
        }
    }
    if (lane == 0) {
        s_loss[wave] = bl;
        s_feat[wave] = bf;
        s_nan[wave] = nan_flag;
    }
    __syncthreads();
    // every wave reduces the waves' bests (the same four records), so all
    // threads know the winner for the guard's pass over the rivals
    bl = lane < kMergeThreads / kWave ? s_loss[lane] : 0.0f;
    bf = lane < kMergeThreads / kWave ? s_feat[lane] : 0xffffffffu;
    nan_flag = lane < kMergeThreads / kWave ? s_nan[lane] : 0u;
#pragma unroll
    for (int d = 2; d >= 1; d >>= 1) {  // kMergeThreads / kWave = 4 candidates
        const float ol = __shfl_xor(bl, d, kWave);
        const uint32_t of = (uint32_t)__shfl_xor((int)bf, d, kWave);
        nan_flag |= (uint32_t)__shfl_xor((int)nan_flag, d, kWave);
        if (merge_better(ol, of, bl, bf)) {
            bl = ol;
            bf = of;
        }
    }
    bf = (uint32_t)__shfl((int)bf, 0, kWave);
    nan_flag = (uint32_t)__shfl((int)nan_flag, 0, kWave);
    float rival = -__builtin_inff();
    if (a.guard) {
        // the best score + error bound of any other partition of the node's rows
        const bool has = bf != 0xffffffffu;
        const int64_t wg = has ? per_node[bf].left.g : 0, wh = has ? per_node[bf].left.h : 0;
        for (uint32_t f = threadIdx.x; f < a.n_features; f += kMergeThreads) {
            const ScanBest c = per_node[f];
            float v = c.rival;
            const bool same = has && c.index != 0xffffffffu && c.left.g == wg && c.left.h == wh;
            if (c.index != 0xffffffffu && !same && f != bf) v = fmaxf(v, up32((double)c.loss + (double)c.err));
            rival = fmaxf(rival, v);
        }
#pragma unroll
        for (int d = 32; d >= 1; d >>= 1) rival = fmaxf(rival, __shfl_xor(rival, d, kWave));
        __syncthreads();  // the first reduction's records are read
        if (lane == 0) s_rival[wave] = rival;
        __syncthreads();
        rival = -__builtin_inff();
#pragma unroll
        for (uint32_t w = 0; w < kMergeThreads / kWave; w++) rival = fmaxf(rival, s_rival[w]);
    }
    if (wave != 0) return;
    if (lane == 0) {
        ScanBest o;
        if (bf == 0xffffffffu) {
            o.loss = 0.0f;
            o.feature = 0;
            o.index = 0xffffffffu;
            o.flags = nan_flag;
            o.left = QBin{0, 0};
            o.right = QBin{0, 0};
            o.err = 0.0f;
        } else {
            o = per_node[bf];
            o.flags |= nan_flag;
        }
        o.rival = rival;
        if (a.guard) {
            // certified when no rival can reach the winner's lower bound and
            // the winner (or, with none, the best rival) stays on one side of
            // the validity threshold (loss > kRtEps and loss >= gamma), the
            // node's own gain included (the root gain is its rounded gain)
            const ScanNode nd = a.nodes[node];
            const uint32_t cls = nd.pad >> kScanClassShift;
            const int eg = a.scale[cls].exp_g, eh = a.scale[cls].exp_h;
            const Bound b = node_bound(node_rows(a, nd), eg, eh, __uint_as_float(a.scale[cls].max_g_bits),
                                       __uint_as_float(a.scale[cls].max_h_bits));
            const bool dev_root = (nd.pad & kScanDeviceRoot) != 0;
            const QBin t = dev_root ? a.root_total[cls] : nd.total;
            const double tg = dequant(t.g, eg), th = dequant(t.h, eh);
            const float w = bounded_weight(tg, th, a.reg, nd.lower, nd.upper);
            float dw;
            const double e_root = th > 0.0 ? (double)gain_err(tg, th, w, (float)b.dg, (float)b.dh, a.reg, &dw) *
                                                     (1.0 + 0x1p-12) +
                                                 2.0 * ulp32(gain_at(tg, th, a.reg, w))
                                           : 0.0;
            const double thr = fmax(1e-6, (double)a.gamma);
            bool near;
            if (bf == 0xffffffffu) {
                near = (double)rival + e_root >= thr;
            } else {
                const double lo = (double)o.loss - (double)o.err - e_root, hi = (double)o.loss + (double)o.err + e_root;
                const bool splits = hi >= thr;
                near = (splits && (double)rival >= (double)o.loss - (double)o.err) || (lo <= thr && hi >= thr) ||
                       (splits && (o.flags & kScanNearTie));
            }
            o.flags = (o.flags & ~kScanNearTie) | (near ? kScanNearTie : 0u);
        }
        a.best[node] = o;
    }
    // a categorical winner's set, for the host's decision and partition
    const uint32_t win = bf;
    if (a.best_sets && a.cat_rank && win != 0xffffffffu && a.cat_rank[win] != 0xffffffffu) {
        const uint32_t *src = a.cat_sets + ((size_t)node * a.n_cat + a.cat_rank[win]) * kCatWords;
        for (uint32_t w = lane; w < kCatWords; w += kWave) a.best_sets[(size_t)node * kCatWords + w] = src[w];
    }
}

extern "C" __global__ __launch_bounds__(kMergeThreads) void hbr_scan_merge(ScanArgs a) {
    const uint32_t node = blockIdx.x;
    if (node >= scan_nodes(a)) return;  // uniform per workgroup
    merge_node(a, node, a.per_feature + (size_t)node * a.n_features);
}

// ---- near ties resolved on the CPU builder's sums -------------------------------
// One workgroup per node: thread f walks feature f's bins in order with f64
// prefix sums, as the reference's host search (builder/split.rs:391-470,
// hist/search.rs:99-127); thread 0 then merges the features in order.
extern "C" __global__ __launch_bounds__(256) void hbr_scan_exact(ExactScanArgs a) {
    const uint32_t f = threadIdx.x;
    const double tg = a.total_g, th = a.total_h;
    const float root_gain = node_gain(tg, th, a.reg, a.lower, a.upper);
    for (uint32_t ff = f; ff < a.n_cols; ff += blockDim.x) {
        const uint32_t fs = a.feature_offset[ff], nb = a.feature_offset[ff + 1] - fs;
        const int dir = a.monotone ? (int)a.monotone[ff] : 0;
        ExactBest b{};
        b.loss = -__builtin_inff();
        b.feature = ff;
        b.index = 0xffffffffu;
        bool nan_seen = false;
        auto offer_exact = [&](uint32_t idx, double lg, double lh, double rg, double rh, uint32_t backward) {
            float loss;
            if (!score(lg, lh, rg, rh, a.reg, a.lower, a.upper, dir, root_gain, &loss)) return;
            if (__builtin_isnan(loss)) {
                nan_seen = true;
                return;
            }
            if (__builtin_isinf(loss) || !(loss > b.loss)) return;  // the first best of the feature
            b.loss = loss;
            b.index = idx;
            b.flags = backward;
            b.lg = lg;
            b.lh = lh;
            b.rg = rg;
            b.rh = rh;
        };
        if (nb > 1) {
            double ag = 0.0, ah = 0.0;
            for (uint32_t k = 0; k < nb; k++) {
                ag += a.hist[2 * (fs + k)];
                ah += a.hist[2 * (fs + k) + 1];
                offer_exact(k, ag, ah, tg - ag, th - ah, 0u);
            }
            if (!a.dense && !(ag == tg && ah == th)) {
                double sg = 0.0, sh = 0.0;
                for (uint32_t o = nb; o-- > 0;) {
                    sg += a.hist[2 * (fs + o)];
                    sh += a.hist[2 * (fs + o) + 1];
                    offer_exact(nb + (nb - 1 - o), tg - sg, th - sh, sg, sh, 1u);
                }
            }
        }
        if (nan_seen) b.flags |= kScanNumericNaN;
        a.per_feature[ff] = b;
    }
    __syncthreads();
    if (threadIdx.x != 0) return;
    ExactBest w{};
    w.loss = 0.0f;
    w.index = 0xffffffffu;
    uint32_t nan_flag = 0;
    for (uint32_t ff = 0; ff < a.n_cols; ff++) {
        const ExactBest c = a.per_feature[ff];
        nan_flag |= c.flags & kScanNumericNaN;
        if (c.index != 0xffffffffu && c.loss > w.loss) w = c;  // only a higher loss displaces a lower feature
    }
    if (w.index != 0xffffffffu) {
        // the winner's partition in fixed point (the sums the next scans take)
        const uint32_t fs = a.feature_offset[w.feature], nb = a.feature_offset[w.feature + 1] - fs;
        const QBin *h = a.fixed + fs;
        int64_t sg = 0, sh = 0;
        if (w.index < nb) {
            for (uint32_t k = 0; k <= w.index; k++) {
                sg += h[k].g;
                sh += h[k].h;
            }
            w.left = QBin{sg, sh};
            w.right = QBin{a.total_fixed.g - sg, a.total_fixed.h - sh};
        } else {
            const uint32_t o = nb - 1 - (w.index - nb);
            for (uint32_t k = o; k < nb; k++) {
                sg += h[k].g;
                sh += h[k].h;
            }
            w.right = QBin{sg, sh};
            w.left = QBin{a.total_fixed.g - sg, a.total_fixed.h - sh};
        }
    }
    w.flags |= nan_flag;
    *a.best = w;
}

// ---- categorical features (builder/categorical.rs:48-170) ---------------------

namespace hbr {

// xgb_calc_weight (builder/shared.rs:86-97): unbounded, f64.
__device__ __forceinline__ double calc_weight(double g, double h, const ScanParams &r) {
    if (h <= 0.0) return 0.0;
    double w = -threshold_l1(g, r.alpha) / (h + r.lambda);
    if (r.max_delta_step != 0.0 && __builtin_fabs(w) > r.max_delta_step) w = __builtin_copysign(r.max_delta_step, w);
    return w;
}

// need_replace (builder/mod.rs:313-326) against the feature's own entry.
__device__ __forceinline__ bool beats(float loss, bool has, float incumbent) {
    if (__builtin_isinf(loss) || __builtin_isnan(loss)) return false;
    return loss > (has ? incumbent : 0.0f);
}

}  // namespace hbr

// One wave per (node, categorical feature): XGBoost's categorical sweep.
// Fewer than 4 categories: each alone, with missing values on either side
// (one-hot). Otherwise the categories stably sorted by their weight
// (CalcWeightCat: 0 below min_child_weight), then at most 64 deep a growing
// prefix of the order on one side scanned forward (missing values on the
// other side) and a growing suffix scanned backward (missing values with
// the prefix). Each candidate is scored as the numeric ones are; a
// direction keeps its first best, the backward best replaces the forward
// one only when strictly greater. Every category of the feature takes part,
// a category the node lacks with zero statistics. The record is written in
// the recorded orientation: `left` is the set's child (the child XGBoost
// calls right), flags bit0 sends missing values left, and the set (local
// bins) goes to cat_sets.
extern "C" __global__ __launch_bounds__(64) void hbr_scan_categorical(ScanArgs a) {
    __shared__ int64_t s_g[kCatMaxBins], s_h[kCatMaxBins];
    __shared__ float s_key[kCatMaxBins];
    __shared__ uint16_t s_order[kCatMaxBins], s_pos[kCatMaxBins];
    const uint32_t pair = blockIdx.x;
    if (pair >= scan_nodes(a) * a.n_cat) return;  // uniform per workgroup
    const uint32_t lane = threadIdx.x;
    const uint32_t node = pair / a.n_cat, rank = pair % a.n_cat;
    const uint32_t f = a.cat_feature[rank];
    const ScanNode nd = a.nodes[node];
    const uint32_t fs = a.feature_offset[f];
    const uint32_t nb = min(a.feature_offset[f + 1] - fs, kCatMaxBins);  // the host refuses wider ones
    const QBin *h = a.hist + (size_t)node_slot(a, nd) * a.total_bins + fs;
    const bool dev_root = (nd.pad & kScanDeviceRoot) != 0;
    const uint32_t cls = nd.pad >> kScanClassShift;
    int64_t tg = nd.total.g, th = nd.total.h;
    if (dev_root) {  // written by hbr_scan_features or hbr_total, earlier on the stream
        tg = a.root_total[cls].g;
        th = a.root_total[cls].h;
    }
    const int eg = a.scale[cls].exp_g, eh = a.scale[cls].exp_h;
    const int dir = a.monotone ? (int)a.monotone[f] : 0;
    const float root_gain =
        dev_root ? node_gain(dequant(tg, eg), dequant(th, eh), a.reg, nd.lower, nd.upper) : nd.root_gain;
    for (uint32_t b = lane; b < nb; b += kWave) {
        const QBin v = h[b];
        s_g[b] = v.g;
        s_h[b] = v.h;
    }
    __syncthreads();

    // the winner: its children in XGBoost's orientation (right = the set)
    bool has = false;
    float best_loss = 0.0f;
    uint32_t xgb_dl = 0, set_size = 0, chosen = 0;
    uint32_t replay = 0;  // kScanCatOrder / kScanCatNaN
    int64_t lg = 0, lh = 0, rg = 0, rh = 0;
    bool onehot = nb < 4;
    if (onehot) {
        if (lane == 0) {
            int64_t pg = 0, ph = 0;
            for (uint32_t i = 0; i < nb; i++) {
                pg += s_g[i];
                ph += s_h[i];
            }
            const int64_t mg = tg - pg, mh = th - ph;
            for (uint32_t i = 0; i < nb; i++) {
                for (uint32_t with_missing = 0; with_missing < 2; with_missing++) {
                    const int64_t cg = s_g[i] + (with_missing ? mg : 0), ch = s_h[i] + (with_missing ? mh : 0);
                    float loss;
                    const bool ok = score(dequant(tg - cg, eg), dequant(th - ch, eh), dequant(cg, eg),
                                          dequant(ch, eh), a.reg, nd.lower, nd.upper, dir, root_gain, &loss);
                    if (ok && loss != loss) replay |= kScanCatNaN;
                    if (ok && beats(loss, has, best_loss)) {
                        has = true;
                        best_loss = loss;
                        xgb_dl = with_missing ? 0u : 1u;
                        lg = tg - cg;
                        lh = th - ch;
                        rg = cg;
                        rh = ch;
                        chosen = i;
                    }
                }
            }
        }
    } else {
        for (uint32_t b = lane; b < nb; b += kWave) {
            const double g = dequant(s_g[b], eg), hh = dequant(s_h[b], eh);
            float k = hh < a.reg.min_child_weight ? 0.0f : (float)calc_weight(g, hh, a.reg);
            if (!__builtin_isfinite(k)) replay |= kScanCatOrder;  // the node is replayed on the host
            s_key[b] = k != k ? 0.0f : k;  // keeps this sort total meanwhile
        }
        __syncthreads();
        // stable ascending order: position = smaller keys + equal keys before
        for (uint32_t b = lane; b < nb; b += kWave) {
            const float k = s_key[b];
            uint32_t pos = 0;
            for (uint32_t j = 0; j < nb; j++) {
                const float kj = s_key[j];
                pos += (kj < k || (kj == k && j < b)) ? 1u : 0u;
            }
            s_pos[b] = (uint16_t)pos;
            s_order[pos] = (uint16_t)b;
        }
        __syncthreads();
        const uint32_t depth = min(nb, 64u), steps = depth - 1;
        float dl_loss[2];
        bool dl_has[2];
        uint32_t dl_step[2];
        int64_t dl_acc[2][2];
        for (uint32_t forward = 0; forward < 2; forward++) {  // 0: forward, 1: backward
            const bool fw = forward == 0;
            int64_t vg = 0, vh = 0;
            if (lane < steps) {
                const uint32_t b = s_order[fw ? lane : nb - 1 - lane];
                vg = s_g[b];
                vh = s_h[b];
            }
            const int64_t ag = wave_inclusive_scan(vg), ah = wave_inclusive_scan(vh);
            float loss = -__builtin_inff();
            bool ok = false;
            if (lane < steps) {
                if (fw)
                    ok = score(dequant(tg - ag, eg), dequant(th - ah, eh), dequant(ag, eg), dequant(ah, eh), a.reg,
                               nd.lower, nd.upper, dir, root_gain, &loss);
                else
                    ok = score(dequant(ag, eg), dequant(ah, eh), dequant(tg - ag, eg), dequant(th - ah, eh), a.reg,
                               nd.lower, nd.upper, dir, root_gain, &loss);
                if (ok && loss != loss) replay |= kScanCatNaN;
                ok = ok && beats(loss, false, 0.0f);
            }
            // the first step of the largest loss
            float bl = ok ? loss : -__builtin_inff();
            uint32_t bi = ok ? lane : 0xffffffffu;
#pragma unroll
            for (int d = 32; d >= 1; d >>= 1) {
                const float ol = __shfl_xor(bl, d, kWave);
                const uint32_t oi = (uint32_t)__shfl_xor((int)bi, d, kWave);
                if (oi != 0xffffffffu && (bi == 0xffffffffu || ol > bl || (ol == bl && oi < bi))) {
                    bl = ol;
                    bi = oi;
                }
            }
            dl_has[forward] = bi != 0xffffffffu;
            dl_loss[forward] = bl;
            dl_step[forward] = bi;
            dl_acc[forward][0] = wave_broadcast(ag, dl_has[forward] ? (int)bi : 0);
            dl_acc[forward][1] = wave_broadcast(ah, dl_has[forward] ? (int)bi : 0);
        }
        const uint32_t pick = dl_has[1] && (!dl_has[0] || dl_loss[1] > dl_loss[0]) ? 1u : 0u;
        if (dl_has[pick]) {
            has = true;
            best_loss = dl_loss[pick];
            const int64_t ag = dl_acc[pick][0], ah = dl_acc[pick][1];
            if (pick == 0) {  // set = the scanned prefix, missing values on the other side
                xgb_dl = 1;
                lg = tg - ag;
                lh = th - ah;
                rg = ag;
                rh = ah;
                set_size = dl_step[0] + 1;
            } else {  // set = the unscanned prefix, missing values with it
                xgb_dl = 0;
                lg = ag;
                lh = ah;
                rg = tg - ag;
                rh = th - ah;
                set_size = nb - 1 - dl_step[1];
            }
        }
    }
    replay = (__ballot((replay & kScanCatOrder) != 0) ? kScanCatOrder : 0u) |
             (__ballot((replay & kScanCatNaN) != 0) ? kScanCatNaN : 0u);
    if (onehot) {  // lane 0 holds the one-hot winner
        has = __shfl((int)has, 0, kWave) != 0;
        best_loss = __shfl(best_loss, 0, kWave);
        xgb_dl = (uint32_t)__shfl((int)xgb_dl, 0, kWave);
        chosen = (uint32_t)__shfl((int)chosen, 0, kWave);
        lg = wave_broadcast(lg, 0);
        lh = wave_broadcast(lh, 0);
        rg = wave_broadcast(rg, 0);
        rh = wave_broadcast(rh, 0);
    }
    uint32_t *set = a.cat_sets + ((size_t)node * a.n_cat + rank) * kCatWords;
    for (uint32_t w = lane; w < kCatWords; w += kWave) {
        uint32_t bits = 0;
        if (has) {
            for (uint32_t i = 0; i < 32; i++) {
                const uint32_t b = 32 * w + i;
                if (b >= nb) break;
                const bool in = onehot ? b == chosen : (uint32_t)s_pos[b] < set_size;
                bits |= in ? 1u << i : 0u;
            }
        }
        set[w] = bits;
    }
    if (lane == 0) {
        ScanBest o;
        o.feature = f;
        if (has) {
            o.loss = best_loss;
            o.index = 0;
            o.flags = kScanCategorical | (xgb_dl ? 0u : 1u) | replay;  // recorded: the set's child on the left
            o.left = QBin{rg, rh};
            o.right = QBin{lg, lh};
        } else {
            o.loss = -__builtin_inff();
            o.index = 0xffffffffu;
            o.flags = replay;
            o.left = QBin{0, 0};
            o.right = QBin{0, 0};
        }
        o.err = 0.0f;  // categorical sweeps are not bounded by the guard
        o.rival = -__builtin_inff();
        a.per_feature[(size_t)node * a.n_features + f] = o;
    }
}
