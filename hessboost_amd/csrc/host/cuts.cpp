#include "cuts.h"

#include <algorithm>
#include <cmath>
#include <cstring>

namespace hbr {

namespace {

// A weighted-quantile summary entry: value with rank bounds [rmin, rmax]
// and its own weight wmin, every quantity f32 (sketch.rs:24-56).
struct Entry {
    float rmin, rmax, wmin, value;
    float rmin_next() const { return rmin + wmin; }
    float rmax_prev() const { return rmax - wmin; }
};

using Summary = std::vector<Entry>;

// SketchEpsilon / LimitSizeLevel / SketchSummaryBudget (sketch.rs:59-85).
size_t budget(size_t max_bin, size_t n) {
    const size_t samples = std::max<size_t>(n, 1);
    const double eps = 1.0 / (double)std::min(max_bin, samples);
    if (n == 0) return 1;
    const double half = eps / 2.0;
    for (unsigned level = 1;; level++) {
        const size_t limit = std::min((size_t)std::ceil((double)level / half) + 1, n);
        if ((size_t(1) << level) * limit >= n) return limit;
    }
}

// SetPrune (sketch.rs:131-181): answer maxsize - 1 evenly spaced rank
// queries, keeping the chosen entries in place, plus the last.
void prune(Summary &s, size_t maxsize) {
    const size_t src = s.size();
    if (maxsize == 0) {
        s.clear();
        return;
    }
    if (src <= maxsize) return;
    if (maxsize == 1) {
        s.resize(1);
        return;
    }
    const float begin = s[0].rmax;
    const float range = s[src - 1].rmin - s[0].rmax;
    const size_t n = maxsize - 1;
    const Entry tail = s[src - 1];
    Entry left = s[1], right = s[2];
    size_t kept = 1, i = 1, last = 0;
    for (size_t k = 1; k < n; k++) {
        const float dx2 = 2.0f * (((float)k * range) / (float)n + begin);
        while (i < src - 1 && dx2 >= right.rmax + right.rmin) {
            ++i;
            left = right;
            if (i < src - 1) right = s[i + 1];
        }
        if (i == src - 1) break;
        if (dx2 < left.rmin_next() + right.rmax_prev()) {
            if (i != last) {
                s[kept++] = left;
                last = i;
            }
        } else if (i + 1 != last) {
            s[kept++] = right;
            last = i + 1;
        }
    }
    if (last != src - 1) s[kept++] = tail;
    s.resize(kept);
}

// FixError (sketch.rs:184-201).
void fix_error(Summary &s) {
    float pmin = 0.0f, pmax = 0.0f;
    for (Entry &e : s) {
        if (e.rmin < pmin)
            e.rmin = pmin;
        else
            pmin = e.rmin;
        if (e.rmax < pmax) e.rmax = pmax;
        const float next = e.rmin_next();
        if (e.rmax < next) e.rmax = next;
        pmax = e.rmax;
    }
}

// SetCombine (sketch.rs:218-345): merge b into a.
void combine(Summary &a, const Summary &b, Summary &scratch) {
    if (b.empty()) return;
    if (a.empty()) {
        a = b;
        return;
    }
    scratch.clear();
    scratch.reserve(a.size() + b.size());
    size_t ia = 0, ib = 0;
    float aprev = 0.0f, bprev = 0.0f;
    while (ia < a.size() && ib < b.size()) {
        const Entry &x = a[ia], &y = b[ib];
        const bool eq = x.value == y.value, lt = x.value < y.value;
        const bool ta = eq || lt, tb = !lt;
        Entry o;
        o.rmin = (ta ? x.rmin : aprev) + (tb ? y.rmin : bprev);
        o.rmax = (ta ? x.rmax : x.rmax_prev()) + (tb ? y.rmax : y.rmax_prev());
        o.wmin = eq ? x.wmin + y.wmin : (lt ? x.wmin : y.wmin);
        o.value = ta ? x.value : y.value;
        scratch.push_back(o);
        if (ta) aprev = x.rmin_next();
        if (tb) bprev = y.rmin_next();
        ia += ta;
        ib += tb;
    }
    for (; ia < a.size(); ia++) {
        const Entry &x = a[ia];
        const float next = ib < b.size() ? b[ib].rmax_prev() : b.back().rmax;
        scratch.push_back(Entry{x.rmin + bprev, x.rmax + next, x.wmin, x.value});
        aprev = x.rmin_next();
    }
    for (; ib < b.size(); ib++) {
        const Entry &y = b[ib];
        const float next = ia < a.size() ? a[ia].rmax_prev() : a.back().rmax;
        scratch.push_back(Entry{y.rmin + aprev, y.rmax + next, y.wmin, y.value});
        bprev = y.rmin_next();
    }
    fix_error(scratch);
    a.swap(scratch);
}

// QueryCutValues (sketch.rs:458-509).
void query(const Summary &s, size_t max_bin, std::vector<float> &out) {
    const size_t n = s.size();
    if (n == 0) {
        out.push_back(1e-5f);
        return;
    }
    auto skip = [&](size_t c, float v) {
        while (c < n && s[c].value <= v) c++;
        return c;
    };
    float last = s[0].value;
    size_t next = skip(1, last);
    if (n <= max_bin) {
        while (next < n) {
            const float c = s[next].value;
            out.push_back(c);
            last = c;
            next = skip(next + 1, last);
        }
    } else {
        const double total = (double)s[n - 1].rmax;
        size_t q = 0;
        for (size_t i = 1; i < max_bin; i++) {
            const double rank2 = 2.0 * ((double)i * total / (double)max_bin);
            while (q < n - 2 && rank2 >= (double)(s[q + 1].rmin + s[q + 1].rmax)) q++;
            const Entry &e = rank2 < (double)(s[q].rmin_next() + s[q + 1].rmax_prev()) ? s[q] : s[q + 1];
            float c = e.value;
            if (c <= last) {
                next = skip(next, last);
                if (next == n) break;
                c = s[next].value;
            } else if (next < n && s[next].value <= c) {
                next = skip(next + 1, c);
            }
            out.push_back(c);
            last = c;
        }
    }
    const float top = s[n - 1].value;
    out.push_back(top + (std::fabs(top) + 1e-5f));
}

uint32_t order_key(float v) {
    uint32_t b;
    std::memcpy(&b, &v, 4);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// One feature's streaming sketch (WQuantileSketch, sketch.rs:512-708).
class Sketch {
public:
    Sketch(size_t n_values, size_t max_bin) : max_bin_(max_bin), limit_(budget(max_bin, n_values)) {
        queue_.reserve(2 * limit_);
    }

    void push(float v, float w) {
        if (w == 0.0f) return;
        count_++;
        if (!queue_.empty() && queue_.back().first == v) {
            queue_.back().second += w;
            return;
        }
        if (queue_.size() == 2 * limit_) flush();
        queue_.push_back({v, w});
    }

    std::vector<float> cut_values() {
        const size_t b = budget(max_bin_, count_);
        flush();
        const size_t prune_size = std::max(b, limit_);
        Summary all, scratch;
        for (const Summary &lv : levels_) {
            combine(all, lv, scratch);
            prune(all, prune_size);
        }
        prune(all, b);
        std::vector<float> out;
        query(all, std::min(all.size(), max_bin_), out);
        return out;
    }

private:
    // Queue::PopSummary (sorted by f32 total order, equal values merged
    // with their weights summed in order) and PushSummary (carry up levels).
    void flush() {
        std::stable_sort(queue_.begin(), queue_.end(),
                         [](const auto &x, const auto &y) { return order_key(x.first) < order_key(y.first); });
        Summary fresh;
        float wsum = 0.0f;
        for (size_t i = 0; i < queue_.size();) {
            const float v = queue_[i].first;
            float w = queue_[i].second;
            size_t j = i + 1;
            while (j < queue_.size() && queue_[j].first == v) w += queue_[j++].second;
            fresh.push_back(Entry{wsum, wsum + w, w, v});
            wsum += w;
            i = j;
        }
        queue_.clear();
        Summary scratch;
        for (size_t l = 0;; l++) {
            if (levels_.size() <= l) levels_.emplace_back();
            prune(fresh, limit_);
            combine(fresh, levels_[l], scratch);
            levels_[l].clear();
            if (fresh.size() <= limit_) {
                levels_[l].swap(fresh);
                break;
            }
        }
    }

    size_t max_bin_, limit_, count_ = 0;
    std::vector<std::pair<float, float>> queue_;
    std::vector<Summary> levels_;
};

bool absent(float v, float missing) { return std::isnan(missing) ? std::isnan(v) : v == missing; }

Cuts assemble(std::vector<std::vector<float>> &per, const uint8_t *categorical) {
    Cuts c;
    c.feature_offset.push_back(0);
    for (auto &v : per) {
        c.values.insert(c.values.end(), v.begin(), v.end());
        c.feature_offset.push_back((uint32_t)c.values.size());
    }
    if (categorical)
        for (size_t j = 0; j < per.size(); j++) c.categorical.push_back(categorical[j] ? 1 : 0);
    return c;
}

// f32::total_cmp as an unsigned key
uint32_t total_order(float v) {
    uint32_t b;
    std::memcpy(&b, &v, 4);
    return (b >> 31) ? ~b : (b | 0x80000000u);
}

// A categorical feature's cuts (quantile.rs:524-672, build_categorical_cuts
// :676-689): the present values sorted by total_cmp, deduplicated by bit
// pattern, then one bin per value that differs (`!=`) from the one before;
// a feature without a present value keeps one degenerate bin at 0.
std::vector<float> category_cuts(std::vector<float> vals) {
    std::sort(vals.begin(), vals.end(), [](float a, float b) { return total_order(a) < total_order(b); });
    vals.erase(std::unique(vals.begin(), vals.end(),
                           [](float a, float b) { return std::memcmp(&a, &b, 4) == 0; }),
               vals.end());
    std::vector<float> out;
    if (vals.empty()) return {0.0f};
    out.push_back(vals[0]);
    for (size_t i = 1; i < vals.size(); i++)
        if (vals[i - 1] != vals[i]) out.push_back(vals[i]);
    return out;
}

}  // namespace

uint32_t Cuts::bin_of(uint32_t f, float v) const {
    const float *lo = values.data() + feature_offset[f];
    const float *hi = values.data() + feature_offset[f + 1];
    if (is_categorical(f)) {
        // the bin whose category equals v, else the feature's first bin
        const float *at = std::lower_bound(lo, hi, v);
        return feature_offset[f] + (at != hi && *at == v ? (uint32_t)(at - lo) : 0u);
    }
    const size_t n = (size_t)(hi - lo);
    size_t k = (size_t)(std::upper_bound(lo, hi, v) - lo);
    if (k > n - 1) k = n - 1;
    return feature_offset[f] + (uint32_t)k;
}

Cuts cuts_from_dense(const float *x, uint64_t n, uint64_t f, uint32_t max_bin, const float *weights, float missing,
                     const uint8_t *categorical) {
    std::vector<std::vector<float>> per(f);
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t j = 0; j < (int64_t)f; j++) {
        size_t present = 0;
        for (uint64_t r = 0; r < n; r++) present += !absent(x[r * f + j], missing);
        if (categorical && categorical[j]) {
            std::vector<float> vals;
            vals.reserve(present);
            for (uint64_t r = 0; r < n; r++)
                if (!absent(x[r * f + j], missing)) vals.push_back(x[r * f + j]);
            per[j] = category_cuts(std::move(vals));
            continue;
        }
        Sketch s(present, max_bin);
        for (uint64_t r = 0; r < n; r++) {
            const float v = x[r * f + j];
            if (!absent(v, missing)) s.push(v, weights ? weights[r] : 1.0f);
        }
        per[j] = s.cut_values();
    }
    return assemble(per, categorical);
}

Cuts cuts_from_csr(const uint64_t *row_ptr, const uint32_t *col, const float *val, uint64_t n, uint64_t f,
                   uint32_t max_bin, const float *weights, const uint8_t *categorical) {
    std::vector<std::vector<std::pair<uint32_t, float>>> csc(f);
    for (uint64_t r = 0; r < n; r++)
        for (uint64_t e = row_ptr[r]; e < row_ptr[r + 1]; e++) csc[col[e]].push_back({(uint32_t)r, val[e]});
    std::vector<std::vector<float>> per(f);
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t j = 0; j < (int64_t)f; j++) {
        if (categorical && categorical[j]) {
            std::vector<float> vals;
            vals.reserve(csc[j].size());
            for (auto &rv : csc[j]) vals.push_back(rv.second);
            per[j] = category_cuts(std::move(vals));
            continue;
        }
        Sketch s(csc[j].size(), max_bin);
        for (auto &rv : csc[j]) s.push(rv.second, weights ? weights[rv.first] : 1.0f);
        per[j] = s.cut_values();
    }
    return assemble(per, categorical);
}

namespace {

void layout(Index &ix) {
    const uint64_t cells = ix.n_rows * ix.n_cols;
    const uint64_t entries = ix.row_ptr[ix.n_rows];
    ix.row_width = ix.cuts.total_bins() <= 65536 ? 2 : 4;
    if (ix.row_width == 2)
        ix.rows16.assign(entries, 0);
    else
        ix.rows32.assign(entries, 0);
    uint32_t widest = 0;
    for (uint32_t f = 0; f < ix.n_cols; f++)
        widest = std::max(widest, ix.cuts.feature_offset[f + 1] - ix.cuts.feature_offset[f]);
    ix.col_width = 0;
    if (cells <= 2 * entries) {
        ix.col_width = widest <= 256 ? 1 : (widest <= 65536 ? 2 : 4);
        if (ix.col_width == 1) ix.cols8.assign(cells, 0);
        if (ix.col_width == 2) ix.cols16.assign(cells, 0);
        if (ix.col_width == 4) ix.cols32.assign(cells, 0);
        if (entries < cells) {
            const uint64_t words = (ix.n_rows + 63) / 64;
            ix.missing.assign(words * ix.n_cols, 0);
            for (uint64_t f = 0; f < ix.n_cols; f++)
                for (uint64_t w = 0; w < words; w++) {
                    const uint64_t valid = std::min<uint64_t>(64, ix.n_rows - w * 64);
                    ix.missing[f * words + w] = valid == 64 ? ~0ull : ((1ull << valid) - 1);
                }
        }
    }
}

// Store one present cell; rows are binned in blocks of 64 so each block
// owns whole words of every feature's missing bitmap.
inline void put(Index &ix, uint64_t r, uint64_t e, uint32_t f, uint32_t global) {
    if (ix.row_width == 2)
        ix.rows16[e] = (uint16_t)global;
    else
        ix.rows32[e] = global;
    if (ix.col_width) {
        const uint32_t local = global - ix.cuts.feature_offset[f];
        const uint64_t at = (uint64_t)f * ix.n_rows + r;
        if (ix.col_width == 1) ix.cols8[at] = (uint8_t)local;
        if (ix.col_width == 2) ix.cols16[at] = (uint16_t)local;
        if (ix.col_width == 4) ix.cols32[at] = local;
        if (!ix.missing.empty()) {
            const uint64_t words = (ix.n_rows + 63) / 64;
            ix.missing[f * words + (r >> 6)] &= ~(1ull << (r & 63));
        }
    }
}

}  // namespace

Index index_from_dense(const float *x, uint64_t n, uint64_t f, float missing, const Cuts &cuts) {
    Index ix;
    ix.cuts = cuts;
    ix.n_rows = n;
    ix.n_cols = f;
    ix.row_ptr.assign(n + 1, 0);
    for (uint64_t r = 0; r < n; r++) {
        uint64_t c = 0;
        for (uint64_t j = 0; j < f; j++) c += !absent(x[r * f + j], missing);
        ix.row_ptr[r + 1] = ix.row_ptr[r] + c;
    }
    layout(ix);
    ix.dense = ix.row_ptr[n] == n * f;
    const int64_t blocks = (int64_t)((n + 63) / 64);
#pragma omp parallel for schedule(static)
    for (int64_t b = 0; b < blocks; b++) {
        const uint64_t end = std::min<uint64_t>(n, (uint64_t)(b + 1) * 64);
        for (uint64_t r = (uint64_t)b * 64; r < end; r++) {
            uint64_t e = ix.row_ptr[r];
            for (uint32_t j = 0; j < f; j++) {
                const float v = x[r * f + j];
                if (!absent(v, missing)) put(ix, r, e++, j, cuts.bin_of(j, v));
            }
        }
    }
    return ix;
}

Index index_from_csr(const uint64_t *row_ptr, const uint32_t *col, const float *val, uint64_t n, uint64_t f,
                     const Cuts &cuts) {
    Index ix;
    ix.cuts = cuts;
    ix.n_rows = n;
    ix.n_cols = f;
    ix.row_ptr.assign(row_ptr, row_ptr + n + 1);
    layout(ix);
    bool dense = true;
    for (uint64_t r = 0; r < n && dense; r++) {
        if (row_ptr[r + 1] - row_ptr[r] != f) dense = false;
        for (uint64_t e = row_ptr[r]; e < row_ptr[r + 1] && dense; e++)
            if (col[e] != e - row_ptr[r]) dense = false;
    }
    ix.dense = dense;
    const int64_t blocks = (int64_t)((n + 63) / 64);
#pragma omp parallel for schedule(static)
    for (int64_t b = 0; b < blocks; b++) {
        const uint64_t end = std::min<uint64_t>(n, (uint64_t)(b + 1) * 64);
        for (uint64_t r = (uint64_t)b * 64; r < end; r++)
            for (uint64_t e = row_ptr[r]; e < row_ptr[r + 1]; e++) put(ix, r, e, col[e], cuts.bin_of(col[e], val[e]));
    }
    return ix;
}

}  // namespace hbr
