// The extern "C" boundary (include/hessboost_rocm.h): argument checks,
// status codes, per-handle locking and the sticky failure flag.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <memory>
#include <string>

#include "cuts.h"
#include "engine.h"
#include "forest.h"
#include "noalloc.h"
#include "split_math.h"
#include "hessboost_rocm.h"
#include "trainer.h"

using namespace hbr;

struct hbr_cuts {
    Cuts c;
};
struct hbr_index {
    Index ix;
};
struct hbr_engine {
    std::unique_ptr<Engine> e;
    std::vector<uint32_t> scan_categories;  // the last scan's category pool
};
struct hbr_trainer {
    hbr_engine *engine;
    std::unique_ptr<Trainer> t;
};
struct hbr_forest {
    std::unique_ptr<Forest> f;
};

namespace {

thread_local std::string g_error;

int set_error(int status, const std::string &msg) {
    g_error = msg;
    return status;
}

template <typename F>
int guard(F &&fn) {
    try {
        g_error.clear();
        fn();
        return HBR_OK;
    } catch (const Error &e) {
        return set_error(e.status, e.what());
    } catch (const std::bad_alloc &) {
        return set_error(HBR_REFUSED, "host allocation failed");
    } catch (const std::exception &e) {
        return set_error(HBR_INVALID, e.what());
    }
}

// Run fn under the engine's lock; a device error poisons the engine. Rows
// a trainer reordered go back to the caller's order first, except for the
// trainer's own calls and those that touch no row (keep_order).
template <typename F>
int with_engine(hbr_engine *h, F &&fn, bool keep_order = false) {
    if (!h || !h->e) return set_error(HBR_INVALID, "null engine");
    Engine &e = *h->e;
    std::lock_guard<std::mutex> lock(e.mu);
    if (e.failed) return set_error(HBR_DEVICE_ERROR, "the engine failed earlier; every call is refused");
    int st = guard([&] {
        e.dev().activate();
        if (!keep_order) e.restore_row_order();
        fn(e);
    });
    if (st == HBR_DEVICE_ERROR) e.failed = true;
    return st;
}

template <typename F>
int with_forest(hbr_forest *h, F &&fn) {
    if (!h || !h->f) return set_error(HBR_INVALID, "null forest");
    Forest &f = *h->f;
    std::lock_guard<std::mutex> lock(f.mu);
    if (f.failed) return set_error(HBR_DEVICE_ERROR, "the forest's device failed earlier");
    int st = guard([&] {
        f.dev().activate();
        fn(f);
    });
    if (st == HBR_DEVICE_ERROR) f.failed = true;
    return st;
}

Segment seg_of(const Engine &e, const hbr_segment &s) {
    if (s.tree != e.tree()) fail(kRefused, "segment of an earlier tree");
    if (s.buffer > 1 || s.offset + s.len > e.n_rows()) fail(kInvalid, "segment outside the row buffers");
    return Segment{(uint32_t)s.offset, (uint32_t)s.len, s.buffer};
}

hbr_segment seg_out(const Engine &e, const Segment &s) {
    hbr_segment o{};
    o.offset = s.offset;
    o.len = s.len;
    o.buffer = s.buf;
    o.contiguous = 0;
    o.tree = e.tree();
    return o;
}

void dequant_hist(const Engine &e, const std::vector<QBin> &q, double *out) {
    const int eg = e.scale().exp_g, eh = e.scale().exp_h;
    for (size_t b = 0; b < q.size(); b++) {
        out[2 * b] = std::ldexp((double)q[b].g, eg);
        out[2 * b + 1] = std::ldexp((double)q[b].h, eh);
    }
}

// The trait's promise (src/tree/hist/mod.rs:205-207, :220-224): histograms
// and root totals equal the CPU's f64 sums bit for bit. The engine keeps it
// by refusing (the trait's None: the host sums itself, as the CUDA backend
// does outside its exact domain, src/backend/cuda/mod.rs:2758-2776) unless
// every sum of `m` staged pairs is exact, or the caller has chosen
// fixed-point sums (hbr_engine_set_sums).
void require_exact(const Engine &e, uint64_t m, const char *what) {
    if (e.exact_sums_only && !e.sums_exact(m))
        fail(kRefused, std::string(what) + ": the staged gradients are outside the exact domain, where fixed-point "
                                           "sums can differ from the CPU's f64 sums (hbr_engine_set_sums selects them)");
}

std::string stats_string(Device &d) {
    std::string s;
    for (auto &kv : d.kernel_stats()) {
        char buf[160];
        std::snprintf(buf, sizeof buf, "%s=%.6f,%llu,%llu;", kv.first.c_str(), kv.second.total_ms,
                      (unsigned long long)kv.second.launches, (unsigned long long)kv.second.calls);
        s += buf;
    }
    return s;
}

size_t copy_string(const std::string &s, char *buf, size_t len) {
    if (buf && len) {
        const size_t n = std::min(len - 1, s.size());
        std::memcpy(buf, s.data(), n);
        buf[n] = 0;
    }
    return s.size();
}

}  // namespace

extern "C" {

size_t hbr_last_error(char *buf, size_t len) { return copy_string(g_error, buf, len); }

int hbr_pred_transform(int kind, float *values, uint64_t n_rows, uint32_t n_outputs) {
    return guard([&] {
        if (!values && n_rows) fail(kInvalid, "transform: null values");
        if (n_outputs == 0) fail(kInvalid, "transform: no outputs");
        const int64_t rows = (int64_t)n_rows;
        const uint32_t k = n_outputs;
        switch (kind) {
        case HBR_TRANSFORM_SIGMOID: {
            const int64_t n = rows * (int64_t)k;
#pragma omp parallel for schedule(static) if (n >= (1 << 15))
            for (int64_t i = 0; i < n; i++) values[i] = 1.0f / (expf(fminf(-values[i], 88.7f)) + 1.0f);
            break;
        }
        case HBR_TRANSFORM_SOFTMAX:
#pragma omp parallel for schedule(static) if (rows * k >= (1 << 15))
            for (int64_t r = 0; r < rows; r++) {
                float *v = values + r * k;
                float wmax = v[0];
                for (uint32_t c = 1; c < k; c++) wmax = fmaxf(v[c], wmax);
                double wsum = 0.0;
                for (uint32_t c = 0; c < k; c++) {
                    v[c] = expf(v[c] - wmax);
                    wsum += (double)v[c];
                }
                const float s = (float)wsum;
                for (uint32_t c = 0; c < k; c++) v[c] /= s;
            }
            break;
        case HBR_TRANSFORM_CLASS_INDEX:
            // row r lands at index r, at or before its own values
            for (int64_t r = 0; r < rows; r++) {
                const float *v = values + r * k;
                uint32_t best = 0;
                for (uint32_t c = 1; c < k; c++)
                    if (v[c] > v[best]) best = c;
                values[r] = (float)best;
            }
            break;
        default:
            fail(kInvalid, "transform: unknown kind");
        }
    });
}

int hbr_device_count(int *count) {
    return guard([&] {
        if (!count) fail(kInvalid, "null count");
        *count = device_count();
    });
}

int hbr_device_name(int ordinal, char *buf, size_t len) {
    return guard([&] {
        if (!buf && len) fail(kInvalid, "device_name: null buffer");
        if (ordinal < 0 || ordinal >= device_count()) fail(kInvalid, "device_name: no such device");
        hipDeviceProp_t p;
        HBR_HIP(hipGetDeviceProperties(&p, ordinal));
        copy_string(std::string(p.name) + " (" + p.gcnArchName + ")", buf, len);
    });
}

// ---- cuts and index -----------------------------------------------------------

int hbr_cuts_from_dense(const float *x, uint64_t n, uint64_t f, uint32_t max_bin, const float *weights,
                        float missing, hbr_cuts **out) {
    return guard([&] {
        if (!out || (!x && n > 0 && f > 0) || max_bin < 2) fail(kInvalid, "cuts: bad arguments");
        *out = new hbr_cuts{cuts_from_dense(x, n, f, max_bin, weights, missing)};
    });
}

int hbr_cuts_from_csr(const uint64_t *row_ptr, const uint32_t *col, const float *val, uint64_t n, uint64_t f,
                      uint32_t max_bin, const float *weights, hbr_cuts **out) {
    return guard([&] {
        if (!out || !row_ptr || max_bin < 2) fail(kInvalid, "cuts: bad arguments");
        if (row_ptr[n] && (!col || !val)) fail(kInvalid, "cuts: null col or val with entries present");
        for (uint64_t e = 0; e < row_ptr[n]; e++)
            if (col[e] >= f) fail(kInvalid, "cuts: column index beyond n_cols");
        *out = new hbr_cuts{cuts_from_csr(row_ptr, col, val, n, f, max_bin, weights)};
    });
}

int hbr_cuts_from_dense_typed(const float *x, uint64_t n, uint64_t f, uint32_t max_bin, const float *weights,
                              float missing, const uint8_t *categorical, hbr_cuts **out) {
    return guard([&] {
        if (!out || (!x && n > 0 && f > 0) || max_bin < 2) fail(kInvalid, "cuts: bad arguments");
        *out = new hbr_cuts{cuts_from_dense(x, n, f, max_bin, weights, missing, categorical)};
    });
}

int hbr_cuts_from_csr_typed(const uint64_t *row_ptr, const uint32_t *col, const float *val, uint64_t n, uint64_t f,
                            uint32_t max_bin, const float *weights, const uint8_t *categorical, hbr_cuts **out) {
    return guard([&] {
        if (!out || !row_ptr || max_bin < 2) fail(kInvalid, "cuts: bad arguments");
        if (row_ptr[n] && (!col || !val)) fail(kInvalid, "cuts: null col or val with entries present");
        for (uint64_t e = 0; e < row_ptr[n]; e++)
            if (col[e] >= f) fail(kInvalid, "cuts: column index beyond n_cols");
        *out = new hbr_cuts{cuts_from_csr(row_ptr, col, val, n, f, max_bin, weights, categorical)};
    });
}

int hbr_cuts_categorical(const hbr_cuts *c, uint8_t *out) {
    return guard([&] {
        if (!c || !out) fail(kInvalid, "null cuts");
        for (uint32_t f = 0; f < c->c.n_cols(); f++) out[f] = c->c.is_categorical(f) ? 1 : 0;
    });
}

int hbr_cuts_from_values(const uint32_t *fo, const float *values, uint64_t n_cols, hbr_cuts **out) {
    return guard([&] {
        if (!out || !fo || !values) fail(kInvalid, "cuts: bad arguments");
        hbr_cuts *c = new hbr_cuts;
        c->c.feature_offset.assign(fo, fo + n_cols + 1);
        for (uint64_t f = 0; f < n_cols; f++)
            if (fo[f + 1] <= fo[f]) {
                delete c;
                fail(kInvalid, "cuts: every feature owns at least one bin");
            }
        c->c.values.assign(values, values + fo[n_cols]);
        *out = c;
    });
}

int hbr_cuts_info(const hbr_cuts *c, uint64_t *n_cols, uint64_t *total_bins) {
    return guard([&] {
        if (!c) fail(kInvalid, "null cuts");
        if (n_cols) *n_cols = c->c.n_cols();
        if (total_bins) *total_bins = c->c.total_bins();
    });
}

int hbr_cuts_copy(const hbr_cuts *c, uint32_t *fo, float *values) {
    return guard([&] {
        if (!c) fail(kInvalid, "null cuts");
        if (fo) std::memcpy(fo, c->c.feature_offset.data(), c->c.feature_offset.size() * 4);
        if (values) std::memcpy(values, c->c.values.data(), c->c.values.size() * 4);
    });
}

void hbr_cuts_free(hbr_cuts *c) { delete c; }

int hbr_index_from_dense(const float *x, uint64_t n, uint64_t f, float missing, const hbr_cuts *cuts,
                         hbr_index **out) {
    return guard([&] {
        if (!out || !cuts || cuts->c.n_cols() != f) fail(kInvalid, "index: cuts do not match the matrix");
        *out = new hbr_index{index_from_dense(x, n, f, missing, cuts->c)};
    });
}

int hbr_index_from_csr(const uint64_t *row_ptr, const uint32_t *col, const float *val, uint64_t n, uint64_t f,
                       const hbr_cuts *cuts, hbr_index **out) {
    return guard([&] {
        if (!out || !cuts || cuts->c.n_cols() != f) fail(kInvalid, "index: cuts do not match the matrix");
        *out = new hbr_index{index_from_csr(row_ptr, col, val, n, f, cuts->c)};
    });
}

void hbr_index_free(hbr_index *ix) { delete ix; }

int hbr_index_describe(const hbr_index *h, hbr_index_desc *d) {
    return guard([&] {
        if (!h || !d) fail(kInvalid, "null index");
        const Index &ix = h->ix;
        *d = hbr_index_desc{};
        d->n_rows = ix.n_rows;
        d->n_cols = ix.n_cols;
        d->feature_offset = ix.cuts.feature_offset.data();
        d->cut_values = ix.cuts.values.data();
        d->row_ptr = ix.row_ptr.data();
        d->row_bin_width = ix.row_width;
        d->row_bins = ix.row_width == 2 ? (const void *)ix.rows16.data() : (const void *)ix.rows32.data();
        d->dense = ix.dense ? 1u : 0u;
        d->col_bin_width = ix.col_width;
        d->col_bins = ix.col_width == 1   ? (const void *)ix.cols8.data()
                      : ix.col_width == 2 ? (const void *)ix.cols16.data()
                      : ix.col_width == 4 ? (const void *)ix.cols32.data()
                                          : nullptr;
        d->missing = ix.missing.empty() ? nullptr : ix.missing.data();
        d->is_categorical = ix.cuts.categorical.empty() ? nullptr : ix.cuts.categorical.data();
    });
}

// ---- engine -----------------------------------------------------------------------

int hbr_engine_open(int ordinal, const hbr_index_desc *index, hbr_engine **out) {
    return guard([&] {
        if (!index || !out) fail(kInvalid, "engine: null argument");
        auto *h = new hbr_engine;
        try {
            h->e = std::make_unique<Engine>(ordinal, *index);
        } catch (...) {
            delete h;
            throw;
        }
        *out = h;
    });
}

void hbr_engine_close(hbr_engine *e) { delete e; }

int hbr_engine_open_dense(int ordinal, const float *x, uint64_t n_rows, uint64_t n_cols, float missing,
                          const hbr_cuts *cuts, int x_on_device, hbr_engine **out) {
    return guard([&] {
        if (!x || !cuts || !out) fail(kInvalid, "engine: null argument");
        if (n_cols != cuts->c.n_cols()) fail(kInvalid, "engine: the cuts are for another number of features");
        Engine::DenseSource src;
        src.x = x;
        src.on_device = x_on_device != 0;
        src.n_rows = n_rows;
        src.n_cols = n_cols;
        src.missing = missing;
        src.feature_offset = cuts->c.feature_offset.data();
        src.cut_values = cuts->c.values.data();
        auto *h = new hbr_engine;
        try {
            h->e = std::make_unique<Engine>(ordinal, src);
        } catch (...) {
            delete h;
            throw;
        }
        *out = h;
    });
}

int hbr_engine_index_info(hbr_engine *h, hbr_index_info *out) {
    return with_engine(h, [&](Engine &e) {
        if (!out) fail(kInvalid, "index_info: null argument");
        const Engine::IndexInfo i = e.index_info();
        *out = hbr_index_info{i.dense, i.dense_u8, i.has_cols, i.has_missing, i.stride, 0, i.entries};
    });
}

int hbr_engine_index_read(hbr_engine *h, uint8_t *rows8, uint8_t *cols8, uint64_t *missing, uint64_t *row_ptr,
                          uint32_t *gbins) {
    return with_engine(h, [&](Engine &e) { e.read_index(rows8, cols8, missing, row_ptr, gbins); });
}

int hbr_prepare(hbr_engine *h, const float *gpair, uint64_t n) {
    return with_engine(h, [&](Engine &e) { e.prepare(gpair, n); });
}

int hbr_build(hbr_engine *h, const uint32_t *rows, uint64_t m, double *out) {
    return with_engine(h, [&](Engine &e) {
        if (!out || (!rows && m)) fail(kInvalid, "build: null argument");
        require_exact(e, m, "build");
        dequant_hist(e, e.build_rows(rows, m), out);
    });
}

int hbr_build_device_noalloc(hbr_engine *h, const uint32_t *rows, uint64_t m, double *out) {
    // the rows stay where they are: putting a trainer's reordered rows back
    // would allocate and free
    return with_engine(
        h,
        [&](Engine &e) {
            if (!out || (!rows && m)) fail(kInvalid, "build: null argument");
            if (e.rows_permuted())
                fail(kRefused, "build (no allocation): a trainer holds the rows in a tree's leaf order; any other "
                               "engine call puts them back");
            require_exact(e, m, "build");
            const auto held = fixed_scratch_lock(e.dev().ordinal());
            uint64_t bytes = 0;
            uint8_t *scratch = fixed_scratch(e.dev().ordinal(), &bytes);
            if (!e.build_rows_fixed(rows, m, out, scratch, bytes)) fail(kInvalid, "build: a row beyond the index");
        },
        true);
}

int hbr_begin_tree(hbr_engine *h, uint64_t n_rows, hbr_segment *root) {
    return with_engine(h, [&](Engine &e) {
        if (n_rows != e.n_rows()) fail(kRefused, "begin_tree: only an unsampled tree over every row");
        e.begin_tree();
        *root = seg_out(e, Segment{0, (uint32_t)n_rows, 0});
        root->contiguous = 1;
    });
}

int hbr_root_total_fixed(hbr_engine *h, const hbr_segment *seg, double out[2], int64_t fixed[2]) {
    return with_engine(h, [&](Engine &e) {
        const Segment sg = seg_of(e, *seg);
        require_exact(e, sg.len, "root_total");
        const QBin t = e.root_total(sg);
        out[0] = std::ldexp((double)t.g, e.scale().exp_g);
        out[1] = std::ldexp((double)t.h, e.scale().exp_h);
        if (fixed) {
            fixed[0] = t.g;
            fixed[1] = t.h;
        }
    });
}

int hbr_root_total(hbr_engine *h, const hbr_segment *seg, double out[2]) {
    return hbr_root_total_fixed(h, seg, out, nullptr);
}

int hbr_partition(hbr_engine *h, const hbr_row_split *splits, uint64_t n, hbr_partitioned *out) {
    return with_engine(h, [&](Engine &e) {
        std::vector<LevelSplit> ls(n);
        const auto &fo = e.feature_offset();
        for (uint64_t i = 0; i < n; i++) {
            const hbr_row_split &sp = splits[i];
            ls[i].seg = seg_of(e, sp.seg);
            if (sp.feature >= e.n_cols()) fail(kInvalid, "partition: feature beyond the index");
            ls[i].feature = sp.feature;
            ls[i].limit = sp.below;
            ls[i].default_left = sp.default_left ? 1u : 0u;
            if (sp.table) {
                // RowRule::Table: the local bins that go left
                const uint32_t nb = fo[sp.feature + 1] - fo[sp.feature];
                if (sp.n_table != nb) fail(kInvalid, "partition: a table must hold one entry per bin of its feature");
                if (!e.is_categorical(sp.feature)) fail(kRefused, "partition: a table on a numeric feature");
                ls[i].categorical = true;
                ls[i].limit = 0;
                for (uint32_t b = 0; b < nb; b++)
                    if (sp.table[b]) ls[i].table[b / 32] |= 1u << (b % 32);
            }
        }
        auto kids = e.level(ls, true);
        for (uint64_t i = 0; i < n; i++) {
            out[i].left = seg_out(e, kids[2 * i].seg);
            out[i].right = seg_out(e, kids[2 * i + 1].seg);
        }
    });
}

int hbr_histograms(hbr_engine *h, const hbr_segment *segs, uint64_t n, double *out) {
    return with_engine(h, [&](Engine &e) {
        std::vector<Segment> ss;
        std::vector<uint32_t> slots;
        for (uint64_t i = 0; i < n; i++) {
            ss.push_back(seg_of(e, segs[i]));
            require_exact(e, ss.back().len, "histograms");
        }
        for (uint64_t i = 0; i < n; i++) slots.push_back(e.alloc_slot());
        e.build_nodes(ss, slots);
        for (uint64_t i = 0; i < n; i++) {
            dequant_hist(e, e.read_slot(slots[i]), out + i * 2 * (uint64_t)e.total_bins());
            e.free_slot(slots[i]);
        }
    });
}

int hbr_rows(hbr_engine *h, const hbr_segment *seg, uint32_t *out) {
    return with_engine(h, [&](Engine &e) {
        auto r = e.rows_of(seg_of(e, *seg));
        std::memcpy(out, r.data(), r.size() * 4);
    });
}

int hbr_load_margins(hbr_engine *h, const float *m, uint64_t n, uint32_t k) {
    return with_engine(h, [&](Engine &e) { e.load_margins(m, n, k ? k : 1); });
}

int hbr_gradients(hbr_engine *h, const hbr_device_loss *loss, const float *labels, const float *weights,
                  uint64_t n, int *all_finite) {
    return with_engine(h, [&](Engine &e) {
        if (!loss || !labels) fail(kInvalid, "gradients: null argument");
        if (!e.labels_loaded()) e.set_labels(labels, weights, n);
        bool ok;
        if (loss->kind == HBR_LOSS_SOFTMAX) {
            e.softmax_gradients_async(loss->min_hess);
            ok = e.softmax_all_finite();
        } else {
            ok = e.compute_gradients(*loss, 0);
        }
        if (all_finite) *all_finite = ok ? 1 : 0;
    });
}

int hbr_read_gradients(hbr_engine *h, float *out, uint64_t n) {
    return with_engine(h, [&](Engine &e) {
        if (!out) fail(kInvalid, "read_gradients: null output");
        e.read_gradients(out, n);
    });
}

int hbr_add_leaf_values(hbr_engine *h, const hbr_segment *segs, const float *values, uint64_t n) {
    return with_engine(h, [&](Engine &e) {
        std::vector<Segment> ss;
        for (uint64_t i = 0; i < n; i++) ss.push_back(seg_of(e, segs[i]));
        e.add_leaves(ss, std::vector<float>(values, values + n), 0);
    });
}

int hbr_read_margins(hbr_engine *h, float *out, uint64_t n) {
    return with_engine(h, [&](Engine &e) { e.read_margins(out, n); });
}

int hbr_engine_add_eval(hbr_engine *h, const float *x, uint64_t n_rows, uint64_t n_cols, float missing,
                        const float *init_margins, uint32_t n_outputs, uint32_t *index) {
    return with_engine(h, [&](Engine &e) {
        if (!x || !init_margins || !index) fail(kInvalid, "evaluation set: null argument");
        *index = e.add_eval_set(x, n_rows, n_cols, missing, init_margins, n_outputs);
    });
}

// The eval walk of a caller's tree (numeric, or with categorical nodes and
// their pool of codes).
static void eval_add_tree(Engine &e, const uint32_t *split_feature, const float *split_cond,
                          const uint8_t *default_left, const int32_t *left, const int32_t *right,
                          const float *leaf_value, uint64_t n_nodes, uint32_t output, const uint8_t *is_categorical,
                          const uint32_t *cat_begin, const uint32_t *cat_end, const uint32_t *categories,
                          uint64_t n_categories) {
    if (!split_feature || !split_cond || !default_left || !left || !right || !leaf_value)
        fail(kInvalid, "evaluation walk: null argument");
    if (n_nodes == 0) fail(kInvalid, "evaluation walk: a tree without nodes");
    std::vector<GrowTreeNode> nodes(n_nodes);
    std::vector<float> cond(n_nodes, 0.0f);
    std::unique_ptr<Engine::EvalCats> cats;
    std::vector<uint32_t> pool;
    if (is_categorical) {
        if (!cat_begin || !cat_end || (n_categories && !categories))
            fail(kInvalid, "evaluation walk: categorical nodes need cat_begin, cat_end and categories");
        cats = std::make_unique<Engine::EvalCats>();
        cats->span.assign(2 * n_nodes, 0u);
        pool.assign(categories, categories + n_categories);
        cats->categories = &pool;
    }
    for (uint64_t i = 0; i < n_nodes; i++) {
        GrowTreeNode &g = nodes[i];
        g = GrowTreeNode{};
        g.left = left[i] < 0 ? -1 : left[i];
        g.value = leaf_value[i];
        if (left[i] < 0) continue;
        if ((uint64_t)left[i] + 1 >= n_nodes || right[i] != left[i] + 1)
            fail(kInvalid, "evaluation walk: children must be a pair of existing nodes (right = left + 1)");
        if (split_feature[i] >= e.n_cols()) fail(kInvalid, "evaluation walk: split feature out of range");
        g.feature = split_feature[i];
        g.default_left = default_left[i] ? 1u : 0u;
        cond[i] = split_cond[i];
        if (cats && is_categorical[i]) {
            if (cat_begin[i] > cat_end[i] || cat_end[i] > n_categories || cat_end[i] >= (1u << 31))
                fail(kInvalid, "evaluation walk: a categorical split's categories are out of range");
            cats->span[2 * i] = cat_begin[i];
            cats->span[2 * i + 1] = cat_end[i] | (1u << 31);
        }
    }
    e.walk_evals(nodes, output, &cond, cats.get());
}

int hbr_engine_eval_add_tree(hbr_engine *h, const uint32_t *split_feature, const float *split_cond,
                             const uint8_t *default_left, const int32_t *left, const int32_t *right,
                             const float *leaf_value, uint64_t n_nodes, uint32_t output) {
    return with_engine(h, [&](Engine &e) {
        eval_add_tree(e, split_feature, split_cond, default_left, left, right, leaf_value, n_nodes, output, nullptr,
                      nullptr, nullptr, nullptr, 0);
    });
}

int hbr_engine_eval_add_tree_categorical(hbr_engine *h, const uint32_t *split_feature, const float *split_cond,
                                         const uint8_t *default_left, const int32_t *left, const int32_t *right,
                                         const float *leaf_value, const uint8_t *is_categorical,
                                         const uint32_t *cat_begin, const uint32_t *cat_end,
                                         const uint32_t *categories, uint64_t n_categories, uint64_t n_nodes,
                                         uint32_t output) {
    return with_engine(h, [&](Engine &e) {
        if (!is_categorical) fail(kInvalid, "evaluation walk: null argument");
        eval_add_tree(e, split_feature, split_cond, default_left, left, right, leaf_value, n_nodes, output,
                      is_categorical, cat_begin, cat_end, categories, n_categories);
    });
}

int hbr_engine_eval_margins(hbr_engine *h, uint32_t index, float *out) {
    return with_engine(h, [&](Engine &e) {
        if (!out) fail(kInvalid, "evaluation set: null argument");
        e.read_eval_margins(index, out);
    });
}

int hbr_reserve_hists(hbr_engine *h, uint64_t slots, int *fits) {
    return with_engine(h, [&](Engine &e) { *fits = e.reserve_slots(slots) ? 1 : 0; });
}

int hbr_build_resident(hbr_engine *h, const hbr_segment *segs, const uint32_t *slots, uint64_t n,
                       const uint32_t *sib_parent, const uint32_t *sib_built, uint64_t n_sib) {
    return with_engine(h, [&](Engine &e) {
        std::vector<Segment> ss;
        for (uint64_t i = 0; i < n; i++) ss.push_back(seg_of(e, segs[i]));
        const std::vector<uint32_t> built(slots, slots + n);
        const std::vector<uint32_t> parents(sib_parent, sib_parent + n_sib), sib(sib_built, sib_built + n_sib);
        e.build_nodes(ss, built);
        e.subtract(parents, sib);
        e.note_built(ss, built);
        e.note_siblings(parents, sib);
        // nothing comes back: the histograms stay resident for the next
        // call on the same stream, which waits for them (a device error
        // surfaces at the next synchronising call)
    });
}

int hbr_scan_resident(hbr_engine *h, const hbr_reg_params *reg, const hbr_scan_request *req, uint64_t n,
                      hbr_node_scan *out) {
    return with_engine(h, [&](Engine &e) {
        if (!reg || (!req && n)) fail(kInvalid, "scan: null argument");
        require_exact(e, e.n_rows(), "scan_resident");
        std::vector<int8_t> dirs;
        if (n && req[0].directions) {
            dirs.assign(e.n_cols(), 0);
            for (uint32_t i = 0; i < req[0].n_features; i++)
                if (req[0].features[i] < e.n_cols()) dirs[req[0].features[i]] = req[0].directions[i];
        }
        e.set_scan_params(ScanParams{reg->lambda, reg->alpha, reg->max_delta_step, reg->min_child_weight}, dirs);
        // fixed-point sums beyond the exact domain: the guard certifies each winner
        e.guard_active = e.guard_on() && !e.sums_exact(e.n_rows());
        std::vector<ScanInput> in(n);
        for (uint64_t i = 0; i < n; i++) {
            if (req[i].n_features != e.n_cols()) fail(kRefused, "scan: a feature subset (column sampling)");
            QBin t;
            if (req[i].has_fixed) {
                t = QBin{req[i].fixed_g, req[i].fixed_h};
            } else {
                t = QBin{(int64_t)std::llrint(std::ldexp(req[i].total_g, -e.scale().exp_g)),
                         (int64_t)std::llrint(std::ldexp(req[i].total_h, -e.scale().exp_h))};
            }
            in[i] = ScanInput{req[i].slot, t, req[i].root_gain, req[i].lower, req[i].upper};
        }
        std::vector<uint32_t> sets;
        auto best = e.scan(in, &sets);
        const auto &fo = e.feature_offset();
        const float *cuts = e.cut_values().data();
        const int eg = e.scale().exp_g, eh = e.scale().exp_h;
        h->scan_categories.clear();
        for (uint64_t i = 0; i < n; i++) {
            hbr_node_scan o{};
            const ScanBest &b = best[i];
            if ((b.flags & kScanNearTie) && !(b.flags & kScanReplay) && e.guard_mode == Engine::kGuardResolve) {
                // resolved on the device: the node searched on the CPU builder's sums
                e.counters.near_ties++;
                ExactBest x;
                if (e.resolve_exact(in[i].slot, req[i].total_g, req[i].total_h, in[i].total, in[i].lower,
                                    in[i].upper, &x) &&
                    !(x.flags & kScanNumericNaN)) {
                    e.counters.near_ties_resolved++;
                    if (x.index == 0xffffffffu) {
                        o.kind = HBR_SCAN_EMPTY;
                        out[i] = o;
                        continue;
                    }
                    const uint32_t nb = fo[x.feature + 1] - fo[x.feature];
                    o.kind = HBR_SCAN_NUMERIC;
                    o.feature = x.feature;
                    o.loss_chg = x.loss;
                    o.loss_err = 0.0f;
                    o.left_g = x.lg;
                    o.left_h = x.lh;
                    o.right_g = x.rg;
                    o.right_h = x.rh;
                    o.fixed_left_g = x.left.g;
                    o.fixed_left_h = x.left.h;
                    o.fixed_right_g = x.right.g;
                    o.fixed_right_h = x.right.h;
                    o.backward = x.index >= nb ? 1u : 0u;
                    o.offset = o.backward ? nb - 1 - (x.index - nb) : x.index;
                    o.acc_g = o.backward ? o.right_g : o.left_g;
                    o.acc_h = o.backward ? o.right_h : o.left_h;
                    out[i] = o;
                    continue;
                }
                o.kind = HBR_SCAN_REPLAY;
                o.fallback = HBR_FALLBACK_NEAR_TIE;
                out[i] = o;
                continue;
            }
            if (b.flags & (kScanReplay | kScanNearTie)) {
                // a NaN score, a categorical order that is not total, or a
                // winner the fixed-point sums cannot certify: the host
                // replays the node from its histogram (NodeScan::Replay),
                // which hbr_read_hist gives in the reference's own order
                o.kind = HBR_SCAN_REPLAY;
                o.fallback = (b.flags & kScanCatOrder)     ? HBR_FALLBACK_CATEGORICAL_ORDER
                             : (b.flags & kScanCatNaN)     ? HBR_FALLBACK_CATEGORICAL_SCORE
                             : (b.flags & kScanNumericNaN) ? HBR_FALLBACK_NUMERIC_SCORE
                                                           : HBR_FALLBACK_NEAR_TIE;
                if (b.flags & kScanNearTie) e.counters.near_ties++;
                out[i] = o;
                continue;
            }
            if (b.index == 0xffffffffu) {
                o.kind = HBR_SCAN_EMPTY;
                out[i] = o;
                continue;
            }
            o.feature = b.feature;
            o.loss_chg = b.loss;
            o.loss_err = b.err;
            o.left_g = std::ldexp((double)b.left.g, eg);
            o.left_h = std::ldexp((double)b.left.h, eh);
            o.right_g = std::ldexp((double)b.right.g, eg);
            o.right_h = std::ldexp((double)b.right.h, eh);
            o.fixed_left_g = b.left.g;
            o.fixed_left_h = b.left.h;
            o.fixed_right_g = b.right.g;
            o.fixed_right_h = b.right.h;
            const uint32_t nb = fo[b.feature + 1] - fo[b.feature];
            if (b.flags & kScanCategorical) {
                // the set's category codes, ascending (BestSplit's sorted set)
                o.kind = HBR_SCAN_CATEGORICAL;
                o.default_left = b.flags & 1u;
                const uint32_t *set = sets.data() + i * kCatWords;
                std::vector<uint32_t> codes;
                for (uint32_t k = 0; k < nb; k++)
                    if (set[k / 32] >> (k % 32) & 1u) codes.push_back(category_code(cuts[fo[b.feature] + k]));
                std::sort(codes.begin(), codes.end());
                o.cat_begin = (uint32_t)h->scan_categories.size();
                h->scan_categories.insert(h->scan_categories.end(), codes.begin(), codes.end());
                o.cat_end = (uint32_t)h->scan_categories.size();
                out[i] = o;
                continue;
            }
            o.kind = HBR_SCAN_NUMERIC;
            o.backward = b.index >= nb ? 1u : 0u;
            o.offset = o.backward ? nb - 1 - (b.index - nb) : b.index;
            o.acc_g = o.backward ? o.right_g : o.left_g;
            o.acc_h = o.backward ? o.right_h : o.left_h;
            out[i] = o;
        }
    });
}

int hbr_scan_categories(hbr_engine *h, uint32_t *out, uint64_t n) {
    return with_engine(h, [&](Engine &) {
        if (n != h->scan_categories.size()) fail(kInvalid, "scan categories: n must equal the pool's length");
        if (n) std::memcpy(out, h->scan_categories.data(), n * sizeof(uint32_t));
    });
}

int hbr_read_hist(hbr_engine *h, uint32_t slot, double *out) {
    return with_engine(h, [&](Engine &e) {
        if (!out) fail(kInvalid, "read_hist: null output");
        if (slot >= e.slot_capacity()) fail(kInvalid, "read_hist: no such slot");
        // in the exact domain the fixed-point bins are the CPU's f64 sums;
        // beyond it, the slot's rows summed on the device in the CPU's order
        if (e.sums_exact(e.n_rows())) {
            dequant_hist(e, e.read_slot(slot), out);
            return;
        }
        if (e.exact_hist(slot, out)) return;
        require_exact(e, e.n_rows(), "read_hist");
        dequant_hist(e, e.read_slot(slot), out);
    });
}

int hbr_node_gain(const hbr_reg_params *reg, double g, double h, double lower, double upper, float *out) {
    return guard([&] {
        if (!reg || !out) fail(kInvalid, "node_gain: null argument");
        const Reg r = reg_from(reg->lambda, reg->alpha, reg->max_delta_step, reg->min_child_weight);
        *out = xgb_node_gain(g, h, r, lower, upper);
    });
}

int hbr_leaf_weight(const hbr_reg_params *reg, double g, double h, double lower, double upper, float *out) {
    return guard([&] {
        if (!reg || !out) fail(kInvalid, "leaf_weight: null argument");
        const Reg r = reg_from(reg->lambda, reg->alpha, reg->max_delta_step, reg->min_child_weight);
        *out = (float)calc_weight_bounded(g, h, r, lower, upper);
    });
}

int hbr_engine_set_guard(hbr_engine *h, int mode, double gamma) {
    return with_engine(h, [&](Engine &e) {
        if (!(gamma >= 0.0)) fail(kInvalid, "set_guard: gamma must be a non-negative number");
        if (mode != HBR_GUARD_OFF && mode != HBR_GUARD_REPLAY && mode != HBR_GUARD_RESOLVE)
            fail(kInvalid, "set_guard: unknown mode");
        e.guard_mode = mode;
        e.guard_gamma = (float)gamma;
    }, true);
}

int hbr_engine_set_sums(hbr_engine *h, int mode) {
    return with_engine(h, [&](Engine &e) {
        if (mode != HBR_SUMS_EXACT && mode != HBR_SUMS_FIXED_POINT) fail(kInvalid, "set_sums: unknown mode");
        e.exact_sums_only = mode == HBR_SUMS_EXACT;
    }, true);
}

int hbr_engine_counters_read(hbr_engine *h, hbr_engine_counters *out) {
    return with_engine(h, [&](Engine &e) {
        if (!out) fail(kInvalid, "counters: null output");
        *out = e.counters;
    }, true);
}

int hbr_set_profiling(hbr_engine *h, int on, const char *prefix) {
    return with_engine(
        h, [&](Engine &e) { e.dev().set_profiling(on > 0 ? (uint32_t)on : 0u, prefix ? prefix : ""); }, true);
}

int hbr_kernel_stats(hbr_engine *h, char *buf, size_t len) {
    return with_engine(h, [&](Engine &e) { copy_string(stats_string(e.dev()), buf, len); }, true);
}

// ---- training ------------------------------------------------------------------------

int hbr_trainer_create(hbr_engine *h, const hbr_train_params *p, const float *labels, const float *weights,
                       uint64_t n, hbr_trainer **out) {
    return with_engine(h, [&](Engine &e) {
        if (!p || !labels || !out) fail(kInvalid, "trainer: null argument");
        TrainParams tp;
        tp.grow.reg = reg_from(p->lambda, p->alpha, p->max_delta_step, p->min_child_weight);
        tp.grow.gamma = p->gamma;
        tp.grow.max_depth = p->max_depth > 0 ? (uint64_t)p->max_depth : UINT64_MAX;
        tp.grow.max_leaves = p->max_leaves > 0 ? (uint64_t)p->max_leaves : UINT64_MAX;
        tp.grow.policy = p->grow_policy;
        tp.grow.eta = (float)p->eta;
        if (p->monotone) tp.grow.monotone.assign(p->monotone, p->monotone + p->n_monotone);
        tp.objective = p->objective;
        tp.num_class = p->num_class > 0 ? (uint32_t)p->num_class : 0;
        tp.scale_pos_weight = p->scale_pos_weight;
        tp.has_base_score = p->has_base_score != 0;
        tp.base_score = p->base_score;
        if (tp.objective < 0 || tp.objective > 3) fail(kInvalid, "trainer: unknown objective");
        auto *t = new hbr_trainer{h, nullptr};
        try {
            t->t = std::make_unique<Trainer>(e, tp, labels, weights, n);
        } catch (...) {
            delete t;
            throw;
        }
        *out = t;
    });
}

int hbr_trainer_boost(hbr_trainer *t, uint64_t rounds) {
    if (!t) return set_error(HBR_INVALID, "null trainer");
    return with_engine(t->engine, [&](Engine &) { t->t->boost(rounds); }, true);
}

int hbr_trainer_num_trees(hbr_trainer *t, uint64_t *n) {
    if (!t) return set_error(HBR_INVALID, "null trainer");
    return guard([&] { *n = t->t->trees().size(); });
}

int hbr_trainer_num_outputs(hbr_trainer *t, uint32_t *k) {
    if (!t) return set_error(HBR_INVALID, "null trainer");
    return guard([&] { *k = t->t->outputs(); });
}

int hbr_trainer_base_score(hbr_trainer *t, float *out) {
    if (!t) return set_error(HBR_INVALID, "null trainer");
    return guard([&] {
        const auto &b = t->t->base_score();
        std::memcpy(out, b.data(), b.size() * 4);
    });
}

int hbr_trainer_tree_size(hbr_trainer *t, uint64_t tree, uint64_t *n_nodes) {
    if (!t) return set_error(HBR_INVALID, "null trainer");
    return guard([&] {
        if (tree >= t->t->trees().size()) fail(kInvalid, "no such tree");
        *n_nodes = t->t->trees()[tree].nodes.size();
    });
}

int hbr_trainer_tree(hbr_trainer *t, uint64_t tree, uint32_t *split_feature, float *split_cond, uint8_t *default_left,
                     int32_t *left, int32_t *right, float *leaf_value, float *sum_hess, float *split_gain,
                     int64_t *split_bin) {
    if (!t) return set_error(HBR_INVALID, "null trainer");
    return guard([&] {
        if (tree >= t->t->trees().size()) fail(kInvalid, "no such tree");
        const auto &nodes = t->t->trees()[tree].nodes;
        for (size_t i = 0; i < nodes.size(); i++) {
            const TreeNode &n = nodes[i];
            if (split_feature) split_feature[i] = n.split_feature;
            if (split_cond) split_cond[i] = n.split_cond;
            if (default_left) default_left[i] = n.default_left;
            if (left) left[i] = n.left;
            if (right) right[i] = n.right;
            if (leaf_value) leaf_value[i] = n.leaf_value;
            if (sum_hess) sum_hess[i] = n.sum_hess;
            if (split_gain) split_gain[i] = n.split_gain;
            if (split_bin) split_bin[i] = n.split_bin;
        }
    });
}

int hbr_trainer_tree_categories(hbr_trainer *t, uint64_t tree, uint8_t *is_categorical, uint32_t *cat_begin,
                                uint32_t *cat_end, uint32_t *categories, uint64_t *n_categories) {
    if (!t) return set_error(HBR_INVALID, "null trainer");
    return guard([&] {
        if (tree >= t->t->trees().size()) fail(kInvalid, "no such tree");
        const Tree &tr = t->t->trees()[tree];
        for (size_t i = 0; i < tr.nodes.size(); i++) {
            if (is_categorical) is_categorical[i] = tr.nodes[i].is_categorical;
            if (cat_begin) cat_begin[i] = tr.nodes[i].cat_begin;
            if (cat_end) cat_end[i] = tr.nodes[i].cat_end;
        }
        if (categories) std::memcpy(categories, tr.categories.data(), tr.categories.size() * sizeof(uint32_t));
        if (n_categories) *n_categories = tr.categories.size();
    });
}

int hbr_trainer_margins(hbr_trainer *t, float *out) {
    if (!t) return set_error(HBR_INVALID, "null trainer");
    return with_engine(t->engine, [&](Engine &) { t->t->margins(out); }, true);
}

int hbr_trainer_add_eval(hbr_trainer *t, const float *x, uint64_t n_rows, uint64_t n_cols, float missing,
                         const float *base_margin, uint32_t *index) {
    if (!t || !x || !index) return set_error(HBR_INVALID, "trainer: null argument");
    return with_engine(t->engine,
                       [&](Engine &) { *index = t->t->add_eval(x, n_rows, n_cols, missing, base_margin); }, true);
}

int hbr_trainer_eval_margins(hbr_trainer *t, uint32_t index, float *out) {
    if (!t || !out) return set_error(HBR_INVALID, "trainer: null argument");
    return with_engine(t->engine, [&](Engine &) { t->t->eval_margins(index, out); }, true);
}

void hbr_trainer_free(hbr_trainer *t) { delete t; }

// ---- prediction -------------------------------------------------------------------------

int hbr_forest_upload(int ordinal, const hbr_forest_desc *fd, hbr_forest **out) {
    return guard([&] {
        if (!fd || !out) fail(kInvalid, "forest: null argument");
        auto *f = new hbr_forest;
        try {
            f->f = std::make_unique<Forest>(ordinal, *fd);
        } catch (...) {
            delete f;
            throw;
        }
        *out = f;
    });
}

void hbr_forest_free(hbr_forest *f) { delete f; }

int hbr_predict_margin_device(hbr_forest *h, const float *x, uint64_t n, uint64_t n_cols, float missing, float *out,
                              int32_t *leaf_out) {
    return with_forest(h, [&](Forest &f) {
        f.predict_device(x, n, n_cols, missing, out, leaf_out);
        f.dev().sync();  // the outputs are complete when the call returns
    });
}

int hbr_predict_margin(hbr_forest *h, const float *x, uint64_t n, uint64_t n_cols, float missing, float *out) {
    return hbr_predict_margin_from(h, x, n, n_cols, missing, nullptr, out);
}

int hbr_predict_margin_from(hbr_forest *h, const float *x, uint64_t n, uint64_t n_cols, float missing,
                            const float *init_margins, float *out) {
    return with_forest(h, [&](Forest &f) {
        if (n == 0) return;
        if (!x || !out) fail(kInvalid, "predict: null argument");
        f.predict_host(x, n, n_cols, missing, out, init_margins);
    });
}

int hbr_predict_leaf(hbr_forest *h, const float *x, uint64_t n, uint64_t n_cols, float missing, int32_t *out) {
    return with_forest(h, [&](Forest &f) {
        if (n == 0) return;
        DBuf<float> dx(n * n_cols), dout(n * f.n_outputs());
        DBuf<int32_t> dleaf(std::max<uint64_t>(1, n * f.n_trees()));
        dx.upload(x, n * n_cols, f.dev().stream());
        f.predict_device(dx.get(), n, n_cols, missing, dout.get(), dleaf.get());
        dleaf.download(out, n * f.n_trees(), f.dev().stream());
        f.dev().sync();
    });
}

int hbr_forest_set_profiling(hbr_forest *h, int on, const char *prefix) {
    return with_forest(h, [&](Forest &f) { f.dev().set_profiling(on > 0 ? (uint32_t)on : 0u, prefix ? prefix : ""); });
}

int hbr_forest_kernel_stats(hbr_forest *h, char *buf, size_t len) {
    return with_forest(h, [&](Forest &f) { copy_string(stats_string(f.dev()), buf, len); });
}

int hbr_device_alloc(int ordinal, uint64_t bytes, void **out) {
    return guard([&] {
        device(ordinal);
        HBR_HIP(hipMalloc(out, bytes ? bytes : 1));
    });
}

int hbr_device_free(int ordinal, void *p) {
    return guard([&] {
        device(ordinal);
        HBR_HIP(hipFree(p));
    });
}

int hbr_device_upload(int ordinal, void *dst, const void *src, uint64_t bytes) {
    return guard([&] {
        device(ordinal);
        HBR_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    });
}

int hbr_device_download(int ordinal, void *dst, const void *src, uint64_t bytes) {
    return guard([&] {
        device(ordinal);
        HBR_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    });
}

int hbr_device_copy(int ordinal, void *dst, const void *src, uint64_t bytes) {
    return guard([&] {
        device(ordinal);
        HBR_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToDevice));
    });
}

}  // extern "C"
