"""Pins of the CPU oracle against the reference's own fixtures and known answers.

Every check here compares the oracle with something it does not compute
itself: the reference's saved models and recorded margins, the reference's
own unit-test known answers, brute-force formulations, or closed forms.
"""
import json
import math

import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import (bits_to_f32, categorical_features, four_features, golden_forest, load_saved_models,
                           random_tree, train_labels)


@pytest.fixture(scope="module")
def saved():
    return load_saved_models()


def test_early_stopping_model_reproduced_bit_for_bit(saved):
    """tests/native_format.rs:660-669: `train(base(), matrix(1), 4)` is the saved
    early-stopping model; every field of its four trees must match."""
    x = four_features()
    y = train_labels(x)
    ds = O.Dataset(x, max_bin=256)
    model = O.Model(ds, y, O.params(max_depth=3), 4)
    for ver in ("0.2.0", "0.4.3", "0.4.9"):
        case = saved[f"{ver}/early_stopping"]
        assert np.array_equal(model.base_score().view(np.uint32),
                              np.array(case["base_score"], np.uint32))
        trees = model.trees()
        assert len(trees) == len(case["trees"])
        for t, (mine, ref) in enumerate(zip(trees, case["trees"])):
            assert len(mine) == len(ref["left"]), f"tree {t}"
            for key in ("split_feature", "default_left", "left", "right"):
                got = [int(n[key]) for n in mine]
                assert got == [int(v) for v in ref[key]], f"tree {t} {key}"
            for key in ("split_cond", "leaf_value", "sum_hess", "split_gain"):
                got = np.array([n[key] for n in mine], np.float32).view(np.uint32)
                want = np.array(ref[key], np.uint32)
                leaf = np.array([n["left"] for n in mine]) == -1
                if key == "split_cond":
                    got, want = got[~leaf], want[~leaf]
                if key == "split_gain":
                    got, want = got[~leaf], want[~leaf]
                assert np.array_equal(got, want), f"tree {t} {key}"


@pytest.mark.parametrize("name", ["early_stopping", "dart", "multiclass_forest", "quantiles",
                                  "expectiles", "aft", "dist_normal", "dist_negbinomial",
                                  "multi_target", "categorical_splits"])
def test_saved_model_margins_bit_exact(saved, name):
    """tests/native_format.rs:822-860: each saved model reproduces its recorded
    little-endian f32 margins on the closed-form rows."""
    x = categorical_features() if name == "categorical_splits" else four_features()
    for ver in ("0.2.0", "0.4.3", "0.4.9"):
        case = saved[f"{ver}/{name}"]
        forest = golden_forest(case)
        out = O.predict_margin(forest, x)
        want = np.array(case["margins"], np.uint32)
        assert np.array_equal(out.view(np.uint32), want), f"{ver}/{name}"


@pytest.mark.parametrize("name", ["early_stopping", "dart", "multiclass_forest", "quantiles", "expectiles", "aft",
                                  "dist_normal", "dist_negbinomial"])
def test_lockstep_walk_reproduces_saved_margins(saved, name):
    """The reference's 16-row lock-step compact walk (compact/mod.rs:963-1095)
    restated for the CPU baseline gives each saved numeric model's recorded
    margins; 160 rows are ten full lane groups, 13 leave a tail only."""
    x = four_features()
    for ver in ("0.2.0", "0.4.3", "0.4.9"):
        case = saved[f"{ver}/{name}"]
        want = np.array(case["margins"], np.uint32).reshape(len(x), -1)
        forest = golden_forest(case)
        for rows in (slice(None), slice(0, 13), slice(5, 160)):
            out = O.predict_margin_lockstep(forest, x[rows])
            assert np.array_equal(out.view(np.uint32), want[rows].reshape(-1)), f"{ver}/{name} {rows}"


@pytest.mark.parametrize("seed", range(6))
def test_lockstep_walk_equals_the_scalar_walk(seed):
    """Unbalanced forests (depth 0 to 20: deeper than 16 takes the early-exit
    walk), several outputs and tree weights, NaN cells, signed zeros and
    values equal to a threshold, row counts around the 16-row lanes and the
    256-row blocks, widths beyond 64 features."""
    rng = np.random.default_rng(900 + seed)
    f = int(rng.choice([1, 7, 100]))
    n_trees = int(rng.integers(1, 40))
    k = int(rng.choice([1, 3]))
    trees = [random_tree(rng, f, int(rng.integers(0, 21 if seed == 5 else 12))) for _ in range(n_trees)]
    arrs = O.forest_arrays(trees)
    arrs["tree_output"] = (np.arange(n_trees) % k).astype(np.uint32)
    arrs["tree_weight"] = rng.uniform(0.5, 1.5, n_trees).astype(np.float32)
    arrs["n_outputs"] = k
    arrs["base_score"] = rng.normal(0, 1, k).astype(np.float32)
    conds = arrs["split_cond"][arrs["left"] != -1]
    conds[: len(conds) // 3] = 0.0
    arrs["split_cond"][np.nonzero(arrs["left"] != -1)[0]] = conds
    O.set_threads(3)
    for n in (0, 1, 15, 16, 17, 255, 256, 257, 1_000):
        x = rng.standard_normal((n, f)).astype(np.float32)
        x[rng.random((n, f)) < 0.1] = np.nan
        x[rng.random((n, f)) < 0.05] = -0.0
        x[rng.random((n, f)) < 0.05] = 0.0
        if n and len(conds):
            hit = rng.random((n, f)) < 0.1
            x[hit] = rng.choice(conds, int(hit.sum()))
        want = O.predict_margin(arrs, x)
        got = O.predict_margin_lockstep(arrs, x)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (seed, n)
    O.set_threads(0)


def test_lockstep_walk_refuses_what_it_does_not_take(saved):
    with pytest.raises(ValueError):
        O.predict_margin_lockstep(golden_forest(saved["0.4.9/categorical_splits"]), categorical_features())
    with pytest.raises(ValueError):
        O.predict_margin_lockstep(golden_forest(saved["0.4.9/multiclass_forest"]), four_features()[:, :3])


def test_categorical_casts_saturate_and_missing_follows_default():
    """src/backend/cuda/predict.rs:702-724: the set {0, 2, u32::MAX} on one
    feature, rows -2.5, -0.0, 0.8, 1.9, 2.9, 2^32 and NaN; Rust's saturating
    `as u32` puts the first three in category 0, 1.9 in 1, 2.9 in 2 and 2^32
    in u32::MAX; NaN is missing."""
    x = np.array([[-2.5], [-0.0], [0.8], [1.9], [2.9], [4294967296.0], [np.nan]], np.float32)
    for dl in (0, 1):
        arrs = O.forest_arrays([[dict(split_feature=0, split_cond=0.0, default_left=bool(dl), left=1, right=2,
                                      leaf_value=1.0),
                                 dict(split_feature=0, split_cond=0.0, default_left=True, left=-1, right=-1,
                                      leaf_value=0.25),
                                 dict(split_feature=0, split_cond=0.0, default_left=True, left=-1, right=-1,
                                      leaf_value=-0.75)]])
        arrs.update(is_categorical=np.array([1, 0, 0], np.uint8), cat_begin=np.array([0, 0, 0], np.uint32),
                    cat_end=np.array([3, 0, 0], np.uint32), categories=np.array([0, 2, 2**32 - 1], np.uint32))
        got = O.predict_margin(arrs, x)
        want = np.array([0.25, 0.25, 0.25, -0.75, 0.25, 0.25, 0.25 if dl else -0.75], np.float32)
        np.testing.assert_array_equal(got, want)


def test_splits_on_separating_feature():
    """builder/hist/mod.rs:1065-1082: four rows, one separating feature."""
    x = np.array([[0.0], [0.0], [1.0], [1.0]], np.float32)
    ds = O.Dataset(x)
    gp = np.array([[1, 1], [1, 1], [-1, 1], [-1, 1]], np.float32)
    p = O.params(max_depth=1, reg_lambda=0.0, min_child_weight=0.0, gamma=0.0, eta=1.0)
    nodes, leaf = ds.grow_tree(gp, p)
    assert len(nodes) == 3
    vals = [nodes[leaf[r]]["leaf_value"] for r in range(4)]
    assert abs(vals[0] + 1.0) < 1e-6 and abs(vals[2] - 1.0) < 1e-6


def test_gain_closed_forms():
    """tree/gain.rs:148-196: w = 4/3 and gain 16/3 at G=-4, H=2, lambda=1;
    L1 shrinks, max_delta_step clamps 100 to 1, min_child_weight zeroes."""
    L = O.lib()
    p = O.params(reg_lambda=1.0, min_child_weight=0.0)
    assert abs(L.or_calc_weight(-4.0, 2.0, p) - 4.0 / 3.0) < 1e-12
    # root_gain at the f32-rounded weight: -(2Gw + (H+l) w^2) = 16/3 to f32 precision
    assert abs(L.or_node_gain(-4.0, 2.0, -math.inf, math.inf, p) - 16.0 / 3.0) < 1e-5
    p1 = O.params(reg_lambda=1.0, alpha=1.0, min_child_weight=0.0)
    assert L.or_node_gain(-4.0, 2.0, -math.inf, math.inf, p1) < L.or_node_gain(-4.0, 2.0, -math.inf, math.inf, p)
    assert abs(L.or_calc_weight(-5.0, 1.0, O.params(reg_lambda=0.0, alpha=2.0, min_child_weight=0.0)) - 3.0) < 1e-12
    pm = O.params(reg_lambda=0.0, max_delta_step=1.0, min_child_weight=0.0)
    assert L.or_calc_weight(-100.0, 1.0, pm) == 1.0
    pc = O.params(reg_lambda=1.0, min_child_weight=1.0)
    assert L.or_calc_weight(-4.0, 0.5, pc) == 0.0


def _sparse_one_feature(values):
    """A CSR index of n rows holding only feature 0 of 3 (hist/mod.rs:776-786)."""
    n = len(values)
    return O.Dataset(csr=(np.arange(n + 1), np.zeros(n, np.uint32), np.asarray(values, np.float32)),
                     n_cols=3)


@pytest.mark.parametrize("threads", [1, 4])
def test_blocked_sum_does_not_depend_on_threads(threads):
    """tree/hist/mod.rs:937-958: 8,192 rows in one bin with g = 2^54, -2^54, 1
    at rows 0, 4096, 4097: the two blocks sum to 0, never the chain's 1."""
    n = 8192
    ds = _sparse_one_feature(np.ones(n))
    assert not ds.dense and ds.columns() is None
    gp = np.zeros((n, 2), np.float32)
    gp[:, 1] = 1.0
    gp[0, 0] = 2.0 ** 54
    gp[4096, 0] = -(2.0 ** 54)
    gp[4097, 0] = 1.0
    O.set_threads(threads)
    try:
        h = ds.build_hist(np.arange(n), gp)
    finally:
        O.set_threads(8)
    assert h[0, 0] == 0.0 and h[0, 1] == float(n)
    assert np.all(h[1:] == 0.0)


def test_blocked_build_matches_block_order_reference():
    """tree/hist/mod.rs:965-1005: blocks of `grain` rows each chained from zero,
    partials added in block order; the case separates block from chain."""
    n = 6 * 4096 + 123
    x = (np.arange(n) % 7).astype(np.float32)
    ds = _sparse_one_feature(x)
    i = np.arange(n)
    scale = np.float32(2.0) ** ((i * 37 % 61) - 30).astype(np.float32)
    g = ((i * 7919) % 1237).astype(np.float32) / np.float32(331.0) * scale - np.float32(1.0)
    gp = np.stack([g, scale], axis=1).astype(np.float32)
    rows = i[i % 11 != 3].astype(np.uint32)
    grain = -(-len(rows) // (len(rows) // 4096))
    bins = np.array([O.lib().or_index_feature_bin(ds.index, int(r), 0) for r in range(n)])
    total = ds.total_bins
    expect = np.zeros((total, 2))
    for start in range(0, len(rows), grain):
        part = np.zeros((total, 2))
        for r in rows[start:start + grain]:
            part[bins[r], 0] += float(gp[r, 0])
            part[bins[r], 1] += float(gp[r, 1])
        expect += part if start else 0.0
        if not start:
            expect = part.copy()
    chain = np.zeros((total, 2))
    for r in rows:
        chain[bins[r], 0] += float(gp[r, 0])
        chain[bins[r], 1] += float(gp[r, 1])
    assert not np.array_equal(expect, chain)
    got = ds.build_hist(rows, gp)
    assert np.array_equal(got, expect)


def test_sum_order_describes_the_build():
    """tree/hist/mod.rs:877-903 (sum_order known answers)."""
    L = O.lib()
    big = (1 << 18) + 1
    pt = 8192
    assert L.or_sum_order_grain(0, big, pt - 1, 0) == 0
    assert L.or_sum_order_grain(0, big, pt, 1) == -(-pt // 2)
    assert L.or_sum_order_grain(1, big, pt, 1) == 0
    assert L.or_sum_order_grain(1, big, pt, 0) == -(-pt // 2)
    assert L.or_sum_order_grain(1, 1 << 18, pt, 0) == 0
    m = 6 * 4096 + 123
    assert L.or_sum_order_grain(0, big, m, 0) == -(-m // 6)


def test_dense_sweeps_match_row_order_reference():
    """tree/hist/mod.rs:757-773, :775-826: every bin receives its rows in
    ascending order, for the whole range, a subset and an offset range."""
    n, f = 3 * 8192 + 129, 7
    x = (((np.arange(n * f) * 2654435761) % 1009).astype(np.float32) / np.float32(7.0)).reshape(n, f)
    ds = O.Dataset(x, max_bin=64)
    assert ds.dense and ds.columns() is not None
    i = np.arange(n)
    gp = np.stack([((i * 7919) % 1237).astype(np.float32) / np.float32(331.0) - np.float32(1.9),
                   np.float32(0.25) + (i % 5).astype(np.float32)], axis=1).astype(np.float32)
    row_ptr, gbins = ds.row_bins()
    gbins = gbins.reshape(n, f)
    for rows in (i, i[i % 3 != 1], np.arange(1000, 1000 + 8192)):
        ref = np.zeros((ds.total_bins, 2))
        # one row-order chain per bin (np.add.at adds in index order)
        for c in range(f):
            np.add.at(ref[:, 0], gbins[rows, c], gp[rows, 0].astype(np.float64))
            np.add.at(ref[:, 1], gbins[rows, c], gp[rows, 1].astype(np.float64))
        got = ds.build_hist(rows, gp)
        assert np.array_equal(got, ref)


def test_cuts_closed_form_for_few_distinct_values():
    """sketch.rs:914-930, quantile.rs:926-996: with at most max_bin distinct
    values the cuts are every distinct value but the minimum, then the
    sentinel max + (|max| + 1e-5); a constant feature has one bin."""
    rng = np.random.default_rng(0)
    vals = np.round(rng.normal(size=40) * 100).astype(np.float32)
    x = np.stack([rng.choice(vals, size=5000), np.full(5000, 3.0, np.float32)], axis=1)
    ds = O.Dataset(x, max_bin=256)
    off = ds.feature_offset
    cuts = ds.cut_values
    d = np.unique(x[:, 0])
    mx = d[-1]
    want = np.concatenate([d[1:], [np.float32(mx + (abs(mx) + np.float32(1e-5)))]]).astype(np.float32)
    assert np.array_equal(cuts[off[0]:off[1]], want)
    assert off[2] - off[1] == 1
    c3 = np.float32(3.0)
    assert cuts[off[1]] == np.float32(c3 + (abs(c3) + np.float32(1e-5)))


def test_cuts_quantile_properties_on_continuous_data():
    """quantile.rs:926-996 invariants: strictly increasing cuts, at most
    max_bin + 1 per feature, and bins of near-equal mass (rank error within
    the sketch's eps = 1/max_bin)."""
    rng = np.random.default_rng(1)
    n = 200_000
    x = rng.normal(size=(n, 3)).astype(np.float32)
    for max_bin in (16, 256):
        ds = O.Dataset(x, max_bin=max_bin)
        off = ds.feature_offset
        cuts = ds.cut_values
        _, gb = ds.row_bins()
        gb = gb.reshape(n, 3)
        for f in range(3):
            c = cuts[off[f]:off[f + 1]]
            assert len(c) <= max_bin + 1 and np.all(np.diff(c) > 0)
            counts = np.bincount(gb[:, f] - off[f], minlength=len(c))
            assert counts.max() <= n / max_bin * 1.5 + 2


def test_bin_assignment_is_upper_bound_count():
    """quantile.rs:285-296: bin = #{cuts <= v}, clamped to the last bin."""
    rng = np.random.default_rng(2)
    x = rng.normal(size=(3000, 2)).astype(np.float32)
    x[::17, 1] = np.nan
    ds = O.Dataset(x, max_bin=32)
    off = ds.feature_offset
    cuts = ds.cut_values
    fb = ds.feature_bins()
    for f in range(2):
        c = cuts[off[f]:off[f + 1]]
        v = x[:, f]
        present = ~np.isnan(v)
        want = np.minimum(np.searchsorted(c, v[present], side="right"), len(c) - 1) + off[f]
        assert np.array_equal(fb[present, f], want)
        assert np.all(fb[~present, f] == -1)


def test_partition_matches_per_row_routing():
    """builder/partition.rs:325+: stable, each row where its own bin decides,
    missing rows following default_left, on dense columns and on CSR rows."""
    rng = np.random.default_rng(3)
    n = 5000
    x = rng.normal(size=(n, 4)).astype(np.float32)
    x[rng.random((n, 4)) < 0.1] = np.nan
    ds = O.Dataset(x, max_bin=64)
    fb = ds.feature_bins()
    rows = np.sort(rng.choice(n, size=3000, replace=False)).astype(np.uint32)
    off = ds.feature_offset
    for feat in range(4):
        for b in (-1, int(off[feat]) + 5, int(off[feat + 1]) - 1):
            for dl in (0, 1):
                L, R = ds.partition(rows, feat, b, dl)
                v = fb[rows, feat]
                go = np.where(v < 0, bool(dl), (v >= 0) & (v <= b) & (b >= 0))
                assert np.array_equal(L, rows[go]) and np.array_equal(R, rows[~go])


def test_logistic_gradient_vector_and_scalar_paths():
    """simd/x86_64.rs:106-160 vs simd/scalar.rs:8-29: vectors of 8 rows with
    all |m| <= 80 take the polynomial, the tail (n % 8 rows, or every row
    when n < 16) and out-of-range vectors the libm sigmoid; both are within
    a few f32 ulps of the exact logistic."""
    rng = np.random.default_rng(4)
    for n in (7, 15, 16, 23, 1000):
        m = (rng.normal(size=n) * 6).astype(np.float32)
        if n == 1000:
            m[100] = 95.0  # one vector leaves the polynomial's range
        y = (rng.random(n) < 0.5).astype(np.float32)
        g = O.gradient(O.OBJ_LOGISTIC, m, y)
        p = 1.0 / (1.0 + np.exp(-m.astype(np.float64)))
        pf = (g[:, 0] + y).astype(np.float64)
        ulp = np.spacing(p.astype(np.float32)).astype(np.float64)
        assert np.all(np.abs(pf - p) <= 8 * ulp + 1e-7)
        vec = n - n % 8 if n >= 16 else 0
        tail = np.arange(vec, n)
        for r in tail:
            s = O.lib().or_sigmoid(float(m[r]))
            assert np.float32(s - y[r]) == g[r, 0]
        h = g[:, 1]
        assert np.all(h >= np.float32(1e-16))


def test_logistic_dispatch_is_close_to_scalar_as_the_reference_tests_it():
    """The reference's own pin of its vector logistic path
    (simd/tests.rs:53-75, logistic_gradient_dispatch_is_close_to_scalar):
    4,103 sawtooth margins over [-20, 20], labels i % 2, no weights and
    sawtooth weights, scale_pos_weight 1.5, min_hess 1e-16; every pair within
    5e-7 (g) and 3e-7 (h) of the scalar rows (the C library's expf)."""
    n = 4_103
    preds = _sawtooth(n, 4_103, -20.0, 40.0 / 4_102.0)
    labels = (np.arange(n) % 2).astype(np.float32)
    for weights in (None, _sawtooth(n, 13, 0.5, 0.125)):
        g = O.gradient(O.OBJ_LOGISTIC, preds, labels, weights, scale_pos_weight=1.5)
        w = np.ones(n, np.float32) if weights is None else weights
        w = np.where(labels == 1.0, w * np.float32(1.5), w).astype(np.float32)
        p = np.array([O.lib().or_sigmoid(float(m)) for m in preds], np.float32)
        eg = ((p - labels) * w).astype(np.float32)
        eh = (np.maximum(p * (np.float32(1) - p), np.float32(1e-16)) * w).astype(np.float32)
        assert np.all(np.abs(g[:, 0] - eg) <= 5.0e-7)
        assert np.all(np.abs(g[:, 1] - eh) <= 3.0e-7)


def test_softmax_gradient_closed_form():
    """objective/multiclass.rs:124-139: zero margins give p = 1/3, g = p - 1 on
    the label, h = 2p(1-p)."""
    g = O.gradient(O.OBJ_SOFTMAX, np.zeros(6, np.float32), np.array([0, 2], np.float32), num_class=3)
    assert abs(g[0, 0, 0] - (1 / 3 - 1)) < 1e-6 and abs(g[0, 1, 0] - 1 / 3) < 1e-6
    assert abs(g[1, 2, 0] - (1 / 3 - 1)) < 1e-6
    assert abs(g[0, 0, 1] - 2 * (1 / 3) * (2 / 3)) < 1e-6


def test_base_margins():
    """classification.rs:276-339 and multiclass base margins: the logit of the
    positive rate; centered log frequencies for softmax (uniform -> zeros)."""
    p = O.params(objective=O.OBJ_LOGISTIC)
    assert O.base_margins(np.array([1, 0], np.float32), p)[0] == 0.0
    q = O.base_margins(np.array([1, 0, 0, 0], np.float32), p)[0]
    assert abs(q - math.log(0.25 / 0.75)) < 1e-6
    ps = O.params(objective=O.OBJ_SOFTMAX, num_class=3)
    assert np.all(O.base_margins(np.array([0, 1, 2], np.float32), ps) == 0.0)


def _libm():
    import ctypes
    m = ctypes.CDLL("libm.so.6")
    for fn in (m.expf, m.logf):
        fn.restype, fn.argtypes = ctypes.c_float, [ctypes.c_float]
    return m


def _logit_of_sigmoid(step):
    """sigmoid_scalar (simd/mod.rs:425-427) then the logistic link
    (classification.rs:74-77), each in f32 with the host libm the reference
    calls through f32::exp / f32::ln."""
    m = _libm()
    f = np.float32
    p = f(1.0) / (f(m.expf(f(min(-f(step), f(88.7))))) + f(1.0))
    p = min(max(p, f(1e-6)), f(1.0) - f(1e-6))
    return -f(m.logf(f(1.0) / p - f(1.0)))


def test_logitraw_intercept_is_the_label_mean():
    """classification.rs:298-303: binary:logitraw's intercept is the label
    mean itself (the identity link); a given base_score is kept as is."""
    p = O.params(objective=O.OBJ_LOGITRAW)
    assert O.base_margins(np.array([1, 0, 0, 0], np.float32), p)[0] == np.float32(0.25)
    pb = O.params(objective=O.OBJ_LOGITRAW, base_score=-3.5)
    assert O.base_margins(np.array([1, 0], np.float32), pb)[0] == np.float32(-3.5)


def test_newton_intercepts_closed_forms():
    """classification.rs:132-141 and regression.rs:66-74: with
    scale_pos_weight away from 1 the intercept is one Newton step from zero
    margins (objective/mod.rs:528-566). Labels [1, 0] with spw 3 give the
    reference's gradient KAT pairs (classification.rs:262-273: (-1.5, 0.75),
    (0.5, 0.25)), so -G/H = 1.0, then sigmoid and logit; logitraw keeps the
    step; squared error over [1, 0, 2] with spw 2 weighs the 1 twice:
    -G/H = 4/4."""
    y = np.array([1, 0], np.float32)
    lg = O.base_margins(y, O.params(objective=O.OBJ_LOGISTIC, scale_pos_weight=3.0))[0]
    assert lg == _logit_of_sigmoid(1.0)
    assert O.base_margins(y, O.params(objective=O.OBJ_LOGITRAW, scale_pos_weight=3.0))[0] == np.float32(1.0)
    ys = np.array([1, 0, 2], np.float32)
    assert O.base_margins(ys, O.params(objective=O.OBJ_SQUARED_ERROR, scale_pos_weight=2.0))[0] == np.float32(1.0)
    # 25% positives: spw 1.5 -> G = 3 * 0.5 - 0.75 = 0.75, H = 0.75 + 0.375
    y4 = np.array([1, 0, 0, 0], np.float32)
    step = np.float32(-0.75 / 1.125)
    got = O.base_margins(y4, O.params(objective=O.OBJ_LOGISTIC, scale_pos_weight=1.5))[0]
    assert got == _logit_of_sigmoid(step)
    assert abs(got - np.float32(-np.log(3.0))) > 0.1  # not the logit of the positive rate
    # |spw - 1| <= 1e-6 (f32) keeps the label-mean path
    mean_path = O.base_margins(y4, O.params(objective=O.OBJ_LOGISTIC, scale_pos_weight=1.0000005))[0]
    assert mean_path == O.base_margins(y4, O.params(objective=O.OBJ_LOGISTIC))[0]


@pytest.mark.parametrize("spw,weighted", [(0.5, True), (2.0, False), (3.0, True)])
def test_newton_intercept_over_the_vector_gradient_path(spw, weighted):
    """1,001 rows (125 AVX2 vectors and a scalar tail) through the oracle's
    gradient at zero margins equal the per-row closed form at p = 0.5,
    summed as one f64 chain in row order (fit_stump, objective/mod.rs:552-566)."""
    rng = np.random.default_rng(int(spw * 10))
    y = (rng.random(1001) < 0.3).astype(np.float32)
    y[::97] = 0.25  # labels other than 0 and 1 are not reweighted
    w = (rng.random(1001) * 3 + 0.1).astype(np.float32) if weighted else np.ones(1001, np.float32)
    wp = np.where(y == 1.0, w * np.float32(spw), w).astype(np.float32)
    g = np.cumsum(((np.float32(0.5) - y) * wp).astype(np.float32).astype(np.float64))[-1]
    h = np.cumsum((np.float32(0.25) * wp).astype(np.float32).astype(np.float64))[-1]
    step = np.float32(-g / max(h, 1e-6))
    for obj, want in ((O.OBJ_LOGISTIC, _logit_of_sigmoid(step)), (O.OBJ_LOGITRAW, step)):
        got = O.base_margins(y, O.params(objective=obj, scale_pos_weight=spw), weights=w if weighted else None)[0]
        assert got == want, (obj, got, want)
    gs = np.cumsum(((np.float32(0.0) - y) * wp).astype(np.float32).astype(np.float64))[-1]
    hs = np.cumsum(wp.astype(np.float64))[-1]
    sq = O.base_margins(y, O.params(objective=O.OBJ_SQUARED_ERROR, scale_pos_weight=spw),
                        weights=w if weighted else None)[0]
    assert sq == np.float32(-gs / hs)


def _sawtooth(n, period, start, step):
    """start + (i % period) * step in f32 (simd/tests.rs:24-30)."""
    i = (np.arange(n) % period).astype(np.float32)
    return (np.float32(start) + i * np.float32(step)).astype(np.float32)


def _close_pairs(actual, expected):
    """simd/tests.rs:3-16: within 1e-6 of max(|expected|, 1)."""
    tol = 1e-6 * np.maximum(np.abs(expected.astype(np.float64)), 1.0)
    assert np.all(np.abs(actual.astype(np.float64) - expected) <= tol)


def test_softmax_vector_batches_are_taken_and_close_to_scalar_rows():
    """simd/tests.rs:116-161: the whole-matrix gradient (with the 2- and
    4-class vector batches) against every row on the scalar path, across
    batch boundaries; the batches differ from the scalar rows in some
    bits, so they are the path taken."""
    for k in (2, 3, 4, 8, 17, 32, 33, 128, 131):
        rows = 257
        preds = _sawtooth(rows * k, 211, -2.5, 0.025)
        labels = (np.arange(rows) % k).astype(np.float32)
        wv = _sawtooth(rows, 11, 0.5, 0.125)
        for w in (None, wv):
            full = O.gradient(O.OBJ_SOFTMAX, preds, labels, w, num_class=k)
            scal = O.gradient(O.OBJ_SOFTMAX, preds, labels, w, num_class=k, scalar_rows=True)
            _close_pairs(full, scal)
            differs = not np.array_equal(full.view(np.uint32), scal.view(np.uint32))
            assert differs == (k in (2, 4)), k
    for k in (2, 3, 4):
        for rows in list(range(18)) + [127, 256, 257]:
            i = np.arange(rows * k)
            preds = (((i * 71) % 211).astype(np.float32) * np.float32(0.375) - np.float32(39.0)).astype(np.float32)
            labels = (np.arange(rows) % k).astype(np.float32)
            wv = ((np.arange(rows) % 7).astype(np.float32) * np.float32(0.25)).astype(np.float32)
            for w in (None, wv):
                full = O.gradient(O.OBJ_SOFTMAX, preds, labels, w, num_class=k)
                scal = O.gradient(O.OBJ_SOFTMAX, preds, labels, w, num_class=k, scalar_rows=True)
                _close_pairs(full, scal)
                if rows * k < 16 or k == 3:  # no batch: the scalar rows themselves
                    assert np.array_equal(full.view(np.uint32), scal.view(np.uint32))


def test_softmax_exceptional_rows_and_label_casts():
    """simd/tests.rs:163-215: one exceptional margin at every position, with
    labels and weights that exercise the casts: NaN stays NaN, infinities
    equal, the rest within 3e-7 of the scalar rows."""
    labels = np.array([np.nan, -2.0, np.inf, 1.5, np.finfo(np.float32).max, float(2**32 - 1), 2.0, 3.0, -np.inf],
                      np.float32)
    weights = np.array([0.0, 0.25, 1.0, np.nan, np.inf, -1.0, 2.0, 0.5, 1.0], np.float32)
    fmax = np.finfo(np.float32).max
    with np.errstate(invalid="ignore"):
        for k in (2, 3, 4):
            for pos in range(len(labels) * k):
                for exc in (np.nan, np.inf, -np.inf, -81.0, 81.0, -80.0, 80.0, fmax):
                    preds = np.zeros(len(labels) * k, np.float32)
                    preds[pos] = exc
                    for w in (None, weights):
                        full = O.gradient(O.OBJ_SOFTMAX, preds, labels, w, num_class=k).astype(np.float64)
                        scal = O.gradient(O.OBJ_SOFTMAX, preds, labels, w, num_class=k,
                                          scalar_rows=True).astype(np.float64)
                        nan = np.isnan(scal)
                        assert np.array_equal(np.isnan(full), nan)
                        inf = np.isinf(scal)
                        assert np.array_equal(full[inf], scal[inf])
                        ok = ~nan & ~inf
                        assert np.all(np.abs(full[ok] - scal[ok]) <= 3e-7)


def test_softmax_underflowing_rows_are_nan_bit_for_bit():
    """simd/tests.rs:217-285: rows of -200 underflow every exponential under
    the f32::MIN_POSITIVE shift (0/0): the gradient is that NaN, bit for bit
    with the scalar rows; rows of -30 and ordinary rows stay close."""
    for k in (2, 3, 4, 8):
        rows = 24
        preds = np.empty(rows * k, np.float32)
        for r in range(rows):
            for c in range(k):
                preds[r * k + c] = (-200.0, -30.0, ((r * 7 + c * 5) % 11) * np.float32(0.4) - 2.0)[r % 3]
        labels = np.array([(r * 5) % k for r in range(rows)], np.float32)
        wv = np.array([0.5 + (r % 4) * 0.25 for r in range(rows)], np.float32)
        for w in (None, wv):
            with np.errstate(invalid="ignore"):
                full = O.gradient(O.OBJ_SOFTMAX, preds, labels, w, num_class=k)
                scal = O.gradient(O.OBJ_SOFTMAX, preds, labels, w, num_class=k, scalar_rows=True)
            for r in range(rows):
                if r % 3 == 0:
                    assert np.all(np.isnan(scal[r, :, 0]))
                    assert np.array_equal(full[r].view(np.uint32), scal[r].view(np.uint32))
                else:
                    _close_pairs(full[r], scal[r])


# ---- loss-guided growth: expansion order and node numbering ----------------------------

def _canon(nodes, i=0):
    """A tree up to node numbering: splits (feature, threshold bits, default
    direction) and leaf values, recursively."""
    nd = nodes[i]
    if nd["left"] == -1:
        return ("leaf", np.float32(nd["leaf_value"]).view(np.uint32).item())
    return ("split", nd["split_feature"], np.float32(nd["split_cond"]).view(np.uint32).item(),
            bool(nd["default_left"]), _canon(nodes, nd["left"]), _canon(nodes, nd["right"]))


def _lossguide_data(seed, n=3_000, f=5):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, f)).astype(np.float32)
    x[rng.random((n, f)) < 0.05] = np.nan
    z = np.nan_to_num(x)
    y = (1.5 * z[:, 0] - z[:, 1] ** 2 + np.sin(2 * z[:, 2]) + 0.1 * rng.standard_normal(n)).astype(np.float32)
    gp = np.stack([-y, np.ones(n, np.float32)], 1).astype(np.float32)  # squared error at zero margins
    return O.Dataset(x, max_bin=64), gp


@pytest.mark.parametrize("seed,depth", [(0, 3), (1, 4), (2, 5)])
def test_lossguide_with_room_for_every_leaf_is_the_depthwise_tree(seed, depth):
    """With max_leaves >= 2^depth, loss-guided growth expands every
    expandable node (builder/hist/mod.rs:505-573), so it grows the depthwise
    tree (:459-503) up to node numbering; with max_leaves = 2 it grows the
    depth-1 stump."""
    ds, gp = _lossguide_data(seed)
    dw, _ = ds.grow_tree(gp, O.params(max_depth=depth, eta=0.3, max_bin=64))
    lg, _ = ds.grow_tree(gp, O.params(grow_policy=O.GROW_LOSSGUIDE, max_depth=depth, max_leaves=1 << depth,
                                      eta=0.3, max_bin=64))
    assert _canon(lg) == _canon(dw)
    stump, _ = ds.grow_tree(gp, O.params(max_depth=1, eta=0.3, max_bin=64))
    two, _ = ds.grow_tree(gp, O.params(grow_policy=O.GROW_LOSSGUIDE, max_depth=0, max_leaves=2, eta=0.3,
                                       max_bin=64))
    assert _canon(two) == _canon(stump) and len(two) == 3


def _best_first(dw, max_leaves):
    """Brute-force best-first growth over the depthwise tree's own splits:
    the frontier node of largest split gain among those the depthwise tree
    split is expanded next, its children numbered next (left, then right),
    until max_leaves leaves. Returns (new node -> depthwise node, children)."""
    of = [0]
    kids = {}
    frontier = [0]
    leaves = 1
    while leaves < max_leaves:
        cand = [v for v in frontier if dw[of[v]]["left"] != -1]
        if not cand:
            break
        gains = [dw[of[v]]["split_gain"] for v in cand]
        best = int(np.argmax(gains))
        assert gains.count(gains[best]) == 1, "tied gains: the check needs distinct ones"
        v = cand[best]
        frontier.remove(v)
        left = len(of)
        of += [dw[of[v]]["left"], dw[of[v]]["right"]]
        kids[v] = (left, left + 1)
        frontier += [left, left + 1]
        leaves += 1
    return of, kids


@pytest.mark.parametrize("seed,depth,leaves", [(3, 6, 9), (4, 7, 23), (5, 5, 14), (6, 8, 40)])
def test_lossguide_expands_in_gain_order_and_numbers_children_next(seed, depth, leaves):
    """The loss-guided tree equals a brute-force best-first expansion of the
    depthwise tree's splits (a node's best split does not depend on when it
    is expanded): node for node, including the ids, which the reference
    assigns in expansion order (max-heap on loss_chg, hist/mod.rs:132-149)."""
    ds, gp = _lossguide_data(seed)
    dw, _ = ds.grow_tree(gp, O.params(max_depth=depth, eta=0.3, max_bin=64))
    lg, _ = ds.grow_tree(gp, O.params(grow_policy=O.GROW_LOSSGUIDE, max_depth=depth, max_leaves=leaves, eta=0.3,
                                      max_bin=64))
    of, kids = _best_first(dw, leaves)
    assert len(lg) == len(of)
    for v, d in enumerate(of):
        a, b = lg[v], dw[d]
        assert np.float32(a["sum_hess"]) == np.float32(b["sum_hess"]), v
        if v in kids:
            assert (a["left"], a["right"]) == kids[v], v
            assert a["split_feature"] == b["split_feature"] and a["default_left"] == b["default_left"], v
            assert np.float32(a["split_cond"]).view(np.uint32) == np.float32(b["split_cond"]).view(np.uint32), v
            assert np.float32(a["split_gain"]) == np.float32(b["split_gain"]), v
        else:
            assert a["left"] == -1, v
            if b["left"] == -1:
                assert np.float32(a["leaf_value"]) == np.float32(b["leaf_value"]), v


def test_lossguide_respects_max_leaves():
    """builder/hist/mod.rs:1322-1343: 64 rows of alternating gradients on
    one feature, max_leaves 4, unlimited depth, no regularisation."""
    x = np.arange(64, dtype=np.float32).reshape(-1, 1)
    g = np.where(np.arange(64) % 2 == 0, 1.0, -1.0).astype(np.float32)
    gp = np.stack([g, np.ones(64, np.float32)], 1)
    ds = O.Dataset(x, max_bin=256)
    t, _ = ds.grow_tree(gp, O.params(grow_policy=O.GROW_LOSSGUIDE, max_leaves=4, max_depth=0, min_child_weight=0.0,
                                     gamma=0.0, reg_lambda=0.0))
    assert sum(nd["left"] == -1 for nd in t) <= 4


# ---- categorical splits --------------------------------------------------------------------

def test_categorical_splits_model_retrained_bit_for_bit(saved):
    """tests/native_format.rs:508-540: the saved categorical-splits model
    (base(): hist, depth 3, eta 0.3; four_features with column 0 the
    category codes i % 5, categorical; y = [0, 2, -1, 3, 1][i % 5] + x1)
    grown again by the oracle: every tree's structure, category sets, split
    gains, Hessian sums and leaf values bit for bit, in three versions."""
    x = categorical_features()
    y = (np.array([0.0, 2.0, -1.0, 3.0, 1.0], np.float32)[np.arange(len(x)) % 5] + x[:, 1]).astype(np.float32)
    ds = O.Dataset(x, max_bin=256, feature_types=["c", "q", "q", "q"])
    for ver in ("0.2.0", "0.4.3", "0.4.9"):
        case = saved[f"{ver}/categorical_splits"]
        model = O.Model(ds, y, O.params(max_depth=3), len(case["trees"]))
        assert np.array_equal(model.base_score().view(np.uint32), np.array(case["base_score"], np.uint32))
        for t, (mine, ref) in enumerate(zip(model.trees(), case["trees"])):
            assert [n["left"] for n in mine] == ref["left"] and [n["right"] for n in mine] == ref["right"], t
            pool = ref["categories"]
            for i, n in enumerate(mine):
                assert n["is_categorical"] == bool(ref["is_categorical"][i]), (t, i)
                if n["is_categorical"]:
                    assert n["categories"] == pool[ref["cat_begin"][i]:ref["cat_end"][i]], (t, i)
                if n["left"] != -1:
                    assert n["split_feature"] == ref["split_feature"][i], (t, i)
                    assert bool(n["default_left"]) == bool(ref["default_left"][i]), (t, i)
                    assert np.float32(n["split_cond"]).view(np.uint32) == ref["split_cond"][i], (t, i)
                    assert np.float32(n["split_gain"]).view(np.uint32) == ref["split_gain"][i], (t, i)
                assert np.float32(n["leaf_value"]).view(np.uint32) == ref["leaf_value"][i], (t, i)
                assert np.float32(n["sum_hess"]).view(np.uint32) == ref["sum_hess"][i], (t, i)
        assert np.array_equal(model.margins().view(np.uint32), np.array(case["margins"], np.uint32))


def _sweep(cats, total, reg_lambda=0.0):
    """builder/categorical.rs:180-201: sweep_categorical unregularized over
    (G, H) per category, against the node total; the winner's set by bin."""
    p = O.params(reg_lambda=reg_lambda, alpha=0.0, max_delta_step=0.0, min_child_weight=0.0)
    best = O.Split()
    best.loss_chg, best.feature, best.bin, best.default_left = 0.0, 0, -1, 1
    st = np.ascontiguousarray(np.array(cats, np.float64).reshape(-1))
    O.lib().or_sweep_categorical(st.ctypes.data, len(cats), total[0], total[1], -math.inf, math.inf, 0, p, 0, best)
    chosen = [i for i in range(len(cats)) if best.cat_left[i // 32] >> (i % 32) & 1]
    return best, chosen


def test_categorical_sweep_known_answers():
    """builder/categorical.rs:211-263: a lone category splits from the
    missing values (loss 4, missing to the other child); four categories of
    weights -2, -1, 1, 2 with missing gradients -3 and 3 both choose {0, 1},
    missing with the set only when its weight fits them, loss 4.5 + 12 - 1.8."""
    best, chosen = _sweep([(2.0, 2.0)], (0.0, 4.0))
    assert best.categorical and chosen == [0] and not best.default_left
    assert abs(best.loss_chg - 4.0) < 1e-6
    cats = [(2.0, 1.0), (1.0, 1.0), (-1.0, 1.0), (-2.0, 1.0)]
    for missing_grad, with_set in ((-3.0, False), (3.0, True)):
        best, chosen = _sweep(cats, (missing_grad, 5.0))
        assert chosen == [0, 1], missing_grad
        assert bool(best.default_left) == with_set, missing_grad
        assert abs(best.loss_chg - (4.5 + 12.0 - 1.8)) < 1e-5


def test_categorical_sweep_brute_force():
    """Every candidate the reference enumerates, scored in closed form in
    f64 (loss = G_l^2/H_l + G_r^2/H_r - G^2/H, unregularized): the sweep's
    winner is the maximum over one-hot sets (fewer than 4 categories) or
    over prefixes and suffixes of the weight order (4 or more), with missing
    values on either side."""
    rng = np.random.default_rng(21)
    for trial in range(200):
        n = int(rng.integers(1, 9))
        g = rng.normal(0, 1, n).round(2)
        h = rng.uniform(0.5, 2, n).round(2)
        mg, mh = round(float(rng.normal(0, 1)), 2), round(float(rng.uniform(0, 1)), 2)
        total = (float(g.sum() + mg), float(h.sum() + mh))
        best, chosen = _sweep(list(zip(g, h)), total)

        def loss(sg, sh):
            ogh = total[1] - sh
            if sh <= 0 or ogh <= 0:
                return -np.inf
            return sg * sg / sh + (total[0] - sg) ** 2 / ogh - total[0] ** 2 / total[1]
        cands = []
        if n < 4:
            for i in range(n):
                cands += [(loss(g[i], h[i]), [i]), (loss(g[i] + mg, h[i] + mh), [i])]
        else:
            order = sorted(range(n), key=lambda i: -g[i] / h[i])
            for k in range(1, n):
                s = order[:k]
                cands += [(loss(g[s].sum(), h[s].sum()), sorted(s)),
                          (loss(g[s].sum() + mg, h[s].sum() + mh), sorted(s))]
        top = max(c[0] for c in cands)
        if top <= 1e-3:
            continue
        assert best.categorical, trial
        assert abs(best.loss_chg - top) <= 1e-3 * max(1.0, abs(top)), (trial, best.loss_chg, top)
        assert any(abs(c[0] - top) <= 1e-3 * max(1.0, abs(top)) and c[1] == chosen for c in cands), trial


def _mirrored_data(seed, n_half=2_000):
    """Rows in mirrored pairs: feature 0 is 0 or 1, the other features are
    shared, and the second row's gradient is the first's negated, so every
    node under the root's split on feature 0 has a mirror image with the
    same loss change bit for bit (f64 sums of negated values in the same
    order are exact negations; gains square them)."""
    rng = np.random.default_rng(seed)
    base = rng.standard_normal((n_half, 3)).astype(np.float32)
    x = np.zeros((2 * n_half, 4), np.float32)
    x[0::2, 1:] = base
    x[1::2, 1:] = base
    x[1::2, 0] = 1.0
    h = (1.5 + base[:, 0] + np.sin(2.0 * base[:, 1]) * base[:, 2]).astype(np.float32)
    g = np.empty(2 * n_half, np.float32)
    g[0::2], g[1::2] = -h, h
    gp = np.stack([g, np.ones_like(g)], 1)
    return x, gp


class RustBinaryHeap:
    """std::collections::BinaryHeap as the Rust standard library implements
    it (library/alloc/src/collections/binary_heap/mod.rs): push appends and
    sifts up, stopping at a parent the element is <= to; pop swaps the last
    element into the root, sifts the hole down to the bottom through the
    larger child (the right one when the left is <= it), then sifts up.
    Elements are (key, payload) ordered by key alone."""

    def __init__(self):
        self.d = []

    def _sift_up(self, start, pos):
        elem = self.d[pos]
        while pos > start:
            parent = (pos - 1) // 2
            if elem[0] <= self.d[parent][0]:
                break
            self.d[pos] = self.d[parent]
            pos = parent
        self.d[pos] = elem

    def push(self, key, payload):
        self.d.append((key, payload))
        self._sift_up(0, len(self.d) - 1)

    def pop(self):
        item = self.d.pop()
        if self.d:
            item, self.d[0] = self.d[0], item
            end, pos = len(self.d), 0
            elem = self.d[0]
            child = 1
            while child <= max(end - 2, 0) and end >= 2:
                if self.d[child][0] <= self.d[child + 1][0]:
                    child += 1
                self.d[pos] = self.d[child]
                pos, child = child, 2 * child + 1
            if child == end - 1:
                self.d[pos] = self.d[child]
                pos = child
            self.d[pos] = elem
            self._sift_up(0, pos)
        return item


def _total_key(x):
    """f64::total_cmp as an integer key."""
    b = int(np.array([x], np.float64).view(np.int64)[0])
    return b ^ ((b >> 63) & 0x7FFFFFFFFFFFFFFF)


@pytest.mark.parametrize("leaves", [3, 5, 6, 9, 14])
def test_lossguide_with_equal_gains_is_best_first_in_rust_heap_order(leaves):
    """Loss-guided growth on mirrored data, where every node below the root
    has a twin of equal loss change, with leaf budgets that cut between
    twins. Brute force: every pop takes a candidate whose loss change is the
    largest left in the queue (ties allowed), an expanded node's two
    children get the next two ids, and the budget stops expansion. Tie
    order: the pops equal those of Rust's BinaryHeap (the reference's
    queue, builder/hist/mod.rs:505-573, keyed by loss_chg.total_cmp,
    :132-148) fed the same pushes."""
    x, gp = _mirrored_data(4)
    ds = O.Dataset(x, max_bin=64)
    p = O.params(grow_policy=O.GROW_LOSSGUIDE, max_depth=0, max_leaves=leaves, eta=0.3)
    nodes, ev = O.lossguide_events(ds, gp, p)
    pushed = {nid: chg for kind, nid, chg, _ in ev if kind == "push"}
    assert nodes[0]["split_feature"] == 0 and pushed[1] == pushed[2] > 0
    queue, heap = {}, RustBinaryHeap()
    next_id, n_leaves, ties, expanded = 1, 1, 0, []
    i = 0
    while i < len(ev):
        kind, nid, chg, expandable = ev[i]
        if kind == "push":
            queue[nid] = chg
            heap.push(_total_key(chg), nid)
            i += 1
            continue
        best = max(_total_key(c) for c in queue.values())
        assert _total_key(chg) == best, (i, nid)
        ties += sum(_total_key(c) == best for c in queue.values()) - 1
        assert heap.pop()[1] == nid, (i, nid)
        del queue[nid]
        i += 1
        if n_leaves >= leaves:
            assert i == len(ev), "growth continues past the leaf budget"
            break
        if not expandable:
            continue
        expanded.append(nid)
        n_leaves += 1
        assert [e[:2] for e in ev[i:i + 2]] == [("push", next_id), ("push", next_id + 1)], (i, nid)
        assert nodes[nid]["left"] == next_id and nodes[nid]["right"] == next_id + 1
        next_id += 2
    assert ties > 0, "the data must put equal gains in the queue"
    assert sum(nd["left"] == -1 for nd in nodes) == min(leaves, len(nodes))
    assert len(expanded) == leaves - 1
