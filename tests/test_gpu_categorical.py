"""Categorical features trained on the GPU: the device's categorical sweep
(one-hot below 4 categories, else the weight-sorted partition scans of
builder/categorical.rs:48-170), routing by category tables in the partition
(RowRule::Table) and the trees' category sets, against the reference's own
saved categorical model and the oracle."""
import numpy as np
import pytest

import hessboost_amd as hb
from hessboost_amd import _capi as A
from oracle import oracle as O
from tests.helpers import categorical_features, load_saved_models
from tests.test_gpu_train import compare_trees

pytestmark = pytest.mark.gpu


def compare_categories(gpu_trees, ref_trees):
    """Categorical nodes hold the oracle's category sets (codes, sorted)."""
    for t, (g, r) in enumerate(zip(gpu_trees, ref_trees)):
        isc = g.get("is_categorical", np.zeros(len(g["left"]), np.uint8))
        for i, nd in enumerate(r):
            assert bool(isc[i]) == bool(nd["is_categorical"]), (t, i)
            if nd["is_categorical"]:
                got = g["categories"][g["cat_begin"][i]:g["cat_end"][i]].tolist()
                assert got == nd["categories"], (t, i)


def test_reference_categorical_model_retrained_on_gpu():
    """tests/native_format.rs:508-540: the saved categorical-splits model
    (hist, depth 3, four_features with column 0 the codes i % 5 as a
    categorical feature) grown again on the GPU: every tree node for node,
    its category sets, split gains, Hessian sums and leaf values bit for bit."""
    saved = load_saved_models()["0.4.9/categorical_splits"]
    x = categorical_features()
    y = (np.array([0.0, 2.0, -1.0, 3.0, 1.0], np.float32)[np.arange(len(x)) % 5] + x[:, 1]).astype(np.float32)
    model = hb.train({"max_depth": 3}, hb.DMatrix(x, label=y, feature_types=["c", "q", "q", "q"]), 4)
    assert np.float32(model.base_score[0]).view(np.uint32) == np.uint32(saved["base_score"][0])
    for t, (g, ref) in enumerate(zip(model.trees, saved["trees"])):
        assert list(g["left"]) == ref["left"] and list(g["right"]) == ref["right"], t
        internal = np.array(ref["left"]) != -1
        assert np.array_equal(g["split_feature"][internal], np.array(ref["split_feature"])[internal]), t
        assert np.array_equal(g["split_cond"].view(np.uint32)[internal], np.array(ref["split_cond"], np.uint32)[internal])
        assert np.array_equal(g["default_left"][internal], np.array(ref["default_left"], np.uint8)[internal]), t
        assert np.array_equal(g["split_gain"].view(np.uint32)[internal], np.array(ref["split_gain"], np.uint32)[internal])
        assert np.array_equal(g["leaf_value"].view(np.uint32), np.array(ref["leaf_value"], np.uint32)), t
        assert np.array_equal(g["sum_hess"].view(np.uint32), np.array(ref["sum_hess"], np.uint32)), t
        assert np.array_equal(g["is_categorical"], np.array(ref["is_categorical"], np.uint8)), t
        pool = ref["categories"]
        for i in np.nonzero(g["is_categorical"])[0]:
            assert g["categories"][g["cat_begin"][i]:g["cat_end"][i]].tolist() == \
                pool[ref["cat_begin"][i]:ref["cat_end"][i]], (t, i)
    m = model.predict(x, output_margin=True)
    assert np.array_equal(m.view(np.uint32), np.array(saved["margins"], np.uint32))


def categorical_data(seed, n, n_cats, objective="reg:squarederror", k=3, missing=0.05):
    """Numeric features plus categorical ones whose effects are not
    monotone in the code (a shuffled effect per category)."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, 2 + len(n_cats))).astype(np.float32)
    z = 0.5 * x[:, 0]
    for j, c in enumerate(n_cats):
        codes = rng.integers(0, c, n)
        x[:, 2 + j] = codes
        z = z + rng.standard_normal(c)[codes]
    if missing:
        x[rng.random(x.shape) < missing] = np.nan
    if objective == "reg:squarederror":
        y = (z + 0.1 * rng.standard_normal(n)).astype(np.float32)
    elif objective == "binary:logistic":
        y = (rng.random(n) < 1 / (1 + np.exp(-z))).astype(np.float32)
    else:
        y = np.clip(np.floor((z - z.min()) / (np.ptp(z) + 1e-9) * k), 0, k - 1).astype(np.float32)
    types = ["q", "q"] + ["c"] * len(n_cats)
    return x, y, types


OBJ = {"reg:squarederror": O.OBJ_SQUARED_ERROR, "binary:logistic": O.OBJ_LOGISTIC, "multi:softprob": O.OBJ_SOFTMAX}

CASES = [
    # name, n, categories per categorical feature, params, missing
    ("one-hot", 5_000, [3, 2], {"objective": "reg:squarederror", "max_depth": 4}, 0.05),
    ("partition", 20_000, [12, 9], {"objective": "reg:squarederror", "max_depth": 6}, 0.1),
    ("beyond the 64-deep scan", 30_000, [300], {"objective": "binary:logistic", "max_depth": 5}, 0.02),
    ("300 categories on u16 rows", 30_000, [300], {"objective": "binary:logistic", "max_depth": 5}, 0.0),
    ("lossguide", 12_000, [7, 40], {"objective": "reg:squarederror", "grow_policy": "lossguide", "max_depth": 0,
                                    "max_leaves": 24}, 0.05),
    ("softmax", 9_000, [6], {"objective": "multi:softprob", "num_class": 3, "max_depth": 4}, 0.0),
    ("regularised", 10_000, [5, 17], {"objective": "reg:squarederror", "max_depth": 5, "lambda": 3.0,
                                      "alpha": 0.5, "min_child_weight": 4.0, "gamma": 0.1}, 0.05),
]


@pytest.mark.parametrize("name,n,n_cats,params,missing", CASES, ids=[c[0] for c in CASES])
def test_categorical_training_matches_oracle(name, n, n_cats, params, missing):
    x, y, types = categorical_data(len(name), n, n_cats, params["objective"], params.get("num_class", 3), missing)
    w = np.random.default_rng(3).random(n).astype(np.float32) + 0.5 if name == "lossguide" else None
    p = dict(params, eta=0.3)
    op = O.params(objective=OBJ[p["objective"]], eta=0.3, max_depth=p["max_depth"],
                  max_leaves=p.get("max_leaves", 0), num_class=p.get("num_class", 0),
                  grow_policy=O.GROW_LOSSGUIDE if p.get("grow_policy") == "lossguide" else O.GROW_DEPTHWISE,
                  reg_lambda=p.get("lambda", 1.0), alpha=p.get("alpha", 0.0),
                  min_child_weight=p.get("min_child_weight", 1.0), gamma=p.get("gamma", 0.0))
    ref = O.Model(O.Dataset(x, weights=w, feature_types=types), y, op, 3, weights=w)
    model = hb.train(p, hb.DMatrix(x, label=y, weight=w, feature_types=types), 3)
    ref_trees = ref.trees()
    compare_trees(model.trees, ref_trees)
    compare_categories(model.trees, ref_trees)
    assert any(nd["is_categorical"] for t in ref_trees for nd in t), "no categorical split"
    m = model.predict(x, output_margin=True).reshape(-1)
    assert np.max(np.abs(m - ref.margins())) <= 1e-5


def test_categorical_csr_input_matches_oracle():
    x, y, types = categorical_data(9, 8_000, [11], "reg:squarederror", missing=0.3)
    present = ~np.isnan(x)
    rp = np.zeros(x.shape[0] + 1, np.uint64)
    rp[1:] = np.cumsum(present.sum(1))
    r, c = np.nonzero(present)
    csr = (rp, c.astype(np.uint32), x[r, c])
    ref = O.Model(O.Dataset(csr=csr, n_cols=x.shape[1], feature_types=types), y, O.params(max_depth=5, eta=0.3), 3)
    model = hb.train({"max_depth": 5, "eta": 0.3}, hb.DMatrix(csr, label=y, n_cols=x.shape[1], feature_types=types),
                     3)
    compare_trees(model.trees, ref.trees())
    compare_categories(model.trees, ref.trees())


def test_categorical_models_save_load(tmp_path):
    """A trained categorical model round-trips through the native format and
    predicts the same margins."""
    x, y, types = categorical_data(4, 6_000, [8], "reg:squarederror")
    model = hb.train({"max_depth": 4}, hb.DMatrix(x, label=y, feature_types=types), 3)
    model.save_model(tmp_path / "cat.bin")
    back = hb.Booster(objective="reg:squarederror", base_score=np.zeros(1, np.float32)).load_model(tmp_path / "cat.bin")
    assert np.array_equal(back.predict(x, output_margin=True).view(np.uint32),
                          model.predict(x, output_margin=True).view(np.uint32))


@pytest.mark.parametrize("objective,k", [("reg:squarederror", 1), ("binary:logistic", 1), ("multi:softprob", 3)])
def test_categorical_eval_sets_follow_the_model(objective, k):
    """Evaluation sets on an index with categorical features
    (training/margins.rs:148-152, :186-196): the device walk routes each
    categorical split by its category set (a present value's saturating
    cast among the node's categories; missing values the default way, codes
    never seen in training and negative or fractional values too), so after
    every round the set's margins equal the model's own prediction bit for
    bit; a set added after trees were grown takes them first."""
    x, y, types = categorical_data(7, 8_000, [6, 40], objective, k)
    xe, _, _ = categorical_data(8, 3_001, [9, 45], objective, k)  # codes beyond training's
    xe[::7, 2] = -1.5
    xe[::11, 3] = 2.5
    xe[::13, 3] = 1e10
    params = {"objective": objective, "max_depth": 5, "eta": 0.3}
    if k > 1:
        params["num_class"] = k
    model = hb.train(params, hb.DMatrix(x, label=y, feature_types=types), 4,
                     evals=[(hb.DMatrix(xe, feature_types=types), "eval"),
                            (hb.DMatrix(x, feature_types=types), "train")])
    assert any(np.any(t.get("is_categorical", ())) for t in model.trees)
    for name, data in (("eval", xe), ("train", x)):
        got = model.eval_margins[name].reshape(-1)
        want = model.predict(data, output_margin=True).reshape(-1)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), name
    eng = hb.DMatrix(x, label=y, feature_types=types).engine(256)
    t = hb.Trainer(eng, params, y)
    t.boost(2)
    late = t.add_eval(hb.DMatrix(xe, feature_types=types))
    t.boost(2)
    b = t.booster(x.shape[1])
    assert np.array_equal(t.eval_margins(late).reshape(-1).view(np.uint32),
                          b.predict(xe, output_margin=True).reshape(-1).view(np.uint32))


def exact_categorical_node(seed, n, n_cats, outlier_code=None):
    """An engine and the oracle over numeric + categorical features, with
    dyadic gradients (every sum exact) driven by the first categorical
    feature's codes, staged and built at the root. outlier_code: that
    category's rows get g = 2^100 and h = 2^-30, the others g scaled by 2^96,
    so its weight G / H = 2^130 overflows f32 while every sum stays exact."""
    x, _, types = categorical_data(seed, n, n_cats, missing=0.1)
    rng = np.random.default_rng(seed)
    effect = np.round(rng.standard_normal(n_cats[0]) * 16) / 8
    codes = np.nan_to_num(x[:, 2], nan=-1).astype(np.int64)
    g = np.where(codes >= 0, effect[np.maximum(codes, 0)], 0.0) + rng.integers(-2, 3, n) / 16
    h = np.ones(n)
    if outlier_code is not None:
        g = g * 2.0 ** 96
        g[codes == outlier_code] = 2.0 ** 100
        h[codes == outlier_code] = 2.0 ** -30
    gp = np.stack([g, h], 1).astype(np.float32)
    eng = hb.DMatrix(x, feature_types=types).engine()
    ref = O.Dataset(x, feature_types=types)
    eng.prepare(gp)
    root = eng.begin_tree()
    tot, fixed = eng.root_total(root, fixed=True)
    eng.reserve_hists(8)
    eng.build_resident([(root, 0)])
    hist = eng.read_hist(0)
    want_hist = ref.build_hist(np.arange(n, dtype=np.uint32), gp)
    assert np.array_equal(hist, want_hist)
    return eng, ref, gp, root, tot, fixed, want_hist


def oracle_partition_categorical(ref, rows, feature, cat_left, default_left):
    rows = np.ascontiguousarray(rows, np.uint32)
    left, right = np.empty(len(rows), np.uint32), np.empty(len(rows), np.uint32)
    words = np.ascontiguousarray(cat_left, np.uint32)
    nl = O.lib().or_partition_categorical(ref.index, rows.ctypes.data, len(rows), feature, words.ctypes.data,
                                          int(default_left), left.ctypes.data, right.ctypes.data)
    return left[:nl], right[:len(rows) - nl]


@pytest.mark.parametrize("n_cats", [[12, 3], [3, 40]], ids=["partition-sweep", "one-hot"])
def test_engine_categorical_scan_and_table_partition_match_oracle(n_cats):
    """The resident search's NodeScan::Categorical (hbr_scan_resident: the
    winning feature, loss, children in the tree's orientation, missing-value
    direction and ascending category codes) against the oracle's sequential
    search (builder/categorical.rs:48-170), then RowRule::Table routing
    (hbr_partition with a table) against the oracle's categorical partition,
    over two levels with a numeric split beside a table."""
    n = 30_000
    eng, ref, gp, root, tot, fixed, want_hist = exact_categorical_node(len(n_cats) + n_cats[0], n, n_cats)
    p = O.params()
    reg = (1.0, 0.0, 0.0, 1.0)
    rg = O.lib().or_node_gain(tot[0], tot[1], -np.inf, np.inf, p)
    scan, = eng.scan_resident(reg, [dict(slot=0, total=tuple(tot), fixed=tuple(fixed), root_gain=rg)])
    want = ref.evaluate(want_hist, tot, p)
    assert want.categorical and want.feature == 2
    assert scan.kind == A.SCAN_CATEGORICAL
    assert scan.feature == want.feature and np.float32(scan.loss_chg) == np.float32(want.loss_chg)
    assert bool(scan.default_left) == bool(want.default_left)
    assert (scan.left_g, scan.left_h, scan.right_g, scan.right_h) == \
        (want.left_g, want.left_h, want.right_g, want.right_h)
    fo, cuts = ref.feature_offset, ref.cut_values
    fs, nb = int(fo[2]), int(fo[3] - fo[2])
    in_set = [bool(want.cat_left[b // 32] >> (b % 32) & 1) for b in range(nb)]
    codes = sorted(int(cuts[fs + b]) for b in range(nb) if in_set[b])
    assert eng.scan_categories[scan.cat_begin:scan.cat_end].tolist() == codes

    all_rows = np.arange(n, dtype=np.uint32)
    (left, right), = eng.partition([(root, 2, in_set, scan.default_left)])
    wl, wr = oracle_partition_categorical(ref, all_rows, 2, want.cat_left, want.default_left)
    assert np.array_equal(eng.rows(left), wl) and np.array_equal(eng.rows(right), wr)
    # the next level: a numeric split (RowRule::Below) beside a table on the other feature
    nb3 = int(fo[4] - fo[3])
    table3 = [b % 2 == 0 for b in range(nb3)]
    words3 = np.zeros(32, np.uint32)
    for b in range(nb3):
        if table3[b]:
            words3[b // 32] |= np.uint32(1 << (b % 32))
    (l2, r2), (l3, r3) = eng.partition([(left, 0, 7, 1), (right, 3, table3, 0)])
    a, b = ref.partition(wl, 0, int(fo[0]) + 6, 1)
    c, d = oracle_partition_categorical(ref, wr, 3, words3, 0)
    assert np.array_equal(eng.rows(l2), a) and np.array_equal(eng.rows(r2), b)
    assert np.array_equal(eng.rows(l3), c) and np.array_equal(eng.rows(r3), d)


def test_engine_scan_asks_for_replay_on_non_finite_category_weights():
    """A category whose weight overflows f32 (lambda = 0, min_child_weight =
    0) makes the sort's order not total: the node comes back as
    NodeScan::Replay (src/tree/hist/mod.rs:313-331) rather than a winner, as
    the reference's device search answers it (the same node's numeric scores
    overflow too, which asks for the replay as well)."""
    eng, ref, gp, root, tot, fixed, _ = exact_categorical_node(5, 20_000, [9, 2], outlier_code=4)
    reg = (0.0, 0.0, 0.0, 0.0)
    p = O.params(reg_lambda=0.0, min_child_weight=0.0)
    rg = O.lib().or_node_gain(tot[0], tot[1], -np.inf, np.inf, p)
    scan, = eng.scan_resident(reg, [dict(slot=0, total=tuple(tot), fixed=tuple(fixed), root_gain=rg)])
    assert scan.kind == A.SCAN_REPLAY
    assert scan.fallback in (A.FALLBACK_CATEGORICAL_ORDER, A.FALLBACK_NUMERIC_SCORE)
    # ordinary gradients on the same features: a winner
    eng, ref, gp, root, tot, fixed, _ = exact_categorical_node(5, 20_000, [9, 2])
    p = O.params()
    rg = O.lib().or_node_gain(tot[0], tot[1], -np.inf, np.inf, p)
    scan, = eng.scan_resident((1.0, 0.0, 0.0, 1.0), [dict(slot=0, total=tuple(tot), fixed=tuple(fixed),
                                                          root_gain=rg)])
    assert scan.kind == A.SCAN_CATEGORICAL


def test_table_partition_refuses_numeric_features_and_wrong_lengths():
    eng, ref, gp, root, *_ = exact_categorical_node(6, 5_000, [5, 3])
    nb0 = int(ref.feature_offset[1] - ref.feature_offset[0])
    with pytest.raises(A.HbrError) as e:
        eng.partition([(root, 0, [True] * nb0, 0)])
    assert e.value.status == A.REFUSED
    root = eng.begin_tree()
    with pytest.raises(A.HbrError) as e:
        eng.partition([(root, 2, [True, False], 0)])
    assert e.value.status == A.INVALID
