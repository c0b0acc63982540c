"""GPU training parity: whole trees and boosting runs against the oracle and
the reference's own saved model."""
import numpy as np
import pytest

import hessboost_amd as hb
from hessboost_amd import synthetic
from hessboost_amd._capi import LOSS_LOGISTIC
from oracle import oracle as O
from tests.helpers import four_features, load_saved_models, train_labels

pytestmark = pytest.mark.gpu


def compare_trees(gpu_trees, ref_trees, leaf_rtol=1e-5, exact=False):
    """Identical structure (split feature, threshold, default direction,
    children), leaf values within leaf_rtol (bit-exact when `exact`)."""
    assert len(gpu_trees) == len(ref_trees)
    for t, (g, r) in enumerate(zip(gpu_trees, ref_trees)):
        assert len(g["left"]) == len(r), f"tree {t}: node count"
        for i, nd in enumerate(r):
            assert g["left"][i] == nd["left"] and g["right"][i] == nd["right"], (t, i)
            if nd["left"] != -1:
                assert g["split_feature"][i] == nd["split_feature"], (t, i)
                assert np.float32(g["split_cond"][i]) == np.float32(nd["split_cond"]), (t, i)
                assert bool(g["default_left"][i]) == bool(nd["default_left"]), (t, i)
            else:
                a, b = np.float32(g["leaf_value"][i]), np.float32(nd["leaf_value"])
                if exact:
                    assert a == b, (t, i, a, b)
                else:
                    assert abs(a - b) <= leaf_rtol * abs(b) + 1e-12, (t, i, a, b)


def test_saved_model_retrained_on_gpu():
    """tests/native_format.rs:660-669: the reference's saved early-stopping
    model (hist, depth 3, 4 rounds, squared error, a feature with missing
    values) is grown again on the GPU: the same trees node for node."""
    saved = load_saved_models()["0.4.9/early_stopping"]
    x = four_features()
    y = train_labels(x)
    model = hb.train({"max_depth": 3}, hb.DMatrix(x, label=y), 4)
    assert np.float32(model.base_score[0]).view(np.uint32) == np.uint32(saved["base_score"][0])
    for t, (g, ref) in enumerate(zip(model.trees, saved["trees"])):
        assert list(g["left"]) == ref["left"] and list(g["right"]) == ref["right"], t
        internal = np.array(ref["left"]) != -1
        assert np.array_equal(g["split_feature"][internal], np.array(ref["split_feature"])[internal])
        assert np.array_equal(g["split_cond"].view(np.uint32)[internal], np.array(ref["split_cond"], np.uint32)[internal])
        assert np.array_equal(g["default_left"][internal], np.array(ref["default_left"], np.uint8)[internal])
        assert np.array_equal(g["split_gain"].view(np.uint32)[internal], np.array(ref["split_gain"], np.uint32)[internal])
        lv = g["leaf_value"].view(np.uint32)[~internal]
        want = np.array(ref["leaf_value"], np.uint32)[~internal]
        assert np.array_equal(lv, want), t
        assert np.array_equal(g["sum_hess"].view(np.uint32), np.array(ref["sum_hess"], np.uint32)), t


@pytest.mark.parametrize("objective", ["reg:squarederror", "binary:logistic"])
def test_boosting_matches_oracle(objective):
    """Several rounds, depthwise, free-running: identical structure every
    round, leaf values within 1e-5, margins within 1e-5."""
    x, y = synthetic.regression_100k(n=20_000, f=16, seed=1)
    if objective == "binary:logistic":
        y = (y > 0).astype(np.float32)
    params = {"objective": objective, "max_depth": 6, "eta": 0.3}
    ds = O.Dataset(x, max_bin=256)
    ref = O.Model(ds, y, O.params(objective=O.OBJ_LOGISTIC if objective != "reg:squarederror" else O.OBJ_SQUARED_ERROR,
                                 max_depth=6, eta=0.3), 8)
    model = hb.train(params, hb.DMatrix(x, label=y), 8)
    compare_trees(model.trees, ref.trees())
    m = model.predict(x, output_margin=True)
    assert np.max(np.abs(m - ref.margins())) <= 1e-5


@pytest.mark.parametrize("objective,spw,weighted", [
    ("binary:logistic", 2.0, False), ("binary:logistic", 0.5, True), ("binary:logitraw", 1.0, False),
    ("binary:logitraw", 2.0, True), ("reg:squarederror", 2.0, True)])
def test_intercepts_match_oracle(objective, spw, weighted):
    """classification.rs:132-141 / regression.rs:66-74: scale_pos_weight away
    from 1 takes one Newton step for the intercept (objective/mod.rs:528-566);
    binary:logitraw keeps the label mean and the step raw
    (classification.rs:67-72). The base score bit for bit, then the trees
    and margins, against the oracle."""
    x, y = synthetic.regression_100k(n=9_003, f=8, seed=11)
    y = (y > 0.7).astype(np.float32) if objective != "reg:squarederror" else y
    if objective == "reg:squarederror":
        y[::5] = 1.0  # labels of exactly 1 are the ones scale_pos_weight reweighs
    w = np.random.default_rng(11).random(len(y)).astype(np.float32) + 0.2 if weighted else None
    obj = {"binary:logistic": O.OBJ_LOGISTIC, "binary:logitraw": O.OBJ_LOGITRAW,
           "reg:squarederror": O.OBJ_SQUARED_ERROR}[objective]
    ref = O.Model(O.Dataset(x, weights=w), y, O.params(objective=obj, max_depth=5, eta=0.3, scale_pos_weight=spw), 4,
                  weights=w)
    model = hb.train({"objective": objective, "max_depth": 5, "eta": 0.3, "scale_pos_weight": spw},
                     hb.DMatrix(x, label=y, weight=w), 4)
    assert np.float32(model.base_score[0]).view(np.uint32) == np.float32(ref.base_score()[0]).view(np.uint32)
    compare_trees(model.trees, ref.trees())
    m = model.predict(x, output_margin=True)
    assert np.max(np.abs(m - ref.margins())) <= 1e-5
    if objective == "binary:logitraw":
        assert np.array_equal(model.predict(x), m)  # predictions stay raw margins


def test_lossguide_matches_oracle():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((8_000, 8), dtype=np.float32)
    x[rng.random(x.shape) < 0.1] = np.nan
    y = (np.nan_to_num(x[:, 0]) * 2 + np.nan_to_num(x[:, 1]) ** 2).astype(np.float32)
    params = {"grow_policy": "lossguide", "max_depth": 0, "max_leaves": 31, "eta": 0.3}
    ref = O.Model(O.Dataset(x), y, O.params(grow_policy=O.GROW_LOSSGUIDE, max_depth=0, max_leaves=31), 3)
    model = hb.train(params, hb.DMatrix(x, label=y), 3)
    compare_trees(model.trees, ref.trees())


def test_softmax_matches_oracle():
    x, y = synthetic.multiclass(n=6_000, f=10, k=4, seed=3)
    params = {"objective": "multi:softprob", "num_class": 4, "max_depth": 4, "eta": 0.3}
    ref = O.Model(O.Dataset(x), y, O.params(objective=O.OBJ_SOFTMAX, num_class=4, max_depth=4), 3)
    model = hb.train(params, hb.DMatrix(x, label=y), 3)
    compare_trees(model.trees, ref.trees())


def test_softmax_two_classes_weighted_deep_and_lossguide_match_oracle():
    """The 2-class vector batches with weights (depth 10: the walk of
    trees too deep for its LDS table), three classes grown level by level
    from the device's class pairs (lossguide), against the oracle."""
    x, y = synthetic.multiclass(n=7_001, f=12, k=2, seed=5)
    w = np.random.default_rng(5).random(len(y)).astype(np.float32) + 0.25
    params = {"objective": "multi:softprob", "num_class": 2, "max_depth": 10, "eta": 0.3}
    ref = O.Model(O.Dataset(x, weights=w), y, O.params(objective=O.OBJ_SOFTMAX, num_class=2, max_depth=10), 3,
                  weights=w)
    model = hb.train(params, hb.DMatrix(x, label=y, weight=w), 3)
    compare_trees(model.trees, ref.trees())
    x, y = synthetic.multiclass(n=5_000, f=7, k=3, seed=6)
    params = {"objective": "multi:softprob", "num_class": 3, "grow_policy": "lossguide", "max_depth": 0,
              "max_leaves": 15, "eta": 0.3}
    ref = O.Model(O.Dataset(x), y, O.params(objective=O.OBJ_SOFTMAX, num_class=3, grow_policy=O.GROW_LOSSGUIDE,
                                            max_depth=0, max_leaves=15), 3)
    model = hb.train(params, hb.DMatrix(x, label=y), 3)
    compare_trees(model.trees, ref.trees())


@pytest.mark.parametrize("k,depth,weighted", [(2, 5, True), (3, 6, False), (10, 4, True)])
def test_batched_class_trees_equal_one_class_at_a_time(k, depth, weighted):
    """A softmax round's class trees grown as one batch (every level of all
    of them in one launch of each kernel) equal, bit for bit, the trees
    grown one class after another, and the final margins too."""
    import os
    x, y = synthetic.multiclass(n=9_001, f=12, k=k, seed=20 + k)
    w = np.random.default_rng(k).random(len(y)).astype(np.float32) + 0.5 if weighted else None
    params = {"objective": "multi:softprob", "num_class": k, "max_depth": depth, "eta": 0.3,
              "lambda": 1.5, "min_child_weight": 0.5}
    dm = hb.DMatrix(x, label=y, weight=w)
    runs = []
    for flag in ("1", "0"):
        os.environ["HBROCM_SOFTMAX_BATCH"] = flag
        try:
            tr = hb.Trainer(dm.engine(256), params, y, w)
            tr.boost(3)
            runs.append((tr.trees(), tr.margins()))
        finally:
            os.environ.pop("HBROCM_SOFTMAX_BATCH", None)
    (ta, ma), (tb, mb) = runs
    assert len(ta) == len(tb) == 3 * k
    for a, b in zip(ta, tb):
        for key in a:
            assert np.array_equal(a[key], b[key]), key
    assert np.array_equal(ma.view(np.uint32), mb.view(np.uint32))


@pytest.mark.parametrize("f,k,depth,kernel", [(12, 3, 5, "hbr_walk_leaves_batch32"),
                                               (50, 10, 6, "hbr_walk_leaves_batch64"),
                                               (50, 10, 7, None)])
def test_one_pass_class_walk_equals_a_walk_per_class_tree(f, k, depth, kernel):
    """A batched softmax round adds its K class trees to the margins in one
    pass over the rows (hbr_walk_leaves_batch32/64, 32- and 64-byte rows);
    the trees and margins equal those of one walk per class tree bit for
    bit. Ten depth-7 trees outgrow the one-pass walk's node tables, and the
    round falls back to a walk per tree."""
    import os
    x, y = synthetic.multiclass(n=20_011, f=f, k=k, seed=40 + f)
    params = {"objective": "multi:softprob", "num_class": k, "max_depth": depth, "eta": 0.3}
    dm = hb.DMatrix(x, label=y)
    runs = []
    for flag in ("1", "0"):
        os.environ["HBROCM_BATCH_WALK"] = flag
        try:
            eng = dm.engine(256)
        finally:
            os.environ.pop("HBROCM_BATCH_WALK", None)
        tr = hb.Trainer(eng, params, y)
        eng.set_profiling(True, "hbr_walk")
        tr.boost(3)
        stats = eng.kernel_stats()
        eng.set_profiling(False)
        runs.append((tr.trees(), tr.margins(), stats))
    (ta, ma, sa), (tb, mb, sb) = runs
    batch = {"hbr_walk_leaves_batch32", "hbr_walk_leaves_batch64"}
    if kernel:
        assert kernel in sa and not batch & set(sb)
    else:
        assert not batch & set(sa)
    assert len(ta) == len(tb) == 3 * k
    for a, b in zip(ta, tb):
        for key in a:
            assert np.array_equal(a[key], b[key]), key
    assert np.array_equal(ma.view(np.uint32), mb.view(np.uint32))


@pytest.mark.parametrize("n,k", [(5, 3), (33, 3), (70, 1), (130, 7)])
def test_batched_class_trees_on_tiny_inputs_match_oracle(n, k):
    """Batched class trees where rows are few (fewer than the classes, or a
    part of one partition tile) and a one-class softmax: the oracle's trees,
    and the same as one class after another."""
    import os
    x, y = synthetic.multiclass(n=n, f=6, k=max(k, 2), seed=n + k)
    y = (y % k).astype(np.float32)
    params = {"objective": "multi:softprob", "num_class": k, "max_depth": 4, "eta": 0.3, "min_child_weight": 0.0}
    ref = O.Model(O.Dataset(x), y, O.params(objective=O.OBJ_SOFTMAX, num_class=k, max_depth=4,
                                            min_child_weight=0.0), 2)
    trees = []
    for flag in ("1", "0"):
        os.environ["HBROCM_SOFTMAX_BATCH"] = flag
        try:
            trees.append(hb.train(params, hb.DMatrix(x, label=y), 2).trees)
        finally:
            os.environ.pop("HBROCM_SOFTMAX_BATCH", None)
    compare_trees(trees[0], ref.trees())
    compare_trees(trees[1], ref.trees())


def test_softmax_labels_must_be_class_indices():
    """multiclass.rs:96-100: a label that is not a class index is refused."""
    x, y = synthetic.multiclass(n=500, f=4, k=3, seed=7)
    params = {"objective": "multi:softprob", "num_class": 3, "max_depth": 3}
    for bad in (1.5, -1.0, 3.0, np.nan):
        yb = y.copy()
        yb[17] = bad
        with pytest.raises(Exception, match="class indices"):
            hb.train(params, hb.DMatrix(x, label=yb), 1)


def test_monotone_and_regularization_match_oracle():
    x, y = synthetic.regression_100k(n=10_000, f=6, seed=4)
    mono = [1, -1, 0, 0, 1, 0]
    params = {"max_depth": 5, "eta": 0.5, "lambda": 2.0, "alpha": 0.5, "gamma": 0.1,
              "min_child_weight": 3.0, "monotone_constraints": mono}
    ref = O.Model(O.Dataset(x), y, O.params(max_depth=5, eta=0.5, reg_lambda=2.0, alpha=0.5, gamma=0.1,
                                            min_child_weight=3.0, monotone=mono), 4)
    model = hb.train(params, hb.DMatrix(x, label=y), 4)
    compare_trees(model.trees, ref.trees())


def _grow_both(x, y, params, rounds):
    """Train twice on one index: trees decided on the device (default for
    a dense u8 index, depthwise) and trees decided by the host level by
    level (HBROCM_DEVICE_GROW=0, read when an engine is made)."""
    import os
    dm = hb.DMatrix(x, label=y)
    index = dm.index(params.get("max_bin", 256))
    out = []
    for flag in (None, "0"):
        old = os.environ.pop("HBROCM_DEVICE_GROW", None)
        if flag is not None:
            os.environ["HBROCM_DEVICE_GROW"] = flag
        try:
            eng = hb.Engine(index, 0)
        finally:
            os.environ.pop("HBROCM_DEVICE_GROW", None)
            if old is not None:
                os.environ["HBROCM_DEVICE_GROW"] = old
        tr = hb.Trainer(eng, params, y)
        eng.set_profiling(True, "hbr_grow_decide")
        tr.boost(rounds)
        launches = sum(n for _, (_, _, n) in eng.kernel_stats().items())
        eng.set_profiling(False)
        out.append((tr.trees(), tr.margins(), launches))
    return out


@pytest.mark.parametrize("depth,params", [
    (1, {"objective": "reg:squarederror"}),
    (3, {"objective": "binary:logistic", "gamma": 0.5, "max_delta_step": 0.7}),
    (8, {"objective": "binary:logistic", "alpha": 0.3, "lambda": 2.0, "min_child_weight": 5.0}),
    (11, {"objective": "reg:squarederror", "monotone_constraints": [1, -1, 0, 1, 0, 0, -1, 0]}),
])
def test_device_decided_growth_equals_host_decided(depth, params):
    """The device's level decisions (split positions, validity, child bounds,
    slot reuse, node ids, final leaf values) give the trees the host's
    decisions give, every field bit for bit, and the same margins; the
    device path is the one that ran (one decision launch per level)."""
    rng = np.random.default_rng(depth)
    n, f = 30_000, 8
    x = rng.standard_normal((n, f)).astype(np.float32)
    x[:, 3] = np.round(x[:, 3] * 2)  # a few distinct values: ties, empty bins
    y = (x[:, 0] - 0.5 * x[:, 1] ** 2 + 0.3 * x[:, 3] + 0.1 * rng.standard_normal(n)).astype(np.float32)
    if params["objective"] == "binary:logistic":
        y = (y > 0).astype(np.float32)
    p = dict(params, max_depth=depth, eta=0.3)
    rounds = 4
    (dev_trees, dev_m, dev_launches), (host_trees, host_m, host_launches) = _grow_both(x, y, p, rounds)
    assert dev_launches == rounds * depth and host_launches == 0
    assert len(dev_trees) == len(host_trees) == rounds
    for t, (a, b) in enumerate(zip(dev_trees, host_trees)):
        for key in ("left", "right", "split_feature", "default_left", "split_bin"):
            assert np.array_equal(a[key], b[key]), (t, key)
        for key in ("split_cond", "leaf_value", "sum_hess", "split_gain"):
            assert np.array_equal(a[key].view(np.uint32), b[key].view(np.uint32)), (t, key)
    assert np.array_equal(dev_m.view(np.uint32), host_m.view(np.uint32))
    # and the oracle's trees
    obj = O.OBJ_LOGISTIC if params["objective"] == "binary:logistic" else O.OBJ_SQUARED_ERROR
    kw = {k: v for k, v in params.items() if k in ("gamma", "max_delta_step", "alpha", "min_child_weight")}
    if "lambda" in params:
        kw["reg_lambda"] = params["lambda"]
    if "monotone_constraints" in params:
        kw["monotone"] = params["monotone_constraints"]
    ref = O.Model(O.Dataset(x, max_bin=256), y, O.params(objective=obj, max_depth=depth, eta=0.3, **kw), rounds)
    compare_trees(dev_trees, ref.trees())


@pytest.mark.parametrize("env", [
    {"HBROCM_HIST_WAVES": "2"},
    {"HBROCM_HIST_FG": "16"},
    {"HBROCM_HIST_FG": "8"},
    {"HBROCM_HIST_BIN_MAJOR": "0", "HBROCM_HIST_THREADS": "512"},
    {"HBROCM_HIST_WAVES": "3", "HBROCM_DEVICE_GROW": "0"},
])
def test_launch_shapes_give_identical_trees(env):
    """Histograms are exact integer sums, so the launch shape (features per
    workgroup, LDS layout, threads, tiles per launch, levels decided on the
    device or the host) cannot change a bit of the trees or the margins."""
    import os
    rng = np.random.default_rng(7)
    n, f = 60_000, 40
    x = rng.standard_normal((n, f)).astype(np.float32)
    x[:, 5] = np.round(x[:, 5])
    y = (x[:, 0] + x[:, 5] * x[:, 1] + 0.2 * rng.standard_normal(n) > 0).astype(np.float32)
    params = {"objective": "binary:logistic", "max_depth": 7, "eta": 0.3}
    index = hb.DMatrix(x, label=y).index(256)
    runs = []
    for e in ({}, env):
        saved = {k: os.environ.pop(k, None) for k in e}
        os.environ.update(e)
        try:
            eng = hb.Engine(index, 0)
        finally:
            for k in e:
                os.environ.pop(k, None)
                if saved[k] is not None:
                    os.environ[k] = saved[k]
        tr = hb.Trainer(eng, params, y)
        tr.boost(3)
        runs.append((tr.trees(), tr.margins()))
    (ta, ma), (tb, mb) = runs
    for a, b in zip(ta, tb):
        for key in a:
            assert np.array_equal(a[key], b[key]), key
    assert np.array_equal(ma.view(np.uint32), mb.view(np.uint32))


def test_pipelined_rounds_with_rows_beyond_the_vector_range():
    """Rows whose logistic margin is beyond the vector kernel's range (|m| >
    80), and a tail of n % 8 rows, take the scalar sigmoid
    (simd/mod.rs:425-427) on the device. Pipelined rounds (device-decided
    trees, the next round's gradients in the margin walk) equal, bit for
    bit, rounds decided by the host level by level."""
    import os
    rng = np.random.default_rng(11)
    n, f = 20_003, 8
    x = rng.standard_normal((n, f)).astype(np.float32)
    y = (x[:, 0] + 0.5 * x[:, 1] > 0).astype(np.float32)
    m0 = np.zeros(n, np.float32)
    far = rng.choice(n, 200, replace=False)
    m0[far] = np.where(rng.random(200) < 0.5, -100.0, 100.0).astype(np.float32)
    params = {"objective": "binary:logistic", "max_depth": 4, "eta": 0.5}
    index = hb.DMatrix(x, label=y).index(256)
    runs = []
    for flag in (None, "0"):
        old = os.environ.pop("HBROCM_DEVICE_GROW", None)
        if flag is not None:
            os.environ["HBROCM_DEVICE_GROW"] = flag
        try:
            eng = hb.Engine(index, 0)
        finally:
            os.environ.pop("HBROCM_DEVICE_GROW", None)
            if old is not None:
                os.environ["HBROCM_DEVICE_GROW"] = old
        tr = hb.Trainer(eng, params, y)
        eng.load_margins(m0)
        eng.gradients(LOSS_LOGISTIC, y)  # labels back on the device after the margins
        tr.boost(3)
        runs.append((tr.trees(), tr.margins()))
    (ta, ma), (tb, mb) = runs
    assert len(ta) == len(tb) == 3
    for a, b in zip(ta, tb):
        for key in a:
            assert np.array_equal(a[key], b[key]), key
    assert np.array_equal(ma.view(np.uint32), mb.view(np.uint32))
    assert np.all(np.abs(ma[far]) > 80)


@pytest.mark.parametrize("far_rows", [False, True])
def test_row_carried_logistic_pairs_give_identical_trees(far_rows):
    """Unit-weight logistic with labels 0 and 1 on rows of at most 28
    features: the rows carry p and y in their padding and the histograms
    derive (g, h) from them, and the margin walk sums the next root's
    histogram as it computes the pairs (the exponents are the loss's bounds,
    known in advance). The trees and margins equal, bit for bit, those grown
    with the root built by the histogram kernel (HBROCM_FUSED_ROOT=0) and
    from the pair array (HBROCM_ROW_PAIRS=0), with rows beyond the vector
    range (deferred to the scalar finish, whose rows the root fix-up sums)
    or without; the root's byte count shows which pair path ran (a 4-byte
    word against an 8-byte pair per row), the kernel statistics that the
    fused walk ran."""
    import os
    rng = np.random.default_rng(23)
    n, f = 50_003, 20
    x = rng.standard_normal((n, f)).astype(np.float32)
    x[:, 3] = np.round(x[:, 3])
    y = (x[:, 0] + 0.5 * x[:, 3] * x[:, 1] + 0.3 * rng.standard_normal(n) > 0).astype(np.float32)
    m0 = np.zeros(n, np.float32)
    far = rng.choice(n, 300, replace=False)
    m0[far] = np.where(rng.random(300) < 0.5, -100.0, 100.0).astype(np.float32)
    params = {"objective": "binary:logistic", "max_depth": 6, "eta": 0.3}
    index = hb.DMatrix(x, label=y).index(256)
    runs = []
    for env in ({}, {"HBROCM_FUSED_ROOT": "0"}, {"HBROCM_ROW_PAIRS": "0"}):
        saved = {k: os.environ.pop(k, None) for k in ("HBROCM_ROW_PAIRS", "HBROCM_FUSED_ROOT")}
        os.environ.update(env)
        try:
            eng = hb.Engine(index, 0)
        finally:
            for k, v in saved.items():
                os.environ.pop(k, None)
                if v is not None:
                    os.environ[k] = v
        tr = hb.Trainer(eng, params, y)
        if far_rows:
            eng.load_margins(m0)
            eng.gradients(LOSS_LOGISTIC, y)
        before = eng.counters()
        tr.boost(1)
        after = eng.counters()
        per_row = (after["hist_bytes"] - before["hist_bytes"]) / (after["hist_rows"] - before["hist_rows"])
        eng.set_profiling(True, "hbr_walk_grad")
        tr.boost(3)
        fused = sum(n for k, (_, _, n) in eng.kernel_stats().items() if k == "hbr_walk_grad_root")
        eng.set_profiling(False)
        runs.append((tr.trees(), tr.margins(), per_row, fused))
    (ta, ma, ra, fa), (tb, mb, rb, fb), (tc, mc, rc, fc) = runs
    assert fa == 3 and fb == 0 and fc == 0, (fa, fb, fc)
    assert ra == rb and rc - ra == 4, (ra, rb, rc)  # the 4-byte word, then the 8-byte pair per row
    for other, mo in ((tb, mb), (tc, mc)):
        for a, b in zip(ta, other):
            for key in a:
                assert np.array_equal(a[key], b[key]), key
        assert np.array_equal(ma.view(np.uint32), mo.view(np.uint32))
    if far_rows:
        assert np.all(np.abs(ma[far]) > 80)


def _engine_with_env(index, env):
    import os
    saved = {k: os.environ.pop(k, None) for k in env}
    os.environ.update(env)
    try:
        return hb.Engine(index, 0)
    finally:
        for k, v in saved.items():
            os.environ.pop(k, None)
            if v is not None:
                os.environ[k] = v


@pytest.mark.parametrize("missing", [False, True])
def test_28_feature_instances_equal_the_32_column_ones(missing):
    """Rows of 25 to 28 features take histogram and fused-walk instances whose
    lanes rotate over the features alone (no atomics into padding columns):
    the trees and margins equal those of the 32-column instances
    (HBROCM_HIST_NF28=0) bit for bit, on dense and on masked rows, and the
    kernel statistics show which instances ran."""
    x, y = synthetic.higgs_like(n=70_000, seed=12)
    if missing:
        rng = np.random.default_rng(12)
        x[rng.random(x.shape) < 0.02] = np.nan
    params = {"objective": "binary:logistic", "max_depth": 7, "eta": 0.3}
    index = hb.DMatrix(x, label=y).index(256)
    runs = []
    for env in ({}, {"HBROCM_HIST_NF28": "0"}):
        eng = _engine_with_env(index, env)
        tr = hb.Trainer(eng, params, y)
        eng.set_profiling(True, "hbr_")
        tr.boost(3)
        names = set(eng.kernel_stats())
        eng.set_profiling(False)
        runs.append((tr.trees(), tr.margins(), names))
    (ta, ma, na), (tb, mb, nb) = runs
    want = "hbr_hist_dense8_fg32_bm_masked_nf28" if missing else "hbr_hist_dense8_fg32_bm_nf28"
    assert want in na and want not in nb, (na, nb)
    if not missing:
        assert "hbr_walk_grad_root_nf28" in na and "hbr_walk_grad_root" in nb
    for a, b in zip(ta, tb):
        for key in a:
            assert np.array_equal(a[key], b[key]), key
    assert np.array_equal(ma.view(np.uint32), mb.view(np.uint32))


@pytest.mark.parametrize("case", ["fused_root", "weights", "no_fused_root", "every_round"])
def test_rows_reordered_by_a_tree_give_identical_trees(case):
    """The whole-round trainer holds the rows in the order of its first
    tree's leaves (every later sum is an integer sum), while the logistic
    8-row vectors stay those of the original rows: a row beyond the vector
    range (|m| > 80) sends the other rows of its original vector to the
    scalar sigmoid (hbr_regroup, which also takes their vector pairs back
    out of the fused root histogram), and the tail of n % 8 rows stays
    scalar. The trees and margins equal, bit for bit, those of the run
    without the reorder; between two boosts, a call of the engine's own puts
    the rows back in their order and the next boost reorders them again
    (every_round: reordered again by each tree, the orders composed)."""
    rng = np.random.default_rng(29)
    n, f = 50_003, 20
    x = rng.standard_normal((n, f)).astype(np.float32)
    x[:, 3] = np.round(x[:, 3])
    y = (x[:, 0] + 0.5 * x[:, 3] * x[:, 1] + 0.3 * rng.standard_normal(n) > 0).astype(np.float32)
    w = rng.uniform(0.5, 2.0, n).astype(np.float32) if case == "weights" else None
    m0 = np.zeros(n, np.float32)
    far = rng.choice(n, 300, replace=False)
    m0[far] = np.where(rng.random(300) < 0.5, -100.0, 100.0).astype(np.float32)
    params = {"objective": "binary:logistic", "max_depth": 6, "eta": 0.3}
    index = hb.DMatrix(x, label=y).index(256)
    extra = {"HBROCM_FUSED_ROOT": "0"} if case == "no_fused_root" else {}
    every = {"HBROCM_ROW_ORDER_EVERY": "1"} if case == "every_round" else {}
    runs = []
    for env in ({"HBROCM_ROW_ORDER_MIN_ROWS": "1", **every}, {"HBROCM_ROW_ORDER": "0"}):
        eng = _engine_with_env(index, {**env, **extra})
        tr = hb.Trainer(eng, params, y, w)
        eng.load_margins(m0)
        eng.gradients(LOSS_LOGISTIC, y, w)
        eng.set_profiling(True, "hbr_")
        tr.boost(2)
        mid = tr.margins()
        back = eng.read_margins(n)  # the engine's own call: the rows in their order again
        tr.boost(2)
        stats = eng.kernel_stats()
        eng.set_profiling(False)
        count = lambda k: stats[k][2] if k in stats else 0
        assert eng.counters()["row_orders"] == count("hbr_order_place")
        runs.append((tr.trees(), tr.margins(), mid, back, count("hbr_regroup"), count("hbr_walk_grad_root"),
                     count("hbr_order_place")))
    (ta, ma, mida, backa, ra, fa, oa), (tb, mb, midb, backb, rb, fb, ob) = runs
    assert ra == 4 and rb == 0, (ra, rb)
    assert oa == (4 if case == "every_round" else 2) and ob == 0, (oa, ob)
    assert fa == fb == (0 if case in ("weights", "no_fused_root") else 4), (fa, fb)
    assert len(ta) == len(tb) == 4
    for a, b in zip(ta, tb):
        for key in a:
            assert np.array_equal(a[key], b[key]), key
    for u, v in ((ma, mb), (mida, midb), (backa, backb), (mida, backa)):
        assert np.array_equal(u.view(np.uint32), v.view(np.uint32))
    assert np.all(np.abs(ma[far]) > 80)


@pytest.mark.parametrize("objective,device_grow", [("binary:logistic", "1"), ("reg:squarederror", "1"),
                                                   ("binary:logistic", "0")])
def test_missing_values_on_masked_dense_rows_match_oracle_and_csr_path(objective, device_grow):
    """A matrix of 28 features with 2% missing cells trains on the masked
    dense rows (bins plus a missing mask per row: the histogram kernel skips
    masked cells, the margin walks send them the default way): the oracle's
    trees, and the CSR path's (HBROCM_MASKED_ROWS=0) trees and margins bit
    for bit, with the levels decided on the device and on the host."""
    import os
    x, y = synthetic.higgs_like(n=40_000, seed=4)
    rng = np.random.default_rng(4)
    x[rng.random(x.shape) < 0.02] = np.nan
    if objective == "reg:squarederror":
        y = (np.nan_to_num(x[:, 0]) + 0.5 * np.nan_to_num(x[:, 5]) + y).astype(np.float32)
    params = {"objective": objective, "max_depth": 6, "eta": 0.3}
    ref = O.Model(O.Dataset(x), y, O.params(objective=O.OBJ_LOGISTIC if objective != "reg:squarederror"
                                            else O.OBJ_SQUARED_ERROR, max_depth=6, eta=0.3), 4)
    runs = []
    for masked in ("1", "0"):
        saved = {k: os.environ.pop(k, None) for k in ("HBROCM_MASKED_ROWS", "HBROCM_DEVICE_GROW")}
        os.environ.update({"HBROCM_MASKED_ROWS": masked, "HBROCM_DEVICE_GROW": device_grow})
        try:
            eng = hb.DMatrix(x, label=y).engine(256)
            info = eng.index_info()
            tr = hb.Trainer(eng, params, y)
            tr.boost(4)
        finally:
            for k, v in saved.items():
                os.environ.pop(k, None)
                if v is not None:
                    os.environ[k] = v
        assert info["dense_u8"] == (1 if masked == "1" else 0) and info["dense"] == 0
        runs.append((tr.trees(), tr.margins()))
    compare_trees(runs[0][0], ref.trees())
    for a, b in zip(runs[0][0], runs[1][0]):
        for key in a:
            assert np.array_equal(a[key], b[key]), key
    assert np.array_equal(runs[0][1].view(np.uint32), runs[1][1].view(np.uint32))
    assert np.max(np.abs(runs[0][1] - ref.margins())) <= 1e-5


def _masked_and_csr_runs(x, y, params, rounds, device_grow="1"):
    """Trees, margins and index info of the masked dense rows and of the CSR
    path (HBROCM_MASKED_ROWS=0) for the same data."""
    import os
    runs = []
    for masked in ("1", "0"):
        saved = {k: os.environ.pop(k, None) for k in ("HBROCM_MASKED_ROWS", "HBROCM_DEVICE_GROW")}
        os.environ.update({"HBROCM_MASKED_ROWS": masked, "HBROCM_DEVICE_GROW": device_grow})
        try:
            eng = hb.DMatrix(x, label=y).engine(256)
            info = eng.index_info()
            tr = hb.Trainer(eng, params, y)
            tr.boost(rounds)
        finally:
            for k, v in saved.items():
                os.environ.pop(k, None)
                if v is not None:
                    os.environ[k] = v
        runs.append((tr.trees(), tr.margins(), info))
    return runs


@pytest.mark.parametrize("n_features,objective,device_grow", [
    (50, "binary:logistic", "1"), (50, "reg:squarederror", "1"), (50, "multi:softprob", "1"),
    (30, "binary:logistic", "0"), (97, "reg:squarederror", "1"), (256, "binary:logistic", "1")])
def test_missing_values_on_wide_masked_rows_match_oracle_and_csr_path(n_features, objective, device_grow):
    """Wider than 28 features, a matrix with 2% missing cells still trains
    on masked dense rows: G = ceil(F / 32) groups of 32 bins, then a 32-byte
    chunk of one mask word per group (row stride 32 G + 32). The oracle's
    trees, and the CSR path's trees and margins bit for bit, with the levels
    decided on the device and on the host."""
    k = 4 if objective == "multi:softprob" else 1
    x, y = synthetic.multiclass(n=20_000, f=n_features, k=max(k, 2), seed=n_features)
    reg, _ = synthetic.regression_100k(n=20_000, f=n_features, seed=n_features)
    rng = np.random.default_rng(7)
    x[rng.random(x.shape) < 0.02] = np.nan
    if objective == "reg:squarederror":
        y = (2 * np.nan_to_num(x[:, 0]) - np.nan_to_num(x[:, n_features - 1]) + 0.1 * reg[:, 1]).astype(np.float32)
    elif objective == "binary:logistic":
        y = ((np.nan_to_num(x[:, 3]) + np.nan_to_num(x[:, n_features - 2]) + 0.5 * reg[:, 2]) > 0).astype(np.float32)
    params = {"objective": objective, "max_depth": 6, "eta": 0.3}
    if k > 1:
        params["num_class"] = k
    obj = {"binary:logistic": O.OBJ_LOGISTIC, "reg:squarederror": O.OBJ_SQUARED_ERROR,
           "multi:softprob": O.OBJ_SOFTMAX}[objective]
    ref = O.Model(O.Dataset(x), y, O.params(objective=obj, num_class=k, max_depth=6, eta=0.3), 3)
    (tm, mm, im), (tc, mc, ic) = _masked_and_csr_runs(x, y, params, 3, device_grow)
    groups = (n_features + 31) // 32
    assert im["dense_u8"] == 1 and im["dense"] == 0
    assert im["stride"] == (32 if n_features <= 28 else 32 * groups + 32), im
    assert ic["dense_u8"] == 0
    compare_trees(tm, ref.trees())
    for a, b in zip(tm, tc):
        for key in a:
            assert np.array_equal(a[key], b[key]), key
    assert np.array_equal(mm.view(np.uint32), mc.view(np.uint32))
    assert np.max(np.abs(mm - ref.margins().reshape(mm.shape))) <= 1e-5


@pytest.mark.parametrize("max_bin,objective,kernel", [(512, "binary:logistic", "hbr_hist_dense16_fg16"),
                                                      (1024, "reg:squarederror", "hbr_hist_dense16_fg8"),
                                                      (3000, "reg:squarederror", "hbr_hist_dense16_fg2")])
def test_features_of_more_than_256_bins_train_on_u16_rows(max_bin, objective, kernel):
    """A dense matrix whose features take more than 256 bins (max_bin 512,
    1024, 3000; local bins u16 as in GHistIndex's columns) builds its
    histograms from rows of u16 local bins, 16, 8 or 2 features per
    workgroup: the oracle's trees, and the CSR path's
    (HBROCM_WIDE_ROWS=0) trees and margins bit for bit."""
    import os
    x, y = synthetic.regression_100k(n=30_000, f=21, seed=max_bin)
    x[:, 5] = np.round(x[:, 5] * 3)  # a feature of few bins beside the wide ones
    if objective == "binary:logistic":
        y = (y > 0).astype(np.float32)
    params = {"objective": objective, "max_depth": 6, "eta": 0.3, "max_bin": max_bin}
    obj = O.OBJ_LOGISTIC if objective == "binary:logistic" else O.OBJ_SQUARED_ERROR
    ref = O.Model(O.Dataset(x, max_bin=max_bin), y, O.params(objective=obj, max_depth=6, eta=0.3, max_bin=max_bin), 3)
    runs = []
    for wide in ("1", "0"):
        saved = os.environ.pop("HBROCM_WIDE_ROWS", None)
        os.environ["HBROCM_WIDE_ROWS"] = wide
        try:
            eng = hb.DMatrix(x, label=y).engine(max_bin)
            eng.set_profiling(True, "hbr_hist")
            tr = hb.Trainer(eng, params, y)
            tr.boost(3)
            launched = set(eng.kernel_stats())
            eng.set_profiling(False)
        finally:
            os.environ.pop("HBROCM_WIDE_ROWS", None)
            if saved is not None:
                os.environ["HBROCM_WIDE_ROWS"] = saved
        assert (kernel in launched) == (wide == "1"), launched
        runs.append((tr.trees(), tr.margins()))
    compare_trees(runs[0][0], ref.trees())
    for a, b in zip(runs[0][0], runs[1][0]):
        for key in a:
            assert np.array_equal(a[key], b[key]), key
    assert np.array_equal(runs[0][1].view(np.uint32), runs[1][1].view(np.uint32))
    assert np.max(np.abs(runs[0][1] - ref.margins())) <= 1e-5


@pytest.mark.parametrize("objective,f,depth", [("binary:logistic", 40, 7), ("reg:squarederror", 33, 6),
                                               ("binary:logistic", 20, 11)])
def test_device_rounds_on_wide_rows_and_deep_trees(objective, f, depth):
    """Depthwise rounds decided on the device for rows wider than 32 bytes
    or trees deeper than the fused walk takes (depth 11): the tree's leaves
    walked onto the margins on any row layout, then the next gradients, all
    queued ahead of the host: the host-decided rounds' trees, margins and
    eval-set margins bit for bit (HBROCM_DEVICE_GROW=0), and the oracle's
    trees."""
    import os
    x, y = synthetic.regression_100k(n=25_000, f=f, seed=f + depth)
    if objective == "binary:logistic":
        y = (y > 0).astype(np.float32)
    xe = synthetic.regression_100k(n=3_000, f=f, seed=99)[0]
    params = {"objective": objective, "max_depth": depth, "eta": 0.3}
    obj = O.OBJ_LOGISTIC if objective == "binary:logistic" else O.OBJ_SQUARED_ERROR
    ref = O.Model(O.Dataset(x), y, O.params(objective=obj, max_depth=depth, eta=0.3), 4)
    runs = []
    for grow in ("1", "0"):
        saved = os.environ.pop("HBROCM_DEVICE_GROW", None)
        os.environ["HBROCM_DEVICE_GROW"] = grow
        try:
            eng = hb.DMatrix(x, label=y).engine(256)
            eng.set_profiling(True, "hbr_")
            tr = hb.Trainer(eng, params, y)
            ev = tr.add_eval(hb.DMatrix(xe))
            tr.boost(4)
            launched = set(eng.kernel_stats())
            eng.set_profiling(False)
        finally:
            os.environ.pop("HBROCM_DEVICE_GROW", None)
            if saved is not None:
                os.environ["HBROCM_DEVICE_GROW"] = saved
        assert ("hbr_grow_decide" in launched) == (grow == "1"), launched
        if grow == "1":  # the walk of any layout, then the gradient pass
            assert "hbr_walk_leaves" in launched and "hbr_gradients" in launched, launched
            assert not any(k.startswith("hbr_walk_grad") for k in launched), launched
        runs.append((tr.trees(), tr.margins(), tr.eval_margins(ev)))
    compare_trees(runs[0][0], ref.trees())
    for a, b in zip(runs[0][0], runs[1][0]):
        for key in a:
            assert np.array_equal(a[key], b[key]), key
    assert np.array_equal(runs[0][1].view(np.uint32), runs[1][1].view(np.uint32))
    assert np.array_equal(runs[0][2].view(np.uint32), runs[1][2].view(np.uint32))
    assert np.max(np.abs(runs[0][1] - ref.margins())) <= 1e-5


def test_u16_rows_softmax_lossguide_and_weights_match_oracle():
    """The u16 rows under the other growth paths: 3-class softmax
    (per-class pairs), loss-guided growth with sample weights, both at
    max_bin 700, against the oracle."""
    x, y = synthetic.multiclass(n=12_000, f=9, k=3, seed=12)
    params = {"objective": "multi:softprob", "num_class": 3, "max_depth": 5, "eta": 0.3, "max_bin": 700}
    ref = O.Model(O.Dataset(x, max_bin=700), y, O.params(objective=O.OBJ_SOFTMAX, num_class=3, max_depth=5,
                                                         max_bin=700), 2)
    eng = hb.DMatrix(x, label=y).engine(700)
    eng.set_profiling(True, "hbr_hist")
    tr = hb.Trainer(eng, params, y)
    tr.boost(2)
    assert "hbr_hist_dense16_fg8" in eng.kernel_stats()
    compare_trees(tr.trees(), ref.trees())
    x, y = synthetic.regression_100k(n=15_000, f=7, seed=13)
    w = np.random.default_rng(13).random(len(y)).astype(np.float32) + 0.25
    params = {"grow_policy": "lossguide", "max_depth": 0, "max_leaves": 40, "eta": 0.3, "max_bin": 700}
    ref = O.Model(O.Dataset(x, max_bin=700, weights=w), y,
                  O.params(grow_policy=O.GROW_LOSSGUIDE, max_depth=0, max_leaves=40, max_bin=700), 3, weights=w)
    model = hb.train(params, hb.DMatrix(x, label=y, weight=w), 3)
    compare_trees(model.trees, ref.trees())
    assert np.max(np.abs(model.predict(x, output_margin=True) - ref.margins())) <= 1e-5


@pytest.mark.parametrize("leaves", [3, 6, 14])
def test_lossguide_with_equal_gains_matches_oracle(leaves):
    """Mirrored rows give every node below the root a twin of equal loss
    change, and the leaf budgets cut between twins: the device-side
    loss-guided growth breaks the ties as the oracle's restatement of the
    reference's BinaryHeap does, for two rounds (the second round's
    gradients are mirrored too)."""
    from tests.test_oracle import _mirrored_data
    x, gp = _mirrored_data(4)
    y = -gp[:, 0]
    params = {"grow_policy": "lossguide", "max_depth": 0, "max_leaves": leaves, "eta": 0.3, "max_bin": 64,
              "base_score": 0.0}
    ref = O.Model(O.Dataset(x, max_bin=64), y, O.params(grow_policy=O.GROW_LOSSGUIDE, max_depth=0, max_leaves=leaves,
                                                        eta=0.3, max_bin=64, base_score=0.0), 2)
    model = hb.train(params, hb.DMatrix(x, label=y), 2)
    compare_trees(model.trees, ref.trees())
    assert np.max(np.abs(model.predict(x, output_margin=True) - ref.margins())) <= 1e-5
