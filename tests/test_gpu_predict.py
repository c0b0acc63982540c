"""GPU batch prediction against the reference's recorded margins and the oracle."""
import numpy as np
import pytest

import hessboost_amd as hb
from hessboost_amd import synthetic
from oracle import oracle as O
from tests.helpers import categorical_features, four_features, golden_forest, load_saved_models, random_tree

pytestmark = pytest.mark.gpu

CASES = ["early_stopping", "dart", "multiclass_forest", "quantiles", "expectiles", "aft", "dist_normal",
         "dist_negbinomial", "multi_target", "categorical_splits"]


def rows_for(name):
    """The rows each saved model's margins were recorded on (the categorical
    case's column 0 holds category codes)."""
    return categorical_features() if name == "categorical_splits" else four_features()


@pytest.mark.parametrize("name", CASES)
def test_saved_models_reproduce_recorded_margins(name):
    """tests/native_format.rs:822-860: recorded f32 margins, bit for bit."""
    saved = load_saved_models()
    x = rows_for(name)
    for ver in ("0.2.0", "0.4.3", "0.4.9"):
        case = saved[f"{ver}/{name}"]
        arrs = golden_forest(case)
        f = hb.Forest(arrs, case["n_outputs"])
        got = f.predict_margin(x)
        assert np.array_equal(got.view(np.uint32), np.array(case["margins"], np.uint32)), f"{ver}/{name}"


@pytest.mark.parametrize("name", CASES)
def test_reference_json_models_predict_recorded_margins(name):
    """The reference's saved JSON models (tests/golden/models, read with
    Booster.load_model_json) predict the recorded f32 margins bit for bit."""
    import os
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "models", name + ".json")
    b = hb.Booster.load_model_json(open(path).read())
    got = b.predict(rows_for(name), output_margin=True)
    want = np.array(load_saved_models()[f"0.4.9/{name}"]["margins"], np.uint32)
    assert np.array_equal(np.asarray(got, np.float32).reshape(-1).view(np.uint32), want)


@pytest.mark.parametrize("ver", ["0.2.0", "0.4.3", "0.4.9"])
def test_reference_native_models_predict_recorded_margins(ver):
    """The reference's saved native binary files (zstd frames of the HBM
    container, tests/golden/native) load with Booster.load_model and
    predict the recorded f32 margins bit for bit on the GPU."""
    import os
    for name in CASES:
        path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "native", ver, name + ".bin")
        b = hb.Booster(objective="reg:squarederror", base_score=np.zeros(1, np.float32)).load_model(path)
        got = b.predict(rows_for(name), output_margin=True)
        want = np.array(load_saved_models()[f"{ver}/{name}"]["margins"], np.uint32)
        assert np.array_equal(np.asarray(got, np.float32).reshape(-1).view(np.uint32), want), name


def test_trained_model_survives_native_round_trip(tmp_path):
    """A trained model written in the native binary format and read back
    predicts the same margins bit for bit; its container re-saves byte for
    byte."""
    from hessboost_amd import native_model as N
    x = synthetic.predict_rows(n=5_000, f=9, seed=13)
    y = (np.nan_to_num(x[:, 0]) > 0).astype(np.float32)
    for params in ({"objective": "binary:logistic", "max_depth": 5, "scale_pos_weight": 2.0},
                   {"objective": "reg:squarederror", "grow_policy": "lossguide", "max_depth": 0, "max_leaves": 12}):
        model = hb.train(params, hb.DMatrix(x, label=y), 4)
        model.save_model(tmp_path / "m.bin")
        back = hb.Booster(objective="reg:squarederror", base_score=np.zeros(1, np.float32)).load_model(
            tmp_path / "m.bin")
        assert N.container(back) == N.container(model)
        a = model.predict(x, output_margin=True)
        c = back.predict(x, output_margin=True)
        assert np.array_equal(np.asarray(a).view(np.uint32), np.asarray(c).view(np.uint32)), params


def test_categorical_casts_saturate_and_missing_follows_default():
    """src/backend/cuda/predict.rs:702-724: the set {0, 2, u32::MAX}; rows
    -2.5, -0.0, 0.8, 1.9, 2.9, 2^32 and NaN, on the GPU as in the oracle,
    for both default directions and a non-NaN missing marker."""
    x = np.array([[-2.5], [-0.0], [0.8], [1.9], [2.9], [4294967296.0], [np.nan], [np.inf], [-np.inf],
                  [4294967040.0], [3.0]], np.float32)
    for dl in (0, 1):
        for missing in (np.nan, 3.0):
            arrs = O.forest_arrays([[dict(split_feature=0, split_cond=0.0, default_left=bool(dl), left=1, right=2,
                                          leaf_value=1.0),
                                     dict(split_feature=0, split_cond=0.0, default_left=True, left=-1, right=-1,
                                          leaf_value=0.25),
                                     dict(split_feature=0, split_cond=0.0, default_left=True, left=-1, right=-1,
                                          leaf_value=-0.75)]])
            arrs.update(is_categorical=np.array([1, 0, 0], np.uint8), cat_begin=np.array([0, 0, 0], np.uint32),
                        cat_end=np.array([3, 0, 0], np.uint32), categories=np.array([0, 2, 2**32 - 1], np.uint32))
            want = O.predict_margin(arrs, x, missing=missing)
            got = hb.Forest(arrs, 1).predict_margin(x, missing)
            np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_random_categorical_forests_match_oracle():
    """Unbalanced random trees mixing numeric and categorical splits (sets of
    up to 70 categories from 0..99), several outputs, category codes with
    fractions, negatives and missing values; margins and leaf ids."""
    rng = np.random.default_rng(31)
    f, k = 6, 3
    trees, pool = [], []
    for t in range(40):
        nodes = [dict(leaf_value=float(rng.standard_normal()))]
        for _ in range(int(rng.integers(0, 30))):
            i = int(rng.choice([j for j, nd in enumerate(nodes) if "left" not in nd]))
            nodes[i].update(left=len(nodes), right=len(nodes) + 1, split_feature=int(rng.integers(0, f)),
                            split_cond=float(np.float32(rng.standard_normal() * 20)),
                            default_left=bool(rng.random() < 0.5), is_categorical=bool(rng.random() < 0.5))
            nodes += [dict(leaf_value=float(rng.standard_normal())), dict(leaf_value=float(rng.standard_normal()))]
        for nd in nodes:
            for key, v in (("left", -1), ("right", -1), ("split_feature", 0), ("split_cond", 0.0),
                           ("default_left", True), ("is_categorical", False)):
                nd.setdefault(key, v)
            if nd["is_categorical"]:
                cats = rng.choice(100, size=int(rng.integers(1, 71)), replace=False)
                nd["cat_begin"], nd["cat_end"] = len(pool), len(pool) + len(cats)
                pool.extend(int(c) for c in cats)
            else:
                nd["cat_begin"] = nd["cat_end"] = 0
        trees.append(nodes)
    arrs = O.forest_arrays(trees, tree_output=[t % k for t in range(len(trees))], n_outputs=k,
                           base_score=[0.5, -0.5, 0.0])
    flat = [nd for nodes in trees for nd in nodes]
    arrs.update(is_categorical=np.array([nd["is_categorical"] for nd in flat], np.uint8),
                cat_begin=np.array([nd["cat_begin"] for nd in flat], np.uint32),
                cat_end=np.array([nd["cat_end"] for nd in flat], np.uint32), categories=np.array(pool, np.uint32))
    x = (rng.integers(-5, 110, (20_000, f)) + rng.choice([0.0, 0.25, 0.99], (20_000, f))).astype(np.float32)
    x[rng.random(x.shape) < 0.05] = np.nan
    want, want_leaf = O.predict_margin(arrs, x, with_leaf=True)
    forest = hb.Forest(arrs, k)
    np.testing.assert_array_equal(forest.predict_margin(x).reshape(-1).view(np.uint32), want.view(np.uint32))
    np.testing.assert_array_equal(forest.predict_leaf(x).reshape(want_leaf.shape), want_leaf)


def test_trained_model_survives_json_round_trip():
    x = synthetic.predict_rows(n=5_000, f=9, seed=12)
    y = (np.nan_to_num(x[:, 0]) > 0).astype(np.float32) + (np.nan_to_num(x[:, 1]) > 0.5).astype(np.float32)
    for params in ({"objective": "binary:logistic", "max_depth": 5, "scale_pos_weight": 2.0},
                   {"objective": "multi:softprob", "num_class": 3, "max_depth": 4},
                   {"objective": "reg:squarederror", "grow_policy": "lossguide", "max_depth": 0, "max_leaves": 12}):
        yy = (y > 0).astype(np.float32) if params["objective"] == "binary:logistic" else y
        model = hb.train(params, hb.DMatrix(x, label=yy), 4)
        back = hb.Booster.load_model_json(model.save_model_json())
        a = model.predict(x, output_margin=True)
        c = back.predict(x, output_margin=True)
        assert np.array_equal(np.asarray(a).view(np.uint32), np.asarray(c).view(np.uint32)), params


def test_synthetic_forest_leaves_and_margins_match_oracle():
    trees = synthetic.forest(n_trees=50, depth=8, n_features=100, seed=7)
    x = synthetic.predict_rows(n=20_000, f=100, seed=8)
    arrs = O.forest_arrays(trees)
    want, want_leaf = O.predict_margin(arrs, x, with_leaf=True)
    f = hb.Forest(arrs, 1)
    got = f.predict_margin(x)
    leaf = f.predict_leaf(x)
    assert np.array_equal(leaf, want_leaf)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_resident_and_chunked_walks_agree_with_the_oracle():
    """The rows-resident walk (the default: 16 trees in flight per lane,
    nodes through the caches) and the LDS-chunked walk: margins bit for bit
    with the oracle, leaves exact, on a ragged row count, a non-NaN missing
    value (with NaN, inf and -0 cells) and a multi-output forest."""
    import os
    trees = synthetic.forest(n_trees=37, depth=6, n_features=23, seed=9)
    x = synthetic.predict_rows(n=3_001, f=23, seed=10)
    arrs = O.forest_arrays(trees)
    want, want_leaf = O.predict_margin(arrs, x, with_leaf=True)
    x9 = np.where(np.isnan(x), np.float32(-9.0), x).astype(np.float32)
    x9[::97, 3] = np.nan  # NaN that is not the missing value: every comparison false, so right
    x9[::89, 5] = np.inf
    x9[::83, 7] = -0.0
    want9 = O.predict_margin(arrs, x9, missing=-9.0)
    multi = dict(arrs)
    multi["tree_output"] = (np.arange(len(trees)) % 3).astype(np.uint32)
    multi["n_outputs"] = 3
    multi["base_score"] = np.array([0.1, -0.2, 0.3], np.float32)
    want3 = O.predict_margin(multi, x)
    for kind in ("pairs", "mirror", "resident", "chunked", "staged", "generic"):
        os.environ["HBROCM_PRED_KERNEL"] = kind
        try:
            f = hb.Forest(arrs, 1)
            assert np.array_equal(f.predict_margin(x).view(np.uint32), want.view(np.uint32)), kind
            assert np.array_equal(f.predict_leaf(x), want_leaf), kind
            assert np.array_equal(f.predict_margin(x9, missing=-9.0).view(np.uint32), want9.view(np.uint32)), kind
            f3 = hb.Forest(multi, 3)
            assert np.array_equal(f3.predict_margin(x).view(np.uint32), want3.view(np.uint32)), kind
        finally:
            os.environ.pop("HBROCM_PRED_KERNEL", None)


def test_rows_start_from_their_own_margins_in_every_walk():
    """hbr_predict_margin_from: each row starts from its own margins (the
    reference's initial margins, a DMatrix's base_margin: plan_margins,
    backend/shared.rs:218-239) and adds the trees' weighted leaf values in
    tree order, as the f32 chain formed here from the oracle's leaf ids;
    starting margins equal to the base scores give the base-score call's bits."""
    import os
    trees = synthetic.forest(n_trees=41, depth=6, n_features=19, seed=21)
    x = synthetic.predict_rows(n=2_777, f=19, seed=22)
    rng = np.random.default_rng(23)
    for k in (1, 3):
        arrs = dict(O.forest_arrays(trees))
        arrs["tree_output"] = (np.arange(len(trees)) % k).astype(np.uint32)
        arrs["n_outputs"] = k
        arrs["base_score"] = np.linspace(-0.25, 0.5, k).astype(np.float32)
        arrs["tree_weight"] = rng.choice([1.0, 0.5, 0.3], len(trees)).astype(np.float32)
        _, leaf = O.predict_margin(arrs, x, with_leaf=True)
        init = (rng.standard_normal((len(x), k)) * 3).astype(np.float32)
        want = init.copy()
        lv = np.asarray(arrs["leaf_value"], np.float32)
        off = np.asarray(arrs["tree_offset"], np.int64)
        for t in range(len(trees)):
            o = arrs["tree_output"][t]
            contrib = (arrs["tree_weight"][t] * lv[off[t] + leaf[:, t]]).astype(np.float32)
            want[:, o] = (want[:, o] + contrib).astype(np.float32)
        base = np.broadcast_to(arrs["base_score"], (len(x), k))
        for kind in ("pairs", "mirror", "resident", "chunked", "staged", "generic"):
            os.environ["HBROCM_PRED_KERNEL"] = kind
            try:
                f = hb.Forest(arrs, k)
                got = f.predict_margin(x, init_margins=init)
                assert np.array_equal(got.view(np.uint32), want.reshape(-1).view(np.uint32)), (kind, k)
                plain = f.predict_margin(x)
                assert np.array_equal(f.predict_margin(x, init_margins=base).view(np.uint32),
                                      plain.view(np.uint32)), (kind, k)
            finally:
                os.environ.pop("HBROCM_PRED_KERNEL", None)


def test_host_rows_in_chunks_equal_device_rows():
    """Rows in host memory beyond two 128 MiB chunks go to the device in
    chunks (copied by the host's threads into two pinned staging buffers,
    then by a copy stream, while the walk runs on the chunks already there):
    the margins equal, bit for bit, those of the same rows already on the
    device and those of slices small enough for one plain copy, across the
    chunk boundaries, with and without starting margins, for one and three
    outputs (a row of 37 features: 906,816 rows a chunk, the last ragged)."""
    trees = synthetic.forest(n_trees=24, depth=8, n_features=37, seed=31)
    n = 2_000_003
    x = synthetic.predict_rows(n=n, f=37, seed=32)
    arrs = O.forest_arrays(trees)
    f = hb.Forest(arrs, 1)
    got = f.predict_margin(x)
    dx = hb.DeviceBuffer(x.nbytes)
    dx.upload(x)
    dout = hb.DeviceBuffer(4 * n)
    f.predict_margin_device(dx.ptr, n, 37, dout.ptr)
    assert np.array_equal(got.view(np.uint32), dout.download(np.float32, n).view(np.uint32))
    del dx, dout
    # rows of too few columns are refused at the first chunk (its copy
    # already queued); the next call starts clean
    if int(np.max(arrs["split_feature"])) >= 36:
        with pytest.raises(hb.HbrError):
            f.predict_margin(np.ascontiguousarray(x[:, :36]))
        assert np.array_equal(f.predict_margin(x).view(np.uint32), got.view(np.uint32))
    chunk = (128 << 20) // (37 * 4) // 64 * 64
    rng = np.random.default_rng(33)
    for k in (1, 3):
        multi = dict(arrs)
        multi["tree_output"] = (np.arange(len(trees)) % k).astype(np.uint32)
        multi["n_outputs"] = k
        multi["base_score"] = np.linspace(-0.5, 0.5, k).astype(np.float32)
        fk = hb.Forest(multi, k)
        init = rng.standard_normal((n, k)).astype(np.float32)
        whole = fk.predict_margin(x, init_margins=init).reshape(n, k)
        plain = fk.predict_margin(x).reshape(n, k)
        for a in (0, chunk - 1000, 2 * chunk - 1, n - 3000):
            b = min(n, a + 3000)
            part = fk.predict_margin(x[a:b], init_margins=init[a:b]).reshape(-1, k)
            assert np.array_equal(part.view(np.uint32), whole[a:b].view(np.uint32)), (k, a)
            part = fk.predict_margin(x[a:b]).reshape(-1, k)
            assert np.array_equal(part.view(np.uint32), plain[a:b].view(np.uint32)), (k, a)


def test_device_resident_prediction():
    trees = synthetic.forest(n_trees=20, depth=6, n_features=30, seed=9)
    x = synthetic.predict_rows(n=5_000, f=30, seed=10)
    arrs = O.forest_arrays(trees)
    want = O.predict_margin(arrs, x)
    f = hb.Forest(arrs, 1)
    dx = hb.DeviceBuffer(x.nbytes)
    dx.upload(x)
    dout = hb.DeviceBuffer(4 * len(x))
    f.predict_margin_device(dx.ptr, len(x), 30, dout.ptr)
    got = dout.download(np.float32, len(x))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_trained_model_predictions_match_training_margins():
    x, y = synthetic.regression_100k(n=5_000, f=8, seed=11)
    dm = hb.DMatrix(x, label=y)
    params = {"max_depth": 4}
    index = dm.index(256)
    eng = hb.Engine(index)
    t = hb.Trainer(eng, params, y)
    t.boost(5)
    model = t.booster(8)
    assert np.array_equal(model.predict(x, output_margin=True).view(np.uint32), t.margins().view(np.uint32))


@pytest.mark.parametrize("objective", ["binary:logistic", "multi:softprob", "multi:softmax"])
def test_booster_predict_transforms_margins_with_the_hosts_expf(objective):
    """Booster.predict: the margins from the GPU, then the objective's
    transform on the host (Transform::apply, model/transform.rs:74-104):
    XGBoost's sigmoid bit for bit as the oracle forms it with the C library's
    expf, softmax rows summed in f64, multi:softmax's first largest class."""
    import ctypes as C
    import ctypes.util
    libm = C.CDLL(ctypes.util.find_library("m"))
    libm.expf.restype, libm.expf.argtypes = C.c_float, [C.c_float]
    rng = np.random.default_rng(7)
    x = rng.standard_normal((3_000, 6)).astype(np.float32)
    if objective == "binary:logistic":
        y = (x[:, 0] + 0.5 * x[:, 1] > 0).astype(np.float32)
        params = {"objective": objective, "max_depth": 4}
    else:
        y = np.digitize(x[:, 0] + 0.3 * x[:, 2], [-0.5, 0.5]).astype(np.float32)
        params = {"objective": objective, "num_class": 3, "max_depth": 3}
    model = hb.train(params, hb.DMatrix(x, label=y), 4)
    m = model.predict(x, output_margin=True)
    p = model.predict(x)
    if objective == "binary:logistic":
        want = np.array([O.lib().or_sigmoid(float(v)) for v in m], np.float32)
        assert np.array_equal(p.view(np.uint32), want.view(np.uint32))
    elif objective == "multi:softprob":
        want = np.empty_like(m)
        for r, row in enumerate(m):
            e = [np.float32(libm.expf(float(np.float32(v - row.max())))) for v in row]
            s = np.float32(sum(float(v) for v in e))
            want[r] = [np.float32(v / s) for v in e]
        assert p.shape == m.shape and np.array_equal(p.view(np.uint32), want.view(np.uint32))
    else:
        assert p.shape == (len(x),) and np.array_equal(p, np.argmax(m, 1).astype(np.float32))


def test_malformed_forest_is_refused():
    arrs = O.forest_arrays([[dict(split_feature=0, split_cond=0.0, default_left=True, left=0, right=0,
                                  leaf_value=0.0)]])
    with pytest.raises(hb.HbrError):
        hb.Forest(arrs, 1)


@pytest.mark.parametrize("seed", range(12))
def test_random_forests_match_oracle(seed):
    """Random unbalanced forests (depth 0 to 12, several outputs, tree
    weights, NaN or a non-NaN missing value), every walk, bit for bit; the
    rows hold values equal to thresholds, signed zeros, infinities and (with
    a non-NaN missing value) present NaNs."""
    import os
    rng = np.random.default_rng(500 + seed)
    f = int(rng.integers(1, 40))
    n_trees = int(rng.integers(1, 90))
    k = int(rng.choice([1, 1, 3]))
    trees = [random_tree(rng, f, int(rng.integers(0, 13))) for _ in range(n_trees)]
    arrs = O.forest_arrays(trees)
    arrs["tree_output"] = (np.arange(n_trees) % k).astype(np.uint32)
    arrs["tree_weight"] = rng.uniform(0.5, 1.5, n_trees).astype(np.float32)
    arrs["n_outputs"] = k
    arrs["base_score"] = rng.normal(0, 1, k).astype(np.float32)
    n = int(rng.choice([1, 63, 64, 65, 2_049]))
    x = rng.standard_normal((n, f)).astype(np.float32)
    missing = np.nan if rng.random() < 0.6 else -7.0
    conds = arrs["split_cond"][arrs["left"] != -1]
    if len(conds):
        conds[: len(conds) // 4] = 0.0
        arrs["split_cond"][np.nonzero(arrs["left"] != -1)[0]] = conds
        hit = rng.random((n, f)) < 0.1
        x[hit] = rng.choice(conds, int(hit.sum()))
    x[rng.random((n, f)) < 0.03] = -0.0
    x[rng.random((n, f)) < 0.03] = 0.0
    x[rng.random((n, f)) < 0.02] = np.inf
    x[rng.random((n, f)) < 0.02] = -np.inf
    x[rng.random((n, f)) < 0.1] = missing
    if missing == missing:
        x[rng.random((n, f)) < 0.03] = np.nan
    want, want_leaf = O.predict_margin(arrs, x, missing=missing, with_leaf=True)
    for kind in ("pairs", "mirror", "resident", "chunked", "staged", "generic"):
        os.environ["HBROCM_PRED_KERNEL"] = kind
        try:
            fo = hb.Forest(arrs, k)
            got = fo.predict_margin(x, missing=missing)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (seed, kind)
            assert np.array_equal(fo.predict_leaf(x, missing=missing), want_leaf), (seed, kind)
        finally:
            os.environ.pop("HBROCM_PRED_KERNEL", None)
