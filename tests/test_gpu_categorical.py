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


def test_categorical_models_save_load_and_refuse_eval_sets(tmp_path):
    """A trained categorical model round-trips through the native format and
    predicts the same margins; an evaluation set on an index with
    categorical features is refused (the device's value walk does not route
    category sets), leaving the caller to score it by prediction."""
    x, y, types = categorical_data(4, 6_000, [8], "reg:squarederror")
    model = hb.train({"max_depth": 4}, hb.DMatrix(x, label=y, feature_types=types), 3)
    model.save_model(tmp_path / "cat.bin")
    back = hb.Booster(objective="reg:squarederror", base_score=np.zeros(1, np.float32)).load_model(tmp_path / "cat.bin")
    assert np.array_equal(back.predict(x, output_margin=True).view(np.uint32),
                          model.predict(x, output_margin=True).view(np.uint32))
    with pytest.raises(A.HbrError) as refused:
        hb.train({"max_depth": 4}, hb.DMatrix(x, label=y, feature_types=types), 1,
                 evals=[(hb.DMatrix(x, feature_types=types), "train")])
    assert refused.value.status == A.REFUSED
