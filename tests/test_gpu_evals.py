"""Evaluation sets on the device: after training, each eval set's margins are
the base score (or its base margin) plus every tree walked over its raw
rows, which the oracle's margin walk computes from the same trees
(or_predict_margin: base, then one f32 add per tree in order). Bit-exact,
for every growth path that grows the trees: the pipelined scalar losses
(guarded device walks), the batched and per-class softmax rounds, and the
host-driven growth (lossguide, CSR training input)."""
import numpy as np
import pytest

import hessboost_amd as hb
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def expected(booster, x, missing=np.nan, base_margin=None):
    k = booster.n_outputs
    arrs = O.forest_arrays(booster.trees, tree_output=[t % k for t in range(len(booster.trees))], n_outputs=k,
                           base_score=booster.base_score if base_margin is None else np.zeros(k))
    out = O.predict_margin(arrs, x, missing=missing).reshape(-1, k)
    if base_margin is not None:
        # base margin first, then the trees in order (the walk's order of adds)
        out = np.asarray(base_margin, np.float32).reshape(-1, k).copy()
        for t, tree in enumerate(booster.trees):
            one = O.forest_arrays([tree], tree_output=[t % k], n_outputs=k, base_score=np.zeros(k))
            out = (out + O.predict_margin(one, x, missing=missing).reshape(-1, k)).astype(np.float32)
    return out


def data(n, f, seed, objective="reg:squarederror", k=1, missing=0.0):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, f)).astype(np.float32)
    z = x[:, 0] - 0.5 * x[:, 1 % f] + np.sin(2 * x[:, 2 % f])
    if objective == "reg:squarederror":
        y = (z + 0.1 * rng.standard_normal(n)).astype(np.float32)
    elif objective == "binary:logistic":
        y = (rng.random(n) < 1 / (1 + np.exp(-2 * z))).astype(np.float32)
    else:
        y = np.clip(np.floor((z - z.min()) / (np.ptp(z) + 1e-9) * k), 0, k - 1).astype(np.float32)
    if missing > 0:
        x[rng.random((n, f)) < missing] = np.nan
    return x, y


def eval_matrix(n, f, seed):
    """Rows beyond the training range, infinities and missing values."""
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((n, f)) * 1.5).astype(np.float32)
    x[rng.random((n, f)) < 0.1] = np.nan
    x[0, :] = np.inf
    x[1, :] = -np.inf
    x[2, :] = 1e30
    x[3, :] = -1e30
    return x


CASES = [
    # name, params, n_features, training missing fraction
    ("pipelined squared error", {"objective": "reg:squarederror", "max_depth": 6}, 28, 0.0),
    ("pipelined logistic", {"objective": "binary:logistic", "max_depth": 5}, 20, 0.0),
    ("batched softmax", {"objective": "multi:softprob", "num_class": 3, "max_depth": 4}, 12, 0.0),
    ("lossguide", {"objective": "reg:squarederror", "grow_policy": "lossguide", "max_depth": 0,
                   "max_leaves": 17}, 10, 0.0),
    ("missing values in training", {"objective": "binary:logistic", "max_depth": 4}, 9, 0.2),
    ("wide rows", {"objective": "reg:squarederror", "max_depth": 7}, 40, 0.0),
    ("deep tree off LDS", {"objective": "reg:squarederror", "max_depth": 12, "min_child_weight": 0.0,
                           "lambda": 0.0}, 6, 0.0),
    ("rows wider than the staged walk", {"objective": "reg:squarederror", "max_depth": 5}, 70, 0.0),
]


def test_in_place_walk_matches_staged(monkeypatch):
    """The in-place walk (rows read from HBM per step) and the staged one
    (64-row blocks in LDS) give the same bits."""
    x, y = data(9_000, 28, 29, "binary:logistic")
    ev = eval_matrix(4_099, 28, 30)
    out = []
    for in_place in (False, True):
        if in_place:
            monkeypatch.setenv("HBROCM_EVAL_IN_PLACE", "1")
        model = hb.train({"objective": "binary:logistic", "max_depth": 6}, hb.DMatrix(x, label=y), 5,
                         evals=[(hb.DMatrix(ev), "e")])
        out.append(model.eval_margins["e"])
        np.testing.assert_array_equal(out[-1].view(np.uint32), expected(model, ev).view(np.uint32))
    np.testing.assert_array_equal(out[0].view(np.uint32), out[1].view(np.uint32))


@pytest.mark.parametrize("name,params,f,miss", CASES, ids=[c[0] for c in CASES])
def test_eval_margins_match_oracle_walk(name, params, f, miss):
    print("eval case", name, flush=True)
    k = params.get("num_class", 1)
    x, y = data(20_000, f, 7, params["objective"], k, miss)
    ev1 = eval_matrix(3_001, f, 8)
    ev2 = data(777, f, 9, params["objective"], k)[0]
    dtrain = hb.DMatrix(x, label=y)
    model = hb.train(dict(params, eta=0.3), dtrain, 6,
                     evals=[(hb.DMatrix(ev1), "a"), (hb.DMatrix(ev2), "b")])
    assert set(model.eval_margins) == {"a", "b"}
    if name == "deep tree off LDS":  # trees beyond the walk's LDS node table
        assert max(len(t["left"]) for t in model.trees) > 2048
    for ev, key in ((ev1, "a"), (ev2, "b")):
        got = model.eval_margins[key]
        want = expected(model, ev)
        assert got.shape == want.shape
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32), err_msg=f"{name} {key}")
        # and the product's own prediction of the same rows
        np.testing.assert_array_equal(got.reshape(-1), model.predict(ev, output_margin=True).reshape(-1))


def test_softmax_per_class_rounds(monkeypatch):
    monkeypatch.setenv("HBROCM_SOFTMAX_BATCH", "0")
    x, y = data(8_000, 10, 11, "multi:softprob", 4)
    ev = eval_matrix(1_500, 10, 12)
    model = hb.train({"objective": "multi:softprob", "num_class": 4, "max_depth": 5}, hb.DMatrix(x, label=y), 4,
                     evals=[(hb.DMatrix(ev), "e")])
    np.testing.assert_array_equal(model.eval_margins["e"].view(np.uint32), expected(model, ev).view(np.uint32))


def test_csr_training_input():
    x, y = data(6_000, 15, 13, "reg:squarederror", 1, 0.4)
    present = ~np.isnan(x)
    rp = np.zeros(x.shape[0] + 1, np.uint64)
    rp[1:] = np.cumsum(present.sum(1))
    rows, cols = np.nonzero(present)
    dtrain = hb.DMatrix((rp, cols.astype(np.uint32), x[rows, cols]), label=y, n_cols=15)
    ev = eval_matrix(900, 15, 14)
    model = hb.train({"objective": "reg:squarederror", "max_depth": 5}, dtrain, 5, evals=[(hb.DMatrix(ev), "e")])
    np.testing.assert_array_equal(model.eval_margins["e"].view(np.uint32), expected(model, ev).view(np.uint32))


def test_csr_eval_set_with_a_non_nan_marker_and_dmatrix_predict():
    """A CSR eval set's absent entries are its missing values whatever marker
    the DMatrix was given (DMatrix::from_csr keeps NaN as the marker and
    stores only finite values, src/data/dmatrix.rs:459-510), so explicit
    zeros stay present values; Booster.predict of a DMatrix reads the
    matrix's own marker (-999 here) instead of NaN."""
    x, y = data(6_000, 12, 33, "reg:squarederror", 1, 0.0)
    ev = eval_matrix(900, 12, 34)
    ev[np.isinf(ev)] = np.copysign(np.float32(3e38), ev[np.isinf(ev)])  # CSR stores finite values only
    ev[5:50, :4] = 0.0  # explicit zeros: present in CSR
    present = ~np.isnan(ev)
    rp = np.zeros(ev.shape[0] + 1, np.uint64)
    rp[1:] = np.cumsum(present.sum(1))
    rows, cols = np.nonzero(present)
    dcsr = hb.DMatrix((rp, cols.astype(np.uint32), ev[rows, cols]), n_cols=12, missing=0.0)
    model = hb.train({"objective": "reg:squarederror", "max_depth": 5}, hb.DMatrix(x, label=y), 4,
                     evals=[(dcsr, "csr")])
    np.testing.assert_array_equal(model.eval_margins["csr"].view(np.uint32), expected(model, ev).view(np.uint32))
    np.testing.assert_array_equal(model.predict(dcsr, output_margin=True).view(np.uint32),
                                  expected(model, ev).reshape(-1).view(np.uint32))
    marked = np.where(np.isnan(ev), np.float32(-999.0), ev).astype(np.float32)
    got = model.predict(hb.DMatrix(marked, missing=-999.0), output_margin=True)
    np.testing.assert_array_equal(got.view(np.uint32), expected(model, ev).reshape(-1).view(np.uint32))


def test_added_after_rounds_with_base_margin_and_missing_marker():
    """A set added after some rounds takes the trees already grown; a base
    margin replaces the base score; a non-NaN missing marker is honoured."""
    x, y = data(10_000, 16, 15, "binary:logistic")
    dtrain = hb.DMatrix(x, label=y)
    engine = dtrain.engine(256)
    t = hb.Trainer(engine, {"objective": "binary:logistic", "max_depth": 6}, y)
    ev = eval_matrix(2_000, 16, 16)
    ev[np.isnan(ev)] = -999.0
    bm = np.linspace(-1, 1, ev.shape[0], dtype=np.float32)
    first = t.add_eval(hb.DMatrix(ev, missing=-999.0), base_margin=bm)
    t.boost(3)
    late = t.add_eval(hb.DMatrix(ev, missing=-999.0))
    t.boost(4)
    booster = t.booster(16)
    assert booster.num_trees() == 7
    np.testing.assert_array_equal(t.eval_margins(first).view(np.uint32),
                                  expected(booster, ev, -999.0, bm).view(np.uint32))
    np.testing.assert_array_equal(t.eval_margins(late).view(np.uint32),
                                  expected(booster, ev, -999.0).view(np.uint32))
    # the training rows as an eval set: their margins are the trainer's own
    tr = t.add_eval(dtrain)
    np.testing.assert_array_equal(t.eval_margins(tr).reshape(-1), t.margins())


def test_a_new_trainer_drops_the_engine_eval_sets():
    x, y = data(4_000, 8, 27)
    engine = hb.DMatrix(x, label=y).engine(256)
    ev = eval_matrix(500, 8, 28)
    first = hb.Trainer(engine, {"max_depth": 4}, y)
    first.add_eval(hb.DMatrix(ev))
    first.boost(2)
    before = first.eval_margins(0).copy()
    second = hb.Trainer(engine, {"max_depth": 3}, y)
    i = second.add_eval(hb.DMatrix(ev))
    assert i == 0
    second.boost(3)
    np.testing.assert_array_equal(second.eval_margins(0).view(np.uint32),
                                  expected(second.booster(8), ev).view(np.uint32))
    np.testing.assert_array_equal(before.view(np.uint32),
                                  expected(first.booster(8), ev).view(np.uint32))
    with pytest.raises(hb.HbrError, match="newer trainer"):
        first.eval_margins(0)


def test_rejects_other_features():
    x, y = data(2_000, 8, 17)
    with pytest.raises(ValueError):
        hb.train({"max_depth": 3}, hb.DMatrix(x, label=y), 1, evals=[(hb.DMatrix(x[:, :5]), "bad")])
    t = hb.Trainer(hb.DMatrix(x, label=y).engine(256), {"max_depth": 3}, y)
    with pytest.raises(hb.HbrError):
        t.add_eval(hb.DMatrix(x[:, :5]))


def test_engine_level_eval_sets_take_caller_trees():
    """The engine-level entry points a caller driving its own rounds binds:
    trees passed as node arrays with their own thresholds (here the
    thresholds of unbalanced random trees, not cut values) added to two
    sets of two outputs."""
    rng = np.random.default_rng(21)
    f = 7
    x, y = data(3_000, f, 22)
    engine = hb.DMatrix(x, label=y).engine(64)
    ev = [eval_matrix(1_234, f, 23), eval_matrix(99, f, 24)]
    init = [rng.standard_normal((e.shape[0], 2)).astype(np.float32) for e in ev]
    ids = [engine.add_eval(e, i) for e, i in zip(ev, init)]
    trees, outputs = [], []
    for t in range(9):
        nodes = [dict(leaf_value=float(rng.standard_normal()))]
        n_splits = int(rng.integers(0, 40))
        for _ in range(n_splits):  # split a random leaf into a pair of leaves
            leaves = [i for i, nd in enumerate(nodes) if "left" not in nd]
            i = int(rng.choice(leaves))
            nodes[i].update(left=len(nodes), right=len(nodes) + 1, split_feature=int(rng.integers(0, f)),
                            split_cond=float(np.float32(rng.standard_normal())), default_left=bool(rng.random() < 0.5))
            nodes += [dict(leaf_value=float(rng.standard_normal())), dict(leaf_value=float(rng.standard_normal()))]
        for nd in nodes:
            nd.setdefault("left", -1)
            nd.setdefault("right", -1)
            nd.setdefault("split_feature", 0)
            nd.setdefault("split_cond", 0.0)
            nd.setdefault("default_left", True)
        tree = {k: np.array([nd[k] for nd in nodes]) for k in nodes[0]}
        out = t % 2
        engine.eval_add_tree(tree, out)
        trees.append(nodes)
        outputs.append(out)
    for i, e, m0 in zip(ids, ev, init):
        want = m0.copy()
        for nodes, out in zip(trees, outputs):
            one = O.forest_arrays([nodes], tree_output=[out], n_outputs=2, base_score=np.zeros(2))
            want = (want + O.predict_margin(one, e).reshape(-1, 2)).astype(np.float32)
        np.testing.assert_array_equal(engine.eval_margins(i).view(np.uint32), want.view(np.uint32))
    with pytest.raises(hb.HbrError):  # children not a pair
        engine.eval_add_tree(dict(split_feature=[0, 0, 0], split_cond=[0.0, 0, 0], default_left=[1, 1, 1],
                                  left=[2, -1, -1], right=[1, -1, -1], leaf_value=[0.0, 1, 2]))


def test_engine_level_eval_sets_take_categorical_caller_trees():
    """hbr_engine_eval_add_tree_categorical: random trees mixing numeric and
    categorical splits (sets of up to 40 codes from 0..59, pools per tree)
    added to an eval set of two outputs, rows with fractional, negative and
    missing codes: the oracle's prediction walk bit for bit; a categorical
    node whose range leaves the pool is refused."""
    rng = np.random.default_rng(41)
    f = 5
    x, y = data(2_000, f, 42)
    engine = hb.DMatrix(x, label=y).engine(64)
    e = (rng.integers(-3, 70, (3_333, f)) + rng.choice([0.0, 0.5], (3_333, f))).astype(np.float32)
    e[rng.random(e.shape) < 0.05] = np.nan
    init = rng.standard_normal((e.shape[0], 2)).astype(np.float32)
    idx = engine.add_eval(e, init)
    want = init.copy()
    for t in range(12):
        nodes, pool = [dict(leaf_value=float(rng.standard_normal()))], []
        for _ in range(int(rng.integers(0, 25))):
            i = int(rng.choice([j for j, nd in enumerate(nodes) if "left" not in nd]))
            nodes[i].update(left=len(nodes), right=len(nodes) + 1, split_feature=int(rng.integers(0, f)),
                            split_cond=float(np.float32(rng.standard_normal() * 20)),
                            default_left=bool(rng.random() < 0.5), is_categorical=bool(rng.random() < 0.6))
            nodes += [dict(leaf_value=float(rng.standard_normal())), dict(leaf_value=float(rng.standard_normal()))]
        for nd in nodes:
            for key, v in (("left", -1), ("right", -1), ("split_feature", 0), ("split_cond", 0.0),
                           ("default_left", True), ("is_categorical", False)):
                nd.setdefault(key, v)
            if nd["is_categorical"] and nd["left"] != -1:
                cats = np.sort(rng.choice(60, size=int(rng.integers(1, 41)), replace=False))
                nd["cat_begin"], nd["cat_end"] = len(pool), len(pool) + len(cats)
                pool.extend(int(c) for c in cats)
            else:
                nd["is_categorical"] = False
                nd["cat_begin"] = nd["cat_end"] = 0
        tree = {k: np.array([nd[k] for nd in nodes]) for k in nodes[0] if k not in ("cat_begin", "cat_end")}
        tree.update(is_categorical=np.array([nd["is_categorical"] for nd in nodes], np.uint8),
                    cat_begin=np.array([nd["cat_begin"] for nd in nodes], np.uint32),
                    cat_end=np.array([nd["cat_end"] for nd in nodes], np.uint32),
                    categories=np.array(pool, np.uint32))
        out = t % 2
        engine.eval_add_tree(tree, out)
        one = O.forest_arrays([nodes], tree_output=[out], n_outputs=2, base_score=np.zeros(2))
        one.update(is_categorical=tree["is_categorical"], cat_begin=tree["cat_begin"], cat_end=tree["cat_end"],
                   categories=tree["categories"])
        want = (want + O.predict_margin(one, e).reshape(-1, 2)).astype(np.float32)
    np.testing.assert_array_equal(engine.eval_margins(idx).view(np.uint32), want.view(np.uint32))
    bad = dict(split_feature=[0, 0, 0], split_cond=[0.0, 0, 0], default_left=[1, 1, 1], left=[1, -1, -1],
               right=[2, -1, -1], leaf_value=[0.0, 1, 2], is_categorical=[1, 0, 0], cat_begin=[0, 0, 0],
               cat_end=[3, 0, 0], categories=[1, 2])
    with pytest.raises(hb.HbrError):
        engine.eval_add_tree(bad)


def test_trees_discarded_by_the_device_are_added_to_no_eval_set():
    """Pipelined rounds whose gradients overflow: with eta 1e30 the second
    tree's leaves overflow to infinity, so the third round's gradients are
    not finite and the device skips that tree's walks and those of every
    tree queued after it. Training stops with an error; each eval set then
    holds exactly the kept trees, like the training margins."""
    x, y = data(6_000, 10, 25)
    dtrain = hb.DMatrix(x, label=y)
    t = hb.Trainer(dtrain.engine(256), {"objective": "reg:squarederror", "max_depth": 3, "eta": 1e30,
                                        "lambda": 0.0}, y)
    own = t.add_eval(dtrain)
    other = t.add_eval(hb.DMatrix(eval_matrix(1_000, 10, 26)))
    with pytest.raises(hb.HbrError, match="not finite"):
        t.boost(6)
    booster = t.booster(10)
    assert 1 <= booster.num_trees() < 6
    np.testing.assert_array_equal(t.eval_margins(own).reshape(-1).view(np.uint32), t.margins().view(np.uint32))
    np.testing.assert_array_equal(t.eval_margins(own).view(np.uint32), expected(booster, x).view(np.uint32))
    ev = eval_matrix(1_000, 10, 26)
    np.testing.assert_array_equal(t.eval_margins(other).view(np.uint32), expected(booster, ev).view(np.uint32))


@pytest.mark.parametrize("batched", ["1", "0"], ids=["batched", "pipelined"])
def test_softmax_trees_discarded_by_the_device_reach_no_margins(batched, monkeypatch):
    """Softmax rounds whose gradients overflow (eta 1e30, lambda 0): once a
    class's margins reach infinity its next gradients are not finite. The
    device skips the walks of that tree (batched: of that whole round) and
    of every tree queued after it; training stops with an error, and the
    training margins and each eval set hold exactly the kept trees."""
    monkeypatch.setenv("HBROCM_SOFTMAX_BATCH", batched)
    x, y = data(6_000, 10, 27, "multi:softprob", k=3)
    dtrain = hb.DMatrix(x, label=y)
    t = hb.Trainer(dtrain.engine(256), {"objective": "multi:softprob", "num_class": 3, "max_depth": 3,
                                        "eta": 1e30, "lambda": 0.0}, y)
    own = t.add_eval(dtrain)
    other = t.add_eval(hb.DMatrix(eval_matrix(1_000, 10, 28)))
    with pytest.raises(hb.HbrError, match="not finite"):
        t.boost(8)
    booster = t.booster(10)
    assert 1 <= booster.num_trees() < 24
    if batched == "1":
        assert booster.num_trees() % 3 == 0  # a round is kept or dropped whole
    want = expected(booster, x)
    np.testing.assert_array_equal(t.margins().reshape(-1, 3).view(np.uint32), want.view(np.uint32))
    np.testing.assert_array_equal(t.eval_margins(own).view(np.uint32), want.view(np.uint32))
    ev = eval_matrix(1_000, 10, 28)
    np.testing.assert_array_equal(t.eval_margins(other).view(np.uint32), expected(booster, ev).view(np.uint32))
