"""GPU parity on the shapes of the benchmark configurations.

Every workload runs at its full size against the oracle: the regression
(100,000 x 32 squared error, depth 6, 100 rounds), the higgs-like logistic
(10,500,000 x 28, depth 8, 10 rounds), the sparse wide loss-guided one
(500,000 x 2,000 CSR, 90% missing, 64 bins, 255 leaves, 2 rounds), the
10-class softmax (2,000,000 x 50, depth 6, 2 rounds) and batch prediction
(1,000 depth-8 trees over 1,000,000 x 100 rows): trees node for node, leaf
values within 1e-5, margins within 1e-5 (prediction: bit for bit, and leaf
ids exact). Smaller cases of the sparse and softmax shapes add row orders
and class counts."""
import numpy as np
import pytest

import hessboost_amd as hb
from hessboost_amd import synthetic
from oracle import oracle as O
from tests.test_gpu_train import compare_trees

pytestmark = pytest.mark.gpu


def test_c1_full_size_matches_oracle():
    x, y = synthetic.regression_100k(n=100_000, f=32, seed=0)
    params = {"objective": "reg:squarederror", "max_depth": 6, "eta": 0.1, "max_bin": 256}
    O.set_threads(8)
    ref = O.Model(O.Dataset(x, max_bin=256), y, O.params(max_depth=6, eta=0.1), 100)
    model = hb.train(params, hb.DMatrix(x, label=y), 100)
    compare_trees(model.trees, ref.trees())
    m = model.predict(x, output_margin=True)
    assert np.max(np.abs(m - ref.margins())) <= 1e-5


def test_c2_full_size_matches_oracle():
    """The binary logistic workload at its full size: 10,500,000 x 28
    higgs-like rows, depth 8, eta 0.1, 256 bins, free-running for 10 rounds.
    At this row count the per-tree fixed-point unit is 2^(e_max - 38), the
    regime where integer sums and the reference's f64 chains differ in their
    last bits: every tree must still match node for node (split feature,
    threshold, default direction, children), leaves within 1e-5, and the
    final margins within 1e-5."""
    x, y = synthetic.higgs_like(n=10_500_000, seed=0)
    O.set_threads(16)
    ref = O.Model(O.Dataset(x, max_bin=256), y, O.params(objective=O.OBJ_LOGISTIC, max_depth=8, eta=0.1), 10)
    params = {"objective": "binary:logistic", "max_depth": 8, "eta": 0.1, "max_bin": 256}
    d = hb.DMatrix(x, label=y)
    t = hb.Trainer(d.engine(256), params, y)
    t.boost(10)
    compare_trees(t.trees(), ref.trees())
    assert np.max(np.abs(t.margins() - ref.margins())) <= 1e-5


def test_c3_shape_sparse_missing_lossguide_matches_oracle():
    (row_ptr, col, val), y, _ = synthetic.sparse_wide(n=20_000, f=300, density=0.1, seed=7)
    params = {"grow_policy": "lossguide", "max_depth": 0, "max_leaves": 255, "eta": 0.3, "max_bin": 64}
    ds = O.Dataset(csr=(row_ptr, col, val), n_cols=300, max_bin=64)
    ref = O.Model(ds, y, O.params(grow_policy=O.GROW_LOSSGUIDE, max_depth=0, max_leaves=255, eta=0.3, max_bin=64), 3)
    model = hb.train(params, hb.DMatrix((row_ptr, col, val), label=y, n_cols=300), 3)
    compare_trees(model.trees, ref.trees())
    assert any(nd == 1 for t in model.trees for nd in t["default_left"][np.asarray(t["left"]) != -1]), \
        "no split sent missing values left"


def test_c3_full_size_matches_oracle():
    """500,000 x 2,000 CSR (90% missing, Exp(1) values), 64 bins (128,000
    bins in 16 ranges of 8,192), loss-guided to 255 leaves, 2 rounds."""
    (row_ptr, col, val), y, _ = synthetic.sparse_wide(n=500_000, f=2_000, density=0.1, seed=0)
    O.set_threads(16)
    params = {"grow_policy": "lossguide", "max_depth": 0, "max_leaves": 255, "eta": 0.3, "max_bin": 64}
    ds = O.Dataset(csr=(row_ptr, col, val), n_cols=2_000, max_bin=64)
    ref = O.Model(ds, y, O.params(grow_policy=O.GROW_LOSSGUIDE, max_depth=0, max_leaves=255, eta=0.3, max_bin=64), 2)
    model = hb.train(params, hb.DMatrix((row_ptr, col, val), label=y, n_cols=2_000), 2)
    assert ds.total_bins > 16 * 8_192 - 8_192
    compare_trees(model.trees, ref.trees())


def test_c4_full_size_matches_oracle():
    """2,000,000 x 50, 10-class softmax, depth 6, eta 0.3, 2 rounds (20
    class trees grown as batches)."""
    x, y = synthetic.multiclass(n=2_000_000, f=50, k=10, seed=0)
    O.set_threads(16)
    params = {"objective": "multi:softprob", "num_class": 10, "max_depth": 6, "eta": 0.3, "max_bin": 256}
    ref = O.Model(O.Dataset(x, max_bin=256), y, O.params(objective=O.OBJ_SOFTMAX, num_class=10, max_depth=6,
                                                         eta=0.3), 2)
    d = hb.DMatrix(x, label=y)
    t = hb.Trainer(d.engine(256), params, y)
    t.boost(2)
    compare_trees(t.trees(), ref.trees())
    assert np.max(np.abs(t.margins() - ref.margins())) <= 1e-5


def test_c5_full_forest_matches_oracle():
    """The 1,000-tree depth-8 forest over 1,000,000 x 100 rows with 2% NaN:
    margins bit for bit (tree order f32 adds), leaf ids exact on the first
    200,000 rows."""
    trees = synthetic.forest(n_trees=1000, depth=8, n_features=100, seed=0)
    x = synthetic.predict_rows(n=1_000_000, f=100, seed=1)
    O.set_threads(16)
    arrs = O.forest_arrays(trees)
    want = O.predict_margin(arrs, x)
    f = hb.Forest(arrs, 1)
    got = f.predict_margin(x)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    head = np.ascontiguousarray(x[:200_000])
    _, want_leaf = O.predict_margin(arrs, head, with_leaf=True)
    assert np.array_equal(f.predict_leaf(head), want_leaf)


def test_csr_rows_in_any_column_order_give_the_same_trees():
    """Routing binary-searches a row's ascending global bins; a CSR whose
    rows list their columns out of order keeps the caller's entry order in
    the index, so routing scans the row instead. Both give the oracle's
    trees (two 8,192-bin ranges per tile: 150 features x 64 bins)."""
    (row_ptr, col, val), y, _ = synthetic.sparse_wide(n=12_000, f=150, density=0.2, seed=8)
    rng = np.random.default_rng(8)
    col_s, val_s = col.copy(), val.copy()
    for r in range(len(row_ptr) - 1):
        a, b = int(row_ptr[r]), int(row_ptr[r + 1])
        p = rng.permutation(b - a)
        col_s[a:b], val_s[a:b] = col[a:b][p], val[a:b][p]
    params = {"grow_policy": "lossguide", "max_depth": 0, "max_leaves": 63, "eta": 0.3, "max_bin": 64}
    ds = O.Dataset(csr=(row_ptr, col, val), n_cols=150, max_bin=64)
    ref = O.Model(ds, y, O.params(grow_policy=O.GROW_LOSSGUIDE, max_depth=0, max_leaves=63, eta=0.3, max_bin=64), 2)
    for c, v in ((col, val), (col_s, val_s)):
        model = hb.train(params, hb.DMatrix((row_ptr, c, v), label=y, n_cols=150), 2)
        compare_trees(model.trees, ref.trees())


def test_c4_shape_softmax_matches_oracle():
    x, y = synthetic.multiclass(n=50_000, f=50, k=10, seed=0)
    params = {"objective": "multi:softprob", "num_class": 10, "max_depth": 6, "eta": 0.3, "max_bin": 256}
    ref = O.Model(O.Dataset(x, max_bin=256), y, O.params(objective=O.OBJ_SOFTMAX, num_class=10, max_depth=6,
                                                         eta=0.3), 2)
    model = hb.train(params, hb.DMatrix(x, label=y), 2)
    compare_trees(model.trees, ref.trees())
    assert len(model.trees) == 20
