"""GPU parity on the shapes of the benchmark configurations.

C1 runs at its full size (100,000 x 32 squared error, depth 6, 256 bins,
eta 0.1, 100 rounds): every tree node for node against the oracle, leaf
values within 1e-5, final margins within 1e-5. C3 (wide CSR with 90%
missing, 64 bins, loss-guided 255 leaves) and C4 (10-class softmax, depth 6)
run scaled down in rows and rounds so the oracle finishes in seconds; they
take the sparse histogram kernel with the backward (missing-left) pass and
the per-class trees."""
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
