"""Every training workload at its full size and its full round count on the
GPU, against the oracle's run of the same workload (trees and a sample of
the final margins, written by tests/golden/make_full_runs.py on the CPU):

* 10,500,000 x 28 higgs-like binary logistic, depth 8, eta 0.1, 256 bins,
  500 rounds (the pipelined device rounds with the fused margin walk);
* 500,000 x 2,000 CSR, 90% missing, 64 bins, loss-guided to 255 leaves,
  eta 0.3, 200 rounds;
* 2,000,000 x 50 10-class softmax, depth 6, eta 0.3, 100 rounds (1,000
  class trees grown ten to a batch).

Every tree node for node (split feature, threshold bits, default direction,
children), leaf values within 1e-5 relative, margins within 1e-5 absolute.
The histogram sums are fixed point on the device and f64 chains in the
oracle; these runs show the fixed-point error does not flip a split over a
whole fit of each workload.
"""
import os

import numpy as np
import pytest

import hessboost_amd as hb
from hessboost_amd import synthetic
from tests.golden.make_full_runs import unpack
from tests.test_gpu_train import compare_trees

pytestmark = pytest.mark.gpu

FIXTURES = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "full_runs")


def fixture(name):
    path = os.path.join(FIXTURES, f"{name}.npz")
    if not os.path.exists(path):
        pytest.fail(f"missing fixture {path}: run tests/golden/make_full_runs.py {name}")
    return np.load(path)


def check(trees, margins, z, n_outputs):
    want = unpack(z)
    assert len(trees) == len(want)
    compare_trees(trees, want)
    m = np.asarray(margins, np.float32).reshape(-1, n_outputs)[z["margin_rows"]]
    assert np.max(np.abs(m - z["margins"])) <= 1e-5


def test_higgs_500_rounds_match_oracle():
    z = fixture("c2")
    x, y = synthetic.higgs_like(n=10_500_000, seed=0)
    params = {"objective": "binary:logistic", "max_depth": 8, "eta": 0.1, "max_bin": 256}
    t = hb.Trainer(hb.DMatrix(x, label=y).engine(256), params, y)
    del x
    t.boost(500)
    assert t.base_score().view(np.uint32)[0] == z["base_score"].view(np.uint32)[0]
    check(t.trees(), t.margins(), z, 1)


def test_sparse_lossguide_200_rounds_match_oracle():
    z = fixture("c3")
    (row_ptr, col, val), y, _ = synthetic.sparse_wide(n=500_000, f=2_000, density=0.1, seed=0)
    params = {"grow_policy": "lossguide", "max_depth": 0, "max_leaves": 255, "eta": 0.3, "max_bin": 64}
    d = hb.DMatrix((row_ptr, col, val), label=y, n_cols=2_000)
    t = hb.Trainer(d.engine(64), params, y)
    t.boost(200)
    check(t.trees(), t.margins(), z, 1)


def test_softmax_100_rounds_match_oracle():
    z = fixture("c4")
    x, y = synthetic.multiclass(n=2_000_000, f=50, k=10, seed=0)
    params = {"objective": "multi:softprob", "num_class": 10, "max_depth": 6, "eta": 0.3, "max_bin": 256}
    t = hb.Trainer(hb.DMatrix(x, label=y).engine(256), params, y)
    t.boost(100)
    check(t.trees(), t.margins(), z, 10)
