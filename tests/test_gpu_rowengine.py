"""hessboost's device-resident rounds through the row-engine calls of the C
ABI (the call sequence of build_device_staged, as hessboost_amd.rowengine
issues it) with fixed-point sums and the guard that certifies each winner:

* hbr_read_hist gives a node's histogram as the reference's CPU builder
  has it, bit for bit: built nodes summed in the CPU build's f64 order (one
  chain, or blocks of rows beyond 2^18 index rows), siblings as their
  parent's minus the built child's;
* the guard catches a designed near tie (two features whose best
  partitions differ by one row of small gradient): it resolves it on the
  device to the winner of the CPU builder's sums (the oracle's split, bit
  for bit), or reports it for a host replay; it certifies exact ties of
  duplicate features; every winner it certifies is the one the host would
  pick from the exact sums, within the loss bound it reports;
* three rounds of the 10,500,000 x 28 logistic workload grown this way
  match the oracle's first three trees node for node.
"""
import numpy as np
import pytest

import hessboost_amd as hb
from hessboost_amd import _capi as A
from hessboost_amd import synthetic
from oracle import oracle as O
from tests.golden.make_full_runs import unpack
from hessboost_amd.rowengine import RowEngineRounds, as_tree
from tests.test_gpu_full_runs import fixture
from tests.test_gpu_train import compare_trees

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, np.float64).view(np.uint64)


def logistic_engine(x, y, margins):
    e = hb.DMatrix(x, label=y).engine(256)
    e.set_sums("fixed_point")
    e.load_margins(margins)
    assert e.gradients(A.LOSS_LOGISTIC, y)
    return e


@pytest.mark.parametrize("n", [200_000, 300_000])
def test_read_hist_gives_the_cpu_builders_sums(n):
    """200,000 rows: every node one chain (an index of at most 2^18 rows);
    300,000: gathered nodes of 8,192 rows or more in blocks of ~4,096."""
    x, y = synthetic.higgs_like(n=n, seed=2)
    m0 = np.zeros(n, np.float32)
    e = logistic_engine(x, y, m0)
    ds = O.Dataset(x, max_bin=256)
    gp = O.gradient(O.OBJ_LOGISTIC, m0, y)
    root = e.begin_tree()
    assert e.reserve_hists(8)
    e.build_resident([(root, 0)])
    want_root = ds.build_hist(np.arange(n, dtype=np.uint32), gp)
    assert np.array_equal(bits(e.read_hist(0)), bits(want_root))
    fo = ds.feature_offset
    (left, right), = e.partition([(root, 0, 100, False)])
    small, big = (left, right) if left.len <= right.len else (right, left)
    e.build_resident([(small, 1)], [(0, 1)])
    want_small = ds.build_hist(e.rows(small), gp)
    want_big = want_root - want_small  # with_sibling: the parent's minus the built child's
    assert small.len >= 8_192
    assert np.array_equal(bits(e.read_hist(1)), bits(want_small))
    assert np.array_equal(bits(e.read_hist(0)), bits(want_big))
    # the larger child split again: its sibling is the root minus two built children
    (bl, br), (sl, sr) = e.partition([(big, 3, 60, True), (small, 5, 200, False)])
    b_small = bl if bl.len <= br.len else br
    s_small = sl if sl.len <= sr.len else sr
    e.build_resident([(b_small, 2), (s_small, 3)], [(0, 2), (1, 3)])
    w_bs = ds.build_hist(e.rows(b_small), gp)
    w_ss = ds.build_hist(e.rows(s_small), gp)
    assert np.array_equal(bits(e.read_hist(2)), bits(w_bs))
    assert np.array_equal(bits(e.read_hist(0)), bits(want_big - w_bs))
    assert np.array_equal(bits(e.read_hist(3)), bits(w_ss))
    assert np.array_equal(bits(e.read_hist(1)), bits(want_small - w_ss))
    assert fo[1] > fo[0]


def near_tie_data(n=100_000, perturb=True, seed=4):
    """Feature 1 duplicates feature 0; with `perturb`, one row's feature 1
    value moves to the far end, and that row's margin makes its logistic
    pair small (|g|, h ~ 1e-6, far above the fixed-point unit): the two
    features' best partitions then differ by that row alone, and their
    scores by less than the sums' error bound."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, 4)).astype(np.float32)
    x[:, 1] = x[:, 0]
    y = (rng.random(n) < 1.0 / (1.0 + np.exp(-2.0 * x[:, 0]))).astype(np.float32)
    m = np.zeros(n, np.float32)
    r = int(np.argmin(np.abs(x[:, 0] + 1.5)))  # a row left of feature 0's best threshold (near 0)
    y[r] = 1.0
    m[r] = 13.8
    if perturb:
        x[r, 1] = 9.0
    return x, y, m


def root_scan(e, y, m):
    ds_root = e.begin_tree()
    tot, fx = e.root_total(ds_root, fixed=True)
    assert e.reserve_hists(2)
    e.build_resident([(ds_root, 0)])
    p = O.params(objective=O.OBJ_LOGISTIC)
    gain = O.lib().or_node_gain(tot[0], tot[1], -np.inf, np.inf, p)
    root_scan.total = tuple(tot)
    return e.scan_resident((1.0, 0.0, 0.0, 1.0), [dict(slot=0, total=tuple(tot), fixed=tuple(fx), root_gain=gain)])[0]


def test_guard_resolves_or_replays_a_near_tie_and_certifies_duplicate_features():
    x, y, m = near_tie_data(perturb=True)
    ds = O.Dataset(x, max_bin=256)
    gp = O.gradient(O.OBJ_LOGISTIC, m, y)
    rows = np.arange(len(y), dtype=np.uint32)
    nodes, _ = ds.grow_tree(gp, O.params(objective=O.OBJ_LOGISTIC, max_depth=1))
    # the default: resolved on the device, the CPU builder's winner
    e = logistic_engine(x, y, m)
    sc = root_scan(e, y, m)
    assert sc.kind == A.SCAN_NUMERIC
    c = e.counters()
    assert c["near_ties"] == 1 and c["near_ties_resolved"] == 1
    fs = int(ds.feature_offset[sc.feature])
    bin_ = (fs + sc.offset - 1 if sc.offset else -1) if sc.backward else fs + sc.offset
    assert (sc.feature, bin_, bool(sc.backward)) == (nodes[0]["split_feature"], nodes[0]["split_bin"],
                                                   bool(nodes[0]["default_left"]))
    s = ds.evaluate(e.read_hist(0), root_scan.total, O.params(objective=O.OBJ_LOGISTIC))
    assert np.float32(sc.loss_chg) == np.float32(s.loss_chg) and sc.left_g == s.left_g and sc.left_h == s.left_h
    # reported for a host replay: its sums are the CPU's, and the host's choice from them is the oracle's
    e = logistic_engine(x, y, m)
    e.set_guard("replay")
    sc = root_scan(e, y, m)
    assert sc.kind == A.SCAN_REPLAY and sc.fallback == A.FALLBACK_NEAR_TIE
    hist = e.read_hist(0)
    assert np.array_equal(bits(hist), bits(ds.build_hist(rows, gp)))
    s = ds.evaluate(hist, O.sum_rows(gp, rows), O.params(objective=O.OBJ_LOGISTIC))
    assert (s.feature, s.bin) == (nodes[0]["split_feature"], nodes[0]["split_bin"])
    # without the guard the same scan is a plain winner
    e.set_guard("off")
    assert root_scan(e, y, m).kind == A.SCAN_NUMERIC
    # exact duplicates are one partition: certified, the lower feature wins
    x2, y2, m2 = near_tie_data(perturb=False)
    e2 = logistic_engine(x2, y2, m2)
    sc2 = root_scan(e2, y2, m2)
    assert sc2.kind == A.SCAN_NUMERIC and sc2.feature == 0 and sc2.loss_err > 0
    assert e2.counters()["near_ties"] == 0


def test_certified_winners_are_the_exact_sums_winners():
    """Two depth-6 rounds over 300,000 higgs-like rows: for every winner the
    guard certifies, the host's search over the node's exact sums picks the
    same feature, bin and direction, and its loss is within the bound."""
    n = 300_000
    x, y = synthetic.higgs_like(n=n, seed=5)
    e = hb.DMatrix(x, label=y).engine(256)
    e.set_sums("fixed_point")
    ds = O.Dataset(x, max_bin=256)
    fo, cuts = ds.feature_offset, ds.cut_values
    d = RowEngineRounds(e, fo, cuts, {"max_depth": 6, "eta": 0.3})
    d.audit = []
    p = O.params(objective=O.OBJ_LOGISTIC, max_depth=6, eta=0.3)
    m = np.zeros(n, np.float32)
    for _ in range(2):
        d.device_round(m, y)
    assert len(d.audit) > 50
    for a in d.audit:
        exact = ds.evaluate(a["hist"], a["total"], p)
        assert (exact.feature, exact.bin, bool(exact.default_left)) == (a["feature"], a["bin"], a["default_left"])
        assert abs(float(exact.loss_chg) - float(a["loss"])) <= float(a["err"])


def test_three_rounds_of_the_higgs_workload_through_the_row_engine_match_oracle():
    """The 10,500,000 x 28 logistic workload (depth 8, eta 0.1, 256 bins):
    three device_round calls of the reference's row-engine sequence grow the
    oracle's first three trees node for node, leaves within 1e-5."""
    z = fixture("c2")
    want = unpack(z)[:3]
    x, y = synthetic.higgs_like(n=10_500_000, seed=0)
    d_x = hb.DMatrix(x, label=y)
    e = d_x.engine(256)
    e.set_sums("fixed_point")
    cuts = d_x.cuts(256)
    fo, cv = cuts.arrays()
    del x
    d = RowEngineRounds(e, fo, cv, {"max_depth": 8, "eta": 0.1})
    base = np.float32(z["base_score"][0])
    m = np.full(len(y), base, np.float32)
    got = [as_tree(d.device_round(m, y)) for _ in range(3)]
    compare_trees(got, want)
    c = e.counters()
    print(f"near ties {c['near_ties']}, resolved {c['near_ties_resolved']}")
    assert d.replays == 0
