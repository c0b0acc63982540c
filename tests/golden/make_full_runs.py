"""Writes the full-length training fixtures: every tree the oracle grows on
the benchmark workloads at their full sizes and round counts, with a sample
of the final margins.

    python tests/golden/make_full_runs.py [c2|c3|c4 ...]

Workloads (the generators of hessboost_amd.synthetic, seed 0):

* c2: 10,500,000 x 28 higgs-like binary logistic, depth 8, eta 0.1,
  256 bins, depthwise, 500 rounds;
* c3: 500,000 x 2,000 CSR with 90% of the cells missing, 64 bins,
  loss-guided to 255 leaves (max_depth 0), eta 0.3, 200 rounds;
* c4: 2,000,000 x 50, 10-class softmax, depth 6, eta 0.3, 256 bins,
  100 rounds (1,000 class trees).

The oracle is the C restatement of the reference's CPU hist path
(oracle/); it runs here on the CPU (c2 takes about 20 minutes at 8
threads). Each fixture is a compressed npz of the trees' nodes in order,
concatenated: children, split feature, threshold bits, default direction,
leaf value, plus the per-tree node counts, the base score and the margins
of every 1,000th row.
"""
from __future__ import annotations

import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from hessboost_amd import synthetic  # noqa: E402
from oracle import oracle as O  # noqa: E402

OUT = os.path.join(HERE, "full_runs")
MARGIN_STRIDE = 1000


def workload(name):
    """(dataset, labels, oracle params, rounds) of a named workload."""
    if name == "c2":
        x, y = synthetic.higgs_like(n=10_500_000, seed=0)
        ds = O.Dataset(x, max_bin=256)
        return ds, y, O.params(objective=O.OBJ_LOGISTIC, max_depth=8, eta=0.1), 500
    if name == "c3":
        (row_ptr, col, val), y, _ = synthetic.sparse_wide(n=500_000, f=2_000, density=0.1, seed=0)
        ds = O.Dataset(csr=(row_ptr, col, val), n_cols=2_000, max_bin=64)
        return ds, y, O.params(grow_policy=O.GROW_LOSSGUIDE, max_depth=0, max_leaves=255, eta=0.3,
                               max_bin=64), 200
    if name == "c4":
        x, y = synthetic.multiclass(n=2_000_000, f=50, k=10, seed=0)
        ds = O.Dataset(x, max_bin=256)
        return ds, y, O.params(objective=O.OBJ_SOFTMAX, num_class=10, max_depth=6, eta=0.3), 100
    raise ValueError(name)


def pack(trees, margins, n_rows, n_outputs, base_score):
    counts = np.array([len(t) for t in trees], np.int32)
    nodes = [nd for t in trees for nd in t]
    assert max(counts) < (1 << 15) and max(nd["split_feature"] for nd in nodes) < (1 << 16)
    rows = np.arange(0, n_rows, MARGIN_STRIDE, dtype=np.int64)
    m = np.asarray(margins, np.float32).reshape(n_rows, n_outputs)
    return dict(
        n_nodes=counts,
        left=np.array([nd["left"] for nd in nodes], np.int16),
        right=np.array([nd["right"] for nd in nodes], np.int16),
        split_feature=np.array([nd["split_feature"] for nd in nodes], np.uint16),
        split_cond=np.array([nd["split_cond"] for nd in nodes], np.float32).view(np.uint32),
        default_left=np.array([nd["default_left"] for nd in nodes], np.uint8),
        leaf_value=np.array([nd["leaf_value"] for nd in nodes], np.float32),
        margin_rows=rows,
        margins=np.ascontiguousarray(m[rows]),
        base_score=np.asarray(base_score, np.float32),
    )


def unpack(z):
    """The fixture's trees as the node dicts `tests.test_gpu_train.compare_trees` reads."""
    z = {k: np.asarray(z[k]) for k in ("n_nodes", "left", "right", "split_feature", "split_cond", "default_left",
                                       "leaf_value")}
    out, s = [], 0
    for c in z["n_nodes"]:
        e = s + int(c)
        out.append([dict(left=int(z["left"][i]), right=int(z["right"][i]),
                         split_feature=int(z["split_feature"][i]),
                         split_cond=z["split_cond"][i:i + 1].view(np.float32)[0],
                         default_left=bool(z["default_left"][i]), leaf_value=z["leaf_value"][i])
                    for i in range(s, e)])
        s = e
    return out


def make(name, threads):
    t0 = time.time()
    O.set_threads(threads)
    ds, y, p, rounds = workload(name)
    print(f"{name}: data and index in {time.time() - t0:.1f} s", flush=True)
    model = O.Model(ds, y, p, 1)
    done = 1
    while done < rounds:
        k = min(10, rounds - done)
        model.more(k)
        done += k
        print(f"{name}: round {done} at {time.time() - t0:.1f} s", flush=True)
    arrs = pack(model.trees(), model.margins(), ds.n_rows, model.n_outputs, model.base_score())
    os.makedirs(OUT, exist_ok=True)
    path = os.path.join(OUT, f"{name}.npz")
    np.savez_compressed(path, **arrs)
    print(f"{name}: {len(arrs['n_nodes'])} trees -> {path} ({os.path.getsize(path)} bytes)", flush=True)


if __name__ == "__main__":
    names = sys.argv[1:] or ["c4", "c3", "c2"]
    for n in names:
        make(n, int(os.environ.get("ORACLE_THREADS", "8")))
