"""GPU parity over seeded random training configurations: objective,
growth policy, depth or leaves, regularisation, monotone directions,
weights, missing values, dense or CSR input and bin counts drawn from a
fixed seed; every tree against the oracle's (structure exact, leaf values
within 1e-5 relative)."""
import numpy as np
import pytest

import hessboost_amd as hb
from oracle import oracle as O
from tests.test_gpu_train import compare_trees

pytestmark = pytest.mark.gpu

OBJECTIVES = {"reg:squarederror": O.OBJ_SQUARED_ERROR, "binary:logistic": O.OBJ_LOGISTIC,
              "multi:softprob": O.OBJ_SOFTMAX}
ORACLE_OBJECTIVES = dict(OBJECTIVES, **{"binary:logitraw": O.OBJ_LOGITRAW})


def draw(seed):
    rng = np.random.default_rng(1000 + seed)
    n = int(rng.choice([97, 1_000, 6_001, 20_000]))
    f = int(rng.integers(2, 24))
    objective = str(rng.choice(list(OBJECTIVES)))
    k = int(rng.integers(2, 6)) if objective == "multi:softprob" else 1
    lossguide = bool(rng.random() < 0.35)
    cfg = {
        "n": n, "f": f, "objective": objective, "k": k,
        "max_bin": int(rng.choice([16, 64, 256])),
        "missing": float(rng.choice([0.0, 0.0, 0.05, 0.3])),
        "csr": bool(rng.random() < 0.25),
        "weights": bool(rng.random() < 0.4),
        "params": {
            "objective": objective,
            "eta": float(rng.choice([0.1, 0.3, 1.0])),
            "lambda": float(rng.choice([0.0, 1.0, 5.0])),
            "alpha": float(rng.choice([0.0, 0.0, 0.5])),
            "gamma": float(rng.choice([0.0, 0.0, 0.2])),
            "min_child_weight": float(rng.choice([0.0, 1.0, 3.0])),
            "max_delta_step": float(rng.choice([0.0, 0.0, 0.7])),
        },
    }
    if lossguide:
        cfg["params"].update({"grow_policy": "lossguide", "max_depth": 0, "max_leaves": int(rng.integers(2, 40))})
    else:
        cfg["params"]["max_depth"] = int(rng.integers(1, 9))
    if objective == "multi:softprob":
        cfg["params"]["num_class"] = k
    if rng.random() < 0.3:
        cfg["params"]["monotone_constraints"] = [int(v) for v in rng.integers(-1, 2, f)]
    # drawn last, so the draws above keep their values for every seed
    if objective != "multi:softprob" and rng.random() < 0.35:
        cfg["params"]["scale_pos_weight"] = float(rng.choice([0.5, 2.0, 3.0]))
    if objective == "binary:logistic" and rng.random() < 0.3:
        cfg["objective"] = cfg["params"]["objective"] = "binary:logitraw"
    return cfg


def data(cfg, seed):
    rng = np.random.default_rng(2000 + seed)
    n, f = cfg["n"], cfg["f"]
    x = rng.standard_normal((n, f)).astype(np.float32)
    x[:, 0] = np.round(x[:, 0] * 2) / 2  # a feature with few distinct values
    z = x[:, 0] + 0.5 * np.sin(2 * x[:, 1 % f]) - 0.3 * x[:, 2 % f] * x[:, 3 % f]
    if cfg["objective"] == "reg:squarederror":
        y = (z + 0.1 * rng.standard_normal(n)).astype(np.float32)
    elif cfg["objective"] in ("binary:logistic", "binary:logitraw"):
        y = (rng.random(n) < 1 / (1 + np.exp(-2 * z))).astype(np.float32)
    else:
        y = np.clip(np.floor((z - z.min()) / (np.ptp(z) + 1e-9) * cfg["k"]), 0, cfg["k"] - 1).astype(np.float32)
    if cfg["missing"] > 0:
        x[rng.random((n, f)) < cfg["missing"]] = np.nan
    w = (rng.random(n) * 2 + 0.1).astype(np.float32) if cfg["weights"] else None
    return x, y, w


def oracle_params(cfg):
    p = cfg["params"]
    return O.params(objective=ORACLE_OBJECTIVES[cfg["objective"]], eta=p["eta"], gamma=p["gamma"], reg_lambda=p["lambda"],
                    alpha=p["alpha"], min_child_weight=p["min_child_weight"], max_delta_step=p["max_delta_step"],
                    max_depth=p["max_depth"], max_leaves=p.get("max_leaves", 0),
                    grow_policy=O.GROW_LOSSGUIDE if p.get("grow_policy") == "lossguide" else O.GROW_DEPTHWISE,
                    num_class=cfg["k"] if cfg["objective"] == "multi:softprob" else 0,
                    monotone=p.get("monotone_constraints"), max_bin=cfg["max_bin"],
                    scale_pos_weight=p.get("scale_pos_weight", 1.0))


def to_csr(x):
    present = ~np.isnan(x)
    row_ptr = np.zeros(x.shape[0] + 1, np.uint64)
    row_ptr[1:] = np.cumsum(present.sum(1))
    rows, cols = np.nonzero(present)
    return row_ptr, cols.astype(np.uint32), x[rows, cols].astype(np.float32)


@pytest.mark.parametrize("seed", range(48))
def test_random_configuration_matches_oracle(seed):
    cfg = draw(seed)
    x, y, w = data(cfg, seed)
    print("config", seed, {k: v for k, v in cfg.items() if k != "params"}, cfg["params"], flush=True)
    params = dict(cfg["params"], max_bin=cfg["max_bin"])
    if cfg["csr"]:
        row_ptr, col, val = to_csr(x)
        ds = O.Dataset(csr=(row_ptr, col, val), n_cols=cfg["f"], max_bin=cfg["max_bin"], weights=w)
        dm = hb.DMatrix((row_ptr, col, val), label=y, weight=w, n_cols=cfg["f"])
    else:
        ds = O.Dataset(x, max_bin=cfg["max_bin"], weights=w)
        dm = hb.DMatrix(x, label=y, weight=w)
    ref = O.Model(ds, y, oracle_params(cfg), 3, weights=w)
    model = hb.train(params, dm, 3)
    assert np.array_equal(np.asarray(model.base_score, np.float32).view(np.uint32),
                          np.asarray(ref.base_score(), np.float32).view(np.uint32))
    compare_trees(model.trees, ref.trees())
