"""The reference's JSON model document (model/serde.rs): the reference's
own saved models (tests/data/saved/0.4.9, copied as data into
tests/golden/models) are read and written back unchanged, field for field
with every f32 value exact; models with features this path does not carry
are refused by name."""
import json
import os

import numpy as np
import pytest

import hessboost_amd as hb

MODELS = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "models")
CARRIED = ["early_stopping", "dart", "multiclass_forest", "quantiles", "expectiles", "aft", "dist_normal",
           "dist_negbinomial", "multi_target", "categorical_splits"]


def same(a, b, path="doc"):
    """Equal documents; numbers compare as f32 (the document's floats are f32)."""
    if isinstance(a, dict):
        assert isinstance(b, dict) and a.keys() == b.keys(), (path, sorted(a), sorted(b))
        for k in a:
            same(a[k], b[k], f"{path}.{k}")
    elif isinstance(a, list):
        assert isinstance(b, list) and len(a) == len(b), path
        for i, (x, y) in enumerate(zip(a, b)):
            same(x, y, f"{path}[{i}]")
    elif isinstance(a, bool) or a is None or isinstance(a, str):
        assert a == b, (path, a, b)
    else:
        assert np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32), (path, a, b)


@pytest.mark.parametrize("case", CARRIED)
def test_reference_model_documents_round_trip(case):
    text = open(os.path.join(MODELS, case + ".json")).read()
    doc = json.loads(text)
    b = hb.Booster.load_model_json(text)
    out = json.loads(b.save_model_json())
    same(doc, out)
    # and once more from our own document
    same(out, json.loads(hb.Booster.load_model_json(json.dumps(out)).save_model_json()))


@pytest.mark.parametrize("case,what", [("gblinear", "linear"), ("vector_leaves", "vector leaves")])
def test_models_beyond_this_path_are_refused(case, what):
    with pytest.raises(ValueError, match=what):
        hb.Booster.load_model_json(open(os.path.join(MODELS, case + ".json")).read())


def test_malformed_categorical_nodes_are_refused():
    """tests/native_format.rs:391-409: a categorical split needs at least
    one category; a leaf is never categorical."""
    doc = json.loads(open(os.path.join(MODELS, "categorical_splits.json")).read())
    node = doc["trees"][0]["nodes"][0]
    assert node["is_categorical"]
    node["cat_end"] = node["cat_begin"]
    with pytest.raises(ValueError, match="categor"):
        hb.Booster.load_model_json(json.dumps(doc))
    doc = json.loads(open(os.path.join(MODELS, "categorical_splits.json")).read())
    leaf = next(n for n in doc["trees"][0]["nodes"] if n["left"] == -1)
    leaf["is_categorical"] = True
    with pytest.raises(ValueError, match="leaf marked categorical"):
        hb.Booster.load_model_json(json.dumps(doc))


def test_categorical_forest_arrays_take_absolute_ranges():
    b = hb.Booster.load_model_json(open(os.path.join(MODELS, "categorical_splits.json")).read())
    d = b.forest_desc()
    doc = json.loads(open(os.path.join(MODELS, "categorical_splits.json")).read())
    pool = [c for t in doc["trees"] for c in t["categories"]]
    assert list(d["categories"]) == pool
    at, base = 0, 0
    for t in doc["trees"]:
        for n in t["nodes"]:
            assert bool(d["is_categorical"][at]) == n["is_categorical"]
            if n["is_categorical"]:
                assert list(d["categories"][d["cat_begin"][at]:d["cat_end"][at]]) == \
                    t["categories"][n["cat_begin"]:n["cat_end"]]
            at += 1
        base += len(t["categories"])


def test_effective_trees_and_outputs_follow_the_document():
    """model/mod.rs:1238-1242: a best iteration keeps its first
    (best + 1) x outputs x parallel trees; tree t feeds output
    (t / num_parallel_tree) mod n_outputs."""
    es = hb.Booster.load_model_json(open(os.path.join(MODELS, "early_stopping.json")).read())
    assert es.best_iteration == 1 and len(es.trees) == 4 and len(es.effective_trees()) == 2
    mc = hb.Booster.load_model_json(open(os.path.join(MODELS, "multiclass_forest.json")).read())
    d = mc.forest_desc()
    assert mc.num_parallel_tree == 3 and mc.n_outputs == 3
    assert list(d["tree_output"][:9]) == [0, 0, 0, 1, 1, 1, 2, 2, 2]
