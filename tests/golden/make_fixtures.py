"""Extract the reference's saved-model prediction fixtures into small data files.

Reads hessboost's own saved models and recorded margins
(tests/data/saved/<version>/<case>.json and <case>.margins, checked by
tests/native_format.rs:822-860) and writes tests/golden/saved_models.json:
for every scalar-leaf case, the trees as flat node arrays (categorical
splits with their category ranges and each tree's category pool), the
tree weights and outputs, the base score, and the recorded margins, every
f32 stored as its bit pattern. The input rows are not stored: they are
regenerated in closed form (tests/common/mod.rs:28-39, four_features;
the categorical case replaces column 0 by the codes i % 5,
tests/native_format.rs:508-513).

It also copies, minified, the 0.4.9 JSON model documents themselves into
tests/golden/models/ (the JSON model format, model/serde.rs): the saved
models of the cases above, which the JSON reader and writer must reproduce,
and two whose features this path does not carry (a linear booster, vector
leaves), which the reader must refuse; and the native binary files
(<case>.bin, src/model/native.rs) of every version into tests/golden/native/.

Run once in a checkout that has the reference under /root/reference:
    python tests/golden/make_fixtures.py
"""
import json
import os
import struct

import numpy as np

REF = "/root/reference/tests/data/saved"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "saved_models.json")
CASES = ["early_stopping", "dart", "multiclass_forest", "quantiles", "expectiles", "aft",
         "dist_normal", "dist_negbinomial", "multi_target", "categorical_splits"]


def f32_bits(x):
    return struct.unpack("<I", struct.pack("<f", float(x)))[0]


def main():
    out = {}
    for ver in sorted(os.listdir(REF)):
        for case in CASES:
            path = os.path.join(REF, ver, case + ".json")
            if not os.path.exists(path):
                continue
            doc = json.load(open(path))
            trees = []
            for t in doc["trees"]:
                assert t.get("size_leaf_vector", 0) <= 1 and not t.get("linear")
                nodes = t["nodes"]
                trees.append({
                    "is_categorical": [int(n["is_categorical"]) for n in nodes],
                    "cat_begin": [n["cat_begin"] for n in nodes],
                    "cat_end": [n["cat_end"] for n in nodes],
                    "categories": list(t["categories"]),
                    "split_feature": [n["split_feature"] for n in nodes],
                    "split_cond": [f32_bits(n["split_cond"]) for n in nodes],
                    "default_left": [int(n["default_left"]) for n in nodes],
                    "left": [n["left"] for n in nodes],
                    "right": [n["right"] for n in nodes],
                    "leaf_value": [f32_bits(n["leaf_value"]) for n in nodes],
                    "sum_hess": [f32_bits(n["sum_hess"]) for n in nodes],
                    "split_gain": [f32_bits(n["split_gain"]) for n in nodes],
                })
            margins = np.fromfile(os.path.join(REF, ver, case + ".margins"), "<u4")
            tw = doc["tree_weights"]
            out[f"{ver}/{case}"] = {
                "objective": doc["objective"],
                "n_outputs": doc["n_outputs"],
                "num_parallel_tree": doc["num_parallel_tree"],
                "best_iteration": doc["best_iteration"],
                "base_score": [f32_bits(b) for b in doc["base_score"]],
                "tree_weights": [f32_bits(w) for w in tw],
                "trees": trees,
                "margins": margins.tolist(),
            }
    json.dump(out, open(OUT, "w"), separators=(",", ":"))
    print(f"wrote {len(out)} cases to {OUT}")
    models = os.path.join(os.path.dirname(OUT), "models")
    os.makedirs(models, exist_ok=True)
    for case in CASES + ["gblinear", "vector_leaves"]:
        doc = json.load(open(os.path.join(REF, "0.4.9", case + ".json")))
        json.dump(doc, open(os.path.join(models, case + ".json"), "w"), separators=(",", ":"))
    print(f"copied {len(CASES) + 2} JSON models to {models}")
    # the native binary files of every version, as the reference saved them
    # (zstd frames of the HBM container, src/model/native.rs), for the
    # native reader and writer
    native = os.path.join(os.path.dirname(OUT), "native")
    copied = 0
    for ver in sorted(os.listdir(REF)):
        os.makedirs(os.path.join(native, ver), exist_ok=True)
        for case in CASES + ["gblinear", "vector_leaves"]:
            src = os.path.join(REF, ver, case + ".bin")
            if os.path.exists(src):
                with open(src, "rb") as f, open(os.path.join(native, ver, case + ".bin"), "wb") as g:
                    g.write(f.read())
                copied += 1
    print(f"copied {copied} native model files to {native}")


if __name__ == "__main__":
    main()
