"""Shared data generators and fixture loaders for the test suite."""
import json
import os
import struct

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def four_features(n=160):
    """hessboost tests/common/mod.rs:28-39: values in [0, 1), feature 3
    missing on every 7th row, each an f32 quotient."""
    i = np.arange(n)
    a = ((i * 37) % 101).astype(np.float32) / np.float32(101)
    b = ((i * 53) % 97).astype(np.float32) / np.float32(97)
    c = ((i * 11) % 89).astype(np.float32) / np.float32(89)
    d = ((i * 29) % 83).astype(np.float32) / np.float32(83)
    d[i % 7 == 0] = np.nan
    return np.stack([a, b, c, d], axis=1).astype(np.float32)


def categorical_features(n=160):
    """tests/native_format.rs:508-513: four_features with column 0 replaced
    by the category codes i % 5."""
    x = four_features(n)
    x[:, 0] = (np.arange(n) % 5).astype(np.float32)
    return x


def train_labels(x, k=1):
    """tests/native_format.rs:441-454: y_t = 2a - b + t*c + 0.1 in f32."""
    a, b, c = x[:, 0], x[:, 1], x[:, 2]
    ys = [((np.float32(2) * a - b) + np.float32(t) * c + np.float32(0.1)).astype(np.float32)
          for t in range(k)]
    return ys[0] if k == 1 else np.stack(ys, axis=1)


def bits_to_f32(v):
    return np.asarray(v, np.uint32).view(np.float32)


def load_saved_models():
    return json.load(open(os.path.join(GOLDEN, "saved_models.json")))


def golden_forest(case):
    """Flat forest arrays of a saved model, restricted to its effective trees
    (model/mod.rs:1238-1242: best_iteration selects the first iterations)."""
    npt = case["num_parallel_tree"]
    k = case["n_outputs"]
    trees = case["trees"]
    n_trees = len(trees)
    if case["best_iteration"] is not None:
        n_trees = min((case["best_iteration"] + 1) * k * npt, n_trees)
    off = [0]
    cols = {key: [] for key in ("split_feature", "split_cond", "default_left", "left", "right", "leaf_value")}
    cat = {key: [] for key in ("is_categorical", "cat_begin", "cat_end", "categories")}
    for t in trees[:n_trees]:
        for key in cols:
            cols[key].extend(t[key])
        off.append(len(cols["left"]))
        # category ranges made absolute in the forest's concatenated pool
        base = len(cat["categories"])
        cat["is_categorical"].extend(t.get("is_categorical", [0] * len(t["left"])))
        cat["cat_begin"].extend(base + b for b in t.get("cat_begin", [0] * len(t["left"])))
        cat["cat_end"].extend(base + e for e in t.get("cat_end", [0] * len(t["left"])))
        cat["categories"].extend(t.get("categories", []))
    extra = {}
    if any(cat["is_categorical"]):
        extra = dict(is_categorical=np.array(cat["is_categorical"], np.uint8),
                     cat_begin=np.array(cat["cat_begin"], np.uint32), cat_end=np.array(cat["cat_end"], np.uint32),
                     categories=np.array(cat["categories"], np.uint32))
    return dict(**extra,
        tree_offset=np.array(off, np.uint32),
        split_feature=np.array(cols["split_feature"], np.uint32),
        split_cond=bits_to_f32(cols["split_cond"]),
        default_left=np.array(cols["default_left"], np.uint8),
        left=np.array(cols["left"], np.int32),
        right=np.array(cols["right"], np.int32),
        leaf_value=bits_to_f32(cols["leaf_value"]),
        tree_weight=bits_to_f32(case["tree_weights"][:n_trees]),
        tree_output=np.array([(t // npt) % k for t in range(n_trees)], np.uint32),
        base_score=bits_to_f32(case["base_score"]),
        n_outputs=k,
    )


def splitmix64(seed):
    """A splitmix64 stream (the synthetic data generator's source)."""
    state = np.uint64(seed)
    while True:
        state = np.uint64((int(state) + 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF)
        z = int(state)
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & 0xFFFFFFFFFFFFFFFF
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & 0xFFFFFFFFFFFFFFFF
        yield z ^ (z >> 31)


def random_tree(rng, n_features, max_depth):
    """An unbalanced tree in the reference's node layout, nodes numbered in
    depth-first order (the upload re-lays them out breadth-first)."""
    nodes = []

    def grow(depth):
        i = len(nodes)
        nodes.append(None)
        if depth >= max_depth or rng.random() < 0.25 * depth / max(1, max_depth):
            nodes[i] = (-1, -1, 0, 0.0, 0, float(rng.normal(0, 0.1)))
            return i
        f = int(rng.integers(0, n_features))
        cond = float(np.float32(rng.normal()))
        dl = int(rng.integers(0, 2))
        left = grow(depth + 1)
        right = grow(depth + 1)
        nodes[i] = (left, right, f, cond, dl, 0.0)
        return i

    grow(0)
    return dict(left=np.array([n[0] for n in nodes], np.int32), right=np.array([n[1] for n in nodes], np.int32),
                split_feature=np.array([n[2] for n in nodes], np.uint32),
                split_cond=np.array([n[3] for n in nodes], np.float32),
                default_left=np.array([n[4] for n in nodes], np.uint8),
                leaf_value=np.array([n[5] for n in nodes], np.float32))
