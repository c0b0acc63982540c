"""ctypes binding of the CPU oracle (test infrastructure only).

The oracle is a C restatement of hessboost's CPU hist path (see oracle.h for
the reference file:line of each part). Only the test suite, the smoke check
and the benchmark's CPU-baseline leg load it; the product never does.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_DIR = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_DIR, "liboracle.so")

OBJ_SQUARED_ERROR, OBJ_LOGISTIC, OBJ_SOFTMAX, OBJ_LOGITRAW = 0, 1, 2, 3
GROW_DEPTHWISE, GROW_LOSSGUIDE = 0, 1


def build() -> None:
    subprocess.run(["make", "-s", "-C", _DIR], check=True)


class Cuts(C.Structure):
    _fields_ = [("n_features", C.c_size_t), ("feature_offset", C.POINTER(C.c_uint32)),
                ("cut_values", C.POINTER(C.c_float)), ("is_categorical", C.POINTER(C.c_uint8))]

MAX_CAT_BINS = 1024


class Index(C.Structure):
    _fields_ = [("n_rows", C.c_size_t), ("n_cols", C.c_size_t),
                ("row_ptr", C.POINTER(C.c_size_t)), ("row_width", C.c_int),
                ("rows", C.c_void_p), ("col_width", C.c_int), ("cols", C.c_void_p),
                ("missing", C.POINTER(C.c_uint64)), ("dense", C.c_int),
                ("cuts", C.POINTER(Cuts))]


class Params(C.Structure):
    _fields_ = [("eta", C.c_double), ("gamma", C.c_double), ("lambda_", C.c_double),
                ("alpha", C.c_double), ("min_child_weight", C.c_double),
                ("max_delta_step", C.c_double), ("max_depth", C.c_int64),
                ("max_leaves", C.c_int64), ("grow_policy", C.c_int), ("objective", C.c_int),
                ("num_class", C.c_int), ("scale_pos_weight", C.c_float),
                ("monotone", C.POINTER(C.c_int8)), ("n_monotone", C.c_size_t),
                ("max_bin", C.c_int64), ("base_score", C.c_float), ("has_base_score", C.c_int)]


class Split(C.Structure):
    _fields_ = [("loss_chg", C.c_double), ("feature", C.c_uint32), ("bin", C.c_int64),
                ("default_left", C.c_int), ("left_g", C.c_double), ("left_h", C.c_double),
                ("right_g", C.c_double), ("right_h", C.c_double), ("w_left", C.c_double),
                ("w_right", C.c_double), ("categorical", C.c_int), ("cat_left", C.c_uint32 * (1024 // 32))]


class Node(C.Structure):
    _fields_ = [("split_feature", C.c_uint32), ("split_cond", C.c_float),
                ("default_left", C.c_int32), ("left", C.c_int32), ("right", C.c_int32),
                ("leaf_value", C.c_float), ("sum_hess", C.c_float), ("split_gain", C.c_float),
                ("split_bin", C.c_int64), ("stat_g", C.c_double), ("stat_h", C.c_double),
                ("is_categorical", C.c_int32), ("cat_begin", C.c_uint32), ("cat_end", C.c_uint32)]


class ForestDesc(C.Structure):
    _fields_ = [("n_trees", C.c_size_t), ("tree_offset", C.POINTER(C.c_uint32)),
                ("split_feature", C.POINTER(C.c_uint32)), ("split_cond", C.POINTER(C.c_float)),
                ("default_left", C.POINTER(C.c_uint8)), ("left", C.POINTER(C.c_int32)),
                ("right", C.POINTER(C.c_int32)), ("leaf_value", C.POINTER(C.c_float)),
                ("tree_weight", C.POINTER(C.c_float)), ("tree_output", C.POINTER(C.c_uint32)),
                ("n_outputs", C.c_size_t), ("base_score", C.POINTER(C.c_float)),
                ("is_categorical", C.POINTER(C.c_uint8)), ("cat_begin", C.POINTER(C.c_uint32)),
                ("cat_end", C.POINTER(C.c_uint32)), ("categories", C.POINTER(C.c_uint32))]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = C.CDLL(_LIB_PATH)
        P = C.POINTER
        L.or_cuts_from_dense.restype = P(Cuts)
        L.or_cuts_from_dense.argtypes = [C.c_void_p, C.c_size_t, C.c_size_t, C.c_size_t, C.c_void_p, C.c_float]
        L.or_cuts_from_csr.restype = P(Cuts)
        L.or_cuts_from_csr.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t, C.c_size_t, C.c_void_p]
        L.or_cuts_from_dense_typed.restype = P(Cuts)
        L.or_cuts_from_dense_typed.argtypes = L.or_cuts_from_dense.argtypes + [C.c_void_p]
        L.or_cuts_from_csr_typed.restype = P(Cuts)
        L.or_cuts_from_csr_typed.argtypes = L.or_cuts_from_csr.argtypes + [C.c_void_p]
        L.or_cuts_free.argtypes = [P(Cuts)]
        L.or_cuts_total_bins.restype = C.c_size_t
        L.or_cuts_total_bins.argtypes = [P(Cuts)]
        L.or_index_from_dense.restype = P(Index)
        L.or_index_from_dense.argtypes = [C.c_void_p, C.c_size_t, C.c_size_t, C.c_float, P(Cuts)]
        L.or_index_from_csr.restype = P(Index)
        L.or_index_from_csr.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t, P(Cuts)]
        L.or_index_free.argtypes = [P(Index)]
        L.or_index_feature_bin.restype = C.c_int64
        L.or_index_feature_bin.argtypes = [P(Index), C.c_size_t, C.c_size_t]
        L.or_build_hist.argtypes = [P(Index), C.c_void_p, C.c_size_t, C.c_void_p, C.c_void_p]
        L.or_sum_rows.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]
        L.or_sum_order_grain.restype = C.c_size_t
        L.or_sum_order_grain.argtypes = [C.c_int, C.c_size_t, C.c_size_t, C.c_int]
        L.or_evaluate.argtypes = [P(Index), C.c_void_p, C.c_double, C.c_double, C.c_double, C.c_double, P(Params), P(Split)]
        L.or_split_valid.restype = C.c_int
        L.or_split_valid.argtypes = [P(Split), P(Params)]
        L.or_calc_weight.restype = C.c_double
        L.or_calc_weight.argtypes = [C.c_double, C.c_double, P(Params)]
        L.or_node_gain.restype = C.c_float
        L.or_node_gain.argtypes = [C.c_double, C.c_double, C.c_double, C.c_double, P(Params)]
        L.or_sweep_categorical.argtypes = [C.c_void_p, C.c_size_t, C.c_double, C.c_double, C.c_double, C.c_double,
                                           C.c_int, P(Params), C.c_uint32, P(Split)]
        L.or_partition_categorical.restype = C.c_size_t
        L.or_partition_categorical.argtypes = [P(Index), C.c_void_p, C.c_size_t, C.c_uint32, C.c_void_p, C.c_int,
                                               C.c_void_p, C.c_void_p]
        L.or_tree_n_categories.restype = C.c_size_t
        L.or_tree_n_categories.argtypes = [C.c_void_p]
        L.or_tree_categories.restype = P(C.c_uint32)
        L.or_tree_categories.argtypes = [C.c_void_p]
        L.or_partition.restype = C.c_size_t
        L.or_partition.argtypes = [P(Index), C.c_void_p, C.c_size_t, C.c_uint32, C.c_int64, C.c_int, C.c_void_p, C.c_void_p]
        L.or_grow_tree.restype = C.c_void_p
        L.or_grow_tree.argtypes = [P(Index), C.c_void_p, P(Params), C.c_void_p]
        L.or_tree_free.argtypes = [C.c_void_p]
        L.or_tree_n_nodes.restype = C.c_size_t
        L.or_tree_n_nodes.argtypes = [C.c_void_p]
        L.or_tree_nodes.restype = P(Node)
        L.or_tree_nodes.argtypes = [C.c_void_p]
        for name in ("or_gradient_squared_error", "or_gradient_logistic"):
            getattr(L, name).argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t, C.c_float, C.c_void_p]
        L.or_gradient_softmax.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t, C.c_void_p]
        L.or_gradient_softmax_scalar.argtypes = L.or_gradient_softmax.argtypes
        L.or_sigmoid.restype = C.c_float
        L.or_sigmoid.argtypes = [C.c_float]
        L.or_base_margins.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, P(Params), C.c_void_p]
        L.or_predict_margin.argtypes = [P(ForestDesc), C.c_void_p, C.c_size_t, C.c_size_t, C.c_float, C.c_void_p, C.c_void_p]
        L.or_predict_margin_lockstep.restype = C.c_int
        L.or_predict_margin_lockstep.argtypes = [P(ForestDesc), C.c_void_p, C.c_size_t, C.c_size_t, C.c_void_p]
        L.or_train.restype = C.c_void_p
        L.or_train.argtypes = [P(Index), C.c_void_p, C.c_void_p, P(Params), C.c_size_t]
        L.or_train_more.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, P(Params), C.c_size_t]
        L.or_model_n_trees.restype = C.c_size_t
        L.or_model_n_trees.argtypes = [C.c_void_p]
        L.or_model_tree.restype = C.c_void_p
        L.or_model_tree.argtypes = [C.c_void_p, C.c_size_t]
        L.or_model_margins.restype = P(C.c_float)
        L.or_model_margins.argtypes = [C.c_void_p]
        L.or_model_base_score.restype = P(C.c_float)
        L.or_model_base_score.argtypes = [C.c_void_p]
        L.or_model_n_outputs.restype = C.c_size_t
        L.or_model_n_outputs.argtypes = [C.c_void_p]
        L.or_model_last_gpair.restype = P(C.c_float)
        L.or_model_last_gpair.argtypes = [C.c_void_p]
        L.or_model_free.argtypes = [C.c_void_p]
        L.or_set_threads.argtypes = [C.c_int]
        L.or_summary_budget.restype = C.c_size_t
        L.or_summary_budget.argtypes = [C.c_size_t, C.c_size_t]
        L.or_summary_from_sorted.restype = C.c_size_t
        L.or_summary_from_sorted.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]
        L.or_summary_prune.restype = C.c_size_t
        L.or_summary_prune.argtypes = [C.c_void_p, C.c_size_t, C.c_size_t]
        L.or_summary_combine.restype = C.c_size_t
        L.or_summary_combine.argtypes = [C.c_void_p, C.c_size_t, C.c_void_p, C.c_size_t, C.c_void_p]
        L.or_summary_query.restype = C.c_size_t
        L.or_summary_query.argtypes = [C.c_void_p, C.c_size_t, C.c_size_t, C.c_void_p]
        L.or_sketch_trace.restype = C.c_long
        L.or_sketch_trace.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t, C.c_void_p, C.c_size_t,
                                      C.c_void_p, C.c_size_t, C.POINTER(C.c_size_t), C.c_void_p]
        L.or_lossguide_trace.argtypes = [C.c_void_p, C.c_size_t]
        L.or_lossguide_trace_len.restype = C.c_size_t
        _lib = L
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data


def params(objective=OBJ_SQUARED_ERROR, eta=0.3, gamma=0.0, reg_lambda=1.0, alpha=0.0,
           min_child_weight=1.0, max_delta_step=0.0, max_depth=6, max_leaves=0,
           grow_policy=GROW_DEPTHWISE, num_class=0, scale_pos_weight=1.0, monotone=None,
           max_bin=256, base_score=None):
    p = Params(eta, gamma, reg_lambda, alpha, min_child_weight, max_delta_step, max_depth,
               max_leaves, grow_policy, objective, num_class, scale_pos_weight, None, 0,
               max_bin, 0.0 if base_score is None else base_score, base_score is not None)
    if monotone is not None:
        arr = (C.c_int8 * len(monotone))(*monotone)
        p.monotone = C.cast(arr, C.POINTER(C.c_int8))
        p.n_monotone = len(monotone)
        p._keep = arr
    return p


class Dataset:
    """Cuts plus the binned index of a dense f32 matrix (or CSR)."""

    def __init__(self, x=None, max_bin=256, weights=None, missing=np.nan, csr=None, n_cols=None,
                 feature_types=None):
        """feature_types: per feature "c" (categorical) or "q" (numeric),
        or None for every feature numeric."""
        L = lib()
        self._keep = []
        cat = None
        if feature_types is not None:
            cat = np.array([1 if t in ("c", "categorical") else 0 for t in feature_types], np.uint8)
            self._keep.append(cat)
        if csr is not None:
            row_ptr, col, val = (np.ascontiguousarray(csr[0], np.uintp),
                                 np.ascontiguousarray(csr[1], np.uint32),
                                 np.ascontiguousarray(csr[2], np.float32))
            n = len(row_ptr) - 1
            self._keep += [row_ptr, col, val]
            w = None if weights is None else np.ascontiguousarray(weights, np.float32)
            self.cuts = L.or_cuts_from_csr_typed(_ptr(row_ptr), _ptr(col), _ptr(val), n, n_cols, max_bin, _ptr(w),
                                                 _ptr(cat))
            self.index = L.or_index_from_csr(_ptr(row_ptr), _ptr(col), _ptr(val), n, n_cols, self.cuts)
            self.n_rows, self.n_cols = n, n_cols
        else:
            x = np.ascontiguousarray(x, np.float32)
            n, f = x.shape
            w = None if weights is None else np.ascontiguousarray(weights, np.float32)
            self.cuts = L.or_cuts_from_dense_typed(_ptr(x), n, f, max_bin, _ptr(w), missing, _ptr(cat))
            self.index = L.or_index_from_dense(_ptr(x), n, f, missing, self.cuts)
            self.n_rows, self.n_cols = n, f

    def __del__(self):
        try:
            L = lib()
            L.or_index_free(self.index)
            L.or_cuts_free(self.cuts)
        except Exception:
            pass

    @property
    def feature_offset(self):
        c = self.cuts.contents
        return np.ctypeslib.as_array(c.feature_offset, shape=(c.n_features + 1,)).copy()

    @property
    def cut_values(self):
        c = self.cuts.contents
        total = int(self.feature_offset[-1])
        return np.ctypeslib.as_array(c.cut_values, shape=(total,)).copy()

    @property
    def total_bins(self):
        return int(self.feature_offset[-1])

    @property
    def dense(self):
        return bool(self.index.contents.dense)

    def row_bins(self):
        """(row_ptr, global bins) of the CSR row store."""
        ix = self.index.contents
        n = ix.n_rows
        row_ptr = np.ctypeslib.as_array(ix.row_ptr, shape=(n + 1,)).copy()
        nnz = int(row_ptr[-1])
        dt = np.uint16 if ix.row_width == 2 else np.uint32
        buf = (C.c_char * (nnz * ix.row_width)).from_address(ix.rows)
        return row_ptr, np.frombuffer(buf, dtype=dt).copy()

    def columns(self):
        """(local bins [f][r], missing bitmap or None), or None without columns."""
        ix = self.index.contents
        if ix.col_width == 0:
            return None
        n, f = ix.n_rows, ix.n_cols
        dt = {1: np.uint8, 2: np.uint16, 4: np.uint32}[ix.col_width]
        buf = (C.c_char * (n * f * ix.col_width)).from_address(ix.cols)
        cols = np.frombuffer(buf, dtype=dt).reshape(f, n).copy()
        miss = None
        if ix.missing:
            words = (n + 63) // 64
            miss = np.ctypeslib.as_array(ix.missing, shape=(f * words,)).copy()
        return cols, miss

    def feature_bins(self):
        """[n][f] int64 global bins, -1 for missing."""
        L = lib()
        out = np.empty((self.n_rows, self.n_cols), np.int64)
        for r in range(self.n_rows):
            for f in range(self.n_cols):
                out[r, f] = L.or_index_feature_bin(self.index, r, f)
        return out

    def build_hist(self, rows, gpair):
        rows = np.ascontiguousarray(rows, np.uint32)
        gpair = np.ascontiguousarray(gpair, np.float32)
        out = np.empty(2 * self.total_bins, np.float64)
        lib().or_build_hist(self.index, _ptr(rows), len(rows), _ptr(gpair), _ptr(out))
        return out.reshape(-1, 2)

    def evaluate(self, hist, total, p, lower=-np.inf, upper=np.inf):
        hist = np.ascontiguousarray(hist, np.float64)
        s = Split()
        lib().or_evaluate(self.index, _ptr(hist), total[0], total[1], lower, upper, C.byref(p), C.byref(s))
        return s

    def partition(self, rows, feature, bin_, default_left):
        rows = np.ascontiguousarray(rows, np.uint32)
        left = np.empty(len(rows), np.uint32)
        right = np.empty(len(rows), np.uint32)
        nl = lib().or_partition(self.index, _ptr(rows), len(rows), feature, bin_, int(default_left), _ptr(left), _ptr(right))
        return left[:nl].copy(), right[: len(rows) - nl].copy()

    def grow_tree(self, gpair, p):
        gpair = np.ascontiguousarray(gpair, np.float32)
        leaf = np.empty(self.n_rows, np.int32)
        t = lib().or_grow_tree(self.index, _ptr(gpair), C.byref(p), _ptr(leaf))
        nodes = tree_nodes(t)
        lib().or_tree_free(t)
        return nodes, leaf


def tree_nodes(t):
    """A tree's nodes as dicts; a categorical split's node lists its
    categories (going left) under "categories"."""
    L = lib()
    n = L.or_tree_n_nodes(t)
    arr = L.or_tree_nodes(t)
    nc = L.or_tree_n_categories(t)
    pool = np.ctypeslib.as_array(L.or_tree_categories(t), shape=(nc,)).tolist() if nc else []
    out = []
    for i in range(n):
        nd = arr[i]
        out.append(dict(split_feature=nd.split_feature, split_cond=nd.split_cond,
                        default_left=bool(nd.default_left), left=nd.left, right=nd.right,
                        leaf_value=nd.leaf_value, sum_hess=nd.sum_hess, split_gain=nd.split_gain,
                        split_bin=nd.split_bin, stat_g=nd.stat_g, stat_h=nd.stat_h,
                        is_categorical=bool(nd.is_categorical),
                        categories=pool[nd.cat_begin:nd.cat_end] if nd.is_categorical else []))
    return out


def sum_rows(gpair, rows):
    gpair = np.ascontiguousarray(gpair, np.float32)
    rows = np.ascontiguousarray(rows, np.uint32)
    out = np.empty(2, np.float64)
    lib().or_sum_rows(_ptr(gpair), _ptr(rows), len(rows), _ptr(out))
    return out


def gradient(objective, preds, labels, weights=None, scale_pos_weight=1.0, num_class=0, scalar_rows=False):
    preds = np.ascontiguousarray(preds, np.float32)
    labels = np.ascontiguousarray(labels, np.float32)
    w = None if weights is None else np.ascontiguousarray(weights, np.float32)
    n = len(labels)
    L = lib()
    if objective == OBJ_SOFTMAX:
        out = np.empty(2 * n * num_class, np.float32)
        fn = L.or_gradient_softmax_scalar if scalar_rows else L.or_gradient_softmax
        fn(_ptr(preds), _ptr(labels), _ptr(w), n, num_class, _ptr(out))
        return out.reshape(n, num_class, 2)
    out = np.empty(2 * n, np.float32)
    fn = L.or_gradient_squared_error if objective == OBJ_SQUARED_ERROR else L.or_gradient_logistic
    fn(_ptr(preds), _ptr(labels), _ptr(w), n, scale_pos_weight, _ptr(out))
    return out.reshape(n, 2)


def base_margins(labels, p, weights=None):
    labels = np.ascontiguousarray(labels, np.float32)
    w = None if weights is None else np.ascontiguousarray(weights, np.float32)
    out = np.zeros(64, np.float32)
    lib().or_base_margins(_ptr(labels), _ptr(w), len(labels), C.byref(p), _ptr(out))
    k = p.num_class if p.objective == OBJ_SOFTMAX else 1
    return out[:k].copy()


class Model:
    def __init__(self, ds: Dataset, labels, p, rounds, weights=None):
        self.ds = ds
        self.labels = np.ascontiguousarray(labels, np.float32)
        self.weights = None if weights is None else np.ascontiguousarray(weights, np.float32)
        self.p = p
        self.h = lib().or_train(ds.index, _ptr(self.labels), _ptr(self.weights), C.byref(p), rounds)

    def more(self, rounds):
        lib().or_train_more(self.h, _ptr(self.labels), _ptr(self.weights), C.byref(self.p), rounds)

    def __del__(self):
        try:
            lib().or_model_free(self.h)
        except Exception:
            pass

    @property
    def n_outputs(self):
        return lib().or_model_n_outputs(self.h)

    def trees(self):
        L = lib()
        return [tree_nodes(L.or_model_tree(self.h, i)) for i in range(L.or_model_n_trees(self.h))]

    def margins(self):
        k = self.n_outputs
        return np.ctypeslib.as_array(lib().or_model_margins(self.h), shape=(self.ds.n_rows * k,)).copy()

    def base_score(self):
        return np.ctypeslib.as_array(lib().or_model_base_score(self.h), shape=(self.n_outputs,)).copy()

    def last_gpair(self):
        k = self.n_outputs
        return np.ctypeslib.as_array(lib().or_model_last_gpair(self.h), shape=(self.ds.n_rows * k * 2,)).copy()


def forest_arrays(trees, tree_weight=None, tree_output=None, n_outputs=1, base_score=(0.0,)):
    """Flatten per-tree node dicts into the arrays or_predict_margin reads."""
    off = [0]
    feat, cond, dl, left, right, leaf = [], [], [], [], [], []
    isc, cb, ce, pool = [], [], [], []
    for t in trees:
        if isinstance(t, dict):  # one array per field (categories: the tree's pool, by ranges)
            tp = list(t.get("categories", []))
            t = [dict(split_feature=int(t["split_feature"][i]), split_cond=float(t["split_cond"][i]),
                      default_left=bool(t["default_left"][i]), left=int(t["left"][i]), right=int(t["right"][i]),
                      leaf_value=float(t["leaf_value"][i]),
                      is_categorical=bool(t["is_categorical"][i]) if "is_categorical" in t else False,
                      categories=tp[int(t["cat_begin"][i]):int(t["cat_end"][i])] if "is_categorical" in t
                      and t["is_categorical"][i] else [])
                 for i in range(len(t["left"]))]
        for nd in t:
            feat.append(nd["split_feature"])
            cond.append(nd["split_cond"])
            dl.append(1 if nd["default_left"] else 0)
            left.append(nd["left"])
            right.append(nd["right"])
            leaf.append(nd["leaf_value"])
            c = nd.get("categories", []) if nd.get("is_categorical") else []
            isc.append(1 if nd.get("is_categorical") else 0)
            cb.append(len(pool))
            pool.extend(c)
            ce.append(len(pool))
        off.append(len(feat))
    nt = len(trees)
    arrs = dict(
        tree_offset=np.array(off, np.uint32), split_feature=np.array(feat, np.uint32),
        split_cond=np.array(cond, np.float32), default_left=np.array(dl, np.uint8),
        left=np.array(left, np.int32), right=np.array(right, np.int32),
        leaf_value=np.array(leaf, np.float32),
        tree_weight=np.ones(nt, np.float32) if tree_weight is None else np.asarray(tree_weight, np.float32),
        tree_output=np.zeros(nt, np.uint32) if tree_output is None else np.asarray(tree_output, np.uint32),
        base_score=np.asarray(base_score, np.float32), n_outputs=n_outputs)
    if any(isc):
        arrs.update(is_categorical=np.array(isc, np.uint8), cat_begin=np.array(cb, np.uint32),
                    cat_end=np.array(ce, np.uint32), categories=np.array(pool, np.uint32))
    return arrs


def _forest_desc(arrs):
    """The ForestDesc over `arrs` (forest_arrays' layout), and the arrays it
    points into (kept alive by the caller while the walk runs)."""
    P = C.POINTER
    fd = ForestDesc(len(arrs["tree_offset"]) - 1,
                    arrs["tree_offset"].ctypes.data_as(P(C.c_uint32)),
                    arrs["split_feature"].ctypes.data_as(P(C.c_uint32)),
                    arrs["split_cond"].ctypes.data_as(P(C.c_float)),
                    arrs["default_left"].ctypes.data_as(P(C.c_uint8)),
                    arrs["left"].ctypes.data_as(P(C.c_int32)),
                    arrs["right"].ctypes.data_as(P(C.c_int32)),
                    arrs["leaf_value"].ctypes.data_as(P(C.c_float)),
                    arrs["tree_weight"].ctypes.data_as(P(C.c_float)),
                    arrs["tree_output"].ctypes.data_as(P(C.c_uint32)),
                    arrs["n_outputs"], arrs["base_score"].ctypes.data_as(P(C.c_float)))
    cat = {}
    if arrs.get("is_categorical") is not None:
        cat = {key: np.ascontiguousarray(arrs[key], dt) for key, dt in
               (("is_categorical", np.uint8), ("cat_begin", np.uint32), ("cat_end", np.uint32),
                ("categories", np.uint32))}
        if cat["categories"].size == 0:
            cat["categories"] = np.zeros(1, np.uint32)
        fd.is_categorical = cat["is_categorical"].ctypes.data_as(P(C.c_uint8))
        fd.cat_begin = cat["cat_begin"].ctypes.data_as(P(C.c_uint32))
        fd.cat_end = cat["cat_end"].ctypes.data_as(P(C.c_uint32))
        fd.categories = cat["categories"].ctypes.data_as(P(C.c_uint32))
    return fd, cat


def predict_margin(arrs, x, missing=np.nan, with_leaf=False):
    x = np.ascontiguousarray(x, np.float32)
    n, f = x.shape
    fd, keep = _forest_desc(arrs)
    k = arrs["n_outputs"]
    out = np.empty(n * k, np.float32)
    leaf = np.empty(n * fd.n_trees, np.int32) if with_leaf else None
    lib().or_predict_margin(C.byref(fd), _ptr(x), n, f, missing, _ptr(out), _ptr(leaf))
    del keep
    return (out, leaf.reshape(n, -1)) if with_leaf else out


def predict_margin_lockstep(arrs, x):
    """predict_margin's margins (NaN missing, numeric splits) through the
    reference's 16-row lock-step compact walk; ValueError for a forest that
    walk does not take here."""
    x = np.ascontiguousarray(x, np.float32)
    n, f = x.shape
    fd, keep = _forest_desc(arrs)
    out = np.empty(n * arrs["n_outputs"], np.float32)
    if lib().or_predict_margin_lockstep(C.byref(fd), _ptr(x), n, f, _ptr(out)) != 0:
        raise ValueError("the lock-step walk takes numeric splits with finite conditions on features < n_cols")
    del keep
    return out


def set_threads(n: int) -> None:
    lib().or_set_threads(n)


# ---- the sketch's summary operations (test hooks) --------------------------
# A summary is an (k, 4) f32 array of entries (rmin, rmax, wmin, value).

SUMMARY_KINDS = ("from_sorted", "prune", "combine", "summary", "final")


def summary_budget(max_bin, n):
    return lib().or_summary_budget(max_bin, n)


def summary_from_sorted(values, weights):
    v = np.ascontiguousarray(values, np.float32)
    w = np.ascontiguousarray(weights, np.float32)
    out = np.empty((max(len(v), 1), 4), np.float32)
    k = lib().or_summary_from_sorted(_ptr(v), _ptr(w), len(v), _ptr(out))
    return out[:k].copy()


def summary_prune(entries, maxsize):
    e = np.array(entries, np.float32, copy=True).reshape(-1, 4)
    k = lib().or_summary_prune(_ptr(e), len(e), maxsize)
    return e[:k].copy()


def summary_combine(a, b):
    a = np.ascontiguousarray(a, np.float32).reshape(-1, 4)
    b = np.ascontiguousarray(b, np.float32).reshape(-1, 4)
    out = np.empty((max(len(a) + len(b), 1), 4), np.float32)
    k = lib().or_summary_combine(_ptr(a), len(a), _ptr(b), len(b), _ptr(out))
    return out[:k].copy()


def summary_query(entries, max_bin):
    e = np.ascontiguousarray(entries, np.float32).reshape(-1, 4)
    out = np.empty(max_bin + 2, np.float32)
    k = lib().or_summary_query(_ptr(e), len(e), max_bin, _ptr(out))
    return out[:k].copy()


def sketch_trace(values, weights, max_bin, buf_entries=1 << 22, rec_cap=1 << 16):
    """One feature's streaming sketch over `values` (weights None: 1): its
    cut values and every summary it formed, as (kind, lo, hi, entries,
    pruned_to), where [lo, hi) are the indices of the values the summary
    covers and pruned_to the size a prune record was pruned to (else 0)."""
    v = np.ascontiguousarray(values, np.float32)
    w = None if weights is None else np.ascontiguousarray(weights, np.float32)
    buf = np.empty((buf_entries, 4), np.float32)
    recs = np.empty((rec_cap, 6), np.uint64)
    n_recs = C.c_size_t()
    cuts = np.empty(max_bin + 2, np.float32)
    k = lib().or_sketch_trace(_ptr(v), _ptr(w), len(v), max_bin, _ptr(buf), buf_entries, _ptr(recs), rec_cap,
                              C.byref(n_recs), _ptr(cuts))
    if k < 0:
        raise RuntimeError("sketch trace: buffers too small")
    out = []
    for off, cnt, lo, hi, kind, size in recs[:n_recs.value].tolist():
        out.append((SUMMARY_KINDS[kind], lo, hi, buf[off:off + cnt].copy(), size))
    return cuts[:k].copy(), out


def lossguide_events(ds, gpair, p, cap=1 << 16):
    """Grow one tree and return it with its loss-guided queue's events:
    (kind "push" / "pop", node id, loss_chg, expandable) in order."""
    buf = np.zeros((cap, 4), np.uint64)
    lib().or_lossguide_trace(_ptr(buf), cap)
    try:
        nodes, _ = ds.grow_tree(gpair, p)
        n = lib().or_lossguide_trace_len()
    finally:
        lib().or_lossguide_trace(None, 0)
    ev = [("push" if k == 0 else "pop", int(nid), float(np.array([bits], np.uint64).view(np.float64)[0]), bool(x))
          for k, nid, bits, x in buf[:n].tolist()]
    return nodes, ev
