"""ctypes binding of libhbrocm.so (include/hessboost_rocm.h).

The library and its gfx950 code object are built in-tree by
``make -C hessboost_amd/csrc`` (or ``__graft_entry__.build()``); loading
fails loudly when they are missing, so no call silently runs elsewhere.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

LIB_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib")
LIB_PATH = os.path.join(LIB_DIR, "libhbrocm.so")
CODE_OBJECT = os.path.join(LIB_DIR, "hbrocm_gfx950.hsaco")

OK, REFUSED, DEVICE_ERROR, INVALID = 0, 1, 2, 3
SUMS_EXACT, SUMS_FIXED_POINT = 0, 1
GUARD_OFF, GUARD_REPLAY, GUARD_RESOLVE = 0, 1, 2
LOSS_SQUARED_ERROR, LOSS_LOGISTIC, LOSS_SOFTMAX = 0, 1, 2
OBJ_SQUARED_ERROR, OBJ_LOGISTIC, OBJ_SOFTMAX, OBJ_LOGITRAW = 0, 1, 2, 3
GROW_DEPTHWISE, GROW_LOSSGUIDE = 0, 1
SCAN_EMPTY, SCAN_REPLAY, SCAN_NUMERIC, SCAN_CATEGORICAL = 0, 1, 2, 3
FALLBACK_NUMERIC_SCORE, FALLBACK_CATEGORICAL_ORDER, FALLBACK_CATEGORICAL_SCORE, FALLBACK_NEAR_TIE = 1, 2, 3, 4
TRANSFORM_SIGMOID, TRANSFORM_SOFTMAX, TRANSFORM_CLASS_INDEX = 1, 2, 3

P = C.POINTER
u32p, u64p, i64p, f32p, f64p, u8p, i8p, i32p = (P(C.c_uint32), P(C.c_uint64), P(C.c_int64), P(C.c_float),
                                                 P(C.c_double), P(C.c_uint8), P(C.c_int8), P(C.c_int32))


class HbrError(RuntimeError):
    def __init__(self, status, message):
        super().__init__(f"[{ {1: 'refused', 2: 'device error', 3: 'invalid'}.get(status, status)}] {message}")
        self.status = status


class IndexDesc(C.Structure):
    _fields_ = [("n_rows", C.c_uint64), ("n_cols", C.c_uint64), ("feature_offset", u32p),
                ("cut_values", f32p), ("row_ptr", u64p), ("row_bins", C.c_void_p),
                ("row_bin_width", C.c_uint32), ("dense", C.c_uint32), ("col_bins", C.c_void_p),
                ("col_bin_width", C.c_uint32), ("pad", C.c_uint32), ("missing", u64p),
                ("is_categorical", C.POINTER(C.c_uint8))]


class IndexInfo(C.Structure):
    _fields_ = [("dense", C.c_uint32), ("dense_u8", C.c_uint32), ("has_cols", C.c_uint32),
                ("has_missing", C.c_uint32), ("stride", C.c_uint32), ("pad", C.c_uint32),
                ("entries", C.c_uint64)]


class Segment(C.Structure):
    _fields_ = [("offset", C.c_uint64), ("len", C.c_uint64), ("buffer", C.c_uint32),
                ("contiguous", C.c_uint32), ("tree", C.c_uint64)]


class RowSplit(C.Structure):
    _fields_ = [("seg", Segment), ("feature", C.c_uint32), ("below", C.c_uint32),
                ("default_left", C.c_uint32), ("n_table", C.c_uint32), ("table", u8p)]


class Partitioned(C.Structure):
    _fields_ = [("left", Segment), ("right", Segment)]


class DeviceLoss(C.Structure):
    _fields_ = [("kind", C.c_uint32), ("scale_pos_weight", C.c_float), ("min_hess", C.c_float),
                ("max_input", C.c_float), ("vector_rows", C.c_uint64)]


class RegParams(C.Structure):
    _fields_ = [("lambda_", C.c_double), ("alpha", C.c_double), ("max_delta_step", C.c_double),
                ("min_child_weight", C.c_double)]


class ScanRequest(C.Structure):
    _fields_ = [("slot", C.c_uint32), ("has_fixed", C.c_uint32), ("total_g", C.c_double),
                ("total_h", C.c_double), ("fixed_g", C.c_int64), ("fixed_h", C.c_int64),
                ("root_gain", C.c_float), ("lower", C.c_float), ("upper", C.c_float),
                ("n_features", C.c_uint32), ("features", u32p), ("directions", i8p)]


class NodeScan(C.Structure):
    _fields_ = [("kind", C.c_uint32), ("feature", C.c_uint32), ("loss_chg", C.c_float),
                ("backward", C.c_uint32), ("offset", C.c_uint32), ("loss_err", C.c_float),
                ("acc_g", C.c_double), ("acc_h", C.c_double), ("left_g", C.c_double),
                ("left_h", C.c_double), ("right_g", C.c_double), ("right_h", C.c_double),
                ("fixed_left_g", C.c_int64), ("fixed_left_h", C.c_int64),
                ("fixed_right_g", C.c_int64), ("fixed_right_h", C.c_int64),
                ("default_left", C.c_uint32), ("fallback", C.c_uint32), ("cat_begin", C.c_uint32),
                ("cat_end", C.c_uint32)]


class EngineCounters(C.Structure):
    _fields_ = [("hist_nodes", C.c_uint64), ("hist_rows", C.c_uint64), ("hist_bytes", C.c_uint64),
                ("partition_rows", C.c_uint64), ("trees", C.c_uint64), ("near_ties", C.c_uint64),
                ("near_ties_resolved", C.c_uint64), ("row_orders", C.c_uint64)]


class TrainParams(C.Structure):
    _fields_ = [("eta", C.c_double), ("gamma", C.c_double), ("lambda_", C.c_double), ("alpha", C.c_double),
                ("min_child_weight", C.c_double), ("max_delta_step", C.c_double),
                ("max_depth", C.c_int64), ("max_leaves", C.c_int64), ("grow_policy", C.c_int32),
                ("objective", C.c_int32), ("num_class", C.c_int32), ("scale_pos_weight", C.c_float),
                ("monotone", i8p), ("n_monotone", C.c_uint64), ("base_score", C.c_float),
                ("has_base_score", C.c_int32)]


class ForestDesc(C.Structure):
    _fields_ = [("n_trees", C.c_uint64), ("tree_offset", u64p), ("split_feature", u32p),
                ("split_cond", f32p), ("default_left", u8p), ("left", i32p), ("right", i32p),
                ("leaf_value", f32p), ("tree_weight", f32p), ("tree_output", u32p),
                ("n_outputs", C.c_uint32), ("pad", C.c_uint32), ("base_score", f32p),
                ("is_categorical", u8p), ("cat_begin", u32p), ("cat_end", u32p), ("categories", u32p),
                ("n_categories", C.c_uint64)]


# name -> (restype, argtypes); every entry point include/hessboost_rocm.h declares
SIGNATURES = {
    "hbr_last_error": (C.c_size_t, [C.c_char_p, C.c_size_t]),
    "hbr_device_count": (C.c_int, [P(C.c_int)]),
    "hbr_device_name": (C.c_int, [C.c_int, C.c_char_p, C.c_size_t]),
    "hbr_cuts_from_dense": (C.c_int, [C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint32, C.c_void_p, C.c_float, P(C.c_void_p)]),
    "hbr_cuts_from_csr": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint32, C.c_void_p, P(C.c_void_p)]),
    "hbr_cuts_from_values": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint64, P(C.c_void_p)]),
    "hbr_cuts_info": (C.c_int, [C.c_void_p, P(C.c_uint64), P(C.c_uint64)]),
    "hbr_cuts_copy": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p]),
    "hbr_cuts_from_dense_typed": (C.c_int, [C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint32, C.c_void_p, C.c_float,
                                            C.c_void_p, P(C.c_void_p)]),
    "hbr_cuts_from_csr_typed": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint32,
                                          C.c_void_p, C.c_void_p, P(C.c_void_p)]),
    "hbr_cuts_categorical": (C.c_int, [C.c_void_p, C.c_void_p]),
    "hbr_trainer_tree_categories": (C.c_int, [C.c_void_p, C.c_uint64, C.c_void_p, C.c_void_p, C.c_void_p,
                                              C.c_void_p, P(C.c_uint64)]),
    "hbr_cuts_free": (None, [C.c_void_p]),
    "hbr_index_from_dense": (C.c_int, [C.c_void_p, C.c_uint64, C.c_uint64, C.c_float, C.c_void_p, P(C.c_void_p)]),
    "hbr_index_from_csr": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint64, C.c_uint64, C.c_void_p, P(C.c_void_p)]),
    "hbr_index_free": (None, [C.c_void_p]),
    "hbr_index_describe": (C.c_int, [C.c_void_p, P(IndexDesc)]),
    "hbr_engine_open": (C.c_int, [C.c_int, P(IndexDesc), P(C.c_void_p)]),
    "hbr_engine_close": (None, [C.c_void_p]),
    "hbr_engine_open_dense": (C.c_int, [C.c_int, C.c_void_p, C.c_uint64, C.c_uint64, C.c_float, C.c_void_p,
                                        C.c_int, P(C.c_void_p)]),
    "hbr_engine_index_info": (C.c_int, [C.c_void_p, P(IndexInfo)]),
    "hbr_engine_index_read": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                        C.c_void_p]),
    "hbr_prepare": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint64]),
    "hbr_engine_set_sums": (C.c_int, [C.c_void_p, C.c_int]),
    "hbr_build": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint64, C.c_void_p]),
    "hbr_build_device_noalloc": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint64, C.c_void_p]),
    "hbr_begin_tree": (C.c_int, [C.c_void_p, C.c_uint64, P(Segment)]),
    "hbr_root_total": (C.c_int, [C.c_void_p, P(Segment), C.c_void_p]),
    "hbr_root_total_fixed": (C.c_int, [C.c_void_p, P(Segment), C.c_void_p, C.c_void_p]),
    "hbr_partition": (C.c_int, [C.c_void_p, P(RowSplit), C.c_uint64, P(Partitioned)]),
    "hbr_histograms": (C.c_int, [C.c_void_p, P(Segment), C.c_uint64, C.c_void_p]),
    "hbr_rows": (C.c_int, [C.c_void_p, P(Segment), C.c_void_p]),
    "hbr_load_margins": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint64, C.c_uint32]),
    "hbr_gradients": (C.c_int, [C.c_void_p, P(DeviceLoss), C.c_void_p, C.c_void_p, C.c_uint64, P(C.c_int)]),
    "hbr_add_leaf_values": (C.c_int, [C.c_void_p, P(Segment), C.c_void_p, C.c_uint64]),
    "hbr_read_gradients": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint64]),
    "hbr_read_margins": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint64]),
    "hbr_reserve_hists": (C.c_int, [C.c_void_p, C.c_uint64, P(C.c_int)]),
    "hbr_build_resident": (C.c_int, [C.c_void_p, P(Segment), C.c_void_p, C.c_uint64, C.c_void_p, C.c_void_p, C.c_uint64]),
    "hbr_scan_resident": (C.c_int, [C.c_void_p, P(RegParams), P(ScanRequest), C.c_uint64, P(NodeScan)]),
    "hbr_scan_categories": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint64]),
    "hbr_read_hist": (C.c_int, [C.c_void_p, C.c_uint32, C.c_void_p]),
    "hbr_engine_set_guard": (C.c_int, [C.c_void_p, C.c_int, C.c_double]),
    "hbr_node_gain": (C.c_int, [P(RegParams), C.c_double, C.c_double, C.c_double, C.c_double, P(C.c_float)]),
    "hbr_leaf_weight": (C.c_int, [P(RegParams), C.c_double, C.c_double, C.c_double, C.c_double, P(C.c_float)]),
    "hbr_engine_counters_read": (C.c_int, [C.c_void_p, P(EngineCounters)]),
    "hbr_set_profiling": (C.c_int, [C.c_void_p, C.c_int, C.c_char_p]),
    "hbr_kernel_stats": (C.c_int, [C.c_void_p, C.c_char_p, C.c_size_t]),
    "hbr_trainer_create": (C.c_int, [C.c_void_p, P(TrainParams), C.c_void_p, C.c_void_p, C.c_uint64, P(C.c_void_p)]),
    "hbr_trainer_boost": (C.c_int, [C.c_void_p, C.c_uint64]),
    "hbr_trainer_num_trees": (C.c_int, [C.c_void_p, P(C.c_uint64)]),
    "hbr_trainer_num_outputs": (C.c_int, [C.c_void_p, P(C.c_uint32)]),
    "hbr_trainer_base_score": (C.c_int, [C.c_void_p, C.c_void_p]),
    "hbr_trainer_tree_size": (C.c_int, [C.c_void_p, C.c_uint64, P(C.c_uint64)]),
    "hbr_trainer_tree": (C.c_int, [C.c_void_p, C.c_uint64] + [C.c_void_p] * 9),
    "hbr_trainer_margins": (C.c_int, [C.c_void_p, C.c_void_p]),
    "hbr_engine_add_eval": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint64, C.c_uint64, C.c_float, C.c_void_p,
                                      C.c_uint32, P(C.c_uint32)]),
    "hbr_engine_eval_add_tree": (C.c_int, [C.c_void_p] + [C.c_void_p] * 6 + [C.c_uint64, C.c_uint32]),
    "hbr_engine_eval_add_tree_categorical": (C.c_int, [C.c_void_p] + [C.c_void_p] * 10 +
                                             [C.c_uint64, C.c_uint64, C.c_uint32]),
    "hbr_engine_eval_margins": (C.c_int, [C.c_void_p, C.c_uint32, C.c_void_p]),
    "hbr_trainer_add_eval": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint64, C.c_uint64, C.c_float, C.c_void_p,
                                       P(C.c_uint32)]),
    "hbr_trainer_eval_margins": (C.c_int, [C.c_void_p, C.c_uint32, C.c_void_p]),
    "hbr_trainer_free": (None, [C.c_void_p]),
    "hbr_forest_upload": (C.c_int, [C.c_int, P(ForestDesc), P(C.c_void_p)]),
    "hbr_forest_free": (None, [C.c_void_p]),
    "hbr_predict_margin": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint64, C.c_uint64, C.c_float, C.c_void_p]),
    "hbr_predict_margin_device": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint64, C.c_uint64, C.c_float, C.c_void_p, C.c_void_p]),
    "hbr_predict_leaf": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint64, C.c_uint64, C.c_float, C.c_void_p]),
    "hbr_predict_margin_from": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint64, C.c_uint64, C.c_float, C.c_void_p,
                                          C.c_void_p]),
    "hbr_pred_transform": (C.c_int, [C.c_int, C.c_void_p, C.c_uint64, C.c_uint32]),
    "hbr_forest_set_profiling": (C.c_int, [C.c_void_p, C.c_int, C.c_char_p]),
    "hbr_forest_kernel_stats": (C.c_int, [C.c_void_p, C.c_char_p, C.c_size_t]),
    "hbr_device_alloc": (C.c_int, [C.c_int, C.c_uint64, P(C.c_void_p)]),
    "hbr_device_free": (C.c_int, [C.c_int, C.c_void_p]),
    "hbr_device_upload": (C.c_int, [C.c_int, C.c_void_p, C.c_void_p, C.c_uint64]),
    "hbr_device_download": (C.c_int, [C.c_int, C.c_void_p, C.c_void_p, C.c_uint64]),
    "hbr_device_copy": (C.c_int, [C.c_int, C.c_void_p, C.c_void_p, C.c_uint64]),
}

_lib = None


def lib():
    """The loaded library; raises when it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH) or not os.path.exists(CODE_OBJECT):
            raise ImportError(f"the MI355X backend is not built ({LIB_PATH}); run "
                              "`make -C hessboost_amd/csrc` or __graft_entry__.build()")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error() -> str:
    buf = C.create_string_buffer(4096)
    lib().hbr_last_error(buf, len(buf))
    return buf.value.decode(errors="replace")


def check(status: int) -> None:
    if status != OK:
        raise HbrError(status, last_error())


def ptr(a):
    return None if a is None else C.c_void_p(a.ctypes.data)


def typed(a, ctype):
    return None if a is None else a.ctypes.data_as(P(ctype))


def kernel_stats(text: str) -> dict:
    """Parse hbr_kernel_stats' "name=ms,timed,launches;" list into
    name -> (ms over the timed launches, timed launches, launches)."""
    out = {}
    for item in filter(None, text.split(";")):
        name, rest = item.split("=")
        ms, timed, n = rest.split(",")
        out[name] = (float(ms), int(timed), int(n))
    return out
