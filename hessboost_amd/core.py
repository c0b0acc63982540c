"""Python mirror of hessboost's hist training and prediction API on MI355X.

``DMatrix``, ``train`` and ``Booster.predict`` keep the reference's names and
argument meaning (python/python/hessboost/_training.py, _booster.py) for
the `tree_method=hist` path; every computation runs in libhbrocm.so (cuts and
binning on the host, growth and prediction on the GPU).
"""
from __future__ import annotations

import ctypes as C
import json
import math
from dataclasses import dataclass, field

import numpy as np

from . import _capi as A


# ---- cuts and the binned index ---------------------------------------------------

def _categorical_flags(feature_types, n_cols):
    """The DMatrix's feature_types (python/python/hessboost/_data.py: "c" or
    "categorical" marks a categorical feature; "q", "float", "int" numeric)
    as per-feature bytes, or None when every feature is numeric."""
    if feature_types is None:
        return None
    if len(feature_types) != n_cols:
        raise ValueError("feature_types needs one entry per feature")
    flags = np.array([1 if t in ("c", "categorical") else 0 for t in feature_types], np.uint8)
    return flags if flags.any() else None


class Cuts:
    """HistCuts (src/data/quantile.rs:28-296): per-feature cut values."""

    def __init__(self, handle):
        self._h = handle

    @classmethod
    def from_dense(cls, x, max_bin=256, weights=None, missing=np.nan, feature_types=None):
        x = np.ascontiguousarray(x, np.float32)
        w = None if weights is None else np.ascontiguousarray(weights, np.float32)
        cat = _categorical_flags(feature_types, x.shape[1])
        h = C.c_void_p()
        A.check(A.lib().hbr_cuts_from_dense_typed(A.ptr(x), x.shape[0], x.shape[1], max_bin, A.ptr(w),
                                                  float(missing), A.ptr(cat), C.byref(h)))
        return cls(h)

    @classmethod
    def from_csr(cls, row_ptr, col, val, n_cols, max_bin=256, weights=None, feature_types=None):
        row_ptr = np.ascontiguousarray(row_ptr, np.uint64)
        col = np.ascontiguousarray(col, np.uint32)
        val = np.ascontiguousarray(val, np.float32)
        w = None if weights is None else np.ascontiguousarray(weights, np.float32)
        cat = _categorical_flags(feature_types, n_cols)
        h = C.c_void_p()
        A.check(A.lib().hbr_cuts_from_csr_typed(A.ptr(row_ptr), A.ptr(col), A.ptr(val), len(row_ptr) - 1, n_cols,
                                                max_bin, A.ptr(w), A.ptr(cat), C.byref(h)))
        return cls(h)

    def categorical(self):
        """Per feature, whether its bins are categories."""
        n = C.c_uint64()
        A.check(A.lib().hbr_cuts_info(self._h, C.byref(n), None))
        out = np.zeros(n.value, np.uint8)
        A.check(A.lib().hbr_cuts_categorical(self._h, A.ptr(out)))
        return out.astype(bool)

    def __del__(self):
        try:
            A.lib().hbr_cuts_free(self._h)
        except Exception:
            pass

    def arrays(self):
        n, total = C.c_uint64(), C.c_uint64()
        A.check(A.lib().hbr_cuts_info(self._h, C.byref(n), C.byref(total)))
        fo = np.empty(n.value + 1, np.uint32)
        cv = np.empty(total.value, np.float32)
        A.check(A.lib().hbr_cuts_copy(self._h, A.ptr(fo), A.ptr(cv)))
        return fo, cv


class BinnedIndex:
    """GHistIndex (src/data/ghist.rs:195-257) built on the host."""

    def __init__(self, cuts: Cuts, x=None, csr=None, n_cols=None, missing=np.nan):
        self.cuts = cuts
        h = C.c_void_p()
        if csr is not None:
            row_ptr = np.ascontiguousarray(csr[0], np.uint64)
            col = np.ascontiguousarray(csr[1], np.uint32)
            val = np.ascontiguousarray(csr[2], np.float32)
            A.check(A.lib().hbr_index_from_csr(A.ptr(row_ptr), A.ptr(col), A.ptr(val), len(row_ptr) - 1, n_cols,
                                               cuts._h, C.byref(h)))
        else:
            x = np.ascontiguousarray(x, np.float32)
            A.check(A.lib().hbr_index_from_dense(A.ptr(x), x.shape[0], x.shape[1], float(missing), cuts._h,
                                                 C.byref(h)))
        self._h = h
        self.desc = A.IndexDesc()
        A.check(A.lib().hbr_index_describe(h, C.byref(self.desc)))

    def __del__(self):
        try:
            A.lib().hbr_index_free(self._h)
        except Exception:
            pass

    @property
    def n_rows(self):
        return self.desc.n_rows

    @property
    def n_cols(self):
        return self.desc.n_cols

    @property
    def dense(self):
        return bool(self.desc.dense)

    def feature_offset(self):
        return np.ctypeslib.as_array(self.desc.feature_offset, shape=(self.n_cols + 1,)).copy()

    def cut_values(self):
        fo = self.feature_offset()
        return np.ctypeslib.as_array(self.desc.cut_values, shape=(int(fo[-1]),)).copy()

    def row_bins(self):
        d = self.desc
        row_ptr = np.ctypeslib.as_array(d.row_ptr, shape=(d.n_rows + 1,)).copy()
        nnz = int(row_ptr[-1])
        dt = np.uint16 if d.row_bin_width == 2 else np.uint32
        if nnz == 0:
            return row_ptr, np.zeros(0, dt)
        buf = (C.c_char * (nnz * d.row_bin_width)).from_address(d.row_bins)
        return row_ptr, np.frombuffer(buf, dt).copy()

    def columns(self):
        d = self.desc
        if d.col_bin_width == 0:
            return None
        dt = {1: np.uint8, 2: np.uint16, 4: np.uint32}[d.col_bin_width]
        cells = d.n_rows * d.n_cols
        buf = (C.c_char * (cells * d.col_bin_width)).from_address(d.col_bins)
        cols = np.frombuffer(buf, dt).reshape(d.n_cols, d.n_rows).copy()
        miss = None
        if d.missing:
            words = (d.n_rows + 63) // 64
            miss = np.ctypeslib.as_array(d.missing, shape=(words * d.n_cols,)).copy()
        return cols, miss


class DeviceBinnedIndex:
    """The shape and cuts of an index binned on the device
    (Engine.from_dense); its layouts live in the engine only."""

    def __init__(self, cuts: Cuts, n_rows: int, n_cols: int):
        self.cuts = cuts
        self.n_rows = n_rows
        self.n_cols = n_cols
        self._fo, self._cv = cuts.arrays()

    def feature_offset(self):
        return self._fo.copy()

    def cut_values(self):
        return self._cv.copy()


# ---- the device engine (HistogramBackend + RowEngine) ----------------------------------

class Engine:
    """One binned index resident on one GPU (src/tree/hist/mod.rs:73-295)."""

    def __init__(self, index: BinnedIndex, ordinal: int = 0):
        self.index = index
        h = C.c_void_p()
        A.check(A.lib().hbr_engine_open(ordinal, C.byref(index.desc), C.byref(h)))
        self._h = h
        fo = index.feature_offset()
        self.total_bins = int(fo[-1])

    @classmethod
    def from_dense(cls, x, cuts: Cuts, ordinal: int = 0, missing=np.nan, n_rows=None, n_cols=None):
        """The engine over a dense f32 matrix binned on the device against
        `cuts` (hbr_engine_open_dense): the same index hbr_index_from_dense
        builds on the host. `x` is a row-major numpy array, or a DeviceBuffer
        (with n_rows and n_cols) already on this ordinal."""
        self = cls.__new__(cls)
        on_device = isinstance(x, DeviceBuffer)
        if on_device:
            ptr, n, f = C.c_void_p(x.ptr), int(n_rows), int(n_cols)
        else:
            x = np.ascontiguousarray(x, np.float32)
            n, f = x.shape
            ptr = A.ptr(x)
        h = C.c_void_p()
        A.check(A.lib().hbr_engine_open_dense(ordinal, ptr, n, f, float(missing), cuts._h, 1 if on_device else 0,
                                              C.byref(h)))
        self._h = h
        self.index = DeviceBinnedIndex(cuts, n, f)
        self.total_bins = int(self.index.feature_offset()[-1])
        return self

    def index_info(self):
        i = A.IndexInfo()
        A.check(A.lib().hbr_engine_index_info(self._h, C.byref(i)))
        return {k: int(getattr(i, k)) for k in ("dense", "dense_u8", "has_cols", "has_missing", "stride", "entries")}

    def read_index(self):
        """The engine's device layouts as numpy arrays (absent ones are None)."""
        info = self.index_info()
        n, f = self.index.n_rows, self.index.n_cols
        words = (n + 63) // 64
        rows8 = np.empty((n, info["stride"]), np.uint8) if info["dense_u8"] else None
        cols8 = np.empty((f, n), np.uint8) if info["has_cols"] else None
        miss = np.empty(f * words, np.uint64) if info["has_missing"] else None
        row_ptr = np.empty(n + 1, np.uint64) if not info["dense"] else None
        gbins = np.empty(info["entries"], np.uint32) if not info["dense"] else None
        A.check(A.lib().hbr_engine_index_read(self._h, A.ptr(rows8), A.ptr(cols8), A.ptr(miss), A.ptr(row_ptr),
                                              A.ptr(gbins)))
        return {"rows8": rows8, "cols8": cols8, "missing": miss, "row_ptr": row_ptr, "gbins": gbins, **info}

    def close(self):
        if getattr(self, "_h", None):
            A.lib().hbr_engine_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_sums(self, mode):
        """"exact" (the default): build / histograms / root_total / the
        resident scan refuse outside the exact domain, where they could not
        equal the CPU's f64 sums (src/backend/exact_sum.rs:14-37);
        "fixed_point": they return the engine's fixed-point sums anyway."""
        code = {"exact": A.SUMS_EXACT, "fixed_point": A.SUMS_FIXED_POINT}[mode]
        A.check(A.lib().hbr_engine_set_sums(self._h, code))

    def set_guard(self, mode="resolve", gamma=0.0):
        """The fixed-point guard of the resident scan: a node whose winner
        its sums cannot certify is searched again on the CPU builder's sums
        on the device ("resolve", the default), reported for a host replay
        ("replay"), or left as it is ("off"); gamma is the split threshold
        it checks. The trainer counts such nodes."""
        code = {"off": A.GUARD_OFF, "replay": A.GUARD_REPLAY, "resolve": A.GUARD_RESOLVE}[mode]
        A.check(A.lib().hbr_engine_set_guard(self._h, code, float(gamma)))

    def prepare(self, gpair):
        gpair = np.ascontiguousarray(gpair, np.float32).reshape(-1)
        A.check(A.lib().hbr_prepare(self._h, A.ptr(gpair), len(gpair) // 2))

    def build(self, rows):
        rows = np.ascontiguousarray(rows, np.uint32)
        out = np.empty(2 * self.total_bins, np.float64)
        A.check(A.lib().hbr_build(self._h, A.ptr(rows), len(rows), A.ptr(out)))
        return out.reshape(-1, 2)

    def begin_tree(self):
        seg = A.Segment()
        A.check(A.lib().hbr_begin_tree(self._h, self.index.n_rows, C.byref(seg)))
        return seg

    def root_total(self, seg, fixed=False):
        out = np.empty(2, np.float64)
        fx = np.empty(2, np.int64)
        A.check(A.lib().hbr_root_total_fixed(self._h, C.byref(seg), A.ptr(out), A.ptr(fx)))
        return (out, fx) if fixed else out

    def partition(self, splits):
        """splits: [(segment, feature, rule, default_left)] -> [(left, right)];
        rule is RowRule::Below's limit (an int) or RowRule::Table's per-bin
        directions (a sequence of bools, one per bin of the feature)."""
        arr = (A.RowSplit * len(splits))()
        keep = []
        for i, (seg, f, rule, dl) in enumerate(splits):
            arr[i].seg = seg
            arr[i].feature = f
            arr[i].default_left = int(dl)
            if np.ndim(rule) == 0:
                arr[i].below = int(rule)
            else:
                table = np.ascontiguousarray(rule, np.uint8)
                keep.append(table)
                arr[i].n_table = table.size
                arr[i].table = A.typed(table, C.c_uint8)
        out = (A.Partitioned * len(splits))()
        A.check(A.lib().hbr_partition(self._h, arr, len(splits), out))
        return [(out[i].left, out[i].right) for i in range(len(splits))]

    def histograms(self, segs):
        arr = (A.Segment * len(segs))(*segs)
        out = np.empty(len(segs) * 2 * self.total_bins, np.float64)
        A.check(A.lib().hbr_histograms(self._h, arr, len(segs), A.ptr(out)))
        return out.reshape(len(segs), -1, 2)

    def rows(self, seg):
        out = np.empty(seg.len, np.uint32)
        A.check(A.lib().hbr_rows(self._h, C.byref(seg), A.ptr(out)))
        return out

    def load_margins(self, margins, n_outputs=1):
        m = np.ascontiguousarray(margins, np.float32).reshape(-1)
        A.check(A.lib().hbr_load_margins(self._h, A.ptr(m), len(m), n_outputs))

    def gradients(self, kind, labels, weights=None, scale_pos_weight=1.0):
        n = self.index.n_rows
        loss = A.DeviceLoss(kind, scale_pos_weight, 1e-16, 80.0, n - n % 8 if n >= 16 else 0)
        labels = np.ascontiguousarray(labels, np.float32)
        w = None if weights is None else np.ascontiguousarray(weights, np.float32)
        ok = C.c_int()
        A.check(A.lib().hbr_gradients(self._h, C.byref(loss), A.ptr(labels), A.ptr(w), n, C.byref(ok)))
        return bool(ok.value)

    def read_gradients(self, n_classes=1):
        """The staged pairs, (n_rows, 2); after softmax gradients of k
        classes, n_classes=k gives every class's, (k, n_rows, 2)."""
        n = self.index.n_rows * n_classes
        out = np.empty(2 * n, np.float32)
        A.check(A.lib().hbr_read_gradients(self._h, A.ptr(out), n))
        return out.reshape(-1, 2) if n_classes == 1 else out.reshape(n_classes, -1, 2)

    def add_leaf_values(self, segs, values):
        arr = (A.Segment * len(segs))(*segs)
        v = np.ascontiguousarray(values, np.float32)
        A.check(A.lib().hbr_add_leaf_values(self._h, arr, A.ptr(v), len(segs)))

    def read_margins(self, n):
        out = np.empty(n, np.float32)
        A.check(A.lib().hbr_read_margins(self._h, A.ptr(out), n))
        return out

    def add_eval(self, x, init_margins, missing=np.nan) -> int:
        """An evaluation set (dense f32 rows of the index's features) with
        its starting margins [n_rows][n_outputs], kept on the device."""
        x = np.ascontiguousarray(x, np.float32)
        init = np.ascontiguousarray(init_margins, np.float32).reshape(x.shape[0], -1)
        idx = C.c_uint32()
        A.check(A.lib().hbr_engine_add_eval(self._h, A.ptr(x), x.shape[0], x.shape[1], float(missing), A.ptr(init),
                                            init.shape[1], C.byref(idx)))
        self._eval_shapes = getattr(self, "_eval_shapes", [])
        self._eval_shapes.append(init.shape)
        return idx.value

    def eval_add_tree(self, tree: dict, output=0):
        """One tree (node arrays as the trainer returns them, with its
        categorical nodes and pool when it has them) added to every eval
        set's margins of `output`, on the device."""
        arrs = [np.ascontiguousarray(tree[k], dt) for k, dt in
                (("split_feature", np.uint32), ("split_cond", np.float32), ("default_left", np.uint8),
                 ("left", np.int32), ("right", np.int32), ("leaf_value", np.float32))]
        if not np.any(tree.get("is_categorical", ())):
            A.check(A.lib().hbr_engine_eval_add_tree(self._h, *[A.ptr(a) for a in arrs], len(arrs[3]), output))
            return
        cats = [np.ascontiguousarray(tree[k], dt) for k, dt in
                (("is_categorical", np.uint8), ("cat_begin", np.uint32), ("cat_end", np.uint32),
                 ("categories", np.uint32))]
        A.check(A.lib().hbr_engine_eval_add_tree_categorical(self._h, *[A.ptr(a) for a in arrs + cats],
                                                             len(cats[3]), len(arrs[3]), output))

    def eval_margins(self, index):
        out = np.empty(self._eval_shapes[index], np.float32)
        A.check(A.lib().hbr_engine_eval_margins(self._h, index, A.ptr(out)))
        return out

    def reserve_hists(self, slots):
        fits = C.c_int()
        A.check(A.lib().hbr_reserve_hists(self._h, slots, C.byref(fits)))
        return bool(fits.value)

    def build_resident(self, nodes, siblings=()):
        segs = (A.Segment * max(1, len(nodes)))(*[s for s, _ in nodes])
        slots = np.array([sl for _, sl in nodes], np.uint32)
        par = np.array([p for p, _ in siblings], np.uint32)
        blt = np.array([b for _, b in siblings], np.uint32)
        A.check(A.lib().hbr_build_resident(self._h, segs, A.ptr(slots), len(nodes), A.ptr(par), A.ptr(blt),
                                           len(siblings)))

    def scan_resident(self, reg, requests):
        """requests: dicts with slot, total (g, h), fixed (g, h) or None,
        root_gain, lower, upper; every feature, no monotone directions."""
        n_cols = self.index.n_cols
        feats = np.arange(n_cols, dtype=np.uint32)
        arr = (A.ScanRequest * len(requests))()
        for i, r in enumerate(requests):
            q = arr[i]
            q.slot = r["slot"]
            q.total_g, q.total_h = r["total"]
            if r.get("fixed") is not None:
                q.has_fixed = 1
                q.fixed_g, q.fixed_h = (int(v) for v in r["fixed"])
            q.root_gain = r["root_gain"]
            q.lower = r.get("lower", -math.inf)
            q.upper = r.get("upper", math.inf)
            q.n_features = n_cols
            q.features = A.typed(feats, C.c_uint32)
        out = (A.NodeScan * len(requests))()
        rp = A.RegParams(*reg)
        A.check(A.lib().hbr_scan_resident(self._h, C.byref(rp), arr, len(requests), out))
        scans = [out[i] for i in range(len(requests))]
        pool = np.zeros(max([s.cat_end for s in scans if s.kind == A.SCAN_CATEGORICAL], default=0), np.uint32)
        A.check(A.lib().hbr_scan_categories(self._h, A.ptr(pool), pool.size))
        self.scan_categories = pool
        return scans

    def read_hist(self, slot):
        out = np.empty(2 * self.total_bins, np.float64)
        A.check(A.lib().hbr_read_hist(self._h, slot, A.ptr(out)))
        return out.reshape(-1, 2)

    def set_profiling(self, on=True, kernel_prefix=None, every=1):
        """Time kernels (those whose name starts with kernel_prefix) with HIP
        events on the engine's stream: every `every`-th launch of them."""
        A.check(A.lib().hbr_set_profiling(self._h, int(every) if on else 0,
                                          None if kernel_prefix is None else kernel_prefix.encode()))

    def kernel_stats(self):
        buf = C.create_string_buffer(1 << 16)
        A.check(A.lib().hbr_kernel_stats(self._h, buf, len(buf)))
        return A.kernel_stats(buf.value.decode())

    def counters(self):
        c = A.EngineCounters()
        A.check(A.lib().hbr_engine_counters_read(self._h, C.byref(c)))
        return {k: getattr(c, k) for k, _ in A.EngineCounters._fields_}


# ---- data -------------------------------------------------------------------------------

class DMatrix:
    """Training or prediction data (python/python/hessboost/_core.py DMatrix):
    a dense f32 matrix or CSR triplet, labels, optional weights, and the
    missing-value marker (NaN by default)."""

    def __init__(self, data, label=None, weight=None, missing=np.nan, n_cols=None, feature_types=None):
        if isinstance(data, tuple):
            self.csr = (np.ascontiguousarray(data[0], np.uint64), np.ascontiguousarray(data[1], np.uint32),
                        np.ascontiguousarray(data[2], np.float32))
            self.x = None
            self.n_rows = len(self.csr[0]) - 1
            self.n_cols = int(n_cols)
        else:
            self.x = np.ascontiguousarray(data, np.float32)
            self.csr = None
            self.n_rows, self.n_cols = self.x.shape
        self.label = None if label is None else np.ascontiguousarray(label, np.float32)
        self.weight = None if weight is None else np.ascontiguousarray(weight, np.float32)
        self.missing = missing
        self.feature_types = None if feature_types is None else list(feature_types)
        _categorical_flags(self.feature_types, self.n_cols)  # validates the length
        self._index = {}
        self._cuts = {}

    def cuts(self, max_bin=256) -> Cuts:
        """HistCuts for max_bin (src/data/quantile.rs:65-78), cached."""
        if max_bin not in self._cuts:
            if self.csr is not None:
                self._cuts[max_bin] = Cuts.from_csr(*self.csr, self.n_cols, max_bin=max_bin, weights=self.weight,
                                                    feature_types=self.feature_types)
            else:
                self._cuts[max_bin] = Cuts.from_dense(self.x, max_bin=max_bin, weights=self.weight,
                                                      missing=self.missing, feature_types=self.feature_types)
        return self._cuts[max_bin]

    def index(self, max_bin=256) -> BinnedIndex:
        """The binned index for max_bin (DMatrix::hist_index, src/data/dmatrix.rs:931), cached."""
        if max_bin not in self._index:
            cuts = self.cuts(max_bin)
            if self.csr is not None:
                self._index[max_bin] = BinnedIndex(cuts, csr=self.csr, n_cols=self.n_cols)
            else:
                self._index[max_bin] = BinnedIndex(cuts, x=self.x, missing=self.missing)
        return self._index[max_bin]

    def engine(self, max_bin=256, ordinal=0) -> "Engine":
        """A device engine over this matrix: a dense matrix is binned on the
        device against the host cuts (features of at most 256 bins); CSR
        input, wider features, or categorical features (binned by exact
        match) go through the host index."""
        if self.x is not None and _categorical_flags(self.feature_types, self.n_cols) is None:
            cuts = self.cuts(max_bin)
            fo, _ = cuts.arrays()
            if fo.size > 1 and int(np.max(np.diff(fo))) <= 256:
                return Engine.from_dense(self.x, cuts, ordinal, missing=self.missing)
        return Engine(self.index(max_bin), ordinal)

    @property
    def marker(self):
        """The value that marks a missing cell in dense(): the caller's
        marker for dense input; NaN for CSR input, whose absent entries are
        the missing ones (DMatrix::from_csr, src/data/dmatrix.rs:459-510,
        keeps NaN as the marker and stores only finite values)."""
        return np.nan if self.csr is not None else self.missing

    def dense(self):
        if self.x is not None:
            return self.x
        out = np.full((self.n_rows, self.n_cols), np.nan, np.float32)
        rp, col, val = self.csr
        rows = np.repeat(np.arange(self.n_rows), np.diff(rp.astype(np.int64)))
        out[rows, col[:rp[-1]]] = val[:rp[-1]]
        return out


# ---- training ---------------------------------------------------------------------------

_OBJECTIVES = {"reg:squarederror": A.OBJ_SQUARED_ERROR, "binary:logistic": A.OBJ_LOGISTIC,
               "reg:logistic": A.OBJ_LOGISTIC, "binary:logitraw": A.OBJ_LOGITRAW,
               "multi:softprob": A.OBJ_SOFTMAX, "multi:softmax": A.OBJ_SOFTMAX}


def _device_ordinal(device):
    if device in ("rocm", "gpu", "cuda", None):
        return 0
    if isinstance(device, str) and ":" in device:
        return int(device.split(":")[1])
    raise ValueError(f"unsupported device {device!r}: this backend runs rocm[:N]")


@dataclass
class Booster:
    """A trained model: scalar-leaf trees in the reference's Node layout
    (src/tree/regtree.rs:38-66), intercepts and the objective, with the
    fields of the reference's JSON model document (model/serde.rs)."""
    objective: str
    base_score: np.ndarray
    trees: list = field(default_factory=list)
    n_outputs: int = 1
    n_features: int = 0
    tree_weights: np.ndarray | None = None
    num_class: int = 0
    n_targets: int = 1
    best_iteration: int | None = None
    num_parallel_tree: int = 1
    objective_params: dict = field(default_factory=dict)
    _forest: object = None
    _forest_ordinal: int = -1

    def num_trees(self):
        return len(self.trees)

    def effective_trees(self):
        """The trees predictions use (model/mod.rs:1238-1242): with a best
        iteration, the first (best_iteration + 1) x n_outputs x
        num_parallel_tree."""
        if self.best_iteration is None:
            return self.trees
        return self.trees[:(self.best_iteration + 1) * self.n_outputs * self.num_parallel_tree]

    def forest_desc(self, trees=None):
        trees = self.effective_trees() if trees is None else trees
        k, npt = self.n_outputs, max(1, self.num_parallel_tree)
        off = np.zeros(len(trees) + 1, np.uint64)
        cols = {key: [] for key in ("split_feature", "split_cond", "default_left", "left", "right", "leaf_value")}
        for i, t in enumerate(trees):
            for key in cols:
                cols[key].append(np.asarray(t[key]))
            off[i + 1] = off[i] + len(t["left"])
        arrs = dict(tree_offset=off,
                    split_feature=np.concatenate(cols["split_feature"]).astype(np.uint32),
                    split_cond=np.concatenate(cols["split_cond"]).astype(np.float32),
                    default_left=np.concatenate(cols["default_left"]).astype(np.uint8),
                    left=np.concatenate(cols["left"]).astype(np.int32),
                    right=np.concatenate(cols["right"]).astype(np.int32),
                    leaf_value=np.concatenate(cols["leaf_value"]).astype(np.float32),
                    tree_weight=(np.ones(len(trees), np.float32) if self.tree_weights is None
                                 else np.asarray(self.tree_weights[:len(trees)], np.float32)),
                    tree_output=np.array([(t // npt) % k for t in range(len(trees))], np.uint32),
                    base_score=np.asarray(self.base_score, np.float32))
        if any(np.any(t.get("is_categorical", ())) for t in trees):
            # every tree's category pool concatenated, node ranges made absolute
            isc, beg, end, pool = [], [], [], []
            for t in trees:
                n = len(t["left"])
                base = sum(len(p) for p in pool)
                isc.append(np.asarray(t.get("is_categorical", np.zeros(n)), np.uint8))
                beg.append(np.asarray(t.get("cat_begin", np.zeros(n)), np.uint64) + base)
                end.append(np.asarray(t.get("cat_end", np.zeros(n)), np.uint64) + base)
                pool.append(np.asarray(t.get("categories", ()), np.uint32))
            arrs.update(is_categorical=np.concatenate(isc), cat_begin=np.concatenate(beg).astype(np.uint32),
                        cat_end=np.concatenate(end).astype(np.uint32), categories=np.concatenate(pool))
        return arrs

    def forest(self, ordinal=0):
        if self._forest is None or self._forest_ordinal != ordinal:
            self._forest = Forest(self.forest_desc(), self.n_outputs, ordinal)
            self._forest_ordinal = ordinal
        return self._forest

    def predict(self, data, *, output_margin=False, pred_leaf=False, missing=None, device="rocm:0"):
        """Margins, transformed predictions or leaf ids. `missing` marks an
        absent cell of an array input (NaN when None); a DMatrix carries
        its own marker."""
        if isinstance(data, DMatrix):
            x, missing = data.dense(), data.marker
        else:
            x = np.ascontiguousarray(data, np.float32)
            missing = np.nan if missing is None else missing
        f = self.forest(_device_ordinal(device))
        if pred_leaf:
            return f.predict_leaf(x, missing)
        m = f.predict_margin(x, missing)
        m = m if self.n_outputs == 1 else m.reshape(-1, self.n_outputs)
        if output_margin or self.objective in ("reg:squarederror", "binary:logitraw"):
            return m
        # the objective's transform on the host with the C library's expf
        # (Transform::apply, model/transform.rs:74-104)
        kind = {"binary:logistic": A.TRANSFORM_SIGMOID, "reg:logistic": A.TRANSFORM_SIGMOID,
                "multi:softprob": A.TRANSFORM_SOFTMAX, "multi:softmax": A.TRANSFORM_CLASS_INDEX}.get(self.objective)
        if kind is None:
            raise NotImplementedError(f"the {self.objective} transform is not implemented; "
                                      "predict(..., output_margin=True) gives the margins")
        v = np.ascontiguousarray(m, np.float32).reshape(-1).copy()
        n_rows = v.size // self.n_outputs
        A.check(A.lib().hbr_pred_transform(kind, A.ptr(v), n_rows, self.n_outputs))
        if kind == A.TRANSFORM_CLASS_INDEX:
            return v[:n_rows]
        return v if self.n_outputs == 1 else v.reshape(n_rows, self.n_outputs)

    # The reference's JSON model document (model/serde.rs:57-136): every
    # field predictions depend on is written, the nullable ones as null.
    _JSON_UNSUPPORTED = ("linear", "shrinkage", "boulevard", "ebm")

    def save_model_json(self):
        """The reference's JSON model document (model/serde.rs:13-55) of
        scalar-leaf, numeric-split trees; hessboost loads it with
        BoostedModel::load (model/io.rs:119-131)."""
        def f32(v):
            return float(np.float32(v))

        trees = []
        for t in self.trees:
            n = len(t["left"])
            gain = t.get("split_gain", np.zeros(n, np.float32))
            hess = t.get("sum_hess", np.zeros(n, np.float32))
            isc = t.get("is_categorical", np.zeros(n, np.uint8))
            beg = t.get("cat_begin", np.zeros(n, np.uint32))
            end = t.get("cat_end", np.zeros(n, np.uint32))
            nodes = [dict(split_feature=int(t["split_feature"][i]), split_cond=f32(t["split_cond"][i]),
                          default_left=bool(t["default_left"][i]), left=int(t["left"][i]), right=int(t["right"][i]),
                          leaf_value=f32(t["leaf_value"][i]), sum_hess=f32(hess[i]), split_gain=f32(gain[i]),
                          is_categorical=bool(isc[i]), cat_begin=int(beg[i]), cat_end=int(end[i]))
                     for i in range(n)]
            trees.append(dict(nodes=nodes, categories=[int(c) for c in t.get("categories", ())], size_leaf_vector=0,
                              leaf_vectors=[], linear=None))
        weights = np.ones(len(trees), np.float32) if self.tree_weights is None else self.tree_weights
        doc = dict(trees=trees, base_score=[f32(b) for b in np.atleast_1d(self.base_score)],
                   objective=self.objective, objective_params=dict(self.objective_params),
                   num_class=int(self.num_class), n_outputs=int(self.n_outputs), n_targets=int(self.n_targets),
                   n_features=int(self.n_features), best_iteration=self.best_iteration,
                   tree_weights=[f32(w) for w in weights], num_parallel_tree=int(self.num_parallel_tree),
                   linear=None, shrinkage=None, boulevard=None, ebm=None)
        return json.dumps(doc)

    def save_raw(self, format="binary"):
        """The model's bytes (python/python/hessboost/_booster.py save_raw):
        "binary", the reference's native container as one zstd frame
        (src/model/native.rs; an uncompressed container where no libzstd
        is present, which the reference reads as well), or "json", its
        JSON document."""
        if format == "json":
            return self.save_model_json().encode()
        if format != "binary":
            raise ValueError(f"unsupported model format {format!r}")
        from . import native_model
        try:
            return native_model.encode(self)
        except native_model.ModelFormatError:
            return native_model.encode(self, compress=False)

    def save_model(self, fname, *, format=None):
        """Write the model to fname: JSON for a .json name, else the native
        binary format (_booster.py:912-921)."""
        if format is None:
            format = "json" if str(fname).endswith(".json") else "binary"
        with open(fname, "wb") as f:
            f.write(self.save_raw(format))

    def load_model(self, fname, *, format=None):
        """Replace the model with one read from a path or bytes, in the
        format its content has (native binary, zstd or not, or JSON), as
        _booster.py:923-940 does for these two formats."""
        from . import native_model
        data = bytes(fname) if isinstance(fname, (bytes, bytearray, memoryview)) else open(fname, "rb").read()
        if format is None:
            format = "binary" if native_model.is_native(data) else "json"
        if format == "binary":
            fields = native_model.decode(data)
        elif format == "json":
            other = type(self).load_model_json(data.decode())
            fields = {k: getattr(other, k) for k in ("objective", "base_score", "trees", "n_outputs", "n_features",
                                                     "tree_weights", "num_class", "n_targets", "best_iteration",
                                                     "num_parallel_tree", "objective_params")}
        else:
            raise ValueError(f"unsupported model format {format!r}")
        for key, value in fields.items():
            setattr(self, key, value)
        self._forest, self._forest_ordinal = None, -1
        return self

    @classmethod
    def from_bytes(cls, data):
        """A Booster read from a native or JSON model's bytes."""
        return cls(objective="reg:squarederror", base_score=np.zeros(1, np.float32)).load_model(data)

    @classmethod
    def load_model_json(cls, text):
        """A Booster from the reference's JSON model document: scalar-leaf
        trees with numeric or categorical splits. Vector or linear leaves,
        the linear booster, shrinkage, Boulevard and EBM models are refused
        with a ValueError naming the feature, and so are the categorical
        nodes the reference's loader refuses (a leaf marked categorical, a
        split with no categories or a range beyond the tree's pool;
        tests/native_format.rs:391-409)."""
        doc = json.loads(text)
        for key in cls._JSON_UNSUPPORTED:
            if doc.get(key) is not None:
                raise ValueError(f"model: '{key}' is not carried by this backend")
        trees = []
        for i, t in enumerate(doc["trees"]):
            if t.get("size_leaf_vector", 0) > 1 or t.get("leaf_vectors"):
                raise ValueError(f"model: tree {i} has vector leaves")
            if t.get("linear") is not None:
                raise ValueError(f"model: tree {i} has linear leaves")
            nodes = t["nodes"]
            pool = [int(c) for c in t.get("categories", [])]
            for j, n in enumerate(nodes):
                if not n.get("is_categorical"):
                    continue
                if n["left"] < 0:
                    raise ValueError(f"model: tree {i} node {j}: a leaf marked categorical")
                if not (0 <= n["cat_begin"] < n["cat_end"] <= len(pool)):
                    raise ValueError(f"model: tree {i} node {j}: a categorical split needs categories in the pool")
            trees.append({
                "is_categorical": np.array([bool(n.get("is_categorical")) for n in nodes], np.uint8),
                "cat_begin": np.array([n.get("cat_begin", 0) for n in nodes], np.uint32),
                "cat_end": np.array([n.get("cat_end", 0) for n in nodes], np.uint32),
                "categories": np.array(pool, np.uint32),
                "split_feature": np.array([n["split_feature"] for n in nodes], np.uint32),
                "split_cond": np.array([n["split_cond"] for n in nodes], np.float32),
                "default_left": np.array([n["default_left"] for n in nodes], np.uint8),
                "left": np.array([n["left"] for n in nodes], np.int32),
                "right": np.array([n["right"] for n in nodes], np.int32),
                "leaf_value": np.array([n["leaf_value"] for n in nodes], np.float32),
                "sum_hess": np.array([n.get("sum_hess", 0.0) for n in nodes], np.float32),
                "split_gain": np.array([n.get("split_gain", 0.0) for n in nodes], np.float32),
            })
        return cls(objective=doc["objective"], base_score=np.array(doc["base_score"], np.float32), trees=trees,
                   n_outputs=int(doc["n_outputs"]), n_features=int(doc["n_features"]),
                   tree_weights=np.array(doc["tree_weights"], np.float32), num_class=int(doc["num_class"]),
                   n_targets=int(doc.get("n_targets", 1)),
                   best_iteration=doc.get("best_iteration"), num_parallel_tree=int(doc["num_parallel_tree"]),
                   objective_params=dict(doc.get("objective_params") or {}))


class Trainer:
    """Device-resident boosting over an engine (src/training/round.rs:105-148)."""

    def __init__(self, engine: Engine, params: dict, labels, weights=None):
        p = A.TrainParams()
        p.eta = params.get("eta", params.get("learning_rate", 0.3))
        p.gamma = params.get("gamma", 0.0)
        p.lambda_ = params.get("lambda", params.get("reg_lambda", 1.0))
        p.alpha = params.get("alpha", params.get("reg_alpha", 0.0))
        p.min_child_weight = params.get("min_child_weight", 1.0)
        p.max_delta_step = params.get("max_delta_step", 0.0)
        md = params.get("max_depth", 6)
        p.max_depth = 0 if md is None else md
        ml = params.get("max_leaves", 0)
        p.max_leaves = 0 if ml is None else ml
        p.grow_policy = A.GROW_LOSSGUIDE if params.get("grow_policy", "depthwise") == "lossguide" else A.GROW_DEPTHWISE
        self.objective = params.get("objective", "reg:squarederror")
        p.objective = _OBJECTIVES[self.objective]
        p.num_class = params.get("num_class", 0)
        p.scale_pos_weight = params.get("scale_pos_weight", 1.0)
        mono = params.get("monotone_constraints")
        self._mono = None
        if mono:
            self._mono = np.array(mono, np.int8)
            p.monotone = A.typed(self._mono, C.c_int8)
            p.n_monotone = len(mono)
        if params.get("base_score") is not None:
            p.base_score = params["base_score"]
            p.has_base_score = 1
        self.params = p
        self.engine = engine
        self.labels = np.ascontiguousarray(labels, np.float32)
        self.weights = None if weights is None else np.ascontiguousarray(weights, np.float32)
        h = C.c_void_p()
        A.check(A.lib().hbr_trainer_create(engine._h, C.byref(p), A.ptr(self.labels), A.ptr(self.weights),
                                           len(self.labels), C.byref(h)))
        self._h = h

    def __del__(self):
        try:
            A.lib().hbr_trainer_free(self._h)
        except Exception:
            pass

    def boost(self, rounds=1):
        A.check(A.lib().hbr_trainer_boost(self._h, rounds))

    @property
    def n_outputs(self):
        k = C.c_uint32()
        A.check(A.lib().hbr_trainer_num_outputs(self._h, C.byref(k)))
        return k.value

    def base_score(self):
        out = np.empty(self.n_outputs, np.float32)
        A.check(A.lib().hbr_trainer_base_score(self._h, A.ptr(out)))
        return out

    def trees(self):
        n = C.c_uint64()
        A.check(A.lib().hbr_trainer_num_trees(self._h, C.byref(n)))
        out = []
        for t in range(n.value):
            m = C.c_uint64()
            A.check(A.lib().hbr_trainer_tree_size(self._h, t, C.byref(m)))
            k = m.value
            d = dict(split_feature=np.empty(k, np.uint32), split_cond=np.empty(k, np.float32),
                     default_left=np.empty(k, np.uint8), left=np.empty(k, np.int32), right=np.empty(k, np.int32),
                     leaf_value=np.empty(k, np.float32), sum_hess=np.empty(k, np.float32),
                     split_gain=np.empty(k, np.float32), split_bin=np.empty(k, np.int64))
            A.check(A.lib().hbr_trainer_tree(self._h, t, *[A.ptr(d[key]) for key in
                                                           ("split_feature", "split_cond", "default_left", "left",
                                                            "right", "leaf_value", "sum_hess", "split_gain",
                                                            "split_bin")]))
            nc = C.c_uint64()
            cat = dict(is_categorical=np.zeros(k, np.uint8), cat_begin=np.zeros(k, np.uint32),
                       cat_end=np.zeros(k, np.uint32))
            A.check(A.lib().hbr_trainer_tree_categories(self._h, t, A.ptr(cat["is_categorical"]),
                                                        A.ptr(cat["cat_begin"]), A.ptr(cat["cat_end"]), None,
                                                        C.byref(nc)))
            if cat["is_categorical"].any():
                pool = np.zeros(nc.value, np.uint32)
                A.check(A.lib().hbr_trainer_tree_categories(self._h, t, None, None, None, A.ptr(pool), None))
                d.update(cat, categories=pool)
            out.append(d)
        return out

    def margins(self):
        out = np.empty(len(self.labels) * self.n_outputs, np.float32)
        A.check(A.lib().hbr_trainer_margins(self._h, A.ptr(out)))
        return out

    def add_eval(self, data: "DMatrix", base_margin=None) -> int:
        """An evaluation set whose margins the device keeps up to date as
        trees are grown (the host's add_tree_to_evals,
        src/training/margins.rs:148-152, called from round.rs:141-143):
        base score (or `base_margin`, [n_rows][n_outputs]) plus every tree,
        routed by raw value. Returns the set's number."""
        x = np.ascontiguousarray(data.dense(), np.float32)
        self._evals = getattr(self, "_evals", [])
        bm = None
        if base_margin is not None:
            bm = np.ascontiguousarray(base_margin, np.float32).reshape(-1)
            if bm.size != x.shape[0] * self.n_outputs:
                raise ValueError("base_margin must hold n_rows * n_outputs values")
        idx = C.c_uint32()
        A.check(A.lib().hbr_trainer_add_eval(self._h, A.ptr(x), x.shape[0], x.shape[1], float(data.marker),
                                             A.ptr(bm), C.byref(idx)))
        self._evals.append(x.shape[0])
        return idx.value

    def eval_margins(self, index: int):
        """Eval set `index`'s margins, [n_rows][n_outputs]."""
        n = self._evals[index]
        out = np.empty(n * self.n_outputs, np.float32)
        A.check(A.lib().hbr_trainer_eval_margins(self._h, index, A.ptr(out)))
        return out.reshape(n, self.n_outputs)

    def booster(self, n_features):
        softmax = self.objective in ("multi:softprob", "multi:softmax")
        return Booster(objective=self.objective, base_score=self.base_score(), trees=self.trees(),
                       n_outputs=self.n_outputs, n_features=n_features,
                       num_class=self.n_outputs if softmax else 0,
                       objective_params={"scale_pos_weight": float(self.params.scale_pos_weight),
                                         "max_delta_step": float(self.params.max_delta_step)})


def train(params: dict, dtrain: DMatrix, num_boost_round: int = 10, *, evals=(), device="rocm:0") -> Booster:
    """hessboost.train for `tree_method=hist` on one MI355X
    (src/training/api.rs:228-234; python/python/hessboost/_training.py:161-175).

    `evals`: (DMatrix, name) pairs with dtrain's features; their margins are
    updated on the device after every tree and returned as the booster's
    `eval_margins` ({name: [n_rows][n_outputs]}). Metrics over them are the
    caller's."""
    if params.get("tree_method", "hist") not in ("hist", "auto"):
        raise ValueError("this backend trains tree_method=hist")
    engine = dtrain.engine(params.get("max_bin", 256), _device_ordinal(device))
    t = Trainer(engine, params, dtrain.label, dtrain.weight)
    names = []
    for data, name in evals:
        if data.n_cols != dtrain.n_cols:
            raise ValueError(f"eval set {name!r} does not have the training matrix's features")
        names.append((t.add_eval(data), name))
    t.boost(num_boost_round)
    b = t.booster(dtrain.n_cols)
    b.eval_margins = {name: t.eval_margins(i) for i, name in names}
    return b


# ---- prediction -----------------------------------------------------------------------------

class Forest:
    """GpuModel (src/backend/cuda/predict.rs:401-520): a forest uploaded once."""

    def __init__(self, arrs: dict, n_outputs: int = 1, ordinal: int = 0):
        dtypes = dict(tree_offset=np.uint64, split_feature=np.uint32, split_cond=np.float32,
                      default_left=np.uint8, left=np.int32, right=np.int32, leaf_value=np.float32,
                      tree_weight=np.float32, tree_output=np.uint32, base_score=np.float32)
        a = {k: np.ascontiguousarray(arrs[k], dt) for k, dt in dtypes.items()}
        if arrs.get("is_categorical") is not None:  # categorical splits (tree/mod.rs:34-58)
            for k, dt in (("is_categorical", np.uint8), ("cat_begin", np.uint32), ("cat_end", np.uint32),
                          ("categories", np.uint32)):
                a[k] = np.ascontiguousarray(arrs[k], dt)
        self.arrs = a
        self.n_trees = len(a["tree_offset"]) - 1
        self.n_outputs = n_outputs
        fd = A.ForestDesc(self.n_trees, A.typed(a["tree_offset"], C.c_uint64),
                          A.typed(a["split_feature"], C.c_uint32), A.typed(a["split_cond"], C.c_float),
                          A.typed(a["default_left"], C.c_uint8), A.typed(a["left"], C.c_int32),
                          A.typed(a["right"], C.c_int32), A.typed(a["leaf_value"], C.c_float),
                          A.typed(a["tree_weight"], C.c_float), A.typed(a["tree_output"], C.c_uint32),
                          n_outputs, 0, A.typed(a["base_score"], C.c_float),
                          A.typed(a.get("is_categorical"), C.c_uint8), A.typed(a.get("cat_begin"), C.c_uint32),
                          A.typed(a.get("cat_end"), C.c_uint32),
                          A.typed(a["categories"] if a.get("categories") is not None and a["categories"].size else None,
                                  C.c_uint32),
                          0 if a.get("categories") is None else int(a["categories"].size))
        h = C.c_void_p()
        A.check(A.lib().hbr_forest_upload(ordinal, C.byref(fd), C.byref(h)))
        self._h = h
        self.ordinal = ordinal

    def __del__(self):
        try:
            A.lib().hbr_forest_free(self._h)
        except Exception:
            pass

    def predict_margin(self, x, missing=np.nan, init_margins=None):
        """Margins [n_rows * n_outputs]; init_margins (the same shape) are
        each row's starting margins in place of the base scores."""
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty(x.shape[0] * self.n_outputs, np.float32)
        if init_margins is None:
            A.check(A.lib().hbr_predict_margin(self._h, A.ptr(x), x.shape[0], x.shape[1], float(missing),
                                               A.ptr(out)))
        else:
            init = np.ascontiguousarray(init_margins, np.float32).reshape(-1)
            if init.size != out.size:
                raise ValueError("init_margins must hold n_rows * n_outputs values")
            A.check(A.lib().hbr_predict_margin_from(self._h, A.ptr(x), x.shape[0], x.shape[1], float(missing),
                                                    A.ptr(init), A.ptr(out)))
        return out

    def predict_leaf(self, x, missing=np.nan):
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty(x.shape[0] * self.n_trees, np.int32)
        A.check(A.lib().hbr_predict_leaf(self._h, A.ptr(x), x.shape[0], x.shape[1], float(missing), A.ptr(out)))
        return out.reshape(x.shape[0], self.n_trees)

    def predict_margin_device(self, d_x, n_rows, n_cols, d_out, d_leaf=None, missing=np.nan):
        A.check(A.lib().hbr_predict_margin_device(self._h, C.c_void_p(d_x), n_rows, n_cols, float(missing),
                                                  C.c_void_p(d_out), None if d_leaf is None else C.c_void_p(d_leaf)))

    def set_profiling(self, on=True, kernel_prefix=None, every=1):
        A.check(A.lib().hbr_forest_set_profiling(self._h, int(every) if on else 0,
                                                  None if kernel_prefix is None else kernel_prefix.encode()))

    def kernel_stats(self):
        buf = C.create_string_buffer(1 << 16)
        A.check(A.lib().hbr_forest_kernel_stats(self._h, buf, len(buf)))
        return A.kernel_stats(buf.value.decode())


class DeviceBuffer:
    """Device memory held by the library (inputs kept resident in HBM)."""

    def __init__(self, nbytes, ordinal=0):
        p = C.c_void_p()
        A.check(A.lib().hbr_device_alloc(ordinal, nbytes, C.byref(p)))
        self.ptr, self.nbytes, self.ordinal = p.value, nbytes, ordinal

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes
        A.check(A.lib().hbr_device_upload(self.ordinal, C.c_void_p(self.ptr), A.ptr(arr), arr.nbytes))

    def download(self, dtype, count):
        out = np.empty(count, dtype)
        A.check(A.lib().hbr_device_download(self.ordinal, A.ptr(out), C.c_void_p(self.ptr), out.nbytes))
        return out

    def copy_from(self, other, nbytes=None):
        """Device-to-device copy of `nbytes` (default: all of `other`)."""
        n = other.nbytes if nbytes is None else nbytes
        assert n <= self.nbytes and n <= other.nbytes
        A.check(A.lib().hbr_device_copy(self.ordinal, C.c_void_p(self.ptr), C.c_void_p(other.ptr), n))

    def __del__(self):
        try:
            A.lib().hbr_device_free(self.ordinal, C.c_void_p(self.ptr))
        except Exception:
            pass
