"""The reference's native binary model format, written and read unchanged.

Layout (src/model/native.rs:1-60, src/model/sections.rs:1-18,
src/model/container.rs): the magic b"HBM\\0", the container version (3), a
section table (u32 count; per section a u8 name length, the name, a u8 flag
byte and a u64 payload length; then the payloads back to back, all
little-endian), and the XXH64 (seed 0) of every byte before it. Files are one
zstd frame holding that container; uncompressed containers are read as well
(`is_native_container`, native.rs:95-100).

The trees are stored column-wise (native.rs:462-590): one array per node
field across every tree, split by `tree.node_count`, with each tree's
category pool. Scalar-leaf models with numeric or categorical splits are
carried; the linear booster, shrinkage, vector and linear leaves, leaf
divisors, Boulevard and EBM records are refused by name, as the JSON reader
refuses them.

The sections are written in the reference's order with its flags, so the
container a model re-saves is byte for byte the one the reference wrote.
zstd comes from the system's libzstd through ctypes: the reference pins
zstd 1.5.7 (python/Cargo.lock, zstd-sys 2.1.0+zstd.1.5.7); another libzstd
may compress the same container to other (equally valid) frame bytes.
"""
from __future__ import annotations

import ctypes as C
import ctypes.util
import struct

import numpy as np

MAGIC = b"HBM\0"
LEGACY_MAGIC = b"SQB\0"  # hessboost 0.1.x, refused (native.rs:79-81)
CONTAINER_VERSION = 3
ZSTD_MAGIC = bytes([0x28, 0xB5, 0x2F, 0xFD])
REQUIRED = 1
# node.flags bits (native.rs:102-107)
DEFAULT_LEFT, CATEGORICAL = 1, 2
# the zstd level of zstd::bulk::compress(.., DEFAULT_COMPRESSION_LEVEL)
ZSTD_LEVEL = 3
# container.rs: a frame may expand 4096-fold, and always to 256 MiB
ALWAYS_ALLOWED = 256 << 20
MAX_EXPANSION = 1 << 12
# the release whose format this writes; the reference writes its own name
# and version here (container.rs WRITER), a record no reader reads back
DEFAULT_WRITER = "hessboost 0.4.9"

OBJECTIVE_DEFAULTS = {
    "scale_pos_weight": 1.0, "max_delta_step": 0.0, "tweedie_variance_power": 1.5, "huber_slope": 1.0,
    "lambdarank_num_pair_per_sample": 32, "quantile_alpha": [], "expectile_alpha": [],
    "aft_loss_distribution": "normal", "aft_loss_distribution_scale": 1.0, "dist_gradient": "fisher",
    "dist_split_direction": "random", "distribution": None,
}

# objective.distribution holds the family's objective name
# (DistFamily::objective_name, objective/distributional/family.rs:131-189);
# the JSON document and this package name it in snake case (serde rename_all)
DIST_OBJECTIVE = {"normal": "dist:normal", "log_normal": "dist:lognormal", "gamma": "dist:gamma",
                  "poisson": "dist:poisson", "negative_binomial": "dist:negbinomial", "student_t": "dist:student_t"}
DIST_FAMILY = {v: k for k, v in DIST_OBJECTIVE.items()}

# every section name this reader knows (native.rs:116-172, :303-317);
# unknown sections are skipped unless REQUIRED
KNOWN = {
    "model.objective", "model.writer", "model.base_score", "model.num_class", "model.n_outputs",
    "model.n_targets", "model.n_features", "model.best_iteration", "model.tree_weights",
    "model.num_parallel_tree", "shrinkage.factors", "shrinkage.base_score", "gblinear.weights", "gblinear.bias",
    "tree.node_count", "node.split_feature", "node.split_cond", "node.left", "node.right", "node.leaf_value",
    "node.sum_hess", "node.split_gain", "node.cat_begin", "node.cat_end", "node.flags", "tree.category_count",
    "tree.categories", "tree.size_leaf_vector", "tree.leaf_vectors", "tree.has_linear", "tree.leaf_divisor",
    "leaf_linear.offsets", "leaf_linear.intercepts", "leaf_linear.features", "leaf_linear.coeffs",
    "leaf_linear.lower", "leaf_linear.upper", "boulevard.dropout", "boulevard.learning_rate", "boulevard.subsample",
    "boulevard.reg_lambda", "boulevard.truncation", "boulevard.seed", "boulevard.intercept_from_labels",
    "ebm.term_sizes", "ebm.term_features", "ebm.tree_terms", "ebm.term_means", "ebm.boulevard",
} | {"objective." + k for k in OBJECTIVE_DEFAULTS} | {"objective.exceedance_threshold"}


class ModelFormatError(ValueError):
    """A native model the reader refuses (the reference's format_error)."""


# ---- XXH64 and zstd ----------------------------------------------------------------------

def xxh64(data: bytes) -> int:
    import xxhash
    return xxhash.xxh64_intdigest(data, seed=0)


_zstd = None


def _libzstd():
    global _zstd
    if _zstd is None:
        name = ctypes.util.find_library("zstd") or "libzstd.so.1"
        try:
            z = C.CDLL(name)
        except OSError as e:
            raise ModelFormatError(f"zstd: no libzstd on this system ({e})") from e
        z.ZSTD_compressBound.restype = C.c_size_t
        z.ZSTD_compressBound.argtypes = [C.c_size_t]
        z.ZSTD_compress.restype = C.c_size_t
        z.ZSTD_compress.argtypes = [C.c_void_p, C.c_size_t, C.c_void_p, C.c_size_t, C.c_int]
        z.ZSTD_isError.restype = C.c_uint
        z.ZSTD_isError.argtypes = [C.c_size_t]
        z.ZSTD_getErrorName.restype = C.c_char_p
        z.ZSTD_getErrorName.argtypes = [C.c_size_t]
        z.ZSTD_createDStream.restype = C.c_void_p
        z.ZSTD_freeDStream.argtypes = [C.c_void_p]
        z.ZSTD_initDStream.restype = C.c_size_t
        z.ZSTD_initDStream.argtypes = [C.c_void_p]
        z.ZSTD_decompressStream.restype = C.c_size_t
        z.ZSTD_decompressStream.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p]
        _zstd = z
    return _zstd


class _Buffer(C.Structure):
    _fields_ = [("ptr", C.c_void_p), ("size", C.c_size_t), ("pos", C.c_size_t)]


def zstd_compress(data: bytes, level: int = ZSTD_LEVEL) -> bytes:
    z = _libzstd()
    cap = z.ZSTD_compressBound(len(data))
    dst = C.create_string_buffer(cap)
    n = z.ZSTD_compress(dst, cap, data, len(data), level)
    if z.ZSTD_isError(n):
        raise ModelFormatError(f"zstd: {z.ZSTD_getErrorName(n).decode()}")
    return dst.raw[:n]


def zstd_decompress(frame: bytes) -> bytes:
    """One frame, refused past the reference's expansion limit
    (container.rs decompress: max(4096 x the frame, 256 MiB))."""
    z = _libzstd()
    limit = max(len(frame) * MAX_EXPANSION, ALWAYS_ALLOWED)
    ds = z.ZSTD_createDStream()
    if not ds:
        raise ModelFormatError("zstd: no decompression context")
    try:
        z.ZSTD_initDStream(ds)
        src = C.create_string_buffer(frame, len(frame))
        inb = _Buffer(C.cast(src, C.c_void_p), len(frame), 0)
        chunk = 1 << 20
        out = bytearray()
        while True:
            dst = C.create_string_buffer(chunk)
            outb = _Buffer(C.cast(dst, C.c_void_p), chunk, 0)
            r = z.ZSTD_decompressStream(ds, C.byref(outb), C.byref(inb))
            if z.ZSTD_isError(r):
                raise ModelFormatError(f"zstd: {z.ZSTD_getErrorName(r).decode()}")
            out += dst.raw[:outb.pos]
            if len(out) > limit:
                raise ModelFormatError("zstd frame expands too far")
            if r == 0:
                break
            if inb.pos == inb.size and outb.pos < chunk:
                raise ModelFormatError("zstd: truncated frame")
        return bytes(out)
    finally:
        z.ZSTD_freeDStream(ds)


# ---- the section table -------------------------------------------------------------------

class _Writer:
    def __init__(self):
        self.sections = []

    def raw(self, name, flags, payload: bytes):
        self.sections.append((name, flags, bytes(payload)))

    def str(self, name, value: str):
        self.raw(name, REQUIRED, value.encode())

    def u64(self, name, value):
        self.raw(name, REQUIRED, struct.pack("<Q", int(value)))

    def f64(self, name, value):
        self.raw(name, REQUIRED, struct.pack("<d", float(value)))

    def array(self, name, values, dtype):
        self.raw(name, REQUIRED, np.ascontiguousarray(values, dtype).tobytes())

    def finish(self) -> bytes:
        head = [struct.pack("<I", len(self.sections))]
        for name, flags, payload in self.sections:
            nb = name.encode()
            head.append(struct.pack("<B", len(nb)) + nb + struct.pack("<BQ", flags, len(payload)))
        return b"".join(head) + b"".join(p for _, _, p in self.sections)


def _parse_sections(body: bytes):
    """(sections by name, bytes after the last payload); unknown sections
    are skipped unless REQUIRED, duplicates refused (sections.rs parse)."""
    at = 0

    def take(n):
        nonlocal at
        if at + n > len(body):
            raise ModelFormatError("truncated section table")
        out = body[at:at + n]
        at += n
        return out

    (count,) = struct.unpack("<I", take(4))
    table = []
    for _ in range(count):
        (nlen,) = struct.unpack("<B", take(1))
        try:
            name = take(nlen).decode()
        except UnicodeDecodeError as e:
            raise ModelFormatError("section name is not UTF-8") from e
        flags, length = struct.unpack("<BQ", take(9))
        table.append((name, flags, length))
    out = {}
    for name, flags, length in table:
        payload = take(length)
        if name not in KNOWN:
            if flags & REQUIRED:
                raise ModelFormatError(f"the data needs section `{name}`, which this version cannot read")
            continue
        if name in out:
            raise ModelFormatError(f"section `{name}` appears twice")
        out[name] = payload
    return out, body[at:]


class _Sections:
    def __init__(self, d):
        self.d = d

    def has(self, name):
        return name in self.d

    def bytes(self, name):
        if name not in self.d:
            raise ModelFormatError(f"missing section `{name}`")
        return self.d[name]

    def str(self, name):
        try:
            return self.bytes(name).decode()
        except UnicodeDecodeError as e:
            raise ModelFormatError(f"section `{name}` is not UTF-8") from e

    def scalar(self, name, fmt):
        b = self.bytes(name)
        if len(b) != 8:
            raise ModelFormatError(f"section `{name}` is not one value")
        return struct.unpack(fmt, b)[0]

    def u64(self, name):
        return self.scalar(name, "<Q")

    def f64(self, name):
        return self.scalar(name, "<d")

    def array(self, name, dtype, count=None):
        b = self.bytes(name)
        size = np.dtype(dtype).itemsize
        if len(b) % size:
            raise ModelFormatError(f"section `{name}` is not a whole number of values")
        a = np.frombuffer(b, dtype).copy()
        if count is not None and len(a) != count:
            raise ModelFormatError(f"section `{name}` has the wrong length")
        return a


# ---- models --------------------------------------------------------------------------------

def _objective_params(booster):
    p = dict(OBJECTIVE_DEFAULTS)
    p.update({k: v for k, v in (booster.objective_params or {}).items() if k in OBJECTIVE_DEFAULTS or
              k == "exceedance_threshold"})
    return p


def container(booster, writer: str = DEFAULT_WRITER) -> bytes:
    """The uncompressed container of `booster` (native.rs sections(): the
    model, objective and tree sections in the reference's order)."""
    w = _Writer()
    trees = booster.trees
    k = len(trees)
    w.str("model.objective", booster.objective)
    w.raw("model.writer", 0, writer.encode())
    w.array("model.base_score", np.atleast_1d(np.asarray(booster.base_score, np.float32)), "<f4")
    w.u64("model.num_class", booster.num_class)
    w.u64("model.n_outputs", booster.n_outputs)
    w.u64("model.n_targets", booster.n_targets)
    w.u64("model.n_features", booster.n_features)
    if booster.best_iteration is not None:
        w.u64("model.best_iteration", booster.best_iteration)
    weights = np.ones(k, np.float32) if booster.tree_weights is None else booster.tree_weights
    w.array("model.tree_weights", weights, "<f4")
    w.u64("model.num_parallel_tree", booster.num_parallel_tree)
    # native.rs:767-810
    p = _objective_params(booster)
    w.f64("objective.scale_pos_weight", p["scale_pos_weight"])
    w.f64("objective.max_delta_step", p["max_delta_step"])
    w.f64("objective.tweedie_variance_power", p["tweedie_variance_power"])
    w.f64("objective.huber_slope", p["huber_slope"])
    w.u64("objective.lambdarank_num_pair_per_sample", p["lambdarank_num_pair_per_sample"])
    w.array("objective.quantile_alpha", np.asarray(p["quantile_alpha"], np.float64), "<f8")
    w.array("objective.expectile_alpha", np.asarray(p["expectile_alpha"], np.float64), "<f8")
    if p.get("exceedance_threshold"):
        w.array("objective.exceedance_threshold", np.asarray(p["exceedance_threshold"], np.float64), "<f8")
    w.str("objective.aft_loss_distribution", p["aft_loss_distribution"])
    w.f64("objective.aft_loss_distribution_scale", p["aft_loss_distribution_scale"])
    w.str("objective.dist_gradient", p["dist_gradient"])
    w.str("objective.dist_split_direction", p["dist_split_direction"])
    if p.get("distribution") is not None:
        if p["distribution"] not in DIST_OBJECTIVE:
            raise ModelFormatError(f"unknown distribution family {p['distribution']!r}")
        w.str("objective.distribution", DIST_OBJECTIVE[p["distribution"]])

    def col(key, dtype, default=0):
        return np.concatenate([np.asarray(t.get(key, np.full(len(t["left"]), default)), dtype) for t in trees]) \
            if trees else np.zeros(0, dtype)

    counts = np.array([len(t["left"]) for t in trees], "<u4")
    w.array("tree.node_count", counts, "<u4")
    w.array("node.split_feature", col("split_feature", "<u4"), "<u4")
    w.array("node.split_cond", col("split_cond", "<f4"), "<f4")
    w.array("node.left", col("left", "<i4"), "<i4")
    w.array("node.right", col("right", "<i4"), "<i4")
    w.array("node.leaf_value", col("leaf_value", "<f4"), "<f4")
    w.array("node.sum_hess", col("sum_hess", "<f4"), "<f4")
    w.array("node.split_gain", col("split_gain", "<f4"), "<f4")
    w.array("node.cat_begin", col("cat_begin", "<u4"), "<u4")
    w.array("node.cat_end", col("cat_end", "<u4"), "<u4")
    flags = (col("default_left", np.uint8) != 0).astype(np.uint8) * DEFAULT_LEFT | \
        (col("is_categorical", np.uint8) != 0).astype(np.uint8) * CATEGORICAL
    w.array("node.flags", flags, np.uint8)
    w.array("tree.category_count", [len(t.get("categories", ())) for t in trees], "<u4")
    cats = [np.asarray(t.get("categories", ()), "<u4") for t in trees]
    w.array("tree.categories", np.concatenate(cats) if cats else np.zeros(0, "<u4"), "<u4")
    w.array("tree.size_leaf_vector", np.zeros(k, "<u4"), "<u4")
    w.array("tree.leaf_vectors", np.zeros(0, "<f4"), "<f4")
    w.array("tree.has_linear", np.zeros(k, np.uint8), np.uint8)
    w.array("leaf_linear.offsets", np.zeros(0, "<u4"), "<u4")
    w.array("leaf_linear.intercepts", np.zeros(0, "<f8"), "<f8")
    w.array("leaf_linear.features", np.zeros(0, "<u4"), "<u4")
    w.array("leaf_linear.coeffs", np.zeros(0, "<f8"), "<f8")
    body = MAGIC + bytes([CONTAINER_VERSION]) + w.finish()
    return body + struct.pack("<Q", xxh64(body))


def encode(booster, compress: bool = True, writer: str = DEFAULT_WRITER) -> bytes:
    """What BoostedModel::encode(Binary) writes (container.rs seal): one zstd
    frame of the container, or the container itself when the frame would
    expand past what a reader accepts, or when `compress` is False."""
    c = container(booster, writer)
    if not compress:
        return c
    frame = zstd_compress(c)
    return frame if len(c) <= max(len(frame) * MAX_EXPANSION, ALWAYS_ALLOWED) else c


def unpack(data: bytes) -> bytes:
    """The container inside `data` (a zstd frame or the container)."""
    return zstd_decompress(data) if data[:4] == ZSTD_MAGIC else bytes(data)


def is_native(data: bytes) -> bool:
    return data[:4] in (ZSTD_MAGIC, MAGIC, LEGACY_MAGIC)


def decode(data: bytes) -> dict:
    """The model fields of a native file (zstd frame or container), as the
    keyword arguments of a Booster. Refuses what the reference's reader
    refuses (bad magic, version or checksum, trailing bytes, unknown
    REQUIRED sections, undefined node flags) and the model features this
    backend does not carry."""
    c = unpack(data)
    if c.startswith(LEGACY_MAGIC):
        raise ModelFormatError("a native model from hessboost 0.1.x, which 0.2.0 and later cannot read")
    if not c.startswith(MAGIC):
        raise ModelFormatError("invalid native model header")
    if len(c) < 5:
        raise ModelFormatError("truncated native model")
    if c[4] != CONTAINER_VERSION:
        raise ModelFormatError(f"unsupported native model version {c[4]}")
    if len(c) - 8 <= len(MAGIC):
        raise ModelFormatError("truncated native model")
    checked, checksum = c[:-8], c[-8:]
    if struct.pack("<Q", xxh64(checked)) != checksum:
        raise ModelFormatError("native model checksum mismatch")
    table, rest = _parse_sections(checked[5:])
    if rest:
        raise ModelFormatError(f"{len(rest)} unexpected bytes after the last section")
    s = _Sections(table)
    for name, what in (("gblinear.weights", "the linear booster"), ("gblinear.bias", "the linear booster"),
                       ("shrinkage.factors", "shrinkage"), ("tree.leaf_divisor", "leaf divisors"),
                       ("boulevard.dropout", "a Boulevard record"), ("ebm.term_sizes", "an EBM record")):
        if s.has(name):
            raise ModelFormatError(f"model: {what} is not carried by this backend")
    counts = s.array("tree.node_count", "<u4")
    n = int(counts.sum())
    k = len(counts)
    cols = {name: s.array(f"node.{name}", dt, n) for name, dt in (
        ("split_feature", "<u4"), ("split_cond", "<f4"), ("left", "<i4"), ("right", "<i4"), ("leaf_value", "<f4"),
        ("sum_hess", "<f4"), ("split_gain", "<f4"), ("cat_begin", "<u4"), ("cat_end", "<u4"))}
    flags = s.array("node.flags", np.uint8, n)
    if np.any(flags & ~np.uint8(DEFAULT_LEFT | CATEGORICAL)):
        raise ModelFormatError("`node.flags` holds bits this version does not define")
    if np.any(s.array("tree.size_leaf_vector", "<u4", k) > 1) or len(s.array("tree.leaf_vectors", "<f4")):
        raise ModelFormatError("model: vector leaves are not carried by this backend")
    if np.any(s.array("tree.has_linear", np.uint8, k) != 0):
        raise ModelFormatError("model: linear leaves are not carried by this backend")
    cat_counts = s.array("tree.category_count", "<u4", k)
    pool = s.array("tree.categories", "<u4", int(cat_counts.sum()))
    trees = []
    at = cat_at = 0
    for t in range(k):
        m = int(counts[t])
        sl = slice(at, at + m)
        cats = pool[cat_at:cat_at + int(cat_counts[t])]
        tree = {key: cols[key][sl].copy() for key in cols}
        tree["default_left"] = (flags[sl] & DEFAULT_LEFT != 0).astype(np.uint8)
        tree["is_categorical"] = (flags[sl] & CATEGORICAL != 0).astype(np.uint8)
        tree["categories"] = cats.copy()
        for j in np.nonzero(tree["is_categorical"])[0]:
            if tree["left"][j] < 0:
                raise ModelFormatError(f"model: tree {t} node {j}: a leaf marked categorical")
            if not (tree["cat_begin"][j] < tree["cat_end"][j] <= len(cats)):
                raise ModelFormatError(f"model: tree {t} node {j}: a categorical split needs categories in the pool")
        trees.append(tree)
        at += m
        cat_at += int(cat_counts[t])
    params = dict(OBJECTIVE_DEFAULTS)
    for key, default in OBJECTIVE_DEFAULTS.items():
        name = "objective." + key
        if not s.has(name):
            continue
        if isinstance(default, list):
            params[key] = s.array(name, "<f8").tolist()
        elif key == "lambdarank_num_pair_per_sample":
            params[key] = int(s.u64(name))
        elif key == "distribution":
            if s.str(name) not in DIST_FAMILY:
                raise ModelFormatError(f"unknown distribution `{s.str(name)}`")
            params[key] = DIST_FAMILY[s.str(name)]
        elif isinstance(default, str):
            params[key] = s.str(name)
        else:
            params[key] = s.f64(name)
    if s.has("objective.exceedance_threshold"):
        params["exceedance_threshold"] = s.array("objective.exceedance_threshold", "<f8").tolist()
    return dict(objective=s.str("model.objective"), base_score=s.array("model.base_score", "<f4"), trees=trees,
                n_outputs=int(s.u64("model.n_outputs")), n_features=int(s.u64("model.n_features")),
                tree_weights=s.array("model.tree_weights", "<f4", k), num_class=int(s.u64("model.num_class")),
                n_targets=int(s.u64("model.n_targets")),
                best_iteration=int(s.u64("model.best_iteration")) if s.has("model.best_iteration") else None,
                num_parallel_tree=int(s.u64("model.num_parallel_tree")), objective_params=params)
