"""The native binary model format (src/model/native.rs), pinned by the
reference's own saved files (tests/data/saved/<version>/<case>.bin, copied to
tests/golden/native/): every scalar-leaf model of three versions loads,
predicts the margins the reference recorded for it bit for bit, and re-saves
its container byte for byte (tests/native_format.rs:822-990); models this
backend does not carry, and malformed files, are refused."""
import os
import struct

import numpy as np
import pytest

from hessboost_amd import native_model as N
from hessboost_amd.core import Booster
from oracle import oracle as O
from tests.helpers import GOLDEN, categorical_features, four_features, golden_forest, load_saved_models

NATIVE = os.path.join(GOLDEN, "native")
VERSIONS = sorted(os.listdir(NATIVE))
CASES = ["early_stopping", "dart", "multiclass_forest", "quantiles", "expectiles", "aft", "dist_normal",
         "dist_negbinomial", "multi_target", "categorical_splits"]


def stored(ver, case):
    with open(os.path.join(NATIVE, ver, case + ".bin"), "rb") as f:
        return f.read()


def as_case(b: Booster):
    """The decoded model in saved_models.json's layout (f32 as bits)."""
    bits = lambda a: np.asarray(a, np.float32).view(np.uint32).tolist()  # noqa: E731
    trees = [{"is_categorical": t["is_categorical"].tolist(), "cat_begin": t["cat_begin"].tolist(),
              "cat_end": t["cat_end"].tolist(), "categories": t["categories"].tolist(),
              "split_feature": t["split_feature"].tolist(), "split_cond": bits(t["split_cond"]),
              "default_left": t["default_left"].tolist(), "left": t["left"].tolist(), "right": t["right"].tolist(),
              "leaf_value": bits(t["leaf_value"]), "sum_hess": bits(t["sum_hess"]),
              "split_gain": bits(t["split_gain"])} for t in b.trees]
    return {"objective": b.objective, "n_outputs": b.n_outputs, "num_parallel_tree": b.num_parallel_tree,
            "best_iteration": b.best_iteration, "base_score": bits(b.base_score),
            "tree_weights": bits(b.tree_weights), "trees": trees}


@pytest.mark.parametrize("ver", VERSIONS)
@pytest.mark.parametrize("case", CASES)
def test_saved_native_models_load_and_predict_recorded_margins(ver, case):
    """native_format.rs:822-860: the .bin (a zstd frame) loads, holds the
    model its .json holds, and predicts the recorded margins bit for bit."""
    b = Booster.from_bytes(stored(ver, case))
    want = load_saved_models()[f"{ver}/{case}"]
    got = as_case(b)
    for key in ("objective", "n_outputs", "num_parallel_tree", "best_iteration", "base_score", "tree_weights"):
        assert got[key] == want[key], key
    assert got["trees"] == want["trees"]
    x = categorical_features() if case == "categorical_splits" else four_features()
    margins = O.predict_margin(golden_forest(got), x)
    assert np.array_equal(margins.view(np.uint32), np.array(want["margins"], np.uint32))


@pytest.mark.parametrize("ver", VERSIONS)
@pytest.mark.parametrize("case", CASES)
def test_containers_re_save_byte_identically(ver, case):
    """native_format.rs:919-990: a loaded model re-saves the container its
    writer stored, byte for byte (the writer record names the release); the
    JSON document of the same model writes the same container."""
    data = stored(ver, case)
    b = Booster.from_bytes(data)
    assert N.container(b, writer=f"hessboost {ver}") == N.unpack(data)
    with open(os.path.join(GOLDEN, "models", case + ".json")) as f:
        j = Booster.load_model_json(f.read())
    if ver == "0.4.9":
        assert N.container(j, writer="hessboost 0.4.9") == N.unpack(data)


def test_binary_round_trip_through_zstd():
    """save_raw writes one zstd frame (container.rs seal); it decompresses
    to the container, and loads back to the same model. The frame bytes
    depend on the zstd library (the reference pins 1.5.7), the container's
    do not."""
    b = Booster.from_bytes(stored("0.4.9", "multiclass_forest"))
    raw = b.save_raw()
    assert raw[:4] == N.ZSTD_MAGIC
    assert N.zstd_decompress(raw) == N.container(b)
    again = Booster.from_bytes(raw)
    assert N.container(again) == N.container(b)
    plain = N.encode(b, compress=False)
    assert plain[:4] == N.MAGIC and N.container(Booster.from_bytes(plain)) == plain


def test_save_and_load_by_file_name(tmp_path):
    b = Booster.from_bytes(stored("0.4.9", "categorical_splits"))
    for name in ("m.bin", "m.json", "m.model"):
        path = tmp_path / name
        b.save_model(path)
        head = path.read_bytes()[:4]
        assert (head == b'{"tr') if name.endswith(".json") else (head == N.ZSTD_MAGIC)
        c = Booster(objective="reg:squarederror", base_score=np.zeros(1, np.float32)).load_model(path)
        assert N.container(c) == N.container(b)


@pytest.mark.parametrize("case,what", [("gblinear", "linear booster"), ("vector_leaves", "vector leaves")])
def test_models_this_backend_does_not_carry_are_refused(case, what):
    with pytest.raises(N.ModelFormatError, match=what):
        Booster.from_bytes(stored("0.4.9", case))


def _reseal(body):
    return body + struct.pack("<Q", N.xxh64(body))


def test_malformed_files_are_refused():
    good = N.unpack(stored("0.4.9", "early_stopping"))
    flipped = bytearray(good)
    flipped[40] ^= 1
    cases = [
        (bytes(flipped), "checksum"),
        (b"SQB\0" + good[4:], "0.1.x"),
        (good[:4] + b"\x02" + good[5:-8] + struct.pack("<Q", N.xxh64(good[:4] + b"\x02" + good[5:-8])), "version"),
        (_reseal(good[:-8] + b"\0\0"), "unexpected bytes"),
        (b"XYZ\0" + good[4:], "header"),
        (good[:6], "truncated"),
    ]
    for data, what in cases:
        with pytest.raises(N.ModelFormatError, match=what):
            N.decode(data)


def _with_section(name, flags, payload):
    """Early stopping's container with one more section at the table's end."""
    body = N.unpack(stored("0.4.9", "early_stopping"))[:-8]
    count = struct.unpack("<I", body[5:9])[0]
    # the table ends where the first payload begins: walk the entries
    at = 9
    for _ in range(count):
        at += 1 + body[at] + 9
    nb = name.encode()
    entry = bytes([len(nb)]) + nb + struct.pack("<BQ", flags, len(payload))
    new = body[:5] + struct.pack("<I", count + 1) + body[9:at] + entry + body[at:] + payload
    return _reseal(new)


def test_unknown_sections_are_skipped_unless_required():
    """sections.rs:1-18: a reader skips sections it does not know, and
    refuses the data when such a section is REQUIRED."""
    skip = N.decode(_with_section("future.note", 0, b"hello"))
    ref = N.decode(stored("0.4.9", "early_stopping"))
    assert len(skip["trees"]) == len(ref["trees"])
    with pytest.raises(N.ModelFormatError, match="cannot read"):
        N.decode(_with_section("future.leaves", N.REQUIRED, b"\0" * 8))


def test_undefined_node_flags_are_refused():
    """native.rs:38-44: node.flags bits the format does not define."""
    body = bytearray(N.unpack(stored("0.4.9", "early_stopping"))[:-8])
    b = Booster.from_bytes(stored("0.4.9", "early_stopping"))
    flags = b"".join(bytes([int(d)]) for t in b.trees for d in t["default_left"])
    at = bytes(body).rfind(flags)
    assert at > 0
    body[at] |= 4
    with pytest.raises(N.ModelFormatError, match="flags"):
        N.decode(_reseal(bytes(body)))
