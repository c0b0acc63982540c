"""hbr_build_device_noalloc, the histogram build that allocates nothing
(its tile plan and partial sums live in the library's fixed per-device
scratch), against hbr_build on the same rows: bit for bit, on two calls in
a row with the second smaller (the scratch keeps the first call's
contents), for a dense u8 index of one and of two feature groups and for a
CSR index; a row id beyond the index is refused without a launch reading
it."""
import ctypes as C

import numpy as np
import pytest

import hessboost_amd as hb
from hessboost_amd import _capi as A

pytestmark = pytest.mark.gpu


class DeviceArray:
    def __init__(self, host):
        self.host = np.ascontiguousarray(host)
        self.nbytes = max(self.host.nbytes, 1)
        self.p = C.c_void_p()
        A.check(A.lib().hbr_device_alloc(0, self.nbytes, C.byref(self.p)))
        if self.host.nbytes:
            A.check(A.lib().hbr_device_upload(0, self.p, A.ptr(self.host), self.host.nbytes))

    def read(self, like):
        out = np.empty_like(like)
        A.check(A.lib().hbr_device_download(0, A.ptr(out), self.p, out.nbytes))
        return out

    def __del__(self):
        A.lib().hbr_device_free(0, self.p)


def noalloc_build(engine, rows):
    d_rows = DeviceArray(np.asarray(rows, np.uint32))
    out = np.full(2 * engine.total_bins, np.nan)
    d_out = DeviceArray(out)
    st = A.lib().hbr_build_device_noalloc(engine._h, d_rows.p, len(rows), d_out.p)
    msg = A.last_error() if st != A.OK else ""
    return st, d_out.read(out).reshape(-1, 2), msg


def engine_and_pairs(kind, seed):
    rng = np.random.default_rng(seed)
    if kind == "csr":
        n, f = 60_000, 300
        x = rng.exponential(1.0, (n, f)).astype(np.float32)
        x[rng.random((n, f)) < 0.9] = np.nan
        present = ~np.isnan(x)
        rp = np.zeros(n + 1, np.uint64)
        rp[1:] = np.cumsum(present.sum(1))
        r, c = np.nonzero(present)
        d = hb.DMatrix((rp, c.astype(np.uint32), x[r, c]), n_cols=f)
        e = hb.Engine(d.index(64))
    else:
        n, f = 400_000, (28 if kind == "dense" else 45)
        x = rng.standard_normal((n, f)).astype(np.float32)
        x[:, 1] = np.round(x[:, 1])  # a feature with a few heavy bins
        e = hb.DMatrix(x).engine(256)
    g = rng.standard_normal(n).astype(np.float32) * np.float32(0.37)
    h = (rng.random(n).astype(np.float32) + np.float32(0.01))
    e.prepare(np.stack([g, h], 1))
    e.set_sums("fixed_point")  # these pairs are outside the exact domain
    return e, n


@pytest.mark.parametrize("kind", ["dense", "dense_two_groups", "csr"])
def test_noalloc_build_equals_build_on_two_calls(kind):
    e, n = engine_and_pairs(kind, 3)
    rng = np.random.default_rng(4)
    first = np.sort(rng.choice(n, size=int(n * 0.8), replace=False)).astype(np.uint32)
    second = np.sort(rng.choice(n, size=int(n * 0.05), replace=False)).astype(np.uint32)
    for rows in (first, second):
        want = e.build(rows)
        st, got, msg = noalloc_build(e, rows)
        assert st == A.OK, msg
        np.testing.assert_array_equal(got.view(np.uint64), want.view(np.uint64))
    st, got, _ = noalloc_build(e, np.zeros(0, np.uint32))
    assert st == A.OK
    assert np.all(got == 0.0)


def test_noalloc_build_refuses_rows_beyond_the_index():
    e, n = engine_and_pairs("dense", 5)
    rows = np.arange(0, n, 7, dtype=np.uint32)
    rows[-1] = n  # one past the last row
    st, got, msg = noalloc_build(e, rows)
    assert st == A.INVALID and "beyond the index" in msg, msg
    assert np.all(got == 0.0)
    ok = np.arange(0, n, 7, dtype=np.uint32)
    st, got, _ = noalloc_build(e, ok)
    assert st == A.OK
    np.testing.assert_array_equal(got.view(np.uint64), e.build(ok).view(np.uint64))


def test_noalloc_build_after_device_rounds_reads_the_row_carried_pairs():
    """After device-resident logistic rounds the next pairs ride in the
    rows' last word (the pair array holds an earlier round's): the no-alloc
    build reads them there, as hbr_build does, and both equal the oracle's
    histogram of the pairs recomputed from the trainer's margins. While the
    trainer holds the rows in its first tree's leaf order the no-alloc build
    refuses (putting them back would allocate); hbr_build puts them back."""
    from hessboost_amd import synthetic
    from oracle import oracle as O

    import os
    x, y = synthetic.higgs_like(n=200_000, seed=3)
    old = os.environ.get("HBROCM_ROW_ORDER_MIN_ROWS")
    os.environ["HBROCM_ROW_ORDER_MIN_ROWS"] = "1"  # the trainer reorders rows this few
    try:
        e = hb.DMatrix(x, label=y).engine(256)
    finally:
        if old is None:
            os.environ.pop("HBROCM_ROW_ORDER_MIN_ROWS")
        else:
            os.environ["HBROCM_ROW_ORDER_MIN_ROWS"] = old
    t = hb.Trainer(e, {"objective": "binary:logistic", "max_depth": 6, "eta": 0.1}, y)
    t.boost(3)
    e.set_sums("fixed_point")
    assert e.counters()["row_orders"] == 1
    st, _, msg = noalloc_build(e, np.arange(0, len(y), 3, dtype=np.uint32))
    assert st == A.REFUSED and "leaf order" in msg, msg
    gpair = O.gradient(O.OBJ_LOGISTIC, t.margins(), y)
    ds = O.Dataset(x, max_bin=256)
    rng = np.random.default_rng(6)
    for frac in (0.7, 0.1):
        rows = np.sort(rng.choice(len(y), size=int(len(y) * frac), replace=False)).astype(np.uint32)
        want = e.build(rows)
        st, got, msg = noalloc_build(e, rows)
        assert st == A.OK, msg
        np.testing.assert_array_equal(got.view(np.uint64), want.view(np.uint64))
        ref = ds.build_hist(rows, gpair).reshape(-1, 2)
        np.testing.assert_allclose(got, ref, rtol=1e-9, atol=1e-9)
