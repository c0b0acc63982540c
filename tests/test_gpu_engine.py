"""GPU parity of the engine's stages against the CPU oracle, through the C ABI.

Histograms are exact integer sums of the quantized gradients: they are
checked bit for bit against the same integer sums formed on the CPU, bit for
bit against the oracle's f64 histogram when every sum is exact (dyadic
gradients), and within 1e-5 relative of it otherwise.
"""
import math

import numpy as np
import pytest

import hessboost_amd as hb
from hessboost_amd import _capi as A
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def quant_exp(values, rows):
    m = float(np.max(np.abs(values))) if len(values) else 0.0
    if m == 0.0 or not math.isfinite(m):
        return 0
    _, e = math.frexp(np.float32(m))
    log_n = (rows - 1).bit_length() if rows > 1 else 0
    return e + log_n - 62


def integer_histogram(gbins_rows, rows, gpair, total_bins, eg, eh):
    """The exact integer bins of the quantized pairs, formed on the CPU."""
    qg = np.rint(np.ldexp(gpair[:, 0].astype(np.float64), -eg)).astype(np.int64)
    qh = np.rint(np.ldexp(gpair[:, 1].astype(np.float64), -eh)).astype(np.int64)
    out = np.zeros((total_bins, 2), np.int64)
    for r in rows:
        for b in gbins_rows[r]:
            out[b, 0] += qg[r]
            out[b, 1] += qh[r]
    return np.stack([np.ldexp(out[:, 0].astype(np.float64), eg), np.ldexp(out[:, 1].astype(np.float64), eh)], 1)


def make(x, max_bin=256, missing=np.nan):
    cuts = hb.Cuts.from_dense(x, max_bin=max_bin, missing=missing)
    ix = hb.BinnedIndex(cuts, x=x, missing=missing)
    return ix, hb.Engine(ix)


def dense_rows(ix):
    rp, gb = ix.row_bins()
    return [gb[rp[r]:rp[r + 1]] for r in range(ix.n_rows)]


def test_histogram_exact_domain_equals_oracle_bits():
    rng = np.random.default_rng(0)
    n = 20_000
    x = rng.standard_normal((n, 32), dtype=np.float32)
    ix, eng = make(x)
    ref = O.Dataset(x)
    # dyadic gradients: every f64 sum is exact, whatever the order
    g = (rng.integers(-64, 64, n) / 16.0).astype(np.float32)
    h = (rng.integers(1, 32, n) / 8.0).astype(np.float32)
    gp = np.stack([g, h], 1).astype(np.float32)
    eng.prepare(gp)
    for rows in (np.arange(n), np.sort(rng.choice(n, 7_777, replace=False))):
        got = eng.build(rows)
        want = ref.build_hist(rows, gp)
        assert np.array_equal(got, want)


def test_histogram_general_gradients_match_integer_sums_and_oracle():
    rng = np.random.default_rng(1)
    n = 30_000
    x = rng.standard_normal((n, 28), dtype=np.float32)
    ix, eng = make(x)
    ref = O.Dataset(x)
    gp = np.stack([rng.standard_normal(n, dtype=np.float32),
                   rng.random(n, dtype=np.float32) * np.float32(0.25) + np.float32(1e-3)], 1).astype(np.float32)
    gp[3, 0] = np.float32(1e-30)  # a grain of about 2^-123: far outside the exact domain
    eng.prepare(gp)
    eg, eh = quant_exp(gp[:, 0], n), quant_exp(gp[:, 1], n)
    rows = np.sort(np.concatenate([[3], rng.choice(np.arange(4, n), 12_344, replace=False)]))
    with pytest.raises(A.HbrError) as refused:  # the trait's contract: no f64-equal sums here
        eng.build(rows)
    assert refused.value.status == A.REFUSED
    eng.set_sums("fixed_point")
    got = eng.build(rows)
    assert np.array_equal(got, integer_histogram(dense_rows(ix), rows, gp, eng.total_bins, eg, eh))
    want = ref.build_hist(rows, gp)
    scale = np.abs(want).max(axis=0)
    assert np.all(np.abs(got - want) <= 1e-5 * np.maximum(np.abs(want), 1e-12 * scale) + 1e-9 * scale)


def test_histogram_with_missing_values_and_wide_features():
    rng = np.random.default_rng(2)
    n = 10_000
    x = rng.standard_normal((n, 6), dtype=np.float32)
    x[rng.random(x.shape) < 0.15] = np.nan
    ix, eng = make(x, max_bin=1024)  # >256 bins and missing cells: the CSR path
    ref = O.Dataset(x, max_bin=1024)
    g = (rng.integers(-64, 64, n) / 32.0).astype(np.float32)
    gp = np.stack([g, np.ones(n, np.float32)], 1)
    eng.prepare(gp)
    rows = np.arange(n)
    assert np.array_equal(eng.build(rows), ref.build_hist(rows, gp))


def test_histogram_is_independent_of_row_order_and_tiles():
    rng = np.random.default_rng(3)
    n = 40_000
    x = rng.standard_normal((n, 12), dtype=np.float32)
    ix, eng = make(x)
    gp = np.stack([rng.standard_normal(n, dtype=np.float32), rng.random(n, dtype=np.float32)], 1)
    eng.prepare(gp)
    eng.set_sums("fixed_point")
    rows = np.sort(rng.choice(n, 30_000, replace=False))
    a = eng.build(rows)
    b = eng.build(rows[::-1].copy())
    c = eng.build(np.concatenate([rows[1::2], rows[::2]]))
    assert np.array_equal(a, b) and np.array_equal(a, c)


def test_exact_contract_refuses_outside_the_exact_domain():
    """The trait promises the CPU's f64 bits (src/tree/hist/mod.rs:205-207,
    :220-224). Gradients of grain 2^-20 with largest magnitude 2^23 are
    2^43 grains each: a node of 1,024 rows is inside the exact domain
    (backend/exact_sum.rs:14-37: n x max <= 2^53 grains) and its bins equal
    the oracle's f64 sums bit for bit; 1,025 rows are outside, and build,
    histograms and root_total refuse (HBR_REFUSED, the trait's None) until
    fixed-point sums are chosen. Device gradients are folded the same way:
    logistic pairs over margins in [-20, 20] hold Hessians near 2e-9 beside
    0.25 (about 2^51 grains each) and refuse; squared error over quarter
    margins and eighth labels is exact."""
    rng = np.random.default_rng(9)
    n = 2_000
    x = rng.standard_normal((n, 6), dtype=np.float32)
    ix, eng = make(x)
    ref = O.Dataset(x)
    g = (rng.integers(-4, 5, n).astype(np.float32) * np.float32(2.0 ** -20))
    g[7] = np.float32(2.0 ** 23)
    g[1500] = np.float32(-(2.0 ** 23))
    gp = np.stack([g, np.ones(n, np.float32)], 1).astype(np.float32)
    eng.prepare(gp)
    inside = np.arange(1_024, dtype=np.uint32)
    assert np.array_equal(eng.build(inside), ref.build_hist(inside, gp))
    outside = np.arange(1_025, dtype=np.uint32)
    for call in (lambda: eng.build(outside), lambda: eng.root_total(eng.begin_tree())):
        with pytest.raises(A.HbrError) as refused:
            call()
        assert refused.value.status == A.REFUSED
    eng.set_sums("fixed_point")
    assert np.array_equal(eng.build(outside), ref.build_hist(outside, gp))  # sums that happen to be exact
    eng.set_sums("exact")
    # device gradients
    y = (rng.random(n) < 0.5).astype(np.float32)
    eng.load_margins(np.linspace(-20, 20, n).astype(np.float32))
    assert eng.gradients(A.LOSS_LOGISTIC, y)
    with pytest.raises(A.HbrError) as refused:
        eng.build(inside)
    assert refused.value.status == A.REFUSED
    eng.load_margins((rng.integers(-8, 8, n) / 4.0).astype(np.float32))
    assert eng.gradients(A.LOSS_SQUARED_ERROR, (rng.integers(-8, 8, n) / 8.0).astype(np.float32))
    gp2 = eng.read_gradients()
    assert np.array_equal(eng.build(inside), ref.build_hist(inside, gp2.astype(np.float32)))


def test_partition_matches_oracle_routing():
    rng = np.random.default_rng(4)
    n = 50_000
    x = rng.standard_normal((n, 5), dtype=np.float32)
    x[rng.random(x.shape) < 0.1] = np.nan
    for xx in (x, np.nan_to_num(x)):
        ix, eng = make(xx, max_bin=64)
        ref = O.Dataset(xx, max_bin=64)
        fo = ix.feature_offset()
        eng.prepare(np.ones((n, 2), np.float32))
        for feature, local, dl in ((0, 10, 0), (3, 0, 1), (4, 40, 1)):
            root = eng.begin_tree()
            (left, right), = eng.partition([(root, feature, local, dl)])
            L, R = eng.rows(left), eng.rows(right)
            gbin = int(fo[feature]) + local - 1 if local > 0 else -1
            wl, wr = ref.partition(np.arange(n, dtype=np.uint32), feature, gbin, dl)
            assert np.array_equal(L, wl) and np.array_equal(R, wr)
            # a second level from the children's segments
            (l2, r2), (l3, r3) = eng.partition([(left, 1, 20, 0), (right, 2, 5, 1)])
            gb1 = int(fo[1]) + 19
            gb2 = int(fo[2]) + 4
            a, b = ref.partition(wl, 1, gb1, 0)
            c, d = ref.partition(wr, 2, gb2, 1)
            assert np.array_equal(eng.rows(l2), a) and np.array_equal(eng.rows(r2), b)
            assert np.array_equal(eng.rows(l3), c) and np.array_equal(eng.rows(r3), d)


def test_split_scan_matches_oracle_on_exact_histograms():
    rng = np.random.default_rng(5)
    n = 20_000
    x = rng.standard_normal((n, 10), dtype=np.float32)
    for missing in (False, True):
        xx = x.copy()
        if missing:
            xx[rng.random(xx.shape) < 0.2] = np.nan
        ix, eng = make(xx, max_bin=32)
        ref = O.Dataset(xx, max_bin=32)
        g = ((xx[:, 2] > 0.3).astype(np.float32) * 2 - 1 + rng.integers(-8, 8, n) / 16.0).astype(np.float32)
        gp = np.stack([np.nan_to_num(g), np.ones(n, np.float32)], 1).astype(np.float32)
        eng.prepare(gp)
        for reg in ((1.0, 0.0, 0.0, 1.0), (0.5, 0.25, 0.0, 5.0), (2.0, 0.0, 0.7, 1.0)):
            p = O.params(reg_lambda=reg[0], alpha=reg[1], max_delta_step=reg[2], min_child_weight=reg[3])
            root = eng.begin_tree()
            tot, fixed = eng.root_total(root, fixed=True)
            assert np.array_equal(tot, O.sum_rows(gp, np.arange(n)))
            eng.reserve_hists(4)
            eng.build_resident([(root, 0)])
            hist = eng.read_hist(0)
            want_hist = ref.build_hist(np.arange(n), gp)
            assert np.array_equal(hist, want_hist)
            rg = O.lib().or_node_gain(tot[0], tot[1], -math.inf, math.inf, p)
            scan, = eng.scan_resident(reg, [dict(slot=0, total=tuple(tot), fixed=tuple(fixed), root_gain=rg)])
            want = ref.evaluate(want_hist, tot, p)
            assert scan.kind == A.SCAN_NUMERIC
            assert scan.feature == want.feature
            assert np.float32(scan.loss_chg) == np.float32(want.loss_chg)
            assert (scan.left_g, scan.left_h, scan.right_g, scan.right_h) == \
                (want.left_g, want.left_h, want.right_g, want.right_h)
            fo = ix.feature_offset()
            fs = int(fo[want.feature])
            if scan.backward:
                assert want.default_left == 1
                assert (want.bin == -1) == (scan.offset == 0)
                if want.bin >= 0:
                    assert want.bin == fs + scan.offset - 1
            else:
                assert want.default_left == 0 and want.bin == fs + scan.offset


def test_device_gradients_match_oracle_bits():
    rng = np.random.default_rng(6)
    for n in (16, 37, 100_003):
        x = rng.standard_normal((n, 3), dtype=np.float32)
        ix, eng = make(x)
        m = (rng.standard_normal(n) * 5).astype(np.float32)
        if n > 1000:
            m[123] = 90.0  # a vector beyond the polynomial's range
            # the scalar sigmoid's edges: min(-x, 88.7) clamps NaN and -inf too
            m[200:210] = [np.nan, np.inf, -np.inf, 88.7, -88.7, 88.8, -88.8, 1e30, -1e30, 103.9]
        y = (rng.random(n) < 0.4).astype(np.float32)
        w = (rng.random(n) * 2).astype(np.float32)
        for obj, kind in ((O.OBJ_LOGISTIC, A.LOSS_LOGISTIC), (O.OBJ_SQUARED_ERROR, A.LOSS_SQUARED_ERROR)):
            for weights in (None, w):
                eng.load_margins(m)
                ok = eng.gradients(kind, y, weights, scale_pos_weight=1.5)
                got = eng.read_gradients()
                with np.errstate(invalid="ignore", over="ignore"):
                    want = O.gradient(obj, m, y, weights, scale_pos_weight=1.5)
                assert ok == bool(np.all(np.isfinite(want))), (n, obj)
                nan = np.isnan(want)
                assert np.array_equal(np.isnan(got), nan), (n, obj)
                assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32)), (n, obj)


def _softmax_case(rng, n, k, spread=3.0):
    m = (rng.standard_normal(n * k) * spread).astype(np.float32)
    if n > 8:
        m[k * 5 + k - 1] = -90.0   # a row spanning more than 80: its batch leaves the vector path
        m[k * 7: k * 8] = -30.0    # every margin below f32::MIN_POSITIVE
    y = rng.integers(0, k, n).astype(np.float32)
    w = (rng.random(n) * 2).astype(np.float32)
    return m, y, w


def test_device_softmax_gradients_match_oracle_bits():
    """Every class's pairs against the oracle (simd/mod.rs:502-600): the
    2- and 4-class vector batches and their scalar tails, rows that leave a
    batch to the scalar path, and other class counts, bit for bit."""
    rng = np.random.default_rng(16)
    for k in (1, 2, 3, 4, 10, 17):
        for n in (3, 5, 37, 4099):
            x = rng.standard_normal((n, 2), dtype=np.float32)
            ix, eng = make(x)
            m, y, w = _softmax_case(rng, n, k)
            for weights in (None, w):
                eng.load_margins(m, k)
                print("softmax", k, n, weights is not None, flush=True)
                assert eng.gradients(A.LOSS_SOFTMAX, y, weights)
                got = eng.read_gradients(k).reshape(k, n, 2)   # [class][row]
                want = O.gradient(O.OBJ_SOFTMAX, m, y, weights, num_class=k)  # [row][class]
                assert np.array_equal(got.view(np.uint32), want.transpose(1, 0, 2).view(np.uint32)), (k, n)


def test_device_softmax_expf_sweep_matches_host_libm():
    """Margins sweeping the f32 values in [-104, 0] (every 61st bit pattern,
    through the subnormal results and the underflow to 0) against the
    oracle's host expf: 16 classes per row, class 0 at 0."""
    k = 16
    xs = np.arange(0x80000000, 0xC2D00001, 61, dtype=np.uint64).astype(np.uint32).view(np.float32)
    n = -(-len(xs) // (k - 1))
    m = np.zeros((n, k), np.float32)
    flat = np.zeros(n * (k - 1), np.float32)
    flat[:len(xs)] = xs
    m[:, 1:] = flat.reshape(n, k - 1)
    m = m.reshape(-1)
    y = (np.arange(n) % k).astype(np.float32)
    x = np.zeros((n, 1), np.float32)
    x[::2] = 1.0
    ix, eng = make(x)
    eng.load_margins(m, k)
    assert eng.gradients(A.LOSS_SOFTMAX, y)
    got = eng.read_gradients(k)
    want = O.gradient(O.OBJ_SOFTMAX, m, y, num_class=k)
    bad = np.count_nonzero(got.view(np.uint32) != want.transpose(1, 0, 2).view(np.uint32))
    assert bad == 0, f"{bad} of {got.size} values differ"


def test_device_softmax_non_finite_rows_are_reported():
    """Rows of -200 underflow every exponential (0/0): NaN gradients, as
    the host's, and the gradients are reported not finite."""
    rng = np.random.default_rng(17)
    for k in (2, 4, 5):
        n = 64
        m, y, _ = _softmax_case(rng, n, k)
        m[k * 3: k * 4] = -200.0
        x = rng.standard_normal((n, 2), dtype=np.float32)
        ix, eng = make(x)
        eng.load_margins(m, k)
        assert not eng.gradients(A.LOSS_SOFTMAX, y)
        got = eng.read_gradients(k).transpose(1, 0, 2)
        with np.errstate(invalid="ignore"):
            want = O.gradient(O.OBJ_SOFTMAX, m, y, num_class=k)
        assert np.array_equal(np.isnan(got), np.isnan(want)) and np.isnan(want[3, :, 0]).all()
        fin = ~np.isnan(want)
        assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))
