"""Device binning (hbr_engine_open_dense): a dense f32 matrix binned on the GPU
against host cuts must give the index the host builds (HistCuts::bin_of,
src/data/quantile.rs:285-296; GHistIndex::from_dmatrix,
src/data/ghist.rs:213-257) byte for byte, in every layout the engine keeps."""
import numpy as np
import pytest

import hessboost_amd as hb

pytestmark = pytest.mark.gpu


def _layouts(x, max_bin, missing=np.nan, on_device=False):
    dm = hb.DMatrix(x, missing=missing)
    cuts = dm.cuts(max_bin)
    host = hb.Engine(dm.index(max_bin), 0).read_index()
    if on_device:
        buf = hb.DeviceBuffer(x.nbytes)
        buf.upload(x)
        dev = hb.Engine.from_dense(buf, cuts, 0, missing=missing, n_rows=x.shape[0], n_cols=x.shape[1])
    else:
        dev = hb.Engine.from_dense(x, cuts, 0, missing=missing)
    return host, dev.read_index()


def _same(host, dev):
    for k in ("dense", "dense_u8", "has_cols", "has_missing", "entries"):
        assert host[k] == dev[k], k
    for k in ("rows8", "cols8", "missing", "row_ptr", "gbins"):
        if host[k] is None:
            assert dev[k] is None, k
        else:
            assert np.array_equal(host[k], dev[k]), k


def test_dense_matrix_bins_equal_host_bins():
    rng = np.random.default_rng(20)
    x = rng.standard_normal((30_001, 40)).astype(np.float32)  # a ragged last 64-row group
    x[:, 7] = np.round(x[:, 7])                                 # few distinct values
    x[:, 8] = 3.0                                               # a constant feature
    host, dev = _layouts(x, 256)
    assert dev["dense_u8"] == 1
    _same(host, dev)


def test_values_on_cut_points_signed_zeros_and_infinities():
    rng = np.random.default_rng(21)
    x = rng.standard_normal((8_192, 6)).astype(np.float32)
    x[:500, 0] = 0.0
    x[500:1000, 0] = -0.0
    x[1000:1100, 1] = np.inf
    x[1100:1200, 1] = -np.inf
    x[1200:1300, 2] = np.float32(1e-40)                         # subnormal
    dm = hb.DMatrix(x)
    _, cv = dm.cuts(64).arrays()
    x[2000:2000 + len(cv), 3] = cv[:min(len(cv), 6192)]         # exactly the cut values
    host, dev = _layouts(x, 64)
    _same(host, dev)


@pytest.mark.parametrize("frac", [0.1, 0.9])
def test_missing_values_give_the_host_csr_columns_and_bitmap(frac):
    """10% NaN keeps columns and a missing bitmap beside the CSR rows; 90%
    NaN over 300 features keeps CSR rows only (cells > 2 x entries)."""
    rng = np.random.default_rng(22)
    n, f = (20_000, 30) if frac < 0.5 else (6_000, 300)
    x = rng.exponential(size=(n, f)).astype(np.float32)
    x[rng.random(x.shape) < frac] = np.nan
    host, dev = _layouts(x, 64)
    assert dev["dense"] == 0
    assert dev["has_cols"] == (1 if frac < 0.5 else 0)
    _same(host, dev)


def test_missing_marker_other_than_nan():
    """With -999 as the marker, -999 cells are absent and NaN cells present
    (bin_of puts a NaN in the feature's last bin)."""
    rng = np.random.default_rng(23)
    x = rng.standard_normal((10_000, 12)).astype(np.float32)
    x[rng.random(x.shape) < 0.05] = -999.0
    x[rng.random(x.shape) < 0.01] = np.nan
    host, dev = _layouts(x, 128, missing=-999.0)
    _same(host, dev)


@pytest.mark.parametrize("f", [1, 27, 32])
@pytest.mark.parametrize("on_device", [False, True])
def test_rows_of_up_to_32_features_staged_through_lds(f, on_device):
    """hbr_bin_dense32: each wave's rows copied into LDS with 16-byte loads,
    every 32-byte row written whole; a ragged last wave and workgroup, every
    byte of the rows (padding included) against the host index."""
    rng = np.random.default_rng(30 + f)
    x = rng.standard_normal((20_037, f)).astype(np.float32)
    x[:, 0] = np.round(x[:, 0] * 2)  # few distinct values: cells on the cut points
    x[5, :] = np.inf
    x[6, :] = -np.inf
    host, dev = _layouts(x, 256, on_device=on_device)
    assert dev["dense_u8"] == 1
    _same(host, dev)


def test_rows_already_on_the_device():
    rng = np.random.default_rng(24)
    x = rng.standard_normal((12_345, 28)).astype(np.float32)
    host, dev = _layouts(x, 256, on_device=True)
    _same(host, dev)


@pytest.mark.parametrize("f,n", [(28, 2_400_017), (45, 1_600_003)])
def test_host_rows_in_chunks_bin_as_rows_on_the_device(f, n):
    """Host rows beyond two 128 MiB chunks are binned chunk by chunk as they
    arrive through the device's pinned staging buffers (the last chunk
    ragged): every layout equals, byte for byte, the index binned from the
    same rows already on the device, with missing cells (masked rows of 32
    and of 64 bytes)."""
    rng = np.random.default_rng(26 + f)
    x = rng.standard_normal((n, f)).astype(np.float32)
    x[rng.random((n, f)) < 0.02] = np.nan
    x[:, 3] = np.round(x[:, 3])
    cuts = hb.DMatrix(x[:200_000]).cuts(256)
    host_rows = hb.Engine.from_dense(x, cuts, 0).read_index()
    buf = hb.DeviceBuffer(x.nbytes)
    buf.upload(x)
    dev_rows = hb.Engine.from_dense(buf, cuts, 0, n_rows=n, n_cols=f).read_index()
    assert host_rows["dense_u8"] == 1
    _same(dev_rows, host_rows)


def test_features_wider_than_256_bins_are_refused():
    rng = np.random.default_rng(25)
    x = rng.standard_normal((5_000, 3)).astype(np.float32)
    cuts = hb.DMatrix(x).cuts(1024)
    with pytest.raises(hb.HbrError):
        hb.Engine.from_dense(x, cuts, 0)


@pytest.mark.parametrize("on_device", [False, True])
def test_few_features_with_missing_values_keep_masked_dense_rows(on_device):
    """A matrix of at most 28 features with missing cells keeps, beside the
    CSR rows, columns and bitmap the host builds, dense u8 rows of 32 bytes
    whose last word marks the row's missing features; the device-binned rows
    and those the engine makes from a host index's columns agree byte for
    byte, and the masks equal the bitmap."""
    rng = np.random.default_rng(26)
    n, f = 20_011, 28
    x = rng.standard_normal((n, f)).astype(np.float32)
    x[rng.random(x.shape) < 0.03] = np.nan
    host, dev = _layouts(x, 256, on_device=on_device)
    assert dev["dense"] == 0 and dev["dense_u8"] == 1 and dev["stride"] == 32
    _same(host, dev)
    rows = dev["rows8"].reshape(n, 32)
    mask = rows[:, 28:32].copy().view(np.uint32).reshape(-1)
    want = np.zeros(n, np.uint32)
    for j in range(f):
        want |= np.isnan(x[:, j]).astype(np.uint32) << np.uint32(j)
    assert np.array_equal(mask, want)
    assert np.all(rows[:, :28][np.isnan(x)] == 0)  # a missing cell's byte is 0


@pytest.mark.parametrize("f,on_device", [(29, False), (70, True), (256, False)])
def test_wide_matrices_with_missing_values_keep_masked_rows_of_groups(f, on_device):
    """Beyond 28 features, rows of G = ceil(f / 32) groups of 32 bins and a
    32-byte chunk of mask words (stride 32 G + 32): a row's bins (0 where
    missing), zeros up to its mask words, bit j % 32 of mask word j / 32 set
    exactly where feature j is missing; the device-binned rows equal those
    made from a host index's columns."""
    rng = np.random.default_rng(27 + f)
    n = 3_001
    x = rng.standard_normal((n, f)).astype(np.float32)
    x[rng.random(x.shape) < 0.05] = np.nan
    host, dev = _layouts(x, 256, on_device=on_device)
    g = (f + 31) // 32
    assert dev["dense"] == 0 and dev["dense_u8"] == 1 and dev["stride"] == 32 * g + 32
    _same(host, dev)
    rows = dev["rows8"].reshape(n, 32 * g + 32)
    miss = np.isnan(x)
    assert np.all(rows[:, :f][miss] == 0)
    assert np.all(rows[:, f:32 * g] == 0)
    words = rows[:, 32 * g:36 * g].copy().view(np.uint32)
    bits = ((words[:, :, None] >> np.arange(32, dtype=np.uint32)) & 1).reshape(n, 32 * g).astype(bool)
    assert np.array_equal(bits[:, :f], miss)
    assert not bits[:, f:].any()
    assert np.all(rows[:, 36 * g:] == 0)
