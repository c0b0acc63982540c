"""The objective's prediction transform on the host (hbr_pred_transform,
the reference's Transform::apply, src/model/transform.rs:74-104): XGBoost's
sigmoid and softmax through the C library's expf (simd/mod.rs:422-427,
:557-573) and multi:softmax's class index (simd/mod.rs:750-758). Runs on the
CPU: the call touches no device."""
import ctypes as C
import ctypes.util

import numpy as np
import pytest

from hessboost_amd import _capi as A
from oracle import oracle as O

LIBM = C.CDLL(ctypes.util.find_library("m"))
LIBM.expf.restype = C.c_float
LIBM.expf.argtypes = [C.c_float]


def transform(kind, values, n_outputs=1):
    v = np.ascontiguousarray(values, np.float32).reshape(-1).copy()
    A.check(A.lib().hbr_pred_transform(kind, A.ptr(v), v.size // n_outputs, n_outputs))
    return v


def expf(x):
    return np.float32(LIBM.expf(float(x)))


def sweep(rng, n):
    """Margins across the sigmoid's whole range, its clamp at 88.7 and the
    special values."""
    x = np.concatenate([rng.standard_normal(n // 2) * 4, rng.uniform(-120, 120, n // 2),
                        [0.0, -0.0, 88.7, -88.7, 88.70001, -88.70001, 1e-30, -1e-30, np.inf, -np.inf, np.nan]])
    return x.astype(np.float32)


def test_sigmoid_is_the_c_library_expf_formula_and_the_oracle():
    x = sweep(np.random.default_rng(1), 4_000)
    got = transform(A.TRANSFORM_SIGMOID, x)
    one = np.float32(1.0)
    want = np.array([one / (expf(np.fmin(-v, np.float32(88.7))) + one) for v in x], np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    oracle = np.array([O.lib().or_sigmoid(float(v)) for v in x], np.float32)
    assert np.array_equal(got.view(np.uint32), oracle.view(np.uint32))
    # what the mathematics fixes: 1/2 at zero, the NaN margin clamped like -88.7
    # (f32::min returns the number), symmetry to within an ulp of 1
    assert transform(A.TRANSFORM_SIGMOID, [0.0, -0.0]).tolist() == [0.5, 0.5]
    assert transform(A.TRANSFORM_SIGMOID, [np.nan])[0] == transform(A.TRANSFORM_SIGMOID, [-88.7])[0]
    mid = x[np.abs(x) < 10]
    s = transform(A.TRANSFORM_SIGMOID, mid) + transform(A.TRANSFORM_SIGMOID, -mid)
    assert np.max(np.abs(s.astype(np.float64) - 1.0)) <= 2 ** -23


def test_large_inputs_are_transformed_in_parallel_blocks_with_the_same_bits():
    x = sweep(np.random.default_rng(2), 200_000)
    whole = transform(A.TRANSFORM_SIGMOID, x)
    parts = np.concatenate([transform(A.TRANSFORM_SIGMOID, x[i:i + 1000]) for i in range(0, x.size, 1000)])
    assert np.array_equal(whole.view(np.uint32), parts.view(np.uint32))


def softmax_row(row):
    wmax = row[0]
    for v in row[1:]:
        wmax = np.float32(np.fmax(v, wmax))
    e = [expf(np.float32(v - wmax)) for v in row]
    s = np.float32(sum(float(v) for v in e))
    return np.array([np.float32(v / s) for v in e], np.float32)


@pytest.mark.parametrize("k", [1, 2, 3, 4, 7, 10])
def test_softmax_rows_sum_in_f64_and_divide_by_the_f32_sum(k):
    rng = np.random.default_rng(k)
    m = (rng.standard_normal((500, k)) * rng.choice([0.1, 3.0, 40.0], (500, 1))).astype(np.float32)
    m[5] = 0.0
    m[6, 0] = np.nan
    m[7] = np.float32(1e30)
    got = transform(A.TRANSFORM_SOFTMAX, m, k).reshape(-1, k)
    want = np.stack([softmax_row(r) for r in m])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    ok = ~np.isnan(m).any(1)
    assert np.max(np.abs(got[ok].astype(np.float64).sum(1) - 1.0)) <= k * 2 ** -23


@pytest.mark.parametrize("k", [1, 2, 4, 8, 16])
def test_softmax_of_equal_margins_is_exactly_one_over_k(k):
    got = transform(A.TRANSFORM_SOFTMAX, np.full((3, k), 2.5, np.float32), k)
    assert np.all(got == np.float32(1.0 / k))


def test_class_index_takes_the_first_largest_margin():
    m = np.array([[0.1, 0.5, 0.5],           # tie: the first
                  [np.nan, 3.0, 1.0],         # nothing beats a leading NaN
                  [1.0, np.nan, 2.0],         # a NaN is never taken
                  [-np.inf, -np.inf, -1.0],
                  [2.0, 2.0, 2.0]], np.float32)
    got = transform(A.TRANSFORM_CLASS_INDEX, m, 3)
    assert got[:5].tolist() == [1.0, 0.0, 2.0, 2.0, 0.0]
    rng = np.random.default_rng(3)
    r = rng.standard_normal((1000, 5)).astype(np.float32)
    assert np.array_equal(transform(A.TRANSFORM_CLASS_INDEX, r, 5)[:1000], np.argmax(r, 1).astype(np.float32))


def test_transform_refuses_bad_arguments():
    with pytest.raises(A.HbrError) as e:
        transform(99, [1.0])
    assert e.value.status == A.INVALID
    v = np.ones(1, np.float32)
    assert A.lib().hbr_pred_transform(A.TRANSFORM_SOFTMAX, A.ptr(v), 1, 0) == A.INVALID
