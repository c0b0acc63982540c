"""The oracle's weighted quantile sketch (oracle/sketch.c, restating
data/sketch.rs:59-680) on data with more distinct values than max_bin,
where its summaries are pruned and merged, checked three ways that do not
restate the oracle's own code:

* brute force: every summary the streaming sketch forms (each flushed
  queue, each prune and merge of the level-wise carry, each merge of the
  final summary, the final summary) bounds the true ranks of the values it
  covers: rmin <= weight below v, rmax >= weight at or below v, wmin <=
  weight of v, the last entry's rmax is the covered total, and a flushed
  queue's summary holds the exact ranks. With whole-number weights every
  f32 rank is exact, so these hold with no tolerance;
* other formulations: the two-pointer SetPrune (sketch.rs:128-181) equals
  XGBoost's rule answered one query at a time by a plain search, and the
  branch-free merge (sketch.rs:218-345) equals XGBoost's three-case
  SetCombine as a sequential loop (the reference's own cross-check,
  sketch.rs:836-925), bit for bit on every field;
* the approximation guarantee: the final summary's error (XGBoost's
  MaxError) stays within eps * total for eps = 1 / max_bin, and every bin
  of the cuts holds at most 1.5 max_bin-ths of the weight (plus one value's
  weight);
* the budget schedule: the summary budget is the smallest level count's
  size by its definition (XGBoost's LimitSizeLevel with the oversampling
  factor 2, sketch.rs:59-85), the level-wise carry prunes to it, the final
  merge to the larger of it and the budget of the values seen, then to that
  budget (sketch.rs:660-708).

Planted mistakes in a copy of the oracle (a prune that always keeps the
left entry, reads one entry early, drops the gap's wmin terms, the tail or
the query offset; a merge that swaps the cursors' previous ranks, drops
rmax_prev, takes the tail's rmin, drops an equal pair's weight or FixError;
exact ranks off by a weight; the final or carry prune to the wrong size; a
query at the rank instead of twice it) each fail at least one test here.

The product's host sketch (csrc/host/cuts.cpp) is checked against the
oracle's cuts in tests/test_binning.py.
"""
import numpy as np
import pytest

from oracle import oracle as O

f32 = np.float32
RMIN, RMAX, WMIN, VALUE = range(4)


def streams():
    """(name, values, weights or None, max_bin): continuous, heavy repeats,
    signed zeros and infinities, ascending and descending order, weighted."""
    rng = np.random.default_rng(11)
    n = 60_000
    normal = rng.standard_normal(n).astype(f32)
    repeats = np.round(rng.standard_normal(n) * 40).astype(f32) / f32(8)
    special = normal.copy()
    pick = rng.random(n)
    special[pick < 0.05] = f32(-0.0)
    special[(pick >= 0.05) & (pick < 0.1)] = f32(0.0)
    special[(pick >= 0.1) & (pick < 0.11)] = f32(np.inf)
    special[(pick >= 0.11) & (pick < 0.12)] = f32(-np.inf)
    weights = rng.integers(1, 5, n).astype(f32)
    return [
        ("normal", normal, None, 16),
        ("normal_b64", normal, None, 64),
        ("normal_b256", rng.standard_normal(200_000).astype(f32), None, 256),
        ("repeats", repeats, None, 16),
        ("special", special, None, 8),
        ("ascending", np.sort(normal), None, 16),
        ("descending", np.sort(normal)[::-1].copy(), None, 16),
        ("weighted", normal, weights, 16),
        ("weighted_repeats", repeats, weights, 64),
    ]


def true_ranks(values, weights, lo, hi, v):
    """Weight of covered values below, at or below, and equal to each of v."""
    x = values[lo:hi]
    w = np.ones(len(x)) if weights is None else weights[lo:hi].astype(np.float64)
    keep = w != 0
    x, w = x[keep], w[keep]
    o = np.argsort(x, kind="stable")
    xs = x[o].astype(np.float64)
    cw = np.concatenate([[0.0], np.cumsum(w[o])])
    v = v.astype(np.float64)
    below = cw[np.searchsorted(xs, v, "left")]
    at_or_below = cw[np.searchsorted(xs, v, "right")]
    return below, at_or_below, cw[-1]


def max_error(e):
    """XGBoost's WQSummary::MaxError."""
    err = e[0, RMAX] - e[0, RMIN] - e[0, WMIN]
    for i in range(1, len(e)):
        err = max(err, (e[i, RMAX] - e[i, WMIN]) - (e[i - 1, RMIN] + e[i - 1, WMIN]),
                  e[i, RMAX] - e[i, RMIN] - e[i, WMIN])
    return float(err)


@pytest.mark.parametrize("case", streams(), ids=lambda c: c[0])
def test_every_summary_bounds_the_true_ranks(case):
    name, values, weights, max_bin = case
    cuts, recs = O.sketch_trace(values, weights, max_bin)
    kinds = {r[0] for r in recs}
    assert {"from_sorted", "prune", "combine", "final"} <= kinds
    assert sum(r[0] == "combine" for r in recs) > 20, "the stream must force level merges"
    assert len(recs[-1][3]) > max_bin, "the final summary must be queried, not listed"
    for kind, lo, hi, e, _ in recs:
        if len(e) == 0:
            continue
        v = e[:, VALUE]
        assert np.all(v[1:] > v[:-1]), (kind, lo, hi)
        below, at_or_below, total = true_ranks(values, weights, lo, hi, v)
        rmin, rmax, wmin = (e[:, k].astype(np.float64) for k in (RMIN, RMAX, WMIN))
        assert np.all(rmin <= below), (kind, lo, hi)
        assert np.all(rmax >= at_or_below), (kind, lo, hi)
        assert np.all(wmin <= at_or_below - below), (kind, lo, hi)
        assert np.all(rmin + wmin <= rmax), (kind, lo, hi)
        assert rmax[-1] == total, (kind, lo, hi)
        assert rmin[0] == 0.0, (kind, lo, hi)
        if kind == "from_sorted":
            assert np.array_equal(rmin, below) and np.array_equal(rmax, at_or_below), (lo, hi)
    assert recs[-1][1] == 0 and recs[-1][2] == len(values)


@pytest.mark.parametrize("case", streams(), ids=lambda c: c[0])
def test_final_summary_meets_the_rank_guarantee(case):
    name, values, weights, max_bin = case
    cuts, recs = O.sketch_trace(values, weights, max_bin)
    final = recs[-1][3].astype(np.float64)
    total = final[-1, RMAX]
    assert max_error(final) <= total / max_bin
    # the weight between consecutive cuts (bin b holds cuts[b-1] <= v < cuts[b])
    present = values if weights is None else values[weights != 0]
    w = np.ones(len(present)) if weights is None else weights[weights != 0].astype(np.float64)
    o = np.argsort(present, kind="stable")
    xs = present[o].astype(np.float64)
    cw = np.concatenate([[0.0], np.cumsum(w[o])])
    edges = cw[np.searchsorted(xs, cuts[:-1].astype(np.float64), "left")]
    mass = np.diff(np.concatenate([[0.0], edges, [cw[-1]]]))
    heaviest_value = max(np.bincount(np.unique(xs, return_inverse=True)[1], weights=w[o]))
    assert mass.max() <= 1.5 * total / max_bin + heaviest_value, name
    assert np.all(np.diff(cuts) > 0)


def prune_by_queries(e, maxsize):
    """XGBoost's SetPrune, each query answered by a plain search: for query
    k the first entry i >= 1 whose successor's rank midpoint lies above the
    query, then i or i + 1 by the gap's midpoint; f32 arithmetic."""
    src = len(e)
    if maxsize == 0:
        return e[:0]
    if src <= maxsize:
        return e
    if maxsize == 1:
        return e[:1]
    begin = e[0, RMAX]
    rng_ = f32(e[-1, RMIN] - e[0, RMAX])
    n = maxsize - 1
    mid2 = (e[:, RMAX] + e[:, RMIN]).astype(f32)
    out, last = [0], 0
    for k in range(1, n):
        dx2 = f32(2.0) * f32(f32(f32(k) * rng_) / f32(n) + begin)
        above = np.nonzero(dx2 < mid2[2:])[0]
        i = int(above[0]) + 1 if len(above) else src - 1
        if i == src - 1:
            break
        gap = f32(f32(e[i, RMIN] + e[i, WMIN]) + f32(e[i + 1, RMAX] - e[i + 1, WMIN]))
        pick = i if dx2 < gap else i + 1
        if pick != last:
            out.append(pick)
            last = pick
    if last != src - 1:
        out.append(src - 1)
    return e[out]


def fix_error(e):
    prev_rmin = prev_rmax = f32(0.0)
    for r in e:
        if r[RMIN] < prev_rmin:
            r[RMIN] = prev_rmin
        else:
            prev_rmin = r[RMIN]
        if r[RMAX] < prev_rmax:
            r[RMAX] = prev_rmax
        nxt = f32(r[RMIN] + r[WMIN])
        if r[RMAX] < nxt:
            r[RMAX] = nxt
        prev_rmax = r[RMAX]
    return e


def combine_three_cases(a, b):
    """XGBoost's SetCombine as one sequential merge with its three cases and
    tail loops (the formulation of sketch.rs:836-893), then FixError."""
    if len(b) == 0:
        return a.copy()
    if len(a) == 0:
        return b.copy()
    out = []
    ia = ib = 0
    ap = bp = f32(0.0)
    while ia < len(a) and ib < len(b):
        ea, eb = a[ia], b[ib]
        if ea[VALUE] == eb[VALUE]:
            out.append((ea[RMIN] + eb[RMIN], ea[RMAX] + eb[RMAX], ea[WMIN] + eb[WMIN], ea[VALUE]))
            ap, bp = f32(ea[RMIN] + ea[WMIN]), f32(eb[RMIN] + eb[WMIN])
            ia += 1
            ib += 1
        elif ea[VALUE] < eb[VALUE]:
            out.append((ea[RMIN] + bp, ea[RMAX] + f32(eb[RMAX] - eb[WMIN]), ea[WMIN], ea[VALUE]))
            ap = f32(ea[RMIN] + ea[WMIN])
            ia += 1
        else:
            out.append((eb[RMIN] + ap, eb[RMAX] + f32(ea[RMAX] - ea[WMIN]), eb[WMIN], eb[VALUE]))
            bp = f32(eb[RMIN] + eb[WMIN])
            ib += 1
    for ea in a[ia:]:
        out.append((ea[RMIN] + bp, ea[RMAX] + b[-1, RMAX], ea[WMIN], ea[VALUE]))
    for eb in b[ib:]:
        out.append((eb[RMIN] + ap, eb[RMAX] + a[-1, RMAX], eb[WMIN], eb[VALUE]))
    return fix_error(np.array(out, f32).reshape(-1, 4))


def random_summary(rng, pool, n):
    """n values from the pool, sorted by total order, weights 1..3, pruned
    to n / 2 + 1 (the reference's random_summary, sketch.rs:895-909)."""
    v = pool[rng.integers(0, len(pool), n)]
    key = v.view(np.int32) ^ ((v.view(np.int32) >> 31) & 0x7FFFFFFF)
    v = v[np.argsort(key, kind="stable")]
    w = rng.integers(1, 4, n).astype(f32)
    return O.summary_prune(O.summary_from_sorted(v, w), n // 2 + 1)


def test_merge_equals_the_three_case_sequential_merge_bit_for_bit():
    rng = np.random.default_rng(9)
    for case in range(40):
        pool = ((rng.random([50, 4000, 100_000][case % 3]) - 0.5) * 100.0).astype(f32)
        pool = np.concatenate([pool, np.array([-0.0, 0.0, np.inf, -np.inf], f32)])
        if case % 7 == 6:
            pool = np.concatenate([pool, np.array([np.nan], f32)])
        a = random_summary(rng, pool, int(rng.integers(1, 6000)))
        b = random_summary(rng, pool, int(rng.integers(1, 6000)))
        got = O.summary_combine(a, b)
        want = combine_three_cases(a, b)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), case


def test_prune_equals_the_rule_answered_query_by_query():
    """On every summary the sketch formed for the streams above, pruned to
    sizes from 2 to beyond its length."""
    checked = 0
    for name, values, weights, max_bin in streams()[:6]:
        _, recs = O.sketch_trace(values, weights, max_bin)
        for kind, lo, hi, e, _ in recs[::7]:
            for size in (2, 3, max_bin, len(e) // 2 + 1, len(e) - 1, len(e)):
                if size < 2:
                    continue
                got = O.summary_prune(e, size)
                want = prune_by_queries(e, size)
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (name, kind, lo, size)
                checked += 1
    assert checked > 300


def test_flushed_queue_summary_is_exact_with_fractional_weights():
    """SetFromSorted keeps exact prefix sums up to f32 rounding: rmin is the
    f32 running sum of the weights before each distinct value."""
    rng = np.random.default_rng(5)
    v = np.sort(np.round(rng.standard_normal(3000) * 20).astype(f32))
    w = rng.random(3000).astype(f32)
    e = O.summary_from_sorted(v, w)
    u, first = np.unique(v, return_index=True)
    assert np.array_equal(e[:, VALUE], u)
    acc, rmin = f32(0.0), []
    ends = list(first[1:]) + [len(v)]
    for s, t in zip(first, ends):
        rmin.append(acc)
        wi = w[s]
        for j in range(s + 1, t):
            wi = f32(wi + w[j])
        acc = f32(acc + wi)
    assert np.array_equal(e[:, RMIN], np.array(rmin, f32))


def budget_by_definition(max_bin, n):
    eps = 1.0 / min(max_bin, max(n, 1))
    if n == 0:
        return 1
    level = 1
    while True:
        limit = min(int(np.ceil(level / (eps / 2.0))) + 1, n)
        if (1 << level) * limit >= n:
            return limit
        level += 1


def test_summary_budget_follows_its_definition():
    for max_bin in (2, 3, 8, 16, 64, 255, 256, 1024):
        for n in (0, 1, 2, 5, 100, 257, 1000, 4097, 65_536, 1_000_000, 10_500_000, 123_456_789):
            assert O.summary_budget(max_bin, n) == budget_by_definition(max_bin, n), (max_bin, n)


@pytest.mark.parametrize("case", streams()[:5], ids=lambda c: c[0])
def test_the_sketch_prunes_to_its_budgets(case):
    name, values, weights, max_bin = case
    n = len(values) if weights is None else int(np.count_nonzero(weights))
    limit = O.summary_budget(max_bin, n)
    _, recs = O.sketch_trace(values, weights, max_bin)
    prunes = [r for r in recs if r[0] == "prune"]
    assert prunes and all(size == limit and len(e) <= limit for _, _, _, e, size in prunes)
    # a level's summary is pruned before it is merged, so a merge holds at most twice the budget
    assert all(len(r[3]) <= 2 * limit for r in recs if r[0] == "combine")
    assert all(r[4] == max(limit, O.summary_budget(max_bin, n)) for r in recs if r[0] == "summary")
    assert recs[-1][4] == O.summary_budget(max_bin, n) and len(recs[-1][3]) <= recs[-1][4]
    # a full queue (2 x the budget distinct entries) was summarised at every flush but the last
    flushes = [r for r in recs if r[0] == "from_sorted"]
    assert all(hi - lo >= 2 * limit for _, lo, hi, _, _ in flushes[:-1]) or name == "repeats"


def test_merge_of_loose_summaries_equals_the_three_case_merge():
    """Summaries that merges have loosened (rmax above rmin + wmin), taken
    from the sketch's own level merges, merged pairwise."""
    for name, values, weights, max_bin in streams()[:4]:
        _, recs = O.sketch_trace(values, weights, max_bin)
        loose = [r[3] for r in recs if r[0] in ("combine", "summary") and len(r[3]) > 2]
        loose = [e for e in loose if np.any(e[:, RMAX] > e[:, RMIN] + e[:, WMIN])]
        assert len(loose) >= 4, name
        for a, b in zip(loose[::3], loose[1::3][::-1]):
            got = O.summary_combine(a, b)
            want = combine_three_cases(a, b)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), name


def test_merge_of_inconsistent_ranks_applies_fix_error():
    """Entries whose rank fields break monotonicity (not a valid summary):
    the merge's FixError pass decides every rmin and rmax."""
    rng = np.random.default_rng(12)
    for case in range(30):
        def entries(n):
            v = np.unique(rng.standard_normal(n).astype(f32))
            r = rng.integers(0, 50, (len(v), 3)).astype(f32)
            return np.column_stack([r[:, 0], r[:, 1], r[:, 2] + 1, v]).astype(f32)
        a, b = entries(int(rng.integers(1, 400))), entries(int(rng.integers(1, 400)))
        got = O.summary_combine(a, b)
        want = combine_three_cases(a, b)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), case
