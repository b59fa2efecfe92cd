"""The oracle's draft-head argmax picks (crates/cuda/csrc/dsv4_mtp_gpu.cu:503-539, crates/cuda/csrc/mtp.cu:78-117)
against numpy restatements: the argmax is the first index of the largest value above -inf (NaN never counts, +0 and -0
tie, 0 for a row with none), and the pick's probability is the float64 softmax of the maximum."""
import numpy as np
import pytest

from oracle import oracle as O


def _np_argmax(x):
    x = np.asarray(x, dtype=np.float32)
    ok = x > -np.inf  # False for NaN and -inf
    if not ok.any():
        return 0
    m = x[ok].max()
    return int(np.flatnonzero(ok & (x == m))[0])


def _bf16(a):
    return (np.asarray(a, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)


def _from_bf16(b):
    return (b.astype(np.uint32) << 16).view(np.float32)


def test_row_argmax_matches_numpy_with_ties_nan_inf_and_signed_zero():
    rng = np.random.default_rng(3)
    rows = []
    for _ in range(40):
        x = rng.integers(-3, 4, size=257).astype(np.float32)  # many ties
        rows.append(x)
    a = np.full(300, -np.inf, np.float32)
    rows.append(a)                                    # no value above -inf -> 0
    b = np.full(300, np.nan, np.float32)
    b[7] = -np.inf
    rows.append(b)                                    # NaN and -inf only -> 0
    c = np.zeros(300, np.float32)
    c[:5] = -0.0
    rows.append(c)                                    # -0 first: it stays (ties with +0)
    d = rng.normal(size=300).astype(np.float32)
    d[[11, 200]] = np.inf
    d[3] = np.nan
    rows.append(d)                                    # +inf wins, first of two
    e = np.full(300, -1.0, np.float32)
    e[299] = np.nan
    rows.append(e)
    X = np.stack([r[:257] for r in rows])
    got = O.row_argmax(X)
    want = np.array([_np_argmax(r) for r in X], dtype=np.int32)
    assert np.array_equal(got, want)
    assert got[40] == 0 and got[41] == 0 and got[42] == 0 and got[43] == 11


@pytest.mark.parametrize("n", [1, 7, 4096, 129280])
def test_mtp_pick_matches_numpy(n):
    rng = np.random.default_rng(n)
    x = _bf16(rng.normal(scale=3.0, size=n))
    if n > 10:
        x[5] = x[n - 1] = _bf16([50.0])[0]  # a tie at the maximum: the first one
    i, p = O.mtp_pick(x)
    f = _from_bf16(x).astype(np.float64)
    assert i == _np_argmax(f.astype(np.float32))
    want = 1.0 / np.exp(f - f.max()).sum()
    assert p == pytest.approx(want, rel=1e-6)


def test_mtp_pick_nan_and_empty_rows():
    x = _bf16(np.array([1.0, np.nan, 3.0], np.float32))
    i, p = O.mtp_pick(x)
    assert i == 2 and np.isnan(p)
    x = _bf16(np.full(5, -np.inf, np.float32))
    i, p = O.mtp_pick(x)
    assert i == 0 and np.isnan(p)
