"""Shared fixtures and comparison helpers.

GPU tests (marker ``gpu``) call libneural_hip.so through the pyneural ctypes
layer and compare against the CPU oracle (oracle/ora.py).  CPU tests check
the oracle itself against closed forms, the reference's own C and the
committed golden fixtures.
"""

import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT / "neural-assembly_amd", ROOT / "oracle", ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libneural_hip.so)")


@pytest.fixture(scope="session")
def ora():
    import ora as _ora
    _ora.lib()
    return _ora


@pytest.fixture(scope="session")
def pn():
    import pyneural
    pyneural.init()
    return pyneural


def same_bits(got, want):
    """Bitwise equality with NaNs compared by class (payload and sign of NaN
    differ between x86 and AMD defaults)."""
    got = np.asarray(got)
    want = np.asarray(want)
    assert got.shape == want.shape, (got.shape, want.shape)
    assert got.dtype == want.dtype, (got.dtype, want.dtype)
    if got.dtype.kind == "f":
        gn, wn = np.isnan(got), np.isnan(want)
        assert np.array_equal(gn, wn), f"NaN positions differ ({int(np.sum(gn != wn))} elements)"
        u = np.uint32 if got.dtype == np.float32 else np.uint64
        gb, wb = got.view(u)[~gn], want.view(u)[~wn]
        bad = np.nonzero(gb != wb)[0]
        assert bad.size == 0, f"{bad.size} elements differ; first: got {got[~gn][bad[0]]!r} want {want[~wn][bad[0]]!r}"
    else:
        bad = np.nonzero(got != want)[0] if got.ndim == 1 else np.argwhere(got != want)
        assert len(bad) == 0, f"{len(bad)} elements differ; first at {bad[0]}"


def rel_close(got, want, rtol, atol=0.0, what=""):
    """|g - w| <= rtol*|w| + atol elementwise, NaN/Inf by class."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    gn, wn = np.isnan(got), np.isnan(want)
    assert np.array_equal(gn, wn), f"{what}: NaN positions differ"
    gi, wi = np.isinf(got), np.isinf(want)
    assert np.array_equal(gi & (got > 0), wi & (want > 0)) and np.array_equal(gi & (got < 0), wi & (want < 0)), \
        f"{what}: Inf positions differ"
    m = ~(gn | gi)
    err = np.abs(got[m] - want[m])
    lim = rtol * np.abs(want[m]) + atol
    bad = np.nonzero(err > lim)[0]
    assert bad.size == 0, (f"{what}: {bad.size} elements out of tolerance; worst rel "
                           f"{np.max(err / np.maximum(np.abs(want[m]), 1e-300)):.3e} at got={got[m][bad[0]]!r} "
                           f"want={want[m][bad[0]]!r}")


def special_f32(n, rng, frac=0.01):
    """Uniform[-1,1] data salted with NaN, +-Inf, +-0, denormals and extremes."""
    x = rng.uniform(-1, 1, n).astype(np.float32)
    k = max(1, int(n * frac)) if n >= 16 else 0
    if k:
        idx = rng.choice(n, size=min(k, n), replace=False)
        pool = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 1e-45, -1e-45, 3.4e38, -3.4e38, 1e-38],
                        dtype=np.float32)
        x[idx] = pool[rng.integers(0, pool.size, idx.size)]
    return x


def special_f64(n, rng, frac=0.01):
    x = rng.uniform(-1, 1, n)
    k = max(1, int(n * frac)) if n >= 16 else 0
    if k:
        idx = rng.choice(n, size=min(k, n), replace=False)
        pool = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 5e-324, -5e-324, 1.7e308, -1.7e308, 2.2e-308])
        x[idx] = pool[rng.integers(0, pool.size, idx.size)]
    return x


def fmaf_exact(a, b, c):
    """Correctly rounded float32 fma(a, b, c), elementwise.  a*b of two floats
    is exact in double; the sum with c is rounded to odd in double (TwoSum's
    error term says whether it was inexact and on which side), and a value
    rounded to odd with at least two bits more than the target rounds to the
    target as the exact value would.  Plain (double)a*b + c, rounded to
    float afterwards, rounds twice and misses fmaf when the exact sum lies
    just past a float tie."""
    a64, b64, c64 = (np.asarray(v, dtype=np.float32).astype(np.float64) for v in (a, b, c))
    with np.errstate(all="ignore"):
        p = a64 * b64
        s = p + c64
        bb = s - p
        err = (p - (s - bb)) + (c64 - bb)
        inexact = np.isfinite(s) & (err != 0)
        # truncate toward zero: step back one double when the exact value is smaller in magnitude
        rz = np.where(inexact & (np.sign(err) != np.sign(s)), np.nextafter(s, 0.0), s)
        bits = rz.view(np.uint64)
        odd = np.where(inexact, bits | np.uint64(1), bits).view(np.float64)
        return odd.astype(np.float32)


_KEEP = []


def keep(t):
    """Pointer of a wrapper object that stays alive until the test ends (a
    temporary's pointer would be freed before the ctypes call runs)."""
    _KEEP.append(t)
    return t._ptr


@pytest.fixture(autouse=True)
def _release_kept():
    yield
    _KEEP.clear()


@pytest.fixture
def rng():
    return np.random.default_rng(1234)


GPU = pytest.mark.gpu
