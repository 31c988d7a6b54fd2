"""CPU checks of the dropout oracle and the random stream it draws from.

ora_dropout_forward is the reference's dropout_forward (training_ops.asm:
718-790) written in C over the C library's own rand(), the generator the
reference calls.  What pins it:
  - rand() after srand(s) equals ora.glibc_rand, a restatement of glibc's
    TYPE_3 generator (the model the GPU stream implements), for several seeds,
    including 0 and seeds with the sign bit set;
  - hand-derived thresholds: p = 0.5 gives 0.5 * 2147483647 = 1073741823.5,
    which cvtsd2si rounds half to even to 1073741824; p = 0 keeps every
    element; p = 1 keeps only draws equal to RAND_MAX (scale inf); a NaN p
    gives the integer indefinite (keep all) with a NaN scale;
  - out = x * (float)(1 / (1 - p)) where kept and +0 where dropped, and the
    keep rate of a million draws within 5 sigma of 1 - p;
  - backward: any nonzero mask byte keeps.
ora_glibc_window (positions far into the stream by the jump x^k mod
x^31 - x^28 - 1, used to check GPU windows 2^31 draws in) is pinned against
rand() itself (ora_rand_n) at skips up to 3 * 10^6 + 7, against ora.glibc_rand
at skips around the 31-value period and the 344-value warm-up, and by the
jump's composition (skip a then b equals skip a + b).
"""

import ctypes
import math

import numpy as np
import pytest

import ora

libc = ctypes.CDLL("libc.so.6")


@pytest.mark.parametrize("seed", [1, 0, 7, 12345, 2 ** 31 - 1, 2 ** 31, 2 ** 32 - 1])
def test_libc_rand_is_the_modelled_stream(seed):
    libc.srand(ctypes.c_uint(seed))
    got = np.array([libc.rand() for _ in range(5000)], dtype=np.uint32)
    assert np.array_equal(got, ora.glibc_rand(seed, 5000))
    # a later window of the same stream
    assert np.array_equal(ora.glibc_rand(seed, 100, skip=4900), got[4900:])


def _expect(x, p, draws):
    pd = float(np.float32(p))
    th = 1073741824 if pd == 0.5 else round(pd * 2147483647.0)
    keep = draws.astype(np.int64) >= th
    scale = np.float32(1.0 / (1.0 - pd))
    return np.where(keep, x * scale, np.float32(0.0)).astype(np.float32), keep.astype(np.uint8)


@pytest.mark.parametrize("p", [0.5, 0.1, 0.25, 0.9])
def test_forward_matches_stream(p):
    rng = np.random.default_rng(5)
    x = rng.normal(0, 1, 10_007).astype(np.float32)
    ora.srand(99)
    rc, out, mask = ora.dropout_forward(x, p)
    assert rc == 0
    want_out, want_mask = _expect(x, p, ora.glibc_rand(99, x.size))
    assert np.array_equal(mask, want_mask)
    assert np.array_equal(out.view(np.uint32), want_out.view(np.uint32))
    # the stream continues across calls
    rc, out2, mask2 = ora.dropout_forward(x[:333], p)
    assert np.array_equal(mask2, _expect(x[:333], p, ora.glibc_rand(99, 333, skip=x.size))[1])


def test_threshold_half_rounds_to_even():
    assert round(0.5 * 2147483647.0) == 1073741824  # Python rounds half to even, as cvtsd2si does
    draws = ora.glibc_rand(3, 200_000)
    ora.srand(3)
    _, _, mask = ora.dropout_forward(np.ones(draws.size, np.float32), 0.5)
    assert np.array_equal(mask == 0, draws < 1073741824)


def test_edge_probabilities():
    x = np.linspace(-2, 2, 4096).astype(np.float32)
    ora.srand(11)
    _, out, mask = ora.dropout_forward(x, 0.0)
    assert mask.all() and np.array_equal(out, x)
    ora.srand(11)
    draws = ora.glibc_rand(11, x.size)
    _, out, mask = ora.dropout_forward(x, 1.0)
    assert np.array_equal(mask.astype(bool), draws == 2147483647)
    assert np.all(out[mask == 0] == 0)
    ora.srand(11)
    _, out, mask = ora.dropout_forward(x, float("nan"))
    assert mask.all() and np.isnan(out).all()
    ora.srand(11)
    _, out, mask = ora.dropout_forward(x, -0.5)  # negative p: threshold < 0, nothing dropped
    assert mask.all() and np.array_equal(out, x * np.float32(1.0 / 1.5))


def test_keep_rate():
    n = 1_000_000
    ora.srand(2024)
    _, _, mask = ora.dropout_forward(np.ones(n, np.float32), 0.3)
    rate = mask.mean()
    assert abs(rate - 0.7) < 5 * math.sqrt(0.21 / n)


def test_dropped_is_positive_zero_and_backward():
    x = np.full(1000, -3.0, np.float32)
    x[::7] = np.nan
    ora.srand(5)
    _, out, mask = ora.dropout_forward(x, 0.5)
    dropped = out[mask == 0]
    assert np.all(dropped.view(np.uint32) == 0)  # +0, also where the input was NaN
    m = np.array([0, 1, 2, 255, 0, 1], np.uint8)
    go = np.array([1.5, -2.0, 3.0, np.nan, np.inf, 0.25], np.float32)
    rc, gi = ora.dropout_backward(go, m, 0.2)
    s = np.float32(1.0 / (1.0 - float(np.float32(0.2))))
    assert rc == 0
    assert gi[0] == 0 and gi[4] == 0 and math.copysign(1, gi[0]) > 0
    assert gi[1] == np.float32(-2.0) * s and gi[2] == np.float32(3.0) * s and np.isnan(gi[3])
    assert gi[5] == np.float32(0.25) * s


def test_add_relu():
    a = np.array([1.0, -1.0, 0.5, -0.0, np.nan, 3.0, -2.0], np.float32)
    b = np.array([1.0, 0.5, -0.5, 0.0, 1.0, -np.inf, 2.0], np.float32)
    c = ora.add_relu(a, b)
    assert c.tolist()[:4] == [2.0, 0.0, 0.0, 0.0]
    assert c[4] == 0 and c[5] == 0 and c[6] == 0
    assert all(math.copysign(1, v) > 0 for v in c if v == 0)


@pytest.mark.parametrize("seed", [1, 0, 2024, 2 ** 31 + 5, 2 ** 32 - 1])
def test_jump_window_matches_rand(seed):
    for skip, n in [(0, 1000), (1, 64), (30, 70), (31, 31), (32, 5), (313, 100), (344, 100), (12345, 700)]:
        assert np.array_equal(ora.glibc_window(seed, skip, n), ora.glibc_rand(seed, n, skip=skip)), (seed, skip)
    # the C library itself, three million draws in
    k = 3_000_007
    ora.srand(seed)
    libc_draws = ora.rand_n(k + 500)
    assert np.array_equal(ora.glibc_window(seed, k, 500), libc_draws[k:])
    assert np.array_equal(ora.glibc_window(seed, 0, 500), libc_draws[:500])


def test_jump_window_composes():
    # x^(a+b) = x^a x^b: a window at a + b equals the window reached from the
    # stream at a, stepped b further -- checked at offsets past 2^32
    a, b = (1 << 32) + 12345, 999_983
    w = ora.glibc_window(77, a, b + 300)
    assert np.array_equal(ora.glibc_window(77, a + b, 300), w[b:])


def test_dropout_window_matches_forward():
    rng = np.random.default_rng(8)
    x = rng.normal(0, 1, 5000).astype(np.float32)
    ora.srand(31)
    ora.rand_n(123_456)
    rc, out, mask = ora.dropout_forward(x, 0.3)
    wout, wmask = ora.dropout_window(31, 123_456, x, 0.3)
    assert np.array_equal(mask, wmask)
    assert np.array_equal(out.view(np.uint32), wout.view(np.uint32))
