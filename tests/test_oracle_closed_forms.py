"""Pin the oracle's restatement of the asm kernels (which cannot be built here:
no nasm) to closed forms and brute force.

- ew_* / scalar / neg / relu / bias add: IEEE-754 correctly rounded numpy
  operations give the same bits (math_kernels.asm:66-945, activations.asm:
  153-171, nn_layers.asm:472-539).
- reduce_sum lane orders (math_kernels.asm:1124-1196) and the 4-lane L2 norm
  (training_ops.asm:646-690): a Python lane-by-lane emulation in float32 /
  float64 scalars, bit for bit, plus the classic sequential error bound
  against math.fsum.
- running max (activations.asm:888-895) and argmax (main.asm:3245-3292,
  3598-3640): brute force over all small arrays of a value pool including
  NaN and signed zeros.
- has_nan / has_inf: numpy isnan / isinf.
- softmax rows: fp64 closed form.
Each section also checks that a plausible mistake (dropped term, swapped
operand, wrong tie rule) would be caught.
"""

import itertools
import math

import numpy as np
import pytest

from conftest import same_bits, special_f32, special_f64


def test_unit_values_from_reference_tests(ora):
    """tests.asm:337-405,470-519."""
    three, two = np.full(8, 3, np.float32), np.full(8, 2, np.float32)
    assert ora.ew(ora.ADD, three, two)[0] == 5 and ora.ew(ora.SUB, three, two)[0] == 1
    assert ora.ew(ora.MUL, three, two)[0] == 6
    assert ora.relu(np.array([-1, 0, 1, 2], np.float32)).tolist() == [0, 0, 1, 2]


@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_elementwise_closed_forms(ora, rng, dt):
    gen = special_f32 if dt == np.float32 else special_f64
    a, b = gen(50021, rng, 0.05), gen(50021, rng, 0.05)
    with np.errstate(all="ignore"):
        same_bits(ora.ew(ora.ADD, a, b), a + b)
        same_bits(ora.ew(ora.SUB, a, b), a - b)
        same_bits(ora.ew(ora.MUL, a, b), a * b)
        same_bits(ora.ew(ora.DIV, a, b), a / b)
        same_bits(ora.ew(ora.MAX, a, b), np.where(a > b, a, b))
        for s in (0.1, -2.5, 1e-30):
            sc = dt(s)
            same_bits(ora.scalar(0, a, s), a + sc)
            same_bits(ora.scalar(2, a, s), a * sc)
    u = np.uint32 if dt == np.float32 else np.uint64
    sign = u(1) << u(31 if dt == np.float32 else 63)
    same_bits(ora.neg(a).view(u), a.view(u) ^ sign)
    same_bits(ora.relu(a), np.where(a > 0, a, dt(0)))
    # a max that takes the first operand on ties would differ on signed zeros
    z = np.array([0.0, -0.0], dtype=dt)
    assert np.signbit(ora.ew(ora.MAX, z[::-1].copy(), z)[0]) == False  # noqa: E712  (max(-0, +0) -> +0)
    assert np.signbit(ora.ew(ora.MAX, z, z[::-1].copy())[0])            # max(+0, -0) -> -0 (second operand)


@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_bias_add_closed_form(ora, rng, dt):
    """out[i,j] = x[i,j] + b[j] correctly rounded (addss / addsd,
    nn_layers.asm:472-539): numpy's broadcast add in the same dtype, with
    NaN, +-Inf, signed zeros and a row/column transposition planted so a
    swapped index or a dropped row stride fails."""
    x = rng.normal(0, 3, (33, 77)).astype(dt)
    b = rng.normal(0, 3, 77).astype(dt)
    x[0, :4] = [np.nan, np.inf, -0.0, 0.0]
    b[:4] = [1.0, -np.inf, -0.0, -0.0]
    got = ora.bias_add(x, b)
    same_bits(got, x + b)
    assert np.signbit(got[0, 2]) and not np.signbit(got[0, 3])  # -0 + -0 = -0, +0 + -0 = +0
    assert np.isnan(got[0, 1])                                   # inf + -inf
    assert not np.array_equal(got[1:], (x + b[::-1])[1:])
    sq = rng.normal(size=(40, 40)).astype(dt)
    bq = rng.normal(size=40).astype(dt)
    assert not np.array_equal(ora.bias_add(sq, bq), sq + bq[:, None])  # broadcast over rows, not columns


def _emulate_sum_f32(x):
    l = [np.float32(0)] * 8
    nv = len(x) // 8
    for i in range(nv):
        for k in range(8):
            l[k] = np.float32(l[k] + x[i * 8 + k])
    acc = np.float32(0)
    if nv:
        s = [np.float32(l[k] + l[k + 4]) for k in range(4)]
        acc = np.float32(np.float32(s[0] + s[1]) + np.float32(s[2] + s[3]))
    for i in range(nv * 8, len(x)):
        acc = np.float32(acc + x[i])
    return acc


def _emulate_sum_f64(x):
    l = [0.0] * 4
    nv = len(x) // 4
    for i in range(nv):
        for k in range(4):
            l[k] = l[k] + float(x[i * 4 + k])
    acc = (l[0] + l[2]) + (l[1] + l[3]) if nv else 0.0
    for i in range(nv * 4, len(x)):
        acc = acc + float(x[i])
    return acc


def _emulate_l2(x):
    l = [np.float32(0)] * 4
    nv = len(x) // 4
    for i in range(nv):
        for k in range(4):
            l[k] = np.float32(l[k] + np.float32(x[i * 4 + k] * x[i * 4 + k]))
    s = np.float32(np.float32(l[0] + l[2]) + np.float32(l[1] + l[3])) if nv else np.float32(0)
    for i in range(nv * 4, len(x)):
        s = np.float32(s + np.float32(x[i] * x[i]))
    return np.sqrt(s, dtype=np.float32)


@pytest.mark.parametrize("n", [0, 1, 5, 7, 8, 9, 15, 16, 17, 100, 1001])
def test_lane_orders(ora, n):
    rng = np.random.default_rng(n)
    x = rng.uniform(-1, 1, n).astype(np.float32)
    assert np.float32(ora.sum_ref(x)).tobytes() == _emulate_sum_f32(x).tobytes()
    y = rng.normal(size=n)
    assert ora.sum_ref(y) == _emulate_sum_f64(y)
    g = (rng.normal(size=n) * 1e-3).astype(np.float32)
    assert np.float32(ora.l2_ref(g)).tobytes() == _emulate_l2(g).tobytes()
    if n:
        e = math.fsum(x.astype(np.float64))
        assert abs(ora.sum_ref(x) - e) <= n * 6e-8 * float(np.sum(np.abs(x))) + 1e-30
        assert abs(ora.sum_exact(x) - e) <= 1e-15 * abs(e) + 1e-300
        assert abs(ora.sum_exact(y) - math.fsum(y)) <= 2e-16 * abs(math.fsum(y)) + 1e-300
        assert abs(ora.sumsq_exact(g) - math.fsum(g.astype(np.float64) ** 2)) <= 1e-15 * math.fsum(g.astype(np.float64) ** 2)
    if n >= 16:  # a sequential sum would not reproduce the lane order
        seq = np.float32(0)
        for v in x:
            seq = np.float32(seq + v)
        x2 = np.float32(_emulate_sum_f32(x))
        assert x2 == np.float32(ora.sum_ref(x))


def test_row_and_column_orders(ora, rng):
    x = rng.uniform(-1, 1, (6, 13)).astype(np.float32)
    rs = ora.rowsum_ref(x)
    for i in range(6):
        acc = np.float32(0)
        for v in x[i]:
            acc = np.float32(acc + v)
        assert rs[i] == acc
    cs = ora.colsum_ref(x)
    for j in range(13):
        acc = np.float32(0)
        for i in range(6):
            acc = np.float32(x[i, j] + acc)
        assert cs[j] == acc
    e = ora.rowsum_exact(x)
    for i in range(6):
        assert e[i] == math.fsum(x[i].astype(np.float64)) or abs(e[i] - math.fsum(x[i])) < 1e-15


POOL = [np.nan, -0.0, 0.0, 1.0, -1.0, 2.0]


def _chain(xs):
    m = xs[0]
    for v in xs[1:]:
        m = m if m > v else v
    return m


def _argmax(xs):
    idx, m = 0, xs[0]
    for j in range(1, len(xs)):
        if xs[j] > m:
            idx, m = j, xs[j]
    return idx


@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_max_argmax_brute_force(ora, dt):
    """Every array of length 1..4 over a pool with NaN and signed zeros, in
    both dtypes: the f32 chain is activations.asm:888-895 (maxss) and
    main.asm:3598-3640 (comiss), the f64 chain activations.asm:815-823
    (maxsd) and the same argmax rule on doubles."""
    pool = np.array(POOL, dtype=dt)
    for n in range(1, 5):
        for combo in itertools.product(range(len(pool)), repeat=n):
            x = pool[list(combo)].copy()
            want = dt(_chain(list(x)))
            got = dt(ora.max_chain(x))
            assert (np.isnan(want) and np.isnan(got)) or got.tobytes() == want.tobytes(), x
            assert ora.argmax(x) == _argmax(list(x)), x
            # closed form used by the GPU reduction: after the last NaN,
            # rightmost maximum; NaN if the array ends with NaN
            nan_idx = [i for i in range(n) if np.isnan(x[i])]
            L = nan_idx[-1] if nan_idx else -1
            if L == n - 1:
                assert np.isnan(got)
            else:
                seg = x[L + 1:]
                best = max(range(len(seg)), key=lambda i: (seg[i], i))
                assert got.tobytes() == seg[best].tobytes()
            # argmax closed form: 0 if x0 is NaN, else first index of the max non-NaN value
            if np.isnan(x[0]):
                assert ora.argmax(x) == 0
            else:
                vals = [(v, -i) for i, v in enumerate(x) if not np.isnan(v)]
                assert ora.argmax(x) == -max(vals)[1]


@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_rowwise_matches_flat(ora, rng, dt):
    x = rng.normal(size=(9, 31)).astype(dt)
    x[2, 4] = np.nan
    x[5, 0] = np.nan
    x[6, :] = 0.0
    x[6, 3] = -0.0
    rm, ra = ora.rowmax_chain(x), ora.rowargmax(x)
    for i in range(9):
        assert dt(ora.max_chain(x[i].copy())).tobytes() == rm[i].tobytes()
        assert ora.argmax(x[i].copy()) == ra[i]


def test_scans(ora, rng):
    x = rng.normal(size=1000).astype(np.float32)
    assert ora.has_nan(x) == 0 and ora.has_inf(x) == 0
    for v, nan, inf in ((np.nan, 1, 0), (np.inf, 0, 1), (-np.inf, 0, 1), (3.4e38, 0, 0)):
        y = x.copy()
        y[777] = v
        assert (ora.has_nan(y), ora.has_inf(y)) == (nan, inf) == (int(np.isnan(y).any()), int(np.isinf(y).any()))


@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_softmax_closed_form(ora, rng, dt):
    x = rng.normal(0, 3, (50, 300)).astype(dt)
    x64 = x.astype(np.float64)
    e = np.exp(x64 - x64.max(axis=1, keepdims=True))
    want = e / e.sum(axis=1, keepdims=True)
    lwant = (x64 - x64.max(axis=1, keepdims=True)) - np.log(e.sum(axis=1, keepdims=True))
    tol = 1e-5 if dt == np.float32 else 1e-13
    assert np.max(np.abs(ora.softmax_rows(x) - want) / want) < tol
    assert np.max(np.abs(ora.softmax_rows(x, True) - lwant) / np.abs(lwant)) < tol
    # the intended f32 softmax normalises by the sum (the asm's slot-aliasing
    # bug would divide by the max): rows must sum to 1
    assert np.allclose(ora.softmax_rows(x).sum(axis=1), 1.0, rtol=1e-5)
