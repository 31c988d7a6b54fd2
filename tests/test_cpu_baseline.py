"""The CPU-baseline loops (oracle/cpu_baseline.c: the reference's AVX-256,
AVX-512 and SSE paths restated with intrinsics) compute what the pinned oracle
computes, bit for bit, so the baseline bench.py times is the reference's
arithmetic and not a faster shortcut: ew add / mul against IEEE closed forms,
the 8-lane and 16-lane sums against a lane-by-lane emulation of their fold
orders, the 4-lane SSE L2 norm against ora_l2_ref_f32, and the node_relu
pass structure against the maxss rule (NaN and -0 give +0)."""

import numpy as np
import pytest

from conftest import same_bits


@pytest.fixture(scope="module")
def cpu(ora):
    return ora.cpu()


def _emulate_lanes(x, lanes):
    """Sequential float32 lane sums, folded 16 -> 8 (if 16 lanes), then
    (l_k + l_{k+4}), two horizontal adds, then the scalar tail."""
    nv = x.size // lanes
    l = np.zeros(lanes, dtype=np.float32)
    for i in range(nv):
        l = (l + x[i * lanes:(i + 1) * lanes]).astype(np.float32)
    acc = np.float32(0)
    if nv:
        if lanes == 16:
            l = (l[:8] + l[8:]).astype(np.float32)
        a = (l[:4] + l[4:8]).astype(np.float32)
        h1 = [np.float32(a[0] + a[1]), np.float32(a[2] + a[3])]
        acc = np.float32(h1[0] + h1[1])
    for v in x[nv * lanes:]:
        acc = np.float32(acc + v)
    return acc


@pytest.mark.parametrize("n", [0, 1, 7, 8, 15, 16, 17, 1000, 4099])
def test_avx256_loops(ora, cpu, rng, n):
    if not cpu.cpu_has_avx():
        pytest.skip("host has no AVX")
    a = rng.uniform(-1, 1, n).astype(np.float32)
    b = rng.uniform(-1, 1, n).astype(np.float32)
    same_bits(ora.cpu_binary("cpu_ew_add_avx", a, b), a + b)
    same_bits(ora.cpu_binary("cpu_ew_mul_avx", a, b), a * b)
    got = np.float32(ora.cpu_sum("cpu_reduce_sum_avx", a))
    assert got.tobytes() == _emulate_lanes(a, 8).tobytes()
    if n:
        assert got.tobytes() == np.float32(ora.sum_ref(a)).tobytes()


@pytest.mark.parametrize("n", [0, 1, 15, 16, 17, 33, 4099])
def test_avx512_loops(ora, cpu, rng, n):
    if not cpu.cpu_has_avx512f():
        pytest.skip("host has no AVX-512F")
    a = rng.uniform(-1, 1, n).astype(np.float32)
    b = rng.uniform(-1, 1, n).astype(np.float32)
    same_bits(ora.cpu_binary("cpu_simd_add_avx512", a, b), a + b)
    same_bits(ora.cpu_binary("cpu_simd_mul_avx512", a, b), a * b)
    got = np.float32(ora.cpu_sum("cpu_simd_sum_avx512", a))
    assert got.tobytes() == _emulate_lanes(a, 16).tobytes()


@pytest.mark.parametrize("n", [1, 3, 4, 5, 1001, 65536 + 3])
def test_sse_l2_and_relu(ora, cpu, rng, n):
    g = rng.normal(0, 1e-3, n).astype(np.float32)
    assert np.float32(ora.cpu_l2(g)).tobytes() == np.float32(ora.l2_ref(g)).tobytes()
    x = rng.normal(size=n).astype(np.float32)
    x[:3] = [np.nan, -0.0, -1.0][: min(3, n)]
    got = ora.cpu_relu_node(x)
    same_bits(got, ora.relu(x))
    assert not np.signbit(got[: min(3, n)]).any()
