"""Randomised raw-pointer float32 kernels (simd.asm:190-784).

Seeded cases: 1 to 4 M values (log-uniform), every pointer starting 0-3
floats past a 16-byte boundary on its own, host buffers or device buffers,
values with exponents spread over 2^-40..2^40 (products and sums reach the
subnormal range and round in every way), NaN / +-Inf planted in some cases,
and in some cases triples whose exact a*b + c lies just past a float tie.
simd_add / simd_mul must equal numpy's IEEE float32 results bit for bit,
simd_fma the correctly rounded fma (one rounding of the exact a*b + c);
simd_dot / simd_sum within REDUCE (1e-5 * sum|terms|) of the fp64-exact
value, non-finite results by class.
"""

import math

import numpy as np

from conftest import GPU, fmaf_exact, same_bits

pytestmark = GPU

CASES = 40


def _vals(rng, n, specials):
    x = (rng.uniform(-2, 2, n) * 2.0 ** rng.integers(-40, 41, n)).astype(np.float32)
    if specials and n > 3:
        x[rng.integers(0, n, 3)] = rng.choice(np.array([np.nan, np.inf, -np.inf], dtype=np.float32), 3)
    return x


def _place(torch, x, off, dev):
    """(pointer, holder, view) of x's values starting `off` floats into a buffer."""
    if dev:
        t = torch.zeros(x.size + 4, dtype=torch.float32, device="cuda")
        t[off:off + x.size] = torch.from_numpy(x).cuda()
        return t.data_ptr() + 4 * off, t
    buf = np.zeros(x.size + 4, dtype=np.float32)
    buf[off:off + x.size] = x
    return buf.ctypes.data + 4 * off, buf


def _read(h, off, n):
    return (h.cpu().numpy() if hasattr(h, "cpu") else h)[off:off + n].copy()


def _reduce_ok(got, terms):
    t = terms.astype(np.float64)
    if not np.all(np.isfinite(t)):
        e = float(np.sum(t))  # NaN, or the infinity (or NaN for both signs), in any order
        assert (math.isnan(got) and math.isnan(e)) or got == e, (got, e)
        return
    e = math.fsum(t.tolist())
    assert abs(got - e) <= 1e-5 * float(np.sum(np.abs(t))) + 1e-37, (got, e)


def test_random_simd_kernels(pn):
    import torch
    lib = pn.core._lib
    rng = np.random.default_rng(1717)
    for case in range(CASES):
        n = int(np.exp(rng.uniform(0, np.log(4_000_000))))
        dev = rng.random() < 0.5
        specials = rng.random() < 0.3
        a, b, c = (_vals(rng, n, specials) for _ in range(3))
        if rng.random() < 0.3:  # exact a*b on a float tie, c far below it
            k = max(1, n // 100)
            i = rng.integers(0, n, k)
            u = np.float32(1 + 2.0 ** -12)
            a[i], b[i] = u, u * np.float32(rng.choice([1, -1]))
            c[i] = np.float32(2.0 ** -80) * rng.choice(np.array([1, -1], dtype=np.float32), k)
        offs = rng.integers(0, 4, 4)
        pa, ha = _place(torch, a, int(offs[0]), dev)
        pb, hb = _place(torch, b, int(offs[1]), dev)
        pc, hc = _place(torch, c, int(offs[2]), dev)
        po, ho = _place(torch, np.zeros(n, dtype=np.float32), int(offs[3]), dev)
        torch.cuda.synchronize()
        what = (case, n, dev, tuple(int(o) for o in offs))
        with np.errstate(all="ignore"):
            assert lib.simd_add_f32(po, pa, pb, n) == 0, what
            pn.synchronize()
            same_bits(_read(ho, int(offs[3]), n), a + b)
            assert lib.simd_mul_f32(po, pa, pb, n) == 0, what
            pn.synchronize()
            same_bits(_read(ho, int(offs[3]), n), a * b)
            assert lib.simd_fma_f32(po, pa, pb, pc, n) == 0, what
            pn.synchronize()
            same_bits(_read(ho, int(offs[3]), n), fmaf_exact(a, b, c))
            _reduce_ok(lib.simd_dot_f32(pa, pb, n), a.astype(np.float64) * b.astype(np.float64))
            _reduce_ok(lib.simd_sum_f32(pa, n), a)
