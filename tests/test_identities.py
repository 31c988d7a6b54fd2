"""Exhaustive CPU checks of arithmetic identities that the device kernels rely
on where they evaluate the reference's expression in a cheaper but
bit-identical form.  tests/identities.c restates both forms in C and is built
here with gcc (-O2 -std=c11 as the reference's Makefile:12, plus
-ffp-contract=off)."""

import ctypes
import math
import subprocess
import threading
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent


@pytest.fixture(scope="module")
def ident(tmp_path_factory):
    so = tmp_path_factory.mktemp("ident") / "libidentities.so"
    subprocess.run(["gcc", "-O2", "-std=c11", "-ffp-contract=off", "-fPIC", "-shared", "-o", str(so),
                    str(HERE / "identities.c"), "-lm"], check=True)
    lib = ctypes.CDLL(str(so))
    lib.hardswish_f32_mismatches.restype = ctypes.c_int64
    lib.hardswish_f32_mismatches.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_double,
                                             ctypes.POINTER(ctypes.c_uint32)]
    lib.hardswish_f32_mismatches_planted.restype = ctypes.c_int64
    lib.hardswish_f32_mismatches_planted.argtypes = [ctypes.c_uint64, ctypes.c_uint64]
    return lib


def _sweep(fn, lo, hi, parts=16):
    """fn(a, b) over [lo, hi) cut into parts, run on threads (ctypes releases the GIL)."""
    step = -(-(hi - lo) // parts)
    spans = [(a, min(hi, a + step)) for a in range(lo, hi, step)]
    out = [None] * len(spans)

    def work(i):
        out[i] = fn(*spans[i])

    threads = [threading.Thread(target=work, args=(i,)) for i in range(len(spans))]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    return out


def test_hardswish_f32_product_form_every_float(ident):
    """HardswishF32Fn (activations.hip) divides by 6 as a product with RN(1/6);
    after the rounding to float it equals the reference's
    (float)(x * (x + 3.0) / 6.0) (activations_c.c:154, 71-77) for all 2^32
    float inputs, signed zeros, denormals, +-3 and NaN included."""
    def count(a, b):
        first = ctypes.c_uint32(0)
        return ident.hardswish_f32_mismatches(a, b, 1.0 / 6.0, ctypes.byref(first)), first.value

    res = _sweep(count, 0, 1 << 32)
    bad = [hex(f) for n, f in res if n]
    assert sum(n for n, _ in res) == 0, f"first mismatching inputs (bits): {bad}"


def test_hardswish_check_catches_planted_mistakes(ident):
    """The same sweep flags a constant one ulp above RN(1/6) (on the positive
    denormals) and the formula evaluated in float arithmetic (on [-1.5, -1))."""
    first = ctypes.c_uint32(0)
    assert ident.hardswish_f32_mismatches(0, 1 << 23, math.nextafter(1.0 / 6.0, 1.0), ctypes.byref(first)) > 1000
    assert sum(_sweep(ident.hardswish_f32_mismatches_planted, 0xBF800000, 0xBFC00000)) > 1000
