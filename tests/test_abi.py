"""CPU-side checks of the C ABI: the library loads, exports every function
include/neural_api.h declares, and the structs keep the reference layouts
(tensor.asm:7-24, quantize.c:39-45, neural_api.h:209-217).  No compute calls
(there is no GPU here)."""

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "neural_api.h"
LIB = ROOT / "neural-assembly_amd" / "libneural_hip.so"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"\b([A-Za-z_][A-Za-z0-9_]*)\s*\([^;{}]*\)\s*;", text)
    return sorted(set(n for n in names if n not in ("if", "sizeof")))


@pytest.fixture(scope="module")
def lib():
    if not LIB.exists():
        pytest.fail(f"{LIB} not built: run __graft_entry__.build()")
    return ctypes.CDLL(str(LIB))


def test_every_declared_symbol_is_exported(lib):
    names = declared_functions()
    assert len(names) > 100, names
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_struct_layouts():
    import sys
    sys.path.insert(0, str(ROOT / "neural-assembly_amd"))
    from pyneural.core import QuantParamsC, NeuralBufferInfo
    assert ctypes.sizeof(QuantParamsC) == 40
    assert [QuantParamsC.scale.offset, QuantParamsC.zero_point.offset, QuantParamsC.min_val.offset,
            QuantParamsC.max_val.offset, QuantParamsC.symmetric.offset] == [0, 8, 16, 24, 32]
    assert [NeuralBufferInfo.data.offset, NeuralBufferInfo.itemsize.offset, NeuralBufferInfo.ndim.offset,
            NeuralBufferInfo.shape.offset, NeuralBufferInfo.strides.offset, NeuralBufferInfo.readonly.offset,
            NeuralBufferInfo.format.offset] == [0, 8, 16, 24, 32, 40, 44]


def test_init_fails_loudly_without_gpu(lib):
    """On a machine without a GPU the runtime refuses to start (no CPU fallback)."""
    import subprocess
    import sys
    code = ("import ctypes,sys; l=ctypes.CDLL(sys.argv[1]); print(l.neural_init())")
    out = subprocess.run([sys.executable, "-c", code, str(LIB)], capture_output=True, text=True, timeout=120)
    rc = int(out.stdout.strip().splitlines()[-1])
    try:
        import torch
        has_gpu = torch.cuda.is_available()
    except Exception:
        has_gpu = False
    assert rc == (0 if has_gpu else 15)


def test_no_oracle_in_product():
    """The product sources never reference the oracle."""
    for p in list((ROOT / "neural-assembly_amd").rglob("*.py")) + list((ROOT / "neural-assembly_amd").rglob("*.hip")) \
            + list((ROOT / "neural-assembly_amd").rglob("*.hpp")):
        t = p.read_text()
        assert "liboracle" not in t and "import ora" not in t and "_ref/" not in t, p


def _bound():
    import json
    return json.loads((ROOT / "tests" / "golden" / "reference_bound_symbols.json").read_text())


def test_reference_loader_symbols_are_exported(lib):
    """Every name the reference's pyneural binds at import (core.py, tensor.py;
    list made by tests/golden/make_bound_symbols.py) resolves in this library."""
    names = _bound()
    assert len(names) == 215
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_out_of_scope_stubs(lib):
    """Entry points outside the hot path answer without touching a device:
    NOT_IMPLEMENTED / -1 / NULL / 0 / NaN, and NOT_IMPLEMENTED as last error."""
    import math
    ct = ctypes
    lib.neural_get_last_error.restype = ct.c_int

    def check(name, restype, argtypes, args, want):
        f = getattr(lib, name)
        f.restype, f.argtypes = restype, argtypes
        got = f(*args)
        if isinstance(want, float) and math.isnan(want):
            assert math.isnan(got), (name, got)
        else:
            assert got == want, (name, got)
        assert lib.neural_get_last_error() == 14, name

    check("neural_matmul", ct.c_int, [ct.c_void_p] * 3, [None] * 3, 14)
    check("neural_mse_loss", ct.c_int, [ct.c_void_p, ct.c_void_p, ct.POINTER(ct.c_double)], [None, None, None], 14)
    check("layernorm_forward", ct.c_int, [ct.c_void_p] * 3 + [ct.c_int64], [None, None, None, 4], -1)
    check("layernorm_create", ct.c_void_p, [ct.c_int64, ct.c_double], [4, 1e-5], None)
    check("neural_sgd_create", ct.c_void_p, [ct.c_double, ct.c_double], [0.1, 0.9], None)
    check("conv2d_output_size", ct.c_int64, [ct.c_int64] * 4, [32, 3, 1, 1], -1)
    check("neural_dataset_size", ct.c_uint64, [ct.c_void_p], [None], 0)
    check("compute_sparsity", ct.c_double, [ct.c_void_p, ct.c_int64], [None, 0], float("nan"))
    check("neural_lr_step_decay", ct.c_double, [ct.c_double, ct.c_int, ct.c_int, ct.c_double], [0.1, 3, 2, 0.5],
          float("nan"))
    check("tb_get_logdir", ct.c_char_p, [ct.c_int], [0], None)
    check("apply_mask", None, [ct.c_void_p, ct.c_void_p, ct.c_int64], [None, None, 0], None)
    # real entry points outside the hot path reject bad arguments before touching a device
    lib.calibrate_percentile.restype = ct.c_int
    lib.calibrate_percentile.argtypes = [ct.c_void_p, ct.c_int64, ct.c_double, ct.c_int, ct.c_void_p]
    assert lib.calibrate_percentile(None, 10, 0.01, 0, None) == -1
    lib.quantized_matmul.restype = ct.c_int
    lib.quantized_matmul.argtypes = [ct.c_void_p] * 3 + [ct.c_int64] * 3 + [ct.c_void_p] * 2
    assert lib.quantized_matmul(None, None, None, 1, 1, 1, None, None) == -1
    lib.layernorm_free.argtypes = [ct.c_void_p]
    lib.layernorm_free(None)
    lib.neural_get_simd_name.restype = ct.c_char_p
    assert b"HIP" in lib.neural_get_simd_name()
