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


# ---- signatures of the reference's bindings --------------------------------------------------

def _ref_type(expr):
    """The ctypes object a reference binding string names (ctypes.c_uint64 and
    ctypes.c_ulong are one type on LP64, so aliases compare equal)."""
    import sys
    sys.path.insert(0, str(ROOT / "neural-assembly_amd"))
    from pyneural.core import QuantParamsC, NeuralBufferInfo
    if expr == "None":
        return None
    return eval(expr, {"ctypes": ctypes, "QuantParamsC": QuantParamsC, "NeuralBufferInfo": NeuralBufferInfo})


def test_python_bindings_match_reference_signatures():
    """Every entry point this package binds that the reference's pyneural also
    binds has the reference's restype and argtypes (pyneural/core.py:89-1373,
    tensor.py:40-59), so the reference's own ctypes declarations call this
    library with the same argument widths."""
    import sys
    sys.path.insert(0, str(ROOT / "neural-assembly_amd"))
    from pyneural.core import _SIGS
    ref = _bound()
    both = [n for n in _SIGS if n in ref]
    assert len(both) >= 70, len(both)
    bad = []
    for n in both:
        res, args = _SIGS[n]
        want_res = _ref_type(ref[n]["restype"])
        want_args = [_ref_type(a) for a in ref[n]["argtypes"]]
        if res is not want_res or list(args) != want_args:
            bad.append((n, (res, args), (want_res, want_args)))
    assert not bad, bad


_C_SCALARS = {
    "int": ctypes.c_int, "int32_t": ctypes.c_int32, "int64_t": ctypes.c_int64, "uint64_t": ctypes.c_uint64,
    "uint32_t": ctypes.c_uint32, "double": ctypes.c_double, "float": ctypes.c_float, "size_t": ctypes.c_size_t,
}


def _header_decls():
    """name -> (return type text, [parameter type texts]) for every function
    include/neural_api.h declares."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    text = re.sub(r"#[^\n]*", "", text)
    out = {}
    for m in re.finditer(r"([A-Za-z_][A-Za-z0-9_ \t\*]*?[\s\*])([A-Za-z_][A-Za-z0-9_]*)\s*\(([^;{}()]*)\)\s*;", text):
        ret, name, params = m.group(1), m.group(2), m.group(3).strip()
        ret = ret.split(";")[-1].split("}")[-1].strip()
        plist = [] if params in ("", "void") else [p.strip() for p in params.split(",")]
        types = []
        for p in plist:
            p = re.sub(r"\[\s*\]", "*", p)
            toks = re.findall(r"[A-Za-z_][A-Za-z0-9_]*|\*", p)
            # drop the parameter name (last identifier after the type)
            if len(toks) >= 2 and toks[-1] != "*" and toks[-2] not in ("const",):
                toks = toks[:-1]
            types.append(" ".join(toks))
        out[name] = (ret, types)
    return out


def _c_matches(ctext, want):
    """A C type from the header is ABI-compatible with a ctypes binding: equal
    scalar widths; pointers bind as c_void_p, c_char_p (char *) or
    POINTER(T) where T is the pointee."""
    # the multi-word spellings by their LP64 widths
    ctext = re.sub(r"\bunsigned\s+long\s+long\b", "uint64_t", ctext)
    ctext = re.sub(r"\blong\s+long\b", "int64_t", ctext)
    toks = [t for t in re.findall(r"[A-Za-z_][A-Za-z0-9_]*|\*", ctext) if t not in ("const", "struct", "unsigned")]
    npt = toks.count("*")
    base = [t for t in toks if t != "*"]
    base = base[0] if base else ""
    if npt == 0:
        if base == "void":
            return want is None
        return want is _C_SCALARS.get(base, object())
    if want is ctypes.c_void_p:
        return True
    if want is ctypes.c_char_p:
        return base == "char" and npt == 1
    if hasattr(want, "_type_") and getattr(want, "__name__", "").startswith("LP_"):
        inner = want._type_
        if npt == 2:
            return inner is ctypes.c_void_p
        if base == "QuantParams":
            return inner.__name__ == "QuantParamsC"
        if base == "NeuralBufferInfo":
            return inner.__name__ == "NeuralBufferInfo"
        return inner is _C_SCALARS.get(base, object())
    return False


def test_header_matches_reference_signatures():
    """Every declaration in include/neural_api.h of a name the reference's
    pyneural binds is ABI-compatible with that binding: same argument count,
    same scalar widths, pointers where the reference passes pointers."""
    decls = _header_decls()
    ref = _bound()
    both = [n for n in ref if n in decls]
    assert len(both) >= 70, len(both)
    bad = []
    for n in both:
        ret, params = decls[n]
        want_res = _ref_type(ref[n]["restype"])
        want_args = [_ref_type(a) for a in ref[n]["argtypes"]]
        ok = _c_matches(ret, want_res) and len(params) == len(want_args) and \
            all(_c_matches(p, w) for p, w in zip(params, want_args))
        if not ok:
            bad.append((n, ret, params, ref[n]["restype"], ref[n]["argtypes"]))
    assert not bad, bad


def test_noalloc_entry_refuses_before_init(lib):
    """calibrate_minmax_f32_dev_noalloc never initialises the library (that
    would allocate): in a process that has not called neural_init it returns
    -1 with NEURAL_ERR_INVALID_CONFIG, without touching a device."""
    import subprocess
    import sys
    code = ("import ctypes,sys; l=ctypes.CDLL(sys.argv[1]); f=l.calibrate_minmax_f32_dev_noalloc; "
            "f.argtypes=[ctypes.c_void_p,ctypes.c_int64,ctypes.c_int,ctypes.c_void_p]; "
            "x=(ctypes.c_float*8)(); p=(ctypes.c_double*5)(); "
            "print(f(ctypes.addressof(x),8,1,ctypes.addressof(p)), l.neural_get_last_error())")
    out = subprocess.run([sys.executable, "-c", code, str(LIB)], capture_output=True, text=True, timeout=120)
    assert out.stdout.split() == ["-1", "10"], (out.stdout, out.stderr)


def test_python_bindings_match_header():
    """Every binding in pyneural/core.py's table, the entry points without a
    reference counterpart included, is declared in include/neural_api.h and
    ABI-compatible with that declaration (argument count, scalar widths,
    pointers where the header has pointers)."""
    import sys
    sys.path.insert(0, str(ROOT / "neural-assembly_amd"))
    from pyneural.core import _SIGS
    decls = _header_decls()
    missing = [n for n in _SIGS if n not in decls]
    assert not missing, missing
    bad = []
    for n, (res, args) in _SIGS.items():
        ret, params = decls[n]
        ok = _c_matches(ret, res) and len(params) == len(args) and \
            all(_c_matches(p, a) for p, a in zip(params, args))
        if not ok:
            bad.append((n, ret, params, res, args))
    assert not bad, bad
