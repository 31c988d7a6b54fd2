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
