"""The package has no CPU fallback: without libneural_hip.so, importing
pyneural raises ImportError naming the library (nothing routes through the
oracle or any host implementation instead)."""

import os
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def test_missing_library_fails_loudly(tmp_path):
    env = dict(os.environ)
    env["NEURAL_HIP_LIB"] = str(tmp_path / "libneural_hip.so")  # does not exist
    env["PYTHONPATH"] = str(ROOT / "neural-assembly_amd")
    code = "import pyneural"
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=120)
    assert r.returncode != 0
    assert "ImportError" in r.stderr and "libneural_hip.so" in r.stderr, r.stderr[-2000:]


def test_package_does_not_import_the_oracle():
    """No module of the package names the oracle or its libraries."""
    for p in (ROOT / "neural-assembly_amd" / "pyneural").glob("*.py"):
        text = p.read_text()
        for word in ("import ora", "from ora", "liboracle", "libcpu_baseline", "neural_ref"):
            assert word not in text, (p.name, word)
