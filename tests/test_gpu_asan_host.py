"""The library's host code under AddressSanitizer and UndefinedBehaviorSanitizer.

`tests/asan/host_checks` (built by `__graft_entry__.build()`) links
libneural_hip_asan.so, the same sources with the host side instrumented for
both (the GPU code is built as usual), and walks the C ABI through the paths whose host
code handles caller memory: descriptors, shapes and byte strides, host
mirrors and raw pointers into them, staged host buffers, the optimizer state
blob (corrupt blobs included), gradient-list tables, the dropout stream
state, the measurement hooks and error returns.  It runs as a child process
with leak detection on (the ROCm runtime's own allocations held until exit
are suppressed, `asan/lsan.supp`); any sanitizer report (an undefined
behaviour's "runtime error" included) or failed check fails the test.
"""

import os
import subprocess
from pathlib import Path

from conftest import GPU

pytestmark = GPU

EXE = Path(__file__).resolve().parent / "asan" / "host_checks"


def test_host_code_under_asan():
    assert EXE.exists(), f"{EXE} is not built (run __graft_entry__.build())"
    env = dict(os.environ)
    env["ASAN_OPTIONS"] = "detect_leaks=1:halt_on_error=1:abort_on_error=0:verify_asan_link_order=0"
    env["LSAN_OPTIONS"] = f"suppressions={EXE.parent / 'lsan.supp'}:print_suppressions=0"
    env["UBSAN_OPTIONS"] = "print_stacktrace=1:halt_on_error=1"
    r = subprocess.run([str(EXE)], capture_output=True, text=True, timeout=300, env=env)
    out = r.stdout + r.stderr
    print(out[-4000:])
    assert "AddressSanitizer" not in out and "runtime error" not in out, out[-8000:]
    assert r.returncode == 0, out[-8000:]
    assert "host checks:" in out and ", 0 failed" in out
