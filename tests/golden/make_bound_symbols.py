"""Writes reference_bound_symbols.json: every C symbol the reference's Python
layer binds through ctypes at import (pyneural/core.py, pyneural/tensor.py),
with the declared restype / argtypes and the line of the binding.  Run in a
container that holds the reference checkout (the text is parsed; nothing is
imported or executed):

    python tests/golden/make_bound_symbols.py /root/reference
"""

import json
import re
import sys
from pathlib import Path


def parse(ref: Path) -> dict:
    out = {}
    for rel in ("pyneural/core.py", "pyneural/tensor.py"):
        text = (ref / rel).read_text()
        for m in re.finditer(r"_lib\.([A-Za-z_][A-Za-z0-9_]*)\.(restype|argtypes)\s*=\s*", text):
            name, what = m.group(1), m.group(2)
            line = text.count("\n", 0, m.start()) + 1
            ent = out.setdefault(name, {"file": rel, "line": line})
            rest = text[m.end():]
            if what == "restype":
                ent["restype"] = rest.split("\n", 1)[0].strip()
            else:
                depth, i = 0, 0
                while True:  # the bracketed list, comments dropped
                    c = rest[i]
                    depth += c == "["
                    depth -= c == "]"
                    i += 1
                    if depth == 0:
                        break
                body = re.sub(r"#[^\n]*", "", rest[:i])
                ent["argtypes"] = [a.strip() for a in body.strip()[1:-1].split(",") if a.strip()]
        for m in re.finditer(r"_lib\.([A-Za-z_][A-Za-z0-9_]*)\b", text):
            out.setdefault(m.group(1), {"file": rel, "line": text.count("\n", 0, m.start()) + 1})
    return out


if __name__ == "__main__":
    ref = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    syms = parse(ref)
    dst = Path(__file__).with_name("reference_bound_symbols.json")
    dst.write_text(json.dumps(dict(sorted(syms.items())), indent=1) + "\n")
    print(len(syms), "symbols ->", dst)
