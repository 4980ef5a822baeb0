"""Build the oracle's native parts (TEST INFRASTRUCTURE).

1. oracle/oc_port.c -> oracle/_build/liboc_port.so (gcc, OpenMP): the C
   restatement used as the CPU baseline and as a second checker.
2. When the reference tree is present (in the build container only), the
   reference's own C++ CPU attention - the XLA custom call embedded as a
   source string in notebooks/phase_d_kaggle.py:184-294 - is compiled into
   oracle/_ref/libref_custom_call.so.  The source is read from the
   reference and compiled from a temporary file outside the repository; only
   the shared object is kept.  It checks the oracle's attention semantics
   against the reference's own code.
"""

from __future__ import annotations

import os
import re
import subprocess
import sys
import tempfile
from pathlib import Path

HERE = Path(__file__).resolve().parent
BUILD = HERE / "_build"
REF_OUT = HERE / "_ref"
PORT_LIB = BUILD / "liboc_port.so"
REF_LIB = REF_OUT / "libref_custom_call.so"
REFERENCE = Path(os.environ.get("OC_REFERENCE", "/root/reference"))
REF_NOTEBOOK = REFERENCE / "notebooks" / "phase_d_kaggle.py"


def build_port() -> Path:
    BUILD.mkdir(exist_ok=True)
    tmp = PORT_LIB.with_suffix(".so.tmp")
    cmd = ["gcc", "-O3", "-march=x86-64-v3", "-fopenmp", "-fPIC", "-shared", str(HERE / "oc_port.c"),
           "-o", str(tmp), "-lm"]
    subprocess.run(cmd, check=True)
    os.replace(tmp, PORT_LIB)
    return PORT_LIB


def build_ref() -> Path | None:
    if not REF_NOTEBOOK.exists():
        return None
    text = REF_NOTEBOOK.read_text()
    m = re.search(r"custom_call_src\s*=\s*r'''(.*?)'''", text, re.S)
    if not m:
        print("oracle/build: reference custom call source not found; skipping _ref", file=sys.stderr)
        return None
    REF_OUT.mkdir(exist_ok=True)
    with tempfile.TemporaryDirectory() as td:
        src = Path(td) / "ref_custom_call.cc"
        src.write_text(m.group(1))
        tmp = REF_LIB.with_suffix(".so.tmp")
        # The reference's own recipe is g++ -shared -fPIC -O3 -march=native
        # (phase_d_kaggle.py:303); -march is left at the default here so the
        # object runs on any x86-64 host.
        subprocess.run(["g++", "-O3", "-shared", "-fPIC", str(src), "-o", str(tmp)], check=True)
        os.replace(tmp, REF_LIB)
    return REF_LIB


def build() -> None:
    p = build_port()
    r = build_ref()
    print(f"oracle/build: {p}" + (f", {r}" if r else " (reference not present: _ref not rebuilt)"), file=sys.stderr)


if __name__ == "__main__":
    build()
