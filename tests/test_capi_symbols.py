"""libmoehip.so loads and exports every function include/*.h declares, and the
Python binding's table covers them.  No compute calls: CPU only."""
import ctypes
import glob
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "moe.cc_amd", "libmoehip.so")


def declared_functions():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        text = re.sub(r"typedef\s+struct\s*\{.*?\}\s*\w+\s*;", "", text, flags=re.S)
        for m in re.finditer(r"\b([A-Za-z_]\w*)\s*\(([^;{}]*)\)\s*;", text):
            name = m.group(1)
            if name not in ("if", "while", "for", "sizeof", "return"):
                names.add(name)
    return sorted(names)


def test_header_parses():
    names = declared_functions()
    assert "matmul_adaptive" in names and "moe_init" in names


@pytest.mark.skipif(not os.path.exists(LIB), reason="libmoehip.so not built")
def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(LIB)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    assert set(declared_functions()) <= exported


@pytest.mark.skipif(not os.path.exists(LIB), reason="libmoehip.so not built")
def test_binding_covers_header():
    import moehip
    assert set(declared_functions()) <= set(moehip.exported_symbols())


def test_drop_in_signature_matches_reference_header():
    # kernels.h:16-17: void matmul_adaptive(const float*, const float*, const void*, float*, int, int, int)
    text = open(os.path.join(ROOT, "include", "moehip.h")).read()
    flat = " ".join(text.split())
    assert ("void matmul_adaptive(const float* A, const float* W_fp32, const void* W_q_ptr, "
            "float* C, int M, int N, int K);") in flat
