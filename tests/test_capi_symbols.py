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


def _undefined_and_needed(binary):
    nm = subprocess.run(["nm", "-D", binary], capture_output=True, text=True, check=True).stdout
    undef = {l.split()[-1] for l in nm.splitlines() if l.split()[0] == "U"}
    defined = {l.split()[-1] for l in nm.splitlines() if len(l.split()) == 3}
    rd = subprocess.run(["readelf", "-d", binary], capture_output=True, text=True, check=True).stdout
    needed = set(re.findall(r"Shared library: \[([^\]]+)\]", rd))
    return undef, defined, needed


@pytest.mark.skipif(not os.path.exists(LIB), reason="libmoehip.so not built")
def test_c_caller_compiles_and_links():
    """tests/c_caller/moe_caller.c, plain C99 with gcc against
    include/moehip.h: builds and resolves the library's symbols from
    libmoehip.so (it is run by the GPU test test_gpu_c_caller.py)."""
    d = os.path.join(ROOT, "tests", "c_caller")
    subprocess.run(["make", "-B", "-C", d], check=True, capture_output=True)
    undef, defined, needed = _undefined_and_needed(os.path.join(d, "moe_caller"))
    assert "libmoehip.so" in needed
    assert {"matmul_adaptive", "moe_layer_create", "moe_layer_forward"} <= undef


@pytest.mark.skipif(not (os.path.exists(LIB) and os.path.isdir("/root/reference")),
                    reason="needs libmoehip.so and the reference tree (build container only)")
def test_reference_links_against_library():
    """INTEGRATION.md's relink: the reference's own test_model_trace.o, io.o
    and utils.o (Makefile:9-10 without kernels.o) link against libmoehip.so,
    which supplies matmul_adaptive.  Built out of tree into oracle/_ref,
    never run."""
    subprocess.run(["make", "-B", "-C", os.path.join(ROOT, "oracle"), "ref-link"], check=True,
                   capture_output=True)
    exe = os.path.join(ROOT, "oracle", "_ref", "test_model_trace_moehip")
    undef, defined, needed = _undefined_and_needed(exe)
    assert "libmoehip.so" in needed
    assert "matmul_adaptive" in undef and "matmul_adaptive" not in defined
