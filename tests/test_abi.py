"""The C-ABI boundary without a GPU: the library loads, exports exactly what the
headers declare, and the host-side entry points reject bad input before touching
a device.  No compute call is made here."""
import ctypes as C
import os
import re
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "jieyu_amd", "libjieyu_amd.so")


def declared(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    names = re.findall(r"\b((?:jyhip|jysyn)_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


def exported():
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True, check=True).stdout
    return {ln.split()[-1] for ln in out.splitlines() if ln.split()[-2] in ("T", "W")}


@pytest.fixture(scope="module")
def syms():
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} missing: run __graft_entry__.build()")
    return exported()


@pytest.mark.parametrize("header", ["jieyu_amd.h", "jieyu_synth.h"])
def test_header_symbols_exported(syms, header):
    names = declared(header)
    assert names, header
    missing = [n for n in names if n not in syms]
    assert not missing, f"declared in include/{header} but not exported: {missing}"


def test_no_undeclared_exports(syms):
    ours = {s for s in syms if s.startswith(("jyhip_", "jysyn_"))}
    decl = set(declared("jieyu_amd.h")) | set(declared("jieyu_synth.h"))
    assert ours <= decl, f"exported but not declared: {sorted(ours - decl)}"
    # C++ internals stay hidden
    assert not any(s.startswith("_ZN2jy") for s in syms)


def test_library_loads_and_binds():
    import jieyu_amd
    lib = jieyu_amd.lib()
    for name in declared("jieyu_amd.h"):
        assert getattr(lib, name) is not None
    assert isinstance(lib.jyhip_last_error(), (bytes, type(None)))


def test_package_fails_loudly_without_library(tmp_path):
    """With the shared library absent the package raises instead of falling back to a CPU path."""
    code = ("import sys, os; sys.path.insert(0, %r); import jieyu_amd; "
            "jieyu_amd.LIB_PATH = os.path.join(%r, 'nope.so'); jieyu_amd._lib = None\n"
            "try:\n    jieyu_amd.lib()\nexcept ImportError as e:\n    print('raised', e)\n") % (ROOT, str(tmp_path))
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert "raised" in r.stdout, r.stdout + r.stderr


def test_bench_refuses_several_gpus():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=300)
    assert r.returncode != 0
    assert "one GPU" in r.stderr or "--gpus 1" in r.stderr
