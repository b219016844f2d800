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
    names = re.findall(r"\b((?:jyhip|jysyn|jytext|jieyu)_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


def exported():
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True, check=True).stdout
    return {ln.split()[-1] for ln in out.splitlines() if ln.split()[-2] in ("T", "W")}


@pytest.fixture(scope="module")
def syms():
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} missing: run __graft_entry__.build()")
    return exported()


HEADERS = ["jieyu_amd.h", "jieyu_synth.h", "jieyu_api.h", "jieyu_text.h"]


@pytest.mark.parametrize("header", HEADERS)
def test_header_symbols_exported(syms, header):
    names = declared(header)
    assert names, header
    missing = [n for n in names if n not in syms]
    assert not missing, f"declared in include/{header} but not exported: {missing}"


def test_no_undeclared_exports(syms):
    ours = {s for s in syms if s.startswith(("jyhip_", "jysyn_", "jytext_", "jieyu_"))}
    decl = set().union(*(declared(h) for h in HEADERS))
    assert ours <= decl, f"exported but not declared: {sorted(ours - decl)}"
    # C++ internals stay hidden
    assert not any(s.startswith(("_ZN2jy", "_ZN6jytext")) for s in syms)


def test_text_abi_matches_reference_header():
    """the eight entry points of JieyuAI_api.h:47-67, and the public handle layout
    {char dir[512]; char error[256]; int max_seq} (JieyuAI_api.h:42-46)"""
    assert declared("jieyu_api.h") == sorted(
        ["jieyu_load", "jieyu_free", "jieyu_last_error", "jieyu_version", "jieyu_context_length",
         "jieyu_model_dir", "jieyu_generate", "jieyu_generate_jsonl"])
    text = open(os.path.join(ROOT, "include", "jieyu_api.h")).read()
    assert re.search(r"char dir\[JIEYU_PATH_MAX\];\s*/\*[^*]*\*/\s*char error\[JIEYU_ERR_MAX\];"
                     r"\s*/\*[^*]*\*/\s*int max_seq;", text)
    assert "#define JIEYU_PATH_MAX 512" in text and "#define JIEYU_ERR_MAX 256" in text


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


def test_bench_kv_packing_matches_oracle(oracle_lib):
    """bench.py fills the long-context cache with rows packed like the cache's own: the
    oracle's packing of attention_q8.h:20-37 (absmax int8 per position and head)."""
    import importlib.util
    import ctypes as C
    import numpy as np
    from conftest import ptr
    spec = importlib.util.spec_from_file_location("bench_mod", os.path.join(ROOT, "bench.py"))
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    x = np.random.default_rng(7).standard_normal((50, 4, 128)).astype(np.float32)
    x[3, 1] = 0.0          # an all-zero row: scale 0, codes 0
    x[4, 2, 5] = 1e30      # one huge value
    q, sc = bench.pack_kv_rows(x)
    q8 = np.zeros(x.size, np.int8)
    s8 = np.zeros(50 * 4, np.float32)
    oracle_lib.jyo_kv_pack(ptr(x), ptr(q8), ptr(s8), 4, 128, 50)
    assert np.array_equal(q.reshape(-1), q8)
    assert np.array_equal(sc.reshape(-1).view(np.uint32), s8.view(np.uint32))
