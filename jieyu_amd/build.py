"""Build libjieyu_amd.so in-tree (hipcc, gfx950) — the product library.

    python -m jieyu_amd.build        # or: from jieyu_amd.build import build; build()

Sources: csrc/*.hip and csrc/*.cpp through hipcc, csrc/*.c through gcc, and the
host-only text layer csrc/*.cc through g++.  The library lands next to this
file so it travels with the source tree.

    python -m jieyu_amd.build --sanitize

builds libjieyu_amd_asan.so instead: the host code (the runtime, the text layer)
instrumented with AddressSanitizer and UBSan, device code unchanged, for the CPU
tests (the loader takes it from JIEYU_AMD_LIB; the sanitizer runtime must be
preloaded, see asan_runtime()).
"""
import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIB = os.path.join(HERE, "libjieyu_amd.so")
LIB_ASAN = os.path.join(HERE, "libjieyu_amd_asan.so")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("JIEYU_AMD_ARCH", "gfx950")

# -ffp-contract=off: fused multiply-adds only where a kernel asks for one.
# -packed-fp32-ops off: no v_pk_*_f32 generation.
HIP_FLAGS = [
    "-O3", "-std=c++17", f"--offload-arch={ARCH}", "-fPIC", "-fvisibility=hidden",
    "-ffp-contract=off", "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument", "-I", INCLUDE, "-I", CSRC,
]
C_FLAGS = ["-std=c11", "-O2", "-ffp-contract=off", "-fno-fast-math", "-fopenmp", "-fPIC", "-I", INCLUDE]
CXX_FLAGS = ["-std=c++17", "-O2", "-fPIC", "-fvisibility=hidden", "-Wall", "-I", INCLUDE, "-I", CSRC]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout)
        raise RuntimeError("build step failed: " + " ".join(cmd[:3]) + " ...")
    return r.stdout


# host-side sanitizers: on hipcc lines each flag applies to the host compilation only
SAN_FLAGS = ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined", "-fno-omit-frame-pointer", "-g"]
CLANGXX = os.path.join(os.path.dirname(os.path.realpath(HIPCC)), "..", "llvm", "bin", "clang++")


def asan_runtime():
    """The clang AddressSanitizer runtime the sanitized library links against (preload it:
    LD_PRELOAD=<this> ASAN_OPTIONS=detect_leaks=0)."""
    import glob
    hits = sorted(glob.glob(os.path.join(os.path.dirname(CLANGXX), "..", "lib", "clang", "*", "lib", "linux",
                                         "libclang_rt.asan-x86_64.so")))
    if not hits:
        raise RuntimeError("no clang AddressSanitizer runtime next to " + CLANGXX)
    return os.path.realpath(hits[-1])


def build(verbose=False, jobs=None, sanitize=False):
    srcs = sorted(os.listdir(CSRC))
    lib_out = LIB_ASAN if sanitize else LIB
    host_san = [y for f in SAN_FLAGS for y in ("-Xarch_host", f)] if sanitize else []
    tmp = tempfile.mkdtemp(prefix="jyamd_build_")
    try:
        objs, cmds = [], []
        for s in srcs:
            path = os.path.join(CSRC, s)
            obj = os.path.join(tmp, s + ".o")
            if s.endswith((".hip", ".cpp")):
                cmd = [HIPCC, *HIP_FLAGS, *host_san, "-c", path, "-o", obj]
                if s.endswith(".cpp"):
                    cmd[1:1] = ["-x", "hip"]
            elif s.endswith(".c"):
                cmd = ["gcc", *C_FLAGS, "-c", path, "-o", obj]
            elif s.endswith(".cc"):
                # (clang++ with the sanitizers: one sanitizer runtime for the whole library)
                cmd = [CLANGXX, *CXX_FLAGS, *SAN_FLAGS, "-c", path, "-o", obj] if sanitize else \
                    ["g++", *CXX_FLAGS, "-c", path, "-o", obj]
            else:
                continue
            if verbose:
                print(" ".join(cmd))
            cmds.append(cmd)
            objs.append(obj)
        # one compiler per source file, at most `jobs` (default: the CPU count, capped at 8) at once
        jobs = jobs or min(8, os.cpu_count() or 1)
        with ThreadPoolExecutor(max_workers=jobs) as ex:
            for f in [ex.submit(_run, c) for c in cmds]:
                f.result()
        out_tmp = lib_out + ".tmp"
        rt = [asan_runtime()] if sanitize else []
        _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", out_tmp, *objs, *rt, "-lgomp", "-lm"])
        os.replace(out_tmp, lib_out)
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    return lib_out


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv, sanitize="--sanitize" in sys.argv))
