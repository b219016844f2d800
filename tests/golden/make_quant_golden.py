"""Write tests/golden/quant.npz and tests/golden/quant_generate.json from jieyu's own
code: matmul_w (libs/model_libs/wmat_kernel.h:9-16) and wmat_row (:18-29) on f16,
Q4_K, Q5_K and Q6_K matrices, and generate() (libs/model_libs/generate.h:90-112)
on the mixed-type synthetic models of quant_models.py.  Runs the reference
compiled by oracle/Makefile (`make -C oracle ref` -> oracle/_ref/libjyref.so);
only the data is committed.

    python tests/golden/make_quant_golden.py
"""
import ctypes as C
import json
import os
import platform
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, HERE)

import oracle  # noqa: E402
import quant_models as QM  # noqa: E402
from jieyu_amd.model import WMat  # noqa: E402

GEN = dict(prompt=9, new=20, max_seq=48)
SAMPLED = [("kq-mixed", 0.8, 1.1), ("kq-tied", 0.0, 1.3)]


def ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def rope(ref, max_seq, hd, theta):
    c = np.zeros(max_seq * hd // 2, np.float32)
    s = np.zeros_like(c)
    ref.jyref_rope_table(max_seq, hd, theta, ptr(c), ptr(s))
    return c, s


def kernels(ref):
    rng = np.random.default_rng(20261202)
    out = {}
    for (t, m, n, k) in QM.KERNEL_CASES:
        key = f"{QM.NAMES[t]}_m{m}_{n}x{k}"
        w = QM.rand_matrix(rng, t, n, k)
        a = rng.standard_normal((m, k)).astype(np.float32)
        c = np.zeros((m, n), np.float32)
        wm = WMat(ptr(w), t)
        ref.jyref_matmul_w(C.byref(wm), m, n, k, ptr(a), ptr(c))
        out[key + ".w"], out[key + ".a"], out[key + ".c"] = w, a, c
        out[key + ".meta"] = np.array([t, m, n, k], np.int64)
    # embedding rows (wmat_row) of every type: [rows][width] quantized or f16
    for t, width in ((QM.JY_Q4_K, 512), (QM.JY_Q5_K, 256), (QM.JY_Q6_K, 768), (QM.JY_F16, 72)):
        key = f"row_{QM.NAMES[t]}_{width}"
        rows = 6
        if t == QM.JY_F16:
            w = (0.02 * rng.standard_normal((rows, width))).astype(np.float16).view(np.uint16)
        else:
            w = QM.rand_blocks(rng, t, rows, width)
        ids = np.array([0, 5, 3], np.int32)
        y = np.zeros((len(ids), width), np.float32)
        wm = WMat(ptr(w), t)
        for i, r in enumerate(ids):
            ref.jyref_wmat_row(C.byref(wm), int(r), width, ptr(y[i]))
        out[key + ".w"], out[key + ".ids"], out[key + ".y"] = w, ids, y
        out[key + ".meta"] = np.array([t, rows, width], np.int64)
    return out


def generate_cases(ref):
    res = {}
    for name in QM.SPECS:
        m = QM.build_model(name)
        d, keep = QM.desc_of(m)
        prompt = QM.prompt_of(m, GEN["prompt"])
        c, s = rope(ref, GEN["max_seq"], m["hd"], m["theta"])
        runs = [(0.0, 1.0)] + [(t, rp) for (nm, t, rp) in SAMPLED if nm == name]
        for (t, rp) in runs:
            ids = np.zeros(GEN["max_seq"] + 1, np.int32)
            n = ref.jyref_generate(C.byref(d), ptr(prompt), len(prompt), None, 0, ptr(c), ptr(s), GEN["max_seq"],
                                   GEN["new"], t, rp, ptr(ids), None, None, 0)
            assert n > len(prompt), (name, n)
            key = name if (t, rp) == (0.0, 1.0) else f"{name}-T{t}-rp{rp}"
            res[key] = dict(model=name, prompt=prompt.tolist(), max_seq=GEN["max_seq"], max_new=GEN["new"],
                            temperature=t, repetition_penalty=rp, ids=ids[:n].tolist())
        del keep
    return res


def main():
    if not oracle.ref_available():
        sys.exit("oracle/_ref/libjyref.so is missing: run `make -C oracle ref` where the reference tree exists")
    ref = oracle.load_ref()
    isa = ref.jyref_init()
    meta = dict(reference_version=ref.jyref_version().decode(), isa_avx2=bool(isa & 1), isa_fma=bool(isa & 2),
                libc=" ".join(platform.libc_ver()), numpy=np.__version__,
                note="models rebuilt by quant_models.build_model(name) (numpy PCG64, seed 7)")
    np.savez_compressed(os.path.join(HERE, "quant.npz"), **kernels(ref))
    with open(os.path.join(HERE, "quant_generate.json"), "w") as f:
        json.dump(dict(meta=meta, cases=generate_cases(ref)), f, indent=1)
    print("wrote quant.npz, quant_generate.json")


if __name__ == "__main__":
    main()
