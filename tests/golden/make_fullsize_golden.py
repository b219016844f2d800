"""Write tests/golden/fullsize.json: greedy token ids of the full-size benchmark models
from jieyu's own decode loop, compiled from the reference sources by oracle/Makefile
(`make -C oracle ref` -> oracle/_ref/libjyref.so).

    python tests/golden/make_fullsize_golden.py

Models come from the repository's deterministic generator (include/jieyu_synth.h) with
the benchmark configurations of jieyu_amd.model.CONFIGS; prompts are the first ids of
the benchmark's prompt stream (jysyn_uniform_int_fill(seed, 99, 0, vocab - 1)).  Only
the ids are committed.
"""
import ctypes as C
import json
import os
import platform
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from jieyu_amd.model import Synth, synth_config  # noqa: E402

# name: (configuration, prompt tokens, new tokens, max_seq)
CASES = {
    # Llama-3-8B shape, Q8_0, seed 3: a 48-token prompt through the prompt GEMMs, 32 greedy tokens
    "llama3-8b-full": ("llama3-8b", 48, 32, 96),
    # Qwen2.5-0.5B shape, Q8_0, tied head, biases: the benchmark's 512-token prompt, 64 greedy tokens
    "qwen2.5-0.5b-full-512": ("qwen2.5-0.5b", 512, 64, 600),
    # Qwen2.5-7B shape, Q8_0, biases, theta 1e6: a 24-token prompt, 16 greedy tokens
    "qwen2.5-7b-full": ("qwen2.5-7b", 24, 16, 48),
}


def ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def main():
    if not oracle.ref_available():
        sys.exit("oracle/_ref/libjyref.so is missing: run `make -C oracle ref` where the reference tree exists")
    ref = oracle.load_ref()
    olib = oracle.load_oracle()
    isa = ref.jyref_init()
    meta = dict(reference_version=ref.jyref_version().decode(), isa_avx2=bool(isa & 1), isa_fma=bool(isa & 2),
                isa_avxvnni=bool(isa & 4), libc=" ".join(platform.libc_ver()), machine=platform.machine(),
                threads=os.environ.get("OMP_NUM_THREADS", str(os.cpu_count())))
    out = {}
    for name, (cname, plen, new, max_seq) in CASES.items():
        t0 = time.time()
        cfg = synth_config(cname)
        syn = Synth(olib, cfg)
        d = syn.desc
        prompt = np.zeros(plen, np.int32)
        olib.jysyn_uniform_int_fill(cfg.seed, 99, 0, d.vocab_size - 1, ptr(prompt), plen)
        c = np.zeros(max_seq * d.head_dim // 2, np.float32)
        s = np.zeros_like(c)
        ref.jyref_rope_table(max_seq, d.head_dim, d.rope_theta, ptr(c), ptr(s))
        ids = np.zeros(max_seq + 1, np.int32)
        n = ref.jyref_generate(C.byref(d), ptr(prompt), plen, None, 0, ptr(c), ptr(s), max_seq, new, 0.0, 1.0,
                               ptr(ids), None, None, 0)
        out[name] = dict(config=cname, prompt_len=plen, max_seq=max_seq, max_new=new, ids=ids[:n].tolist())
        syn.close()
        print(f"{name}: {n - plen} tokens in {time.time() - t0:.1f} s", flush=True)
    with open(os.path.join(HERE, "fullsize.json"), "w") as f:
        json.dump(dict(meta=meta, cases=out), f, indent=1)
    print("wrote", os.path.join(HERE, "fullsize.json"))


if __name__ == "__main__":
    main()
