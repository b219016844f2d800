"""A workload to profile the decode attention kernels at long context (not a test): one
layer of the Qwen2.5-7B shape (28 heads, 4 kv heads, head_dim 128) over a cache pre-filled
to 32768 positions with N(0,1) K / V, 10 fast-mode decode rows by direct launches
(forward_cached).  Usage: python3 tests/prof_attention_32768.py [config positions]."""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, HERE)
import jieyu_amd as jy  # noqa: E402
import oracle  # noqa: E402
from conftest import prefill_kv  # noqa: E402
from jieyu_amd.model import Synth, synth_config  # noqa: E402

olib = oracle.load_oracle()
name, pre = (sys.argv[1], int(sys.argv[2])) if len(sys.argv) > 2 else ("qwen2.5-7b", 32768)
syn = Synth(olib, synth_config(name, num_layers=1, vocab_size=1000))
d = syn.desc
g = jy.GpuModel(d, pre + 64)
g.mode = jy.MODE_FAST
kv = g.kv(pre + 64)
prefill_kv(olib, d, pre, pre + 64, kv, one_draw=True)
x = np.random.default_rng(0).standard_normal((1, d.hidden)).astype(np.float32)
for i in range(10):
    kv.set_len(pre)
    g.forward_cached(kv, x, pre)
print(name, "done", flush=True)
kv.close()
g.close()
syn.close()
