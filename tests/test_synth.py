"""The synthetic-model generator (include/jieyu_synth.h): deterministic bytes and
a Q8_0 quantizer that meets the block format's invariants.  Both the product
library and the oracle link the same generator, so a model built on the GPU host
is the model the golden vectors were written from."""
import ctypes as C
import hashlib
import os
import subprocess
import sys

import numpy as np

from conftest import ptr

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

HASH_SNIPPET = r"""
import ctypes as C, hashlib, sys
sys.path.insert(0, %r)
import oracle
from jieyu_amd.model import Synth, synth_config
lib = oracle.load_oracle()
s = Synth(lib, synth_config("qwen2.5-0.5b", num_layers=2, vocab_size=3000))
m = s.ptr.contents
print(hashlib.sha256(C.string_at(m.arena, m.arena_bytes)).hexdigest())
"""


def test_generator_deterministic_across_thread_counts():
    digests = set()
    for threads in ("1", "3", "8"):
        env = dict(os.environ, OMP_NUM_THREADS=threads)
        r = subprocess.run([sys.executable, "-c", HASH_SNIPPET % ROOT], capture_output=True, text=True, env=env,
                           timeout=300, check=True)
        digests.add(r.stdout.strip())
    assert len(digests) == 1


def test_product_and_oracle_generators_agree(oracle_lib):
    import jieyu_amd
    from jieyu_amd.model import Synth, synth_config
    cfg = synth_config("llama3-8b", num_layers=1, hidden=256, num_heads=4, num_kv_heads=2, head_dim=64,
                       intermediate=512, vocab_size=500)
    a = Synth(oracle_lib, cfg)
    b = Synth(jieyu_amd.lib(), cfg)
    try:
        ma, mb = a.ptr.contents, b.ptr.contents
        assert ma.arena_bytes == mb.arena_bytes
        assert C.string_at(ma.arena, ma.arena_bytes) == C.string_at(mb.arena, mb.arena_bytes)
    finally:
        a.close()
        b.close()


def test_normal_fill_moments(oracle_lib):
    x = np.zeros(1 << 20, np.float32)
    oracle_lib.jysyn_normal_fill(42, 3, 0.5, ptr(x), x.size)
    assert abs(x.mean()) < 0.003 and abs(x.std() - 0.5) < 0.003
    y = np.zeros(1 << 10, np.float32)  # a prefix of the same stream is the same values
    oracle_lib.jysyn_normal_fill(42, 3, 0.5, ptr(y), y.size)
    assert np.array_equal(x[:y.size], y)
    z = np.zeros(1 << 10, np.float32)  # another stream differs
    oracle_lib.jysyn_normal_fill(42, 4, 0.5, ptr(z), z.size)
    assert not np.array_equal(y, z)


def test_uniform_int_fill_range(oracle_lib):
    q = np.zeros(200000, np.int32)
    oracle_lib.jysyn_uniform_int_fill(1, 11, -127, 127, ptr(q), q.size)
    assert q.min() == -127 and q.max() == 127
    counts = np.bincount(q + 127)
    assert counts.min() > 0.8 * q.size / 255


def test_quantize_q8_0_block_invariants(oracle_lib):
    rng = np.random.default_rng(0)
    nb = 512
    x = (rng.standard_normal((nb, 32)) * rng.uniform(1e-4, 10, (nb, 1))).astype(np.float32)
    x[3] = 0.0
    out = np.zeros(nb * 34, np.uint8)
    oracle_lib.jysyn_quantize_q8_0(ptr(x), ptr(out), x.size)
    blk = out.reshape(nb, 34)
    d = blk[:, 0:2].copy().view(np.float16)[:, 0]
    q = blk[:, 2:].view(np.int8).astype(np.int32)
    amax = np.abs(x).max(axis=1)
    # d is amax/127 rounded to the nearest half; q = round(x/d) within +-127
    assert np.array_equal(d, (amax / np.float32(127)).astype(np.float16))
    assert np.all(np.abs(q) <= 127)
    live = amax > 0
    assert np.all(q[~live] == 0) and np.all(d[~live] == 0)
    # q rounds x * 127/amax (the unrounded scale), so dequantizing with the stored half
    # errs by at most half a step plus 127 times the half's rounding of the scale
    d32 = (amax / np.float32(127)).astype(np.float64)[:, None]
    bound = 0.5 * d32 + 127 * np.abs(d.astype(np.float64)[:, None] - d32) + 1e-6 * d32
    err = np.abs(q * d.astype(np.float64)[:, None] - x)
    assert np.all(err[live] <= bound[live])
    assert np.all(np.abs(q[live]).max(axis=1) == 127)
    # half conversion helpers agree with numpy's round-to-nearest-even conversion
    vals = np.concatenate([x.reshape(-1)[:4096], [65504, 65520, 1e-8, -6.1e-5, 0.0]]).astype(np.float32)
    mine = np.array([oracle_lib.jysyn_f32_to_f16(float(v)) for v in vals], np.uint16)
    with np.errstate(over="ignore"):  # 65520 rounds to inf, as in the C conversion
        assert np.array_equal(mine, vals.astype(np.float16).view(np.uint16))
    back = np.array([oracle_lib.jysyn_f16_to_f32(int(h)) for h in mine], np.float32)
    assert np.array_equal(back, mine.view(np.float16).astype(np.float32))


def test_synth_models_match_config_shapes(oracle_lib):
    from jieyu_amd.model import CONFIGS, Synth, synth_config
    for name in CONFIGS:
        cfg = synth_config(name, num_layers=1, vocab_size=64)
        s = Synth(oracle_lib, cfg)
        try:
            d = s.desc
            assert (d.hidden, d.num_heads, d.num_kv_heads, d.head_dim, d.intermediate) == (
                cfg.hidden, cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, cfg.intermediate)
            per_layer_q8 = (d.hidden * (d.num_heads + 2 * d.num_kv_heads) * d.head_dim +
                            d.num_heads * d.head_dim * d.hidden + 3 * d.hidden * d.intermediate) // 32 * 34
            if cfg.wtype == 3:
                assert s.weight_bytes >= per_layer_q8
        finally:
            s.close()
