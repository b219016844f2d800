"""Shared fixtures.  GPU tests are marked `gpu`; everything else runs on the CPU."""
import ctypes as C
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


def ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle
    return oracle.load_oracle()


@pytest.fixture(scope="session")
def ref_lib():
    import oracle
    if not oracle.ref_available():
        pytest.skip("oracle/_ref/libjyref.so not built (needs the reference tree)")
    return oracle.load_ref()


def rope_tables(olib, max_seq, head_dim, theta):
    half = head_dim // 2
    c = np.zeros(max_seq * half, np.float32)
    s = np.zeros_like(c)
    olib.jyo_rope_table(max_seq, head_dim, theta, ptr(c), ptr(s))
    return c, s


def q8_random_normal(olib, rows, cols, seed, std=0.02):
    """Q8_0 rows [rows][cols/32]x34 from N(0, std) (the synthetic-model quantizer)."""
    x = np.zeros(rows * cols, np.float32)
    olib.jysyn_normal_fill(seed, 7, std, ptr(x), x.size)
    out = np.zeros(rows * (cols // 32) * 34, np.uint8)
    olib.jysyn_quantize_q8_0(ptr(x), ptr(out), x.size)
    return out


def q8_random_uniform(olib, rows, cols, seed):
    """Isolated-matvec inputs: int8 ~ U[-127, 127], per-block scale ~ U(0.001, 0.01) as fp16."""
    nb = rows * (cols // 32)
    q = np.zeros(nb * 32, np.int32)
    olib.jysyn_uniform_int_fill(seed, 11, -127, 127, ptr(q), q.size)
    d = np.zeros(nb, np.float32)
    olib.jysyn_uniform_fill(seed, 12, 0.001, 0.01, ptr(d), d.size)
    dh = d.astype(np.float16).view(np.uint16)  # round to nearest even, as jysyn_f32_to_f16
    blk = np.zeros((nb, 34), np.uint8)
    blk[:, 0:2] = dh.view(np.uint8).reshape(nb, 2)
    blk[:, 2:] = q.astype(np.int8).view(np.uint8).reshape(nb, 32)
    return blk.reshape(-1)


def kv_views(okv, L, max_seq, nkv, hd):
    """numpy views of an oracle cache (jyo_kv): int8 K, V [L][max_seq][nkv][hd], fp32 scales."""
    import ctypes as C_
    k = np.ctypeslib.as_array(C_.cast(okv.k, C_.POINTER(C_.c_int8)), (L, max_seq, nkv, hd))
    v = np.ctypeslib.as_array(C_.cast(okv.v, C_.POINTER(C_.c_int8)), (L, max_seq, nkv, hd))
    ks = np.ctypeslib.as_array(C_.cast(okv.ks, C_.POINTER(C_.c_float)), (L, max_seq, nkv))
    vs = np.ctypeslib.as_array(C_.cast(okv.vs, C_.POINTER(C_.c_float)), (L, max_seq, nkv))
    return k, v, ks, vs


def prefill_kv(olib, d, pre, max_seq, kv, one_draw=False):
    """Fill positions [0, pre) of every layer of the GPU cache `kv` and of a new oracle cache
    (returned) with N(0,1) K and V packed by the oracle's kv_pack_q8 (the long-context
    workload's setup).  one_draw: the same draw in every layer (the benchmark's setup)."""
    import ctypes as C_
    import oracle as O_
    L, nkv, hd = d.num_layers, d.num_kv_heads, d.head_dim
    okv = O_.JyoKV()
    assert olib.jyo_kv_init(C_.byref(okv), L, max_seq, nkv, hd) == 0
    ok8, ov8, oks, ovs = kv_views(okv, L, max_seq, nkv, hd)
    packed = None
    for l in range(L):
        if packed is None or not one_draw:
            kf = np.zeros(pre * nkv * hd, np.float32)
            vf = np.zeros_like(kf)
            olib.jysyn_normal_fill(9, 1000 + (0 if one_draw else 2 * l), 1.0, ptr(kf), kf.size)
            olib.jysyn_normal_fill(9, 1001 + (0 if one_draw else 2 * l), 1.0, ptr(vf), vf.size)
            k8 = np.zeros(kf.size, np.int8)
            v8 = np.zeros(kf.size, np.int8)
            ks = np.zeros(pre * nkv, np.float32)
            vs = np.zeros_like(ks)
            olib.jyo_kv_pack(ptr(kf), ptr(k8), ptr(ks), nkv, hd, pre)
            olib.jyo_kv_pack(ptr(vf), ptr(v8), ptr(vs), nkv, hd, pre)
            del kf, vf
            packed = (k8.reshape(pre, nkv, hd), ks.reshape(pre, nkv), v8.reshape(pre, nkv, hd), vs.reshape(pre, nkv))
        k8, ks, v8, vs = packed
        ok8[l, :pre] = k8
        ov8[l, :pre] = v8
        oks[l, :pre] = ks
        ovs[l, :pre] = vs
        kv.write(l, 0, k8, ks, v8, vs)
    kv.set_len(pre)
    return okv
