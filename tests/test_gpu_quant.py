"""f16 and k-quant (Q4_K / Q5_K / Q6_K) weights on the GPU, bit-exact with jieyu.

  * jyhip_wmat_matmul (matmul_w, libs/model_libs/wmat_kernel.h:9-16) against the
    reference's own outputs (tests/golden/quant.npz) and against the oracle at
    Llama-3-8B matrix shapes, decode (m == 1) and prompt (m > 1);
  * whole models of mixed weight types: per-layer hidden states and the int8 KV
    cache after a prefill then decode steps against the oracle, and greedy /
    sampled token ids against the reference's generate() (quant_generate.json).
"""
import ctypes as C
import json
import os
import sys

import numpy as np
import pytest

import oracle
from conftest import ptr, rope_tables

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = os.path.join(HERE, "golden")
sys.path.insert(0, GOLD)

import quant_models as QM  # noqa: E402

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)


@pytest.fixture(scope="module")
def jy():
    import jieyu_amd
    if jieyu_amd.device_count() < 1:
        pytest.fail("no HIP device visible")
    return jieyu_amd


def bits_equal(a, b):
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    return a.shape == b.shape and np.array_equal(a.view(np.uint8), b.view(np.uint8))


def first_diff(a, b):
    d = np.flatnonzero(np.ascontiguousarray(a).view(np.uint32).reshape(-1) !=
                       np.ascontiguousarray(b).view(np.uint32).reshape(-1))
    return d[:5]


# ---------------------------------------------------------------- single matrices

def test_wmat_matmul_reference_golden(jy):
    z = np.load(os.path.join(GOLD, "quant.npz"))
    cases = sorted({k.split(".")[0] for k in z.files if not k.startswith("row_")})
    for key in cases:
        t, m, n, k = (int(v) for v in z[key + ".meta"])
        say(f"matmul_w golden {key}")
        W = jy.WeightMatrix(z[key + ".w"], t, n, k)
        got = W.matmul(z[key + ".a"])
        W.close()
        assert bits_equal(got, z[key + ".c"]), f"{key}: first diffs {first_diff(got, z[key + '.c'])}"


SHAPES = [(JT, n, k) for JT in (QM.JY_Q4_K, QM.JY_Q5_K, QM.JY_Q6_K)
          for (n, k) in ((4096, 4096), (14336, 4096), (4096, 14336), (1031, 768))] + \
         [(QM.JY_F16, 1024, 4096), (QM.JY_F16, 4096, 1031), (QM.JY_Q8_0, 4096, 4096)] + \
         [(QM.JY_F32, 1031, 1001), (QM.JY_F16, 70, 1003), (QM.JY_F32, 5, 3), (QM.JY_F16, 129, 7)]


@pytest.mark.parametrize("t,n,k", SHAPES)
def test_wmat_matmul_matches_oracle(jy, oracle_lib, t, n, k):
    say(f"matmul_w {QM.NAMES[t]} n={n} k={k}")
    rng = np.random.default_rng(n + k + t)
    w = QM.rand_matrix(rng, t, n, k)
    W = jy.WeightMatrix(w, t, n, k)
    wm = QM.WMat(w.ctypes.data_as(C.c_void_p), t)
    for m in (1, 3):
        if m > 1 and n * k > 4096 * 4096:
            continue  # the oracle's generic path is scalar; keep the CPU side to seconds
        a = rng.standard_normal((m, k)).astype(np.float32)
        want = np.zeros((m, n), np.float32)
        oracle_lib.jyo_matmul_w(C.byref(wm), m, n, k, ptr(a), ptr(want))
        got = W.matmul(a)
        assert bits_equal(got, want), f"m={m}: first diffs {first_diff(got, want)}"
    W.close()


# prompts of 128 rows or more take the 128 x 128 tile of the prompt GEMM: ragged m and n
@pytest.mark.parametrize("t,m,n,k", [(QM.JY_Q8_0, 160, 1031, 1024), (QM.JY_Q8_0, 256, 384, 4096),
                                     (QM.JY_Q4_K, 130, 300, 768), (QM.JY_Q6_K, 129, 257, 512)])
def test_prompt_gemm_big_tile_matches_oracle(jy, oracle_lib, t, m, n, k):
    say(f"prompt gemm {QM.NAMES[t]} m={m} n={n} k={k}")
    rng = np.random.default_rng(m + n + k + t)
    w = QM.rand_matrix(rng, t, n, k)
    W = jy.WeightMatrix(w, t, n, k)
    wm = QM.WMat(w.ctypes.data_as(C.c_void_p), t)
    a = rng.standard_normal((m, k)).astype(np.float32)
    want = np.zeros((m, n), np.float32)
    oracle_lib.jyo_matmul_w(C.byref(wm), m, n, k, ptr(a), ptr(want))
    got = W.matmul(a)
    W.close()
    assert bits_equal(got, want), f"first diffs {first_diff(got, want)}"


def test_wmat_rejects_bad_shapes(jy):
    rng = np.random.default_rng(0)
    w = QM.rand_blocks(rng, QM.JY_Q4_K, 4, 256)
    with pytest.raises(jy.JyError):
        jy.WeightMatrix(w, QM.JY_Q4_K, 4, 320)  # not a multiple of the 256-weight block
    with pytest.raises(jy.JyError):
        jy.WeightMatrix(w, 99, 4, 256)


# ---------------------------------------------------------------- whole models

@pytest.mark.parametrize("name", list(QM.SPECS))
def test_forward_cached_layers_and_kv(jy, oracle_lib, name):
    say(f"forward_cached {name}")
    m = QM.build_model(name)
    d, keep = QM.desc_of(m)
    L, H, nkv, hd = d.num_layers, d.hidden, d.num_kv_heads, d.head_dim
    max_seq = 24
    cos, sin = rope_tables(oracle_lib, max_seq, hd, d.rope_theta)
    okv = oracle.JyoKV()
    assert oracle_lib.jyo_kv_init(C.byref(okv), L, max_seq, nkv, hd) == 0
    g = jy.GpuModel(d, max_seq)
    kv = g.kv(max_seq)
    rng = np.random.default_rng(4)
    start = 0
    try:
        for seq in (6, 1, 1, 4):
            X = rng.standard_normal((seq, H)).astype(np.float32)
            Xo = X.copy()
            lo = np.zeros((L, seq, H), np.float32)
            assert oracle_lib.jyo_forward_cached(C.byref(d), ptr(Xo), ptr(cos), ptr(sin), seq, start, C.byref(okv),
                                                 ptr(lo)) == 0
            Xg, log = g.forward_cached(kv, X, start, layer_out=True)
            assert bits_equal(log, lo), f"layers differ at seq={seq} start={start}: {first_diff(log, lo)}"
            assert bits_equal(Xg, Xo)
            start += seq
        ok8 = np.ctypeslib.as_array(C.cast(okv.k, C.POINTER(C.c_int8)), (L, max_seq, nkv, hd))
        ov8 = np.ctypeslib.as_array(C.cast(okv.v, C.POINTER(C.c_int8)), (L, max_seq, nkv, hd))
        for l in range(L):
            k, ks, v, vs = kv.read(l, 0, start)
            assert np.array_equal(k, ok8[l, :start]) and np.array_equal(v, ov8[l, :start])
    finally:
        oracle_lib.jyo_kv_free(C.byref(okv))
        kv.close()
        g.close()


@pytest.fixture(scope="module")
def qgen():
    with open(os.path.join(GOLD, "quant_generate.json")) as f:
        return json.load(f)


@pytest.mark.parametrize("case", ["kq-mixed", "kq-mixed-T0.8-rp1.1", "kq-tied", "kq-tied-T0.0-rp1.3", "f16",
                                  "f32-f16-q8"])
def test_generate_matches_reference(jy, qgen, case):
    g0 = qgen["cases"][case]
    say(f"generate {case}")
    m = QM.build_model(g0["model"])
    d, keep = QM.desc_of(m)
    g = jy.GpuModel(d, g0["max_seq"])
    try:
        ids, _ = g.generate(np.array(g0["prompt"], np.int32), g0["max_new"], temperature=g0["temperature"],
                            repetition_penalty=g0["repetition_penalty"])
    finally:
        g.close()
    assert ids.tolist() == g0["ids"]
