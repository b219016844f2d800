"""The oracle's f16 and k-quant paths (Q4_K, Q5_K, Q6_K) pinned against jieyu.

  * bit-exact against golden vectors the compiled reference wrote
    (tests/golden/quant.npz, quant_generate.json; make_quant_golden.py): matmul_w
    at m == 1 (dot_row_avx2) and m > 1 (the generic path), wmat_row, and greedy /
    sampled ids of four mixed-type models;
  * bit-exact against the reference library on fresh inputs where it is built
    (forward_cached layer outputs and the int8 cache of a mixed model);
  * an independent float64 decode of GGML's block formats written from the
    format description (not from the restatement), so a wrong scale index, nibble
    or bit position fails even without the reference.
"""
import ctypes as C
import json
import os
import sys

import numpy as np
import pytest

from conftest import ptr, rope_tables

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = os.path.join(HERE, "golden")
sys.path.insert(0, GOLD)

import quant_models as QM  # noqa: E402
from jieyu_amd.model import WMat  # noqa: E402


@pytest.fixture(scope="module")
def qz():
    return np.load(os.path.join(GOLD, "quant.npz"))


@pytest.fixture(scope="module")
def qgen():
    with open(os.path.join(GOLD, "quant_generate.json")) as f:
        return json.load(f)


def assert_bits(got, want, what=""):
    g = np.ascontiguousarray(got).view(np.uint32)
    w = np.ascontiguousarray(want).view(np.uint32)
    assert g.shape == w.shape, what
    bad = np.flatnonzero(g.reshape(-1) != w.reshape(-1))
    assert bad.size == 0, f"{what}: {bad.size} mismatches, first at {bad[:5]}"


def keys(z, prefix):
    return sorted({k.split(".")[0] for k in z.files if k.startswith(prefix)})


# ---------------------------------------------------------------- reference goldens

def test_matmul_w_golden(oracle_lib, qz):
    cases = [k for k in keys(qz, "") if not k.startswith("row_")]
    assert len(cases) == len(QM.KERNEL_CASES)
    for key in cases:
        t, m, n, k = (int(v) for v in qz[key + ".meta"])
        w, a = np.ascontiguousarray(qz[key + ".w"]), np.ascontiguousarray(qz[key + ".a"])
        got = np.zeros((m, n), np.float32)
        wm = WMat(ptr(w), t)
        oracle_lib.jyo_matmul_w(C.byref(wm), m, n, k, ptr(a), ptr(got))
        assert_bits(got, qz[key + ".c"], key)


def test_embed_row_golden(oracle_lib, qz):
    for key in keys(qz, "row_"):
        t, rows, width = (int(v) for v in qz[key + ".meta"])
        w = np.ascontiguousarray(qz[key + ".w"])
        wm = WMat(ptr(w), t)
        for i, r in enumerate(qz[key + ".ids"]):
            y = np.zeros(width, np.float32)
            oracle_lib.jyo_embed_row(C.byref(wm), int(r), width, ptr(y))
            assert_bits(y, qz[key + ".y"][i], f"{key} row {r}")


def oracle_generate(olib, desc, prompt, max_seq, max_new, T=0.0, rp=1.0):
    import oracle
    c, s = rope_tables(olib, max_seq, desc.head_dim, desc.rope_theta)
    p = np.asarray(prompt, np.int32)
    ids = np.zeros(max_seq + 1, np.int32)
    kv = oracle.JyoKV()
    assert olib.jyo_kv_init(C.byref(kv), desc.num_layers, max_seq, desc.num_kv_heads, desc.head_dim) == 0
    try:
        n = olib.jyo_generate(C.byref(desc), ptr(p), len(p), None, 0, ptr(c), ptr(s), max_seq, max_new, T, rp,
                              ptr(ids), C.byref(kv), None)
    finally:
        olib.jyo_kv_free(C.byref(kv))
    return ids[:n].tolist()


@pytest.mark.parametrize("case", ["kq-mixed", "kq-mixed-T0.8-rp1.1", "kq-tied", "kq-tied-T0.0-rp1.3", "f16",
                                  "f32-f16-q8"])
def test_generate_golden(oracle_lib, qgen, case):
    g = qgen["cases"][case]
    m = QM.build_model(g["model"])
    d, keep = QM.desc_of(m)
    assert g["prompt"] == QM.prompt_of(m, len(g["prompt"])).tolist()  # the model rebuilds as recorded
    got = oracle_generate(oracle_lib, d, g["prompt"], g["max_seq"], g["max_new"], g["temperature"],
                          g["repetition_penalty"])
    assert got == g["ids"]


# ---------------------------------------------------------------- against the reference library

@pytest.mark.parametrize("seed", [1, 2])
def test_matmul_w_matches_reference_random(oracle_lib, ref_lib, seed):
    rng = np.random.default_rng(seed)
    for t in (QM.JY_Q4_K, QM.JY_Q5_K, QM.JY_Q6_K, QM.JY_F16):
        for m in (1, 2, 7):
            n, k = 19, (512 if t != QM.JY_F16 else 200)
            w = QM.rand_matrix(rng, t, n, k)
            a = rng.standard_normal((m, k)).astype(np.float32)
            c1 = np.zeros((m, n), np.float32)
            c2 = np.zeros_like(c1)
            wm = WMat(ptr(w), t)
            oracle_lib.jyo_matmul_w(C.byref(wm), m, n, k, ptr(a), ptr(c1))
            ref_lib.jyref_matmul_w(C.byref(wm), m, n, k, ptr(a), ptr(c2))
            assert_bits(c1, c2, f"{QM.NAMES[t]} m={m}")


def test_forward_cached_matches_reference(oracle_lib, ref_lib):
    """prefill 5 rows then 1 row through the mixed k-quant model: layer outputs and cache"""
    import oracle
    m = QM.build_model("kq-mixed")
    d, keep = QM.desc_of(m)
    max_seq = 16
    c, s = rope_tables(oracle_lib, max_seq, d.head_dim, d.rope_theta)
    rng = np.random.default_rng(9)
    kv = oracle.JyoKV()
    assert oracle_lib.jyo_kv_init(C.byref(kv), d.num_layers, max_seq, d.num_kv_heads, d.head_dim) == 0
    rkv = ref_lib.jyref_kv_create(d.num_layers, max_seq, d.num_kv_heads, d.head_dim)
    try:
        start = 0
        for seq in (5, 1):
            X = rng.standard_normal((seq, d.hidden)).astype(np.float32)
            X1, X2 = X.copy(), X.copy()
            lo1 = np.zeros((d.num_layers, seq, d.hidden), np.float32)
            lo2 = np.zeros_like(lo1)
            assert oracle_lib.jyo_forward_cached(C.byref(d), ptr(X1), ptr(c), ptr(s), seq, start, C.byref(kv),
                                                 ptr(lo1)) == 0
            assert ref_lib.jyref_forward_cached(C.byref(d), ptr(c), ptr(s), ptr(X2), seq, start, rkv, ptr(lo2)) == 0
            assert_bits(lo1, lo2, f"layer_out seq {seq}")
            assert_bits(X1, X2, f"X seq {seq}")
            start += seq
        n = d.num_layers * max_seq * d.num_kv_heads * d.head_dim
        a = np.ctypeslib.as_array(C.cast(kv.k, C.POINTER(C.c_int8)), (n,))
        b = np.ctypeslib.as_array(C.cast(ref_lib.jyref_kv_k(rkv), C.POINTER(C.c_int8)), (n,))
        assert np.array_equal(a, b)
    finally:
        oracle_lib.jyo_kv_free(C.byref(kv))
        ref_lib.jyref_kv_free(rkv)


# ---------------------------------------------------------------- the block formats from their description

def _h(b, off):
    return b[:, off:off + 2].copy().view(np.float16).astype(np.float64).reshape(-1)


def _k4_scales(sc):
    """6-bit scales and mins of the 8 sub-blocks: j < 4 in the low 6 bits of bytes j
    (scale) and j+4 (min); j >= 4 from the nibbles of byte j+4 with the top two bits
    of bytes j-4 (scale) and j (min)"""
    s = np.zeros((sc.shape[0], 8), np.int64)
    mn = np.zeros_like(s)
    for j in range(8):
        if j < 4:
            s[:, j] = sc[:, j] & 63
            mn[:, j] = sc[:, j + 4] & 63
        else:
            s[:, j] = (sc[:, j + 4] & 15) | ((sc[:, j - 4] >> 6) << 4)
            mn[:, j] = (sc[:, j + 4] >> 4) | ((sc[:, j] >> 6) << 4)
    return s, mn


def decode_f64(t, blocks):
    """[nb, 256] float64 weights of raw k-quant blocks"""
    b = blocks.astype(np.int64)
    nb = b.shape[0]
    out = np.zeros((nb, 256))
    e = np.arange(256)
    if t in (QM.JY_Q4_K, QM.JY_Q5_K):
        d, dmin = _h(blocks, 0), _h(blocks, 2)
        s, mn = _k4_scales(b[:, 4:16])
        qs = b[:, 16:144] if t == QM.JY_Q4_K else b[:, 48:176]
        sub = e // 32            # sub-block: 64-element groups of 32 low then 32 high nibbles
        byte = (e // 64) * 32 + e % 32
        q = np.where(sub % 2 == 0, qs[:, byte] & 15, qs[:, byte] >> 4)
        if t == QM.JY_Q5_K:
            q = q + 16 * ((b[:, 16:48][:, e % 32] >> sub) & 1)
        out = d[:, None] * s[:, sub] * q - dmin[:, None] * mn[:, sub]
    else:  # Q6_K: two halves of 128; quarter t' of a half takes low nibbles of ql[l] / ql[l+32]
        ql, qh = b[:, 0:128], b[:, 128:192]
        sc = blocks[:, 192:208].view(np.int8).astype(np.int64)
        d = _h(blocks, 208)
        half, r = e // 128, e % 128
        quarter, l = r // 32, r % 32
        lo_byte = half * 64 + l + 32 * (quarter % 2)
        lo = np.where(quarter < 2, ql[:, lo_byte] & 15, ql[:, lo_byte] >> 4)
        hi = (qh[:, half * 32 + l] >> (2 * quarter)) & 3
        q = (lo | (hi << 4)) - 32
        out = d[:, None] * sc[:, half * 8 + l // 16 + 2 * quarter] * q
    return out


@pytest.mark.parametrize("t", [QM.JY_Q4_K, QM.JY_Q5_K, QM.JY_Q6_K])
def test_dequant_matches_format_description(oracle_lib, t):
    """every product is exact in float64 and float32 (at most 24 significant bits), so
    the restatement's values equal the float64 decode rounded once"""
    rng = np.random.default_rng(t)
    blocks = QM.rand_blocks(rng, t, 64, 256).reshape(64, -1)
    # extremes: all-ones bytes (largest scales, mins and quants) and all-zero quants
    blocks[0, 4:] = 255 if t != QM.JY_Q6_K else blocks[0, 4:]
    if t == QM.JY_Q6_K:
        blocks[0, :192] = 255
        blocks[1, 192:208] = np.array([-128, 127] * 8, np.int8).view(np.uint8)
    want = decode_f64(t, blocks).astype(np.float32)
    got = np.zeros((64, 256), np.float32)
    for i in range(64):
        oracle_lib.jyo_dequant_block(t, ptr(np.ascontiguousarray(blocks[i])), ptr(got[i]))
    assert_bits(got, want, QM.NAMES[t])


@pytest.mark.parametrize("t", [QM.JY_Q4_K, QM.JY_Q5_K, QM.JY_Q6_K])
def test_row_dot_close_to_float64(oracle_lib, t):
    """the 32-lane dot against a float64 dot of the decoded weights (rel 1e-5)"""
    rng = np.random.default_rng(100 + t)
    k = 2048
    row = QM.rand_blocks(rng, t, 1, k)
    x = rng.standard_normal(k).astype(np.float32)
    w = decode_f64(t, row.reshape(k // 256, -1)).reshape(-1)
    want = float(np.dot(x.astype(np.float64), w))
    got = oracle_lib.jyo_q_row_dot(ptr(x), ptr(row), t, k)
    assert abs(got - want) <= 1e-5 * np.sum(np.abs(x.astype(np.float64) * w))


def test_f16_matmul_is_f32_matmul_of_converted(oracle_lib):
    """f16 weights are converted exactly, then the f32 chain: same bits as the f32
    matmul of the converted matrix"""
    rng = np.random.default_rng(3)
    for (m, n, k) in ((1, 37, 40), (4, 16, 9)):
        w16 = (0.05 * rng.standard_normal((k, n))).astype(np.float16)
        a = rng.standard_normal((m, k)).astype(np.float32)
        c1 = np.zeros((m, n), np.float32)
        c2 = np.zeros_like(c1)
        oracle_lib.jyo_matmul_f16(m, n, k, ptr(a), ptr(w16.view(np.uint16)), ptr(c1))
        oracle_lib.jyo_matmul_f32(m, n, k, ptr(a), ptr(w16.astype(np.float32)), ptr(c2))
        assert_bits(c1, c2)
