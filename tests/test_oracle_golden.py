"""The CPU oracle pinned against jieyu's own outputs and against mathematics.

Three kinds of checks, so that a plausible slip in the restatement (a dropped
term, a wrong index, a different summation order) fails at least one:
  * bit-exact against golden vectors the compiled reference wrote
    (tests/golden/kernels.npz, tests/golden/generate.json; make_golden.py),
  * bit-exact against the reference library itself on fresh random inputs when
    oracle/_ref/libjyref.so is built,
  * closed forms, invariants and float64 restatements with stated tolerances,
    including the reference's own known-answer tests (text.h:737-843, :993-1002).
"""
import ctypes as C
import json
import math
import os

import numpy as np
import pytest

from conftest import ptr, rope_tables

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = os.path.join(HERE, "golden")


@pytest.fixture(scope="module")
def kz():
    return np.load(os.path.join(GOLD, "kernels.npz"))


@pytest.fixture(scope="module")
def gen_gold():
    with open(os.path.join(GOLD, "generate.json")) as f:
        return json.load(f)


def bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint32) if a.dtype == np.float32 else a


def assert_bits(got, want, what=""):
    g, w = bits(got), bits(want)
    assert g.shape == w.shape, what
    bad = np.flatnonzero(g.reshape(-1) != w.reshape(-1))
    assert bad.size == 0, f"{what}: {bad.size} mismatches, first at {bad[:5]}"


def keys(kz, prefix):
    return sorted({k.split(".")[0] for k in kz.files if k.startswith(prefix)})


# ---------------------------------------------------------------- kernel goldens

def test_q8_matmul_golden(oracle_lib, kz):
    for key in keys(kz, "q8_"):
        w, a, c = kz[key + ".w"], kz[key + ".a"], kz[key + ".c"]
        m, n = c.shape
        k = a.shape[1]
        got = np.zeros((m, n), np.float32)
        oracle_lib.jyo_matmul_q8(ptr(np.ascontiguousarray(a)), ptr(w), ptr(got), m, n, k)
        assert_bits(got, c, key)


def test_f32_matmul_golden(oracle_lib, kz):
    for key in keys(kz, "f32_"):
        A, B, Cw = kz[key + ".A"], kz[key + ".B"], kz[key + ".C"]
        m, k = A.shape
        n = B.shape[1]
        got = np.zeros((m, n), np.float32)
        oracle_lib.jyo_matmul_f32(m, n, k, ptr(A), ptr(B), ptr(got))
        assert_bits(got, Cw, key)


def test_rmsnorm_golden(oracle_lib, kz):
    for key in keys(kz, "rms_"):
        x, w, y = kz[key + ".x"], kz[key + ".w"], kz[key + ".y"]
        got = np.zeros_like(y)
        oracle_lib.jyo_rmsnorm(ptr(x.copy()), ptr(got), ptr(w), x.size, 1e-5)
        assert_bits(got, y, key)


def test_rope_golden(oracle_lib, kz):
    for key in keys(kz, "rope_hd"):
        if "_seq" in key:
            continue
        ms, hd, theta = kz[key + ".meta"]
        c, s = rope_tables(oracle_lib, int(ms), int(hd), float(theta))
        assert_bits(c, kz[key + ".cos"], key + " cos")
        assert_bits(s, kz[key + ".sin"], key + " sin")
        for seq_key in (key + "_seq1", key + "_seq5"):
            seq, sp, nh = (int(v) for v in kz[seq_key + ".meta"])
            y = kz[seq_key + ".q"].copy()
            oracle_lib.jyo_rope(ptr(y), seq, sp, nh, int(hd), ptr(c), ptr(s))
            assert_bits(y, kz[seq_key + ".y"], seq_key)


def test_silu_golden(oracle_lib, kz):
    for key in keys(kz, "silu_"):
        x, y = kz[key + ".x"], kz[key + ".y"]
        got = np.zeros_like(y)
        oracle_lib.jyo_silu(ptr(x.copy()), ptr(got), x.size)
        assert_bits(got, y, key)


def test_kv_pack_golden(oracle_lib, kz):
    src = kz["kvpack.src"]
    dst = np.zeros(src.size, np.int8)
    sc = np.zeros(src.shape[0] * src.shape[1], np.float32)
    oracle_lib.jyo_kv_pack(ptr(src.copy()), ptr(dst), ptr(sc), src.shape[1], src.shape[2], src.shape[0])
    assert_bits(dst, kz["kvpack.dst"], "kv_pack q")
    assert_bits(sc, kz["kvpack.sc"], "kv_pack scale")


def test_attention_golden(oracle_lib, kz):
    for key in keys(kz, "attn_"):
        seq, sp, nh, nkv, hd, cap = (int(v) for v in kz[key + ".meta"])
        kc, vc = kz[key + ".kc_in"].copy(), kz[key + ".vc_in"].copy()
        ks, vs = kz[key + ".ks_in"].copy(), kz[key + ".vs_in"].copy()
        o = np.zeros((seq, nh, hd), np.float32)
        rc = oracle_lib.jyo_attention(ptr(kz[key + ".Q_in"].copy()), ptr(kz[key + ".K_in"].copy()),
                                      ptr(kz[key + ".V_in"].copy()), ptr(o), seq, sp, nh, nkv, hd, ptr(kc), ptr(ks),
                                      ptr(vc), ptr(vs), cap)
        assert rc == 0
        assert_bits(o, kz[key + ".out"], key + " out")
        for nm, arr in (("kc", kc), ("vc", vc), ("ks", ks), ("vs", vs)):
            assert_bits(arr, kz[f"{key}.{nm}"], f"{key} {nm}")


# ---------------------------------------------------------------- end-to-end goldens

def _synth(oracle_lib, case):
    from jieyu_amd.model import Synth, synth_config
    cfg = synth_config(case["config"], **case.get("overrides", {}))
    return Synth(oracle_lib, cfg)


def _oracle_generate(olib, desc, prompt, max_seq, max_new, T=0.0, rp=1.0, theta=None, eos=()):
    import oracle
    c, s = rope_tables(olib, max_seq, desc.head_dim, desc.rope_theta if theta is None else theta)
    p = np.asarray(prompt, np.int32)
    e = np.asarray(eos, np.int32) if eos else None
    ids = np.zeros(max_seq + 1, np.int32)
    kv = oracle.JyoKV()
    assert olib.jyo_kv_init(C.byref(kv), desc.num_layers, max_seq, desc.num_kv_heads, desc.head_dim) == 0
    try:
        n = olib.jyo_generate(C.byref(desc), ptr(p), len(p), ptr(e), len(eos), ptr(c), ptr(s), max_seq, max_new,
                              T, rp, ptr(ids), C.byref(kv), None)
    finally:
        olib.jyo_kv_free(C.byref(kv))
    return ids[:n].tolist()


GEN_NAMES = ["tiny-f32", "qwen-like-small", "llama-like-small", "llama-like-small-T0.0-rp1.3",
             "llama-like-small-T0.8-rp1.0", "llama-like-small-T0.7-rp1.1", "qwen2.5-0.5b-full"]


@pytest.mark.parametrize("name", GEN_NAMES)
def test_generate_golden(oracle_lib, gen_gold, name):
    case = gen_gold["cases"][name]
    syn = _synth(oracle_lib, case)
    try:
        got = _oracle_generate(oracle_lib, syn.desc, case["prompt"], case["max_seq"], case["max_new"],
                               case.get("temperature", 0.0), case.get("repetition_penalty", 1.0))
    finally:
        syn.close()
    assert got == case["ids"]


def test_bind_test_kat(oracle_lib, gen_gold):
    """check_bind_weights (text.h:817-843): generate() must equal the float64 model's greedy ids."""
    from golden.kat_models import bind_model_desc, bind_test_model, reference_ids_f64
    bm = bind_test_model()
    desc, keep = bind_model_desc(bm)
    for prompt in ([1, 2, 3], [5, 6, 7]):
        want_f64 = reference_ids_f64(bm, prompt, 3, 8)
        got = _oracle_generate(oracle_lib, desc, prompt, 8, 3, theta=10000.0)
        assert got == want_f64 == gen_gold["cases"]["bind_test_kat"][str(prompt)]
    del keep


def test_demo_model_kat(oracle_lib, gen_gold):
    """make_demo_model (converter.h:412-503) decodes "abcdefgh" to "ijklmnop..." (text.h:993-1002)."""
    from golden.kat_models import demo_model_desc
    desc, keep = demo_model_desc()
    prompt = [256] + list(b"abcdefgh")
    got = _oracle_generate(oracle_lib, desc, prompt, 64, 16, theta=10000.0)
    del keep
    assert bytes(got[len(prompt):len(prompt) + 16]) == b"ijklmnopqrstuvwx"
    assert got == gen_gold["cases"]["demo_abcdefgh"]["ids"]


# ---------------------------------------------------------------- oracle == reference on fresh inputs

@pytest.mark.parametrize("seed", [1, 2, 3])
def test_oracle_matches_reference_random(oracle_lib, ref_lib, seed):
    rng = np.random.default_rng(seed)
    # Q8 matvec and generic path, odd shapes
    from conftest import q8_random_normal
    for (m, n, k) in ((1, 33, 96), (3, 7, 64), (1, 5, 4096 + 32 * seed)):
        w = q8_random_normal(oracle_lib, n, k, seed=seed * 100 + k)
        a = rng.standard_normal((m, k)).astype(np.float32)
        c1 = np.zeros((m, n), np.float32)
        c2 = np.zeros((m, n), np.float32)
        oracle_lib.jyo_matmul_q8(ptr(a), ptr(w), ptr(c1), m, n, k)
        ref_lib.jyref_matmul_q8(ptr(a), ptr(w), ptr(c2), m, n, k)
        assert_bits(c1, c2, f"q8 {m}x{n}x{k}")
    for (m, n, k) in ((1, 1, 1), (1, 7, 13), (2, 9, 33), (5, 15, 64), (1, 64 + seed, 40), (6, 23, 100)):
        A = rng.standard_normal((m, k)).astype(np.float32)
        B = rng.standard_normal((k, n)).astype(np.float32)
        c1 = np.zeros((m, n), np.float32)
        c2 = np.zeros((m, n), np.float32)
        oracle_lib.jyo_matmul_f32(m, n, k, ptr(A), ptr(B), ptr(c1))
        ref_lib.jyref_matmul_f32(m, n, k, ptr(A), ptr(B), ptr(c2))
        assert_bits(c1, c2, f"f32 {m}x{n}x{k}")
    for n in list(range(1, 40)) + [1000 + seed]:
        x = (rng.standard_normal(n) * 10 ** rng.uniform(-3, 3)).astype(np.float32)
        w = rng.standard_normal(n).astype(np.float32)
        y1, y2 = np.zeros(n, np.float32), np.zeros(n, np.float32)
        oracle_lib.jyo_rmsnorm(ptr(x.copy()), ptr(y1), ptr(w), n, 1e-5)
        ref_lib.jyref_rmsnorm(ptr(x.copy()), ptr(y2), ptr(w), n, 1e-5)
        assert_bits(y1, y2, f"rms {n}")
    x = (rng.standard_normal(5000) * 20).astype(np.float32)
    y1, y2 = np.zeros_like(x), np.zeros_like(x)
    oracle_lib.jyo_silu(ptr(x), ptr(y1), x.size)
    ref_lib.jyref_silu(ptr(x), ptr(y2), x.size)
    assert_bits(y1, y2, "silu")
    # attention with a long history (exercises the softmax over many keys)
    seq, sp, nh, nkv, hd, cap = 2, 300 + seed, 4, 2, 64, 310
    kc = rng.integers(-127, 128, cap * nkv * hd).astype(np.int8)
    vc = rng.integers(-127, 128, cap * nkv * hd).astype(np.int8)
    ks = (rng.random(cap * nkv) * 0.05).astype(np.float32)
    vs = (rng.random(cap * nkv) * 0.05).astype(np.float32)
    Q = rng.standard_normal((seq, nh, hd)).astype(np.float32)
    K = rng.standard_normal((seq, nkv, hd)).astype(np.float32)
    V = rng.standard_normal((seq, nkv, hd)).astype(np.float32)
    outs = []
    for lib, fn in ((oracle_lib, "jyo_attention"), (ref_lib, "jyref_attention")):
        bufs = [kc.copy(), ks.copy(), vc.copy(), vs.copy()]
        o = np.zeros((seq, nh, hd), np.float32)
        assert getattr(lib, fn)(ptr(Q.copy()), ptr(K.copy()), ptr(V.copy()), ptr(o), seq, sp, nh, nkv, hd,
                                ptr(bufs[0]), ptr(bufs[1]), ptr(bufs[2]), ptr(bufs[3]), cap) == 0
        outs.append([o] + bufs)
    for a, b in zip(*outs):
        assert_bits(a, b, "attention")


def test_oracle_matches_reference_forward_cached(oracle_lib, ref_lib):
    """forward_cached in two calls (prefill 5, then 1 row) -- layer output and the int8 cache."""
    import oracle
    from jieyu_amd.model import Synth, synth_config
    cfg = synth_config("llama3-8b", num_layers=2, hidden=256, num_heads=4, num_kv_heads=2, head_dim=64,
                       intermediate=512, vocab_size=300)
    syn = Synth(oracle_lib, cfg)
    d = syn.desc
    try:
        max_seq = 16
        c, s = rope_tables(oracle_lib, max_seq, d.head_dim, d.rope_theta)
        rng = np.random.default_rng(5)
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
                assert ref_lib.jyref_forward_cached(C.byref(d), ptr(c), ptr(s), ptr(X2), seq, start, rkv,
                                                    ptr(lo2)) == 0
                assert_bits(X1, X2, f"X seq {seq}")
                assert_bits(lo1, lo2, f"layer_out seq {seq}")
                start += seq
            n = d.num_layers * max_seq * d.num_kv_heads * d.head_dim
            for attr, fn, dt, cnt in (("k", "jyref_kv_k", C.c_int8, n), ("v", "jyref_kv_v", C.c_int8, n),
                                      ("ks", "jyref_kv_ks", C.c_float, n // d.head_dim),
                                      ("vs", "jyref_kv_vs", C.c_float, n // d.head_dim)):
                a = np.ctypeslib.as_array(C.cast(getattr(kv, attr), C.POINTER(dt)), (cnt,))
                b = np.ctypeslib.as_array(C.cast(getattr(ref_lib, fn)(rkv), C.POINTER(dt)), (cnt,))
                assert_bits(a, b, "kv " + attr)
        finally:
            oracle_lib.jyo_kv_free(C.byref(kv))
            ref_lib.jyref_kv_free(rkv)
    finally:
        syn.close()


# ---------------------------------------------------------------- closed forms and invariants

def test_f16_to_f32_exhaustive(oracle_lib):
    """Every finite half (subnormals included) converts exactly; numpy's conversion is exact too."""
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32)
    fn = oracle_lib.jyo_f16_to_f32
    got = np.array([fn(int(v)) for v in h], np.float32)
    fin = np.isfinite(want)
    assert_bits(got[fin], want[fin], "f16")
    assert np.all(np.isinf(got[np.isinf(want)]) & (np.sign(got[np.isinf(want)]) == np.sign(want[np.isinf(want)])))
    assert np.all(np.isnan(got[np.isnan(want)]))


def test_q8_dot_closed_forms(oracle_lib):
    # one block, one non-zero weight: exact product q*d*x
    k = 64
    row = np.zeros((k // 32, 34), np.uint8)
    row[:, 0:2] = np.array([0.5, 0.25], np.float16).view(np.uint8).reshape(2, 2)
    row[1, 2 + 7] = np.uint8(np.int8(-3).view(np.uint8))
    x = np.zeros(k, np.float32)
    x[32 + 7] = 1.75
    assert oracle_lib.jyo_q8_row_dot(ptr(x), ptr(row.reshape(-1)), k) == np.float32(-3 * 0.25 * 1.75)
    # random rows: within a float64 error bound (n * eps * sum |terms|)
    from conftest import q8_random_normal
    rng = np.random.default_rng(7)
    n, k = 64, 4096
    w = q8_random_normal(oracle_lib, n, k, seed=3)
    a = rng.standard_normal(k).astype(np.float32)
    got = np.zeros(n, np.float32)
    oracle_lib.jyo_matmul_q8(ptr(a), ptr(w), ptr(got), 1, n, k)
    blk = w.reshape(n, k // 32, 34)
    d = blk[:, :, 0:2].copy().view(np.float16).astype(np.float64)[..., 0]
    q = blk[:, :, 2:].view(np.int8).astype(np.float64)
    wf = (q * d[:, :, None]).reshape(n, k)
    exact = wf @ a.astype(np.float64)
    bound = (k // 32 + 8) * np.finfo(np.float32).eps * (np.abs(wf) @ np.abs(a.astype(np.float64)))
    assert np.all(np.abs(got - exact) <= bound)


def test_q8_summation_order_is_pinned(oracle_lib, kz):
    """A plausible slip -- summing the row in another order -- does not reproduce the golden bits,
    so the golden test above pins the reference's 32-lane block order."""
    key = "q8_m1_16x14336"
    w, a, c = kz[key + ".w"], kz[key + ".a"], kz[key + ".c"]
    n, k = c.shape[1], a.shape[1]
    blk = w.reshape(n, k // 32, 34)
    d = blk[:, :, 0:2].copy().view(np.float16).astype(np.float32)[..., 0]
    q = blk[:, :, 2:].view(np.int8).astype(np.float32)
    naive = np.zeros(n, np.float32)
    for j in range(k // 32):  # block-sequential, lanes summed in order, one rounding per add
        wj = q[:, j, :] * d[:, j, None]
        for i in range(32):
            naive = naive + wj[:, i] * a[0, 32 * j + i]
    assert np.any(naive.view(np.uint32) != c[0].view(np.uint32))
    assert np.allclose(naive, c[0], rtol=1e-4, atol=1e-5)


def test_rmsnorm_float64(oracle_lib):
    rng = np.random.default_rng(11)
    for n in (1, 8, 4096):
        x = rng.standard_normal(n).astype(np.float32)
        w = rng.standard_normal(n).astype(np.float32)
        y = np.zeros(n, np.float32)
        oracle_lib.jyo_rmsnorm(ptr(x.copy()), ptr(y), ptr(w), n, 1e-5)
        x64 = x.astype(np.float64)
        want = x64 / np.sqrt(np.mean(x64 * x64) + 1e-5) * w
        assert np.allclose(y, want, rtol=4e-6, atol=1e-7)
    y = np.zeros(16, np.float32)  # all-zero input: scale 1/sqrt(eps), output 0
    oracle_lib.jyo_rmsnorm(ptr(np.zeros(16, np.float32)), ptr(y), ptr(np.ones(16, np.float32)), 16, 1e-5)
    assert not np.any(y)


def test_rope_closed_forms(oracle_lib):
    hd, ms = 128, 50
    c, s = rope_tables(oracle_lib, ms, hd, 500000.0)
    half = hd // 2
    # table: cos/sin of pos * theta^(-2i/hd), within float32 rounding of the float64 angle
    pos = np.arange(ms)[:, None]
    i = np.arange(half)[None, :]
    ang = pos * np.power(500000.0, -2.0 * i / hd)
    assert np.allclose(c.reshape(ms, half), np.cos(ang), atol=2e-6)
    assert np.allclose(s.reshape(ms, half), np.sin(ang), atol=2e-6)
    assert np.all(c[:half] == 1.0) and np.all(s[:half] == 0.0)
    rng = np.random.default_rng(3)
    q = rng.standard_normal((1, 2, hd)).astype(np.float32)
    y = q.copy()
    # position 0 rotates by nothing, so only the store order of x86_classic.txt:23-29 shows:
    # within each group of 8 pairs, pairs (2,3) and (4,5) exchange slots
    oracle_lib.jyo_rope(ptr(y), 1, 0, 2, hd, ptr(c), ptr(s))
    pairs = q.reshape(2, hd // 16, 8, 2)
    want = pairs[:, :, [0, 1, 4, 5, 2, 3, 6, 7], :].reshape(q.shape)
    assert_bits(y, want, "rope pos 0")
    # any position preserves each rotated pair's norm (pairs stored in the same slot order)
    y = q.copy()
    oracle_lib.jyo_rope(ptr(y), 1, 37, 2, hd, ptr(c), ptr(s))
    n0 = np.hypot(want[..., 0::2].astype(np.float64), want[..., 1::2])
    n1 = np.hypot(y[..., 0::2].astype(np.float64), y[..., 1::2])
    assert np.allclose(n0, n1, rtol=1e-6)


def test_kv_pack_invariants(oracle_lib):
    rng = np.random.default_rng(4)
    src = (rng.standard_normal((9, 3, 64)) * rng.uniform(0.01, 10, (9, 3, 1))).astype(np.float32)
    src[2, 1] = 0.0
    src[3, 0] = 1e-9  # below the 1e-8 threshold: scale and values 0
    dst = np.zeros(src.size, np.int8)
    sc = np.zeros(27, np.float32)
    oracle_lib.jyo_kv_pack(ptr(src.copy()), ptr(dst), ptr(sc), 3, 64, 9)
    q = dst.reshape(9, 3, 64).astype(np.float64)
    scale = sc.reshape(9, 3)
    amax = np.abs(src).max(axis=2)
    live = amax > 1e-8
    assert np.all(scale[~live] == 0) and np.all(q[~live] == 0)
    assert np.all(np.abs(q[live]).max(axis=1) == 127)
    assert np.allclose(scale[live], amax[live] / 127, rtol=1e-7)
    err = np.abs(q * scale[..., None] - src)
    assert np.all(err[live] <= 0.5 * scale[live][:, None] * (1 + 1e-5) + 1e-12)


def test_attention_float64(oracle_lib):
    """Decode attention equals softmax over exact int8 dot products within float32 rounding."""
    rng = np.random.default_rng(9)
    nh, nkv, hd, sp, cap = 8, 2, 64, 77, 80
    kc = rng.integers(-127, 128, (cap, nkv, hd)).astype(np.int8)
    vc = rng.integers(-127, 128, (cap, nkv, hd)).astype(np.int8)
    ks = (rng.random((cap, nkv)) * 0.02).astype(np.float32)
    vs = (rng.random((cap, nkv)) * 0.02).astype(np.float32)
    Q = rng.standard_normal((1, nh, hd)).astype(np.float32)
    K = rng.standard_normal((1, nkv, hd)).astype(np.float32)
    V = rng.standard_normal((1, nkv, hd)).astype(np.float32)
    o = np.zeros((1, nh, hd), np.float32)
    kc2, vc2, ks2, vs2 = kc.copy(), vc.copy(), ks.copy(), vs.copy()
    assert oracle_lib.jyo_attention(ptr(Q.copy()), ptr(K), ptr(V), ptr(o), 1, sp, nh, nkv, hd, ptr(kc2), ptr(ks2),
                                    ptr(vc2), ptr(vs2), cap) == 0
    n = sp + 1
    kq, kscale = kc2[:n].astype(np.float64), ks2[:n].astype(np.float64)
    vq, vscale = vc2[:n].astype(np.float64), vs2[:n].astype(np.float64)
    for h in range(nh):
        g = h // (nh // nkv)
        amax = np.abs(Q[0, h]).max()
        qs = np.float32(amax) / np.float32(127)
        qq = np.clip(np.rint(Q[0, h] * (np.float32(127) / np.float32(amax))), -127, 127).astype(np.float64)
        dots = kq[:, g, :] @ qq
        sc = dots * kscale[:, g] * float(qs) / math.sqrt(hd)
        p = np.exp(sc - sc.max())
        p /= p.sum()
        want = (p * vscale[:, g]) @ vq[:, g, :]
        assert np.allclose(o[0, h], want, rtol=2e-5, atol=1e-6), h


def test_silu_float64(oracle_lib):
    x = np.linspace(-80, 80, 100001).astype(np.float32)
    y = np.zeros_like(x)
    oracle_lib.jyo_silu(ptr(x), ptr(y), x.size)
    x64 = x.astype(np.float64)
    want = x64 / (1 + np.exp(-x64))
    assert np.allclose(y, want, rtol=4e-7, atol=1e-30)


def test_planted_mistake_in_oracle_is_caught(kz):
    """A plausible slip in a restatement -- RoPE without the reference's slot exchange within
    each group of 8 pairs -- disagrees with the golden vectors."""
    key = "rope_hd128"
    c, s = kz[key + ".cos"], kz[key + ".sin"]
    seq, sp, nh = (int(v) for v in kz[key + "_seq1.meta"])
    q = kz[key + "_seq1.q"]
    half = 64
    cc, ss = c[sp * half:(sp + 1) * half], s[sp * half:(sp + 1) * half]
    x0, x1 = q[..., 0::2], q[..., 1::2]
    plain = np.empty_like(q)
    plain[..., 0::2] = x0 * cc - x1 * ss
    plain[..., 1::2] = x0 * ss + x1 * cc
    assert not np.allclose(plain, kz[key + "_seq1.y"], atol=1e-3)
