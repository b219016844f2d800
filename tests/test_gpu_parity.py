"""HIP decode path vs the CPU oracle on identical seeded inputs (bit-exact).

Every comparison here is exact: token ids, logits, per-layer hidden states and
KV-cache bytes must equal the oracle's bit for bit, because every kernel
reproduces the reference's operation order and rounding.  (The tolerance the
path is specified to, 1e-3 relative on hidden states, is therefore met with
zero error.)
"""
import ctypes as C
import sys

import numpy as np
import pytest

import oracle
from conftest import prefill_kv, ptr, q8_random_normal, q8_random_uniform, rope_tables

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


# ---------------------------------------------------------------- Q8 matvec


@pytest.mark.parametrize("rows,cols", [(8, 32), (13, 96), (100, 896), (1000, 4864), (517, 1408), (64, 14336),
                                       (300, 3584), (40, 18944)])
def test_q8_matvec_bitexact(jy, oracle_lib, rows, cols):
    say(f"q8 matvec {rows}x{cols}")
    w = q8_random_normal(oracle_lib, rows, cols, seed=rows * 7 + cols)
    x = np.random.default_rng(rows).standard_normal(cols).astype(np.float32)
    ref = np.zeros(rows, np.float32)
    oracle_lib.jyo_matmul_q8(ptr(x), ptr(w), ptr(ref), 1, rows, cols)
    m = jy.Q8Matrix(w, rows, cols)
    y = m.matvec(x)
    m.close()
    assert bits_equal(y, ref), f"max abs diff {np.abs(y - ref).max()}"


@pytest.mark.parametrize("rows,cols", [(4096, 4096), (14336, 4096), (4096, 14336)])
def test_q8_matvec_isolated_shapes(jy, oracle_lib, rows, cols):
    """The isolated-kernel workload: int8 ~ U[-127,127], scales ~ U(0.001,0.01), x ~ N(0,1), seed 1."""
    say(f"q8 matvec isolated {rows}x{cols}")
    w = q8_random_uniform(oracle_lib, rows, cols, seed=1)
    x = np.zeros(cols, np.float32)
    oracle_lib.jysyn_normal_fill(1, 13, 1.0, ptr(x), cols)
    ref = np.zeros(rows, np.float32)
    oracle_lib.jyo_matmul_q8(ptr(x), ptr(w), ptr(ref), 1, rows, cols)
    m = jy.Q8Matrix(w, rows, cols)
    y = m.matvec(x)
    m.close()
    assert bits_equal(y, ref)
    # closed form in float64: the fp32 result is within a few ulp-sums of the exact dot
    q = w.reshape(rows, cols // 32, 34)
    d = q[:, :, :2].copy().view(np.float16).astype(np.float64)[:, :, 0]
    wf = q[:, :, 2:].view(np.int8).astype(np.float64) * d[:, :, None]
    exact = wf.reshape(rows, cols) @ x.astype(np.float64)
    tol = 1e-5 * (np.abs(wf.reshape(rows, cols)) @ np.abs(x.astype(np.float64)))
    assert np.all(np.abs(y - exact) <= tol)


# ---------------------------------------------------------------- model level

SMALL = {
    "llama-like-q8": dict(name="llama3-8b", num_layers=2, hidden=512, num_heads=8, num_kv_heads=2, head_dim=64,
                          intermediate=1408, vocab_size=3000),
    "qwen-like-q8": dict(name="qwen2.5-0.5b", num_layers=2, hidden=896, num_heads=14, num_kv_heads=2,
                         head_dim=64, intermediate=4864, vocab_size=5000),
    "hd128-q8": dict(name="qwen2.5-7b", num_layers=1, hidden=1024, num_heads=8, num_kv_heads=2, head_dim=128,
                     intermediate=2048, vocab_size=2000),
    "tiny-f32": dict(name="tiny-f32", num_layers=2, vocab_size=4000),
    # FFN width 1004: silu's libm tail on the last 4 gate values of a decode step and the
    # last (rows * 1004) % 8 of a prompt (silu/x86/x86_classic.txt:30-31)
    "f32-ffn-tail": dict(name="tiny-f32", num_layers=2, vocab_size=3000, intermediate=1004),
}


def make_synth(oracle_lib, key):
    from jieyu_amd.model import Synth, synth_config
    spec = dict(SMALL[key])
    name = spec.pop("name")
    return Synth(oracle_lib, synth_config(name, **spec))


def oracle_generate(olib, desc, prompt, max_seq, max_new, temperature=0.0, rp=1.0, eos=None):
    cos, sin = rope_tables(olib, max_seq, desc.head_dim, desc.rope_theta)
    out = np.zeros(max_seq + 1, np.int32)
    logits = np.zeros(desc.vocab_size, np.float32)
    eos_a = None if eos is None else np.asarray(eos, np.int32)
    n = olib.jyo_generate(C.byref(desc), ptr(prompt), len(prompt), ptr(eos_a), 0 if eos is None else len(eos),
                          ptr(cos), ptr(sin), max_seq, max_new, temperature, rp, ptr(out), None, ptr(logits))
    return out[:n].copy(), logits


@pytest.mark.parametrize("key", list(SMALL))
def test_generate_greedy_matches_oracle(jy, oracle_lib, key):
    say(f"generate greedy {key}")
    s = make_synth(oracle_lib, key)
    d = s.desc
    prompt = np.zeros(11, np.int32)
    oracle_lib.jysyn_uniform_int_fill(5, 99, 0, d.vocab_size - 1, ptr(prompt), len(prompt))
    max_seq, max_new = 64, 24
    ref_ids, ref_logits = oracle_generate(oracle_lib, d, prompt, max_seq, max_new)
    g = jy.GpuModel(d, max_seq)
    ids, st, logits = g.generate(prompt, max_new, want_logits=True)
    g.close()
    s.close()
    assert np.array_equal(ids, ref_ids), f"gpu {ids[len(prompt):]} vs oracle {ref_ids[len(prompt):]}"
    assert bits_equal(logits, ref_logits)


def test_generate_prompt_of_one(jy, oracle_lib):
    """prompt_len 1: the first step takes the m == 1 matvec path (matmul_q.h:139)."""
    say("generate prompt_len=1")
    s = make_synth(oracle_lib, "llama-like-q8")
    d = s.desc
    prompt = np.array([17], np.int32)
    ref_ids, _ = oracle_generate(oracle_lib, d, prompt, 40, 12)
    g = jy.GpuModel(d, 40)
    ids, _ = g.generate(prompt, 12)
    g.close()
    s.close()
    assert np.array_equal(ids, ref_ids)


def test_forward_cached_layers_and_kv(jy, oracle_lib):
    """Per-layer hidden states and the int8 cache after a prefill then a decode step."""
    say("forward_cached layers + kv")
    s = make_synth(oracle_lib, "qwen-like-q8")
    d = s.desc
    L, H, nkv, hd = d.num_layers, d.hidden, d.num_kv_heads, d.head_dim
    max_seq = 32
    cos, sin = rope_tables(oracle_lib, max_seq, hd, d.rope_theta)
    okv = oracle.JyoKV()
    assert oracle_lib.jyo_kv_init(C.byref(okv), L, max_seq, nkv, hd) == 0
    g = jy.GpuModel(d, max_seq)
    kv = g.kv(max_seq)
    rng = np.random.default_rng(3)
    start = 0
    for seq in (7, 1, 1, 5):
        X = rng.standard_normal((seq, H)).astype(np.float32)
        Xo = X.copy()
        lo = np.zeros((L, seq, H), np.float32)
        assert oracle_lib.jyo_forward_cached(C.byref(d), ptr(Xo), ptr(cos), ptr(sin), seq, start, C.byref(okv),
                                             ptr(lo)) == 0
        Xg, log = g.forward_cached(kv, X, start, layer_out=True)
        assert bits_equal(log, lo), f"layers differ at seq={seq} start={start}"
        assert bits_equal(Xg, Xo)
        assert len(kv) == start + seq
        start += seq
    ok8 = np.ctypeslib.as_array(C.cast(okv.k, C.POINTER(C.c_int8)), (L, max_seq, nkv, hd))
    ov8 = np.ctypeslib.as_array(C.cast(okv.v, C.POINTER(C.c_int8)), (L, max_seq, nkv, hd))
    oks = np.ctypeslib.as_array(C.cast(okv.ks, C.POINTER(C.c_float)), (L, max_seq, nkv))
    ovs = np.ctypeslib.as_array(C.cast(okv.vs, C.POINTER(C.c_float)), (L, max_seq, nkv))
    for l in range(L):
        k, ks, v, vs = kv.read(l, 0, start)
        assert np.array_equal(k, ok8[l, :start]) and np.array_equal(v, ov8[l, :start])
        assert bits_equal(ks, oks[l, :start]) and bits_equal(vs, ovs[l, :start])
    oracle_lib.jyo_kv_free(C.byref(okv))
    kv.close()
    g.close()
    s.close()


def prefill_cache(oracle_lib, d, pre, max_seq, kv):
    return prefill_kv(oracle_lib, d, pre, max_seq, kv)


# 766: 767 / 768 keys (scores inside the softmax/PV kernel) then 769 (two kernels);
# 1534: 1535 / 1536 keys (every score in LDS) then 1537 (the first of the windowed
# form); 3000: two windows and three chunks; 9000: windows and chunks with ragged ends
@pytest.mark.parametrize("pre", [766, 1534, 3000, 9000])
def test_prefilled_cache_long_context(jy, oracle_lib, pre):
    """Decode steps at start_pos pre.. over a cache pre-filled with packed N(0,1) K/V (the
    long-context workload's setup, at a reduced model size)."""
    say(f"pre-filled cache decode at {pre}")
    s = make_synth(oracle_lib, "hd128-q8")
    d = s.desc
    H, hd = d.hidden, d.head_dim
    max_seq = pre + 8
    cos, sin = rope_tables(oracle_lib, max_seq, hd, d.rope_theta)
    g = jy.GpuModel(d, max_seq)
    kv = g.kv(max_seq)
    okv = prefill_cache(oracle_lib, d, pre, max_seq, kv)
    rng = np.random.default_rng(4)
    for i in range(3):
        X = rng.standard_normal((1, H)).astype(np.float32)
        Xo = X.copy()
        assert oracle_lib.jyo_forward_cached(C.byref(d), ptr(Xo), ptr(cos), ptr(sin), 1, pre + i, C.byref(okv),
                                             None) == 0
        Xg = g.forward_cached(kv, X, pre + i)
        assert bits_equal(Xg, Xo), f"step {i}: max abs diff {np.abs(Xg - Xo).max()}"
    oracle_lib.jyo_kv_free(C.byref(okv))
    kv.close()
    g.close()
    s.close()


# 760: the session's steps cross from the one-kernel graph (up to 768 keys) to the
# two-kernel one; 6000: the windowed form throughout
@pytest.mark.parametrize("pre,n_new", [(760, 16), (6000, 8)])
def test_resume_over_long_prefilled_cache(jy, oracle_lib, pre, n_new):
    """The decode graphs (positions read on the device) over a pre-filled cache:
    jyhip_session_resume's greedy tokens against the oracle driven token by token
    (embedding row, forward_cached at the next position, lm_head, first maximum)."""
    say(f"session resume over a {pre}-position cache")
    s = make_synth(oracle_lib, "hd128-q8")
    d = s.desc
    H, V, hd = d.hidden, d.vocab_size, d.head_dim
    max_seq = pre + n_new + 8
    cos, sin = rope_tables(oracle_lib, max_seq, hd, d.rope_theta)
    g = jy.GpuModel(d, max_seq)
    kv = g.kv(max_seq)
    okv = prefill_cache(oracle_lib, d, pre, max_seq, kv)
    ids = np.zeros(pre + 1, np.int32)
    oracle_lib.jysyn_uniform_int_fill(8, 99, 0, V - 1, ptr(ids), len(ids))
    want = []
    tok = int(ids[-1])
    for i in range(n_new):
        X = np.zeros((1, H), np.float32)
        oracle_lib.jyo_embed_row(C.byref(d.embed), tok, H, ptr(X))
        assert oracle_lib.jyo_forward_cached(C.byref(d), ptr(X), ptr(cos), ptr(sin), 1, pre + i, C.byref(okv),
                                             None) == 0
        logits = np.zeros(V, np.float32)
        oracle_lib.jyo_matmul_w(C.byref(d.lm_head), 1, V, H, ptr(X), ptr(logits))
        tok = int(np.argmax(logits))
        want.append(tok)
    ss = g.session(ids, n_new, max_seq=max_seq, kv=kv, resume=True)
    ss.step(n_new)
    got = ss.ids()[pre + 1:]
    ss.close()
    assert list(got) == want
    oracle_lib.jyo_kv_free(C.byref(okv))
    kv.close()
    g.close()
    s.close()


@pytest.mark.parametrize("key", ["hd128-q8", "tiny-f32"])
def test_session_resume_matches_oracle(jy, oracle_lib, key):
    """jyhip_session_resume over a cache holding the prompt's first c positions (written by
    an earlier session) gives the oracle's tokens for the whole prompt: c = 0, a chunk
    run at start_pos c (the prefill path), and c = n - 1 (the single-row decode path)."""
    say(f"session resume {key}")
    s = make_synth(oracle_lib, key)
    d = s.desc
    prompt = np.zeros(19, np.int32)
    oracle_lib.jysyn_uniform_int_fill(6, 99, 0, d.vocab_size - 1, ptr(prompt), len(prompt))
    max_seq, max_new = 64, 16
    ref_ids, _ = oracle_generate(oracle_lib, d, prompt, max_seq, max_new)
    g = jy.GpuModel(d, max_seq)
    kv = g.kv(max_seq)
    for c in (0, 7, len(prompt) - 1):
        if c:
            g.session(prompt[:c], 1, kv=kv).close()
        kv.set_len(c)
        ss = g.session(prompt, max_new, kv=kv, resume=True)
        ss.step(max_new)
        ids = ss.ids()
        ss.close()
        assert np.array_equal(ids, ref_ids), f"c={c}: gpu {ids[len(prompt):]} vs oracle {ref_ids[len(prompt):]}"
    kv.set_len(len(prompt))
    with pytest.raises(jy.JyError):
        g.session(prompt, 4, kv=kv, resume=True)  # the cache already holds the whole prompt
    with pytest.raises(jy.JyError):
        g.session(prompt, 4, resume=True)  # nothing to resume from
    kv.close()
    g.close()
    s.close()


def test_session_survives_workspace_growth(jy, oracle_lib):
    """A forward_cached chunk longer than the session's prompt replaces the shared
    workspace between two steps; the session captures its decode graphs again and
    still gives the oracle's tokens."""
    say("session across a workspace reallocation")
    s = make_synth(oracle_lib, "llama-like-q8")
    d = s.desc
    prompt = np.arange(30, 35, dtype=np.int32)
    ref_ids, _ = oracle_generate(oracle_lib, d, prompt, 64, 20)
    g = jy.GpuModel(d, 64)
    ss = g.session(prompt, 20)
    ss.step(4)
    kv2 = g.kv(64)
    g.forward_cached(kv2, np.random.default_rng(1).standard_normal((48, d.hidden)).astype(np.float32), 0)
    ss.step(20)
    ids = ss.ids()
    ss.close()
    kv2.close()
    g.close()
    s.close()
    assert np.array_equal(ids, ref_ids)


def test_superseded_session_refuses_to_step(jy, oracle_lib):
    """The device holds one generation's ids and length per model: once a second session
    begins, the first one's step is an error, and the second runs as if alone."""
    say("superseded session")
    s = make_synth(oracle_lib, "llama-like-q8")
    d = s.desc
    p1 = np.arange(40, 47, dtype=np.int32)
    p2 = np.arange(3, 12, dtype=np.int32)
    ref2, _ = oracle_generate(oracle_lib, d, p2, 64, 12)
    g = jy.GpuModel(d, 64)
    s1 = g.session(p1, 12)
    s1.step(3)
    s2 = g.session(p2, 12)
    with pytest.raises(jy.JyError):
        s1.step(1)
    s2.step(12)
    ids2 = s2.ids()
    s1.close()
    s2.close()
    g.close()
    s.close()
    assert np.array_equal(ids2, ref2)


def test_sampling_and_penalty(jy, oracle_lib):
    """Temperature sampling (LCG, seed 12345) and the per-occurrence repetition penalty."""
    say("sampling + repetition penalty")
    s = make_synth(oracle_lib, "llama-like-q8")
    d = s.desc
    prompt = np.arange(5, 14, dtype=np.int32)
    g = jy.GpuModel(d, 64)
    for (t, rp) in [(0.0, 1.3), (0.8, 1.0), (0.7, 1.1)]:
        ref_ids, _ = oracle_generate(oracle_lib, d, prompt, 64, 20, temperature=t, rp=rp)
        ids, _ = g.generate(prompt, 20, temperature=t, repetition_penalty=rp)
        assert np.array_equal(ids, ref_ids), f"T={t} rp={rp}"
    g.close()
    s.close()


def test_eos_and_callback_stop(jy, oracle_lib):
    say("eos + callback")
    s = make_synth(oracle_lib, "llama-like-q8")
    d = s.desc
    prompt = np.arange(20, 27, dtype=np.int32)
    ref_ids, _ = oracle_generate(oracle_lib, d, prompt, 64, 30)
    eos_tok = int(ref_ids[len(prompt) + 5])
    ref_eos, _ = oracle_generate(oracle_lib, d, prompt, 64, 30, eos=[eos_tok])
    g = jy.GpuModel(d, 64)
    ids, _ = g.generate(prompt, 30, eos=[eos_tok])
    assert np.array_equal(ids, ref_eos)
    seen = []
    ids2, _ = g.generate(prompt, 30, callback=lambda t: (seen.append(t), len(seen) >= 4)[1])
    assert np.array_equal(ids2, ref_ids[:len(prompt) + 4]) and len(seen) == 4
    g.close()
    s.close()


def test_edge_cases(jy, oracle_lib):
    say("edge cases")
    s = make_synth(oracle_lib, "llama-like-q8")
    d = s.desc
    g = jy.GpuModel(d, 16)
    ids, _ = g.generate(np.arange(16, dtype=np.int32), 5)       # prompt fills max_seq -> prompt only
    assert len(ids) == 16
    ids, _ = g.generate(np.arange(3, dtype=np.int32), 0)        # max_new 0 -> prompt only
    assert len(ids) == 3
    ids, _ = g.generate(np.arange(10, dtype=np.int32), 50)      # clamp at max_seq
    ref, _ = oracle_generate(oracle_lib, d, np.arange(10, dtype=np.int32), 16, 50)
    assert np.array_equal(ids, ref) and len(ids) == 16
    with pytest.raises(jy.JyError):
        g.generate(np.array([d.vocab_size], np.int32), 2)       # id outside the vocabulary
    kv = g.kv(8)
    with pytest.raises(jy.JyError):
        g.forward_cached(kv, np.zeros((9, d.hidden), np.float32), 0)  # capacity exceeded
    kv.close()
    g.close()
    s.close()
