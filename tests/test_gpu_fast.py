"""The tolerance modes (jyhip_model_set_mode) against the CPU oracle.

The specification allows floating-point reordering within 1e-3 relative on per-layer
fp32 hidden states, with identical greedy token ids.  Here "within 1e-3 relative" is
checked per layer output as max|gpu - oracle| <= 1e-3 * max|oracle| (an element-wise
ratio is meaningless at values near zero).  Int8 KV bytes are checked exactly where the
fp32 values they quantise are the reference's: without the split matvec and the
matrix-core prompt GEMMs the first layer's K and V come from the exact QKV products of the
unchanged inputs.  With either their scales may differ in the last bits and a value on a
rounding boundary by one step.
"""
import ctypes as C

import numpy as np
import pytest

import oracle
from conftest import kv_views, prefill_kv, ptr, rope_tables

pytestmark = pytest.mark.gpu

TOL = 1e-3


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)


@pytest.fixture(scope="module")
def jy():
    import jieyu_amd
    if jieyu_amd.device_count() < 1:
        pytest.fail("no HIP device visible")
    return jieyu_amd


MODELS = {
    "llama-like": dict(name="llama3-8b", num_layers=2, hidden=512, num_heads=8, num_kv_heads=2, head_dim=64,
                       intermediate=1408, vocab_size=3000),
    "qwen-like": dict(name="qwen2.5-0.5b", num_layers=2, hidden=896, num_heads=14, num_kv_heads=2, head_dim=64,
                      intermediate=4864, vocab_size=5000),
    "hd128": dict(name="qwen2.5-7b", num_layers=2, hidden=1024, num_heads=8, num_kv_heads=2, head_dim=128,
                  intermediate=2048, vocab_size=2000),
    "llama-hd128-g4": dict(name="llama3-8b", num_layers=2, hidden=2048, num_heads=16, num_kv_heads=4, head_dim=128,
                           intermediate=3072, vocab_size=4000),
}
# the other query heads per kv head the attention slices specialise on (1, 2 and a full 8
# at both head sizes; the models above have 4 and 7): forward_cached only (per-layer
# tolerance)
HEAD_GROUPS = {
    "mha-hd64": dict(name="llama3-8b", num_layers=2, hidden=256, num_heads=4, num_kv_heads=4, head_dim=64,
                     intermediate=768, vocab_size=1500),
    "mha-hd128": dict(name="llama3-8b", num_layers=2, hidden=512, num_heads=4, num_kv_heads=4, head_dim=128,
                      intermediate=1024, vocab_size=1500),
    "g2-hd64": dict(name="qwen2.5-0.5b", num_layers=2, hidden=512, num_heads=8, num_kv_heads=4, head_dim=64,
                    intermediate=1024, vocab_size=1500),
    "g2-hd128-bias": dict(name="qwen2.5-7b", num_layers=2, hidden=1024, num_heads=8, num_kv_heads=4, head_dim=128,
                          intermediate=2048, vocab_size=2000),
    "g8-hd128": dict(name="llama3-8b", num_layers=2, hidden=2048, num_heads=16, num_kv_heads=2, head_dim=128,
                     intermediate=2048, vocab_size=2000),
}


def make(oracle_lib, key):
    from jieyu_amd.model import Synth, synth_config
    spec = dict(MODELS[key] if key in MODELS else HEAD_GROUPS[key])
    name = spec.pop("name")
    return Synth(oracle_lib, synth_config(name, **spec))


def rel_err(got, want):
    return float(np.abs(got - want).max() / max(np.abs(want).max(), 1e-30))


def layer_errs(got, want):
    return [rel_err(got[l], want[l]) for l in range(got.shape[0])]


# the isolated-kernel workload (int8 ~ U[-127,127], scales U(0.001,0.01), x ~ N(0,1), seed 1)
# and ragged shapes: rows not a multiple of 4, K with padded chunks (896: 28 blocks)
@pytest.mark.parametrize("rows,cols", [(4096, 4096), (14336, 4096), (4096, 14336), (13, 96), (517, 896),
                                       (300, 3584), (40, 18944), (1000, 4864)])
def test_split_matvec_within_tolerance(jy, oracle_lib, rows, cols):
    """The split-dot matvec against the oracle's dot_row_avx2 order: within a bound of the
    float64 dot that only a reordered fp32 sum meets (a dropped block or a wrong scale
    misses it by orders of magnitude)."""
    from conftest import q8_random_uniform
    say(f"split matvec {rows}x{cols}")
    w = q8_random_uniform(oracle_lib, rows, cols, seed=1)
    x = np.zeros(cols, np.float32)
    oracle_lib.jysyn_normal_fill(1, 13, 1.0, ptr(x), cols)
    ref = np.zeros(rows, np.float32)
    oracle_lib.jyo_matmul_q8(ptr(x), ptr(w), ptr(ref), 1, rows, cols)
    m = jy.Q8Matrix(w, rows, cols)
    m.set_mode(jy.MODE_SPLIT_MV)
    y = m.matvec(x)
    m.close()
    q = w.reshape(rows, cols // 32, 34)
    d = q[:, :, :2].copy().view(np.float16).astype(np.float64)[:, :, 0]
    wf = (q[:, :, 2:].view(np.int8).astype(np.float64) * d[:, :, None]).reshape(rows, cols)
    exact = wf @ x.astype(np.float64)
    bound = 1e-5 * (np.abs(wf) @ np.abs(x.astype(np.float64)))
    assert np.all(np.abs(y - exact) <= bound)
    assert rel_err(y, ref) <= TOL


def dequant(w, rows, cols):
    q = w.reshape(rows, cols // 32, 34)
    d = q[:, :, :2].copy().view(np.float16).astype(np.float64)[:, :, 0]
    return (q[:, :, 2:].view(np.int8).astype(np.float64) * d[:, :, None]).reshape(rows, cols)


# prompt GEMMs: ragged token counts (not multiples of the 128-row tile), rows not multiples of
# 16, blocks not multiples of 4 (1184 = 37 blocks), the benchmark's 4096 x 4096 at 1024 tokens
# (the narrow tile), and enough column tiles for the wide tile (1000 x 8200: 520 workgroups);
# token counts either side of a workgroup's 64 rows and of the 128-row padding, on grids
# split over K (1000 x 896: 3 slices; 2048 x 4096: up to 8), and either side of the narrow /
# wide switch (8200 x 320 at 896 and 897 tokens: 896 and 1024 padded rows) and past it
# (1025); activation rows spread over 10^-3 .. 10^3 with one zero row
@pytest.mark.parametrize("m,rows,cols", [(2, 13, 96), (37, 300, 1184), (200, 517, 896), (130, 1000, 4864),
                                         (1024, 4096, 4096), (1000, 8200, 320),
                                         (3, 1000, 896), (63, 1000, 896), (64, 1000, 896), (65, 1000, 896),
                                         (127, 2048, 4096), (128, 2048, 4096), (129, 2048, 4096),
                                         (257, 2048, 4096), (896, 8200, 320), (897, 8200, 320),
                                         (1025, 8200, 320)])
def test_mfma_gemm_within_tolerance(jy, oracle_lib, m, rows, cols):
    """The matrix-core prompt GEMM (fp16 high/low split of the activations, fp16 weights,
    fp32 block sums times the block scales) within 1e-5 of sum |a| |w| of the float64
    product, element by element; the exact tiles bit-equal to the oracle's matmul."""
    from conftest import q8_random_uniform
    say(f"mfma gemm m={m} {rows}x{cols}")
    w = q8_random_uniform(oracle_lib, rows, cols, seed=3)
    A = np.zeros((m, cols), np.float32)
    oracle_lib.jysyn_normal_fill(3, 17, 1.0, ptr(A), A.size)
    A *= (10.0 ** (np.arange(m) % 7 - 3)).astype(np.float32)[:, None]
    A[m // 2] = 0.0
    M = jy.Q8Matrix(w, rows, cols)
    M.set_mode(jy.MODE_MFMA_PREFILL)
    got = M.gemm(A)
    M.set_mode(jy.MODE_EXACT)
    tiles = M.gemm(A) if m * rows * cols <= 1 << 28 else None
    M.close()
    wf = dequant(w, rows, cols)
    A64 = A.astype(np.float64)
    exact = A64 @ wf.T
    bound = 1e-5 * (np.abs(A64) @ np.abs(wf).T)
    assert np.all(np.abs(got - exact) <= bound), f"worst excess {np.max(np.abs(got - exact) - bound):.3g}"
    assert np.all(got[m // 2] == 0.0)
    if tiles is not None:
        ref = np.zeros((m, rows), np.float32)
        oracle_lib.jyo_matmul_q8(ptr(A), ptr(w), ptr(ref), m, rows, cols)
        assert np.array_equal(tiles.view(np.uint32), ref.view(np.uint32))


MODES = {"SPLIT_ATTN": 1, "SPLIT_MV": 2, "MFMA_PREFILL": 4, "FAST": 7, "PERSIST": 7 | 8}


@pytest.mark.parametrize("mode_name", list(MODES))
@pytest.mark.parametrize("key", list(MODELS) + list(HEAD_GROUPS))
def test_forward_cached_within_tolerance(jy, oracle_lib, key, mode_name):
    """A prompt chunk then decode steps through forward_cached: every layer's output within
    1e-3 of the oracle's, the first layer's int8 K/V bytes equal to the oracle's."""
    say(f"forward_cached {key} mode {mode_name}")
    s = make(oracle_lib, key)
    d = s.desc
    L, H, nkv, hd = d.num_layers, d.hidden, d.num_kv_heads, d.head_dim
    max_seq = 48
    cos, sin = rope_tables(oracle_lib, max_seq, hd, d.rope_theta)
    okv = oracle.JyoKV()
    assert oracle_lib.jyo_kv_init(C.byref(okv), L, max_seq, nkv, hd) == 0
    g = jy.GpuModel(d, max_seq)
    g.mode = MODES[mode_name]
    kv = g.kv(max_seq)
    rng = np.random.default_rng(7)
    start = 0
    worst = 0.0
    for seq in (9, 1, 1, 1, 1, 3, 1, 1):
        X = rng.standard_normal((seq, H)).astype(np.float32)
        Xo = X.copy()
        lo = np.zeros((L, seq, H), np.float32)
        assert oracle_lib.jyo_forward_cached(C.byref(d), ptr(Xo), ptr(cos), ptr(sin), seq, start, C.byref(okv),
                                             ptr(lo)) == 0
        Xg, log = g.forward_cached(kv, X, start, layer_out=True)
        errs = layer_errs(log, lo) + [rel_err(Xg, Xo)]
        worst = max(worst, max(errs))
        assert max(errs) <= TOL, f"seq={seq} start={start}: relative errors {errs}"
        start += seq
    ok8, ov8, oks, ovs = kv_views(okv, L, max_seq, nkv, hd)
    k, ks, v, vs = kv.read(0, 0, start)
    if not g.mode & (jy.MODE_SPLIT_MV | jy.MODE_MFMA_PREFILL):
        assert np.array_equal(k, ok8[0, :start]) and np.array_equal(v, ov8[0, :start])
        assert np.array_equal(ks, oks[0, :start]) and np.array_equal(vs, ovs[0, :start])
    else:
        for a8, b8 in ((k, ok8[0, :start]), (v, ov8[0, :start])):
            diff = np.abs(a8.astype(np.int32) - b8.astype(np.int32))
            assert diff.max() <= 1 and np.count_nonzero(diff) <= max(2, diff.size // 1000)
        for a_s, b_s in ((ks, oks[0, :start]), (vs, ovs[0, :start])):
            assert np.all(np.abs(a_s - b_s) <= 1e-5 * np.abs(b_s))
    say(f"  worst relative error {worst:.3g}")
    oracle_lib.jyo_kv_free(C.byref(okv))
    kv.close()
    g.close()
    s.close()


@pytest.mark.parametrize("mode_name", ["FAST", "PERSIST"])
@pytest.mark.parametrize("key", list(MODELS))
def test_generate_fast_ids_match_oracle(jy, oracle_lib, key, mode_name):
    """Greedy ids of a whole generation in the tolerance modes equal the oracle's."""
    say(f"generate {key} in MODE_{mode_name}")
    s = make(oracle_lib, key)
    d = s.desc
    prompt = np.zeros(13, np.int32)
    oracle_lib.jysyn_uniform_int_fill(5, 99, 0, d.vocab_size - 1, ptr(prompt), len(prompt))
    max_seq, max_new = 80, 40
    cos, sin = rope_tables(oracle_lib, max_seq, d.head_dim, d.rope_theta)
    ref = np.zeros(max_seq + 1, np.int32)
    n = oracle_lib.jyo_generate(C.byref(d), ptr(prompt), len(prompt), None, 0, ptr(cos), ptr(sin), max_seq, max_new,
                                0.0, 1.0, ptr(ref), None, None)
    g = jy.GpuModel(d, max_seq)
    g.mode = MODES[mode_name]
    ids, _ = g.generate(prompt, max_new)
    g.close()
    s.close()
    assert np.array_equal(ids, ref[:n]), f"gpu {ids[len(prompt):]} vs oracle {ref[len(prompt):n]}"


@pytest.mark.parametrize("key", ["llama-like", "qwen-like"])
def test_fast_penalty_and_eos(jy, oracle_lib, key):
    """The tolerance mode with the repetition penalty applied on the device (greedy, rp 1.3)
    and with an EOS id that ends the generation early: ids equal to the oracle's."""
    say(f"fast mode: repetition penalty and EOS ({key})")
    s = make(oracle_lib, key)
    d = s.desc
    prompt = np.arange(5, 14, dtype=np.int32)
    max_seq = 64
    cos, sin = rope_tables(oracle_lib, max_seq, d.head_dim, d.rope_theta)

    def ref(max_new, rp=1.0, eos=None):
        out = np.zeros(max_seq + 1, np.int32)
        eos_a = None if eos is None else np.asarray(eos, np.int32)
        n = oracle_lib.jyo_generate(C.byref(d), ptr(prompt), len(prompt), ptr(eos_a), 0 if eos is None else len(eos),
                                    ptr(cos), ptr(sin), max_seq, max_new, 0.0, rp, ptr(out), None, None)
        return out[:n].copy()

    g = jy.GpuModel(d, max_seq)
    g.mode = MODES["FAST"]
    want = ref(20, rp=1.3)
    ids, _ = g.generate(prompt, 20, repetition_penalty=1.3)
    assert np.array_equal(ids, want), f"rp 1.3: gpu {ids[len(prompt):]} vs oracle {want[len(prompt):]}"
    eos_tok = int(ref(30)[len(prompt) + 5])
    want = ref(30, eos=[eos_tok])
    ids, _ = g.generate(prompt, 30, eos=[eos_tok])
    assert np.array_equal(ids, want), f"eos {eos_tok}: gpu {ids[len(prompt):]} vs oracle {want[len(prompt):]}"
    assert len(want) < len(prompt) + 30
    g.close()
    s.close()


def prefill_cache(oracle_lib, d, pre, max_seq, kv):
    return prefill_kv(oracle_lib, d, pre, max_seq, kv)


# the whole-range kernel up to 1024 keys (40 .. 1023: most of its 8 waves idle, one to
# four steps per wave, the last step partial or full), the slices and the merge past it:
# 128-key slices of 4 waves (3000, 5000), 256-key slices of 8 waves (20000), and past 256
# such slices two steps for some waves (70000)
@pytest.mark.parametrize("pre", [40, 700, 1023, 3000, 5000, 20000, 70000])
def test_split_attention_long_context(jy, oracle_lib, pre):
    """Decode steps over a cache pre-filled with packed N(0,1) K/V: hidden states within
    tolerance, the appended K/V bytes of the first layer equal to the oracle's."""
    say(f"split attention over a {pre}-position cache")
    s = make(oracle_lib, "hd128")
    d = s.desc
    L, H, nkv, hd = d.num_layers, d.hidden, d.num_kv_heads, d.head_dim
    max_seq = pre + 8
    cos, sin = rope_tables(oracle_lib, max_seq, hd, d.rope_theta)
    g = jy.GpuModel(d, max_seq)
    g.mode = jy.MODE_SPLIT_ATTN
    kv = g.kv(max_seq)
    okv = prefill_cache(oracle_lib, d, pre, max_seq, kv)
    rng = np.random.default_rng(4)
    for i in range(4):
        X = rng.standard_normal((1, H)).astype(np.float32)
        Xo = X.copy()
        lo = np.zeros((L, 1, H), np.float32)
        assert oracle_lib.jyo_forward_cached(C.byref(d), ptr(Xo), ptr(cos), ptr(sin), 1, pre + i, C.byref(okv),
                                             ptr(lo)) == 0
        Xg, log = g.forward_cached(kv, X, pre + i, layer_out=True)
        errs = layer_errs(log, lo) + [rel_err(Xg, Xo)]
        assert max(errs) <= TOL, f"step {i}: relative errors {errs}"
    ok8, ov8, _, _ = kv_views(okv, L, max_seq, nkv, hd)
    k, _, v, _ = kv.read(0, pre, 4)
    assert np.array_equal(k, ok8[0, pre:pre + 4]) and np.array_equal(v, ov8[0, pre:pre + 4])
    oracle_lib.jyo_kv_free(C.byref(okv))
    kv.close()
    g.close()
    s.close()


# (1490, 12) in a 4096-position cache: the session's slices are sized for the capacity (32
# of them), so at 1491..1502 keys each holds 48 and the last one 3..14: the slice before it
# ends in a partial step whose keys past its end include the token's own (masked there;
# only the last slice takes the token's key from its copy)
@pytest.mark.parametrize("mode_name", ["FAST", "PERSIST"])
@pytest.mark.parametrize("pre,n_new,cap", [(700, 24, 0), (1018, 12, 0), (1490, 12, 4096), (6000, 12, 0)])
def test_fast_resume_over_long_cache(jy, oracle_lib, pre, n_new, cap, mode_name):
    """The graph-replayed decode step in MODE_FAST over a pre-filled cache: greedy ids equal
    the oracle driven token by token (embedding row, forward_cached, lm_head, first maximum)."""
    say(f"MODE_FAST session resume over a {pre}-position cache (capacity {cap or pre + n_new + 8})")
    s = make(oracle_lib, "hd128")
    d = s.desc
    H, V, hd = d.hidden, d.vocab_size, d.head_dim
    max_seq = cap or pre + n_new + 8
    cos, sin = rope_tables(oracle_lib, max_seq, hd, d.rope_theta)
    g = jy.GpuModel(d, max_seq)
    g.mode = MODES[mode_name]
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


def test_mode_switch_recaptures(jy, oracle_lib):
    """A session's decode graphs follow a mode change between steps; an exact-mode run of the
    same prompt afterwards is still bit-identical to the oracle."""
    say("mode switch within a session")
    s = make(oracle_lib, "llama-like")
    d = s.desc
    prompt = np.arange(30, 41, dtype=np.int32)
    cos, sin = rope_tables(oracle_lib, 64, d.head_dim, d.rope_theta)
    ref = np.zeros(65, np.int32)
    logits = np.zeros(d.vocab_size, np.float32)
    n = oracle_lib.jyo_generate(C.byref(d), ptr(prompt), len(prompt), None, 0, ptr(cos), ptr(sin), 64, 30, 0.0,
                                1.0, ptr(ref), None, ptr(logits))
    g = jy.GpuModel(d, 64)
    ss = g.session(prompt, 30)
    ss.step(5)
    g.mode = jy.MODE_SPLIT_ATTN | jy.MODE_SPLIT_MV | jy.MODE_PERSIST
    ss.step(10)
    g.mode = jy.MODE_EXACT
    ss.step(30)
    assert np.array_equal(ss.ids(), ref[:n])
    ss.close()
    ids, _, lg = g.generate(prompt, 30, want_logits=True)
    assert np.array_equal(ids, ref[:n]) and np.array_equal(lg.view(np.uint32), logits.view(np.uint32))
    with pytest.raises(jy.JyError):
        g.mode = 64
    g.close()
    s.close()


@pytest.mark.parametrize("key,seq", [("llama-like", 9), ("llama-like", 37), ("qwen-like", 64), ("hd128", 130)])
def test_deferred_split_sums_bit_equal(jy, oracle_lib, key, seq):
    """Prompt GEMMs whose small grids run split over K leave their sums to the next kernel
    (rope_pack adds the QKV partials, the RMSNorm + split adds a residual product's into X).
    A pass that copies every layer's output out adds them with the sum kernel instead, before
    each copy: the final states and the K/V cache must be bit-identical either way, at prompt
    lengths below, across and above the 128-row tile."""
    say(f"deferred split-K sums {key} seq={seq}")
    s = make(oracle_lib, key)
    d = s.desc
    L, H, nkv, hd = d.num_layers, d.hidden, d.num_kv_heads, d.head_dim
    g = jy.GpuModel(d, seq + 8)
    g.mode = MODES["FAST"]
    X = np.random.default_rng(seq).standard_normal((seq, H)).astype(np.float32)
    kv_a, kv_b = g.kv(seq + 8), g.kv(seq + 8)
    ya = g.forward_cached(kv_a, X, 0)
    yb, lo = g.forward_cached(kv_b, X, 0, layer_out=True)
    assert np.array_equal(ya.view(np.uint32), yb.view(np.uint32))
    for layer in range(L):
        a, b = kv_a.read(layer, 0, seq), kv_b.read(layer, 0, seq)
        assert all(np.array_equal(np.asarray(u).view(np.uint8), np.asarray(v).view(np.uint8)) for u, v in zip(a, b))
    assert np.all(np.isfinite(lo))
    kv_a.close()
    kv_b.close()
    g.close()
    s.close()
