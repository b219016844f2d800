"""The benchmark models at full size on the GPU, against the reference and the oracle.

* The benchmarks' own runs against jieyu's decode loop compiled from the reference sources
  (tests/golden/fullsize.json, tests/golden/make_fullsize_golden.py): Llama-3-8B, the
  1024-token prompt and 512 greedy tokens in a 4096-position cache; Qwen2.5-0.5B, the
  512-token prompt and 256 tokens; Qwen2.5-7B, 128 tokens after a cache pre-filled to 32768
  positions.  The exact mode must give every id.  The fast mode must give every id up to the
  first divergence recorded in tests/golden/fast_ties.json (none where every id was equal),
  and a divergence must be a near tie: the reference's own top-2 logit gap there at most twice
  the fast logits' largest deviation from the exact ones at that step (same prefix), and that
  deviation within LOGIT_TOL * max|logit| (2e-2; measured 6.4e-3 and 1.4e-2).  The ids after a tie
  follow a different prefix and are not compared.  The Llama-3-8B prompt's last row after
  the 1024-row prefill (the prompt GEMMs; on the matrix cores in the fast mode) against the
  reference's: bit-equal in the exact mode, within HIDDEN_BENCH relative in the fast mode.
* Shorter runs of the same three models against the reference (48 + 32, 512 + 64, 24 + 16
  tokens), by the same rules with the exact-mode logits in place of the reference's gap.
  (These random-init models amplify a change of rounding: per-layer deviations of ~1e-3
  compound over the stack and the positions through the int8 requantization of q / k / v.)
* Each layer on its own (the same input for the GPU's layer and the oracle's): a 16-row
  prompt and one decode row of Llama-3-8B through forward_cached, and at layers 0, 1, 15
  and 31 the oracle running that one layer on the GPU's input to it; bit-exact in the exact
  mode, within 1e-3 relative in the fast mode.
* Decode steps at the benchmark positions through forward_cached: Llama-3-8B over a cache
  filled to 1024 positions, Qwen2.5-7B over 32768; per-layer hidden states bit-exact with
  the oracle in the exact mode, within 1e-3 relative (max|gpu - oracle| <= 1e-3 *
  max|oracle| per layer) in the fast mode.
* The benchmark sessions' captured decode graphs pass the host-side checks (kernel nodes in
  one chain, every buffer they address live and unchanged) with the expected kernel count.
The pre-filled caches hold packed N(0, 1) K and V, as the long-context benchmark sets up.
"""
import ctypes as C
import json
import os

import numpy as np
import pytest

import oracle

from conftest import prefill_kv, ptr, rope_tables

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
TOL = 1e-3
# The fast logits' largest deviation from the exact ones at a divergence step, as a fraction
# of max|logit| (per-layer deviations of ~1e-3 compounded over 32 layers and the positions
# through the int8 K/V): measured 6.41e-3 on the Llama-3-8B benchmark run (generated token
# 112 after the 1024-token prompt) and 1.40e-2 on its 48-token run (generated token 2);
# the bound leaves 1.4x over the larger.
LOGIT_TOL = 2e-2
LOGIT_BENCH = LOGIT_TOL
# the last prompt row's relative error after the 32-layer, 1024-row fast prefill: measured
# 4.19e-3
HIDDEN_BENCH = 1e-2
MODES = {"exact": 0, "fast": 7}


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)


@pytest.fixture(scope="module")
def jy():
    import jieyu_amd
    if jieyu_amd.device_count() < 1:
        pytest.fail("no HIP device visible")
    return jieyu_amd


@pytest.fixture(scope="module")
def golden():
    with open(os.path.join(HERE, "golden", "fullsize.json")) as f:
        return json.load(f)["cases"]


def bits_equal(a, b):
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    return a.shape == b.shape and np.array_equal(a.view(np.uint8), b.view(np.uint8))


def rel_err(got, want):
    return float(np.abs(got - want).max() / max(np.abs(want).max(), 1e-30))


class Full:
    """One benchmark model, built on the host and uploaded once for a group of tests."""

    def __init__(self, jy, olib, name, max_seq):
        from jieyu_amd.model import Synth, synth_config
        say(f"building the {name} model")
        self.cfg = synth_config(name)
        self.syn = Synth(olib, self.cfg)
        self.d = self.syn.desc
        self.g = jy.GpuModel(self.d, max_seq)
        self.max_seq = max_seq

    def prompt(self, olib, n):
        p = np.zeros(n, np.int32)
        olib.jysyn_uniform_int_fill(self.cfg.seed, 99, 0, self.d.vocab_size - 1, ptr(p), n)
        return p

    def close(self):
        self.g.close()
        self.syn.close()


def check_near_tie(got, want, n0, exact_logits, fast_logits=None, name=None):
    """got (fast mode) against want (exact): equal, or equal up to index i where the step's
    fast logits (fast_logits(i), same prefix) are within LOGIT_TOL of the exact ones
    (exact_logits(i)) and the exact-logit gap of the two picks is within twice their largest
    difference.  Without fast logits the gap is bounded by LOGIT_TOL * max|logit|.  With a
    case name, i may not come before the tie recorded for it in fast_ties.json (and a case
    recorded with every id equal may not diverge)."""
    if got == want:
        return
    assert len(got) == len(want), f"lengths {len(got)} vs {len(want)}"
    i = next(k for k in range(len(got)) if got[k] != want[k])
    assert i >= n0, f"prompt ids differ at {i}"
    if name is not None:
        ties = fast_ties()
        assert not (name in ties and ties[name] is None), \
            f"{name}: fast mode diverged at generated token {i - n0}; every id was equal when this case was recorded"
        if ties.get(name) is not None:
            assert i - n0 >= ties[name], f"{name}: diverged at {i - n0}, before the recorded tie at {ties[name]}"
    lg = exact_logits(i)
    assert int(np.argmax(lg)) == want[i]
    scale = float(np.abs(lg).max())
    gap = float(lg[want[i]] - lg[got[i]])
    if fast_logits is not None:
        lf = fast_logits(i)
        assert int(np.argmax(lf)) == got[i]
        diff = float(np.abs(lf - lg).max())
        say(f"  fast mode: near tie at generated token {i - n0}: exact-logit gap {gap:.3g}, fast vs exact "
            f"logits max|diff| {diff:.3g} ({diff / scale:.2g} of max|logit|)")
        assert diff <= LOGIT_TOL * scale, f"fast logits off by {diff:.3g} at {i}"
        assert gap <= 2 * diff, f"fast mode picked {got[i]} at {i}: gap {gap:.3g} > 2 x {diff:.3g}"
    else:
        say(f"  fast mode: near tie at generated token {i - n0}: exact-logit gap {gap:.3g}")
        assert gap <= LOGIT_TOL * scale, f"fast mode picked {got[i]} at {i}: gap {gap:.3g}"


def check_generate(jy, olib, full, case, name=None):
    prompt = full.prompt(olib, case["prompt_len"])
    n0 = case["prompt_len"]
    assert prompt.tolist() == case["ids"][:n0]
    for mode in MODES:
        full.g.mode = MODES[mode]
        say(f"  {mode} mode: {n0}-token prompt, {case['max_new']} greedy tokens")
        ids, _ = full.g.generate(prompt, case["max_new"], max_seq=case["max_seq"])
        if mode == "exact":
            assert ids.tolist() == case["ids"], f"exact: gpu {ids[n0:].tolist()} vs reference {case['ids'][n0:]}"
            continue

        def logits_in(m):
            def at(i):
                full.g.mode = MODES[m]
                _, _, lg = full.g.generate(prompt, i - n0 + 1, max_seq=case["max_seq"], want_logits=True)
                return lg
            return at

        check_near_tie(ids.tolist(), case["ids"], n0, logits_in("exact"), logits_in(mode), name)


def check_decode_layers(jy, olib, full, pre, steps):
    """forward_cached steps at positions pre, pre+1, ... over a cache pre-filled to pre."""
    d = full.d
    L, H = d.num_layers, d.hidden
    cos, sin = rope_tables(olib, full.max_seq, d.head_dim, d.rope_theta)
    kv = full.g.kv(full.max_seq)
    okv = prefill_kv(olib, d, pre, full.max_seq, kv, one_draw=True)
    rng = np.random.default_rng(pre)
    xs = [rng.standard_normal((1, H)).astype(np.float32) for _ in range(steps)]
    want = []
    for i, X in enumerate(xs):
        Xo = X.copy()
        lo = np.zeros((L, 1, H), np.float32)
        assert olib.jyo_forward_cached(C.byref(d), ptr(Xo), ptr(cos), ptr(sin), 1, pre + i, C.byref(okv),
                                       ptr(lo)) == 0
        want.append((Xo, lo))
    for mode in MODES:
        full.g.mode = MODES[mode]
        kv.set_len(pre)
        for i, X in enumerate(xs):
            Xg, log = full.g.forward_cached(kv, X, pre + i, layer_out=True)
            Xo, lo = want[i]
            if mode == "exact":
                assert bits_equal(log, lo) and bits_equal(Xg, Xo), f"exact, step at {pre + i}"
            else:
                errs = [rel_err(log[l], lo[l]) for l in range(L)] + [rel_err(Xg, Xo)]
                assert max(errs) <= TOL, f"fast, step at {pre + i}: worst layer error {max(errs):.3g}"
                say(f"  fast mode at {pre + i}: worst per-layer relative error {max(errs):.3g}")
    olib.jyo_kv_free(C.byref(okv))
    kv.close()


def one_layer(desc, l):
    """A descriptor of layer l alone (the weights stay where they are)."""
    from jieyu_amd.model import LayerWeights, ModelDesc
    d1 = ModelDesc()
    C.memmove(C.byref(d1), C.byref(desc), C.sizeof(ModelDesc))
    d1.num_layers = 1
    d1.layers = C.cast(C.addressof(desc.layers.contents) + l * C.sizeof(LayerWeights), C.POINTER(LayerWeights))
    return d1


def check_layers_alone(jy, olib, full, layers, rows=16):
    d = full.d
    H = d.hidden
    cos, sin = rope_tables(olib, full.max_seq, d.head_dim, d.rope_theta)
    rng = np.random.default_rng(11)
    X = rng.standard_normal((rows, H)).astype(np.float32)
    x1 = rng.standard_normal((1, H)).astype(np.float32)
    for mode in MODES:
        full.g.mode = MODES[mode]
        kv = full.g.kv(full.max_seq)
        _, lo = full.g.forward_cached(kv, X, 0, layer_out=True)
        _, lo1 = full.g.forward_cached(kv, x1, rows, layer_out=True)
        kv.close()
        got = np.concatenate([lo, lo1], axis=1)  # [L][rows + 1][H]
        worst = 0.0
        for l in layers:
            inp = np.concatenate([X, x1]) if l == 0 else got[l - 1].copy()
            okv = oracle.JyoKV()
            assert olib.jyo_kv_init(C.byref(okv), 1, full.max_seq, d.num_kv_heads, d.head_dim) == 0
            d1 = one_layer(d, l)
            # the prompt rows as one chunk, then the decode row (the m = 1 path), as the GPU ran them
            out = np.zeros((1, rows + 1, H), np.float32)
            xa = np.ascontiguousarray(inp[:rows])
            xb = np.ascontiguousarray(inp[rows:])
            oa = np.zeros((1, rows, H), np.float32)
            ob = np.zeros((1, 1, H), np.float32)
            assert olib.jyo_forward_cached(C.byref(d1), ptr(xa), ptr(cos), ptr(sin), rows, 0, C.byref(okv),
                                           ptr(oa)) == 0
            assert olib.jyo_forward_cached(C.byref(d1), ptr(xb), ptr(cos), ptr(sin), 1, rows, C.byref(okv),
                                           ptr(ob)) == 0
            out[0, :rows], out[0, rows] = oa[0], ob[0, 0]
            olib.jyo_kv_free(C.byref(okv))
            if mode == "exact":
                assert bits_equal(got[l], out[0]), f"exact, layer {l}"
            else:
                err = rel_err(got[l], out[0])
                worst = max(worst, err)
                assert err <= TOL, f"fast, layer {l} alone: relative error {err:.3g}"
        say(f"  {mode} mode: layers {layers} alone, worst relative error {worst:.3g}")


def fast_ties():
    """The first fast-mode divergence measured per benchmark-length case (generated-token
    index; None where every id was equal): a later run may diverge there or later, never
    earlier, and a case recorded as equal may not diverge at all."""
    with open(os.path.join(HERE, "golden", "fast_ties.json")) as f:
        return json.load(f)["ties"]


def first_diff(got, want):
    return next((k for k in range(min(len(got), len(want))) if got[k] != want[k]), None)


def check_bench_tie(name, k, case, exact_logits, fast_logits, pick):
    """Fast mode diverged from the reference at generated token k (same prefix before it):
    it must not come earlier than the recorded tie, the reference's own top-2 gap there must
    be small (rel_gap from the golden), the fast logits must be within LOGIT_BENCH of the
    exact ones, and the gap no larger than twice their largest difference."""
    ties = fast_ties()
    assert not (name in ties and ties[name] is None), \
        f"{name}: fast mode diverged at generated token {k}; every id was equal when this case was recorded"
    known = ties.get(name)
    gap_rel = case["rel_gap"][k]
    lg, lf = exact_logits(), fast_logits()
    scale = float(np.abs(lg).max())
    diff = float(np.abs(lf - lg).max())
    say(f"  fast mode: {name} first differs at generated token {k} (recorded: {known}): reference top-2 gap "
        f"{gap_rel:.3g} of max|logit|, fast vs exact logits {diff / scale:.3g} of max|logit|")
    if known is not None:
        assert k >= known, f"{name}: fast mode diverged at generated token {k}, before the recorded tie at {known}"
    if pick is not None:
        assert int(np.argmax(lf)) == pick
    assert diff <= LOGIT_BENCH * scale, f"{name}: fast logits off by {diff / scale:.3g} of max|logit| at {k}"
    assert gap_rel * scale <= 2 * diff, f"{name}: gap {gap_rel:.3g} of max|logit| at {k} is no tie"


def check_bench_generate(jy, olib, full, name, case):
    """The benchmark's prompt and generation length: every id in the exact mode; in the fast
    mode every id up to a certified near tie (check_bench_tie)."""
    n0 = case["prompt_len"]
    prompt = full.prompt(olib, n0)
    assert prompt.tolist() == case["ids"][:n0]
    new = case["max_new"]
    for mode in MODES:
        full.g.mode = MODES[mode]
        say(f"  {mode} mode: {n0}-token prompt, {new} greedy tokens")
        ids, _ = full.g.generate(prompt, new, max_seq=case["max_seq"])
        got = ids[n0:].tolist()
        want = case["ids"][n0:]
        assert len(got) == len(want)
        if mode == "exact":
            k = first_diff(got, want)
            assert k is None, f"exact: generated token {k} is {got[k]}, the reference's {want[k]}"
            continue
        k = first_diff(got, want)
        if k is None:
            say(f"  fast mode: all {new} ids equal the reference's")
            continue

        def logits(m):
            def at():
                full.g.mode = MODES[m]
                _, _, lg = full.g.generate(prompt, k + 1, max_seq=case["max_seq"], want_logits=True)
                return lg
            return at

        check_bench_tie(name, k, case, logits("exact"), logits(mode), got[k])


def step_nodes(d, mode, keys):
    """Kernel launches of one captured decode step past the short-context threshold: the
    embedding row, per layer QKV, the attention (fast: slices + merge; exact past 768 keys:
    scores + softmax/PV), O, gate/up and down, then the lm_head and the pick."""
    assert (mode == "fast" and keys > 1024) or (mode == "exact" and keys > 768)
    return 1 + 6 * d.num_layers + 2


def check_session_graph(full, ids, n_pre, kv=None):
    """The session's captured decode graph passes the host-side checks (kernel nodes in one
    chain, launch shapes, every buffer it addresses live and unchanged since capture) and
    has the expected number of kernels, in both modes."""
    for mode in MODES:
        full.g.mode = MODES[mode]
        if kv is not None:
            kv.set_len(n_pre)
        s = full.g.session(ids, 4, max_seq=full.max_seq, kv=kv, resume=kv is not None)
        s.step(2)
        info = s.graph_info(0)
        assert info is not None, f"{mode}: no graph captured"
        nodes, edges, bufs = info
        want = step_nodes(full.d, mode, n_pre + 1)
        say(f"  {mode} mode: decode graph {nodes} kernel nodes, {edges} edges, {bufs} device buffers checked")
        assert nodes == want and edges == nodes - 1, f"{mode}: {nodes} nodes / {edges} edges, want {want}"
        assert bufs >= 9 * full.d.num_layers
        assert s.graph_info(1) is None  # the short-context graph is never needed here
        s.close()


class TestLlama3_8B:
    @pytest.fixture(scope="class")
    def full(self, jy, oracle_lib):
        f = Full(jy, oracle_lib, "llama3-8b", 4096)
        yield f
        f.close()

    def test_session_graph_checked(self, jy, oracle_lib, full):
        say("llama3-8b: the benchmark session's captured decode graph, host-side checks")
        check_session_graph(full, full.prompt(oracle_lib, 1024), 1024)

    def test_bench_generate_matches_reference(self, jy, oracle_lib, full, golden):
        say("llama3-8b: the benchmark's 1024-token prompt + 512 greedy tokens vs the reference")
        check_bench_generate(jy, oracle_lib, full, "llama3-8b-bench", golden["llama3-8b-bench"])

    def test_bench_prefill_last_row(self, jy, oracle_lib, full, golden):
        """The 1024-row prompt through the whole stack (the prompt GEMMs, on the matrix cores
        in the fast mode): the last row's final-normed state against the reference's, bit for
        bit in the exact mode, within HIDDEN_BENCH relative in the fast mode (the stack's
        compounded deviation); its lm_head pick is the reference's first token."""
        case = golden["llama3-8b-bench"]
        n0 = case["prompt_len"]
        with np.load(os.path.join(HERE, "golden", "fullsize_hidden.npz")) as z:
            want = z["llama3-8b-bench"]
        d = full.d
        prompt = full.prompt(oracle_lib, n0)
        X = np.zeros((n0, d.hidden), np.float32)
        for i, t in enumerate(prompt):
            oracle_lib.jyo_embed_row(C.byref(d.embed), int(t), d.hidden, ptr(X[i]))
        for mode in MODES:
            full.g.mode = MODES[mode]
            kv = full.g.kv(full.max_seq)
            out = full.g.forward_cached(kv, X, 0)
            kv.close()
            last = out[n0 - 1]
            if mode == "exact":
                assert bits_equal(last, want), f"exact: max abs diff {np.abs(last - want).max()}"
            else:
                err = rel_err(last, want)
                say(f"  fast mode: last prompt row after 32 layers, relative error {err:.3g}")
                assert err <= HIDDEN_BENCH, f"fast: last row relative error {err:.3g}"
            logits = np.zeros(d.vocab_size, np.float32)
            oracle_lib.jyo_matmul_w(C.byref(d.lm_head), 1, d.vocab_size, d.hidden, ptr(last), ptr(logits))
            pick = int(np.argmax(logits))
            if mode == "exact" or case["rel_gap"][0] > 2 * LOGIT_BENCH:
                assert pick == case["ids"][n0], f"{mode}: first token {pick} vs the reference's {case['ids'][n0]}"

    def test_generate_matches_reference(self, jy, oracle_lib, full, golden):
        say("llama3-8b: greedy ids vs the reference")
        check_generate(jy, oracle_lib, full, golden["llama3-8b-full"], "llama3-8b-full")

    def test_layers_alone(self, jy, oracle_lib, full):
        say("llama3-8b: layers 0, 1, 15, 31 alone (16 prompt rows + 1 decode row) vs the oracle")
        check_layers_alone(jy, oracle_lib, full, (0, 1, 15, 31))

    def test_decode_at_1024(self, jy, oracle_lib, full):
        say("llama3-8b: decode steps at 1024..1025 vs the oracle, per layer")
        check_decode_layers(jy, oracle_lib, full, 1024, 2)


class TestQwen05B:
    @pytest.fixture(scope="class")
    def full(self, jy, oracle_lib):
        f = Full(jy, oracle_lib, "qwen2.5-0.5b", 768)
        yield f
        f.close()

    def test_bench_generate_matches_reference(self, jy, oracle_lib, full, golden):
        say("qwen2.5-0.5b: the benchmark's 512-token prompt + 256 greedy tokens vs the reference")
        check_bench_generate(jy, oracle_lib, full, "qwen2.5-0.5b-bench", golden["qwen2.5-0.5b-bench"])

    def test_512_prompt_matches_reference(self, jy, oracle_lib, full, golden):
        say("qwen2.5-0.5b: 512-token prompt + 64 greedy tokens vs the reference")
        check_generate(jy, oracle_lib, full, golden["qwen2.5-0.5b-full-512"], "qwen2.5-0.5b-full-512")


class TestQwen7B:
    PRE = 32768

    @pytest.fixture(scope="class")
    def full(self, jy, oracle_lib):
        f = Full(jy, oracle_lib, "qwen2.5-7b", self.PRE + 136)
        yield f
        f.close()

    def test_generate_matches_reference(self, jy, oracle_lib, full, golden):
        say("qwen2.5-7b: greedy ids vs the reference")
        check_generate(jy, oracle_lib, full, golden["qwen2.5-7b-full"], "qwen2.5-7b-full")

    def test_session_graph_checked(self, jy, oracle_lib, full):
        say("qwen2.5-7b: the long-context session's captured decode graph, host-side checks")
        kv = full.g.kv(full.max_seq)
        okv = prefill_kv(oracle_lib, full.d, self.PRE, full.max_seq, kv, one_draw=True)
        oracle_lib.jyo_kv_free(C.byref(okv))
        check_session_graph(full, full.prompt(oracle_lib, self.PRE + 1), self.PRE, kv)
        kv.close()

    def test_decode_at_32768(self, jy, oracle_lib, full):
        say("qwen2.5-7b: decode steps at 32768..32769 vs the oracle, per layer")
        check_decode_layers(jy, oracle_lib, full, self.PRE, 2)

    def test_resume_after_32768(self, jy, oracle_lib, full, golden):
        """jyhip_session_resume over the pre-filled cache: the benchmark's 128 graph-replayed
        greedy steps give the reference's tokens (its forward_cached driven row by row over
        the same cache bytes, tests/golden/make_fullsize_golden.py): every id in the exact
        mode, up to a certified near tie in the fast mode."""
        case = golden["qwen2.5-7b-32768"]
        n_new = case["max_new"]
        say(f"qwen2.5-7b: {n_new} greedy tokens after a 32768-position cache vs the reference")
        assert case["prefilled"] == self.PRE
        d = full.d
        H, V = d.hidden, d.vocab_size
        kv = full.g.kv(full.max_seq)
        okv = prefill_kv(oracle_lib, d, self.PRE, full.max_seq, kv, one_draw=True)
        oracle_lib.jyo_kv_free(C.byref(okv))
        ids = full.prompt(oracle_lib, self.PRE + 1)
        assert ids[-1] == case["ids"][0]
        want = case["ids"][1:]

        def run(mode):
            full.g.mode = MODES[mode]
            kv.set_len(self.PRE)
            s = full.g.session(ids, n_new, max_seq=full.max_seq, kv=kv, resume=True)
            s.step(n_new)
            got = s.ids()[self.PRE + 1:].tolist()
            s.close()
            return got

        def logits_at(mode, toks):
            """forward_cached rows over the cache (the session's kernels), then the oracle's
            lm_head product on the final state: the logits after the prefix toks."""
            def at():
                full.g.mode = MODES[mode]
                kv.set_len(self.PRE)
                for j, t in enumerate(toks):
                    X = np.zeros((1, H), np.float32)
                    oracle_lib.jyo_embed_row(C.byref(d.embed), int(t), H, ptr(X))
                    X = full.g.forward_cached(kv, X, self.PRE + j)
                lg = np.zeros(V, np.float32)
                oracle_lib.jyo_matmul_w(C.byref(d.lm_head), 1, V, H, ptr(X), ptr(lg))
                return lg
            return at

        for mode in MODES:
            got = run(mode)
            assert len(got) == len(want), f"{mode}: {len(got)} tokens"
            k = first_diff(got, want)
            if mode == "exact":
                assert k is None, f"exact: generated token {k} is {got[k]}, the reference's {want[k]}"
            elif k is None:
                say(f"  fast mode: all {n_new} ids equal the reference's")
            else:
                prefix = [ids[-1]] + want[:k]
                check_bench_tie("qwen2.5-7b-32768", k, case, logits_at("exact", prefix), logits_at("fast", prefix),
                                None)
        kv.close()
