"""Write tests/golden/fullsize.json: greedy token ids of the full-size benchmark models
from jieyu's own decode loop, compiled from the reference sources by oracle/Makefile
(`make -C oracle ref` -> oracle/_ref/libjyref.so).

    python tests/golden/make_fullsize_golden.py [case ...]   # default: every case

With case names only those are (re)written; the other cases already in the file stay.

Models come from the repository's deterministic generator (include/jieyu_synth.h) with
the benchmark configurations of jieyu_amd.model.CONFIGS; prompts are the first ids of
the benchmark's prompt stream (jysyn_uniform_int_fill(seed, 99, 0, vocab - 1)).

Kinds of case:

* "generate": the reference's own generate() (generate.h:90-112) writes the ids.  The
  benchmark-length cases are also driven step by step through the reference's
  forward_cached (forward.h:47-96) and its lm_head product (matmul_w), which must give the
  same ids, and from that loop the file keeps, per generated token, the gap between the
  largest and the second-largest logit over max|logit| (`rel_gap`): a fast-mode check uses
  it to tell a near tie from a real error.  With `hidden` the last prompt row's state after
  the final RMSNorm (the row the first token's logits come from) goes to fullsize_hidden.npz.
* "driven": the same driven loop alone, its prompt through forward_cached in chunks of
  `chunk` rows.  The reference's m > 1 product (matmul_q.h:145-161) computes every output
  element from its own activation row in ascending k, and its attention packs a chunk's K/V
  into the int8 cache before any row reads it, so a prompt in chunks of m >= 2 rows gives
  the one-chunk result bit for bit; the chunks keep the activations cache-resident, where
  one 1024-row chunk re-streams 16 MB of activations per output column (hours per layer
  of the 8B shape).  The script checks that equivalence on the case's own model first: 64
  prompt rows as one chunk and as four chunks of 16, hidden states and K/V bit-equal.
* "resume": the cache first holds `prefilled` positions of N(0,1) K and V (one draw,
  packed by the reference's kv_pack_q8, written to every layer: the long-context
  benchmark's setup), then the prompt stream's id at `prefilled` is decoded greedily for
  `max_new` tokens, one forward_cached row at a time (generate_cached's loop body,
  generate.h:36-89, with the cache not restarted).
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

# name: dict(kind, config, prompt_len, max_new, max_seq[, prefilled][, hidden][, driven])
CASES = {
    # Llama-3-8B shape, Q8_0, seed 3: a 48-token prompt through the prompt GEMMs, 32 greedy tokens
    "llama3-8b-full": dict(kind="generate", config="llama3-8b", prompt_len=48, max_new=32, max_seq=96),
    # Qwen2.5-0.5B shape, Q8_0, tied head, biases: the benchmark's 512-token prompt, 64 greedy tokens
    "qwen2.5-0.5b-full-512": dict(kind="generate", config="qwen2.5-0.5b", prompt_len=512, max_new=64, max_seq=600),
    # Qwen2.5-7B shape, Q8_0, biases, theta 1e6: a 24-token prompt, 16 greedy tokens
    "qwen2.5-7b-full": dict(kind="generate", config="qwen2.5-7b", prompt_len=24, max_new=16, max_seq=48),
    # the Llama-3-8B benchmark: 1024-token prompt, 512 greedy tokens, a 4096-position cache
    "llama3-8b-bench": dict(kind="driven", config="llama3-8b", prompt_len=1024, max_new=512, max_seq=4096,
                            hidden=True, chunk=32),
    # the Qwen2.5-0.5B benchmark: 512-token prompt, 256 greedy tokens
    "qwen2.5-0.5b-bench": dict(kind="generate", config="qwen2.5-0.5b", prompt_len=512, max_new=256, max_seq=768,
                               driven=True),
    # the Qwen2.5-7B long-context benchmark: 128 greedy tokens after 32768 pre-filled positions
    "qwen2.5-7b-32768": dict(kind="resume", config="qwen2.5-7b", prompt_len=1, max_new=128, max_seq=32768 + 136,
                             prefilled=32768),
}


def ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def rel_gap(lg):
    """(largest - second largest logit) / max|logit|; the first maximum is the pick."""
    i = int(np.argmax(lg))
    rest = np.delete(lg, i)
    return float((lg[i] - rest.max()) / max(float(np.abs(lg).max()), 1e-30))


def embed(ref, d, tok, X):
    ref.jyref_wmat_row(C.byref(d.embed), int(tok), d.hidden, ptr(X))


def lm_head(ref, d, X):
    logits = np.zeros(d.vocab_size, np.float32)
    ref.jyref_matmul_w(C.byref(d.lm_head), 1, d.vocab_size, d.hidden, ptr(X), ptr(logits))
    return logits


def prefill_ref_kv(ref, olib, d, kvp, pre, max_seq):
    """positions [0, pre) of every layer: one N(0,1) draw each for K and V (seeds 9 / 1000
    and 9 / 1001), packed by the reference's kv_pack_q8."""
    L, nkv, hd = d.num_layers, d.num_kv_heads, d.head_dim
    packed = []
    for sub in (1000, 1001):
        f = np.zeros(pre * nkv * hd, np.float32)
        olib.jysyn_normal_fill(9, sub, 1.0, ptr(f), f.size)
        q = np.zeros(f.size, np.int8)
        s = np.zeros(pre * nkv, np.float32)
        ref.jyref_kv_pack(ptr(f), ptr(q), ptr(s), nkv, hd, pre)
        packed.append((q.reshape(pre, nkv, hd), s.reshape(pre, nkv)))
        del f
    views = []
    for fn, shape, ct in (("jyref_kv_k", (L, max_seq, nkv, hd), C.c_int8), ("jyref_kv_v", (L, max_seq, nkv, hd), C.c_int8),
                          ("jyref_kv_ks", (L, max_seq, nkv), C.c_float), ("jyref_kv_vs", (L, max_seq, nkv), C.c_float)):
        views.append(np.ctypeslib.as_array(C.cast(getattr(ref, fn)(kvp), C.POINTER(ct)), shape))
    k, v, ks, vs = views
    for l in range(L):
        k[l, :pre] = packed[0][0]
        ks[l, :pre] = packed[0][1]
        v[l, :pre] = packed[1][0]
        vs[l, :pre] = packed[1][1]
    ref.jyref_kv_set_len(kvp, pre)


def prefill(ref, d, X, start, cos, sin, kvp, chunk):
    """forward_cached over the rows of X from position `start`, in chunks of `chunk` rows
    (every chunk m >= 2 rows: the m > 1 product) or as one chunk (chunk = 0)."""
    n = X.shape[0]
    step = chunk or n
    for r0 in range(0, n, step):
        r1 = min(n, r0 + step)
        assert chunk == 0 or r1 - r0 >= 2, "a chunk of one row would take the m = 1 product"
        Xc = np.ascontiguousarray(X[r0:r1])
        assert ref.jyref_forward_cached(C.byref(d), ptr(cos), ptr(sin), ptr(Xc), r1 - r0, start + r0, kvp, None) == 0
        X[r0:r1] = Xc


def check_chunking(ref, d, prompt, cos, sin, max_seq, rows=64, chunk=16):
    """the first `rows` prompt rows as one chunk and in chunks: final states and K/V bit-equal"""
    H = d.hidden
    L, nkv, hd = d.num_layers, d.num_kv_heads, d.head_dim
    outs = []
    for ch in (0, chunk):
        X = np.zeros((rows, H), np.float32)
        for i, t in enumerate(prompt[:rows]):
            embed(ref, d, t, X[i])
        kvp = ref.jyref_kv_create(L, max_seq, nkv, hd)
        prefill(ref, d, X, 0, cos, sin, kvp, ch)
        k = np.ctypeslib.as_array(C.cast(ref.jyref_kv_k(kvp), C.POINTER(C.c_int8)), (L, max_seq, nkv, hd))[:, :rows].copy()
        v = np.ctypeslib.as_array(C.cast(ref.jyref_kv_v(kvp), C.POINTER(C.c_int8)), (L, max_seq, nkv, hd))[:, :rows].copy()
        ks = np.ctypeslib.as_array(C.cast(ref.jyref_kv_ks(kvp), C.POINTER(C.c_float)), (L, max_seq, nkv))[:, :rows].copy()
        ref.jyref_kv_free(kvp)
        outs.append((X, k, v, ks))
    (x0, k0, v0, s0), (x1, k1, v1, s1) = outs
    same = (np.array_equal(x0.view(np.uint32), x1.view(np.uint32)) and np.array_equal(k0, k1) and np.array_equal(v0, v1)
            and np.array_equal(s0.view(np.uint32), s1.view(np.uint32)))
    assert same, "a chunked prompt differs from the one-chunk prompt"
    print(f"    {rows} prompt rows: one chunk and chunks of {chunk} are bit-equal", flush=True)


def driven(ref, olib, d, prompt, start, n_new, max_seq, cos, sin, kvp, want_hidden=False, chunk=0):
    """greedy ids, per-step rel_gap and (optionally) the last prompt row's final state from
    forward_cached steps over the reference cache kvp, the prompt starting at `start`."""
    H = d.hidden
    n = len(prompt)
    X = np.zeros((n, H), np.float32)
    for i, t in enumerate(prompt):
        embed(ref, d, t, X[i])
    t0 = time.time()
    prefill(ref, d, X, start, cos, sin, kvp, chunk if n > 1 else 0)
    print(f"    prompt of {n} rows in {time.time() - t0:.1f} s", flush=True)
    hidden = X[n - 1].copy() if want_hidden else None
    ids, gaps = [], []
    x = np.ascontiguousarray(X[n - 1:n])
    pos = start + n
    for i in range(n_new):
        lg = lm_head(ref, d, x)
        tok = int(np.argmax(lg))
        ids.append(tok)
        gaps.append(rel_gap(lg))
        if i + 1 == n_new:
            break
        x = np.zeros((1, H), np.float32)
        embed(ref, d, tok, x[0])
        assert ref.jyref_forward_cached(C.byref(d), ptr(cos), ptr(sin), ptr(x), 1, pos, kvp, None) == 0
        pos += 1
        if i % 32 == 31:
            print(f"    {i + 1} of {n_new} driven steps", flush=True)
    return ids, gaps, hidden


def run_case(ref, olib, name, cs):
    cname, plen, new, max_seq = cs["config"], cs["prompt_len"], cs["max_new"], cs["max_seq"]
    t0 = time.time()
    cfg = synth_config(cname)
    syn = Synth(olib, cfg)
    d = syn.desc
    pre = cs.get("prefilled", 0)
    stream = np.zeros(pre + plen, np.int32)
    olib.jysyn_uniform_int_fill(cfg.seed, 99, 0, d.vocab_size - 1, ptr(stream), len(stream))
    prompt = stream[pre:]
    c = np.zeros(max_seq * d.head_dim // 2, np.float32)
    s = np.zeros_like(c)
    ref.jyref_rope_table(max_seq, d.head_dim, d.rope_theta, ptr(c), ptr(s))
    rec = dict(kind=cs["kind"], config=cname, prompt_len=plen, max_seq=max_seq, max_new=new)
    hidden = None
    if cs["kind"] == "driven":
        check_chunking(ref, d, prompt, c, s, max_seq)
        kvp = ref.jyref_kv_create(d.num_layers, max_seq, d.num_kv_heads, d.head_dim)
        got, gaps, hidden = driven(ref, olib, d, prompt, 0, new, max_seq, c, s, kvp, cs.get("hidden", False),
                                   cs["chunk"])
        ref.jyref_kv_free(kvp)
        rec["ids"] = prompt.tolist() + got
        rec["rel_gap"] = [round(g, 7) for g in gaps]
        rec["chunk"] = cs["chunk"]
    elif cs["kind"] == "generate":
        ids = np.zeros(max_seq + 1, np.int32)
        n = ref.jyref_generate(C.byref(d), ptr(prompt), plen, None, 0, ptr(c), ptr(s), max_seq, new, 0.0, 1.0,
                               ptr(ids), None, None, 0)
        rec["ids"] = ids[:n].tolist()
        print(f"  {name}: generate gave {n - plen} tokens in {time.time() - t0:.1f} s", flush=True)
        if cs.get("driven"):
            kvp = ref.jyref_kv_create(d.num_layers, max_seq, d.num_kv_heads, d.head_dim)
            got, gaps, hidden = driven(ref, olib, d, prompt, 0, new, max_seq, c, s, kvp, cs.get("hidden", False))
            ref.jyref_kv_free(kvp)
            assert got == rec["ids"][plen:], f"{name}: the driven loop's ids differ from generate()'s"
            rec["rel_gap"] = [round(g, 7) for g in gaps]
    else:
        kvp = ref.jyref_kv_create(d.num_layers, max_seq, d.num_kv_heads, d.head_dim)
        prefill_ref_kv(ref, olib, d, kvp, pre, max_seq)
        got, gaps, _ = driven(ref, olib, d, prompt, pre, new, max_seq, c, s, kvp)
        ref.jyref_kv_free(kvp)
        rec["prefilled"] = pre
        rec["ids"] = prompt.tolist() + got
        rec["rel_gap"] = [round(g, 7) for g in gaps]
    if "rel_gap" in rec:
        g = np.array(rec["rel_gap"])
        print(f"  {name}: smallest top-2 logit gap {g.min():.3g} of max|logit| at generated token {int(g.argmin())}",
              flush=True)
    syn.close()
    print(f"{name}: {new} tokens in {time.time() - t0:.1f} s", flush=True)
    return rec, hidden


def main():
    if not oracle.ref_available():
        sys.exit("oracle/_ref/libjyref.so is missing: run `make -C oracle ref` where the reference tree exists")
    names = sys.argv[1:] or list(CASES)
    for n in names:
        if n not in CASES:
            sys.exit(f"unknown case {n}; cases: {', '.join(CASES)}")
    ref = oracle.load_ref()
    olib = oracle.load_oracle()
    isa = ref.jyref_init()
    meta = dict(reference_version=ref.jyref_version().decode(), isa_avx2=bool(isa & 1), isa_fma=bool(isa & 2),
                isa_avxvnni=bool(isa & 4), libc=" ".join(platform.libc_ver()), machine=platform.machine(),
                threads=os.environ.get("OMP_NUM_THREADS", str(os.cpu_count())))
    path = os.path.join(HERE, "fullsize.json")
    hpath = os.path.join(HERE, "fullsize_hidden.npz")
    out = {}
    if os.path.exists(path):
        with open(path) as f:
            out = json.load(f)["cases"]
    hid = dict(np.load(hpath)) if os.path.exists(hpath) else {}
    for name in names:
        rec, hidden = run_case(ref, olib, name, CASES[name])
        out[name] = rec
        if hidden is not None:
            hid[name] = hidden
        with open(path, "w") as f:  # after every case: a long run keeps what it finished
            json.dump(dict(meta=meta, cases={k: out[k] for k in CASES if k in out}), f, indent=1)
        if hid:
            np.savez(hpath, **hid)
    print("wrote", path)


if __name__ == "__main__":
    main()
