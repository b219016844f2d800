"""Write the golden fixtures of tests/golden/ from jieyu's own code.

Runs the reference's decode-path functions, compiled from the reference sources
by oracle/Makefile (`make -C oracle ref` -> oracle/_ref/libjyref.so), on seeded
inputs and stores inputs and outputs as small .npz / .json files.  Only data is
committed; the reference source and library are not.

    python tests/golden/make_golden.py

Inputs come from the repository's deterministic generator (include/jieyu_synth.h)
or from numpy's PCG64 with fixed seeds; every case records what it was.
"""
import ctypes as C
import json
import os
import platform
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

sys.path.insert(0, HERE)
import oracle  # noqa: E402
from jieyu_amd.model import Synth, synth_config  # noqa: E402
from kat_models import bind_model_desc, bind_test_model, demo_model_desc  # noqa: E402


def ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def q8_normal(olib, rows, cols, seed, std=0.02):
    x = np.zeros(rows * cols, np.float32)
    olib.jysyn_normal_fill(seed, 7, std, ptr(x), x.size)
    out = np.zeros(rows * (cols // 32) * 34, np.uint8)
    olib.jysyn_quantize_q8_0(ptr(x), ptr(out), x.size)
    return out


def q8_uniform(olib, rows, cols, seed):
    nb = rows * (cols // 32)
    q = np.zeros(nb * 32, np.int32)
    olib.jysyn_uniform_int_fill(seed, 11, -127, 127, ptr(q), q.size)
    d = np.zeros(nb, np.float32)
    olib.jysyn_uniform_fill(seed, 12, 0.001, 0.01, ptr(d), d.size)
    blk = np.zeros((nb, 34), np.uint8)
    blk[:, 0:2] = d.astype(np.float16).view(np.uint8).reshape(nb, 2)
    blk[:, 2:] = q.astype(np.int8).view(np.uint8).reshape(nb, 32)
    return blk.reshape(-1)


def rope_tables(ref, max_seq, hd, theta):
    c = np.zeros(max_seq * hd // 2, np.float32)
    s = np.zeros_like(c)
    ref.jyref_rope_table(max_seq, hd, theta, ptr(c), ptr(s))
    return c, s


def kernels(ref, olib):
    rng = np.random.default_rng(20261201)
    out = {}
    # Q8_0 matvec (decode, m == 1) and the generic m > 1 path
    for name, (m, n, k, src) in {
        "q8_m1_100x896": (1, 100, 896, "normal"),
        "q8_m1_37x4864": (1, 37, 4864, "normal"),
        "q8_m1_16x14336": (1, 16, 14336, "normal"),
        "q8_m1_isolated_4096x4096_rows0_15": (1, 16, 4096, "uniform"),
        "q8_m5_40x512": (5, 40, 512, "normal"),
        "q8_m17_24x256": (17, 24, 256, "normal"),
    }.items():
        w = q8_normal(olib, n, k, seed=n + k) if src == "normal" else q8_uniform(olib, n, k, seed=1)
        if src == "uniform":
            a = np.zeros(k, np.float32)
            olib.jysyn_normal_fill(1, 13, 1.0, ptr(a), k)
            a = a.reshape(1, k)
        else:
            a = rng.standard_normal((m, k)).astype(np.float32)
        c = np.zeros((m, n), np.float32)
        ref.jyref_matmul_q8(ptr(a), ptr(w), ptr(c), m, n, k)
        out[name + ".w"], out[name + ".a"], out[name + ".c"] = w, a, c
    # f32 matmul, B = [k][n] (includes the n % 8 tail)
    for name, (m, n, k) in {"f32_1x12x8": (1, 12, 8), "f32_2x4x8": (2, 4, 8), "f32_5x136x64": (5, 136, 64),
                            "f32_1x200x512": (1, 200, 512)}.items():
        A = rng.standard_normal((m, k)).astype(np.float32)
        B = rng.standard_normal((k, n)).astype(np.float32)
        Cm = np.zeros((m, n), np.float32)
        ref.jyref_matmul_f32(m, n, k, ptr(A), ptr(B), ptr(Cm))
        out[name + ".A"], out[name + ".B"], out[name + ".C"] = A, B, Cm
    # rmsnorm, eps 1e-5 (includes the 8-wide remainder and scalar tails)
    for n in (8, 20, 24, 512, 896, 3584, 4096):
        x = rng.standard_normal(n).astype(np.float32)
        w = (1.0 + 0.02 * rng.standard_normal(n)).astype(np.float32)
        y = np.zeros(n, np.float32)
        ref.jyref_rmsnorm(ptr(x.copy()), ptr(y), ptr(w), n, 1e-5)
        out[f"rms_{n}.x"], out[f"rms_{n}.w"], out[f"rms_{n}.y"] = x, w, y
    # RoPE table + rotation (full groups of 8 pairs and remainder pairs)
    for (ms, hd, theta) in ((40, 128, 500000.0), (64, 64, 1000000.0), (8, 4, 10000.0), (12, 6, 10000.0)):
        c, s = rope_tables(ref, ms, hd, theta)
        key = f"rope_hd{hd}"
        out[key + ".cos"], out[key + ".sin"] = c, s
        out[key + ".meta"] = np.array([ms, hd, theta], np.float64)
        for (seq, sp, nh) in ((1, ms - 1, 3), (5, 2, 2)):
            q = rng.standard_normal((seq, nh, hd)).astype(np.float32)
            y = q.copy()
            ref.jyref_rope(ptr(y), seq, sp, nh, hd, ptr(c), ptr(s))
            out[f"{key}_seq{seq}.q"], out[f"{key}_seq{seq}.y"] = q, y
            out[f"{key}_seq{seq}.meta"] = np.array([seq, sp, nh], np.int64)
    # SiLU (vector body and libm tail)
    for n in (8, 13, 4864):
        x = (3.0 * rng.standard_normal(n)).astype(np.float32)
        x[:6] = [0.0, -0.0, 90.0, -90.0, 1e-30, -100.0]
        y = np.zeros(n, np.float32)
        ref.jyref_silu(ptr(x.copy()), ptr(y), n)
        out[f"silu_{n}.x"], out[f"silu_{n}.y"] = x, y
    # kv_pack_q8: random rows, a zero row, exact .5 ties after scaling
    src = rng.standard_normal((3, 2, 16)).astype(np.float32)
    src[1, 0, :] = 0.0
    src[2, 1, :] = np.array([127, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5] * 2, np.float32)
    dst = np.zeros(src.size, np.int8)
    sc = np.zeros(6, np.float32)
    ref.jyref_kv_pack(ptr(src), ptr(dst), ptr(sc), 2, 16, 3)
    out["kvpack.src"], out["kvpack.dst"], out["kvpack.sc"] = src, dst, sc
    # attention_q8 (decode and prefill rows, GQA groups, hd 4/64/128)
    for (seq, sp, nh, nkv, hd, cap) in ((1, 0, 8, 2, 64, 40), (1, 37, 8, 2, 64, 40), (7, 0, 4, 1, 4, 8),
                                        (5, 10, 14, 2, 64, 20), (1, 200, 32, 8, 128, 210)):
        key = f"attn_{seq}_{sp}_{nh}_{nkv}_{hd}"
        kc = np.zeros(cap * nkv * hd, np.int8)
        kc[:sp * nkv * hd] = rng.integers(-127, 128, sp * nkv * hd)
        vc = np.zeros_like(kc)
        vc[:sp * nkv * hd] = rng.integers(-127, 128, sp * nkv * hd)
        ks = np.zeros(cap * nkv, np.float32)
        ks[:sp * nkv] = (rng.random(sp * nkv) * 0.05).astype(np.float32)
        vs = np.zeros_like(ks)
        vs[:sp * nkv] = (rng.random(sp * nkv) * 0.05).astype(np.float32)
        Q = rng.standard_normal((seq, nh, hd)).astype(np.float32)
        K = rng.standard_normal((seq, nkv, hd)).astype(np.float32)
        V = rng.standard_normal((seq, nkv, hd)).astype(np.float32)
        for nm, arr in (("kc", kc), ("vc", vc), ("ks", ks), ("vs", vs), ("Q", Q), ("K", K), ("V", V)):
            out[f"{key}.{nm}_in"] = arr.copy()
        o = np.zeros((seq, nh, hd), np.float32)
        rc = ref.jyref_attention(ptr(Q.copy()), ptr(K.copy()), ptr(V.copy()), ptr(o), seq, sp, nh, nkv, hd, ptr(kc),
                                 ptr(ks), ptr(vc), ptr(vs), cap)
        assert rc == 0
        out[f"{key}.out"], out[f"{key}.kc"], out[f"{key}.ks"] = o, kc, ks
        out[f"{key}.vc"], out[f"{key}.vs"] = vc, vs
        out[f"{key}.meta"] = np.array([seq, sp, nh, nkv, hd, cap], np.int64)
    return out


GEN_CASES = {
    # the tiny f32 configuration in full: 4 layers, d 512, 8/2 heads, FFN 1408, V 32000, seed 0
    "tiny-f32": dict(cfg=("tiny-f32", {}), prompt=16, new=128, max_seq=160),
    "qwen-like-small": dict(cfg=("qwen2.5-0.5b", dict(num_layers=2, vocab_size=5000)), prompt=11, new=24, max_seq=64),
    "llama-like-small": dict(cfg=("llama3-8b", dict(num_layers=2, hidden=512, num_heads=8, num_kv_heads=2,
                                                    head_dim=64, intermediate=1408, vocab_size=3000)),
                             prompt=9, new=24, max_seq=64),
    # Qwen2.5-0.5B shape in full (24 layers, tied embeddings, biases), short run
    "qwen2.5-0.5b-full": dict(cfg=("qwen2.5-0.5b", {}), prompt=16, new=16, max_seq=48),
}


def generate_cases(ref, olib):
    res = {}
    for name, case in GEN_CASES.items():
        cname, over = case["cfg"]
        cfg = synth_config(cname, **over)
        syn = Synth(olib, cfg)
        d = syn.desc
        prompt = np.zeros(case["prompt"], np.int32)
        olib.jysyn_uniform_int_fill(cfg.seed, 99, 0, d.vocab_size - 1, ptr(prompt), len(prompt))
        c, s = rope_tables(ref, case["max_seq"], d.head_dim, d.rope_theta)
        ids = np.zeros(case["max_seq"] + 1, np.int32)
        n = ref.jyref_generate(C.byref(d), ptr(prompt), len(prompt), None, 0, ptr(c), ptr(s), case["max_seq"],
                               case["new"], 0.0, 1.0, ptr(ids), None, None, 0)
        res[name] = dict(config=cname, overrides=over, prompt=prompt.tolist(), max_seq=case["max_seq"],
                         max_new=case["new"], ids=ids[:n].tolist())
        # sampling and repetition penalty on the small llama-like model
        if name == "llama-like-small":
            for (t, rp) in ((0.0, 1.3), (0.8, 1.0), (0.7, 1.1)):
                ids2 = np.zeros(case["max_seq"] + 1, np.int32)
                n2 = ref.jyref_generate(C.byref(d), ptr(prompt), len(prompt), None, 0, ptr(c), ptr(s),
                                        case["max_seq"], case["new"], t, rp, ptr(ids2), None, None, 0)
                res[f"{name}-T{t}-rp{rp}"] = dict(config=cname, overrides=over, prompt=prompt.tolist(),
                                                  max_seq=case["max_seq"], max_new=case["new"], temperature=t,
                                                  repetition_penalty=rp, ids=ids2[:n2].tolist())
        syn.close()
    return res


def main():
    if not oracle.ref_available():
        sys.exit("oracle/_ref/libjyref.so is missing: run `make -C oracle ref` where the reference tree exists")
    ref = oracle.load_ref()
    olib = oracle.load_oracle()
    isa = ref.jyref_init()
    meta = dict(reference_version=ref.jyref_version().decode(), isa_avx2=bool(isa & 1), isa_fma=bool(isa & 2),
                isa_avxvnni=bool(isa & 4), libc=" ".join(platform.libc_ver()), machine=platform.machine())
    k = kernels(ref, olib)
    np.savez_compressed(os.path.join(HERE, "kernels.npz"), **k)
    gen = generate_cases(ref, olib)
    # the reference's own known-answer model (check_bind_weights, text.h:737-843): pseudo weights,
    # prompts {1,2,3} and {5,6,7}, 3 greedy tokens, max_seq 8, f32, int8 KV cache
    bm = bind_test_model()
    desc, keep = bind_model_desc(bm)
    c, s = rope_tables(ref, 8, bm["hd"], 10000.0)
    kat = {}
    for prompt in ([1, 2, 3], [5, 6, 7]):
        p = np.array(prompt, np.int32)
        ids = np.zeros(9, np.int32)
        n = ref.jyref_generate(C.byref(desc), ptr(p), 3, None, 0, ptr(c), ptr(s), 8, 3, 0.0, 1.0, ptr(ids), None,
                               None, 0)
        kat[str(prompt)] = ids[:n].tolist()
    del keep
    ddesc, dkeep = demo_model_desc()
    c2, s2 = rope_tables(ref, 64, 32, 10000.0)
    p = np.array([256] + list(b"abcdefgh"), np.int32)  # BOS-prefixed byte ids of "abcdefgh"
    ids = np.zeros(65, np.int32)
    n = ref.jyref_generate(C.byref(ddesc), ptr(p), len(p), None, 0, ptr(c2), ptr(s2), 64, 16, 0.0, 1.0, ptr(ids),
                           None, None, 0)
    del dkeep
    gen["bind_test_kat"] = kat
    gen["demo_abcdefgh"] = dict(prompt=p.tolist(), ids=ids[:n].tolist())
    with open(os.path.join(HERE, "generate.json"), "w") as f:
        json.dump(dict(meta=meta, cases=gen), f, indent=1)
    print("wrote", os.path.join(HERE, "kernels.npz"), os.path.join(HERE, "generate.json"))


if __name__ == "__main__":
    main()
