"""Synthetic models and matrices in every weight type jieyu binds: f32, f16, Q8_0,
Q4_K, Q5_K, Q6_K (libs/model_libs/load_weights.h:26-35, libs/matmul_libs/matmul_q.h:15-45).

Quantized matrices are random blocks in GGML's layouts with scales chosen so the
weights stay near the 0.02 scale of the other synthetic models:
  Q8_0 (34 B):  fp16 d, 32 int8
  Q4_K (144 B): fp16 d, fp16 dmin, 12 B of 6-bit scales/mins, 128 B of nibbles
  Q5_K (176 B): fp16 d, fp16 dmin, 12 B scales/mins, 32 B high bits, 128 B nibbles
  Q6_K (210 B): 128 B low nibbles, 64 B high 2-bit pairs, 16 int8 scales, fp16 d
f32 / f16 matrices are [in][out] (matmul's B operand), quantized ones [out][in].
Test infrastructure: used by the golden script and the tests only.
"""
import ctypes as C

import numpy as np

from jieyu_amd.model import JY_F16, JY_F32, JY_Q4_K, JY_Q5_K, JY_Q6_K, JY_Q8_0, LayerWeights, ModelDesc, WMat

BLOCK = {JY_Q8_0: (32, 34), JY_Q4_K: (256, 144), JY_Q5_K: (256, 176), JY_Q6_K: (256, 210)}
NAMES = {JY_F32: "f32", JY_F16: "f16", JY_Q8_0: "q8_0", JY_Q4_K: "q4_K", JY_Q5_K: "q5_K", JY_Q6_K: "q6_K"}
SLOTS = ("Wq", "Wk", "Wv", "Wo", "W1", "W2", "W3")


def _f16(rng, n, lo, hi):
    return rng.uniform(lo, hi, n).astype(np.float16).view(np.uint8).reshape(n, 2)


def rand_blocks(rng, wtype, rows, cols):
    """rows x cols weights of a quantized type as raw blocks, uint8 [rows * cols/be * bb]"""
    be, bb = BLOCK[wtype]
    assert cols % be == 0
    nb = rows * (cols // be)
    b = rng.integers(0, 256, (nb, bb), dtype=np.uint8)
    if wtype == JY_Q8_0:
        b[:, 0:2] = _f16(rng, nb, 1e-4, 3e-4)
    elif wtype == JY_Q4_K:
        b[:, 0:2] = _f16(rng, nb, 2e-5, 6e-5)
        b[:, 2:4] = _f16(rng, nb, 1e-4, 4e-4)
    elif wtype == JY_Q5_K:
        b[:, 0:2] = _f16(rng, nb, 1e-5, 3e-5)
        b[:, 2:4] = _f16(rng, nb, 1e-4, 4e-4)
    elif wtype == JY_Q6_K:
        b[:, 208:210] = _f16(rng, nb, 4e-6, 1.2e-5)
    return b.reshape(-1)


def rand_matrix(rng, wtype, out_dim, in_dim, std=0.02):
    """one weight matrix in the layout its type is bound with"""
    if wtype == JY_F32:
        return (std * rng.standard_normal((in_dim, out_dim))).astype(np.float32)
    if wtype == JY_F16:
        return (std * rng.standard_normal((in_dim, out_dim))).astype(np.float16).view(np.uint16)
    return rand_blocks(rng, wtype, out_dim, in_dim)


# Model specs: shape, per-layer slot types, embedding and lm_head types (tied: the
# lm_head is the embedding tensor, as jieyu binds a quantized embed_tokens).
SPECS = {
    # every k-quant and Q8_0 in one model, each layer its own mix
    "kq-mixed": dict(hidden=512, heads=8, kv=2, hd=64, inter=1536, vocab=1000, theta=10000.0, bias=False,
                     layers=[dict(Wq=JY_Q4_K, Wk=JY_Q5_K, Wv=JY_Q6_K, Wo=JY_Q8_0, W1=JY_Q4_K, W2=JY_Q6_K, W3=JY_Q5_K),
                             dict(Wq=JY_Q6_K, Wk=JY_Q4_K, Wv=JY_Q5_K, Wo=JY_Q4_K, W1=JY_Q5_K, W2=JY_Q5_K,
                                  W3=JY_Q6_K)],
                     embed=JY_Q6_K, lm=JY_Q4_K, tied=False),
    # Q4_K_M-like: Q4_K matrices, Q6_K V / down, tied Q6_K embedding, q/k/v biases
    "kq-tied": dict(hidden=256, heads=4, kv=1, hd=64, inter=768, vocab=700, theta=1000000.0, bias=True,
                    layers=[dict(Wq=JY_Q4_K, Wk=JY_Q4_K, Wv=JY_Q6_K, Wo=JY_Q4_K, W1=JY_Q4_K, W2=JY_Q6_K,
                                 W3=JY_Q4_K)] * 2,
                    embed=JY_Q6_K, lm=None, tied=True),
    # all f16 ([in][out]), sizes that are not multiples of 32
    "f16": dict(hidden=320, heads=5, kv=1, hd=64, inter=872, vocab=900, theta=10000.0, bias=False,
                layers=[{s: JY_F16 for s in SLOTS}] * 2, embed=JY_F16, lm=JY_F16, tied=False),
    # all f16 with an FFN width that is not a multiple of 8: the last (rows * 1004) % 8
    # gate values of each SwiGLU take silu's libm tail (silu/x86/x86_classic.txt:30-31)
    "f16-tail": dict(hidden=256, heads=4, kv=1, hd=64, inter=1004, vocab=600, theta=10000.0, bias=False,
                     layers=[{s: JY_F16 for s in SLOTS}] * 2, embed=JY_F16, lm=JY_F16, tied=False),
    # f32, f16 and Q8_0 side by side
    "f32-f16-q8": dict(hidden=256, heads=4, kv=2, hd=64, inter=768, vocab=800, theta=500000.0, bias=False,
                       layers=[dict(Wq=JY_F32, Wk=JY_F16, Wv=JY_Q8_0, Wo=JY_F16, W1=JY_Q8_0, W2=JY_F32, W3=JY_F16),
                               dict(Wq=JY_Q8_0, Wk=JY_F32, Wv=JY_F16, Wo=JY_Q8_0, W1=JY_F16, W2=JY_Q8_0,
                                    W3=JY_F32)],
                       embed=JY_Q8_0, lm=JY_F16, tied=False),
}


def build_model(name, seed=7):
    s = SPECS[name]
    rng = np.random.default_rng(seed)
    H, nh, nkv, hd, F, V = s["hidden"], s["heads"], s["kv"], s["hd"], s["inter"], s["vocab"]
    qd, kvd = nh * hd, nkv * hd
    dims = dict(Wq=(qd, H), Wk=(kvd, H), Wv=(kvd, H), Wo=(H, qd), W1=(F, H), W2=(H, F), W3=(F, H))
    layers = []
    for lt in s["layers"]:
        L = dict(rms1=(1.0 + 0.02 * rng.standard_normal(H)).astype(np.float32),
                 rms2=(1.0 + 0.02 * rng.standard_normal(H)).astype(np.float32))
        for slot in SLOTS:
            L[slot] = (lt[slot], rand_matrix(rng, lt[slot], *dims[slot]))
        if s["bias"]:
            L["bq"] = (0.02 * rng.standard_normal(qd)).astype(np.float32)
            L["bk"] = (0.02 * rng.standard_normal(kvd)).astype(np.float32)
            L["bv"] = (0.02 * rng.standard_normal(kvd)).astype(np.float32)
        layers.append(L)
    et = s["embed"]
    if et in (JY_F32, JY_F16):  # embedding rows [vocab][hidden]
        e = (0.02 * rng.standard_normal((V, H)))
        embed = (et, e.astype(np.float32) if et == JY_F32 else e.astype(np.float16).view(np.uint16))
    else:
        embed = (et, rand_blocks(rng, et, V, H))
    if s["tied"]:
        lm = embed
    elif s["lm"] in (JY_F32, JY_F16):  # [hidden][vocab]
        lm = (s["lm"], rand_matrix(rng, s["lm"], V, H))
    else:
        lm = (s["lm"], rand_blocks(rng, s["lm"], V, H))
    final = (1.0 + 0.02 * rng.standard_normal(H)).astype(np.float32)
    return dict(name=name, hidden=H, heads=nh, kv=nkv, hd=hd, inter=F, vocab=V, theta=s["theta"], layers=layers,
                embed=embed, lm=lm, final=final, tied=s["tied"])


def desc_of(m):
    """ModelDesc over the arrays of build_model(); returns (desc, keepalive)"""
    keep = []

    def p(a):
        a = np.ascontiguousarray(a)
        keep.append(a)
        return a.ctypes.data_as(C.c_void_p)

    def w(tw):
        t, a = tw
        return WMat(p(a), t)

    nl = len(m["layers"])
    layers = (LayerWeights * nl)()
    for i, L in enumerate(m["layers"]):
        layers[i].rms1_weight = p(L["rms1"])
        layers[i].rms2_weight = p(L["rms2"])
        for slot in SLOTS:
            setattr(layers[i], slot, w(L[slot]))
        if "bq" in L:
            layers[i].bq, layers[i].bk, layers[i].bv = p(L["bq"]), p(L["bk"]), p(L["bv"])
    keep.append(layers)
    d = ModelDesc()
    d.num_layers, d.hidden, d.num_heads, d.num_kv_heads = nl, m["hidden"], m["heads"], m["kv"]
    d.head_dim, d.intermediate, d.vocab_size, d.rope_theta = m["hd"], m["inter"], m["vocab"], m["theta"]
    d.embed = w(m["embed"])
    d.lm_head = d.embed if m["tied"] else w(m["lm"])
    d.final_rms_weight = p(m["final"])
    d.layers = C.cast(layers, C.POINTER(LayerWeights))
    return d, keep


def prompt_of(m, n, seed=11):
    return np.random.default_rng(seed).integers(0, m["vocab"], n).astype(np.int32)


# kernel cases: (type, m, n, k); f16 shapes include n % 8 tails
KERNEL_CASES = [
    (JY_Q4_K, 1, 40, 1024), (JY_Q4_K, 3, 24, 512), (JY_Q5_K, 1, 40, 768), (JY_Q5_K, 4, 16, 256),
    (JY_Q6_K, 1, 40, 1024), (JY_Q6_K, 3, 24, 512), (JY_F16, 1, 203, 320), (JY_F16, 3, 40, 64),
    (JY_F16, 5, 13, 72),
]
