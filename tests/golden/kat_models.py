"""The reference's own known-answer models, rebuilt as data.

bind_test model: gen_weights::build + pipe_detail::make_weights
(libs/text/text.h:491-541, :604-610) -- pseudo(i) = ((i*37)%19 - 9)/8 weights,
vocab 24, hidden 8, 2 heads, 1 kv head, head_dim 4, FFN 16, 2 layers.  The
reference checks that generate() reproduces a float64 model's greedy ids
(text.h:817-843); reference_ids_f64 restates that float64 model
(text.h:111-148, :190-231, :248-260, :283-324, :365-420, :551-597).

demo model: converter::make_demo_model (libs/model_libs/converter.h:412-503) --
one-hot embedding, zero attention/FFN, lm_head mapping byte v to v+1; the
pipeline KAT greedy-decodes "abcdefgh" to "ijklmnopqrstuvwx" (text.h:993-1002).
"""
import ctypes as C
import math

import numpy as np

from jieyu_amd.model import JY_F32, LayerWeights, ModelDesc, WMat


def _pseudo(i):
    return np.float32((((np.asarray(i, np.int64) * 37) % 19) - 9) / 8.0)


def bind_test_model(vocab=24, hidden=8, heads=2, kv=1, hd=4, inter=16, layers=2):
    qd, kvd = heads * hd, kv * hd
    f = np.float32
    L = []
    for l in range(layers):
        ar = np.arange
        L.append(dict(
            rms1=(f(1.0) + _pseudo(ar(hidden) + 3 * l) * f(0.25)).astype(f),
            rms2=(f(1.0) + _pseudo(ar(hidden) + 5 * l) * f(0.25)).astype(f),
            Wq=(_pseudo(ar(hidden * qd) + 7 * l) * f(0.5)).astype(f).reshape(hidden, qd),
            Wk=(_pseudo(ar(hidden * kvd) + 11 * l) * f(0.5)).astype(f).reshape(hidden, kvd),
            Wv=(_pseudo(ar(hidden * kvd) + 13 * l) * f(0.5)).astype(f).reshape(hidden, kvd),
            Wo=(_pseudo(ar(qd * hidden) + 17 * l) * f(0.5)).astype(f).reshape(qd, hidden),
            W1=(_pseudo(ar(hidden * inter) + 19 * l) * f(0.5)).astype(f).reshape(hidden, inter),
            W2=(_pseudo(ar(inter * hidden) + 23 * l) * f(0.5)).astype(f).reshape(inter, hidden),
            W3=(_pseudo(ar(hidden * inter) + 29 * l) * f(0.5)).astype(f).reshape(hidden, inter)))
    embed = (_pseudo(np.arange(vocab * hidden) + 101) * f(0.5)).astype(f).reshape(vocab, hidden)
    lm = (_pseudo(np.arange(hidden * vocab) + 211) * f(2.0)).astype(f).reshape(hidden, vocab)
    final = (f(1.0) + _pseudo(np.arange(hidden) + 307) * f(0.25)).astype(f)
    return dict(vocab=vocab, hidden=hidden, heads=heads, kv=kv, hd=hd, inter=inter, layers=L, embed=embed,
                lm=lm, final=final, theta=10000.0)


def demo_model(hidden=256, heads=8, hd=32, kv=2, inter=64, layers=2, vocab=259):
    f = np.float32
    qd, kvd = heads * hd, kv * hd
    embed = np.zeros((vocab, hidden), f)
    for v in range(min(256, vocab)):
        embed[v, v] = 1.0
    lm = np.zeros((hidden, vocab), f)  # [hidden][vocab] after the converter's transpose
    for v in range(1, min(256, vocab)):
        lm[v - 1, v] = 1.0
    L = [dict(rms1=np.ones(hidden, f), rms2=np.ones(hidden, f), Wq=np.zeros((hidden, qd), f),
              Wk=np.zeros((hidden, kvd), f), Wv=np.zeros((hidden, kvd), f), Wo=np.zeros((qd, hidden), f),
              W1=np.zeros((hidden, inter), f), W2=np.zeros((inter, hidden), f), W3=np.zeros((hidden, inter), f))
         for _ in range(layers)]
    return dict(vocab=vocab, hidden=hidden, heads=heads, kv=kv, hd=hd, inter=inter, layers=L, embed=embed, lm=lm,
                final=np.ones(hidden, f), theta=10000.0)


def model_desc(m):
    """ModelDesc over f32 arrays of `m`; returns (desc, keepalive)."""
    keep = []

    def p(a):
        a = np.ascontiguousarray(a, np.float32)
        keep.append(a)
        return a.ctypes.data_as(C.c_void_p)

    nl = len(m["layers"])
    layers = (LayerWeights * nl)()
    for i, l in enumerate(m["layers"]):
        layers[i].rms1_weight = p(l["rms1"])
        layers[i].rms2_weight = p(l["rms2"])
        for slot in ("Wq", "Wk", "Wv", "Wo", "W1", "W2", "W3"):
            setattr(layers[i], slot, WMat(p(l[slot]), JY_F32))
    keep.append(layers)
    d = ModelDesc(num_layers=nl, hidden=m["hidden"], num_heads=m["heads"], num_kv_heads=m["kv"],
                  head_dim=m["hd"], intermediate=m["inter"], vocab_size=m["vocab"], rope_theta=m["theta"],
                  embed=WMat(p(m["embed"]), JY_F32), lm_head=WMat(p(m["lm"]), JY_F32),
                  final_rms_weight=p(m["final"]), layers=layers)
    return d, keep


def bind_model_desc(bm):
    return model_desc(bm)


def demo_model_desc():
    return model_desc(demo_model())


# ---- float64 model of libs/text/text.h (reference_ids and the helpers it calls)

def _rms_f64(x, w, eps=1e-5):
    ss = sum(float(v) * float(v) for v in x)
    scale = 1.0 / math.sqrt(ss / len(x) + float(np.float32(eps)))
    return np.array([np.float32(float(x[i]) * scale * float(w[i])) for i in range(len(x))], np.float32)


def _dmatmul(A, B):
    return (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)


def _rope_f64(q, seq, nh, hd, cos_t, sin_t):
    half = hd // 2
    out = q.copy()
    for pos in range(seq):
        for h in range(nh):
            for i in range(half):
                x0, x1 = float(q[pos, h, 2 * i]), float(q[pos, h, 2 * i + 1])
                c, s = float(cos_t[pos * half + i]), float(sin_t[pos * half + i])
                out[pos, h, 2 * i] = np.float32(x0 * c - x1 * s)
                out[pos, h, 2 * i + 1] = np.float32(x0 * s + x1 * c)
    return out


def _attn_f64(Q, K, V, seq, nh, nkv, hd):
    group = nh // nkv
    scale = 1.0 / math.sqrt(hd)
    out = np.zeros((seq, nh, hd), np.float32)
    for h in range(nh):
        kvh = h // group
        for i in range(seq):
            sc = [float(np.dot(Q[i, h].astype(np.float64), K[j, kvh].astype(np.float64))) * scale
                  for j in range(i + 1)]
            mx = max(sc)
            e = [math.exp(v - mx) for v in sc]
            tot = sum(e)
            for d in range(hd):
                out[i, h, d] = np.float32(sum(e[j] / tot * float(V[j, kvh, d]) for j in range(i + 1)))
    return out


def _silu64(v):
    return v / (1.0 + math.exp(-v))


def reference_ids_f64(m, prompt, n_new, max_seq):
    """gen_detail::reference_ids (libs/text/text.h:551-597): no KV cache, full recompute in
    float64 each step, RoPE tables in double (rope_detail::make_tables, text.h:190-203)."""
    H, nh, nkv, hd, F = m["hidden"], m["heads"], m["kv"], m["hd"], m["inter"]
    half = hd // 2
    cos_t = np.zeros(max_seq * half, np.float32)
    sin_t = np.zeros_like(cos_t)
    for pos in range(max_seq):
        for i in range(half):
            th = pos * math.pow(10000.0, -2.0 * i / hd)
            cos_t[pos * half + i] = np.float32(math.cos(th))
            sin_t[pos * half + i] = np.float32(math.sin(th))
    ids = list(prompt)
    for _ in range(n_new):
        if len(ids) >= max_seq:
            break
        n = len(ids)
        X = np.stack([m["embed"][t] for t in ids]).astype(np.float32)
        for l in m["layers"]:
            xn = np.stack([_rms_f64(X[i], l["rms1"]) for i in range(n)])
            Q = _rope_f64(_dmatmul(xn, l["Wq"]).reshape(n, nh, hd), n, nh, hd, cos_t, sin_t)
            K = _rope_f64(_dmatmul(xn, l["Wk"]).reshape(n, nkv, hd), n, nkv, hd, cos_t, sin_t)
            V = _dmatmul(xn, l["Wv"]).reshape(n, nkv, hd)
            att = _attn_f64(Q, K, V, n, nh, nkv, hd).reshape(n, nh * hd)
            X = (X + _dmatmul(att, l["Wo"])).astype(np.float32)
            xn = np.stack([_rms_f64(X[i], l["rms2"]) for i in range(n)])
            g = xn.astype(np.float64) @ l["W1"].astype(np.float64)
            u = xn.astype(np.float64) @ l["W3"].astype(np.float64)
            h = np.vectorize(_silu64)(g) * u
            X = (X + (h @ l["W2"].astype(np.float64)).astype(np.float32)).astype(np.float32)
        last = _rms_f64(X[n - 1], m["final"])
        logits = _dmatmul(last.reshape(1, H), m["lm"])[0]
        best = 0
        for v in range(1, m["vocab"]):
            if logits[v] > logits[best]:
                best = v
        ids.append(best)
    return ids
