"""Model directories for the text C ABI checks (jieyu_load / jieyu_generate).

Each builder writes a complete directory (model.bf, model_info.json, vocab.json,
merges.txt) with jieyu_amd.bfile, whose output is byte-identical to jieyu's own
writer (the bind_test fixtures pin it).  The same builders serve
make_text_golden.py, which records what jieyu's own C ABI returns for each
directory, and the tests, which compare the GPU library with those records.

  demo      converter::make_demo_model (libs/model_libs/converter.h:412-503):
            one-hot embedding, zero attention and FFN, lm_head maps byte v to
            v+1; byte-level vocabulary.  Its KATs: text.h:993-1013.
  bind      the reference's bind_test model.bf fixture (tests/golden/bind_test)
            with a 24-letter vocabulary a..x (ids 0..23).
  bpe_f32   a random 2-layer f32 decoder over a BPE vocabulary trained by
            jieyu's own trainer (tests/golden/tok_bpe), with chat markers.
  bpe_q8    the same vocabulary, Q8_0 weights and a tied embedding.
"""
import json
import os
import shutil

import numpy as np

from jieyu_amd import bfile as B

HERE = os.path.dirname(os.path.abspath(__file__))
TOK_DIR = os.path.join(HERE, "tok_bpe")
BIND_FIXTURES = os.path.join(HERE, "bind_test")
MARKERS = ("<|im_start|>", "<|im_end|>")


def bpe_vocab_size():
    with open(os.path.join(TOK_DIR, "vocab.json"), encoding="utf-8") as f:
        v = json.load(f)
    return max(v.values()) + 1


def demo_dir(path):
    hidden, heads, hd, kv, inter, layers, vocab = 256, 8, 32, 2, 64, 2, 259
    f = np.float32
    embed = np.zeros((vocab, hidden), f)
    for v in range(256):
        embed[v, v] = 1.0
    lm = np.zeros((hidden, vocab), f)          # [hidden][vocab], as the converter transposes it
    for v in range(1, 256):
        lm[v - 1, v] = 1.0
    L = [dict(rms1=np.ones(hidden, f), rms2=np.ones(hidden, f), Wq=np.zeros((hidden, heads * hd), f),
              Wk=np.zeros((hidden, kv * hd), f), Wv=np.zeros((hidden, kv * hd), f),
              Wo=np.zeros((heads * hd, hidden), f), W1=np.zeros((hidden, inter), f),
              W2=np.zeros((inter, hidden), f), W3=np.zeros((hidden, inter), f)) for _ in range(layers)]
    ts = B.decoder_tensors(embed, lm, np.ones(hidden, f), L)
    hp = dict(hidden=hidden, layers=layers, num_heads=heads, num_kv_heads=kv, head_dim=hd, intermediate=inter,
              vocab=vocab)
    return B.write_model_dir(path, ts, hp, info={"rope_theta": 10000, "max_position_embeddings": 1024})


def bind_dir(path, which="model"):
    os.makedirs(path, exist_ok=True)
    shutil.copyfile(os.path.join(BIND_FIXTURES, which, "model.bf"), os.path.join(path, "model.bf"))
    hp = dict(model=(8, 2, 2, 1, 4, 16, 24, 8), wrong_shape=(8, 1, 2, 1, 6, 16, 24, 8),
              missing=(8, 1, 2, 1, 4, 16, 24, 8))[which]
    keys = ("hidden_size", "layer_count", "num_heads", "num_kv_heads", "head_dim", "intermediate_size",
            "vocab_size", "max_position_embeddings")
    info = dict(zip(keys, hp))
    info["rope_theta"] = 10000
    B.write_info(os.path.join(path, "model_info.json"), info)
    letters = "abcdefghijklmnopqrstuvwx"
    with open(os.path.join(path, "vocab.json"), "w", encoding="utf-8") as f:
        f.write("{" + ",".join(f'"{c}":{i}' for i, c in enumerate(letters)) + "}")
    with open(os.path.join(path, "merges.txt"), "w") as f:
        f.write("#version: 0.2\n")
    return path


def _random_layers(rng, layers, hidden, heads, kv, hd, inter, scale):
    f = np.float32
    n = lambda *s: (rng.standard_normal(s) * scale).astype(f)  # noqa: E731
    return [dict(rms1=(1 + 0.1 * rng.standard_normal(hidden)).astype(f),
                 rms2=(1 + 0.1 * rng.standard_normal(hidden)).astype(f),
                 Wq=n(hidden, heads * hd), Wk=n(hidden, kv * hd), Wv=n(hidden, kv * hd), Wo=n(heads * hd, hidden),
                 W1=n(hidden, inter), W2=n(inter, hidden), W3=n(hidden, inter)) for _ in range(layers)]


BPE_HP = dict(hidden=64, layers=2, num_heads=4, num_kv_heads=2, head_dim=16, intermediate=128)
BPE_INFO = {"rope_theta": 10000, "max_position_embeddings": 256, "message_start": MARKERS[0],
            "message_end": MARKERS[1]}


def bpe_f32_dir(path, seed=7):
    rng = np.random.default_rng(seed)
    hp = dict(BPE_HP, vocab=bpe_vocab_size())
    H, V = hp["hidden"], hp["vocab"]
    L = _random_layers(rng, hp["layers"], H, hp["num_heads"], hp["num_kv_heads"], hp["head_dim"],
                       hp["intermediate"], 0.25)
    embed = rng.standard_normal((V, H)).astype(np.float32)
    lm = (rng.standard_normal((H, V)) * 0.5).astype(np.float32)
    final = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    ts = B.decoder_tensors(embed, lm, final, L)
    vocab = (os.path.join(TOK_DIR, "vocab.json"), os.path.join(TOK_DIR, "merges.txt"))
    return B.write_model_dir(path, ts, hp, info=BPE_INFO, vocab=vocab)


def _q8(lib, a):
    """Q8_0 blob of a row-major [rows][cols] float array (the library's quantizer)"""
    import ctypes as C
    a = np.ascontiguousarray(a, np.float32)
    out = np.zeros(a.size // 32 * 34, np.uint8)
    lib.jysyn_quantize_q8_0(a.ctypes.data_as(C.c_void_p), out.ctypes.data_as(C.c_void_p), a.size)
    return out


def bpe_q8_dir(path, lib, seed=11):
    """Q8_0 weights ([out][in] rows quantized per 32), tied Q8_0 embedding / lm_head"""
    rng = np.random.default_rng(seed)
    hp = dict(BPE_HP, vocab=bpe_vocab_size())
    H, V = hp["hidden"], hp["vocab"]
    L = _random_layers(rng, hp["layers"], H, hp["num_heads"], hp["num_kv_heads"], hp["head_dim"],
                       hp["intermediate"], 0.25)
    q8 = {}
    for l, layer in enumerate(L):
        for key, sfx in (("Wq", "self_attn.q_proj.weight"), ("Wk", "self_attn.k_proj.weight"),
                         ("Wv", "self_attn.v_proj.weight"), ("Wo", "self_attn.o_proj.weight"),
                         ("W1", "mlp.gate_proj.weight"), ("W2", "mlp.down_proj.weight"),
                         ("W3", "mlp.up_proj.weight")):
            w = layer[key].T                      # [out][in]
            q8[B.layer_name(l, sfx)] = (w.shape[0], w.shape[1], _q8(lib, w))
    embed = rng.standard_normal((V, H)).astype(np.float32)
    q8["model.embed_tokens.weight"] = (V, H, _q8(lib, embed))
    final = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    ts = B.decoder_tensors(embed, None, final, L, q8=q8)
    vocab = (os.path.join(TOK_DIR, "vocab.json"), os.path.join(TOK_DIR, "merges.txt"))
    return B.write_model_dir(path, ts, hp, info=BPE_INFO, vocab=vocab)


# Byte strings the tokenizer checks encode: ASCII words and punctuation, runs
# of spaces, tabs and newlines, CJK text with full-width punctuation, the chat
# markers, the BOS/EOS pieces, digits, malformed UTF-8, and an empty string.
TOKENIZER_STRINGS = [s.encode("utf-8") for s in [
    "", "a", "abc", "Hello, JieYu AI!", "hello world", "  two  spaces", "tab\there", "line\nbreak\r\n",
    "The quick brown fox jumps over the lazy dog.", "你好，世界！昆仑分词器。", "mixed 中文 and English, ok?",
    "<|im_start|>user\nhi<|im_end|>\n<|im_start|>assistant\n", "x<|im_end|>y<|im_start|>",
    "<｜begin▁of▁sentence｜>start", "end<｜end▁of▁sentence｜>", "1234567890 3.14159",
    " leading space", "trailing space ", "punct!?,.;:'\"()[]{}", "　ideographic　space", "emoji \U0001F600 ok",
    "the theory of the thing: they then thought", "x = f(y) + g[z]; // comment",
]] + [b"\xff\xfe raw bytes", b"cut \xe4\xbd", b"\xc3( bad", b"\x00\x01\x7f ctrl"]


# ------------------------------------------------------------ C ABI scripts
#
# A script is a model directory, the max_seq to load it with, and a list of
# calls.  run_script() executes it against any library that exports jieyu's
# C ABI (jieyu's own, compiled from the reference sources, or libjieyu_amd)
# and returns one record per call.

def jsonl_file(path):
    lines = [{"name": "user", "message": "hello there"},
             {"name": "assistant", "message": "hi, how can I help?"},
             {"other": 1},
             {"name": "user", "message": "tell me about the theory"}]
    with open(path, "w", encoding="utf-8") as f:
        f.write("\n".join(json.dumps(x, ensure_ascii=False) for x in lines) + "\n")
    return path


SCRIPTS = [
    ("demo", 64, [
        ("gen", b"abcdefgh", 16, 0.0, 1.0, 4096),
        ("gen", b"abc", 5, 0.0, 1.0, 4096),
        ("gen", b"xyz", 8, 0.0, 1.0, 4096),
        ("gen", b"xyz", 8, 0.0, 1.0, 4096),
        ("gen", b"k" * 200, 16, 0.0, 1.0, 4096),
        ("gen", b"abcdefgh", 16, 0.0, 1.0, 5),
        ("gen", b"abcdefgh", 16, 0.0, 1.0, 0),
        ("gen", b"", 8, 0.0, 1.0, 4096),
        ("gen", b"abc", 0, 0.0, 1.0, 4096),
        ("gen", b"abc", 12, 0.8, 1.1, 4096),
        ("gen", b"abc", 12, 0.0, 1.3, 4096),
        ("gen", None, 8, 0.0, 1.0, 4096),
        ("info",),
        ("load_again", 0),
    ]),
    ("bind", 8, [
        ("gen", b"bcd", 3, 0.0, 1.0, 4096),
        ("gen", b"bcd", 5, 0.0, 1.0, 4096),
        ("gen", b"hello", 3, 0.0, 1.0, 4096),
        ("gen", b"xyz", 3, 0.0, 1.0, 4096),
        ("gen", b"bcd", 4, 0.9, 1.2, 4096),
        ("info",),
    ]),
    ("bpe_f32", 128, [
        ("gen", b"Hello, JieYu AI!", 24, 0.0, 1.0, 4096),
        ("gen", "你好，世界！".encode(), 24, 0.0, 1.0, 4096),
        ("gen", b"<|im_start|>user\nhi<|im_end|>\n<|im_start|>assistant\n", 32, 0.0, 1.0, 4096),
        ("gen", b"the theory of the thing", 40, 0.7, 1.1, 4096),
        ("gen", b"the theory of the thing", 40, 0.0, 1.1, 4096),
        ("gen", b"the", 200, 0.0, 1.0, 4096),
        ("jsonl", "chat.jsonl", None, None, 24, 0.0, 1.0, 4096),
        ("jsonl", "chat.jsonl", b"[", b"]", 24, 0.8, 1.1, 4096),
        ("jsonl", "missing.jsonl", None, None, 24, 0.0, 1.0, 4096),
        ("info",),
    ]),
    ("bpe_q8", 128, [
        ("gen", b"Hello, JieYu AI!", 24, 0.0, 1.0, 4096),
        ("gen", b"x = f(y) + g[z]; // comment", 48, 0.0, 1.0, 4096),
        ("gen", b"the theory of the thing", 40, 0.7, 1.1, 4096),
        ("jsonl", "chat.jsonl", None, None, 24, 0.0, 1.0, 4096),
    ]),
    # GGUF files converted to model directories (jytext_gguf_convert, quant = true):
    # Q4_K / Q5_K / Q6_K matrices with the Q6_K embedding as the tied head ...
    ("gguf_q4km", 64, [
        ("gen", b"hello world", 16, 0.0, 1.0, 4096),
        ("gen", b"<|im_start|>user\nhi<|im_end|>\n<|im_start|>assistant\n", 24, 0.0, 1.0, 4096),
        ("gen", b"abc", 20, 0.8, 1.1, 4096),
        ("gen", b"abc", 20, 0.0, 1.3, 4096),
        ("info",),
    ]),
    # ... and Q8_0 matrices beside f32 ones dequantized from Q4_0 / Q4_1 / Q5_0 / Q5_1 /
    # f16 / bf16, q/k/v biases, untied Q8_0 head
    ("gguf_qwen", 64, [
        ("gen", b"abcd abc", 16, 0.0, 1.0, 4096),
        ("gen", b"Hello, qwen!", 20, 0.7, 1.1, 4096),
        ("gen", b"<|im_start|>user\ncd ab<|im_end|>\n", 16, 0.0, 1.2, 4096),
        ("jsonl", "chat.jsonl", None, None, 16, 0.0, 1.0, 4096),
    ]),
]

LOAD_ERRORS = ["bind:wrong_shape", "bind:missing", "nodir", "noinfo", "novocab", "badmagic"]


def build_dir(kind, root, lib=None):
    """the directory a script or load-error case names, built under root"""
    path = os.path.join(root, kind.replace(":", "_"))
    if os.path.isdir(path):
        return path
    if kind == "demo":
        demo_dir(path)
    elif kind == "bind":
        bind_dir(path)
    elif kind.startswith("bind:"):
        bind_dir(path, kind.split(":")[1])
    elif kind == "bpe_f32":
        bpe_f32_dir(path)
    elif kind == "bpe_q8":
        bpe_q8_dir(path, lib)
    elif kind in ("gguf_q4km", "gguf_qwen"):
        import gguf_models
        from jieyu_amd import api
        model = {"gguf_q4km": gguf_models.llama_q4km, "gguf_qwen": gguf_models.qwen_mixed}[kind]()
        src = model.write(path + ".gguf")
        api.gguf_convert(src, path, "f32", True)
    elif kind == "nodir":
        return path  # never created
    elif kind == "noinfo":
        bind_dir(path)
        os.remove(os.path.join(path, "model_info.json"))
    elif kind == "novocab":
        bind_dir(path)
        os.remove(os.path.join(path, "vocab.json"))
    elif kind == "badmagic":
        bind_dir(path)
        with open(os.path.join(path, "model.bf"), "r+b") as f:
            f.write(b"JYAIBX")
    jsonl_file(os.path.join(path, "chat.jsonl"))
    return path


def bind_abi(lib):
    import ctypes as C
    P, I, F, S = C.c_void_p, C.c_int, C.c_float, C.c_char_p
    for name, res, args in (("jieyu_load", P, [S, I]), ("jieyu_free", None, [P]), ("jieyu_last_error", S, [P]),
                            ("jieyu_version", S, []), ("jieyu_context_length", I, [P]),
                            ("jieyu_model_dir", S, [P]),
                            ("jieyu_generate", I, [P, S, P, I, I, F, F]),
                            ("jieyu_generate_jsonl", I, [P, S, S, S, P, I, I, F, F])):
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    return lib


def _call(lib, h, root, c):
    import ctypes as C
    if c[0] == "info":
        return {"ctx": lib.jieyu_context_length(h), "dir_tail": os.path.basename(lib.jieyu_model_dir(h).decode()),
                "version": lib.jieyu_version().decode(), "null_ctx": lib.jieyu_context_length(None),
                "null_dir": lib.jieyu_model_dir(None).decode()}
    if c[0] == "load_again":
        h2 = lib.jieyu_load(lib.jieyu_model_dir(h), c[1])
        r = {"ok": bool(h2), "ctx": lib.jieyu_context_length(h2) if h2 else None}
        if h2:
            lib.jieyu_free(h2)
        return r
    cap = c[-1]
    buf = C.create_string_buffer(max(cap, 1))
    out = buf if cap > 0 else None
    if c[0] == "gen":
        _, prompt, max_new, t, rp, _ = c
        ret = lib.jieyu_generate(h, prompt, out, cap, max_new, t, rp)
    else:
        _, name, qb, qe, max_new, t, rp, _ = c
        path = os.path.join(root, name).encode()
        ret = lib.jieyu_generate_jsonl(h, path, qb, qe, out, cap, max_new, t, rp)
    return {"ret": ret, "out_hex": buf.raw[:cap].split(b"\0")[0].hex() if cap > 0 else "",
            "err": lib.jieyu_last_error(h).decode("utf-8", "replace")}


def run_script(lib, root, kind, max_seq, calls, qlib=None):
    """records of one script; root holds the model directories"""
    path = build_dir(kind, root, qlib)
    h = lib.jieyu_load(path.encode(), max_seq)
    if not h:
        return {"load_error": lib.jieyu_last_error(None).decode("utf-8", "replace")}
    try:
        return {"calls": [_call(lib, h, path, c) for c in calls]}
    finally:
        lib.jieyu_free(h)


def run_load_error(lib, root, kind):
    path = build_dir(kind, root)
    h = lib.jieyu_load(path.encode(), 16)
    if h:
        lib.jieyu_free(h)
        return {"loaded": True}
    return {"loaded": False, "err": lib.jieyu_last_error(None).decode("utf-8", "replace")}
