"""GGUF files for the converter checks (test infrastructure): three small models
covering the k-quants, the legacy 32-weight quants, f16 / bf16 / f32 tensors,
v2 and v3 headers, biases, tied and untied heads, skipped tensors, DeepSeek
chat markers and vocabulary escaping; plus malformed files for the error paths
of libs/gguf_libs/gguf.h:495-541 and gguf_convert.h:260-302.
"""
import os
import sys

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import gguf_writer as G  # noqa: E402


def byte_pieces():
    """the 256 byte-level BPE pieces (printable Latin-1 bytes as themselves, the rest
    mapped to U+0100..), ids = byte values"""
    out, nxt = [], 256
    for b in range(256):
        if 33 <= b <= 126 or 161 <= b <= 172 or 174 <= b <= 255:
            out.append(chr(b))
        else:
            out.append(chr(nxt))
            nxt += 1
    return out


def _blocks(g, rng, nl, hidden, heads, kv, hd, ff, types, bias=False):
    for l in range(nl):
        p = f"blk.{l}."
        g.tensor(p + "attn_norm.weight", [hidden], G.T_F32, (1 + 0.02 * rng.standard_normal(hidden)).astype(np.float32).tobytes())
        for nm, shape in (("attn_q", [hidden, heads * hd]), ("attn_k", [hidden, kv * hd]), ("attn_v", [hidden, kv * hd]),
                          ("attn_output", [heads * hd, hidden]), ("ffn_gate", [hidden, ff]), ("ffn_up", [hidden, ff]),
                          ("ffn_down", [ff, hidden])):
            t = types[nm]
            g.tensor(p + nm + ".weight", shape, t, G.tensor_bytes(rng, t, shape))
        if bias:
            for nm, n in (("attn_q", heads * hd), ("attn_k", kv * hd), ("attn_v", kv * hd)):
                g.tensor(p + nm + ".bias", [n], G.T_F32, (0.02 * rng.standard_normal(n)).astype(np.float32).tobytes())
        g.tensor(p + "ffn_norm.weight", [hidden], G.T_F32, (1 + 0.02 * rng.standard_normal(hidden)).astype(np.float32).tobytes())


def llama_q4km():
    """Q4_K_M-like llama, v3: k-quant matrices, Q6_K embedding tied as the head"""
    rng = np.random.default_rng(21)
    hidden, nl, heads, kv, ff = 256, 2, 4, 2, 512
    toks = byte_pieces() + ["<|im_start|>", "<|im_end|>", "<|endoftext|>"]
    g = G.GGUF(3)
    g.add("general.architecture", G.STR, "llama").add("general.name", G.STR, "tiny llama q4km")
    g.add("llama.embedding_length", G.U32, hidden).add("llama.block_count", G.U32, nl)
    g.add("llama.feed_forward_length", G.U32, ff).add("llama.attention.head_count", G.U32, heads)
    g.add("llama.attention.head_count_kv", G.U32, kv).add("llama.rope.freq_base", G.F32, 500000.0)
    g.add("llama.context_length", G.U32, 4096)
    g.add("tokenizer.ggml.tokens", G.ARR, toks, G.STR).add("tokenizer.ggml.merges", G.ARR, [], G.STR)
    g.add("tokenizer.ggml.eos_token_id", G.U32, 257).add("tokenizer.ggml.bos_token_id", G.U32, 256)
    g.tensor("token_embd.weight", [hidden, len(toks)], G.T_Q6_K, G.tensor_bytes(rng, G.T_Q6_K, [hidden, len(toks)]))
    _blocks(g, rng, nl, hidden, heads, kv, hidden // heads, ff,
            dict(attn_q=G.T_Q4_K, attn_k=G.T_Q4_K, attn_v=G.T_Q6_K, attn_output=G.T_Q4_K, ffn_gate=G.T_Q4_K,
                 ffn_up=G.T_Q5_K, ffn_down=G.T_Q6_K))
    g.tensor("output_norm.weight", [hidden], G.T_F32, (1 + 0.02 * rng.standard_normal(hidden)).astype(np.float32).tobytes())
    g.tensor("rope_freqs.weight", [32], G.T_F32, np.ones(32, np.float32).tobytes())  # no Hugging Face name: skipped
    return g


def qwen_mixed():
    """qwen2, v2 header, alignment 64: q/k/v biases, legacy quants, f16 / bf16, Q8_0 head"""
    rng = np.random.default_rng(22)
    hidden, nl, heads, kv, hd, ff, V = 128, 2, 4, 1, 32, 256, 300
    # byte-level pieces, three merged pieces, fillers, then the chat markers
    toks = byte_pieces() + ["ab", "cd", "abcd"]
    toks += [f"x{i}" for i in range(V - 3 - len(toks))] + ["<|endoftext|>", "<|im_start|>", "<|im_end|>"]
    g = G.GGUF(2, alignment=64)
    g.add("general.architecture", G.STR, "qwen2")
    g.add("qwen2.embedding_length", G.U64, hidden).add("qwen2.block_count", G.I32, nl)
    g.add("qwen2.feed_forward_length", G.U32, ff).add("qwen2.attention.head_count", G.U16, heads)
    g.add("qwen2.attention.head_count_kv", G.U8, kv).add("qwen2.attention.key_length", G.U32, hd)
    g.add("qwen2.rope.freq_base", G.F64, 1000000.0).add("qwen2.context_length", G.U64, 2048)
    g.add("qwen2.use_parallel_residual", G.BOOL, True).add("qwen2.some_floats", G.ARR, [0.5, 1.5], G.F32)
    g.add("tokenizer.ggml.tokens", G.ARR, toks, G.STR)
    g.add("tokenizer.ggml.merges", G.ARR, ["a b", "c d", "ab cd"], G.STR)
    g.add("tokenizer.ggml.eos_token_id", G.I32, V - 3)
    g.tensor("token_embd.weight", [hidden, V], G.T_F16, G.tensor_bytes(rng, G.T_F16, [hidden, V]))
    _blocks(g, rng, nl, hidden, heads, kv, hd, ff,
            dict(attn_q=G.T_Q8_0, attn_k=G.T_Q4_0, attn_v=G.T_Q5_1, attn_output=G.T_F16, ffn_gate=G.T_BF16,
                 ffn_up=G.T_Q4_1, ffn_down=G.T_Q5_0), bias=True)
    g.tensor("output_norm.weight", [hidden], G.T_F32, (1 + 0.02 * rng.standard_normal(hidden)).astype(np.float32).tobytes())
    g.tensor("output.weight", [hidden, V], G.T_Q8_0, G.tensor_bytes(rng, G.T_Q8_0, [hidden, V]))
    return g


DS_BAR, DS_SP = "｜", "▁"


def deepseek_f32():
    """f32 tensors, DeepSeek chat markers, vocabulary pieces that need escaping"""
    rng = np.random.default_rng(23)
    hidden, nl, heads, kv, ff, V = 64, 1, 2, 2, 128, 40
    marks = [f"<{DS_BAR}User{DS_BAR}>", f"<{DS_BAR}Assistant{DS_BAR}>",
             f"<{DS_BAR}begin{DS_SP}of{DS_SP}sentence{DS_BAR}>", f"<{DS_BAR}end{DS_SP}of{DS_SP}sentence{DS_BAR}>",
             '"', "\\", 'a"b\\c', "</s>"]
    toks = [f"w{i}" for i in range(V - len(marks))] + marks
    g = G.GGUF(3)
    g.add("general.architecture", G.STR, "llama").add("general.name", G.STR, "")
    g.add("llama.embedding_length", G.U32, hidden).add("llama.feed_forward_length", G.U32, ff)
    g.add("llama.attention.head_count", G.U32, heads).add("llama.rope.freq_base", G.U32, 10000)  # int: reads 0
    g.add("tokenizer.ggml.tokens", G.ARR, toks, G.STR).add("tokenizer.ggml.bos_token_id", G.U32, V - 6)
    g.tensor("token_embd.weight", [hidden, V], G.T_F32, G.tensor_bytes(rng, G.T_F32, [hidden, V]))
    _blocks(g, rng, nl, hidden, heads, kv, hidden // heads, ff,
            {k: G.T_F32 for k in ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down")})
    g.tensor("output_norm.weight", [hidden], G.T_F32, np.ones(hidden, np.float32).tobytes())
    g.tensor("output.weight", [hidden, V], G.T_F32, G.tensor_bytes(rng, G.T_F32, [hidden, V]))
    return g


MODELS = {"llama-q4km": llama_q4km, "qwen-mixed": qwen_mixed, "deepseek-f32": deepseek_f32}

# (case, model, out_dtype, quant, pre-existing model_info.json text or None)
CONVERT_CASES = [
    ("llama-q4km-quant", "llama-q4km", 0, 1, None),
    ("llama-q4km-f32", "llama-q4km", 0, 0, None),
    ("llama-q4km-f16", "llama-q4km", 1, 0, None),
    ("llama-q4km-bf16", "llama-q4km", 2, 0, None),
    ("qwen-mixed-quant", "qwen-mixed", 0, 1, None),
    ("qwen-mixed-f16", "qwen-mixed", 1, 0, None),
    ("deepseek-f32-quant", "deepseek-f32", 0, 1, '{\n  "num_heads": 99,\n  "extra": [1, 2],\n  "note": "kept"\n}\n'),
]

OUT_FILES = ("model.bf", "model_info.json", "vocab.json", "merges.txt")


def bad_files():
    """(name, GGUF bytes): each fails in the reader or the converter"""
    ok = llama_q4km()
    out = [("bad-magic", b"GGUX" + ok.bytes()[4:]),
           ("version-1", b"GGUF" + (1).to_bytes(4, "little") + ok.bytes()[8:]),
           ("truncated-header", ok.bytes(truncate=200)),
           ("truncated-data", ok.bytes(truncate=len(ok.bytes()) - 1000))]
    g = G.GGUF(3).add("general.architecture", G.STR, "llama").add("llama.embedding_length", G.U32, 64)
    out.append(("no-hyper", g.bytes()))
    g = G.GGUF(3).add("x", G.ARR, [], G.ARR)
    out.append(("nested-array", g.bytes()))
    import struct  # one metadata entry of an undefined value type (99)
    out.append(("meta-type", b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1) + b"x" +
                struct.pack("<I", 99) + b"\0" * 8))
    g = llama_q4km()
    g.tensors = [t for t in g.tensors if t[0] != "token_embd.weight"]
    out.append(("no-embed", g.bytes()))
    g = llama_q4km()
    g.kv = [kv for kv in g.kv if kv[0] != "llama.attention.head_count"]
    out.append(("no-heads", g.bytes()))
    g = llama_q4km()
    g.kv = [kv for kv in g.kv if kv[0] != "tokenizer.ggml.tokens"]
    g.add("llama.vocab_size", G.U32, 259)
    out.append(("no-tokens", g.bytes()))
    g = llama_q4km()
    g.tensor("blk.0.extra.weight", [128, 4], G.T_Q4_K, b"\0" * (2 * 144))  # 512 weights, rows of 128
    out.append(("row-not-block", g.bytes()))
    g = llama_q4km()
    g.tensor("blk.0.odd.weight", [100], G.T_Q4_K, b"")
    out.append(("partial-block", g.bytes()))
    g = llama_q4km()
    g.tensor("blk.0.iq.weight", [256], G.T_IQ4_XS, b"\0" * 136)
    out.append(("iq4xs-skipped", g.bytes()))  # unknown name: skipped, so it converts
    g = llama_q4km()
    g.tensor("output.weight", [256, 259], G.T_IQ4_XS, b"\0" * (259 * 136))
    out.append(("iq4xs-dequant", g.bytes()))
    g = llama_q4km()
    g.tensors = [(n, s, 5, d) if n == "output_norm.weight" else (n, s, t, d) for (n, s, t, d) in g.tensors]
    out.append(("unknown-type", g.bytes()))
    return out
