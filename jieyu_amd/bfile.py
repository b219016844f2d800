"""Model directories in jieyu's on-disk format, written from numpy arrays.

A model directory holds model.bf (bfile v2), model_info.json, vocab.json and
merges.txt -- what ``jieyu_load`` (include/jieyu_api.h) reads.  The writer lays
model.bf out the way jieyu's own writer does (libs/model_libs/bfile.h:17-22,
:124-135, :237-307): a 64-byte header, a 104-byte table entry per tensor, the
data area starting at the 64-aligned end of the table, every tensor at a
64-aligned offset.  2-D f32 / f16 weights are stored [in][out], block-quantized
ones (Q8_0, Q4_K, Q5_K, Q6_K) [out][in/block] x block bytes, as jieyu's
bind_model expects (libs/model_libs/pipeline.h:103-117).
"""
import json
import os
import struct

import numpy as np

MAGIC = b"JYAIBF"
VERSION = 2
HEADER = 64
ENTRY = 104
ALIGN = 64

F32, F16, BF16, I8, I32, Q4K, Q5K, Q6K, Q8_0 = range(9)
_ELEM_BYTES = {F32: 4, I32: 4, F16: 2, BF16: 2, I8: 1}
_BLOCK = {Q4K: (256, 144), Q5K: (256, 176), Q6K: (256, 210), Q8_0: (32, 34)}


def _align(n, a=ALIGN):
    return (n + a - 1) // a * a


def tensor_bytes(dtype, shape):
    elems = int(np.prod(shape, dtype=np.int64)) if len(shape) else 1
    if dtype in _BLOCK:
        be, bb = _BLOCK[dtype]
        return 0 if elems % be else elems // be * bb
    return elems * _ELEM_BYTES[dtype]


class Tensor:
    """A named tensor: dtype (F32 / Q8_0 / ...), shape, raw little-endian bytes."""

    def __init__(self, name, dtype, shape, data):
        self.name, self.dtype, self.shape = name, int(dtype), [int(s) for s in shape]
        self.data = bytes(data)
        if not 1 <= len(name.encode()) <= 63:
            raise ValueError(f"tensor name must be 1..63 bytes: {name!r}")
        if len(self.shape) > 4:
            raise ValueError(f"more than 4 dimensions: {name}")
        if tensor_bytes(self.dtype, self.shape) != len(self.data):
            raise ValueError(f"shape does not match the data length: {name}")

    @staticmethod
    def f32(name, arr):
        a = np.ascontiguousarray(arr, dtype="<f4")
        return Tensor(name, F32, a.shape, a.tobytes())

    @staticmethod
    def f16(name, arr):
        a = np.ascontiguousarray(arr, dtype="<f2")
        return Tensor(name, F16, a.shape, a.tobytes())

    @staticmethod
    def q8_0(name, rows, cols, blob):
        """blob: [rows][cols/32] x 34 bytes (fp16 scale + 32 int8), as jieyu stores it"""
        return Tensor(name, Q8_0, (rows, cols), np.asarray(blob, np.uint8).tobytes())

    @staticmethod
    def quant(name, dtype, rows, cols, blob):
        """a block-quantized matrix (Q8_0 / Q4K / Q5K / Q6K): [rows][cols/block] blocks"""
        return Tensor(name, dtype, (rows, cols), np.asarray(blob, np.uint8).tobytes())


def write_bfile(path, tensors, hidden, layers, num_heads, num_kv_heads, head_dim, intermediate, vocab, mode=1):
    """model.bf with a v2 tensor table; returns the file size."""
    table = len(tensors) * ENTRY
    data_off = _align(HEADER + table)
    offs, cur = [], 0
    for t in tensors:
        offs.append(cur)
        cur = _align(cur + len(t.data))
    head = bytearray(HEADER)
    head[0:6] = MAGIC
    struct.pack_into("<QQBBBBIQ", head, 6, hidden, layers, mode, num_heads, num_kv_heads, head_dim, intermediate,
                     vocab)
    struct.pack_into("<IIII", head, 38, VERSION, len(tensors), data_off, ENTRY)
    with open(path, "wb") as f:
        f.write(head)
        for t, off in zip(tensors, offs):
            e = bytearray(ENTRY)
            nb = t.name.encode()
            e[0:len(nb)] = nb
            shape = (t.shape + [0, 0, 0, 0])[:4]
            struct.pack_into("<BBH4IIQQ", e, 64, t.dtype, len(t.shape), 0, *shape, 0, off, len(t.data))
            f.write(e)
        f.write(b"\0" * (data_off - HEADER - table))
        pos = 0
        for t, off in zip(tensors, offs):
            if off > pos:
                f.write(b"\0" * (off - pos))
                pos = off
            f.write(t.data)
            pos += len(t.data)
    return os.path.getsize(path)


def write_info(path, items):
    """model_info.json: a flat object, two-space indented, numbers unquoted"""
    with open(path, "w", encoding="utf-8") as f:
        f.write(json.dumps(items, indent=2, ensure_ascii=False) + "\n")


def byte_level_pieces():
    """the 256 byte-level pieces: printable Latin-1 bytes are themselves, the others
    take code points 256, 257, ... in byte order (tokenizer.h:64-100)"""
    printable = [33 <= b <= 126 or 161 <= b <= 172 or 174 <= b <= 255 for b in range(256)]
    out, nxt = [], 256
    for b in range(256):
        if printable[b]:
            out.append(chr(b))
        else:
            out.append(chr(nxt))
            nxt += 1
    return out


def write_byte_vocab(vocab_path, merges_path):
    """a vocabulary of the 256 byte pieces (ids = byte values) and no merges
    (libs/tokenizer_libs/include/byte_vocab.h:15-38)"""
    parts = []
    for b, p in enumerate(byte_level_pieces()):
        esc = p.replace("\\", "\\\\").replace('"', '\\"')
        parts.append(f'"{esc}":{b}')
    with open(vocab_path, "wb") as f:
        f.write(("{" + ",".join(parts) + "}").encode("utf-8"))
    with open(merges_path, "wb") as f:
        f.write(b"#version: 0.2\n")


def layer_name(l, suffix):
    return f"model.layers.{l}.{suffix}"


def decoder_tensors(embed, lm_head, final_norm, layers, q8=None, quant=None):
    """Tensor list of a decoder in jieyu's names.

    layers: dicts with rms1, rms2 (float [hidden]) and Wq, Wk, Wv, Wo, W1, W2, W3.
    Dense weights are [in][out] arrays, written f16 when the array is float16 and
    f32 otherwise; with q8 (dict name -> (rows, cols, blob)) or quant (dict name ->
    (dtype, rows, cols, blob)) given, the named weights are block-quantized instead.
    embed: [vocab][hidden] dense or quantized; lm_head: dense [hidden][vocab],
    quantized [vocab][hidden], or None (tied to the embedding, which must then be
    quantized)."""
    quant = dict(quant or {})
    for name, (r, c, blob) in (q8 or {}).items():
        quant[name] = (Q8_0, r, c, blob)

    def w(name, arr):
        if name in quant:
            dt, r, c, blob = quant[name]
            return Tensor.quant(name, dt, r, c, blob)
        if arr is not None and np.asarray(arr).dtype == np.float16:
            return Tensor.f16(name, arr)
        return Tensor.f32(name, arr)

    ts = [w("model.embed_tokens.weight", embed)]
    for l, L in enumerate(layers):
        ts += [Tensor.f32(layer_name(l, "input_layernorm.weight"), L["rms1"]),
               w(layer_name(l, "self_attn.q_proj.weight"), L.get("Wq")),
               w(layer_name(l, "self_attn.k_proj.weight"), L.get("Wk")),
               w(layer_name(l, "self_attn.v_proj.weight"), L.get("Wv")),
               w(layer_name(l, "self_attn.o_proj.weight"), L.get("Wo")),
               Tensor.f32(layer_name(l, "post_attention_layernorm.weight"), L["rms2"]),
               w(layer_name(l, "mlp.gate_proj.weight"), L.get("W1")),
               w(layer_name(l, "mlp.down_proj.weight"), L.get("W2")),
               w(layer_name(l, "mlp.up_proj.weight"), L.get("W3"))]
        for b in ("bq", "bk", "bv"):
            if L.get(b) is not None:
                ts.append(Tensor.f32(layer_name(l, f"self_attn.{b[1]}_proj.bias"), L[b]))
    ts.append(Tensor.f32("model.norm.weight", final_norm))
    if lm_head is not None or "lm_head.weight" in quant:
        ts.append(w("lm_head.weight", lm_head))
    return ts


def write_model_dir(path, tensors, hp, info=None, vocab=None):
    """A complete model directory.

    hp: dict hidden, layers, num_heads, num_kv_heads, head_dim, intermediate, vocab.
    info: extra model_info.json keys (rope_theta, max_position_embeddings,
    message_start, ...).  vocab: None for the byte-level vocabulary, or a pair of
    (vocab.json, merges.txt) source paths to copy."""
    os.makedirs(path, exist_ok=True)
    write_bfile(os.path.join(path, "model.bf"), tensors, hp["hidden"], hp["layers"], hp["num_heads"],
                hp["num_kv_heads"], hp["head_dim"], hp["intermediate"], hp["vocab"])
    items = {"hidden_size": hp["hidden"], "layer_count": hp["layers"], "num_heads": hp["num_heads"],
             "num_kv_heads": hp["num_kv_heads"], "head_dim": hp["head_dim"],
             "intermediate_size": hp["intermediate"], "vocab_size": hp["vocab"], "rope_theta": 10000,
             "max_position_embeddings": 1024}
    items.update(info or {})
    write_info(os.path.join(path, "model_info.json"), items)
    if vocab is None:
        write_byte_vocab(os.path.join(path, "vocab.json"), os.path.join(path, "merges.txt"))
    else:
        for src, dst in zip(vocab, ("vocab.json", "merges.txt")):
            with open(src, "rb") as fi, open(os.path.join(path, dst), "wb") as fo:
                fo.write(fi.read())
    return path
