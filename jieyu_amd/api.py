"""Python side of jieyu's text C ABI (include/jieyu_api.h) and tokenizer.

``Jieyu`` mirrors the C++ wrapper class of JieyuAI_api.h:68-146: open / close,
generate / generate_jsonl with options (max_new 256, temperature 0.7,
repetition_penalty 1.1), an output buffer of max_new*16+256 bytes, and an
exception on a negative return.  ``Tokenizer`` wraps the byte-level BPE
tokenizer of include/jieyu_text.h.
"""
import ctypes as C
from dataclasses import dataclass

from . import lib as _lib

P, I, F, S = C.c_void_p, C.c_int, C.c_float, C.c_char_p
_bound = None


def abi():
    """libjieyu_amd.so with the jieyu_* and jytext_* prototypes set."""
    global _bound
    if _bound is not None:
        return _bound
    L = _lib()
    protos = (("jieyu_load", P, [S, I]), ("jieyu_free", None, [P]), ("jieyu_last_error", S, [P]),
              ("jieyu_version", S, []), ("jieyu_context_length", I, [P]), ("jieyu_model_dir", S, [P]),
              ("jieyu_generate", I, [P, S, P, I, I, F, F]),
              ("jieyu_generate_jsonl", I, [P, S, S, S, P, I, I, F, F]),
              ("jytext_last_error", S, []), ("jytext_tokenizer_load", P, [S, S]),
              ("jytext_tokenizer_free", None, [P]), ("jytext_tokenizer_info", I, [P, P, P, P, P]),
              ("jytext_tokenizer_add_special", I, [P, S]),
              ("jytext_tokenizer_encode", I, [P, S, C.c_size_t, P, I]),
              ("jytext_tokenizer_decode", I, [P, P, I, P, I]), ("jytext_info_int", I, [S, S, I]),
              ("jytext_info_str", I, [S, S, S, P, I]), ("jytext_model_bind", I, [S, I, P]),
              ("jytext_gguf_convert", I, [S, S, I, I, I, P]))
    for name, res, args in protos:
        fn = getattr(L, name)
        fn.restype, fn.argtypes = res, args
    _bound = L
    return L


def _b(s):
    return s if isinstance(s, (bytes, type(None))) else str(s).encode("utf-8")


class JieyuError(RuntimeError):
    """jieyu::error (JieyuAI_api.h:70-73)"""


@dataclass
class Options:
    max_new: int = 256
    temperature: float = 0.7
    repetition_penalty: float = 1.1


class Jieyu:
    def __init__(self, dir=None, max_seq=0):
        self._h = None
        if dir is not None:
            self.open(dir, max_seq)

    def open(self, dir, max_seq=0):
        self.close()
        L = abi()
        h = L.jieyu_load(_b(dir), max_seq)
        if not h:
            raise JieyuError("load failed: " + L.jieyu_last_error(None).decode("utf-8", "replace"))
        self._h = h

    def close(self):
        if self._h:
            abi().jieyu_free(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def is_open(self):
        return bool(self._h)

    def context_length(self):
        return abi().jieyu_context_length(self._h) if self._h else 0

    def dir(self):
        return abi().jieyu_model_dir(self._h).decode("utf-8") if self._h else ""

    def last_error(self):
        return abi().jieyu_last_error(self._h).decode("utf-8", "replace")

    @staticmethod
    def version():
        return abi().jieyu_version().decode()

    def _check(self):
        if not self._h:
            raise JieyuError("model not loaded (open first)")

    def _buffer(self, opt):
        return C.create_string_buffer((opt.max_new if opt.max_new > 0 else 4096) * 16 + 256)

    def generate(self, prompt, opt=None, raw=False):
        """generated text (bytes with raw=True)"""
        self._check()
        opt = opt or Options()
        buf = self._buffer(opt)
        n = abi().jieyu_generate(self._h, _b(prompt), buf, len(buf), opt.max_new, opt.temperature,
                                 opt.repetition_penalty)
        if n < 0:
            raise JieyuError(self.last_error())
        return buf.value if raw else buf.value.decode("utf-8", "replace")

    def generate_jsonl(self, jsonl, qb="", qe="", opt=None, raw=False):
        self._check()
        opt = opt or Options()
        buf = self._buffer(opt)
        n = abi().jieyu_generate_jsonl(self._h, _b(jsonl), _b(qb), _b(qe), buf, len(buf), opt.max_new,
                                       opt.temperature, opt.repetition_penalty)
        if n < 0:
            raise JieyuError(self.last_error())
        return buf.value if raw else buf.value.decode("utf-8", "replace")


class Tokenizer:
    """jieyu's byte-level BPE tokenizer over vocab.json + merges.txt"""

    def __init__(self, vocab_json, merges_txt):
        L = abi()
        self._t = L.jytext_tokenizer_load(_b(vocab_json), _b(merges_txt))
        if not self._t:
            raise JieyuError(L.jytext_last_error().decode("utf-8", "replace"))

    def close(self):
        if self._t:
            abi().jytext_tokenizer_free(self._t)
            self._t = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def info(self):
        v = [C.c_int() for _ in range(4)]
        abi().jytext_tokenizer_info(self._t, *[C.byref(x) for x in v])
        return dict(zip(("vocab_size", "bos", "eos", "unk"), (x.value for x in v)))

    def add_special(self, piece):
        return abi().jytext_tokenizer_add_special(self._t, _b(piece))

    def encode(self, text):
        b = _b(text)
        n = abi().jytext_tokenizer_encode(self._t, b, len(b), None, 0)
        ids = (C.c_int32 * max(n, 1))()
        abi().jytext_tokenizer_encode(self._t, b, len(b), ids, n)
        return list(ids)[:n]

    def decode(self, ids):
        arr = (C.c_int32 * max(len(ids), 1))(*ids)
        n = abi().jytext_tokenizer_decode(self._t, arr, len(ids), None, 0)
        buf = C.create_string_buffer(max(n, 1))
        abi().jytext_tokenizer_decode(self._t, arr, len(ids), buf, n)
        return buf.raw[:n]


def model_bind(dir, max_seq=16):
    """install + bind of a model directory on the host: the hyper-parameters, or
    raises with jieyu's error text"""
    hp = (C.c_int * 12)()
    L = abi()
    if L.jytext_model_bind(_b(dir), max_seq, hp) != 0:
        raise JieyuError(L.jytext_last_error().decode("utf-8", "replace"))
    keys = ("layers", "hidden", "heads", "kv_heads", "head_dim", "intermediate", "vocab", "add_bos", "qkv_bias",
            "embed_type", "lm_head_type", "layer_type")
    return dict(zip(keys, list(hp)))


GGUF_INFO = ("hidden", "layers", "heads", "kv_heads", "head_dim", "intermediate", "vocab", "rope_theta",
             "max_position", "tensor_count", "transposed", "permuted", "quant", "tied_lm_head", "eos_id", "file_size")


def gguf_convert(src, out_dir, out_dtype="f32", quant=True, verbose=False):
    """GGUF file -> model directory (ggufc::convert, libs/gguf_libs/gguf_convert.h:260-421):
    model.bf, model_info.json, vocab.json, merges.txt.  out_dtype ("f32", "f16", "bf16"
    or the model.bf dtype code) applies to the non-quantized 2-D weights; quant keeps
    Q4_K / Q5_K / Q6_K / Q8_0 blocks.  Returns the converter's report, or raises with
    jieyu's error text."""
    L = abi()
    code = {"f32": 0, "f16": 1, "bf16": 2}.get(out_dtype, out_dtype)
    info = (C.c_longlong * 16)()
    if L.jytext_gguf_convert(_b(src), _b(out_dir), int(code), 1 if quant else 0, 1 if verbose else 0, info) != 0:
        raise JieyuError(L.jytext_last_error().decode("utf-8", "replace"))
    return dict(zip(GGUF_INFO, list(info)))

