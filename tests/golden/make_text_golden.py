"""Write the text-path fixtures of tests/golden/ from jieyu's own code.

Needs the reference build (`make -C oracle ref` -> oracle/_ref/libjyref.so), which
exports jieyu's tokenizer, JSON lookups, model-directory bind, BPE trainer and
its text C ABI (main.hpp) compiled from the reference sources.

    python tests/golden/make_text_golden.py

Writes
  tok_bpe/vocab.json, tok_bpe/merges.txt  a BPE vocabulary trained by jieyu's
        BPETrainer on the corpus below, plus the two chat markers appended;
  text.json  tokenizer ids, JSON lookups, model-directory binds, and the
        records of every C ABI script of text_models.SCRIPTS / LOAD_ERRORS.
"""
import ctypes as C
import json
import os
import platform
import shutil
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, HERE)
import oracle  # noqa: E402
import text_models as TM  # noqa: E402
import jieyu_amd  # noqa: E402

SENTENCES = [
    "The quick brown fox jumps over the lazy dog.",
    "the theory of the thing is that they then thought about it",
    "Hello, JieYu AI! How are you today?",
    "A language model predicts the next token from the ones before it.",
    "int main(void) { return f(x) + g[y]; } // comment",
    "你好，世界！今天天气很好。",
    "昆仑分词器把文本切成词，再合并成更长的片段。",
    "mixed 中文 and English text, with numbers 1234 and 3.14159.",
    "user: what is the capital of France? assistant: Paris.",
    "they think that the other thing is better than this one",
]


def corpus(n_lines=2000, seed=5):
    rng = np.random.default_rng(seed)
    lines = []
    for _ in range(n_lines):
        k = int(rng.integers(1, 4))
        lines.append(" ".join(SENTENCES[int(i)] for i in rng.integers(0, len(SENTENCES), k)))
    return "\n".join(lines) + "\n"


def train_tokenizer(ref, target_vocab=700):
    tmp = tempfile.mkdtemp(prefix="jy_tok_")
    try:
        cpath = os.path.join(tmp, "corpus.txt")
        with open(cpath, "w", encoding="utf-8") as f:
            f.write(corpus())
        n = ref.jyref_train_bpe(cpath.encode(), target_vocab, tmp.encode())
        assert n > 0, "trainer failed"
        with open(os.path.join(tmp, "vocab.json"), encoding="utf-8") as f:
            vocab = json.load(f)
        nxt = max(vocab.values()) + 1
        for i, m in enumerate(TM.MARKERS):
            vocab[m] = nxt + i
        os.makedirs(TM.TOK_DIR, exist_ok=True)
        with open(os.path.join(TM.TOK_DIR, "vocab.json"), "w", encoding="utf-8") as f:
            json.dump(vocab, f, ensure_ascii=False)
        shutil.copyfile(os.path.join(tmp, "merges.txt"), os.path.join(TM.TOK_DIR, "merges.txt"))
        return n
    finally:
        shutil.rmtree(tmp, ignore_errors=True)


def tok_case(ref, vocab, merges, specials):
    t = ref.jyref_tok_load(vocab.encode(), merges.encode())
    assert t
    for s in specials:
        ref.jyref_tok_add_special(t, s.encode())
    vs, bos, eos, unk = C.c_int(), C.c_int(), C.c_int(), C.c_int()
    ref.jyref_tok_info(t, C.byref(vs), C.byref(bos), C.byref(eos), C.byref(unk))
    out = {"vocab_size": vs.value, "bos": bos.value, "eos": eos.value, "unk": unk.value, "specials": list(specials),
           "cases": []}
    for s in TM.TOKENIZER_STRINGS:
        n = ref.jyref_tok_encode(t, s, len(s), None, 0)
        ids = (C.c_int32 * max(n, 1))()
        ref.jyref_tok_encode(t, s, len(s), ids, n)
        idl = list(ids)[:n]
        nb = ref.jyref_tok_decode(t, (C.c_int32 * max(n, 1))(*idl), n, None, 0)
        buf = C.create_string_buffer(max(nb, 1))
        ref.jyref_tok_decode(t, (C.c_int32 * max(n, 1))(*idl), n, buf, nb)
        out["cases"].append({"text_hex": s.hex(), "ids": idl, "decoded_hex": buf.raw[:nb].hex()})
    ref.jyref_tok_free(t)
    return out


INFO_DOC = {"a": 1, "neg": -7, "big": 99999999999, "float": 500000.0, "exp": 1e6, "str_num": "12",
            "str": "hello", "empty": "", "t": True, "n": None, "nested": {"x": {"y": 42}}, "arr": [1, 2],
            "a.b": 5, "uni": "你好 \\ \" \n", "lead": " 17", "plus": "+3"}
INFO_KEYS = ["a", "neg", "big", "float", "exp", "str_num", "str", "empty", "t", "n", "nested.x.y", "nested.x",
             "arr", "a.b", "uni", "lead", "plus", "missing", "nested.missing", "nested"]


def info_case(ref, tmp):
    path = os.path.join(tmp, "info.json")
    with open(path, "w", encoding="utf-8") as f:
        json.dump(INFO_DOC, f, ensure_ascii=False, indent=2)
    out = {"doc": INFO_DOC, "ints": {}, "strs": {}}
    buf = C.create_string_buffer(256)
    for k in INFO_KEYS:
        out["ints"][k] = ref.jyref_info_int(path.encode(), k.encode(), -99)
        ref.jyref_info_str(path.encode(), k.encode(), b"<fb>", buf, 256)
        out["strs"][k] = buf.value.decode("utf-8")
    return out


def bind_case(ref, path):
    hp = (C.c_int * 9)()
    err = C.create_string_buffer(512)
    rc = ref.jyref_model_bind(path.encode(), 16, hp, err, 512)
    return {"rc": rc, "hp": list(hp) if rc == 0 else None, "err": err.value.decode("utf-8")}


def main():
    ref = oracle.load_ref()
    P, I, S = C.c_void_p, C.c_int, C.c_char_p
    for name, res, args in (("jyref_tok_load", P, [S, S]), ("jyref_tok_free", None, [P]),
                            ("jyref_tok_info", I, [P, P, P, P, P]), ("jyref_tok_add_special", I, [P, S]),
                            ("jyref_tok_encode", I, [P, S, C.c_size_t, P, I]),
                            ("jyref_tok_decode", I, [P, P, I, P, I]), ("jyref_info_int", I, [S, S, I]),
                            ("jyref_info_str", I, [S, S, S, P, I]), ("jyref_model_bind", I, [S, I, P, P, I]),
                            ("jyref_train_bpe", I, [S, I, S]), ("jyref_write_byte_vocab", I, [S, S])):
        fn = getattr(ref, name)
        fn.restype, fn.argtypes = res, args
    TM.bind_abi(ref)
    qlib = jieyu_amd.lib()

    trained = train_tokenizer(ref)
    tmp = tempfile.mkdtemp(prefix="jy_text_golden_")
    try:
        bv, bm = os.path.join(tmp, "bv.json"), os.path.join(tmp, "bm.txt")
        ref.jyref_write_byte_vocab(bv.encode(), bm.encode())
        from jieyu_amd import bfile as B
        mv, mm = os.path.join(tmp, "mv.json"), os.path.join(tmp, "mm.txt")
        B.write_byte_vocab(mv, mm)
        assert open(bv, "rb").read() == open(mv, "rb").read() and open(bm, "rb").read() == open(mm, "rb").read()

        tok = {"bpe": tok_case(ref, os.path.join(TM.TOK_DIR, "vocab.json"), os.path.join(TM.TOK_DIR, "merges.txt"),
                               TM.MARKERS),
               "bpe_plain": tok_case(ref, os.path.join(TM.TOK_DIR, "vocab.json"),
                                     os.path.join(TM.TOK_DIR, "merges.txt"), ()),
               "byte": tok_case(ref, bv, bm, ())}
        info = info_case(ref, tmp)
        dirs = os.path.join(tmp, "dirs")
        binds = {}
        for kind in ("bind", "bind:wrong_shape", "bind:missing", "bpe_f32", "bpe_q8", "demo", "noinfo",
                     "badmagic", "nodir"):
            binds[kind] = bind_case(ref, TM.build_dir(kind, dirs, qlib))
        scripts = {kind: TM.run_script(ref, dirs, kind, ms, calls, qlib) for kind, ms, calls in TM.SCRIPTS}
        load_errors = {kind: TM.run_load_error(ref, dirs, kind) for kind in TM.LOAD_ERRORS}
    finally:
        shutil.rmtree(tmp, ignore_errors=True)

    doc = {"source": "jieyu's tokenizer, json_libs, bind_model, BPETrainer and main.hpp C ABI compiled from the "
                     "reference sources by oracle/Makefile (make ref)",
           "host": {"machine": platform.machine(), "libc": " ".join(platform.libc_ver())},
           "trained_vocab": trained, "tokenizer": tok, "info": info, "bind": binds, "scripts": scripts,
           "load_errors": load_errors}
    with open(os.path.join(HERE, "text.json"), "w", encoding="utf-8") as f:
        json.dump(doc, f, ensure_ascii=False, indent=1)
    print("wrote", os.path.join(HERE, "text.json"))


if __name__ == "__main__":
    main()
