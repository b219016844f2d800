"""The text layer of the C ABI on the CPU: model-directory writer and loader,
tokenizer, model_info.json lookups, and jieyu_load's error behaviour.

Expected values come from jieyu's own code (tests/golden/text.json, written by
make_text_golden.py from the reference compiled in oracle/_ref) and from the
reference's bind_test fixtures (tests/golden/bind_test/*/model.bf).  Where the
reference build is present the tokenizer is also compared on random text.
"""
import ctypes as C
import json
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")
sys.path.insert(0, GOLDEN)

import text_models as TM  # noqa: E402
from jieyu_amd import api  # noqa: E402
from jieyu_amd import bfile as B  # noqa: E402
from kat_models import bind_test_model  # noqa: E402


@pytest.fixture(scope="module")
def gold():
    with open(os.path.join(GOLDEN, "text.json"), encoding="utf-8") as f:
        return json.load(f)


@pytest.fixture(scope="module")
def L():
    return api.abi()


@pytest.fixture(scope="module")
def dirs(tmp_path_factory):
    import jieyu_amd
    root = str(tmp_path_factory.mktemp("models"))
    return root, jieyu_amd.lib()


# ------------------------------------------------------------ model.bf writer

def _ref_order(m, wrong_q=False, drop_norm=False):
    """tensor order of the reference test's write_model_dir (libs/text/text.h:612-656)"""
    ts = [B.Tensor.f32("model.embed_tokens.weight", m["embed"])]
    if not drop_norm:
        ts.append(B.Tensor.f32("model.norm.weight", m["final"]))
    for l, w in enumerate(m["layers"]):
        q = w["Wq"].reshape(w["Wq"].shape[::-1]) if wrong_q else w["Wq"]
        for sfx, a in (("input_layernorm.weight", w["rms1"]), ("self_attn.q_proj.weight", q),
                       ("self_attn.k_proj.weight", w["Wk"]), ("self_attn.v_proj.weight", w["Wv"]),
                       ("self_attn.o_proj.weight", w["Wo"]), ("post_attention_layernorm.weight", w["rms2"]),
                       ("mlp.gate_proj.weight", w["W1"]), ("mlp.down_proj.weight", w["W2"]),
                       ("mlp.up_proj.weight", w["W3"])):
            ts.append(B.Tensor.f32(B.layer_name(l, sfx), a))
    ts.append(B.Tensor.f32("lm_head.weight", m["lm"]))
    return ts


@pytest.mark.parametrize("which,kw,opt", [("model", {}, {}),
                                          ("wrong_shape", dict(hd=6, layers=1), dict(wrong_q=True)),
                                          ("missing", dict(layers=1), dict(drop_norm=True))])
def test_writer_reproduces_reference_fixtures(tmp_path, which, kw, opt):
    """the reference's three bind_test model.bf files, byte for byte, from the
    restated weight generator and this writer"""
    m = bind_test_model(**kw)
    p = str(tmp_path / "model.bf")
    B.write_bfile(p, _ref_order(m, **opt), m["hidden"], len(m["layers"]), m["heads"], m["kv"], m["hd"],
                  m["inter"], m["vocab"])
    with open(p, "rb") as a, open(os.path.join(GOLDEN, "bind_test", which, "model.bf"), "rb") as b:
        assert a.read() == b.read()


def test_byte_vocab_writer(tmp_path, gold):
    v, m = str(tmp_path / "vocab.json"), str(tmp_path / "merges.txt")
    B.write_byte_vocab(v, m)
    with open(v, encoding="utf-8") as f:
        doc = json.load(f)
    assert len(doc) == 256 and sorted(doc.values()) == list(range(256))
    assert doc["a"] == 97 and doc["Ā"] == 0 and doc["Ġ"] == 32  # byte 0 -> U+0100, ' ' -> U+0120
    t = api.Tokenizer(v, m)
    g = gold["tokenizer"]["byte"]
    assert t.info() == {k: g[k] for k in ("vocab_size", "bos", "eos", "unk")}


# ------------------------------------------------------------ model-directory bind

@pytest.mark.parametrize("kind", ["bind", "bind:wrong_shape", "bind:missing", "bpe_f32", "bpe_q8", "demo",
                                  "noinfo", "badmagic", "nodir"])
def test_model_bind_matches_reference(dirs, gold, kind):
    root, qlib = dirs
    g = gold["bind"][kind]
    path = TM.build_dir(kind, root, qlib)
    if g["rc"] == 0:
        hp = api.model_bind(path)
        got = [hp[k] for k in ("layers", "hidden", "heads", "kv_heads", "head_dim", "intermediate", "vocab",
                               "add_bos", "qkv_bias")]
        assert got == g["hp"]
    else:
        with pytest.raises(api.JieyuError) as e:
            api.model_bind(path)
        assert str(e.value) == g["err"]


def test_model_bind_weight_types(dirs):
    root, qlib = dirs
    f32 = api.model_bind(TM.build_dir("bpe_f32", root, qlib))
    q8 = api.model_bind(TM.build_dir("bpe_q8", root, qlib))
    assert (f32["embed_type"], f32["lm_head_type"], f32["layer_type"]) == (0, 0, 0)
    assert (q8["embed_type"], q8["lm_head_type"], q8["layer_type"]) == (3, 3, 3)   # tied Q8_0 lm_head


def test_model_bind_rejects_broken_table(tmp_path):
    p = TM.bind_dir(str(tmp_path / "d"))
    with open(os.path.join(p, "model.bf"), "r+b") as f:   # first entry's nbytes no longer matches its shape
        f.seek(64 + 96)
        f.write((12345).to_bytes(8, "little"))
    with pytest.raises(api.JieyuError) as e:
        api.model_bind(p)
    assert str(e.value) == "装载 model.bf 失败: model.bf tensor table broken"


def test_model_bind_v1_file(tmp_path):
    p = TM.bind_dir(str(tmp_path / "d"))
    with open(os.path.join(p, "model.bf"), "r+b") as f:   # version 1: no tensor table
        f.seek(38)
        f.write((1).to_bytes(4, "little"))
    with pytest.raises(api.JieyuError) as e:
        api.model_bind(p)
    assert str(e.value) == "model.bf 没有张量目录,请先用 jieyu -convert 转化"


# ------------------------------------------------------------ tokenizer

@pytest.mark.parametrize("case", ["bpe", "bpe_plain", "byte"])
def test_tokenizer_matches_reference_golden(tmp_path, gold, case):
    g = gold["tokenizer"][case]
    if case == "byte":
        v, m = str(tmp_path / "v.json"), str(tmp_path / "m.txt")
        B.write_byte_vocab(v, m)
    else:
        v, m = os.path.join(TM.TOK_DIR, "vocab.json"), os.path.join(TM.TOK_DIR, "merges.txt")
    t = api.Tokenizer(v, m)
    for s in g["specials"]:
        assert t.add_special(s) >= 0
    assert t.info() == {k: g[k] for k in ("vocab_size", "bos", "eos", "unk")}
    assert len(g["cases"]) == len(TM.TOKENIZER_STRINGS)
    for c in g["cases"]:
        text = bytes.fromhex(c["text_hex"])
        ids = t.encode(text)
        assert ids == c["ids"], text
        assert t.decode(ids) == bytes.fromhex(c["decoded_hex"]), text


def test_tokenizer_reference_kats(tmp_path):
    """check_pipeline 2-5 (libs/text/text.h:959-990): 259 tokens, lossless round
    trips, encode("abc") = {97, 98, 99}"""
    v, m = str(tmp_path / "v.json"), str(tmp_path / "m.txt")
    B.write_byte_vocab(v, m)
    t = api.Tokenizer(v, m)
    assert t.info()["vocab_size"] == 259
    for s in ("Hello, JieYu AI!", "你好，世界！昆仑分词器。"):
        assert t.decode(t.encode(s)) == s.encode()
    assert t.encode("abc") == [97, 98, 99]


def test_tokenizer_bpe_round_trip_and_merges():
    t = api.Tokenizer(os.path.join(TM.TOK_DIR, "vocab.json"), os.path.join(TM.TOK_DIR, "merges.txt"))
    rng = np.random.default_rng(3)
    words = ["the", "theory", "thing", " they", "你好", "世界", "Paris", "1234", "!", " ", "\n", "token"]
    for _ in range(50):
        s = "".join(words[i] for i in rng.integers(0, len(words), 12))
        ids = t.encode(s)
        assert t.decode(ids) == s.encode()
        assert len(ids) < len(s.encode())  # merges shorten every such string


def _random_text(rng, n):
    pool = ["a", "b", "the", "th", "e", " ", "  ", "\t", "\n", ",", ".", "!", "你", "好", "，", "。", "<|im_start|>",
            "<|im_end|>", "<|", "|>", "<unk>", "</w>", "<｜begin▁of▁sentence｜>", "　", "é", "\U0001F600", "0",
            "42", "x", "Paris", "theory"]
    parts = [pool[int(i)].encode() for i in rng.integers(0, len(pool), n)]
    if rng.random() < 0.3:
        parts.append(bytes([int(rng.integers(0x80, 0x100))]))
    return b"".join(parts)


def test_tokenizer_matches_reference_random(ref_lib):
    """random strings through both tokenizers (needs the reference build)"""
    R = ref_lib
    for name, res, args in (("jyref_tok_load", C.c_void_p, [C.c_char_p, C.c_char_p]),
                            ("jyref_tok_add_special", C.c_int, [C.c_void_p, C.c_char_p]),
                            ("jyref_tok_encode", C.c_int, [C.c_void_p, C.c_char_p, C.c_size_t, C.c_void_p, C.c_int]),
                            ("jyref_tok_free", None, [C.c_void_p])):
        getattr(R, name).restype, getattr(R, name).argtypes = res, args
    v, m = os.path.join(TM.TOK_DIR, "vocab.json"), os.path.join(TM.TOK_DIR, "merges.txt")
    rt = R.jyref_tok_load(v.encode(), m.encode())
    t = api.Tokenizer(v, m)
    for s in TM.MARKERS:
        R.jyref_tok_add_special(rt, s.encode())
        t.add_special(s)
    rng = np.random.default_rng(11)
    try:
        for _ in range(400):
            s = _random_text(rng, int(rng.integers(0, 24)))
            n = R.jyref_tok_encode(rt, s, len(s), None, 0)
            ids = (C.c_int32 * max(n, 1))()
            R.jyref_tok_encode(rt, s, len(s), ids, n)
            assert t.encode(s) == list(ids)[:n], s
    finally:
        R.jyref_tok_free(rt)


def test_tokenizer_load_errors(tmp_path):
    with pytest.raises(api.JieyuError):
        api.Tokenizer(str(tmp_path / "none.json"), str(tmp_path / "none.txt"))
    (tmp_path / "v.json").write_text("{}")
    (tmp_path / "m.txt").write_text("")
    with pytest.raises(api.JieyuError):
        api.Tokenizer(str(tmp_path / "v.json"), str(tmp_path / "m.txt"))   # empty vocabulary


# ------------------------------------------------------------ model_info.json

def test_info_lookups_match_reference(tmp_path, gold, L):
    g = gold["info"]
    p = str(tmp_path / "info.json")
    with open(p, "w", encoding="utf-8") as f:
        json.dump(g["doc"], f, ensure_ascii=False, indent=2)
    buf = C.create_string_buffer(256)
    for k, want in g["ints"].items():
        assert L.jytext_info_int(p.encode(), k.encode(), -99) == want, k
    for k, want in g["strs"].items():
        L.jytext_info_str(p.encode(), k.encode(), b"<fb>", buf, 256)
        assert buf.value.decode("utf-8") == want, k
    assert L.jytext_info_int(str(tmp_path / "absent.json").encode(), b"a", 5) == 5


# ------------------------------------------------------------ jieyu_load without a device

@pytest.mark.parametrize("kind", TM.LOAD_ERRORS)
def test_load_errors_match_reference(dirs, gold, L, kind):
    """directories that fail before any device work: NULL handle, the reference's text"""
    root, qlib = dirs
    g = gold["load_errors"][kind]
    got = TM.run_load_error(L, root, kind)
    assert got["loaded"] is False
    if kind == "novocab":
        # the message names the two files (the golden was made under another temporary root)
        path = os.path.join(root, "novocab")
        want = "分词器加载失败: %s / %s" % (os.path.join(path, "vocab.json"), os.path.join(path, "merges.txt"))
        assert got["err"] == want and g["err"].startswith("分词器加载失败: ")
    else:
        assert got["err"] == g["err"]


def test_null_arguments(L):
    assert not L.jieyu_load(None, 0)
    assert L.jieyu_last_error(None).decode() == "dir 为空"
    assert L.jieyu_generate(None, b"x", None, 0, 4, 0.0, 1.0) == -1
    assert L.jieyu_last_error(None).decode() == "句柄为空"
    assert L.jieyu_generate_jsonl(None, b"x", None, None, None, 0, 4, 0.0, 1.0) == -1
    assert L.jieyu_version().decode() == "1.0.0"
    assert L.jieyu_context_length(None) == 0
    assert L.jieyu_model_dir(None).decode() == ""


def test_load_needs_a_device(dirs, L):
    """a valid directory on a host without a GPU: the load fails loudly at the
    device upload, it does not fall back to the CPU"""
    import jieyu_amd
    if jieyu_amd.device_count() > 0:
        pytest.skip("a GPU is visible")
    root, qlib = dirs
    h = L.jieyu_load(TM.build_dir("bind", root, qlib).encode(), 8)
    assert not h
    assert L.jieyu_last_error(None).decode().startswith("device upload failed")
