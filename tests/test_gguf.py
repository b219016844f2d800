"""GGUF -> model directory (jytext_gguf_convert) against jieyu's own converter
(ggufc::convert, libs/gguf_libs/gguf_convert.h:260-421).

The GGUF inputs are rebuilt from tests/golden/gguf_models.py; tests/golden/gguf.json
holds, per case, what the reference converter wrote (sha256 and size of model.bf,
model_info.json, vocab.json, merges.txt), its report, or its error text
(make_gguf_golden.py).  A failed conversion here writes no file at all (the reference
may leave the files it wrote before the failure; only its error text is compared).  Where oracle/_ref is built the reference also runs on the
same files here and the outputs are compared byte for byte.  CPU only: the
converter is host code.
"""
import ctypes as C
import hashlib
import json
import os
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = os.path.join(HERE, "golden")
sys.path.insert(0, GOLD)

import gguf_models as GM  # noqa: E402
from jieyu_amd import api  # noqa: E402


@pytest.fixture(scope="module")
def gold():
    with open(os.path.join(GOLD, "gguf.json"), encoding="utf-8") as f:
        return json.load(f)


def digest(out):
    res = {}
    for f in GM.OUT_FILES:
        p = os.path.join(out, f)
        if os.path.exists(p):
            data = open(p, "rb").read()
            res[f] = [hashlib.sha256(data).hexdigest(), len(data)]
    return res


def convert(src, out, dtype, quant):
    try:
        info = api.gguf_convert(src, out, dtype, bool(quant))
        return 0, [info[k] for k in api.GGUF_INFO], ""
    except api.JieyuError as e:
        return -1, None, str(e)


@pytest.mark.parametrize("case", [c[0] for c in GM.CONVERT_CASES])
def test_convert_matches_reference(tmp_path, gold, case):
    _, model, dtype, quant, pre = next(c for c in GM.CONVERT_CASES if c[0] == case)
    src = GM.MODELS[model]().write(str(tmp_path / (model + ".gguf")))
    out = str(tmp_path / "out")
    if pre is not None:  # an existing model_info.json is updated, its other keys kept
        os.makedirs(out)
        open(os.path.join(out, "model_info.json"), "w").write(pre)
    rc, info, err = convert(src, out, dtype, quant)
    assert rc == 0, err
    want = gold["convert"][case]
    assert info == want["info"]
    got = digest(out)
    for f in GM.OUT_FILES:
        assert got.get(f) == want["files"].get(f), f"{case}: {f} differs (size {got.get(f, [0, 0])[1]} vs " \
                                                    f"{want['files'].get(f, [0, 0])[1]})"


@pytest.mark.parametrize("name", [b[0] for b in GM.bad_files()])
def test_errors_match_reference(tmp_path, gold, name):
    data = dict(GM.bad_files())[name]
    src = str(tmp_path / (name + ".gguf"))
    open(src, "wb").write(data)
    out = str(tmp_path / "out")
    rc, _, err = convert(src, out, 0, 1)
    want = gold["errors"][name]
    assert rc == want["rc"]
    assert err == want["error"]
    if rc == 0:
        assert digest(out) == want["files"]
    else:  # everything is checked before the first file is written: a failure leaves nothing
        assert digest(out) == {}


def test_converted_model_binds(tmp_path):
    """the quantized conversion binds with jieyu's checks: k-quant matrices, Q6_K
    embedding as the tied head"""
    src = GM.llama_q4km().write(str(tmp_path / "m.gguf"))
    out = str(tmp_path / "m")
    api.gguf_convert(src, out, "f32", True)
    hp = api.model_bind(out, 64)
    assert hp["hidden"] == 256 and hp["vocab"] == 259 and hp["layers"] == 2
    assert hp["embed_type"] == 7 and hp["lm_head_type"] == 7 and hp["layer_type"] == 5  # q6_K, q6_K, q4_K


def test_perm_row_restores_adjacent_pairs(tmp_path):
    """q rows come back in jieyu's adjacent-pair order: f32 output row j of a head is
    GGUF row perm_row(j) = (j odd ? hd/2 + j/2 : j/2) of that head"""
    import numpy as np
    import gguf_writer as G
    hidden, hd = 64, 16
    g = GM.deepseek_f32()
    q = np.arange(hidden * hidden, dtype=np.float32).reshape(hidden, hidden)  # GGUF rows (out) x in
    g.tensors = [(n, s, t, q.tobytes() if n == "blk.0.attn_q.weight" else d) for (n, s, t, d) in g.tensors]
    g.kv.append(("llama.attention.key_length", G.U32, hd, None))
    src = g.write(str(tmp_path / "p.gguf"))
    out = str(tmp_path / "p")
    api.gguf_convert(src, out, "f32", True)
    raw = open(os.path.join(out, "model.bf"), "rb").read()
    n = int.from_bytes(raw[42:46], "little")
    data_off = int.from_bytes(raw[46:50], "little")
    for i in range(n):
        e = raw[64 + 104 * i: 64 + 104 * (i + 1)]
        if e[:64].split(b"\0")[0] == b"model.layers.0.self_attn.q_proj.weight":
            off, nb = int.from_bytes(e[88:96], "little"), int.from_bytes(e[96:104], "little")
            w = np.frombuffer(raw[data_off + off: data_off + off + nb], np.float32).reshape(hidden, hidden)  # [in][out]
            perm = [(j // hd) * hd + ((j % hd) // 2 + (hd // 2 if j % 2 else 0)) for j in range(hidden)]
            assert np.array_equal(w.T, q[perm])
            return
    pytest.fail("q_proj not found")


@pytest.mark.parametrize("hd", [24, 15])
def test_pairs_need_whole_heads(tmp_path, hd):
    """a key_length that does not split the q / k rows into whole heads of an even size is
    refused before any file is written (the row permutation would read past the tensor)"""
    import gguf_writer as G
    g = GM.deepseek_f32()  # hidden 64: q / k have 64 rows
    g.kv.append(("llama.attention.key_length", G.U32, hd, None))
    src = g.write(str(tmp_path / "bad.gguf"))
    out = str(tmp_path / "out")
    rc, _, err = convert(src, out, "f32", True)
    assert rc == -1
    assert "head_dim" in err and "attn_q" in err
    assert digest(out) == {}


def test_reference_live(tmp_path):
    """the reference converter on the same GGUF bytes, compared file by file"""
    import oracle
    if not oracle.ref_available():
        pytest.skip("oracle/_ref/libjyref.so not built")
    ref = oracle.load_ref()
    ref.jyref_gguf_convert.restype = C.c_int
    ref.jyref_gguf_convert.argtypes = [C.c_char_p, C.c_char_p, C.c_int, C.c_int, C.c_void_p, C.c_char_p, C.c_int]
    for case, model, dtype, quant, pre in GM.CONVERT_CASES[:5]:
        src = GM.MODELS[model]().write(str(tmp_path / (model + ".gguf")))
        a, b = str(tmp_path / (case + "-ref")), str(tmp_path / (case + "-ours"))
        err = C.create_string_buffer(256)
        assert ref.jyref_gguf_convert(src.encode(), a.encode(), dtype, quant, None, err, 256) == 0, err.value
        convert(src, b, dtype, quant)
        for f in GM.OUT_FILES:
            assert open(os.path.join(a, f), "rb").read() == open(os.path.join(b, f), "rb").read(), (case, f)


def test_bfile_writer_kquant_directory_binds(tmp_path):
    """jieyu_amd.bfile writes k-quant, Q8_0 and f16 tensors that bind with jieyu's
    checks, each slot keeping its own type"""
    import numpy as np
    import quant_models as QM
    import jieyu_amd.bfile as B
    m = QM.build_model("kq-mixed")
    code = {QM.JY_Q8_0: B.Q8_0, QM.JY_Q4_K: B.Q4K, QM.JY_Q5_K: B.Q5K, QM.JY_Q6_K: B.Q6K}
    names = dict(Wq="self_attn.q_proj.weight", Wk="self_attn.k_proj.weight", Wv="self_attn.v_proj.weight",
                 Wo="self_attn.o_proj.weight", W1="mlp.gate_proj.weight", W2="mlp.down_proj.weight",
                 W3="mlp.up_proj.weight")
    H, F, qd, kvd, V = m["hidden"], m["inter"], m["heads"] * m["hd"], m["kv"] * m["hd"], m["vocab"]
    dims = dict(Wq=(qd, H), Wk=(kvd, H), Wv=(kvd, H), Wo=(H, qd), W1=(F, H), W2=(H, F), W3=(F, H))
    quant, layers = {}, []
    for l, L in enumerate(m["layers"]):
        layers.append(dict(rms1=L["rms1"], rms2=L["rms2"]))
        for slot, nm in names.items():
            t, blob = L[slot]
            quant[B.layer_name(l, nm)] = (code[t], *dims[slot], blob)
    quant["model.embed_tokens.weight"] = (code[m["embed"][0]], V, H, m["embed"][1])
    quant["lm_head.weight"] = (code[m["lm"][0]], V, H, m["lm"][1])
    ts = B.decoder_tensors(None, None, m["final"], layers, quant=quant)
    hp = dict(hidden=H, layers=len(layers), num_heads=m["heads"], num_kv_heads=m["kv"], head_dim=m["hd"],
              intermediate=F, vocab=V)
    d = B.write_model_dir(str(tmp_path / "kq"), ts, hp)
    got = api.model_bind(d, 32)
    assert (got["embed_type"], got["lm_head_type"], got["layer_type"]) == (QM.JY_Q6_K, QM.JY_Q4_K, QM.JY_Q4_K)
    # an f16 tensor round-trips as dtype F16
    t = B.Tensor.f16("x", np.ones((2, 3), np.float16))
    assert t.dtype == B.F16 and len(t.data) == 12


def _patch_tensor(raw, name, dims=None, offset=None):
    """raw GGUF v3 bytes with tensor `name`'s dims and/or data offset replaced in its
    tensor-info record (same dimension count, so the layout is unchanged)"""
    import struct
    key = struct.pack("<Q", len(name)) + name.encode()
    at = raw.index(key) + len(key)
    nd = struct.unpack_from("<I", raw, at)[0]
    b = bytearray(raw)
    if dims is not None:
        assert len(dims) == nd
        struct.pack_into("<" + "Q" * nd, b, at + 4, *dims)
    if offset is not None:
        struct.pack_into("<Q", b, at + 4 + 8 * nd + 4, offset)
    return bytes(b)


# corrupt tensor records and headers that once got past the range checks: a zero dim beside
# a huge one (an endless panel loop), a dim past model.bf's 32 bits, a byte count that wraps
# 64 bits, a data offset that wraps the start of the range, an alignment past the file
@pytest.mark.parametrize("case,want", [("zero_dim", "维度不对"), ("dim_over_32bit", "维度不对"),
                                       ("bytes_wrap", "字节数溢出"), ("offset_wraps", "写张量失败"),
                                       ("align_past_file", "alignment")])
def test_corrupt_records_fail_cleanly(tmp_path, case, want):
    """each is refused with an error before any file is written"""
    import gguf_writer as G
    g = GM.deepseek_f32()
    if case == "align_past_file":
        g.kv.append(("general.alignment", G.U32, 1 << 31, None))
    raw = g.bytes()
    name = "blk.0.attn_output.weight"
    if case == "zero_dim":
        raw = _patch_tensor(raw, name, dims=(2 ** 63 + 64, 0))
    elif case == "dim_over_32bit":
        raw = _patch_tensor(raw, name, dims=(2 ** 32, 1))
    elif case == "bytes_wrap":
        raw = _patch_tensor(raw, name, dims=(2 ** 32 - 1, 2 ** 32 - 1))
    elif case == "offset_wraps":
        raw = _patch_tensor(raw, name, offset=2 ** 64 - 16)
    src = str(tmp_path / "bad.gguf")
    open(src, "wb").write(raw)
    out = str(tmp_path / "out")
    rc, _, err = convert(src, out, "f32", True)
    assert rc == -1 and want in err, err
    assert digest(out) == {}


def _mutate(data, rng):
    """one random corruption: a truncation, byte flips in the first 4 KiB or anywhere, or a
    random 4- / 8-byte value (8-byte ones often edge values) at a header offset"""
    b = bytearray(data)
    kind = rng.randrange(5)
    hdr = min(len(b), 4096)
    if kind == 0:
        return bytes(b[:rng.randrange(len(b))])
    if kind == 1:
        for _ in range(rng.randrange(1, 8)):
            b[rng.randrange(hdr)] = rng.randrange(256)
    elif kind == 2:
        o = rng.randrange(0, max(1, hdr - 8)) & ~7
        v = rng.choice([0, 1, 2 ** 31, 2 ** 32 - 1, 2 ** 63, 2 ** 64 - 1, rng.randrange(2 ** 64)])
        b[o:o + 8] = v.to_bytes(8, "little")
    elif kind == 3:
        o = rng.randrange(0, max(1, hdr - 4))
        b[o:o + 4] = rng.randrange(2 ** 32).to_bytes(4, "little")
    else:
        for _ in range(rng.randrange(1, 32)):
            b[rng.randrange(len(b))] = rng.randrange(256)
    return bytes(b)


@pytest.mark.parametrize("model", list(GM.MODELS))
def test_mutated_files_fail_cleanly(tmp_path, model):
    """150 seeded random corruptions of each synthetic GGUF file: each converts or fails with
    an error and writes nothing (a crash or a hang would end the test run).  The same sweep
    at 3000 corruptions per file, against the host-sanitized library (ASan + UBSan), found
    the cases of test_corrupt_records_fail_cleanly and now reports nothing."""
    import random
    import shutil
    data = open(GM.MODELS[model]().write(str(tmp_path / "m.gguf")), "rb").read()
    src, out = str(tmp_path / "f.gguf"), str(tmp_path / "out")
    ok = 0
    for seed in range(150):
        open(src, "wb").write(_mutate(data, random.Random(seed)))
        shutil.rmtree(out, ignore_errors=True)
        rc, _, _ = convert(src, out, "f32", False)
        if rc == 0:
            ok += 1
        else:
            assert digest(out) == {}, f"seed {seed}: a failed conversion left files"
    assert 0 < ok < 150


@pytest.mark.parametrize("target", ["model.bf", "model_info.json", "vocab.json", "merges.txt"])
def test_mutated_model_directory(tmp_path, target):
    """a converted model directory with one file corrupted (100 seeded corruptions): binding
    it (model.bf, model_info.json) or loading its tokenizer (vocab.json, merges.txt) and
    coding a few texts either works or raises.  The same sweep at 1000 corruptions per file,
    against the host-sanitized library, reports nothing."""
    import random
    import shutil
    base = str(tmp_path / "base")
    api.gguf_convert(GM.MODELS["qwen-mixed"]().write(str(tmp_path / "m.gguf")), base, "f32", True)
    files = {f: open(os.path.join(base, f), "rb").read() for f in os.listdir(base)}
    d = str(tmp_path / "d")
    for seed in range(100):
        shutil.rmtree(d, ignore_errors=True)
        os.makedirs(d)
        for f, b in files.items():
            open(os.path.join(d, f), "wb").write(b)
        open(os.path.join(d, target), "wb").write(_mutate(files[target], random.Random(seed)))
        try:
            if target in ("model.bf", "model_info.json"):
                api.model_bind(d)
            else:
                t = api.Tokenizer(os.path.join(d, "vocab.json"), os.path.join(d, "merges.txt"))
                for text in ("hello world", "abé中文 <|x|> 123", ""):
                    t.decode(t.encode(text) + [0, 1, 2, 10 ** 6, -5])
                t.close()
        except api.JieyuError:
            pass
