"""Write tests/golden/gguf.json from jieyu's own GGUF converter (ggufc::convert,
libs/gguf_libs/gguf_convert.h:260-421, compiled by oracle/Makefile into
oracle/_ref/libjyref.so): for each GGUF file of gguf_models.py the sha256 and size
of the four files it writes, its report, or its error text.  The GGUF inputs are
rebuilt by the tests from gguf_models.py (numpy PCG64 seeds).

    python tests/golden/make_gguf_golden.py
"""
import ctypes as C
import hashlib
import json
import os
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, HERE)

import gguf_models as GM  # noqa: E402
import oracle  # noqa: E402


def ref_convert(ref, src, out, dtype, quant):
    info = (C.c_longlong * 16)()
    err = C.create_string_buffer(512)
    rc = ref.jyref_gguf_convert(src.encode(), out.encode(), dtype, quant, info, err, 512)
    return rc, list(info), err.value.decode("utf-8", "replace")


def digest(out):
    res = {}
    for f in GM.OUT_FILES:
        p = os.path.join(out, f)
        if os.path.exists(p):
            data = open(p, "rb").read()
            res[f] = [hashlib.sha256(data).hexdigest(), len(data)]
    return res


def main():
    if not oracle.ref_available():
        sys.exit("oracle/_ref/libjyref.so is missing: run `make -C oracle ref` where the reference tree exists")
    ref = oracle.load_ref()
    ref.jyref_gguf_convert.restype = C.c_int
    ref.jyref_gguf_convert.argtypes = [C.c_char_p, C.c_char_p, C.c_int, C.c_int, C.c_void_p, C.c_char_p, C.c_int]
    gold = {"convert": {}, "errors": {}}
    with tempfile.TemporaryDirectory() as tmp:
        for case, model, dtype, quant, pre in GM.CONVERT_CASES:
            src = GM.MODELS[model]().write(os.path.join(tmp, model + ".gguf"))
            out = os.path.join(tmp, case)
            if pre is not None:
                os.makedirs(out)
                open(os.path.join(out, "model_info.json"), "w").write(pre)
            rc, info, err = ref_convert(ref, src, out, dtype, quant)
            assert rc == 0, (case, err)
            gold["convert"][case] = {"info": info, "files": digest(out)}
        for name, data in GM.bad_files():
            src = os.path.join(tmp, name + ".gguf")
            open(src, "wb").write(data)
            out = os.path.join(tmp, "bad-" + name)
            rc, info, err = ref_convert(ref, src, out, 0, 1)
            gold["errors"][name] = {"rc": rc, "error": err if rc else "", "files": digest(out)}
    with open(os.path.join(HERE, "gguf.json"), "w", encoding="utf-8") as f:
        json.dump(gold, f, indent=1, ensure_ascii=False)
    print("wrote gguf.json")


if __name__ == "__main__":
    main()
