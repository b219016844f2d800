"""jieyu's text C ABI on the GPU: jieyu_load / jieyu_generate / jieyu_generate_jsonl
against the records jieyu's own C ABI produced for the same model directories
(tests/golden/text.json), call for call: return value, output bytes, error text.

Covers the reference's pipeline KATs (libs/text/text.h:993-1051: "abcdefgh" ->
"ijklmnopqrstuvwx", max_new=5 -> "defgh", repeatability, BOS, over-long prompt),
greedy and sampled decoding with the repetition penalty, stop markers and
special ids, jsonl prompts, f32 and Q8_0 (tied) models, truncated and NULL
output buffers, and handle sharing.
"""
import json
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")
sys.path.insert(0, GOLDEN)

import text_models as TM  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gold():
    with open(os.path.join(GOLDEN, "text.json"), encoding="utf-8") as f:
        return json.load(f)


@pytest.fixture(scope="module")
def env(tmp_path_factory):
    import jieyu_amd
    from jieyu_amd import api
    if jieyu_amd.device_count() < 1:
        pytest.fail("no HIP device visible")
    return str(tmp_path_factory.mktemp("textdirs")), api.abi(), jieyu_amd.lib()


@pytest.mark.parametrize("kind", [s[0] for s in TM.SCRIPTS])
def test_script_matches_reference(env, gold, kind):
    root, L, qlib = env
    _, max_seq, calls = next(s for s in TM.SCRIPTS if s[0] == kind)
    print(f"[text] script {kind} max_seq={max_seq} calls={len(calls)}", flush=True)
    got = TM.run_script(L, root, kind, max_seq, calls, qlib)
    want = gold["scripts"][kind]
    assert "load_error" not in got, got.get("load_error")
    for i, (c, g, w) in enumerate(zip(calls, got["calls"], want["calls"])):
        assert g == w, f"call {i} {c[:2]}: got {g} want {w}"


def test_pipeline_kats(env):
    """check_pipeline 6-10 (libs/text/text.h:993-1051) through the Python wrapper"""
    root, L, qlib = env
    from jieyu_amd.api import Jieyu, Options
    with Jieyu(TM.build_dir("demo", root, qlib), 64) as m:
        assert m.generate("abcdefgh", Options(16, 0.0, 1.0)) == "ijklmnopqrstuvwx"
        assert m.generate("abc", Options(5, 0.0, 1.0)) == "defgh"
        a = m.generate("xyz", Options(8, 0.0, 1.0))
        assert a and a == m.generate("xyz", Options(8, 0.0, 1.0))
        assert m.generate("k" * 200, Options(16, 0.0, 1.0)) == ""
        assert m.context_length() == 64 and Jieyu.version() == "1.0.0"


def test_handles_share_one_model(env):
    """a second load of the same directory shares the model; the last free releases
    it (main.hpp:85-130)"""
    root, L, qlib = env
    d = TM.build_dir("demo", root, qlib).encode()
    h1 = L.jieyu_load(d, 64)
    h2 = L.jieyu_load(d, 32)
    assert h1 and h2 and L.jieyu_context_length(h2) == 32
    L.jieyu_free(h1)
    import ctypes as C
    buf = C.create_string_buffer(64)
    assert L.jieyu_generate(h2, b"abc", buf, 64, 5, 0.0, 1.0) == 5 and buf.value == b"defgh"
    L.jieyu_free(h2)
    # released: a new load of the directory uploads it again
    h3 = L.jieyu_load(d, 64)
    assert h3 and L.jieyu_generate(h3, b"abcdefgh", buf, 64, 16, 0.0, 1.0) == 16
    assert buf.value == b"ijklmnopqrstuvwx"
    L.jieyu_free(h3)
