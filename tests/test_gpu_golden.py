"""HIP decode path against the golden token streams the compiled reference wrote
(tests/golden/generate.json) and against the reference's own known-answer models.

Runs the same synthetic models (include/jieyu_synth.h builds them byte for byte
on any host) through libjieyu_amd.so and requires the reference's ids exactly.
"""
import json
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)


@pytest.fixture(scope="module")
def jy():
    import jieyu_amd
    if jieyu_amd.device_count() < 1:
        pytest.fail("no HIP device visible")
    return jieyu_amd


@pytest.fixture(scope="module")
def gold():
    with open(os.path.join(HERE, "golden", "generate.json")) as f:
        return json.load(f)["cases"]


GEN_NAMES = ["tiny-f32", "qwen-like-small", "llama-like-small", "llama-like-small-T0.0-rp1.3",
             "llama-like-small-T0.8-rp1.0", "llama-like-small-T0.7-rp1.1", "qwen2.5-0.5b-full"]


@pytest.mark.parametrize("name", GEN_NAMES)
def test_generate_matches_reference_golden(jy, oracle_lib, gold, name):
    from jieyu_amd.model import Synth, synth_config
    case = gold[name]
    say(f"golden generate {name}: prompt {len(case['prompt'])} max_new {case['max_new']} max_seq {case['max_seq']}")
    syn = Synth(oracle_lib, synth_config(case["config"], **case["overrides"]))
    try:
        g = jy.GpuModel(syn.desc, case["max_seq"])
        try:
            ids, _ = g.generate(np.array(case["prompt"], np.int32), case["max_new"],
                                temperature=case.get("temperature", 0.0),
                                repetition_penalty=case.get("repetition_penalty", 1.0))
        finally:
            g.close()
    finally:
        syn.close()
    assert ids.tolist() == case["ids"]


def test_bind_test_kat(jy, gold):
    """check_bind_weights (libs/text/text.h:817-843): the pseudo-weight model, prompts {1,2,3}
    and {5,6,7}, 3 greedy tokens at max_seq 8."""
    from golden.kat_models import bind_model_desc, bind_test_model
    desc, keep = bind_model_desc(bind_test_model())
    g = jy.GpuModel(desc, 8)
    try:
        for prompt in ([1, 2, 3], [5, 6, 7]):
            say(f"bind_test KAT {prompt}")
            ids, _ = g.generate(np.array(prompt, np.int32), 3)
            assert ids.tolist() == gold["bind_test_kat"][str(prompt)]
    finally:
        g.close()
    del keep


def test_demo_model_kat(jy, gold):
    """make_demo_model (libs/model_libs/converter.h:412-503): "abcdefgh" -> "ijklmnopqrstuvwx"."""
    from golden.kat_models import demo_model_desc
    say("demo model KAT")
    desc, keep = demo_model_desc()
    g = jy.GpuModel(desc, 64)
    try:
        prompt = [256] + list(b"abcdefgh")
        ids, _ = g.generate(np.array(prompt, np.int32), 16)
    finally:
        g.close()
    del keep
    assert bytes(ids[len(prompt):].tolist()) == b"ijklmnopqrstuvwx"
    assert ids.tolist() == gold["demo_abcdefgh"]["ids"]
