"""jyhip_forward_cached_noalloc (the entry point that allocates nothing) against
jyhip_forward_cached, through the C ABI: the same hidden states and KV-cache bytes,
bit for bit, on two calls in a row (the second with fewer rows), over the static
per-GPU workspace that both calls share."""
import ctypes as C

import numpy as np
import pytest

from conftest import ptr

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def bits_equal(a, b):
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    return a.shape == b.shape and np.array_equal(a.view(np.uint8), b.view(np.uint8))


@pytest.fixture(scope="module")
def jy():
    import jieyu_amd
    if jieyu_amd.device_count() < 1:
        pytest.fail("no HIP device visible")
    return jieyu_amd


def small_model(oracle_lib, name, **kw):
    from jieyu_amd.model import Synth, synth_config
    return Synth(oracle_lib, synth_config(name, **kw))


# the tolerance mode as well: its split attention keeps the slices' partials in the
# workspace, here the static array (both runs use the same kernels in the same order)
@pytest.mark.parametrize("fast", [False, True])
@pytest.mark.parametrize("spec", [
    dict(name="llama3-8b", num_layers=2, hidden=512, num_heads=8, num_kv_heads=2, head_dim=64, intermediate=1408,
         vocab_size=3000),
    dict(name="tiny-f32", num_layers=2, vocab_size=4000),
])
def test_noalloc_matches_forward_cached(jy, oracle_lib, spec, fast):
    spec = dict(spec)
    name = spec.pop("name")
    say(f"forward_cached_noalloc vs forward_cached ({name}, {'fast' if fast else 'exact'} mode)")
    s = small_model(oracle_lib, name, **spec)
    d = s.desc
    L, H = d.num_layers, d.hidden
    max_seq = 40
    g = jy.GpuModel(d, max_seq)
    if fast:
        g.mode = jy.MODE_FAST
    kv_a, kv_b = g.kv(max_seq), g.kv(max_seq)
    rng = np.random.default_rng(11)
    start = 0
    for seq in (9, 2, 1):  # each call after the first has fewer rows than the one before
        X = rng.standard_normal((seq, H)).astype(np.float32)
        want = g.forward_cached(kv_a, X, start)
        Xn = X.copy()
        rc = jy.lib().jyhip_forward_cached_noalloc(g.h, kv_b.h, ptr(Xn), seq, start)
        assert rc == 0, jy.last_error()
        assert bits_equal(Xn, want), f"seq={seq} start={start}: max abs diff {np.abs(Xn - want).max()}"
        assert len(kv_b) == start + seq
        start += seq
    for layer in range(L):
        for a, b in zip(kv_a.read(layer, 0, start), kv_b.read(layer, 0, start)):
            assert bits_equal(a, b), f"layer {layer}: KV caches differ"
    kv_a.close()
    kv_b.close()
    g.close()
    s.close()


def device_free_bytes():
    """hipMemGetInfo's free bytes on the current device (the HIP runtime the library uses)."""
    hip = C.CDLL("libamdhip64.so")
    free, total = C.c_size_t(0), C.c_size_t(0)
    assert hip.hipMemGetInfo(C.byref(free), C.byref(total)) == 0
    return free.value


@pytest.mark.parametrize("fast", [False, True])
def test_noalloc_allocates_nothing(jy, oracle_lib, fast):
    """After one warm-up call, repeated calls (prompt rows, then decode rows) leave the
    device's free memory exactly where it was: no allocation and no growth of any pool."""
    say(f"forward_cached_noalloc: device free memory across calls ({'fast' if fast else 'exact'} mode)")
    s = small_model(oracle_lib, "llama3-8b", num_layers=2, hidden=512, num_heads=8, num_kv_heads=2, head_dim=64,
                    intermediate=1408, vocab_size=3000)
    d = s.desc
    max_seq = 64
    g = jy.GpuModel(d, max_seq)
    if fast:
        g.mode = jy.MODE_FAST
    kv = g.kv(max_seq)
    rng = np.random.default_rng(5)
    xs = [rng.standard_normal((n, d.hidden)).astype(np.float32) for n in (12, 3, 1, 1, 1)]

    def run_all():
        start = 0
        for X in xs:
            Xn = X.copy()
            rc = jy.lib().jyhip_forward_cached_noalloc(g.h, kv.h, ptr(Xn), Xn.shape[0], start)
            assert rc == 0, jy.last_error()
            start += Xn.shape[0]

    run_all()  # warm-up: the first launches of each kernel
    before = device_free_bytes()
    for _ in range(3):
        run_all()
    after = device_free_bytes()
    assert after == before, f"device free memory moved by {before - after} bytes across noalloc calls"
    kv.close()
    g.close()
    s.close()


def test_noalloc_rejects_oversize(jy, oracle_lib):
    """A call whose workspace would pass the static array's size is refused with an error
    that names the size; the library stays usable afterwards."""
    say("forward_cached_noalloc oversize request")
    s = small_model(oracle_lib, "llama3-8b", num_layers=1, hidden=512, num_heads=8, num_kv_heads=2, head_dim=64,
                    intermediate=1408, vocab_size=1000)
    d = s.desc
    max_seq = 1024
    g = jy.GpuModel(d, max_seq)
    kv = g.kv(max_seq)
    X = np.zeros((1000, d.hidden), np.float32)
    rc = jy.lib().jyhip_forward_cached_noalloc(g.h, kv.h, ptr(X), X.shape[0], 0)
    assert rc == -1
    assert "static scratch" in jy.last_error()
    x1 = np.random.default_rng(2).standard_normal((1, d.hidden)).astype(np.float32)
    kv2 = g.kv(max_seq)
    want = g.forward_cached(kv2, x1, 0)
    got = g.forward_cached_noalloc(kv, x1, 0)
    assert bits_equal(got, want)
    kv.close()
    kv2.close()
    g.close()
    s.close()
