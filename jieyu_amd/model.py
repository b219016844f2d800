"""ctypes mirror of include/jieyu_model.h and include/jieyu_synth.h.

Host-side model descriptors in jieyu's in-memory layouts (WMat, LayerWeights:
libs/date_libs/wmat.h:32-44, libs/date_libs/date.h:75-88) plus the synthetic
configurations the decode-path measurements use.
"""
import ctypes as C

JY_F32 = 0
JY_F16 = 1
JY_Q8_0 = 3
JY_Q4_K = 5
JY_Q5_K = 6
JY_Q6_K = 7


class WMat(C.Structure):
    _fields_ = [("data", C.c_void_p), ("type", C.c_int)]


class LayerWeights(C.Structure):
    _fields_ = [
        ("rms1_weight", C.c_void_p),
        ("Wq", WMat), ("Wk", WMat), ("Wv", WMat), ("Wo", WMat),
        ("bq", C.c_void_p), ("bk", C.c_void_p), ("bv", C.c_void_p),
        ("rms2_weight", C.c_void_p),
        ("W1", WMat), ("W2", WMat), ("W3", WMat),
    ]


class ModelDesc(C.Structure):
    _fields_ = [
        ("num_layers", C.c_int), ("hidden", C.c_int), ("num_heads", C.c_int),
        ("num_kv_heads", C.c_int), ("head_dim", C.c_int), ("intermediate", C.c_int),
        ("vocab_size", C.c_int), ("rope_theta", C.c_float),
        ("embed", WMat), ("lm_head", WMat),
        ("final_rms_weight", C.c_void_p),
        ("layers", C.POINTER(LayerWeights)),
    ]


class SynthConfig(C.Structure):
    _fields_ = [
        ("num_layers", C.c_int), ("hidden", C.c_int), ("num_heads", C.c_int),
        ("num_kv_heads", C.c_int), ("head_dim", C.c_int), ("intermediate", C.c_int),
        ("vocab_size", C.c_int), ("rope_theta", C.c_int), ("wtype", C.c_int),
        ("qkv_bias", C.c_int), ("tied", C.c_int), ("seed", C.c_uint64), ("std", C.c_float),
    ]


class SynthModel(C.Structure):
    _fields_ = [
        ("desc", ModelDesc), ("layers", C.POINTER(LayerWeights)),
        ("arena", C.c_void_p), ("arena_bytes", C.c_size_t), ("weight_bytes", C.c_size_t),
    ]


# The model shapes the decode path is measured on.  Norm weights are 1 + N(0, std),
# biases N(0, std), every 2-D weight N(0, std) (Q8_0-quantized where wtype is Q8_0).
CONFIGS = {
    # 4 layers, d 512, 8/2 heads, hd 64, FFN 1408, V 32000, f32, seed 0, theta 10000
    "tiny-f32": dict(num_layers=4, hidden=512, num_heads=8, num_kv_heads=2, head_dim=64,
                     intermediate=1408, vocab_size=32000, rope_theta=10000, wtype=JY_F32,
                     qkv_bias=0, tied=0, seed=0, std=0.02),
    # Qwen2.5-0.5B shape, Q8_0, tied embeddings, q/k/v biases, theta 1e6
    "qwen2.5-0.5b": dict(num_layers=24, hidden=896, num_heads=14, num_kv_heads=2, head_dim=64,
                         intermediate=4864, vocab_size=151936, rope_theta=1000000, wtype=JY_Q8_0,
                         qkv_bias=1, tied=1, seed=2, std=0.02),
    # Llama-3-8B shape, Q8_0, theta 5e5, seed 3
    "llama3-8b": dict(num_layers=32, hidden=4096, num_heads=32, num_kv_heads=8, head_dim=128,
                      intermediate=14336, vocab_size=128256, rope_theta=500000, wtype=JY_Q8_0,
                      qkv_bias=0, tied=0, seed=3, std=0.02),
    # Qwen2.5-7B shape, Q8_0, q/k/v biases, theta 1e6
    "qwen2.5-7b": dict(num_layers=28, hidden=3584, num_heads=28, num_kv_heads=4, head_dim=128,
                       intermediate=18944, vocab_size=152064, rope_theta=1000000, wtype=JY_Q8_0,
                       qkv_bias=1, tied=0, seed=4, std=0.02),
}


def synth_config(name=None, **over):
    """SynthConfig for a named shape (CONFIGS) with optional field overrides."""
    base = dict(CONFIGS[name]) if name else {}
    base.update(over)
    return SynthConfig(**base)


def bind_synth(lib):
    """Declare the jysyn_* prototypes on a loaded library that exports them."""
    lib.jysyn_create.argtypes = [C.POINTER(SynthConfig), C.POINTER(C.POINTER(SynthModel))]
    lib.jysyn_create.restype = C.c_int
    lib.jysyn_free.argtypes = [C.POINTER(SynthModel)]
    lib.jysyn_free.restype = None
    lib.jysyn_normal_fill.argtypes = [C.c_uint64, C.c_uint64, C.c_float, C.c_void_p, C.c_size_t]
    lib.jysyn_normal_fill.restype = None
    lib.jysyn_uniform_int_fill.argtypes = [C.c_uint64, C.c_uint64, C.c_int, C.c_int, C.c_void_p, C.c_size_t]
    lib.jysyn_uniform_int_fill.restype = None
    lib.jysyn_uniform_fill.argtypes = [C.c_uint64, C.c_uint64, C.c_float, C.c_float, C.c_void_p, C.c_size_t]
    lib.jysyn_uniform_fill.restype = None
    lib.jysyn_quantize_q8_0.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t]
    lib.jysyn_quantize_q8_0.restype = None
    lib.jysyn_f32_to_f16.argtypes = [C.c_float]
    lib.jysyn_f32_to_f16.restype = C.c_uint16
    lib.jysyn_f16_to_f32.argtypes = [C.c_uint16]
    lib.jysyn_f16_to_f32.restype = C.c_float
    return lib


class Synth:
    """Owns one synthetic model built by `lib.jysyn_create`."""

    def __init__(self, lib, cfg):
        self.lib = lib
        self.cfg = cfg
        self.ptr = C.POINTER(SynthModel)()
        if lib.jysyn_create(C.byref(cfg), C.byref(self.ptr)) != 0:
            raise RuntimeError("jysyn_create failed")

    @property
    def desc(self):
        return self.ptr.contents.desc

    @property
    def weight_bytes(self):
        return self.ptr.contents.weight_bytes

    def close(self):
        if self.ptr:
            self.lib.jysyn_free(self.ptr)
            self.ptr = C.POINTER(SynthModel)()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
