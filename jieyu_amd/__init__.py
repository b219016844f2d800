"""jieyu_amd — MI355X (gfx950) decode path for jieyu models.

Python host side over libjieyu_amd.so's C ABI (include/jieyu_amd.h).  The
compute path is the HIP library; importing this package without the built
library raises, there is no fallback.
"""
import ctypes as C
import os

import numpy as np

from .model import (CONFIGS, JY_F16, JY_F32, JY_Q4_K, JY_Q5_K, JY_Q6_K, JY_Q8_0, LayerWeights, ModelDesc, Synth,
                    SynthConfig, WMat, bind_synth, synth_config)

HERE = os.path.dirname(os.path.abspath(__file__))
# (JIEYU_AMD_LIB: another build of the library, e.g. the host-sanitized one)
LIB_PATH = os.environ.get("JIEYU_AMD_LIB") or os.path.join(HERE, "libjieyu_amd.so")

P = C.c_void_p
I = C.c_int
F = C.c_float

TOKEN_CB = C.CFUNCTYPE(C.c_int, C.c_int, C.c_void_p)

# arithmetic modes (include/jieyu_amd.h): exact reproduces the reference bit for bit; the
# other bits are the tolerance forms of the decode attention, decode matvecs and prompt GEMMs
MODE_EXACT = 0
MODE_SPLIT_ATTN = 1
MODE_SPLIT_MV = 2
MODE_MFMA_PREFILL = 4
MODE_FAST = MODE_SPLIT_ATTN | MODE_SPLIT_MV | MODE_MFMA_PREFILL
SPLIT_MV_ROWS = 2048  # a model's decode matvecs use the split-dot form below this many rows
MODE_PERSIST = 8  # with the split bits: the decode step as one persistent kernel (opt-in)


class Stats(C.Structure):
    _fields_ = [("prefill_ms", C.c_double), ("decode_ms", C.c_double), ("prompt_len", C.c_int),
                ("decoded", C.c_int), ("upload_ms", C.c_double)]


class JyError(RuntimeError):
    pass


_lib = None


def _proto(lib, name, res, *args):
    fn = getattr(lib, name)
    fn.restype = res
    fn.argtypes = list(args)


def lib():
    """The loaded libjieyu_amd.so (raises if it was not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is missing: run `python -m jieyu_amd.build` first")
    L = C.CDLL(LIB_PATH)
    bind_synth(L)
    _proto(L, "jyhip_last_error", C.c_char_p)
    _proto(L, "jyhip_device_count", I)
    _proto(L, "jyhip_set_device", I, I)
    _proto(L, "jyhip_model_upload", P, C.POINTER(ModelDesc), I)
    _proto(L, "jyhip_model_free", None, P)
    _proto(L, "jyhip_model_weight_bytes", C.c_size_t, P)
    _proto(L, "jyhip_model_upload_ms", C.c_double, P)
    _proto(L, "jyhip_model_set_mode", I, P, I)
    _proto(L, "jyhip_model_mode", I, P)
    _proto(L, "jyhip_kv_create", P, P, I)
    _proto(L, "jyhip_kv_free", None, P)
    _proto(L, "jyhip_kv_len", I, P)
    _proto(L, "jyhip_kv_set_len", I, P, I)
    _proto(L, "jyhip_kv_write", I, P, I, I, I, P, P, P, P)
    _proto(L, "jyhip_kv_read", I, P, I, I, I, P, P, P, P)
    _proto(L, "jyhip_forward_cached", I, P, P, P, I, I, P)
    _proto(L, "jyhip_forward_cached_noalloc", I, P, P, P, I, I)
    _proto(L, "jyhip_generate", I, P, P, P, I, P, I, I, I, F, F, P, TOKEN_CB, P, P, C.POINTER(Stats))
    _proto(L, "jyhip_session_begin", P, P, P, P, I, P, I, I, I, F, F)
    _proto(L, "jyhip_session_graph_info", I, P, I, P)
    _proto(L, "jyhip_session_resume", P, P, P, P, I, P, I, I, I, F, F)
    _proto(L, "jyhip_session_step", I, P, I)
    _proto(L, "jyhip_session_remaining", I, P)
    _proto(L, "jyhip_session_len", I, P)
    _proto(L, "jyhip_session_ids", I, P, P, I)
    _proto(L, "jyhip_session_stats", I, P, C.POINTER(Stats))
    _proto(L, "jyhip_session_end", None, P)
    _proto(L, "jyhip_q8_upload", P, P, I, I, I)
    _proto(L, "jyhip_q8_free", None, P)
    _proto(L, "jyhip_q8_matvec", I, P, P, P)
    _proto(L, "jyhip_q8_set_mode", I, P, I)
    _proto(L, "jyhip_q8_matvec_time", I, P, P, I, I, C.POINTER(C.c_double))
    _proto(L, "jyhip_q8_gemm", I, P, I, P, P)
    _proto(L, "jyhip_q8_gemm_time", I, P, I, P, I, C.POINTER(C.c_double))
    _proto(L, "jyhip_wmat_upload", P, C.POINTER(WMat), I, I, I)
    _proto(L, "jyhip_wmat_free", None, P)
    _proto(L, "jyhip_wmat_matmul", I, P, I, P, P)
    _proto(L, "jyhip_wmat_time", I, P, P, I, C.POINTER(C.c_double))
    _lib = L
    return L


def last_error():
    return lib().jyhip_last_error().decode("utf-8", "replace")


def _check(rc):
    if rc is None or (isinstance(rc, int) and rc < 0):
        raise JyError(last_error())
    return rc


def _ptr(a):
    return None if a is None else a.ctypes.data_as(P)


def device_count():
    return lib().jyhip_device_count()


class KVCache:
    """Device int8 KV cache (__KVcache, libs/date_libs/date.h:89-147)."""

    def __init__(self, model, max_seq):
        self._lib = lib()
        self.model = model
        self.max_seq = max_seq
        self.h = self._lib.jyhip_kv_create(model.h, max_seq)
        if not self.h:
            raise JyError(last_error())

    def __len__(self):
        return self._lib.jyhip_kv_len(self.h)

    def set_len(self, n):
        _check(self._lib.jyhip_kv_set_len(self.h, n))

    def write(self, layer, pos0, k, ks, v, vs):
        """k, v int8 [npos][nkv][hd]; ks, vs float32 [npos][nkv] (jieyu layout)."""
        k = np.ascontiguousarray(k, np.int8)
        v = np.ascontiguousarray(v, np.int8)
        ks = np.ascontiguousarray(ks, np.float32)
        vs = np.ascontiguousarray(vs, np.float32)
        _check(self._lib.jyhip_kv_write(self.h, layer, pos0, k.shape[0], _ptr(k), _ptr(ks), _ptr(v), _ptr(vs)))

    def read(self, layer, pos0, npos):
        m = self.model
        k = np.zeros((npos, m.nkv, m.hd), np.int8)
        v = np.zeros_like(k)
        ks = np.zeros((npos, m.nkv), np.float32)
        vs = np.zeros_like(ks)
        _check(self._lib.jyhip_kv_read(self.h, layer, pos0, npos, _ptr(k), _ptr(ks), _ptr(v), _ptr(vs)))
        return k, ks, v, vs

    def close(self):
        if self.h:
            self._lib.jyhip_kv_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class GpuModel:
    """A model resident in HBM (jyhip_model_upload)."""

    def __init__(self, desc, max_seq):
        self._lib = lib()
        self.desc = desc
        self.max_seq = max_seq
        self.nkv = desc.num_kv_heads
        self.hd = desc.head_dim
        self.hidden = desc.hidden
        self.vocab = desc.vocab_size
        self.num_layers = desc.num_layers
        self.h = self._lib.jyhip_model_upload(C.byref(desc), max_seq)
        if not self.h:
            raise JyError(last_error())

    @property
    def weight_bytes(self):
        return self._lib.jyhip_model_weight_bytes(self.h)

    @property
    def upload_ms(self):
        return self._lib.jyhip_model_upload_ms(self.h)

    @property
    def mode(self):
        """Arithmetic mode bits (MODE_EXACT, or MODE_SPLIT_ATTN | MODE_SPLIT_MV | MODE_MFMA_PREFILL)."""
        return self._lib.jyhip_model_mode(self.h)

    @mode.setter
    def mode(self, bits):
        _check(self._lib.jyhip_model_set_mode(self.h, int(bits)))

    def kv(self, max_seq=None):
        return KVCache(self, max_seq or self.max_seq)

    def forward_cached(self, kv, X, start_pos, layer_out=False):
        """forward_cached: X [seq][hidden] float32 -> final-normed states (new array)."""
        X = np.array(X, np.float32, copy=True, order="C")
        seq = X.shape[0]
        lo = np.zeros((self.num_layers, seq, self.hidden), np.float32) if layer_out else None
        _check(self._lib.jyhip_forward_cached(self.h, kv.h, _ptr(X), seq, start_pos, _ptr(lo)))
        return (X, lo) if layer_out else X

    def forward_cached_noalloc(self, kv, X, start_pos):
        """forward_cached over the GPU's static workspace (jyhip_forward_cached_noalloc)."""
        X = np.array(X, np.float32, copy=True, order="C")
        _check(self._lib.jyhip_forward_cached_noalloc(self.h, kv.h, _ptr(X), X.shape[0], start_pos))
        return X

    def generate(self, prompt, max_new, max_seq=None, temperature=0.0, repetition_penalty=1.0, eos=None,
                 kv=None, callback=None, want_logits=False):
        """generate(): returns (ids up to the returned length, Stats[, last logits])."""
        max_seq = max_seq or self.max_seq
        prompt = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros(max(max_seq, len(prompt)) + 1, np.int32)
        eos_a = None if eos is None else np.ascontiguousarray(eos, np.int32)
        logits = np.zeros(self.vocab, np.float32) if want_logits else None
        st = Stats()
        cb = TOKEN_CB(lambda i, ud: int(bool(callback(i)))) if callback else TOKEN_CB()
        n = self._lib.jyhip_generate(self.h, kv.h if kv is not None else None, _ptr(prompt), len(prompt),
                                     _ptr(eos_a), 0 if eos_a is None else len(eos_a), max_seq, max_new,
                                     temperature, repetition_penalty, _ptr(out), cb, None, _ptr(logits),
                                     C.byref(st))
        _check(n)
        if want_logits:
            return out[:n].copy(), st, logits
        return out[:n].copy(), st

    def session(self, prompt, max_new, max_seq=None, temperature=0.0, repetition_penalty=1.0, eos=None, kv=None,
                resume=False):
        """resume=True: kv already holds the first kv.len positions of `prompt`; only the
        rest runs before decoding (jyhip_session_resume)."""
        return Session(self, prompt, max_new, max_seq or self.max_seq, temperature, repetition_penalty, eos, kv,
                       resume)

    def close(self):
        if self.h:
            self._lib.jyhip_model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Session:
    """A generation driven step by step (jyhip_session_*): the prompt runs on creation."""

    def __init__(self, model, prompt, max_new, max_seq, temperature, repetition_penalty, eos, kv, resume=False):
        self._lib = lib()
        self.model = model
        self.max_seq = max_seq
        prompt = np.ascontiguousarray(prompt, np.int32)
        eos_a = None if eos is None else np.ascontiguousarray(eos, np.int32)
        opener = self._lib.jyhip_session_resume if resume else self._lib.jyhip_session_begin
        self.h = opener(model.h, kv.h if kv is not None else None, _ptr(prompt), len(prompt),
                                               _ptr(eos_a), 0 if eos_a is None else len(eos_a), max_seq, max_new,
                                               temperature, repetition_penalty)
        if not self.h:
            raise JyError(last_error())

    def step(self, n):
        return _check(self._lib.jyhip_session_step(self.h, n))

    @property
    def remaining(self):
        return self._lib.jyhip_session_remaining(self.h)

    def __len__(self):
        return self._lib.jyhip_session_len(self.h)

    def ids(self):
        out = np.zeros(self.max_seq + 1, np.int32)
        n = _check(self._lib.jyhip_session_ids(self.h, _ptr(out), len(out)))
        return out[:n].copy()

    def stats(self):
        st = Stats()
        _check(self._lib.jyhip_session_stats(self.h, C.byref(st)))
        return st

    def graph_info(self, which):
        """(nodes, edges, buffers checked) of captured decode graph `which` (0: past the
        short-context threshold, 1: up to it), None if not captured; raises on a failed check."""
        info = (C.c_longlong * 3)()
        r = _check(self._lib.jyhip_session_graph_info(self.h, which, info))
        return tuple(info) if r == 1 else None

    def close(self):
        if self.h:
            self._lib.jyhip_session_end(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Q8Matrix:
    """Isolated Q8_0 matrix for the decode matvec kernel."""

    def __init__(self, w_q8, rows, cols, copies=1):
        self._lib = lib()
        self.rows, self.cols = rows, cols
        w_q8 = np.ascontiguousarray(w_q8, np.uint8)
        assert w_q8.size == rows * (cols // 32) * 34
        self.h = self._lib.jyhip_q8_upload(_ptr(w_q8), rows, cols, copies)
        if not self.h:
            raise JyError(last_error())

    def matvec(self, x):
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros(self.rows, np.float32)
        _check(self._lib.jyhip_q8_matvec(self.h, _ptr(x), _ptr(y)))
        return y

    def set_mode(self, bits):
        """MODE_EXACT, MODE_SPLIT_MV for matvec(), MODE_MFMA_PREFILL for gemm()."""
        _check(self._lib.jyhip_q8_set_mode(self.h, int(bits)))

    def gemm(self, A):
        """C[m][rows] = A[m][cols] W^T by the prompt GEMM of the matrix's mode."""
        A = np.ascontiguousarray(A, np.float32)
        assert A.ndim == 2 and A.shape[1] == self.cols
        out = np.zeros((A.shape[0], self.rows), np.float32)
        _check(self._lib.jyhip_q8_gemm(self.h, A.shape[0], _ptr(A), _ptr(out)))
        return out

    def gemm_time(self, A, iters):
        """Mean µs per prompt GEMM of A (the activation split included)."""
        A = np.ascontiguousarray(A, np.float32)
        us = C.c_double()
        _check(self._lib.jyhip_q8_gemm_time(self.h, A.shape[0], _ptr(A), iters, C.byref(us)))
        return us.value

    def time(self, x, iters, variant=0):
        """Mean µs per launch over `iters` launches: variant 0 the plain matvec, 1 the decode
        gate/up launch (RMSNorm + SwiGLU); 2 and 3 the same with the split-dot kernel; 4 the
        gate/up launch of the first kernel with the RMSNorm applied after the dot."""
        x = np.ascontiguousarray(x, np.float32)
        us = C.c_double()
        _check(self._lib.jyhip_q8_matvec_time(self.h, _ptr(x), variant, iters, C.byref(us)))
        return us.value

    def close(self):
        if self.h:
            self._lib.jyhip_q8_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class WeightMatrix:
    """One weight matrix of any bound type in HBM (matmul_w's B operand): n outputs,
    k inputs; `data` in the type's host layout (f32 / f16 [k][n], quantized
    [n][k/block] blocks)."""

    def __init__(self, data, wtype, n, k, copies=1):
        self._lib = lib()
        self.n, self.k, self.wtype = n, k, wtype
        self._data = np.ascontiguousarray(data)
        w = WMat(_ptr(self._data), wtype)
        self.h = self._lib.jyhip_wmat_upload(C.byref(w), n, k, copies)
        if not self.h:
            raise JyError(last_error())

    def matmul(self, A):
        """C[m][n] for A[m][k] (m == 1: the decode kernel, m > 1: the prompt GEMM)"""
        A = np.ascontiguousarray(A, np.float32).reshape(-1, self.k)
        out = np.zeros((A.shape[0], self.n), np.float32)
        _check(self._lib.jyhip_wmat_matmul(self.h, A.shape[0], _ptr(A), _ptr(out)))
        return out

    def time(self, x, iters):
        x = np.ascontiguousarray(x, np.float32)
        us = C.c_double()
        _check(self._lib.jyhip_wmat_time(self.h, _ptr(x), iters, C.byref(us)))
        return us.value

    def close(self):
        if self.h:
            self._lib.jyhip_wmat_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


__all__ = ["lib", "last_error", "device_count", "GpuModel", "KVCache", "Q8Matrix", "WeightMatrix", "Stats", "JyError",
           "ModelDesc", "LayerWeights", "SynthConfig", "Synth", "synth_config", "CONFIGS", "JY_F32", "JY_F16",
           "JY_Q8_0", "JY_Q4_K", "JY_Q5_K", "JY_Q6_K"]
