"""CPU oracles for jieyu's decode path.  TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package, and only as the oracle / the timed CPU baseline.  The product
(jieyu_amd, libjieyu_amd.so) never imports or links it.

  Oracle  -- oracle/_build/libjyoracle.so, the C restatement (jy_oracle.c)
  Ref     -- oracle/_ref/libjyref.so, jieyu's own headers compiled by
             oracle/Makefile from the reference sources (present only where
             it was built)
"""
import ctypes as C
import os

from jieyu_amd.model import ModelDesc, bind_synth

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "_build", "libjyoracle.so")
REF_SO = os.path.join(HERE, "_ref", "libjyref.so")

P = C.c_void_p
I = C.c_int
F = C.c_float


def _proto(lib, name, res, *args):
    fn = getattr(lib, name)
    fn.restype = res
    fn.argtypes = list(args)


class JyoKV(C.Structure):
    _fields_ = [("num_layers", I), ("max_seq", I), ("num_kv_heads", I), ("head_dim", I),
                ("current_len", I), ("k", P), ("v", P), ("ks", P), ("vs", P)]


def load_oracle():
    if not os.path.exists(ORACLE_SO):
        raise FileNotFoundError(f"{ORACLE_SO} not built (make -C oracle)")
    lib = bind_synth(C.CDLL(ORACLE_SO))
    _proto(lib, "jyo_f16_to_f32", F, C.c_uint16)
    _proto(lib, "jyo_q8_row_dot", F, P, P, I)
    _proto(lib, "jyo_q_row_dot", F, P, P, I, I)
    _proto(lib, "jyo_block_elems", I, I)
    _proto(lib, "jyo_block_bytes", I, I)
    _proto(lib, "jyo_dequant_block", None, I, P, P)
    _proto(lib, "jyo_matmul_q", None, P, P, P, I, I, I, I)
    _proto(lib, "jyo_matmul_f16", None, I, I, I, P, P, P)
    _proto(lib, "jyo_matmul_w", None, P, I, I, I, P, P)
    _proto(lib, "jyo_embed_row", None, P, I, I, P)
    _proto(lib, "jyo_matmul_q8", None, P, P, P, I, I, I)
    _proto(lib, "jyo_matmul_f32", None, I, I, I, P, P, P)
    _proto(lib, "jyo_rmsnorm", None, P, P, P, I, F)
    _proto(lib, "jyo_rope_table", None, I, I, F, P, P)
    _proto(lib, "jyo_rope", None, P, I, I, I, I, P, P)
    _proto(lib, "jyo_kv_pack", None, P, P, P, I, I, I)
    _proto(lib, "jyo_silu", None, P, P, I)
    _proto(lib, "jyo_kv_init", I, C.POINTER(JyoKV), I, I, I, I)
    _proto(lib, "jyo_kv_free", None, C.POINTER(JyoKV))
    _proto(lib, "jyo_attention", I, P, P, P, P, I, I, I, I, I, P, P, P, P, I)
    _proto(lib, "jyo_forward_cached", I, C.POINTER(ModelDesc), P, P, P, I, I, C.POINTER(JyoKV), P)
    _proto(lib, "jyo_generate", I, C.POINTER(ModelDesc), P, I, P, I, P, P, I, I, F, F, P,
           C.POINTER(JyoKV), P)
    return lib


def ref_available():
    return os.path.exists(REF_SO)


def load_ref():
    if not os.path.exists(REF_SO):
        raise FileNotFoundError(f"{REF_SO} not built (make -C oracle ref)")
    lib = C.CDLL(REF_SO)
    _proto(lib, "jyref_init", I)
    _proto(lib, "jyref_version", C.c_char_p)
    _proto(lib, "jyref_matmul_q8", None, P, P, P, I, I, I)
    _proto(lib, "jyref_matmul_f32", None, I, I, I, P, P, P)
    _proto(lib, "jyref_matmul_w", None, P, I, I, I, P, P)
    _proto(lib, "jyref_wmat_row", None, P, I, I, P)
    _proto(lib, "jyref_rmsnorm", None, P, P, P, I, F)
    _proto(lib, "jyref_rope_table", None, I, I, F, P, P)
    _proto(lib, "jyref_rope", None, P, I, I, I, I, P, P)
    _proto(lib, "jyref_kv_pack", None, P, P, P, I, I, I)
    _proto(lib, "jyref_attention", I, P, P, P, P, I, I, I, I, I, P, P, P, P, I)
    _proto(lib, "jyref_silu", None, P, P, I)
    _proto(lib, "jyref_kv_create", P, I, I, I, I)
    _proto(lib, "jyref_kv_free", None, P)
    for n in ("jyref_kv_k", "jyref_kv_v", "jyref_kv_ks", "jyref_kv_vs"):
        _proto(lib, n, P, P)
    _proto(lib, "jyref_kv_len", I, P)
    _proto(lib, "jyref_kv_set_len", None, P, I)
    _proto(lib, "jyref_forward_cached", I, C.POINTER(ModelDesc), P, P, P, I, I, P, P)
    _proto(lib, "jyref_generate", I, C.POINTER(ModelDesc), P, I, P, I, P, P, I, I, F, F, P, P, P, I)
    lib.jyref_init()
    return lib
