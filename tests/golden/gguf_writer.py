"""Write small GGUF files (v2 / v3) for the converter checks.  Test infrastructure.

GGUF layout (the format GGML publishes; the reader is libs/gguf_libs/gguf.h:495-541):
  "GGUF", u32 version, tensor count and metadata count (u64 in v3, u32 in v2),
  metadata {string key, u32 type, value}, tensor infos {string name, u32 n_dims,
  u64 dims[n_dims] (dims[0] = row length), u32 type, u64 offset}, zero padding to
  general.alignment (default 32), then the tensor data at those offsets.
Strings are a length (u64 in v3, u32 in v2) and UTF-8 bytes.
"""
import struct

import numpy as np

# metadata value types
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
# tensor types (GGML codes)
T_F32, T_F16, T_Q4_0, T_Q4_1, T_Q5_0, T_Q5_1, T_Q8_0 = 0, 1, 2, 3, 6, 7, 8
T_Q4_K, T_Q5_K, T_Q6_K, T_BF16, T_IQ4_XS = 12, 13, 14, 30, 23
BLOCK = {T_F32: (1, 4), T_F16: (1, 2), T_BF16: (1, 2), T_Q4_0: (32, 18), T_Q4_1: (32, 20), T_Q5_0: (32, 22),
         T_Q5_1: (32, 24), T_Q8_0: (32, 34), T_Q4_K: (256, 144), T_Q5_K: (256, 176), T_Q6_K: (256, 210),
         T_IQ4_XS: (256, 136)}
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q", I64: "<q",
        F64: "<d"}


def tensor_bytes(rng, ttype, shape):
    """random data for a tensor of GGUF shape (dims[0] fastest) with sane scales"""
    n = int(np.prod(shape))
    if ttype == T_F32:
        return (0.02 * rng.standard_normal(n)).astype(np.float32).tobytes()
    if ttype == T_F16:
        return (0.02 * rng.standard_normal(n)).astype(np.float16).tobytes()
    if ttype == T_BF16:
        return ((0.02 * rng.standard_normal(n)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16).tobytes()
    be, bb = BLOCK[ttype]
    nb = n // be
    b = rng.integers(0, 256, (nb, bb), dtype=np.uint8)

    def h(lo, hi):
        return rng.uniform(lo, hi, nb).astype(np.float16).view(np.uint8).reshape(nb, 2)

    if ttype in (T_Q4_0, T_Q5_0, T_Q8_0):
        b[:, 0:2] = h(1e-4, 3e-3)
    elif ttype in (T_Q4_1, T_Q5_1):
        b[:, 0:2] = h(1e-4, 3e-3)
        b[:, 2:4] = h(-0.02, 0.02)
    elif ttype in (T_Q4_K, T_Q5_K):
        b[:, 0:2] = h(1e-5, 5e-5)
        b[:, 2:4] = h(1e-4, 4e-4)
    elif ttype == T_Q6_K:
        b[:, 208:210] = h(4e-6, 1.2e-5)
    return b.tobytes()


class GGUF:
    def __init__(self, version=3, alignment=None):
        self.version = version
        self.kv = []       # (key, type, value, elem_type)
        self.tensors = []  # (name, shape, type, bytes)
        self.alignment = alignment
        if alignment is not None:
            self.add("general.alignment", U32, alignment)

    def add(self, key, vtype, value, elem=None):
        self.kv.append((key, vtype, value, elem))
        return self

    def tensor(self, name, shape, ttype, data):
        self.tensors.append((name, list(shape), ttype, data))
        return self

    def _n(self, v):
        return struct.pack("<Q" if self.version == 3 else "<I", v)

    def _str(self, s):
        b = s.encode("utf-8") if isinstance(s, str) else s
        return self._n(len(b)) + b

    def _val(self, vtype, v, elem):
        if vtype == STR:
            return self._str(v)
        if vtype == ARR:
            out = struct.pack("<I", elem) + self._n(len(v))
            for x in v:
                out += self._val(elem, x, None)
            return out
        return struct.pack(_FMT[vtype], v)

    def bytes(self, truncate=None):
        align = self.alignment or 32
        out = b"GGUF" + struct.pack("<I", self.version) + self._n(len(self.tensors)) + self._n(len(self.kv))
        for key, vt, v, el in self.kv:
            out += self._str(key) + struct.pack("<I", vt) + self._val(vt, v, el)
        off, offs = 0, []
        for name, shape, tt, data in self.tensors:
            offs.append(off)
            off = (off + len(data) + align - 1) // align * align
        for (name, shape, tt, data), o in zip(self.tensors, offs):
            out += self._str(name) + struct.pack("<I", len(shape)) + b"".join(struct.pack("<Q", d) for d in shape)
            out += struct.pack("<I", tt) + struct.pack("<Q", o)
        out += b"\0" * ((-len(out)) % align)
        base = len(out)
        for (name, shape, tt, data), o in zip(self.tensors, offs):
            out += b"\0" * (base + o - len(out)) + data
        return out if truncate is None else out[:truncate]

    def write(self, path, truncate=None):
        with open(path, "wb") as f:
            f.write(self.bytes(truncate))
        return path
