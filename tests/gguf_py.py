"""A small, independent GGUF (v2/v3) reader in pure Python for the tests: it cross-checks the
product's C++ reader and writer and feeds the float64 reference model. Layout as documented for
the GGUF format (the reference reads it through gguf_init_from_file, model.cpp:667-784):

    magic "GGUF", u32 version, u64 n_tensors, u64 n_kv,
    n_kv x { string key, u32 type, value },
    n_tensors x { string name, u32 n_dims, u64 ne[n_dims], u32 ggml_type, u64 offset },
    padding to general.alignment (default 32), tensor data (offsets relative to that point).
Strings are u64 length + bytes; arrays are u32 element type + u64 count + elements.
"""
import struct

import numpy as np

_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}
STRING, ARRAY = 8, 9

# ggml type id -> (block elements, block bytes)
BLOCK = {0: (1, 4), 1: (1, 2), 2: (32, 18), 8: (32, 34), 12: (256, 144), 30: (1, 2)}


class GGUFFile:
    def __init__(self, path):
        self.path = path
        with open(path, "rb") as f:
            self.buf = f.read()
        self.pos = 0
        if self.buf[:4] != b"GGUF":
            raise ValueError("not a GGUF file")
        self.pos = 4
        self.version = self._u("<I")
        n_tensors, n_kv = self._u("<Q"), self._u("<Q")
        self.kv = {}
        self.kv_types = {}
        for _ in range(n_kv):
            key = self._str()
            t = self._u("<I")
            self.kv_types[key] = t
            self.kv[key] = self._value(t)
        self.tensors = {}
        for _ in range(n_tensors):
            name = self._str()
            nd = self._u("<I")
            ne = [self._u("<Q") for _ in range(nd)]
            ttype = self._u("<I")
            off = self._u("<Q")
            self.tensors[name] = (ttype, ne, off)
        align = int(self.kv.get("general.alignment", 32))
        self.data_offset = (self.pos + align - 1) // align * align

    def _u(self, fmt):
        v = struct.unpack_from(fmt, self.buf, self.pos)[0]
        self.pos += struct.calcsize(fmt)
        return v

    def _str(self):
        n = self._u("<Q")
        s = self.buf[self.pos:self.pos + n].decode("utf-8")
        self.pos += n
        return s

    def _value(self, t):
        if t in _SCALAR:
            return self._u(_SCALAR[t])
        if t == STRING:
            return self._str()
        if t == ARRAY:
            et = self._u("<I")
            n = self._u("<Q")
            return [self._value(et) for _ in range(n)]
        raise ValueError(f"unknown GGUF value type {t}")

    def raw(self, name):
        ttype, ne, off = self.tensors[name]
        qk, bs = BLOCK[ttype]
        n = int(np.prod(ne))
        nbytes = n // qk * bs
        start = self.data_offset + off
        return np.frombuffer(self.buf, dtype=np.uint8, count=nbytes, offset=start), ttype, ne
