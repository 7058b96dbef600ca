"""A small GGUF v3 reader for the tests (metadata and tensor table; tensor bytes as numpy views). Test helper only:
the product's reader is the C++ one in malkin_amd/csrc/host."""
import struct

import numpy as np

_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<B", 10: "<Q", 11: "<q", 12: "<d"}
_BLOCK = {0: (1, 4), 1: (1, 2), 30: (1, 2), 8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210)}


class Gguf:
    def __init__(self, path):
        with open(path, "rb") as f:
            self.buf = f.read()
        self.pos = 0
        if self._get("<I") != 0x46554747:
            raise ValueError("not a GGUF file")
        self.version = self._get("<I")
        n_tensors, n_kv = self._get("<Q"), self._get("<Q")
        self.kv = {}
        for _ in range(n_kv):
            key = self._str()
            self.kv[key] = self._value(self._get("<I"))
        self.tensors = {}
        for _ in range(n_tensors):
            name = self._str()
            nd = self._get("<I")
            ne = [self._get("<Q") for _ in range(nd)]
            ty = self._get("<I")
            self.tensors[name] = (ne, ty, self._get("<Q"))
        align = self.kv.get("general.alignment", 32)
        self.data_start = (self.pos + align - 1) // align * align

    def _get(self, fmt):
        v = struct.unpack_from(fmt, self.buf, self.pos)[0]
        self.pos += struct.calcsize(fmt)
        return v

    def _str(self):
        n = self._get("<Q")
        s = self.buf[self.pos:self.pos + n].decode()
        self.pos += n
        return s

    def _value(self, t):
        if t == 8:
            return self._str()
        if t == 9:
            et, n = self._get("<I"), self._get("<Q")
            return [self._value(et) for _ in range(n)]
        return self._get(_SCALAR[t])

    def rows(self, name):
        """(type, columns, [rows][row bytes] uint8 view) of a tensor."""
        ne, ty, off = self.tensors[name]
        qk, bs = _BLOCK[ty]
        rb = ne[0] // qk * bs
        n_rows = 1
        for d in ne[1:]:
            n_rows *= d
        a = np.frombuffer(self.buf, np.uint8, rb * n_rows, self.data_start + off)
        return ty, ne[0], a.reshape(n_rows, rb)
