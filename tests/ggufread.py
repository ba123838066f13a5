"""A small GGUF v3 reader for the tests: metadata values and tensors by name, dequantized to float32
(Tensor::read / to_f32, src/gguf.rs:121-287).  Independent of the product's C++ reader and the
oracle's C reader, so the composition checks read the weights a third way."""

import struct

import numpy as np

from wavo_amd import gguf

_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<B", 10: "<Q", 11: "<q", 12: "<d"}


class Gguf:
    def __init__(self, path):
        self.buf = open(path, "rb").read()
        b = self.buf
        assert b[:4] == b"GGUF"
        version, n_t, n_kv = struct.unpack_from("<IQQ", b, 4)
        assert version == 3
        self.at = 24
        self.kv = {}
        for _ in range(n_kv):
            key = self._str()
            ty = self._u32()
            self.kv[key] = self._value(ty)
        infos = []
        for _ in range(n_t):
            name = self._str()
            nd = self._u32()
            dims = list(struct.unpack_from(f"<{nd}Q", b, self.at))
            self.at += 8 * nd
            ty, off = struct.unpack_from("<IQ", b, self.at)
            self.at += 12
            infos.append((name, dims, ty, off))
        align = self.kv.get("general.alignment", 32)
        data = (self.at + align - 1) // align * align
        self.tensors = {n: (dims, ty, data + off) for n, dims, ty, off in infos}

    def _u32(self):
        v = struct.unpack_from("<I", self.buf, self.at)[0]
        self.at += 4
        return v

    def _str(self):
        n = struct.unpack_from("<Q", self.buf, self.at)[0]
        s = self.buf[self.at + 8:self.at + 8 + n].decode()
        self.at += 8 + n
        return s

    def _value(self, ty):
        if ty == 8:
            return self._str()
        if ty == 9:
            it = self._u32()
            n = struct.unpack_from("<Q", self.buf, self.at)[0]
            self.at += 8
            return [self._value(it) for _ in range(n)]
        fmt = _SCALAR[ty]
        v = struct.unpack_from(fmt, self.buf, self.at)[0]
        self.at += struct.calcsize(fmt)
        return v

    def has(self, name):
        return name in self.tensors

    def tensor(self, name):
        """float32 values of a tensor, shaped [dims[-1]]…[dims[0]] (row-major, dims[0] contiguous)."""
        dims, ty, off = self.tensors[name]
        n = int(np.prod(dims))
        raw = self.buf[off:off + gguf.type_size(ty, n)]
        return gguf.dequantize(raw, ty, n).reshape(list(reversed(dims)))

    def matrix(self, name):
        """A linear weight as [rows][k] (ggml dims [k…, rows])."""
        dims, _, _ = self.tensors[name]
        return self.tensor(name).reshape(dims[-1], -1)
