"""GGUF v3 writer and Q8_0/Q4_0 quantizers for synthetic models.

The file layout is the one src/gguf.rs:121-181 reads: magic, version 3, tensor and metadata counts,
typed key/value pairs, tensor infos (ggml dims, dims[0] contiguous; type; offset), then the data at
`general.alignment` (32).  The quantizers are ggml's reference ones, as scripts/convert.py:198-209
documents for Q8_0: d = amax/127 stored as f16, q = round-half-away(x·(1/d)); Q4_0 (absent from the
reference reader) is ggml's block_q4_0: d = max/−8 (max = the value of largest magnitude),
q = min(15, trunc(x·(1/d) + 8.5)), element i < 16 in the low nibble of byte i, 16 + i in the high one.
"""

import struct

import numpy as np

F32, F16, Q4_0, Q8_0 = 0, 1, 2, 8
ALIGN = 32

_U32, _I32, _F32, _BOOL, _STR, _ARR, _U64 = 4, 5, 6, 7, 8, 9, 10


def type_size(wtype, n):
    return {F32: 4 * n, F16: 2 * n, Q8_0: n // 32 * 34, Q4_0: n // 32 * 18}[wtype]


def _round_away(v):
    t = np.trunc(v)
    return t + np.where(np.abs(v - t) >= 0.5, np.sign(v), 0.0).astype(np.float32)


def quantize_q8_0(x):
    """GGUF Q8_0 bytes of float32 values (a multiple of 32)."""
    b = np.ascontiguousarray(x, np.float32).reshape(-1, 32)
    amax = np.abs(b).max(axis=1)
    d = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d != 0, np.float32(1.0) / d, np.float32(0.0)).astype(np.float32)
    q = _round_away(b * inv[:, None]).astype(np.int8)
    out = np.empty((b.shape[0], 34), np.uint8)
    out[:, :2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q.view(np.uint8)
    return out.tobytes()


def quantize_q4_0(x):
    b = np.ascontiguousarray(x, np.float32).reshape(-1, 32)
    idx = np.abs(b).argmax(axis=1)  # the first of equal magnitudes, as ggml's strict `<`
    mx = b[np.arange(b.shape[0]), idx]
    d = (mx / np.float32(-8.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d != 0, np.float32(1.0) / d, np.float32(0.0)).astype(np.float32)
    q = np.trunc(b * inv[:, None] + np.float32(8.5)).astype(np.int32)
    q = np.minimum(q, 15).astype(np.uint8)
    out = np.empty((b.shape[0], 18), np.uint8)
    out[:, :2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q[:, :16] | (q[:, 16:] << 4)
    return out.tobytes()


def encode(x, wtype):
    x = np.ascontiguousarray(x, np.float32)
    if wtype == F32:
        return x.tobytes()
    if wtype == F16:
        return x.astype(np.float16).tobytes()
    if wtype == Q8_0:
        return quantize_q8_0(x)
    if wtype == Q4_0:
        return quantize_q4_0(x)
    raise ValueError(wtype)


def dequantize(raw, wtype, n):
    """float32 values of GGUF bytes (Tensor::to_f32, src/gguf.rs:274-287, + Q4_0)."""
    raw = np.frombuffer(raw, np.uint8)
    if wtype == F32:
        return raw.view(np.float32)[:n].copy()
    if wtype == F16:
        return raw.view(np.float16)[:n].astype(np.float32)
    if wtype == Q8_0:
        b = raw.reshape(-1, 34)
        d = b[:, :2].copy().view(np.float16).astype(np.float32)
        return (b[:, 2:].view(np.int8).astype(np.float32) * d).ravel()[:n]
    if wtype == Q4_0:
        b = raw.reshape(-1, 18)
        d = b[:, :2].copy().view(np.float16).astype(np.float32)
        lo = (b[:, 2:] & 15).astype(np.float32) - 8
        hi = (b[:, 2:] >> 4).astype(np.float32) - 8
        return (np.concatenate([lo, hi], axis=1) * d).ravel()[:n]
    raise ValueError(wtype)


class Writer:
    """Collects metadata and tensors, then writes a GGUF v3 file."""

    def __init__(self):
        self.kv = []
        self.tensors = []

    def u32(self, key, v):
        self.kv.append((key, _U32, struct.pack("<I", int(v))))

    def i32(self, key, v):
        self.kv.append((key, _I32, struct.pack("<i", int(v))))

    def f32(self, key, v):
        self.kv.append((key, _F32, struct.pack("<f", float(v))))

    def bool(self, key, v):
        self.kv.append((key, _BOOL, struct.pack("<B", 1 if v else 0)))

    def str(self, key, v):
        b = v.encode()
        self.kv.append((key, _STR, struct.pack("<Q", len(b)) + b))

    def i32s(self, key, vals):
        self.kv.append((key, _ARR, struct.pack("<IQ", _I32, len(vals)) + struct.pack(f"<{len(vals)}i", *vals)))

    def strs(self, key, vals):
        body = b"".join(struct.pack("<Q", len(s.encode())) + s.encode() for s in vals)
        self.kv.append((key, _ARR, struct.pack("<IQ", _STR, len(vals)) + body))

    def tensor(self, name, dims, wtype, raw):
        """`dims` in ggml order (dims[0] contiguous), `raw` the bytes in type `wtype`."""
        n = int(np.prod(dims))
        assert len(raw) == type_size(wtype, n), (name, dims, wtype, len(raw))
        self.tensors.append((name, list(dims), wtype, raw))

    def write(self, path):
        self.u32("general.alignment", ALIGN)
        head = [b"GGUF", struct.pack("<IQQ", 3, len(self.tensors), len(self.kv))]
        for key, ty, val in self.kv:
            kb = key.encode()
            head.append(struct.pack("<Q", len(kb)) + kb + struct.pack("<I", ty) + val)
        offset = 0
        offsets = []
        for name, dims, wtype, raw in self.tensors:
            nb = name.encode()
            head.append(struct.pack("<Q", len(nb)) + nb + struct.pack("<I", len(dims)) +
                        struct.pack(f"<{len(dims)}Q", *dims) + struct.pack("<IQ", wtype, offset))
            offsets.append(offset)
            offset += (len(raw) + ALIGN - 1) // ALIGN * ALIGN
        header = b"".join(head)
        pad = (-len(header)) % ALIGN
        with open(path, "wb") as f:
            f.write(header + b"\0" * pad)
            for (name, dims, wtype, raw), off in zip(self.tensors, offsets):
                f.write(raw)
                f.write(b"\0" * ((-len(raw)) % ALIGN))
