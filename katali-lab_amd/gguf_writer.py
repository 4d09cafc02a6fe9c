"""A small GGUF writer (synthetic model files for the tests and the expert-tier
benchmark): the public container format (little-endian
header "GGUF", version, tensor and metadata counts; key/value metadata;
tensor infos; the data section at the file's alignment), plus hooks to write
malformed files on purpose."""
import struct

import numpy as np

# metadata value types (public GGUF format)
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q",
        I64: "<q", F64: "<d"}


def gstr(s) -> bytes:
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


class GgufWriter:
    def __init__(self, version=3, alignment=32):
        self.version, self.alignment = version, alignment
        self.kvs = []          # raw encoded key/value entries
        self.tensors = []      # (name, dims, type, data bytes, offset or None)
        self.n_kv = self.n_tensors = None   # header overrides

    # -- metadata ---------------------------------------------------------
    def kv(self, key, t, v):
        self.kvs.append(gstr(key) + struct.pack("<I", t) + (gstr(v) if t == STR else struct.pack(_FMT[t], v)))
        return self

    def kv_array(self, key, et, values):
        body = b"".join(gstr(v) if et == STR else struct.pack(_FMT[et], v) for v in values)
        self.kvs.append(gstr(key) + struct.pack("<IIQ", ARR, et, len(values)) + body)
        return self

    def kv_raw(self, raw: bytes):
        self.kvs.append(raw)
        return self

    # -- tensors ------------------------------------------------------------
    def tensor(self, name, dims, t, data, offset=None):
        """dims in GGUF order (dims[0] contiguous); data bytes (numpy ok)."""
        self.tensors.append((name, list(dims), t, bytes(np.ascontiguousarray(data).view(np.uint8)), offset))
        return self

    def build(self, truncate=0) -> bytes:
        nt = len(self.tensors) if self.n_tensors is None else self.n_tensors
        nk = len(self.kvs) if self.n_kv is None else self.n_kv
        out = bytearray(struct.pack("<IIQQ", 0x46554747, self.version, nt, nk))
        for e in self.kvs:
            out += e
        # data offsets: each tensor at the next aligned position unless given
        offs, pos = [], 0
        for _, _, _, data, off in self.tensors:
            if off is None:
                pos = (pos + self.alignment - 1) // self.alignment * self.alignment
                off = pos
                pos += len(data)
            offs.append(off)
        for (name, dims, t, _, _), off in zip(self.tensors, offs):
            out += gstr(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
            out += struct.pack("<IQ", t, off)
        pad = (-len(out)) % self.alignment
        out += b"\0" * pad
        # the data section (a tensor placed past 1 GiB on purpose gets no bytes)
        spans = [(off, data) for (_, _, _, data, _), off in zip(self.tensors, offs) if off + len(data) < 1 << 30]
        sec = bytearray(max((off + len(d) for off, d in spans), default=0))
        for off, d in spans:
            sec[off:off + len(d)] = d
        out += sec
        return bytes(out[:len(out) - truncate] if truncate else out)

    def write(self, path, truncate=0):
        with open(path, "wb") as f:
            f.write(self.build(truncate))
        return path
