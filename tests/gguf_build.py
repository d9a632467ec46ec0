"""A GGUF writer for tests: builds files of the public GGUF layout (versions 1-3) with chosen
metadata and tensor tables, so the reader is exercised on known bytes (the role of the reference's
tests/gguf_builder.hpp, written here from the format)."""
from __future__ import annotations

import struct

MAGIC = 0x46554747
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q",
        I64: "<q", F64: "<d"}


class GgufBuilder:
    def __init__(self, version: int = 3):
        self.version = version
        self.meta = []     # (key, tag, value)
        self.tensors = []  # (name, dims, type, offset)

    # -- metadata ---------------------------------------------------------------------------------
    def kv(self, key, tag, value):
        self.meta.append((key, tag, value))
        return self

    def str(self, key, v):
        return self.kv(key, STR, v)

    def u32(self, key, v):
        return self.kv(key, U32, v)

    def u64(self, key, v):
        return self.kv(key, U64, v)

    def i32(self, key, v):
        return self.kv(key, I32, v)

    def f32(self, key, v):
        return self.kv(key, F32, v)

    def f64(self, key, v):
        return self.kv(key, F64, v)

    def boolean(self, key, v):
        return self.kv(key, BOOL, 1 if v else 0)

    def array(self, key, elem_tag, values):
        return self.kv(key, ARR, (elem_tag, list(values)))

    def tensor(self, name, dims, ggml_type, offset):
        self.tensors.append((name, list(dims), ggml_type, offset))
        return self

    # -- encoding ---------------------------------------------------------------------------------
    def _wide(self):
        return self.version >= 2

    def _len(self, n):
        return struct.pack("<Q" if self._wide() else "<I", n)

    def _string(self, s):
        b = s.encode() if isinstance(s, str) else bytes(s)
        return self._len(len(b)) + b

    def _scalar(self, tag, v):
        return self._string(v) if tag == STR else struct.pack(_FMT[tag], v)

    def _value(self, tag, v):
        """A value of `tag`; an array value is (element tag, items), nested arrays included."""
        if tag != ARR:
            return self._scalar(tag, v)
        elem, items = v
        return struct.pack("<I", elem) + self._len(len(items)) + b"".join(self._value(elem, it) for it in items)

    def header_and_tables(self):
        out = bytearray(struct.pack("<II", MAGIC, self.version))
        out += self._len(len(self.tensors)) + self._len(len(self.meta))
        for key, tag, v in self.meta:
            out += self._string(key) + struct.pack("<I", tag) + self._value(tag, v)
        for name, dims, t, off in self.tensors:
            out += self._string(name) + struct.pack("<I", len(dims))
            for d in dims:
                out += struct.pack("<Q" if self._wide() else "<I", d)
            out += struct.pack("<IQ", t, off)
        return bytes(out)

    def build(self, alignment: int = 32, data: bytes | None = None, data_bytes: int = 0) -> bytes:
        """Header and tables, padded to `alignment`, then the data section (`data`, or `data_bytes`
        bytes of a repeating pattern)."""
        head = self.header_and_tables()
        pad = (-len(head)) % alignment if alignment else 0
        if data is None:
            data = bytes((i * 7 + 3) & 0xFF for i in range(data_bytes))
        return head + b"\0" * pad + data
