"""GGUF model files for the engine: the reference's ``GgufFile``
(``gguf/include/qorvix/gguf/gguf_file.hpp:47-105``) over ``qvx_gguf_*`` in ``libqvx.so``.

``GgufFile.open(path)`` memory-maps and parses a GGUF file (versions 1-3) with the reference's
checks; malformed data raises ``GgufParseError`` as the reference throws it.  Tensors are located,
not read: ``tensor_bytes`` is a view into the mapping, and ``upload`` copies a tensor's raw blocks to
the device as a ``decode.DevWeight`` that ``qvx_qmatmul`` / ``qvx_qgemm_f16`` take as they are (the
reference's CUDA backend uploads the same bytes, ``cuda/src/cuda_backend.cu:1300-1309``).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

from . import E_FORMAT, E_IO, OK, QvxError, lib

# ggml type names by on-disk id (gguf/include/qorvix/gguf/gguf_types.hpp:17-45; public format).
GGML_TYPE_NAMES = {
    0: "F32", 1: "F16", 2: "Q4_0", 3: "Q4_1", 6: "Q5_0", 7: "Q5_1", 8: "Q8_0", 9: "Q8_1", 10: "Q2_K",
    11: "Q3_K", 12: "Q4_K", 13: "Q5_K", 14: "Q6_K", 15: "Q8_K", 16: "IQ2_XXS", 17: "IQ2_XS", 18: "IQ3_XXS",
    19: "IQ1_S", 20: "IQ4_NL", 21: "IQ3_S", 22: "IQ2_S", 23: "IQ4_XS", 24: "I8", 25: "I16", 26: "I32",
    27: "I64", 28: "F64", 29: "IQ1_M", 30: "BF16",
}
# metadata value type tags (0..12)
M_U8, M_I8, M_U16, M_I16, M_U32, M_I32, M_F32, M_BOOL, M_STR, M_ARR, M_U64, M_I64, M_F64 = range(13)
_SIGNED = (M_I8, M_I16, M_I32, M_I64)


def ggml_type_name(t: int) -> str:
    """ggmlTypeName (gguf/src/gguf_types.cpp): "UNKNOWN(n)" for ids the format does not define."""
    return GGML_TYPE_NAMES.get(t, f"UNKNOWN({t})")


class GgufParseError(ValueError):
    """Malformed GGUF data (the reference's GgufParseError, gguf/include/qorvix/gguf/gguf_error.hpp)."""


@dataclass(frozen=True)
class GgufTensor:
    """One tensor-table entry (gguf_file.hpp:27-35): ggml dimension order (dimensions[0] is the row
    length), offset relative to the data section, on-disk size from the block traits."""
    name: str
    dimensions: tuple
    type_raw: int
    offset: int
    n_elements: int
    n_bytes: int
    index: int

    def type_name(self) -> str:
        return ggml_type_name(self.type_raw)

    @property
    def cols(self) -> int:
        """Row length (elements per row): dimensions[0]."""
        return int(self.dimensions[0]) if self.dimensions else 1

    @property
    def rows(self) -> int:
        """Row count: the product of the other dimensions."""
        n = 1
        for d in self.dimensions[1:]:
            n *= int(d)
        return n


def _check(rc: int, what: str) -> None:
    if rc == OK:
        return
    if rc in (E_FORMAT, E_IO):
        raise GgufParseError(lib().qvx_gguf_last_error().decode(errors="replace"))
    raise QvxError(rc, what)


class GgufFile:
    """Parsed GGUF header, metadata and tensor table (the reference's GgufFile)."""

    def __init__(self, handle, keepalive=None):
        self._h = handle
        self._keep = keepalive  # the caller's buffer of parse(), held while the handle lives
        so = lib()
        n = so.qvx_gguf_tensor_count(handle)
        self._tensors = []
        for i in range(n):
            name, typ, nd = C.c_char_p(), C.c_uint32(), C.c_uint32()
            dims = (C.c_uint64 * 8)()
            off, ne, nb = C.c_uint64(), C.c_uint64(), C.c_uint64()
            _check(so.qvx_gguf_tensor_info(handle, i, C.byref(name), C.byref(typ), C.byref(nd), dims, C.byref(off),
                                           C.byref(ne), C.byref(nb)), "qvx_gguf_tensor_info")
            self._tensors.append(GgufTensor(name.value.decode(), tuple(int(dims[d]) for d in range(nd.value)),
                                            typ.value, off.value, ne.value, nb.value, i))
        self._by_name = {t.name: t for t in self._tensors}  # later duplicates win, as in the reference
        self._meta = []
        for i in range(so.qvx_gguf_meta_count(handle)):
            key = so.qvx_gguf_meta_key(handle, i).decode()
            self._meta.append((key, self._value(key)))
        self._meta_index = {k: v for k, v in self._meta}

    # ---- construction -------------------------------------------------------------------------
    @staticmethod
    def parse(data: bytes) -> "GgufFile":
        """Parses an in-memory buffer (GgufFile::parse, gguf_file.hpp:51-52)."""
        buf = C.create_string_buffer(bytes(data), len(data)) if len(data) else None
        h = C.c_void_p()
        _check(lib().qvx_gguf_parse(buf, len(data), C.byref(h)), "qvx_gguf_parse")
        return GgufFile(h, buf)

    @staticmethod
    def open(path) -> "GgufFile":
        """Memory-maps `path` and parses it (GgufFile::open, gguf_file.hpp:54-55)."""
        h = C.c_void_p()
        _check(lib().qvx_gguf_open(str(path).encode(), C.byref(h)), "qvx_gguf_open")
        return GgufFile(h)

    def close(self) -> None:
        if self._h:
            lib().qvx_gguf_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- header and tables ----------------------------------------------------------------------
    @property
    def version(self) -> int:
        return lib().qvx_gguf_version(self._h)

    @property
    def alignment(self) -> int:
        return lib().qvx_gguf_alignment(self._h)

    @property
    def data_offset(self) -> int:
        """Absolute offset of the tensor-data section (dataOffset(), gguf_file.hpp:62)."""
        return lib().qvx_gguf_data_offset(self._h)

    @property
    def tensors(self):
        return list(self._tensors)

    def tensor(self, name: str):
        return self._by_name.get(name)

    @property
    def metadata(self):
        """(key, value) pairs in file order; arrays as lists."""
        return list(self._meta)

    def find(self, key: str):
        return self._meta_index.get(key)

    def _value(self, key: str):
        so, k = lib(), key.encode()
        tag, elem, cnt = C.c_uint32(), C.c_uint32(), C.c_uint64()
        _check(so.qvx_gguf_meta_type(self._h, k, C.byref(tag), C.byref(elem), C.byref(cnt)), "qvx_gguf_meta_type")
        items = [self._element(k, elem.value, i) for i in range(cnt.value)]
        return items if tag.value == M_ARR else items[0]

    def _element(self, k: bytes, tag: int, i: int):
        so = lib()
        if tag == M_ARR:  # an element of an array of arrays: the format allows them, the engine reads none
            return None
        if tag == M_STR:
            p, n = C.c_void_p(), C.c_size_t()
            _check(so.qvx_gguf_meta_string(self._h, k, i, C.byref(p), C.byref(n)), "qvx_gguf_meta_string")
            return C.string_at(p.value, n.value).decode(errors="replace") if n.value else ""
        if tag == M_BOOL:
            b = C.c_int()
            _check(so.qvx_gguf_meta_bool(self._h, k, i, C.byref(b)), "qvx_gguf_meta_bool")
            return bool(b.value)
        if tag in (M_F32, M_F64):
            f = C.c_double()
            _check(so.qvx_gguf_meta_f64(self._h, k, i, C.byref(f)), "qvx_gguf_meta_f64")
            return f.value
        if tag in _SIGNED:
            v = C.c_int64()
            _check(so.qvx_gguf_meta_i64(self._h, k, i, C.byref(v)), "qvx_gguf_meta_i64")
            return v.value
        u = C.c_uint64()
        _check(so.qvx_gguf_meta_u64(self._h, k, i, C.byref(u)), "qvx_gguf_meta_u64")
        return u.value

    # typed helpers (gguf_file.hpp:74-78): None when absent or of the wrong category
    def get_string(self, key: str):
        v = self.find(key)
        return v if isinstance(v, str) else None

    def get_u64(self, key: str):
        u = C.c_uint64()
        return u.value if self._h and lib().qvx_gguf_meta_u64(self._h, key.encode(), 0, C.byref(u)) == OK \
            and not isinstance(self.find(key), list) else None

    def get_f64(self, key: str):
        f = C.c_double()
        return f.value if self._h and lib().qvx_gguf_meta_f64(self._h, key.encode(), 0, C.byref(f)) == OK \
            and not isinstance(self.find(key), list) else None

    def get_bool(self, key: str):
        v = self.find(key)
        return v if isinstance(v, bool) else None

    @property
    def architecture(self) -> str:
        return self.get_string("general.architecture") or ""

    def name(self):
        return self.get_string("general.name")

    def file_type(self):
        return self.get_u64("general.file_type")

    def arch_u64(self, suffix: str):
        """An "<architecture>.<suffix>" key (archU64, gguf_file.hpp:85-86)."""
        return self.get_u64(f"{self.architecture}.{suffix}") if self.architecture else None

    # ---- tensor data ----------------------------------------------------------------------------
    def tensor_bytes(self, name: str):
        """numpy uint8 view of the tensor's raw bytes in the mapping (valid while the file is open)."""
        import numpy as np
        t = self._need(name)
        p = lib().qvx_gguf_tensor_data(self._h, t.index)
        if not p:
            raise GgufParseError(f"tensor '{name}': the file does not carry its data")
        return np.ctypeslib.as_array((C.c_uint8 * t.n_bytes).from_address(p)) if t.n_bytes else np.zeros(0, np.uint8)

    def upload(self, name: str, device="cuda"):
        """Copies the tensor's raw blocks to a fresh device buffer (16-byte aligned); returns a
        decode.DevWeight of [rows, cols] in the tensor's type."""
        import torch

        from .decode import DevWeight
        t = self._need(name)
        buf = torch.empty(max(t.n_bytes, 1), dtype=torch.uint8, device=device)
        stream = torch.cuda.current_stream(buf.device).cuda_stream
        _check(lib().qvx_gguf_upload(self._h, t.index, buf.data_ptr(), buf.numel(), stream), "qvx_gguf_upload")
        return DevWeight(buf[:t.n_bytes], t.type_raw, t.rows, t.cols)

    def _need(self, name: str) -> GgufTensor:
        t = self._by_name.get(name)
        if t is None:
            raise KeyError(name)
        return t
