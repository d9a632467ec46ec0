"""CPU tests of the GGUF reader (qvx_gguf_*, qorvix_amd/gguf.py): header, metadata and typed
accessors, arrays (nested ones included), the tensor table with computed sizes and data offset,
v1/v2 files, file mapping, and every rejection the public format implies (the cases of the
reference's tests/gguf_file_test.cpp among them).  No GPU is touched."""
from __future__ import annotations

import ctypes as C
import struct

import pytest

import qorvix_amd as qvx
from gguf_build import ARR, F32 as MF32, I32 as MI32, STR, U32 as MU32, GgufBuilder
from qorvix_amd.gguf import GgufFile, GgufParseError, ggml_type_name


def sample_model(version=3):
    b = GgufBuilder(version)
    (b.str("general.architecture", "llama").str("general.name", "tiny-test").u32("general.alignment", 32)
     .u32("general.file_type", 15).u64("llama.context_length", 4096).u32("llama.attention.head_count", 32)
     .f32("llama.rope.freq_base", 10000.0).u32("llama.rope.dimension_count", 128)
     .boolean("tokenizer.ggml.add_bos_token", True)
     .array("tokenizer.ggml.tokens", STR, ["<s>", "</s>", "hello", "world"])
     .array("tokenizer.ggml.token_type", MI32, [1, 1, 1, 1]))
    b.tensor("token_embd.weight", [64, 4], qvx.F32, 0)              # 256 elems * 4 B = 1024 B
    b.tensor("blk.0.ffn_down.weight", [256], qvx.Q4_K, 1024)        # one Q4_K block = 144 B
    return b.build(32, data_bytes=1024 + 144)


def test_header_metadata_and_typed_accessors():
    f = GgufFile.parse(sample_model())
    assert f.version == 3 and f.alignment == 32
    assert f.architecture == "llama" and f.name() == "tiny-test" and f.file_type() == 15
    assert f.get_u64("llama.context_length") == 4096
    assert f.arch_u64("attention.head_count") == 32
    assert f.get_f64("llama.rope.freq_base") == 10000.0
    assert f.get_bool("tokenizer.ggml.add_bos_token") is True
    assert f.get_string("general.architecture") == "llama"
    # wrong category -> None (the reference's optional accessors)
    assert f.get_u64("general.name") is None and f.get_string("llama.context_length") is None
    assert f.get_bool("general.file_type") is None and f.get_u64("no.such.key") is None
    assert [k for k, _ in f.metadata][:3] == ["general.architecture", "general.name", "general.alignment"]


def test_arrays():
    f = GgufFile.parse(sample_model())
    assert f.find("tokenizer.ggml.tokens") == ["<s>", "</s>", "hello", "world"]
    assert f.find("tokenizer.ggml.token_type") == [1, 1, 1, 1]


def test_tensor_table_sizes_and_data_offset():
    data = sample_model()
    f = GgufFile.parse(data)
    assert len(f.tensors) == 2
    e = f.tensor("token_embd.weight")
    assert e.dimensions == (64, 4) and e.n_elements == 256 and e.n_bytes == 1024 and e.type_name() == "F32"
    assert (e.cols, e.rows) == (64, 4)
    d = f.tensor("blk.0.ffn_down.weight")
    assert d.n_elements == 256 and d.n_bytes == 144 and d.offset == 1024 and d.type_name() == "Q4_K"
    assert f.data_offset % 32 == 0 and f.data_offset < len(data)
    # the data views point at the right bytes
    raw = f.tensor_bytes("blk.0.ffn_down.weight")
    assert bytes(raw) == data[f.data_offset + 1024:f.data_offset + 1024 + 144]
    assert f.tensor("missing") is None


@pytest.mark.parametrize("version", [1, 2])
def test_older_versions_parse_identically(version):
    f = GgufFile.parse(sample_model(version))
    assert f.version == version and f.architecture == "llama" and len(f.tensors) == 2
    assert f.tensor("blk.0.ffn_down.weight").n_bytes == 144
    assert f.find("tokenizer.ggml.tokens")[2] == "hello"


def test_rejects_bad_magic():
    with pytest.raises(GgufParseError, match="no GGUF magic"):
        GgufFile.parse(bytes(16))
    with pytest.raises(GgufParseError, match="big-endian"):
        GgufFile.parse(b"FUGG" + bytes(12))
    with pytest.raises(GgufParseError, match="no GGUF magic"):
        GgufFile.parse(b"GG")


def test_rejects_unsupported_version():
    with pytest.raises(GgufParseError, match="version 99 is not one of 1, 2, 3"):
        GgufFile.parse(GgufBuilder(99).build())


def test_rejects_truncation_mid_metadata():
    with pytest.raises(GgufParseError, match="file ends inside"):
        GgufFile.parse(sample_model()[:150])
    # every cut inside the header and tables is refused, never read past
    full = sample_model()
    for cut in range(0, 200, 7):
        with pytest.raises(GgufParseError):
            GgufFile.parse(full[:cut])


def test_rejects_misaligned_tensor_offset():
    b = GgufBuilder(3).str("general.architecture", "llama").u32("general.alignment", 32)
    b.tensor("bad.weight", [32], qvx.F32, 7)
    with pytest.raises(GgufParseError, match="not a multiple of the alignment"):
        GgufFile.parse(b.build())


def test_rejects_block_size_mismatch():
    b = GgufBuilder(3).str("general.architecture", "llama")
    b.tensor("bad.weight", [100], qvx.Q4_K, 0)
    with pytest.raises(GgufParseError, match="not whole blocks of 256"):
        GgufFile.parse(b.build())
    # whole blocks in total but not per row: 100 x 256 elements with rows of 100
    b = GgufBuilder(3)
    b.tensor("bad.weight", [100, 256], qvx.Q4_K, 0)
    with pytest.raises(GgufParseError, match="rows of 100 elements"):
        GgufFile.parse(b.build(32, data_bytes=100 * 144))


def test_nested_arrays_parse_and_are_skipped():
    """The format allows arrays of arrays: they are walked (what follows them parses), reported as
    arrays, and their elements are not exposed as scalars."""
    b = (GgufBuilder(3).array("a", ARR, [(MU32, [1, 2, 3]), (STR, ["x", "yz"])]).array("e", ARR, [])
         .u32("after", 7))
    f = GgufFile.parse(b.build())
    assert f.get_u64("after") == 7
    assert f.find("a") == [None, None] and f.find("e") == []
    lib = qvx.lib()
    out = C.c_uint64()
    assert lib.qvx_gguf_meta_u64(f._h, b"a", 0, C.byref(out)) == qvx.E_TYPE


def test_rejects_unknown_types_and_impossible_lengths():
    with pytest.raises(GgufParseError, match="value type 77 is not defined"):
        GgufFile.parse(_raw_kv_type(77))
    # an array that claims more elements than the buffer could hold
    head = struct.pack("<IIQQ", 0x46554747, 3, 0, 1) + struct.pack("<Q", 1) + b"k" + struct.pack("<IIQ", ARR, MU32, 1 << 40)
    with pytest.raises(GgufParseError, match="runs past the end of the file"):
        GgufFile.parse(head)
    head = struct.pack("<IIQQ", 0x46554747, 3, 0, 1) + struct.pack("<Q", 1) + b"k" + struct.pack("<IIQ", ARR, STR, 1 << 40)
    with pytest.raises(GgufParseError, match="runs past the end of the file"):
        GgufFile.parse(head)
    # counts that cannot fit are refused before anything is reserved
    with pytest.raises(GgufParseError, match="metadata count"):
        GgufFile.parse(struct.pack("<IIQQ", 0x46554747, 3, 0, 1 << 60))
    with pytest.raises(GgufParseError, match="tensor count"):
        GgufFile.parse(struct.pack("<IIQQ", 0x46554747, 3, 1 << 60, 0))


def test_rejects_duplicate_keys_and_tensor_names():
    with pytest.raises(GgufParseError, match="key 'k' appears twice"):
        GgufFile.parse(GgufBuilder(3).u32("k", 1).u32("k", 2).build())
    b = GgufBuilder(3)
    b.tensor("t", [32], qvx.F32, 0).tensor("t", [32], qvx.F32, 128)
    with pytest.raises(GgufParseError, match="tensor name 't' appears twice"):
        GgufFile.parse(b.build(32, data_bytes=256))


def _raw_kv_type(tag):
    return struct.pack("<IIQQ", 0x46554747, 3, 0, 1) + struct.pack("<Q", 1) + b"k" + struct.pack("<I", tag) + b"\0" * 8


def test_rejects_rank_overflow_and_data_extent():
    b = GgufBuilder(3)
    b.tensor("t", [2] * 5, qvx.F32, 0)
    with pytest.raises(GgufParseError, match="5 dimensions"):
        GgufFile.parse(b.build())
    b = GgufBuilder(3)
    b.tensor("t", [2] * 4, qvx.F32, 0)  # four is the format's maximum
    assert GgufFile.parse(b.build(32, data_bytes=64)).tensor("t").n_elements == 16
    b = GgufBuilder(3)
    b.tensor("t", [1 << 40, 1 << 40], qvx.F32, 0)
    with pytest.raises(GgufParseError, match="does not fit in 64 bits"):
        GgufFile.parse(b.build())
    b = GgufBuilder(3)
    b.tensor("t", [1 << 62, 2], qvx.F32, 0)  # elements fit, bytes do not
    with pytest.raises(GgufParseError, match="does not fit in 64 bits"):
        GgufFile.parse(b.build())
    b = GgufBuilder(3)
    b.tensor("t", [256], qvx.F32, 0)  # 1024 bytes, but the file carries 100
    with pytest.raises(GgufParseError, match="outside the file's data section"):
        GgufFile.parse(b.build(32, data_bytes=100))


def test_data_must_be_in_the_file():
    """A buffer that stops after the tables (or whose tensor offset points past its end) is not a
    GGUF file: a tensor's bytes must lie in the data section."""
    b = GgufBuilder(3)
    b.tensor("t", [256], qvx.Q4_K, 0)
    with pytest.raises(GgufParseError, match="outside the file's data section"):
        GgufFile.parse(b.header_and_tables())
    b = GgufBuilder(3)
    b.tensor("t", [256], qvx.Q4_K, (1 << 64) - 32)  # aligned offset near 2^64: no wrap-around
    with pytest.raises(GgufParseError, match="outside the file's data section"):
        GgufFile.parse(b.build(32, data_bytes=144))
    # a tensor of an id without known block size occupies no known bytes and is only listed
    b = GgufBuilder(3)
    b.tensor("odd", [32], 4, 0)
    f = GgufFile.parse(b.build())
    assert f.tensor("odd").n_bytes == 0


def test_alignment_key_and_default():
    b = GgufBuilder(3).u32("general.alignment", 64)
    b.tensor("t", [16], qvx.F32, 64)
    f = GgufFile.parse(b.build(64, data_bytes=128))
    assert f.alignment == 64 and f.data_offset % 64 == 0
    assert GgufFile.parse(GgufBuilder(3).build()).alignment == 32  # default
    for bad in (0, 48):
        with pytest.raises(GgufParseError, match="not a power of two"):
            GgufFile.parse(GgufBuilder(3).u32("general.alignment", bad).build())
    with pytest.raises(GgufParseError, match="must be a u32"):
        GgufFile.parse(GgufBuilder(3).u64("general.alignment", 32).build())


def test_open_maps_a_file(tmp_path):
    p = tmp_path / "m.gguf"
    p.write_bytes(sample_model())
    with GgufFile.open(p) as f:
        assert f.tensor("token_embd.weight").n_bytes == 1024
        assert f.tensor_bytes("token_embd.weight")[:4].tolist() == list(sample_model()[f.data_offset:f.data_offset + 4])
    with pytest.raises(GgufParseError, match="cannot open"):
        GgufFile.open(tmp_path / "absent.gguf")


def test_type_names():
    assert ggml_type_name(12) == "Q4_K" and ggml_type_name(14) == "Q6_K" and ggml_type_name(4) == "UNKNOWN(4)"


def test_c_abi_null_and_range_handling():
    lib = qvx.lib()
    assert lib.qvx_gguf_tensor_count(None) == 0 and lib.qvx_gguf_version(None) == 0
    assert lib.qvx_gguf_find_tensor(None, b"x") == -1
    assert lib.qvx_gguf_tensor_data(None, 0) is None
    assert lib.qvx_gguf_upload(None, 0, None, 0, None) == qvx.E_RANGE
    assert lib.qvx_gguf_parse(None, 4, None) == qvx.E_NULL
    lib.qvx_gguf_close(None)
