"""GGUF reader (native, behind the C ABI) on the CPU: header, metadata with the
reference's Java typing, tensor infos, raw tensor bytes, llamafile ZIP
variants and LlamaConfig.from_gguf.

The llamafile cases are the reference's own (GgufReaderTest.java:576-794):
a stored entry behind an APE stub, the EOCD beyond the backward window (forward
scan), and a stub larger than one 1 MiB scan window.  The expected values are
the reference tests' values.  Float widening of F32 / F16 / BF16 tensors runs
on the host and is checked here; packed types are dequantized on the device
(tests/test_gpu_gguf.py).
"""
import struct

import numpy as np
import pytest

import oracle as O
from gguf_build import (ARRAY, BOOL, FLOAT32, FLOAT64, INT8, INT16, INT32, INT64, STRING, UINT8, UINT16, UINT32,
                        UINT64, big_stub_llamafile, f32_bytes, gguf_bytes, llamafile, minimal_gguf, zip64_llamafile)
from juno_amd import GgufArray, GgufReader, IllegalArgumentException, IOException, UnsupportedOperationException
from juno_amd.decode import LlamaConfig


def write(tmp_path, name, data: bytes):
    p = tmp_path / name
    p.write_bytes(data)
    return p


def open_bytes(tmp_path, data: bytes, name="m.gguf"):
    return GgufReader.open(write(tmp_path, name, data))


# ------------------------------------------------------------------ reference llamafile cases

def test_llamafile_opens_and_reads_tensor(tmp_path):  # GgufReaderTest.java:574-594
    g = minimal_gguf("inner", 0, 4, f32_bytes([1, 2, 3, 4]))
    with open_bytes(tmp_path, llamafile("inner.gguf", g), "inner.llamafile") as r:
        assert r.tensor("inner").tolist() == [1.0, 2.0, 3.0, 4.0]
        assert r.gguf_file_offset() > 0


def test_zip_offset_points_to_gguf_magic(tmp_path):  # GgufReaderTest.java:596-616
    g = minimal_gguf("magic_check", 0, 8, bytes(32))
    data = llamafile("magic_check.gguf", g)
    with open_bytes(tmp_path, data, "x.llamafile") as r:
        off = r.gguf_file_offset()
    assert struct.unpack_from("<I", data, off)[0] == 0x46554747
    assert data[off:off + len(g)] == g


def test_plain_gguf_opens(tmp_path):  # GgufReaderTest.java:618-632
    with open_bytes(tmp_path, minimal_gguf("plain", 0, 4, f32_bytes([-1, 0, 1, 2]))) as r:
        assert r.tensor("plain").tolist() == [-1.0, 0.0, 1.0, 2.0]
        assert r.gguf_file_offset() == 0


def test_llamafile_q8_0_tensor_round_trips(tmp_path, ):  # GgufReaderTest.java:634-656
    block = struct.pack("<H", 0x3800) + bytes(range(32))
    with open_bytes(tmp_path, llamafile("q8test.gguf", minimal_gguf("q8test", 8, 32, block)), "q8.llamafile") as r:
        qt = r.tensor_raw("q8test")
        assert (qt.name, qt.type, qt.nelems, qt.data) == ("q8test", 8, 32, block)
        # dequantized by the oracle here (the device path is covered by the GPU tests)
        assert np.allclose(O.dequantize(8, np.frombuffer(qt.data, np.uint8), 1, 32), 0.5 * np.arange(32), atol=1e-3)


def test_llamafile_overlay_uses_forward_scan(tmp_path):  # GgufReaderTest.java:658-700
    g = minimal_gguf("overlay_test", 0, 4, f32_bytes([5, 6, 7, 8]))
    data = llamafile("overlay_test.gguf", g, overlay=b"\xcc" * 70_000)
    with open_bytes(tmp_path, data, "big.llamafile") as r:
        assert r.tensor("overlay_test").tolist() == [5.0, 6.0, 7.0, 8.0]


def test_llamafile_large_ape_stub_forward_scan(tmp_path):  # GgufReaderTest.java:702-794
    g = minimal_gguf("bigstub", 0, 4, f32_bytes([-3, -2, -1, 0]))
    with open_bytes(tmp_path, big_stub_llamafile("bigstub.gguf", g), "bigstub.llamafile") as r:
        assert r.tensor("bigstub").tolist() == [-3.0, -2.0, -1.0, 0.0]
        assert r.gguf_file_offset() == 1_200_000 + 30 + len("bigstub.gguf")


def test_forward_scan_finds_signature_across_the_1mib_window(tmp_path):
    # the local header starts 2 bytes before the 1 MiB boundary: its signature spans two scan windows
    g = minimal_gguf("edge", 0, 4, f32_bytes([9, 8, 7, 6]))
    data = big_stub_llamafile("edge.gguf", g, stub_len=(1 << 20) - 2)
    with open_bytes(tmp_path, data, "edge.llamafile") as r:
        assert r.tensor("edge").tolist() == [9.0, 8.0, 7.0, 6.0]


def test_zip64_llamafile(tmp_path):
    g = minimal_gguf("z64", 0, 4, f32_bytes([1.5, 2.5, 3.5, 4.5]))
    with open_bytes(tmp_path, zip64_llamafile("z64.gguf", g), "z64.llamafile") as r:
        assert r.tensor("z64").tolist() == [1.5, 2.5, 3.5, 4.5]


def test_llamafile_picks_the_gguf_entry_among_others(tmp_path):
    g = minimal_gguf("w", 0, 2, f32_bytes([4, 5]))
    data = llamafile("model.gguf", g, others=[(".args", b"-m model.gguf\n"), ("readme.txt", b"GGUF is not here")])
    with open_bytes(tmp_path, data, "multi.llamafile") as r:
        assert r.tensor("w").tolist() == [4.0, 5.0]


def test_zip_without_gguf_entry_is_rejected(tmp_path):
    data = llamafile("weights.bin", minimal_gguf("w", 0, 2, f32_bytes([4, 5])))
    with pytest.raises(IOException, match="No .gguf entry"):
        open_bytes(tmp_path, data, "nogguf.llamafile")


def test_neither_gguf_nor_zip_is_rejected(tmp_path):
    with pytest.raises(IOException, match="neither a GGUF nor a llamafile"):
        open_bytes(tmp_path, b"\x7fELF" + bytes(200), "x.bin")
    with pytest.raises(IOException):
        open_bytes(tmp_path, b"GG", "short.bin")
    with pytest.raises(IOException, match="cannot open"):
        GgufReader.open(tmp_path / "missing.gguf")


# ------------------------------------------------------------------ header and layout

def test_version_gate(tmp_path):  # GgufReader.java:131-132
    for v in (2, 3):
        with open_bytes(tmp_path, gguf_bytes(version=v), f"v{v}.gguf") as r:
            assert r.version == v
    for v in (1, 4):
        with pytest.raises(IOException, match=f"Unsupported GGUF version: {v}"):
            open_bytes(tmp_path, gguf_bytes(version=v), f"v{v}.gguf")


def test_data_offset_is_32_aligned_from_the_gguf_start(tmp_path):  # GgufReader.java:168-176
    meta = [("general.name", STRING, "x" * 5)]
    g = gguf_bytes(meta, [("t", [8], 0, f32_bytes(range(8)))])
    with open_bytes(tmp_path, g) as r:
        assert r.data_offset % 32 == 0 and r.data_offset == len(g) - 32
        assert r.metadata_section_end() == 24 + 8 + len("general.name") + 4 + 8 + 5
        assert r.tensor_absolute_offset("t") == r.data_offset
    stub = b"MZ" + bytes(7)  # GGUF image at an odd file offset: alignment is relative to it
    with open_bytes(tmp_path, llamafile("a.gguf", g, stub=stub), "a.llamafile") as r:
        assert (r.data_offset - r.gguf_file_offset()) % 32 == 0
        assert r.data_offset % 32 != 0
        assert r.tensor("t").tolist() == list(map(float, range(8)))


def test_tensor_infos_and_raw_bytes(tmp_path):
    rng = np.random.default_rng(3)
    q4 = rng.integers(0, 256, 144 * 6, dtype=np.uint8).tobytes()
    q6 = rng.integers(0, 256, 210 * 2, dtype=np.uint8).tobytes()
    tensors = [("blk.0.ffn_up.weight", [512, 3], 12, q4), ("blk.0.attn_v.weight", [256, 2], 14, q6),
               ("norm", [5], 0, f32_bytes([1, 2, 3, 4, 5]))]
    with open_bytes(tmp_path, gguf_bytes((), tensors)) as r:
        assert r.tensor_order() == [t[0] for t in tensors]
        assert r.tensor_dims("blk.0.ffn_up.weight") == (512, 3)
        assert r.tensor_nelems("blk.0.ffn_up.weight") == 1536
        assert r.tensor_type("blk.0.attn_v.weight") == 14
        assert r.tensor_raw("blk.0.ffn_up.weight").data == q4
        assert r.tensor_raw("blk.0.attn_v.weight").data == q6
        assert r.has_tensor("norm") and not r.has_tensor("nope")
        offs = [r.tensor_absolute_offset(t[0]) for t in tensors]
        assert all(o % 32 == 0 for o in offs) and offs == sorted(offs)
        with pytest.raises(IllegalArgumentException, match="Tensor not found: nope"):
            r.tensor_raw("nope")
        with pytest.raises(IllegalArgumentException, match="Tensor not found"):
            r.tensor_dims("nope")


def test_f16_and_bf16_tensors_widen_exactly(tmp_path):
    h = np.array([0x3400, 0x3C00, 0xC000, 0x0000, 0x7BFF, 0x0001, 0x8000], dtype="<u2")  # GgufReaderTest.java:35-46 + extremes
    bf = np.array([0x3F80, 0xC040, 0x0001, 0x7F7F], dtype="<u2")
    with open_bytes(tmp_path, gguf_bytes((), [("h", [7], 1, h.tobytes()), ("b", [4], 30, bf.tobytes())])) as r:
        got = r.tensor("h")
        assert got[:4].tolist() == [0.25, 1.0, -2.0, 0.0]
        assert got[4] == 65504.0 and got[5] == 2.0 ** -24 and np.signbit(got[6])
        assert r.tensor("b").view(np.uint32).tolist() == [0x3F800000, 0xC0400000, 0x00010000, 0x7F7F0000]


def test_raw_byte_count_every_reference_type():  # GgufReader.java:347-360
    rb = GgufReader.raw_byte_count
    assert [rb(t, 512) for t in (0, 1, 30, 8, 2, 10, 11, 12, 13, 14)] == \
        [2048, 1024, 1024, 16 * 34, 16 * 18, 2 * 84, 2 * 110, 2 * 144, 2 * 176, 2 * 210]
    with pytest.raises(UnsupportedOperationException, match="No byte-size formula for GGML type 99"):
        rb(99, 512)


def test_tensor_raw_of_q2k_q3k_and_unknown_types(tmp_path):
    q2 = bytes(range(84))
    with open_bytes(tmp_path, gguf_bytes((), [("q2", [256], 10, q2), ("odd", [4], 99, bytes(16))])) as r:
        assert r.tensor_raw("q2").data == q2
        with pytest.raises(UnsupportedOperationException, match="type 99"):
            r.tensor_raw("odd")


def test_truncated_file_is_rejected(tmp_path):
    g = gguf_bytes([("k", STRING, "value")], [("t", [8], 0, f32_bytes(range(8)))])
    for cut in (10, 30, 60):  # header, metadata, tensor info
        with pytest.raises(IOException):
            open_bytes(tmp_path, g[:cut], f"cut{cut}.gguf")
    with open_bytes(tmp_path, g[:-4], "short_data.gguf") as r:  # infos intact, data short
        with pytest.raises(IOException, match="Expected 32 bytes"):
            r.tensor_raw("t")


# ------------------------------------------------------------------ metadata typing (readMetadataValue)

META = [
    ("u8", UINT8, 255), ("i8", INT8, -5), ("u16", UINT16, 65535), ("i16", INT16, -300),
    ("u32", UINT32, 0xFFFFFFFF), ("i32", INT32, -7), ("u64", UINT64, 2**64 - 2), ("i64", INT64, 2**40 + 3),
    ("f32", FLOAT32, 1e-5), ("f64", FLOAT64, 1e300), ("b", BOOL, True), ("b0", BOOL, False), ("s", STRING, "héllo"),
    ("arr", ARRAY, (STRING, ["a", "bb", "ccc"])), ("nested", ARRAY, (ARRAY, [(INT32, [1, 2]), (INT32, [3])])),
    ("big", INT64, 5_000_000_000), ("fneg", FLOAT32, -3.75), ("nan", FLOAT64, float("nan")),
]


def test_metadata_java_typing(tmp_path):  # GgufReader.java:1189-1246
    with open_bytes(tmp_path, gguf_bytes(META)) as r:
        assert r.kv_count == len(META)
        # unsigned 8/16/32-bit values are read as signed Java int / short / byte
        assert (r.meta("u8"), r.meta("i8"), r.meta("u16"), r.meta("i16")) == (-1, -5, -1, -300)
        assert (r.meta("u32"), r.meta("i32")) == (-1, -7)
        assert r.meta("u64") == -2 and r.meta("i64") == 2**40 + 3  # UINT64 as signed long
        assert r.meta("f32") == float(np.float32(1e-5)) and r.meta("f64") == 1e300
        assert r.meta("b") is True and r.meta("b0") is False
        assert r.meta("s") == "héllo" and r.meta_string("s") == "héllo"
        assert r.meta("arr") == GgufArray(STRING, 3) and len(r.meta("arr")) == 3
        assert len(r.meta("nested")) == 2
        assert r.meta("missing") is None and r.meta_string("missing") is None and r.meta_string("u8") is None


def test_metadata_number_conversions(tmp_path):  # metaLong / metaInt / metaFloat, GgufReader.java:194-207
    with open_bytes(tmp_path, gguf_bytes(META)) as r:
        assert r.meta_int("big", 0) == 5_000_000_000 - 2**32  # Long.intValue(): low 32 bits
        assert r.meta_long("big", 0) == 5_000_000_000
        assert r.meta_int("fneg", 0) == -3 and r.meta_long("fneg", 0) == -3  # truncation
        assert r.meta_int("f64", 0) == 2**31 - 1 and r.meta_long("f64", 0) == 2**63 - 1  # saturation
        assert r.meta_int("nan", 9) == 0
        assert r.meta_float("i32", 0.0) == -7.0 and r.meta_float("f32", 0.0) == float(np.float32(1e-5))
        assert r.meta_float("u64", 0.0) == -2.0
        # not a Number -> the default
        assert r.meta_int("s", 42) == 42 and r.meta_long("b", 7) == 7 and r.meta_float("arr", 0.5) == 0.5
        assert r.meta_int("missing", 11) == 11


def test_repeated_key_keeps_the_last_value(tmp_path):  # HashMap.put
    with open_bytes(tmp_path, gguf_bytes([("k", INT32, 1), ("k", STRING, "two")])) as r:
        assert r.meta("k") == "two" and r.kv_count == 2


def test_unknown_metadata_type_is_rejected(tmp_path):
    g = bytearray(gguf_bytes([("k", INT32, 1)]))
    struct.pack_into("<i", g, 24 + 8 + 1, 13)  # the value type of the only entry
    with pytest.raises(IOException, match="bad metadata entry 0"):
        open_bytes(tmp_path, bytes(g))


# ------------------------------------------------------------------ LlamaConfig.from (LlamaConfig.java:58-100)

def test_llama_config_from_gguf_arch_prefix_and_tokenizer_vocab(tmp_path):
    meta = [("general.architecture", STRING, "phi3"), ("phi3.embedding_length", UINT32, 3072),
            ("phi3.block_count", UINT32, 32), ("phi3.attention.head_count", UINT32, 32),
            ("phi3.attention.head_count_kv", UINT32, 32), ("phi3.feed_forward_length", UINT32, 8192),
            ("phi3.vocab_size", UINT32, 32000), ("phi3.attention.layer_norm_rms_epsilon", FLOAT32, 1e-5),
            ("phi3.rope.freq_base", FLOAT32, 10000.0),
            ("tokenizer.ggml.tokens", ARRAY, (STRING, [f"t{i}" for i in range(32064)]))]
    with open_bytes(tmp_path, gguf_bytes(meta)) as r:
        c = LlamaConfig.from_gguf(r)
    assert (c.hidden_dim, c.num_layers, c.num_heads, c.num_kv_heads, c.head_dim) == (3072, 32, 32, 32, 96)
    assert (c.intermediate_size, c.vocab_size, c.architecture) == (8192, 32064, "phi3")
    assert c.rms_norm_eps == float(np.float32(1e-5)) and c.rope_theta == 10000.0


def test_llama_config_from_gguf_llama_fallbacks_and_defaults(tmp_path):
    meta = [("general.architecture", STRING, "mistral"), ("llama.embedding_length", UINT32, 4096),
            ("mistral.attention.head_count", UINT32, 32), ("llama.attention.head_count_kv", UINT32, 8),
            ("llama.rope.freq_base", FLOAT32, 500000.0), ("tokenizer.ggml.tokens", ARRAY, (STRING, ["a"]))]
    with open_bytes(tmp_path, gguf_bytes(meta)) as r:
        c = LlamaConfig.from_gguf(r)
    assert (c.hidden_dim, c.num_layers, c.num_heads, c.num_kv_heads, c.head_dim) == (4096, 22, 32, 8, 128)
    assert (c.intermediate_size, c.vocab_size) == (4096 * 11 // 4, 32000)
    assert c.rms_norm_eps == float(np.float32(1e-5)) and c.rope_theta == 500000.0
    with open_bytes(tmp_path, gguf_bytes(), "empty.gguf") as r:  # every default, architecture "llama"
        c = LlamaConfig.from_gguf(r)
    assert (c.hidden_dim, c.num_layers, c.num_heads, c.num_kv_heads, c.intermediate_size, c.vocab_size,
            c.architecture) == (2048, 22, 32, 32, 5632, 32000, "llama")
