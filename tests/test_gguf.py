"""GGUF reader (include/mlxr_gguf.h, mlxr_amd/gguf.py): the reference's own parser tests
(tests/unit/gguf_parser_test.cpp:14-168) restated over files written by tests/gguf_writer.py,
plus the fixes the build makes (GGUF block sizes, general.alignment, bounds checks)."""
import numpy as np
import pytest

import mlxr_amd as mx
from mlxr_amd import gguf
from tests import gguf_writer as gw
from tests.gguf_writer import ARR, BOOL, F32, F64, I8, I16, I32, I64, STR, U8, U16, U32, U64

T = gguf.GGMLType


def _minimal(version=3):
    """The file of the reference's create_minimal_gguf (gguf_parser_test.cpp:15-77)."""
    w = gw.Writer(version)
    w.add("general.architecture", STR, "llama")
    w.add("llama.context_length", U32, 2048)
    w.add("llama.embedding_length", U32, 4096)
    w.tensors.append(("token_embd.weight", [32000, 4096], T.F16, b""))  # info only, no data
    return w.to_bytes(declared_offsets=[0])[0]


def test_parse_minimal_file(tmp_path):
    p = tmp_path / "test_minimal.gguf"
    p.write_bytes(_minimal())
    g = gguf.GGUFFile()
    assert g.parse(str(p))
    assert not g.has_error()
    h = g.header()
    assert (h.magic, h.version, h.tensor_count, h.metadata_kv_count) == (gguf.GGUF_MAGIC, 3, 1, 3)
    for k in ("general.architecture", "llama.context_length", "llama.embedding_length"):
        assert g.has_metadata(k)
    assert g.get_arch() == "llama"
    assert g.get_context_length() == 2048
    assert g.get_embedding_length() == 4096
    assert len(g.tensors()) == 1
    t = g.find_tensor("token_embd.weight")
    assert t is not None and t.n_dimensions == 2 and t.dimensions == [32000, 4096] and t.type == T.F16
    assert t.size == 32000 * 4096 * 2
    # defaults of the reference getters (gguf_parser.cpp:493-550)
    assert g.get_block_count() == 0 and g.get_attention_head_count_kv() == g.get_attention_head_count() == 0
    assert g.get_rope_freq_base() == 10000.0 and g.get_tokenizer_model() == ""
    # the header describes data that is not in the file: parse succeeds, the view refuses
    with pytest.raises(mx.QGemmError, match="outside"):
        g.tensor_bytes("token_embd.weight")
    assert g.find_tensor("missing") is None
    g.close()


def test_invalid_magic(tmp_path):
    data = bytearray(16)
    data[0:4] = (0x12345678).to_bytes(4, "little")
    p = tmp_path / "test_bad_magic.gguf"
    p.write_bytes(bytes(data))
    g = gguf.GGUFFile()
    assert not g.parse(str(p))
    assert g.has_error() and "magic" in g.error()
    assert not g.parse(str(tmp_path / "absent.gguf"))
    assert "Failed to open" in g.error()


def test_unsupported_version():
    raw = bytearray(_minimal())
    raw[4:8] = (4).to_bytes(4, "little")
    g = gguf.GGUFFile()
    assert not g.parse_bytes(bytes(raw)) and "version" in g.error()


def test_tensor_size_calculation():
    assert gguf.calculate_tensor_size([4096, 11008], T.F16) == 4096 * 11008 * 2
    n = 4096 * 11008
    assert gguf.calculate_tensor_size([4096, 11008], T.Q4_0) == (n + 31) // 32 * 18
    # GGUF block bytes (ggml type traits); the reference has Q6_K 208, Q2_K 80, Q3_K 108
    expect = {T.Q4_0: 18, T.Q4_1: 20, T.Q5_0: 22, T.Q5_1: 24, T.Q8_0: 34, T.Q8_1: 36, T.Q2_K: 84, T.Q3_K: 110,
              T.Q4_K: 144, T.Q5_K: 176, T.Q6_K: 210, T.Q8_K: 292}
    for t, b in expect.items():
        be = gguf.gguf_block_size(t)
        assert be == (256 if t >= T.Q2_K else 32)
        assert gguf.type_bytes(t, be * 3) == 3 * b
    for t, b in {T.F32: 4, T.F16: 2, T.BF16: 2, T.F64: 8, T.I8: 1, T.I16: 2, T.I32: 4, T.I64: 8}.items():
        assert gguf.gguf_block_size(t) == 1 and gguf.type_bytes(t, 5) == 5 * b
    # consistent with the matmul's own size helper for the types it runs
    for t, qt in ((T.Q4_K, mx.QuantType.Q4_K), (T.Q6_K, mx.QuantType.Q6_K), (T.Q8_0, mx.QuantType.Q8_0),
                  (T.Q5_K, mx.QuantType.Q5_K), (T.Q4_0, mx.QuantType.Q4_0), (T.Q4_1, mx.QuantType.Q4_1)):
        assert gguf.calculate_tensor_size([4096, 1024], t) == mx.gguf_size(qt, 1024, 4096)
    with pytest.raises(mx.QGemmError):
        gguf.type_bytes(T.Q4_K, 100)  # not whole blocks
    with pytest.raises(mx.QGemmError):
        gguf.type_bytes(99, 32)


def test_type_names():
    assert gguf.gguf_type_name(T.F32) == "F32"
    assert gguf.gguf_type_name(T.F16) == "F16"
    assert gguf.gguf_type_name(T.Q4_0) == "Q4_0"
    assert gguf.gguf_type_name(T.Q4_K) == "Q4_K"
    assert gguf.gguf_type_name(T.Q6_K) == "Q6_K"
    assert gguf.gguf_type_name(77) == "UNKNOWN"
    assert gguf.quant_type(T.Q4_K) == mx.QuantType.Q4_K
    assert gguf.quant_type(T.Q6_K) == mx.QuantType.Q6_K
    assert gguf.quant_type(T.Q8_0) == mx.QuantType.Q8_0
    assert gguf.quant_type(T.Q5_K) == mx.QuantType.Q5_K
    assert gguf.quant_type(T.Q4_0) == mx.QuantType.Q4_0
    with pytest.raises(mx.QGemmError):
        gguf.quant_type(T.F16)


@pytest.mark.parametrize("version", [1, 2, 3])
def test_metadata_types(version):
    w = gw.Writer(version)
    vals = [("u8", U8, 200), ("i8", I8, -100), ("u16", U16, 60000), ("i16", I16, -30000), ("u32", U32, 4000000000),
            ("i32", I32, -2000000000), ("f32", F32, 1.5), ("b", BOOL, True), ("s", STR, "héllo"),
            ("u64", U64, 2 ** 63 + 5), ("i64", I64, -(2 ** 62)), ("f64", F64, -2.25)]
    for k, t, v in vals:
        w.add(k, t, v)
    w.add("toks", ARR, (STR, ["<s>", "", "world"]))
    w.add("scores", ARR, (F32, [0.5, -1.0, 2.0]))
    w.add("ids", ARR, (I32, [-1, 2, 3]))
    w.add("nested", ARR, (ARR, [(U8, [1, 2]), (U8, [3])]))
    w.add("empty", ARR, (U64, []))
    w.add("tokenizer.ggml.model", STR, "llama")
    g = gguf.GGUFFile()
    assert g.parse_bytes(w.to_bytes()[0]), g.error()
    md = g.metadata()
    assert list(md)[:len(vals)] == [k for k, _, _ in vals]
    for k, t, v in vals:
        assert md[k] == v, k
        assert g.metadata_type(k) == t
    assert md["toks"] == ["<s>", "", "world"]
    assert md["scores"].dtype == np.float32 and md["scores"].tolist() == [0.5, -1.0, 2.0]
    assert md["ids"].tolist() == [-1, 2, 3]
    assert md["nested"] is None and md["empty"].size == 0
    assert g.get_tokenizer_model() == "llama"
    assert g.header().version == version


def test_alignment_and_tensor_views(tmp_path):
    rng = np.random.default_rng(5)
    for align in (None, 64, 4096):
        w = gw.Writer(3, alignment=align)
        w.add("general.architecture", STR, "llama")
        a = rng.standard_normal((3, 40)).astype(np.float32)
        q = mx.synth_gguf(mx.QuantType.Q4_K, 8, 512, 11)
        w.add_tensor("a", [40, 3], T.F32, a.tobytes())
        w.add_tensor("blk.0.ffn_up.weight", [512, 8], T.Q4_K, q.tobytes())
        raw, data_start = w.to_bytes()
        p = tmp_path / f"t{align}.gguf"
        p.write_bytes(raw)
        with gguf.GGUFFile(str(p)) as g:
            assert g.alignment() == (align or 32)
            assert g.data_offset() == data_start and data_start % (align or 32) == 0
            assert g.get_tensor_names() == ["a", "blk.0.ffn_up.weight"]
            ta = g.find_tensor("a")
            assert ta.file_offset == data_start + ta.offset
            assert np.array_equal(g.tensor_bytes("a").view(np.float32).reshape(3, 40), a)
            assert np.array_equal(g.tensor_bytes("blk.0.ffn_up.weight"), q)
            assert g.find_tensor("blk.0.ffn_up.weight").offset % (align or 32) == 0


def test_bad_alignment():
    w = gw.Writer(3, alignment=48)
    g = gguf.GGUFFile()
    assert not g.parse_bytes(w.to_bytes()[0]) and "alignment" in g.error()


def test_every_truncation_fails_cleanly():
    """Each prefix of a valid header is rejected with an error (no read past the end)."""
    w = gw.Writer(3)
    w.add("general.architecture", STR, "llama")
    w.add("toks", ARR, (STR, ["a", "bc"]))
    w.add("ids", ARR, (I16, [1, 2, 3]))
    w.add_tensor("x", [32, 2], T.Q8_0, bytes(68))
    raw, data_start = w.to_bytes()
    g = gguf.GGUFFile()
    # data_start is the header end rounded up to 32, so every prefix below data_start - 31
    # cuts the header itself
    for n in range(0, data_start - 31):
        assert not g.parse_bytes(raw[:n]), n
        assert g.has_error()
    assert g.parse_bytes(raw)


def test_garbage_counts_and_lengths():
    raw = bytearray(_minimal())
    raw[8:16] = (2 ** 60).to_bytes(8, "little")  # tensor count
    g = gguf.GGUFFile()
    assert not g.parse_bytes(bytes(raw)) and "implausible" in g.error()
    raw = bytearray(_minimal())
    raw[24:32] = (2 ** 40).to_bytes(8, "little")  # length of the first key
    assert not g.parse_bytes(bytes(raw))
    raw = bytearray(_minimal())
    raw[24 + 8 + 20:24 + 8 + 20 + 4] = (77).to_bytes(4, "little")  # value type of the first key
    assert not g.parse_bytes(bytes(raw)) and "metadata type" in g.error()
