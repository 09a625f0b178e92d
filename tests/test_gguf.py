"""GGUF reading on the data side of the matmul path (rocmforge_amd/gguf.py).

Restates the reference loader's own tests -- src/loader/parse.rs:360-400,
ggml_type.rs:97-150, file.rs:133-170, metadata.rs:158-203,
tests/loader_integration.rs:14-121 (there on a real Qwen2.5 file, here on a
seeded synthetic one) and src/gpu/weights.rs:1044-1108 -- then pins what they
leave open: byte-identical write->read round trips, the 32-byte data-section
rule, the KV value formatting (Rust Display of the typed value; signed codes
read as unsigned), truncated files, string/array limits, the Q4_K_M layer set
of profiling/results/phase8_q4_k_m_analysis.md:97-103, and real Qwen3-8B
Q4_K blocks (the golden JSON) read back out of a file and dequantized by the
oracle to the JSON's values.
"""
import json
import math
import struct
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O
from rocmforge_amd import gguf as g
from rocmforge_amd import synth
from rocmforge_amd.ops import GgmlType, InvalidWeightLayout, TensorRole, UnsupportedWeightType

GOLDEN = Path(__file__).resolve().parent / "golden" / "q4_k_m_qwen3_8b_ffn_gate_layer0_first3_blocks.json"


def _hdr(version, tensors, kv, magic=b"GGUF"):
    return magic + struct.pack("<IQQ", version, tensors, kv)


def _s(text: bytes):
    return struct.pack("<Q", len(text)) + text


# ---- parse.rs tests -------------------------------------------------------------

def test_valid_header_v3():
    h = g.parse_header(g._Reader(_hdr(3, 42, 10)))
    assert (h.version, h.tensor_count, h.kv_count) == (3, 42, 10)


def test_valid_header_v2():
    assert g.parse_header(g._Reader(_hdr(2, 1, 1))).version == 2


def test_bad_magic():
    with pytest.raises(g.InvalidMagic):
        g.parse_header(g._Reader(_hdr(3, 0, 0, magic=b"XGUF")))


@pytest.mark.parametrize("v", [1, 4])
def test_unsupported_version(v):
    with pytest.raises(g.UnsupportedVersion, match=str(v)):
        g.parse_header(g._Reader(_hdr(v, 0, 0)))


def test_read_string_basic():
    assert g._Reader(_s(b"hello")).string() == "hello"


def test_string_limits_and_utf8():
    with pytest.raises(g.StringTooLong):
        g._Reader(struct.pack("<Q", 100_000_001)).string()
    with pytest.raises(g.InvalidUtf8):
        g._Reader(_s(b"\xff\xfe")).string()
    with pytest.raises(g.LoadError):            # truncated
        g._Reader(struct.pack("<Q", 10) + b"abc").string()


# ---- ggml_type.rs tests -----------------------------------------------------------

def test_type_codes_round_trip():
    for v, t in [(0, "F32"), (1, "F16"), (2, "Q4_0"), (3, "Q4_1"), (6, "Q5_0"), (7, "Q5_1"), (8, "Q8_0"),
                 (10, "Q2_K"), (11, "Q3_K"), (12, "Q4_K"), (13, "Q5_K"), (14, "Q6_K")]:
        assert g.ggml_type_from_u32(v) == GgmlType[t]


@pytest.mark.parametrize("v", [4, 5, 9, 15, 99])
def test_unknown_type_is_error(v):
    with pytest.raises(g.UnknownTensorType):
        g.ggml_type_from_u32(v)


def test_bytes_for_elements():
    assert g.bytes_for_elements(GgmlType.F32, 100) == 400
    assert g.bytes_for_elements(GgmlType.Q4_0, 32) == 18
    assert g.bytes_for_elements(GgmlType.Q4_0, 33) == 36
    assert g.bytes_for_elements(GgmlType.Q4_K, 256) == 144
    assert g.bytes_for_elements(GgmlType.Q3_K, 256) == 110
    assert g.bytes_for_elements(GgmlType.Q3_K, 512) == 220
    assert g.bytes_for_elements(GgmlType.Q3_K, 201326592) == 86507520


def test_block_bytes_agree_with_kernel_layouts():
    # the block sizes the kernels and the oracle index with
    for fmt, t in (("q4_k", GgmlType.Q4_K), ("q6_k", GgmlType.Q6_K)):
        for k in (256, 4096, 14336):
            assert g.bytes_for_elements(t, k) == synth.row_bytes(fmt, k)
    assert json.loads(GOLDEN.read_text())["block_size_bytes"] == g.bytes_for_elements(GgmlType.Q4_K, 256)


# ---- file.rs tests ------------------------------------------------------------------

@pytest.mark.parametrize("dims,n", [([4096], 4096), ([4096, 32000], 4096 * 32000), ([64, 32, 8], 16384)])
def test_tensor_view_element_count(dims, n):
    assert g.TensorView("t", dims, GgmlType.F32, np.zeros(0, np.uint8)).element_count() == n


# ---- metadata.rs tests ------------------------------------------------------------

def _meta(**kv):
    return g.GgufMetadata({k.replace("__", "."): v for k, v in kv.items()})


def test_metadata_arch_prefix():
    assert _meta(general__architecture="qwen2", qwen2__block_count="28").block_count() == 28


def test_metadata_llama_fallback():
    assert _meta(general__architecture="newarch", llama__block_count="32").block_count() == 32


def test_metadata_head_dim_computed():
    m = _meta(general__architecture="llama", llama__embedding_length="4096", llama__attention__head_count="32")
    assert m.head_dim() == 128


def test_metadata_rope_freq_from_kv():
    m = _meta(general__architecture="qwen2", qwen2__rope__freq_base="1000000")
    assert m.rope_freq_base(10000.0) == 1_000_000.0


def test_metadata_kv_heads_gqa():
    m = _meta(general__architecture="qwen2", qwen2__attention__head_count_kv="2")
    assert m.attention_head_count_kv() == 2


def test_metadata_resolution_details():
    m = g.GgufMetadata({})
    assert m.architecture == "unknown"
    assert (m.block_count(), m.context_length(), m.head_dim(), m.attention_head_count_kv()) == (0, 2048, 0, None)
    assert m.rms_norm_eps(1e-5) == pytest.approx(1e-5)
    # zero, negative and non-numeric values fall through to the next key
    m = _meta(general__architecture="qwen3", qwen3__block_count="0", qwen3__n_layers="-3",
              qwen3__num_hidden_layers="36", qwen3__embedding_length="x", hidden_size="+2048")
    assert m.block_count() == 36 and m.embedding_length() == 2048
    # explicit head_dim wins over hidden/heads; llama.* does not shadow the arch key
    m = _meta(general__architecture="qwen3", qwen3__attention__key_length="128", qwen3__embedding_length="2560",
              qwen3__attention__head_count="32", llama__attention__key_length="64")
    assert m.head_dim() == 128
    # f32 parse rounds to f32; rope.freq_base un-prefixed in the raw KV
    m = _meta(general__architecture="qwen3", qwen3__attention__layer_norm_rms_epsilon="0.000001",
              rope__freq_base="500000")
    assert m.rms_norm_eps(1e-5) == float(np.float32(1e-6)) and m.rope_freq_base(1e4) == 500000.0


# ---- weights.rs matrix metadata ------------------------------------------------------

def test_matrix_meta_roles():
    m = g.build_matrix_meta("output.weight", [1024, 32000], GgmlType.Q4_0, is_lm_head=True)
    assert m.role == TensorRole.LM_HEAD and m.dims == [1024, 32000]
    m = g.build_matrix_meta("output.weight", [1024, 32000], GgmlType.Q4_0, is_lm_head=True, is_tied=True)
    assert m.role == TensorRole.TIED_LM_HEAD
    assert g.build_matrix_meta("blk.0.attn_q.weight", [4096, 4096], GgmlType.Q4_K).role == TensorRole.GENERIC
    assert g.derive_tensor_role(False, True) == TensorRole.GENERIC


def test_matrix_meta_rejections():
    with pytest.raises(InvalidWeightLayout):
        g.build_matrix_meta("output.weight", [32000], GgmlType.Q4_0, is_lm_head=True)
    for t in (GgmlType.F16, GgmlType.Q5_0, GgmlType.Q5_1, GgmlType.Q2_K, GgmlType.Q3_K):
        with pytest.raises(UnsupportedWeightType):
            g.build_matrix_meta("blk.0.attn_q.weight", [1024, 1024], t)
    # Q6_K is a supported matrix type (weights.rs:356-366); a Q4_K_M file
    # carries its attn_v / ffn_down / output tensors in it
    assert g.build_matrix_meta("blk.0.ffn_down.weight", [12288, 4096], GgmlType.Q6_K).wtype == GgmlType.Q6_K


# ---- KV values -------------------------------------------------------------------------

def _kv_file(tmp_path, entries, version=3):
    """entries: raw (key, type code, payload bytes); no tensors."""
    body = _hdr(version, 0, len(entries))
    for key, t, payload in entries:
        body += _s(key.encode()) + struct.pack("<I", t) + payload
    p = tmp_path / "kv.gguf"
    p.write_bytes(body)
    return g.GgufFile.open(p)


def test_kv_value_formatting(tmp_path):
    f = _kv_file(tmp_path, [
        ("u8", g.T_U8, b"\xff"), ("i8", g.T_I8, b"\xff"), ("bool", g.T_BOOL, b"\x01"),
        ("u16", g.T_U16, struct.pack("<H", 65535)), ("i32", g.T_I32, struct.pack("<i", -1)),
        ("f32a", g.T_F32, struct.pack("<f", 1e-6)), ("f32b", g.T_F32, struct.pack("<f", 1e6)),
        ("f32c", g.T_F32, struct.pack("<f", 0.1)), ("f32d", g.T_F32, struct.pack("<f", 1.5)),
        ("f32nan", g.T_F32, struct.pack("<f", math.nan)), ("f32inf", g.T_F32, struct.pack("<f", -math.inf)),
        ("u64", g.T_U64, struct.pack("<Q", 2**64 - 1)), ("i64", g.T_I64, struct.pack("<q", -2)),
        ("f64", g.T_F64, struct.pack("<d", 0.1)), ("str", g.T_STRING, _s("äb".encode())),
        ("arr", g.T_ARRAY, struct.pack("<IQ", g.T_U16, 3) + b"\0" * 6),
        ("nested", g.T_ARRAY, struct.pack("<IQ", g.T_ARRAY, 2) + (struct.pack("<IQ", g.T_STRING, 1) + _s(b"x")) * 2),
        ("weird", 77, b"\0\0\0\0"), ("after", g.T_U32, struct.pack("<I", 7)),
    ])
    want = {"u8": "255", "i8": "255", "bool": "1", "u16": "65535", "i32": "4294967295", "f32a": "0.000001",
            "f32b": "1000000", "f32c": "0.1", "f32d": "1.5", "f32nan": "NaN", "f32inf": "-inf",
            "u64": str(2**64 - 1), "i64": str(2**64 - 2), "f64": "0.1", "str": "äb", "arr": "array:3",
            "nested": "array:2", "weird": "unknown", "after": "7"}
    assert f.metadata.raw == want
    assert f.tensor_count() == 0 and f.data_start % 32 == 0


def test_tokenizer_interception(tmp_path):
    toks = struct.pack("<IQ", g.T_STRING, 3) + _s(b"a") + _s(b"\xff\xfe") + _s(b"")
    merges = struct.pack("<IQ", g.T_STRING, 3) + _s(b"a b c") + _s(b"nospace") + _s(b"\xc4\xa0 t")
    f = _kv_file(tmp_path, [
        ("tokenizer.ggml.tokens", g.T_ARRAY, toks), ("tokenizer.ggml.merges", g.T_ARRAY, merges),
        ("tokenizer.ggml.bos_token_id", g.T_U32, struct.pack("<I", 151643)),
        ("tokenizer.ggml.eos_token_id", g.T_STRING, _s(b"x1")),
        ("tokenizer.ggml.add_bos_token", g.T_BOOL, b"\0"), ("tokenizer.ggml.add_eos_token", g.T_BOOL, b"\2"),
        ("tokenizer.ggml.pre", g.T_STRING, _s(b"qwen2")),
    ])
    t = f.tokenizer_data()
    assert t.tokens == [b"a", b"\xff\xfe", b""]             # raw bytes, not UTF-8 checked
    assert t.merges == [(b"a", b"b c"), ("Ġ".encode(), b"t")]
    assert (t.bos_token_id, t.eos_token_id, t.add_bos, t.add_eos, t.pre) == (151643, None, False, True, "qwen2")
    assert "tokenizer.ggml.tokens" not in f.metadata.raw and "tokenizer.ggml.merges" not in f.metadata.raw
    assert f.metadata.raw["tokenizer.ggml.bos_token_id"] == "151643"


def test_tokenizer_array_limit(tmp_path):
    with pytest.raises(g.StringTooLong):
        _kv_file(tmp_path, [("tokenizer.ggml.tokens", g.T_ARRAY, struct.pack("<IQ", g.T_STRING, 2_000_001))])


# ---- files: synthetic Q4_K_M model (loader_integration.rs on a seeded file) ----------------

@pytest.fixture(scope="module")
def model(tmp_path_factory):
    p = tmp_path_factory.mktemp("gguf") / "q4km.gguf"
    tensors = synth.write_q4_k_m_gguf(p, arch="qwen3", n_layers=8, hidden=256, ff=512, n_heads=2, n_kv_heads=1,
                                      vocab=512, seed=3)
    return p, tensors


def test_load_synthetic_model(model):
    p, tensors = model
    f = g.GgufFile.open(p)
    assert f.version == 3 and f.tensor_count() == len(tensors) > 0
    m = f.metadata
    assert m.architecture == "qwen3" and m.block_count() == 8
    assert (m.embedding_length(), m.feed_forward_length(), m.attention_head_count(), m.head_dim()) == (256, 512, 2, 128)
    assert m.attention_head_count_kv() == 1 and m.context_length() == 40960
    assert m.rope_freq_base(1e4) == 1e6 and m.rms_norm_eps(1e-5) == float(np.float32(1e-6))
    assert m.raw["general.file_type"] == "15" and m.raw["tokenizer.ggml.token_type"] == "array:512"
    t = f.tensor("token_embd.weight")
    assert t.element_count() == 256 * 512 and t.data.size == 512 * 144
    tok = f.tokenizer_data()
    assert len(tok.tokens) == 512 and tok.merges == [(b"t", b"0"), (b"t", b"1")] and tok.bos_token_id == 1


def test_tensor_iteration_and_bounds(model):
    p, tensors = model
    f = g.GgufFile.open(p)
    names = f.tensor_names()
    assert names == [t[0] for t in tensors] and len(names) == f.tensor_count()
    assert f.has_tensor("token_embd.weight") and not f.has_tensor("nonexistent_tensor")
    assert f.tensor("nonexistent_tensor") is None
    for name in names:
        assert f.tensor(name) is not None


def test_round_trip_byte_identical(model):
    p, tensors = model
    f = g.GgufFile.open(p)
    assert f.data_start % 32 == 0
    for name, t, dims, data in tensors:
        v = f.tensor(name)
        assert (v.ggml_type, v.dims) == (t, dims) and np.array_equal(v.data, data), name
        assert f.desc(name).offset % 32 == 0
        assert not v.data.flags.owndata                           # a view into the mapping


def test_data_section_alignment_ignores_general_alignment(tmp_path):
    # the data section starts at the next multiple of 32 whatever general.alignment says
    w = synth.q4_k_weights(2, 256, seed=1).reshape(-1)
    p = tmp_path / "a.gguf"
    g.write_gguf(p, [("general.alignment", g.T_U32, 64)], [("w", GgmlType.Q4_K, [512], w)])
    f = g.GgufFile.open(p)
    hdr_end = 24 + (8 + 17 + 4 + 4) + (8 + 1 + 4 + 8 + 4 + 8)
    assert hdr_end == 90 and f.data_start == 96                 # 64-byte alignment would give 128
    assert np.array_equal(f.tensor("w").data, w)


def test_truncated_file_out_of_bounds(model, tmp_path):
    p, tensors = model
    raw = p.read_bytes()
    f0 = g.GgufFile.open(p)
    last = tensors[-1][0]
    cut = f0.data_start + f0.desc(last).offset + f0.desc(last).byte_size() - 1
    q = tmp_path / "cut.gguf"
    q.write_bytes(raw[:cut])
    f = g.GgufFile.open(q)
    with pytest.raises(g.OutOfBounds, match=f"file_size={cut}"):
        f.tensor(last)
    assert np.array_equal(f.tensor(tensors[0][0]).data, tensors[0][3])
    q.write_bytes(raw[:40])                                     # inside the KV section
    with pytest.raises(g.LoadError):
        g.GgufFile.open(q)


def test_unknown_tensor_type_in_file(tmp_path):
    body = _hdr(3, 1, 0) + _s(b"w") + struct.pack("<I", 1) + struct.pack("<Q", 32) + struct.pack("<IQ", 9, 0)
    p = tmp_path / "u.gguf"
    p.write_bytes(body + b"\0" * 64)
    with pytest.raises(g.UnknownTensorType):
        g.GgufFile.open(p)


def test_writer_rejects_wrong_sizes(tmp_path):
    with pytest.raises(ValueError):
        g.write_gguf(tmp_path / "x.gguf", [], [("w", GgmlType.Q4_K, [256, 2], np.zeros(100, np.uint8))])


# ---- Q4_K_M tensor types ----------------------------------------------------------------------

def test_q4_k_m_q6_layers_qwen3_8b():
    # profiling/results/phase8_q4_k_m_analysis.md:97-103 (36-layer Qwen3-8B)
    want = [0, 1, 2, 3, 6, 9, 12, 15, 18, 21, 24, 27, 30, 31, 32, 33, 34, 35]
    assert [i for i in range(36) if g.q4_k_m_uses_q6_k(i, 36)] == want


def test_synthetic_model_tensor_types(model):
    _, tensors = model
    q6 = sorted(n for n, t, _, _ in tensors if t == GgmlType.Q6_K)
    want = sorted([f"blk.{i}.{w}.weight" for i in (0, 3, 6, 7) for w in ("attn_v", "ffn_down")] + ["output.weight"])
    assert q6 == want
    for name, t, dims, _ in tensors:
        if name.endswith("norm.weight"):
            assert t == GgmlType.F32 and len(dims) == 1
        elif t == GgmlType.Q4_K:
            g.build_matrix_meta(name, dims, t)


def test_golden_q4k_blocks_through_a_file(tmp_path):
    # real Qwen3-8B blk.0.ffn_gate.weight blocks written as a 3-block row,
    # read back and dequantized to the values of the reference's JSON
    blocks = json.loads(GOLDEN.read_text())["blocks"]
    raw = np.frombuffer(b"".join(bytes.fromhex(b["raw_hex"]) for b in blocks), np.uint8)
    p = tmp_path / "golden.gguf"
    g.write_gguf(p, [("general.architecture", g.T_STRING, "qwen3")], [("blk.0.ffn_gate.weight", GgmlType.Q4_K,
                                                                        [768, 1], raw)])
    v = g.GgufFile.open(p).tensor("blk.0.ffn_gate.weight")
    vals = O.q4k_dequant(np.ascontiguousarray(v.data), 3, f64=True).reshape(3, 256)
    for i, b in enumerate(blocks):
        np.testing.assert_allclose(vals[i, :64], b["dequantized_first_64"], rtol=0, atol=1e-15)
        np.testing.assert_allclose(vals[i, -8:], b["dequantized_last_8"], rtol=0, atol=1e-15)


def test_lm_head_tied_on_cpu_meta(tmp_path):
    # load_lm_head's role logic without a device: build the tied meta directly
    p = tmp_path / "tied.gguf"
    synth.write_q4_k_m_gguf(p, n_layers=1, hidden=256, ff=256, n_heads=2, n_kv_heads=1, vocab=256, tied=True)
    f = g.GgufFile.open(p)
    assert not f.has_tensor("output.weight")
    emb = f.tensor("token_embd.weight")
    m = g.build_matrix_meta("output.weight", emb.dims, emb.ggml_type, True, True)
    assert m.role == TensorRole.TIED_LM_HEAD and m.wtype == GgmlType.Q4_K


@pytest.mark.parametrize("arch,bias,qk_norm", [("qwen2", True, False), ("qwen3", False, True), ("llama", False, False)])
def test_optional_layer_tensors(tmp_path, arch, bias, qk_norm):
    # biases (attn_{q,k,v}.bias) and per-head norms (attn_{q,k}_norm.weight):
    # the optional tensors load_layer looks up (weights.rs:625-650, :753-770)
    p = tmp_path / f"{arch}.gguf"
    synth.write_q4_k_m_gguf(p, arch, 2, 256, 256, 2, 1, 256)
    f = g.GgufFile.open(p)
    hd = f.metadata.head_dim()
    for i in range(2):
        for t, n in (("q", 256), ("k", 128), ("v", 128)):
            v = f.tensor(f"blk.{i}.attn_{t}.bias")
            assert (v is not None) == bias and (v is None or (v.ggml_type, v.dims) == (GgmlType.F32, [n]))
        for t in ("q", "k"):
            v = f.tensor(f"blk.{i}.attn_{t}_norm.weight")
            assert (v is not None) == qk_norm and (v is None or v.dims == [hd])


def test_file_closes(model):
    p, tensors = model
    with g.GgufFile.open(p) as f:
        assert np.array_equal(f.tensor(tensors[0][0]).data, tensors[0][3])
    assert f._mm.closed
