"""GGUF v2/v3 reading (and writing, for seeded synthetic models) on the data
side of the matmul path: tensor descriptors, zero-copy tensor views, the
metadata the launchers' callers need, and the verbatim upload of a tensor's
bytes into its own device buffer.

Restates ROCmForge's loader (src/loader/):
  parse_header / parse_kv / parse_tensor_descs   parse.rs:28-47, :78-129, :288-321
  value conversion / skipping, read_string        parse.rs:133-260, :325-333
  GgmlType.from_u32 / bytes_for_elements          ggml_type.rs:25-66
  GgufFile.open / tensor / has_tensor / ...       file.rs:51-127
  GgufMetadata (arch-prefix resolution)           metadata.rs:18-145
  LoadError variants                              error.rs:5-24
and the matrix-metadata rules of src/gpu/weights.rs:
  supports_gpu_matrix_type / derive_tensor_role / build_matrix_meta   :355-413
  upload_tensor_bytes (verbatim copy into its own allocation)        :415-419

Like the reference, the tensor data section starts at the next 32-byte
boundary after the descriptors (parse.rs:16-17, :316-318; the general.alignment
key is not consulted), KV values other than the tokenizer arrays are kept as
strings formatted from their typed value, and arrays that are not tokenizer
arrays are kept as "array:<count>".
"""
from __future__ import annotations

import math
import mmap
import os
import re
import struct
from dataclasses import dataclass, field

import numpy as np

from .ops import GgmlType, InvalidWeightLayout, TensorRole, UnsupportedWeightType, WeightMeta

MAGIC = b"GGUF"
VERSION_MIN, VERSION_MAX = 2, 3
TENSOR_ALIGNMENT = 32

# ggml_type.rs:55-66 -- (elements per block, bytes per block)
_BLOCK = {
    GgmlType.F32: (1, 4), GgmlType.F16: (1, 2),
    GgmlType.Q4_0: (32, 18), GgmlType.Q4_1: (32, 20), GgmlType.Q5_0: (32, 22), GgmlType.Q5_1: (32, 24),
    GgmlType.Q8_0: (32, 34),
    GgmlType.Q2_K: (256, 256), GgmlType.Q3_K: (256, 110), GgmlType.Q4_K: (256, 144), GgmlType.Q5_K: (256, 176),
    GgmlType.Q6_K: (256, 210),
}

# GGUF KV value types
T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STRING, T_ARRAY, T_U64, T_I64, T_F64 = range(13)


# ---- errors (error.rs) --------------------------------------------------------

class LoadError(RuntimeError):
    pass


class InvalidMagic(LoadError):
    pass


class UnsupportedVersion(LoadError):
    pass


class UnknownTensorType(LoadError):
    pass


class OutOfBounds(LoadError):
    pass


class InvalidUtf8(LoadError):
    pass


class StringTooLong(LoadError):
    pass


# ---- ggml types ---------------------------------------------------------------

def ggml_type_from_u32(v: int) -> GgmlType:
    try:
        return GgmlType(v)
    except ValueError:
        raise UnknownTensorType(f"unknown tensor type: {v}") from None


def bytes_for_elements(t: GgmlType, n: int) -> int:
    per, nbytes = _BLOCK[GgmlType(t)]
    return -(-n // per) * nbytes


# ---- primitive reader ---------------------------------------------------------

class _Reader:
    def __init__(self, buf):
        self.buf, self.pos = buf, 0

    def take(self, n: int) -> bytes:
        if self.pos + n > len(self.buf):
            raise LoadError(f"I/O error: unexpected end of file at byte {self.pos}")
        b = bytes(self.buf[self.pos:self.pos + n])
        self.pos += n
        return b

    def u32(self) -> int:
        return struct.unpack("<I", self.take(4))[0]

    def u64(self) -> int:
        return struct.unpack("<Q", self.take(8))[0]

    def raw_string(self, limit: int = 100_000_000) -> bytes:
        n = self.u64()
        if n > limit:
            raise StringTooLong(f"string too long: {n} bytes")
        return self.take(n)

    def string(self) -> str:
        b = self.raw_string()
        try:
            return b.decode("utf-8")
        except UnicodeDecodeError:
            raise InvalidUtf8("invalid UTF-8 in string field") from None


_SCALAR = {T_U8: ("<B", 1), T_I8: ("<B", 1), T_BOOL: ("<B", 1), T_U16: ("<H", 2), T_I16: ("<H", 2),
           T_U32: ("<I", 4), T_I32: ("<I", 4), T_F32: ("<f", 4), T_U64: ("<Q", 8), T_I64: ("<Q", 8),
           T_F64: ("<d", 8)}


def _format_float(v, ftype) -> str:
    """Rust's Display for f32/f64: the shortest decimal that reads back to
    the same value, positional (no exponent), no trailing '.0'."""
    x = ftype(v)
    if np.isnan(x):
        return "NaN"
    if np.isinf(x):
        return "inf" if x > 0 else "-inf"
    return np.format_float_positional(x, unique=True, trim="-")


_USIZE = re.compile(r"\+?[0-9]+\Z")
_FLOAT = re.compile(r"[+-]?(inf|infinity|nan|([0-9]+\.?[0-9]*|\.[0-9]+)([eE][+-]?[0-9]+)?)\Z", re.I)


def parse_usize(s: str):
    """Rust's str::parse::<usize>: optional '+', decimal digits only."""
    if not _USIZE.match(s):
        return None
    v = int(s)
    return v if v < 1 << 64 else None


def parse_f32(s: str):
    """Rust's str::parse::<f32>, rounded to f32."""
    if not _FLOAT.match(s):
        return None
    return float(np.float32(float(s)))


def _skip_value(r: _Reader, t: int) -> None:
    """parse.rs:233-259 (unknown types skip 4 bytes)."""
    if t in _SCALAR:
        r.take(_SCALAR[t][1])
    elif t == T_STRING:
        r.raw_string()
    elif t == T_ARRAY:
        et, n = r.u32(), r.u64()
        for _ in range(n):
            _skip_value(r, et)
    else:
        r.take(4)


def _value_as_string(r: _Reader, t: int) -> str:
    """parse.rs:163-231: scalars read as unsigned (signed codes share the
    unsigned reader there), f32/f64 formatted, arrays as 'array:<n>'."""
    if t in _SCALAR:
        fmt, n = _SCALAR[t]
        v = struct.unpack(fmt, r.take(n))[0]
        if t == T_F32:
            return _format_float(v, np.float32)
        if t == T_F64:
            return _format_float(v, np.float64)
        return str(v)
    if t == T_STRING:
        return r.string()
    if t == T_ARRAY:
        et, n = r.u32(), r.u64()
        for _ in range(n):
            _skip_value(r, et)
        return f"array:{n}"
    r.take(4)
    return "unknown"


# ---- header / KV / tensor descriptors ------------------------------------------

@dataclass
class Header:
    version: int
    tensor_count: int
    kv_count: int


def parse_header(r: _Reader) -> Header:
    magic = r.take(4)
    if magic != MAGIC:
        raise InvalidMagic(f"invalid GGUF magic: {list(magic)}")
    version = r.u32()
    if version < VERSION_MIN or version > VERSION_MAX:
        raise UnsupportedVersion(f"unsupported GGUF version: {version}")
    return Header(version, r.u64(), r.u64())


@dataclass
class TokenizerData:
    tokens: list = field(default_factory=list)
    merges: list = field(default_factory=list)
    bos_token_id: int | None = None
    eos_token_id: int | None = None
    unk_token_id: int | None = None
    model: str | None = None
    pre: str | None = None
    add_bos: bool | None = None
    add_eos: bool | None = None


def _u32_or_none(s: str):
    v = parse_usize(s)
    return v if v is not None and v < 1 << 32 else None


def parse_kv(r: _Reader, kv_count: int):
    kv: dict[str, str] = {}
    tok = TokenizerData()
    for _ in range(kv_count):
        key = r.string()
        t = r.u32()
        if key in ("tokenizer.ggml.tokens", "tokenizer.ggml.vocab"):
            if t == T_ARRAY:
                r.u32()
                n = r.u64()
                if n > 2_000_000:
                    raise StringTooLong(f"string too long: {n} bytes")
                tok.tokens = [r.raw_string(10_000_000) for _ in range(n)]
            else:
                _skip_value(r, t)
            continue
        if key == "tokenizer.ggml.merges":
            if t == T_ARRAY:
                r.u32()
                n = r.u64()
                if n > 2_000_000:
                    raise StringTooLong(f"string too long: {n} bytes")
                merges = []
                for _ in range(n):
                    s = r.string()
                    if " " in s:
                        a, b = s.split(" ", 1)
                        merges.append((a.encode(), b.encode()))
                tok.merges = merges
            else:
                _skip_value(r, t)
            continue
        v = _value_as_string(r, t)
        if key == "tokenizer.ggml.model":
            tok.model = v
        elif key == "tokenizer.ggml.pre":
            tok.pre = v
        elif key == "tokenizer.ggml.bos_token_id":
            tok.bos_token_id = _u32_or_none(v)
        elif key == "tokenizer.ggml.eos_token_id":
            tok.eos_token_id = _u32_or_none(v)
        elif key == "tokenizer.ggml.unknown_token_id":
            tok.unk_token_id = _u32_or_none(v)
        elif key == "tokenizer.ggml.add_bos_token":
            tok.add_bos = v != "0"
        elif key == "tokenizer.ggml.add_eos_token":
            tok.add_eos = v != "0"
        kv[key] = v
    return GgufMetadata(kv), tok


@dataclass
class TensorDesc:
    name: str
    dims: list          # GGUF order, innermost first
    ggml_type: GgmlType
    offset: int         # relative to the data section

    def element_count(self) -> int:
        return math.prod(self.dims) if self.dims else 1

    def byte_size(self) -> int:
        return bytes_for_elements(self.ggml_type, self.element_count())


def parse_tensor_descs(r: _Reader, tensor_count: int):
    descs = []
    for _ in range(tensor_count):
        name = r.string()
        n_dims = r.u32()
        dims = [r.u64() for _ in range(n_dims)]
        t = ggml_type_from_u32(r.u32())
        descs.append(TensorDesc(name, dims, t, r.u64()))
    data_start = -(-r.pos // TENSOR_ALIGNMENT) * TENSOR_ALIGNMENT
    return descs, data_start


# ---- metadata (metadata.rs) -----------------------------------------------------

class GgufMetadata:
    def __init__(self, raw: dict):
        self.raw = raw
        self.architecture = raw.get("general.architecture", "unknown")

    def get(self, param: str):
        """<arch>.<param>, then llama.<param> (for other archs), then <param>."""
        v = self.raw.get(f"{self.architecture}.{param}")
        if v is not None:
            return v
        if self.architecture != "llama":
            v = self.raw.get(f"llama.{param}")
            if v is not None:
                return v
        return self.raw.get(param)

    def _resolve(self, keys, parse):
        for k in keys:
            v = self.get(k)
            x = None if v is None else parse(v)
            if x is not None and x > 0:
                return x
        return None

    def _usize(self, keys):
        return self._resolve(keys, parse_usize)

    def block_count(self) -> int:
        return self._usize(["block_count", "n_layers", "num_hidden_layers"]) or 0

    def embedding_length(self) -> int:
        return self._usize(["embedding_length", "hidden_size", "n_embd"]) or 0

    def feed_forward_length(self) -> int:
        return self._usize(["feed_forward_length", "intermediate_size", "ffn_dim"]) or 0

    def attention_head_count(self) -> int:
        return self._usize(["attention.head_count", "n_heads", "num_attention_heads"]) or 0

    def attention_head_count_kv(self):
        return self._usize(["attention.head_count_kv", "n_heads_kv", "num_key_value_heads"])

    def context_length(self) -> int:
        return self._usize(["context_length", "max_position_embeddings", "n_ctx"]) or 2048

    def vocab_size(self) -> int:
        return self._usize(["vocab_size"]) or 0

    def rms_norm_eps(self, default: float) -> float:
        v = self._resolve(["attention.layer_norm_rms_epsilon", "attention_norm_epsilon", "norm_eps",
                           "rms_norm_eps"], parse_f32)
        return default if v is None else v

    def rope_freq_base(self, default: float) -> float:
        v = self._resolve(["rope.freq_base", "rope_theta"], parse_f32)
        if v is None:
            w = parse_f32(self.raw.get("rope.freq_base", ""))
            v = w if w is not None and w > 0 else None
        return default if v is None else v

    def head_dim(self) -> int:
        for k in ("attention.key_length", "head_dim", "rope.dimension_count"):
            v = self._usize([k])
            if v is not None:
                return v
        hidden, heads = self.embedding_length(), self.attention_head_count()
        return hidden // heads if hidden > 0 and heads > 0 else 0


# ---- file (file.rs) -----------------------------------------------------------------

@dataclass
class TensorView:
    name: str
    dims: list
    ggml_type: GgmlType
    data: np.ndarray     # uint8 view into the file mapping (no copy)

    def element_count(self) -> int:
        return math.prod(self.dims) if self.dims else 1


class GgufFile:
    """Parses the header, KV section and tensor descriptors, then maps the
    file read-only; tensor data is exposed as zero-copy uint8 views."""

    def __init__(self, path):
        self.path = os.fspath(path)
        with open(self.path, "rb") as f:
            self._mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
        self._buf = np.frombuffer(self._mm, dtype=np.uint8)
        r = _Reader(self._mm)
        header = parse_header(r)
        self.version = header.version
        self.metadata, self._tokenizer = parse_kv(r, header.kv_count)
        descs, self.data_start = parse_tensor_descs(r, header.tensor_count)
        self._order = [d.name for d in descs]
        self._descs = {d.name: d for d in descs}

    @classmethod
    def open(cls, path) -> "GgufFile":
        return cls(path)

    def tensor_names(self):
        return list(self._order)

    def tensor_count(self) -> int:
        return len(self._descs)

    def has_tensor(self, name: str) -> bool:
        return name in self._descs

    def desc(self, name: str) -> TensorDesc | None:
        return self._descs.get(name)

    def tensor(self, name: str) -> TensorView | None:
        """None if absent; OutOfBounds if its bytes run past the file."""
        d = self._descs.get(name)
        if d is None:
            return None
        start = self.data_start + d.offset
        size = d.byte_size()
        if start + size > len(self._buf):
            raise OutOfBounds(f"slice out of bounds: offset={start} size={size} file_size={len(self._buf)}")
        return TensorView(d.name, d.dims, d.ggml_type, self._buf[start:start + size])

    def tokenizer_data(self) -> TokenizerData:
        return self._tokenizer

    def close(self) -> None:
        """Unmaps the file.  Tensor views still referenced keep the mapping
        exported, and then mmap refuses (BufferError)."""
        self._buf = None
        self._mm.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


# ---- matrix metadata and upload (weights.rs) --------------------------------------

_GPU_MATRIX_TYPES = {GgmlType.F32, GgmlType.Q4_0, GgmlType.Q4_1, GgmlType.Q4_K, GgmlType.Q5_K, GgmlType.Q6_K,
                     GgmlType.Q8_0}


def supports_gpu_matrix_type(t: GgmlType) -> bool:
    return GgmlType(t) in _GPU_MATRIX_TYPES


def derive_tensor_role(is_lm_head: bool, is_tied: bool) -> TensorRole:
    if not is_lm_head:
        return TensorRole.GENERIC
    return TensorRole.TIED_LM_HEAD if is_tied else TensorRole.LM_HEAD


def build_matrix_meta(name: str, dims, wtype: GgmlType, is_lm_head: bool = False,
                      is_tied: bool = False) -> WeightMeta:
    """weights.rs:379-413 without the transpose flag (the kernels here read
    the GGUF layout as stored: row n = output n, K/256 blocks per row)."""
    dims = list(dims)
    if len(dims) < 2:
        raise InvalidWeightLayout(f"{name}: matrix weights must have at least 2 dimensions (dims {dims})")
    if not supports_gpu_matrix_type(wtype):
        raise UnsupportedWeightType(f"{name}: {GgmlType(wtype).name}")
    return WeightMeta(GgmlType(wtype), dims, derive_tensor_role(is_lm_head, is_tied))


def upload_tensor(view: TensorView, device="cuda:0"):
    """The tensor's bytes, verbatim, in a device allocation of their own
    (upload_tensor_bytes); torch's allocations are 256-byte aligned, which
    covers the 16-byte buffer loads of the Q4_K kernels."""
    import warnings

    import torch
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")      # read-only mapping; only read by the copy
        host = torch.from_numpy(view.data)
    return host.to(device)


def load_matrix(f: GgufFile, name: str, device="cuda:0", is_lm_head=False, is_tied=False):
    """(device bytes, WeightMeta) of one matrix -- weights.rs:835-851."""
    v = f.tensor(name)
    if v is None:
        raise LoadError(f"tensor not found: {name}")
    meta = build_matrix_meta(name, v.dims, v.ggml_type, is_lm_head, is_tied)
    return upload_tensor(v, device), meta


def load_lm_head(f: GgufFile, device="cuda:0", lm_head_name="output.weight",
                 token_emb_name="token_embd.weight"):
    """The LM head if the file has one, else the token embeddings marked as a
    tied head (weights.rs:868-887).  Returns (device bytes, meta, tied)."""
    if f.has_tensor(lm_head_name):
        buf, meta = load_matrix(f, lm_head_name, device, True, False)
        return buf, meta, False
    buf, emb = load_matrix(f, token_emb_name, device)
    return buf, build_matrix_meta(lm_head_name, emb.dims, emb.wtype, True, True), True


def load_f32(f: GgufFile, name: str, device="cuda:0", optional=False):
    """A norm / bias vector's bytes on the device (weights.rs load_f32 and
    load_f32_opt): None for an absent optional tensor."""
    v = f.tensor(name)
    if v is None:
        if optional:
            return None
        raise LoadError(f"tensor not found: {name}")
    if v.ggml_type != GgmlType.F32:
        raise UnsupportedWeightType(f"{name}: {GgmlType(v.ggml_type).name} (F32 expected)")
    return upload_tensor(v, device)


# GGUF tensor names of one decoder layer (src/config.rs:141-183)
LAYER_MATRICES = ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down")


@dataclass
class LayerWeights:
    """One layer's device buffers and matrix metadata (GpuLayerWeights,
    weights.rs:515-551): each entry of `matrices` is (bytes, WeightMeta);
    biases and the per-head Q/K norms are None where the file has none."""
    attn_norm: object
    ffn_norm: object
    matrices: dict
    bias: dict
    attn_q_norm: object = None
    attn_k_norm: object = None

    def __getitem__(self, key):
        return self.matrices[key]


def load_layer(f: GgufFile, layer: int, device="cuda:0") -> LayerWeights:
    """weights.rs:558-797 for the GGUF naming scheme (dense models)."""
    p = f"blk.{layer}."
    mats = {m: load_matrix(f, f"{p}{m}.weight", device) for m in LAYER_MATRICES}
    bias = {m: load_f32(f, f"{p}{m}.bias", device, optional=True) for m in ("attn_q", "attn_k", "attn_v")}
    return LayerWeights(load_f32(f, f"{p}attn_norm.weight", device), load_f32(f, f"{p}ffn_norm.weight", device),
                        mats, bias, load_f32(f, f"{p}attn_q_norm.weight", device, optional=True),
                        load_f32(f, f"{p}attn_k_norm.weight", device, optional=True))


@dataclass
class ModelWeights:
    """GpuModelWeights (weights.rs:830-945): embeddings, output norm, LM head
    (explicit or tied) and the layers."""
    token_emb: tuple
    output_norm: object
    lm_head: tuple
    lm_head_tied: bool
    layers: list


def load_model(f: GgufFile, device="cuda:0") -> ModelWeights:
    emb = load_matrix(f, "token_embd.weight", device)
    norm = load_f32(f, "output_norm.weight", device)
    buf, meta, tied = load_lm_head(f, device)
    layers = [load_layer(f, i, device) for i in range(f.metadata.block_count())]
    return ModelWeights(emb, norm, (buf, meta), tied, layers)


# ---- Q4_K_M tensor types ------------------------------------------------------------

def q4_k_m_uses_q6_k(layer: int, n_layers: int) -> bool:
    """Which layers a Q4_K_M file keeps attn_v / ffn_down in Q6_K: the first
    and last eighth of the stack and every third layer in between (llama.cpp's
    Q4_K_M rule).  For Qwen3-8B (36 layers) this is the set the reference
    lists in profiling/results/phase8_q4_k_m_analysis.md:97-103."""
    lo, hi = n_layers // 8, 7 * n_layers // 8
    return layer < lo or layer >= hi or (layer - lo) % 3 == 2


# ---- writer (no reference counterpart: builds seeded synthetic files) ------------------

def _w_string(out: list, s: str | bytes) -> None:
    b = s.encode() if isinstance(s, str) else s
    out.append(struct.pack("<Q", len(b)))
    out.append(b)


def _w_value(out: list, t: int, v) -> None:
    if t in _SCALAR:
        fmt = _SCALAR[t][0]
        if t in (T_I8, T_I16, T_I32, T_I64):
            fmt = fmt.lower()
        out.append(struct.pack(fmt, v))
    elif t == T_STRING:
        _w_string(out, v)
    elif t == T_ARRAY:
        et, items = v
        out.append(struct.pack("<IQ", et, len(items)))
        for it in items:
            _w_value(out, et, it)
    else:
        raise ValueError(f"unsupported KV type {t}")


def write_gguf(path, kv, tensors, version: int = 3) -> None:
    """kv: list of (key, value type, value) -- arrays as (element type,
    items); tensors: list of (name, GgmlType, dims innermost first, bytes).
    Tensor data is laid out at 32-byte aligned offsets after the 32-byte
    aligned end of the descriptors."""
    head = [MAGIC, struct.pack("<IQQ", version, len(tensors), len(kv))]
    for key, t, v in kv:
        _w_string(head, key)
        head.append(struct.pack("<I", t))
        _w_value(head, t, v)
    offsets, off = [], 0
    for name, t, dims, data in tensors:
        if len(data) != bytes_for_elements(t, math.prod(dims)):
            raise ValueError(f"{name}: {len(data)} bytes for dims {dims} of {GgmlType(t).name}")
        offsets.append(off)
        off += -(-len(data) // TENSOR_ALIGNMENT) * TENSOR_ALIGNMENT
    for (name, t, dims, _), o in zip(tensors, offsets):
        _w_string(head, name)
        head.append(struct.pack("<I", len(dims)))
        head.extend(struct.pack("<Q", d) for d in dims)
        head.append(struct.pack("<IQ", int(t), o))
    blob = b"".join(head)
    pad = -(-len(blob) // TENSOR_ALIGNMENT) * TENSOR_ALIGNMENT - len(blob)
    with open(path, "wb") as f:
        f.write(blob + b"\0" * pad)
        for (_, _, _, data), o in zip(tensors, offsets):
            f.write(bytes(data))
            f.write(b"\0" * (-(-len(data) // TENSOR_ALIGNMENT) * TENSOR_ALIGNMENT - len(data)))


def _main(argv=None) -> int:
    """Times open (header/KV/descriptor parse + mapping) and the verbatim
    upload of every matrix of a seeded Qwen3-8B-shaped Q4_K_M file with the
    given number of layers; prints one JSON line."""
    import argparse
    import json
    import tempfile
    import time

    ap = argparse.ArgumentParser()
    ap.add_argument("--layers", type=int, default=2)
    ap.add_argument("--dir", default=None)
    a = ap.parse_args(argv)
    import torch

    from . import synth
    with tempfile.TemporaryDirectory(dir=a.dir) as d:
        path = os.path.join(d, "q4km.gguf")
        t0 = time.perf_counter()
        tensors = synth.write_q4_k_m_gguf(path, "qwen3", a.layers, 4096, 12288, 32, 8, 151936, seed=1)
        t_write = time.perf_counter() - t0
        t0 = time.perf_counter()
        f = GgufFile.open(path)
        t_open = time.perf_counter() - t0
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        bufs = [upload_tensor(f.tensor(n)) for n, _, _, _ in tensors]
        torch.cuda.synchronize()
        t_up = time.perf_counter() - t0
        nbytes = sum(b.numel() for b in bufs)
        ok = all(np.array_equal(b.cpu().numpy(), f.tensor(n).data) for b, (n, _, _, _) in zip(bufs, tensors))
        print(json.dumps({"file_bytes": os.path.getsize(path), "tensors": len(tensors), "layers": a.layers,
                          "write_s": round(t_write, 3), "open_ms": round(t_open * 1e3, 3),
                          "upload_s": round(t_up, 4), "upload_GBps": round(nbytes / t_up / 1e9, 2),
                          "bytes_identical": ok}), flush=True)
        return 0 if ok else 1


if __name__ == "__main__":
    raise SystemExit(_main())
