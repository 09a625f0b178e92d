"""Seeded synthetic GGUF Q4_K / Q6_K weights and activations.

Value distributions follow the benchmark configuration of the reference
hot path: Q4_K d, dmin = fp16(|N(0,1)| * 1e-3), 12 scale bytes and 128
nibble bytes uniform; Q6_K ql/qh uniform bytes, int8 sub-scales uniform in
[-32, 31], d = fp16(|N(0,1)| * 1e-3); activations fp32 N(0,1).

Two generators with the same distributions: numpy (host bytes, used by
tests and fixtures) and torch (generated directly in device memory, used by
the benchmark for multi-GB weight sets).
"""
from __future__ import annotations

import numpy as np

QK_K = 256
Q4K_BYTES = 144
Q6K_BYTES = 210
BLOCK_BYTES = {"q4_k": Q4K_BYTES, "q6_k": Q6K_BYTES}


def row_bytes(fmt: str, k: int) -> int:
    assert k % QK_K == 0
    return (k // QK_K) * BLOCK_BYTES[fmt]


def _fp16_bytes(vals: np.ndarray) -> np.ndarray:
    return vals.astype(np.float16).view(np.uint8).reshape(-1, 2)


def q4_k_weights(n: int, k: int, seed: int = 0) -> np.ndarray:
    """uint8 array [n, (k/256)*144] of random Q4_K super-blocks."""
    rng = np.random.default_rng(seed)
    nb = n * (k // QK_K)
    blk = rng.integers(0, 256, size=(nb, Q4K_BYTES), dtype=np.uint8)
    blk[:, 0:2] = _fp16_bytes(np.abs(rng.standard_normal(nb)) * 1e-3)
    blk[:, 2:4] = _fp16_bytes(np.abs(rng.standard_normal(nb)) * 1e-3)
    return blk.reshape(n, -1)


def q6_k_weights(n: int, k: int, seed: int = 0) -> np.ndarray:
    """uint8 array [n, (k/256)*210] of random Q6_K super-blocks."""
    rng = np.random.default_rng(seed)
    nb = n * (k // QK_K)
    blk = rng.integers(0, 256, size=(nb, Q6K_BYTES), dtype=np.uint8)
    blk[:, 192:208] = rng.integers(-32, 32, size=(nb, 16), dtype=np.int8).view(np.uint8)
    blk[:, 208:210] = _fp16_bytes(np.abs(rng.standard_normal(nb)) * 1e-3)
    return blk.reshape(n, -1)


def activations(k: int, seed: int = 0, m: int | None = None) -> np.ndarray:
    rng = np.random.default_rng(seed)
    shape = (k,) if m is None else (m, k)
    return rng.standard_normal(shape).astype(np.float32)


def weights(fmt: str, n: int, k: int, seed: int = 0) -> np.ndarray:
    return q4_k_weights(n, k, seed) if fmt == "q4_k" else q6_k_weights(n, k, seed)


# ---- device-side generator (torch) -----------------------------------------

def torch_weights(fmt: str, n: int, k: int, seed: int, device="cuda", signed: bool = False):
    """Same distributions, generated in device memory (uint8 [n, row_bytes]).

    signed: negate half the Q4_K super-blocks at random (the sign bit of both
    d and dmin, so w -> -w block by block).  The plain distribution has a
    positive mean per weight (d sc q - dmin m with q, sc, m uniform), which a
    deep stack of such matrices amplifies until the hidden state is one
    common-mode vector; signed blocks have mean zero across a row."""
    import torch

    g = torch.Generator(device=device)
    g.manual_seed(seed)
    bb = BLOCK_BYTES[fmt]
    nb = n * (k // QK_K)
    blk = torch.randint(0, 256, (nb, bb), dtype=torch.uint8, device=device, generator=g)

    def f16(count):
        v = torch.randn(count, device=device, generator=g).abs_().mul_(1e-3).to(torch.float16)
        return v.view(torch.uint8).view(count, 2)

    if fmt == "q4_k":
        blk[:, 0:2] = f16(nb)
        blk[:, 2:4] = f16(nb)
        if signed:
            neg = torch.randint(0, 2, (nb,), dtype=torch.uint8, device=device, generator=g) * 0x80
            blk[:, 1] |= neg
            blk[:, 3] |= neg
    else:
        sc = torch.randint(-32, 32, (nb, 16), dtype=torch.int8, device=device, generator=g)
        blk[:, 192:208] = sc.view(torch.uint8)
        blk[:, 208:210] = f16(nb)
    return blk.view(n, -1)


def q4_k_m_model_tensors(n_layers: int, hidden: int, ff: int, n_heads: int, n_kv_heads: int, vocab: int,
                         head_dim: int | None = None, seed: int = 0, tied: bool = False, qkv_bias: bool = False,
                         qk_norm: bool = False):
    """Seeded random tensors of a llama/qwen-style model in a Q4_K_M file's
    types: Q4_K matrices, Q6_K for attn_v / ffn_down on the layers the
    Q4_K_M rule picks and for output.weight, F32 norms (and, on request, F32
    Q/K/V biases as qwen2 files carry and per-head Q/K norms as qwen3 files
    carry).  Returns a list of
    (name, GgmlType, GGUF dims innermost first, uint8 bytes)."""
    from .gguf import q4_k_m_uses_q6_k
    from .ops import GgmlType

    hd = head_dim or hidden // n_heads
    q_dim, kv_dim = n_heads * hd, n_kv_heads * hd
    out = []
    s = [seed * 1009]

    def mat(name, k, n, q6=False):
        s[0] += 1
        w = q6_k_weights(n, k, s[0]) if q6 else q4_k_weights(n, k, s[0])
        out.append((name, GgmlType.Q6_K if q6 else GgmlType.Q4_K, [k, n], w.reshape(-1)))

    def norm(name, n, centre=1.0):
        s[0] += 1
        v = (centre + 0.1 * np.random.default_rng(s[0]).standard_normal(n)).astype(np.float32)
        out.append((name, GgmlType.F32, [n], v.view(np.uint8)))

    mat("token_embd.weight", hidden, vocab)
    for i in range(n_layers):
        q6 = q4_k_m_uses_q6_k(i, n_layers)
        norm(f"blk.{i}.attn_norm.weight", hidden)
        mat(f"blk.{i}.attn_q.weight", hidden, q_dim)
        mat(f"blk.{i}.attn_k.weight", hidden, kv_dim)
        mat(f"blk.{i}.attn_v.weight", hidden, kv_dim, q6)
        if qkv_bias:
            for t, n in (("q", q_dim), ("k", kv_dim), ("v", kv_dim)):
                norm(f"blk.{i}.attn_{t}.bias", n, 0.0)
        if qk_norm:
            norm(f"blk.{i}.attn_q_norm.weight", hd)
            norm(f"blk.{i}.attn_k_norm.weight", hd)
        mat(f"blk.{i}.attn_output.weight", q_dim, hidden)
        norm(f"blk.{i}.ffn_norm.weight", hidden)
        mat(f"blk.{i}.ffn_gate.weight", hidden, ff)
        mat(f"blk.{i}.ffn_up.weight", hidden, ff)
        mat(f"blk.{i}.ffn_down.weight", ff, hidden, q6)
    norm("output_norm.weight", hidden)
    if not tied:
        mat("output.weight", hidden, vocab, True)
    return out


def write_q4_k_m_gguf(path, arch: str = "qwen3", n_layers: int = 4, hidden: int = 1024, ff: int = 3072,
                      n_heads: int = 8, n_kv_heads: int = 2, vocab: int = 2048, seed: int = 0,
                      tied: bool = False, qkv_bias: bool | None = None, qk_norm: bool | None = None):
    """Writes a synthetic Q4_K_M GGUF (v3) with the metadata keys a loader
    resolves and a small tokenizer; returns the tensor list written.  By
    default qwen2 files get Q/K/V biases and qwen3 files per-head Q/K norms."""
    from . import gguf as g

    qkv_bias = arch == "qwen2" if qkv_bias is None else qkv_bias
    qk_norm = arch == "qwen3" if qk_norm is None else qk_norm
    tensors = q4_k_m_model_tensors(n_layers, hidden, ff, n_heads, n_kv_heads, vocab, seed=seed, tied=tied,
                                   qkv_bias=qkv_bias, qk_norm=qk_norm)
    tokens = [f"t{i}".encode() for i in range(vocab)]
    kv = [
        ("general.architecture", g.T_STRING, arch),
        ("general.file_type", g.T_U32, 15),                      # MOSTLY_Q4_K_M
        (f"{arch}.block_count", g.T_U32, n_layers),
        (f"{arch}.embedding_length", g.T_U32, hidden),
        (f"{arch}.feed_forward_length", g.T_U32, ff),
        (f"{arch}.attention.head_count", g.T_U32, n_heads),
        (f"{arch}.attention.head_count_kv", g.T_U32, n_kv_heads),
        (f"{arch}.context_length", g.T_U64, 40960),
        (f"{arch}.attention.layer_norm_rms_epsilon", g.T_F32, 1e-6),
        (f"{arch}.rope.freq_base", g.T_F32, 1000000.0),
        ("tokenizer.ggml.model", g.T_STRING, "gpt2"),
        ("tokenizer.ggml.tokens", g.T_ARRAY, (g.T_STRING, tokens)),
        ("tokenizer.ggml.merges", g.T_ARRAY, (g.T_STRING, ["t 0", "t 1", "nospace"])),
        ("tokenizer.ggml.token_type", g.T_ARRAY, (g.T_I32, [1] * vocab)),
        ("tokenizer.ggml.bos_token_id", g.T_U32, 1),
        ("tokenizer.ggml.eos_token_id", g.T_U32, 2),
        ("tokenizer.ggml.add_bos_token", g.T_BOOL, 0),
    ]
    g.write_gguf(path, kv, tensors)
    return tensors
