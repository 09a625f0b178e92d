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

def torch_weights(fmt: str, n: int, k: int, seed: int, device="cuda"):
    """Same distributions, generated in device memory (uint8 [n, row_bytes])."""
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
    else:
        sc = torch.randint(-32, 32, (nb, 16), dtype=torch.int8, device=device, generator=g)
        blk[:, 192:208] = sc.view(torch.uint8)
        blk[:, 208:210] = f16(nb)
    return blk.view(n, -1)
