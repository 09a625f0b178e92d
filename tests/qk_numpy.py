"""Independent numpy decoders of the GGUF Q4_K / Q6_K layouts, written from
the ggml loop structure (ggml dequantize_row_q4_K / dequantize_row_q6_K as
documented in docs/q4_k_m_block_format.md and docs/q6_k_block_format.md of
the reference) rather than from the C oracle.  Tests use them to pin the
oracle: the two restatements share no code."""
import numpy as np


def f16(b):
    return np.frombuffer(np.ascontiguousarray(b).tobytes(), np.float16).astype(np.float64)


def q4k_fields(w: np.ndarray):
    """w: uint8 [..., 144] -> d, dmin (float64), sc[8], m[8] (int), nibbles[256]."""
    blk = w.reshape(-1, 144)
    d = f16(blk[:, 0:2])
    dmin = f16(blk[:, 2:4])
    q = blk[:, 4:16].astype(np.int64)
    sc = np.zeros((blk.shape[0], 8), np.int64)
    m = np.zeros((blk.shape[0], 8), np.int64)
    sc[:, 0:4] = q[:, 0:4] & 63
    m[:, 0:4] = q[:, 4:8] & 63
    sc[:, 4:8] = (q[:, 8:12] & 0xF) | ((q[:, 0:4] >> 6) << 4)
    m[:, 4:8] = (q[:, 8:12] >> 4) | ((q[:, 4:8] >> 6) << 4)
    qs = blk[:, 16:144].reshape(-1, 4, 32).astype(np.int64)
    nib = np.empty((blk.shape[0], 4, 2, 32), np.int64)
    nib[:, :, 0, :] = qs & 0xF       # element 64*k + l
    nib[:, :, 1, :] = qs >> 4        # element 64*k + 32 + l
    return d, dmin, sc, m, nib.reshape(-1, 256)


def q4k_dequant(w: np.ndarray) -> np.ndarray:
    d, dmin, sc, m, nib = q4k_fields(w)
    scale = np.repeat(d[:, None] * sc, 32, axis=1)
    mn = np.repeat(dmin[:, None] * m, 32, axis=1)
    return (scale * nib - mn).reshape(-1)


def q6k_dequant(w: np.ndarray) -> np.ndarray:
    blk = w.reshape(-1, 210)
    out = np.empty((blk.shape[0], 256), np.float64)
    d = f16(blk[:, 208:210])
    sc = blk[:, 192:208].view(np.int8).astype(np.int64)
    for n in range(2):                      # y += 128, ql += 64, qh += 32, sc += 8
        ql = blk[:, 64 * n: 64 * n + 64].astype(np.int64)
        qh = blk[:, 128 + 32 * n: 128 + 32 * n + 32].astype(np.int64)
        l = np.arange(32)
        isx = l // 16
        q1 = ((ql[:, l] & 0xF) | (((qh[:, l] >> 0) & 3) << 4)) - 32
        q2 = ((ql[:, l + 32] & 0xF) | (((qh[:, l] >> 2) & 3) << 4)) - 32
        q3 = ((ql[:, l] >> 4) | (((qh[:, l] >> 4) & 3) << 4)) - 32
        q4 = ((ql[:, l + 32] >> 4) | (((qh[:, l] >> 6) & 3) << 4)) - 32
        s = sc[:, 8 * n:8 * n + 8]
        out[:, 128 * n + l] = d[:, None] * s[:, isx + 0] * q1
        out[:, 128 * n + l + 32] = d[:, None] * s[:, isx + 2] * q2
        out[:, 128 * n + l + 64] = d[:, None] * s[:, isx + 4] * q3
        out[:, 128 * n + l + 96] = d[:, None] * s[:, isx + 6] * q4
    return out.reshape(-1)


def q8_0_quantize(x: np.ndarray):
    """numpy float32/float16 semantics of the Q8_0 inline quantiser."""
    xb = x.astype(np.float32).reshape(-1, 32)
    amax = np.max(np.abs(xb), axis=1)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        scale = np.maximum(amax / np.float32(127.0), np.float32(1e-30)).astype(np.float32)
        dh = scale.astype(np.float16)
        sf = dh.astype(np.float32)
        inv = (np.float32(1.0) / sf).astype(np.float32)
        prod = (xb * inv[:, None]).astype(np.float32)
        # np.fmax/fmin return the non-NaN operand, like C fmaxf/fminf
        qf = np.fmin(np.fmax(prod, np.float32(-127.0)), np.float32(127.0))
    q = np.trunc(qf).astype(np.int8)
    return dh.view(np.uint16), q.reshape(-1)
