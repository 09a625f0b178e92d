"""ctypes front-end of the C oracle (qk_oracle.c) and the CPU timing port
(cpu_baseline.c).  TEST INFRASTRUCTURE ONLY: imported by tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg, never by the
product path.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"
REF_LIB = HERE / "_ref" / "libref_gemv.so"
REF_OPS_LIB = HERE / "_ref" / "libref_ops.so"

_p = ctypes.c_void_p
_i = ctypes.c_int
_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = ctypes.CDLL(str(LIB))
        L.or_f32_to_f16.argtypes = [ctypes.c_float]
        L.or_f32_to_f16.restype = ctypes.c_uint16
        L.or_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.or_f16_to_f32.restype = ctypes.c_float
        for name, args in {
            "or_q8_0_quantize": [_p, _i, _p, _p],
            "or_q4k_scale_min": [_i, _p, _p, _p],
            "or_q4k_dequant_row_f64": [_p, _i, _p],
            "or_q4k_dequant_row_f32": [_p, _i, _p],
            "or_q6k_dequant_row_f32": [_p, _i, _p],
            "or_q4k_q8_partials": [_p, _p, _i, _i, _p, _p],
            "or_gemv_q4k_q8": [_p, _p, _i, _i, _p],
            "or_gemv_q4k_f32": [_p, _p, _i, _i, _p],
            "or_gemv_q6k": [_p, _p, _i, _i, _p],
            "or_swiglu": [_p, _p, _i, _p],
            "or_round_f16": [_p, ctypes.c_size_t, _p],
            "or_q4k_dequant_f16": [_p, _i, _i, _p],
            "or_q6k_dequant_f16": [_p, _i, _i, _p],
            "or_rms_norm": [_p, _p, _i, _i, ctypes.c_float, _p],
            "or_rope": [_p, _i, _i, _i, _i, ctypes.c_float, _i, _p],
            "or_attn_decode": [_p, _p, _p, _i, _i, _i, _i, ctypes.c_float, _p],
            "or_attn_prefill_f16": [_p, _p, _p, _i, _i, _i, _i, ctypes.c_float, _p],
            "or_silu_mul": [_p, _p, _i, _p],
            "cb_gemv_q4k_q8k": [_p, _p, _p, _i, _i, _i],
            "cb_gemm_q4k_q8k": [_p, _p, _p, _i, _i, _i, _i],
            "cb_gemv_q6k": [_p, _p, _p, _i, _i, _i],
            "cb_gemm_q6k": [_p, _p, _p, _i, _i, _i, _i],
            "cb_gate_up_swiglu": [_p, _p, _p, _p, _p, _i, _i, _i],
        }.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = None
        L.cb_max_threads.restype = _i
        L.or_rope_theta.argtypes = [_i, _i, ctypes.c_float, _p]
        L.or_rope_theta.restype = ctypes.c_float
        L.or_argmax.argtypes = [_p, _i]
        L.or_argmax.restype = _i
        _lib = L
    return _lib


def _ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def f32_to_f16_bits(x: float) -> int:
    return int(lib().or_f32_to_f16(float(x)))


def f16_bits_to_f32(h: int) -> float:
    return float(lib().or_f16_to_f32(int(h)))


def q8_0_quantize(x: np.ndarray):
    x = np.ascontiguousarray(x, dtype=np.float32)
    d = np.empty(x.size // 32, np.uint16)
    q = np.empty(x.size, np.int8)
    lib().or_q8_0_quantize(_ptr(x), x.size, _ptr(d), _ptr(q))
    return d, q


def q4k_scale_min(j: int, scales: bytes):
    s = np.frombuffer(bytes(scales), np.uint8).copy()
    sc, m = ctypes.c_int(), ctypes.c_int()
    lib().or_q4k_scale_min(j, _ptr(s), ctypes.byref(sc), ctypes.byref(m))
    return sc.value, m.value


def q4k_dequant(w: np.ndarray, n_blocks: int, f64: bool = True) -> np.ndarray:
    w = np.ascontiguousarray(w, np.uint8)
    out = np.empty(n_blocks * 256, np.float64 if f64 else np.float32)
    (lib().or_q4k_dequant_row_f64 if f64 else lib().or_q4k_dequant_row_f32)(_ptr(w), n_blocks, _ptr(out))
    return out


def q6k_dequant(w: np.ndarray, n_blocks: int) -> np.ndarray:
    w = np.ascontiguousarray(w, np.uint8)
    out = np.empty(n_blocks * 256, np.float32)
    lib().or_q6k_dequant_row_f32(_ptr(w), n_blocks, _ptr(out))
    return out


def q4k_q8_partials(w: np.ndarray, xq: np.ndarray, k: int, n: int):
    w = np.ascontiguousarray(w, np.uint8)
    xq = np.ascontiguousarray(xq, np.int8)
    dots = np.empty(n * (k // 32), np.int32)
    sums = np.empty(k // 32, np.int32)
    lib().or_q4k_q8_partials(_ptr(w), _ptr(xq), k, n, _ptr(dots), _ptr(sums))
    return dots.reshape(n, k // 32), sums


def _gemv(fn, w, x, k, n):
    w = np.ascontiguousarray(w, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(n, np.float64)
    fn(_ptr(w), _ptr(x), k, n, _ptr(y))
    return y


def gemv_q4k_q8(w, x, k, n):
    return _gemv(lib().or_gemv_q4k_q8, w, x, k, n)


def gemv_q4k_f32(w, x, k, n):
    return _gemv(lib().or_gemv_q4k_f32, w, x, k, n)


def gemv_q6k(w, x, k, n):
    return _gemv(lib().or_gemv_q6k, w, x, k, n)


def swiglu(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    g = np.ascontiguousarray(g, np.float64)
    u = np.ascontiguousarray(u, np.float64)
    out = np.empty_like(g)
    lib().or_swiglu(_ptr(g), _ptr(u), g.size, _ptr(out))
    return out


def round_f16(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32)
    out = np.empty_like(a)
    lib().or_round_f16(_ptr(a), a.size, _ptr(out))
    return out


def dequant_f16(fmt: str, w: np.ndarray, n: int, k: int) -> np.ndarray:
    """fp16-rounded dequantised weights [n, k] (as float32)."""
    w = np.ascontiguousarray(w, np.uint8)
    out = np.empty((n, k), np.float32)
    fn = lib().or_q4k_dequant_f16 if fmt == "q4_k" else lib().or_q6k_dequant_f16
    fn(_ptr(w), n, k, _ptr(out))
    return out


def gemm(fmt: str, a: np.ndarray, w: np.ndarray, m: int, n: int, k: int) -> np.ndarray:
    """float64 D = fp16(A) @ fp16(dequant W)^T  (the reference GEMM's operands)."""
    af = round_f16(a).astype(np.float64).reshape(m, k)
    wf = dequant_f16(fmt, w, n, k).astype(np.float64)
    return af @ wf.T


def gemm_abs(fmt: str, a: np.ndarray, w: np.ndarray, m: int, n: int, k: int) -> np.ndarray:
    """|fp16(A)| @ |fp16(dequant W)|^T: per output, the sum of the magnitudes
    of the products it adds up -- the scale of its fp32 accumulation error."""
    af = np.abs(round_f16(a).astype(np.float32).reshape(m, k))
    wf = np.abs(dequant_f16(fmt, w, n, k))
    return af.astype(np.float64) @ wf.T.astype(np.float64)


# ---- CPU timing port ---------------------------------------------------------

def cpu_gemv_q4k(w, x, n, k, threads):
    y = np.empty(n, np.float32)
    lib().cb_gemv_q4k_q8k(_ptr(w), _ptr(x), _ptr(y), n, k, threads)
    return y


def cpu_gemv_q6k(w, x, n, k, threads):
    y = np.empty(n, np.float32)
    lib().cb_gemv_q6k(_ptr(w), _ptr(x), _ptr(y), n, k, threads)
    return y


def cpu_gate_up(wg, wu, x, n, k, threads):
    g = np.empty(n, np.float32)
    out = np.empty(n, np.float32)
    lib().cb_gate_up_swiglu(_ptr(wg), _ptr(wu), _ptr(x), _ptr(g), _ptr(out), n, k, threads)
    return out


def cpu_gemm(fmt, w, a, m, n, k, threads):
    y = np.empty((m, n), np.float32)
    fn = lib().cb_gemm_q4k_q8k if fmt == "q4_k" else lib().cb_gemm_q6k
    fn(_ptr(w), _ptr(a), _ptr(y), m, n, k, threads)
    return y


def cpu_threads() -> int:
    return int(lib().cb_max_threads())


# ---- layer operations -------------------------------------------------------------

def _f32(a):
    return np.ascontiguousarray(a, np.float32)


def rms_norm(x, w, eps: float, rows: int = 1) -> np.ndarray:
    x, w = _f32(x), _f32(w)
    n = x.size // rows
    out = np.empty(x.size, np.float64)
    lib().or_rms_norm(_ptr(x), _ptr(w), n, rows, eps, _ptr(out))
    return out


def rope_theta(i: int, d: int, base: float, freq_scale=None) -> float:
    fs = None if freq_scale is None else _f32(freq_scale)
    return lib().or_rope_theta(i, d, base, None if fs is None else _ptr(fs))


def rope(x, seq: int, nh: int, d: int, pos0: int, base: float, neox: bool, freq_scale=None) -> np.ndarray:
    out = np.ascontiguousarray(x, np.float64).copy()
    fs = None if freq_scale is None else _f32(freq_scale)
    lib().or_rope(_ptr(out), seq, nh, d, pos0, base, int(neox), None if fs is None else _ptr(fs))
    return out


def attn_decode(q, kc16, vc16, seq: int, nh: int, nkv: int, d: int, scale: float) -> np.ndarray:
    q = _f32(q)
    kc16, vc16 = np.ascontiguousarray(kc16, np.uint16), np.ascontiguousarray(vc16, np.uint16)
    out = np.empty(nh * d, np.float64)
    lib().or_attn_decode(_ptr(q), _ptr(kc16), _ptr(vc16), seq, nh, nkv, d, scale, _ptr(out))
    return out


def attn_prefill_f16(q, k, v, seq: int, nh: int, nkv: int, d: int, scale: float) -> np.ndarray:
    q, k, v = _f32(q), _f32(k), _f32(v)
    out = np.empty(seq * nh * d, np.float64)
    lib().or_attn_prefill_f16(_ptr(q), _ptr(k), _ptr(v), seq, nh, nkv, d, scale, _ptr(out))
    return out


def silu_mul(g, u) -> np.ndarray:
    g, u = _f32(g), _f32(u)
    out = np.empty(g.size, np.float64)
    lib().or_silu_mul(_ptr(g), _ptr(u), g.size, _ptr(out))
    return out


def argmax(x) -> int:
    x = _f32(x)
    return lib().or_argmax(_ptr(x), x.size)
