"""Host routing of the Q4_K / Q6_K matmul arms -- the Python face of the
C dispatch functions in librocmforge_cdna4.so (include/rocmforge_cdna4.h),
which restate ROCmForge's src/gpu/ops.rs routing.

Function names, argument order and error behaviour follow ops.rs:
  gpu_dispatch_gemv / gpu_dispatch_gemv_on_stream      (ops.rs:455, :484)
  gpu_dispatch_gemv_residual_on_stream -> bool         (ops.rs:509)
  gpu_dispatch_fused_gate_up_on_stream (Q4_K arm)      (ops.rs:1441, :1316-1355)
  gpu_dispatch_fused_qkv_on_stream (Q4_K fused arm)    (ops.rs:748, individual GEMVs :851-853)
  gpu_dispatch_gemm                                    (ops.rs:1591)
  refresh_runtime_env_flags                            (safety.rs:123)
Errors map to the reference's GpuError variants: InvalidWeightLayout,
UnsupportedWeightType, HipApiError(code).  An arm whose kernel is not part
of this library (Q4_0 / Q4_1 / Q8_0 / Q5_K, the scalar Q4_K GEMM, the
unfused gate/up path) raises NotInLibrary, so a caller can keep its own
route for it.

Pointers are device addresses: ints, ctypes.c_void_p, or objects with a
data_ptr() method (torch tensors).
"""
from __future__ import annotations

import ctypes
import enum
from dataclasses import dataclass, field

from ._lib import load

RF_DISPATCH_OK = 0
RF_DISPATCH_INVALID_LAYOUT = -1001
RF_DISPATCH_UNSUPPORTED_TYPE = -1002
RF_DISPATCH_NOT_IN_LIBRARY = -1003


class GgmlType(enum.IntEnum):
    """GGUF tensor type codes (src/loader/ggml_type.rs:6-19)."""
    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q4_1 = 3
    Q5_0 = 6
    Q5_1 = 7
    Q8_0 = 8
    Q2_K = 10
    Q3_K = 11
    Q4_K = 12
    Q5_K = 13
    Q6_K = 14


class TensorRole(enum.IntEnum):
    """src/gpu/weights.rs:22-26."""
    GENERIC = 0
    LM_HEAD = 1
    TIED_LM_HEAD = 2


@dataclass
class WeightMeta:
    """src/gpu/weights.rs:29-40: type and GGUF dims (innermost first)."""
    wtype: GgmlType
    dims: list = field(default_factory=list)
    role: TensorRole = TensorRole.GENERIC


class GpuError(RuntimeError):
    pass


class InvalidWeightLayout(GpuError):
    pass


class UnsupportedWeightType(GpuError):
    pass


class NotInLibrary(GpuError):
    pass


class HipApiError(GpuError):
    def __init__(self, code: int, what: str):
        super().__init__(f"{what}: hipError {code}")
        self.code = code


class _CMeta(ctypes.Structure):
    _fields_ = [("wtype", ctypes.c_int32), ("n_dims", ctypes.c_int32), ("dims", ctypes.c_uint64 * 4),
                ("role", ctypes.c_int32)]


def _cmeta(meta: WeightMeta) -> _CMeta:
    m = _CMeta()
    m.wtype = int(meta.wtype)
    dims = list(meta.dims)[:4]
    m.n_dims = len(meta.dims)
    for i, d in enumerate(dims):
        m.dims[i] = int(d)
    m.role = int(meta.role)
    return m


def _ptr(p) -> ctypes.c_void_p:
    if p is None:
        return ctypes.c_void_p(0)
    if isinstance(p, ctypes.c_void_p):
        return p
    if hasattr(p, "data_ptr"):
        return ctypes.c_void_p(p.data_ptr())
    return ctypes.c_void_p(int(p))


_vp, _sz, _i = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
_SIGS = {
    "rf_gpu_dispatch_gemv": [_vp, ctypes.POINTER(_CMeta), _vp, _vp, _sz, _sz, _vp],
    "rf_gpu_dispatch_gemv_residual": [_vp, ctypes.POINTER(_CMeta), _vp, _vp, _vp, _sz, _sz, _vp,
                                      ctypes.POINTER(_i)],
    "rf_gpu_dispatch_fused_gate_up": [_vp, ctypes.POINTER(_CMeta), _vp, ctypes.POINTER(_CMeta), _vp, _vp, _sz, _sz,
                                      _vp],
    "rf_gpu_dispatch_gemm": [_vp, ctypes.POINTER(_CMeta), _vp, _vp, _sz, _sz, _sz],
    "rf_gpu_dispatch_fused_qkv": [_vp, ctypes.POINTER(_CMeta), _vp, _vp, ctypes.POINTER(_CMeta), _vp, _vp,
                                  ctypes.POINTER(_CMeta), _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _vp],
    "rf_dispatch_parse_env_flag": [ctypes.c_char_p, _i],
}


def _lib():
    lib = load()
    if not getattr(lib, "_rf_dispatch_sigs", False):
        for name, args in _SIGS.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int
        lib.rf_dispatch_refresh_flags.argtypes = []
        lib.rf_dispatch_refresh_flags.restype = None
        lib._rf_dispatch_sigs = True
    return lib


def _check(rc: int, what: str, meta: WeightMeta) -> None:
    if rc == RF_DISPATCH_OK:
        return
    if rc == RF_DISPATCH_INVALID_LAYOUT:
        raise InvalidWeightLayout(f"{what}: matrix dims {list(meta.dims)} do not match the vector lengths")
    if rc == RF_DISPATCH_UNSUPPORTED_TYPE:
        raise UnsupportedWeightType(f"{what}: {GgmlType(meta.wtype).name}")
    if rc == RF_DISPATCH_NOT_IN_LIBRARY:
        raise NotInLibrary(f"{what}: the {GgmlType(meta.wtype).name} arm is served outside this library")
    raise HipApiError(rc, what)


def gpu_dispatch_gemv_on_stream(weights, meta: WeightMeta, input, output, out_dim: int, in_dim: int,
                                stream=None) -> None:
    m = _cmeta(meta)
    rc = _lib().rf_gpu_dispatch_gemv(_ptr(weights), ctypes.byref(m), _ptr(input), _ptr(output), out_dim, in_dim,
                                     _ptr(stream))
    _check(rc, "gpu_dispatch_gemv_on_stream", meta)


def gpu_dispatch_gemv(weights, meta: WeightMeta, input, output, out_dim: int, in_dim: int) -> None:
    gpu_dispatch_gemv_on_stream(weights, meta, input, output, out_dim, in_dim, None)


def gpu_dispatch_gemv_residual_on_stream(weights, meta: WeightMeta, input, residual, output, in_dim: int,
                                         out_dim: int, stream=None) -> bool:
    """True when a fused residual kernel ran; False (nothing launched) for
    weight types without one -- the caller then runs GEMV + add."""
    m = _cmeta(meta)
    done = ctypes.c_int(0)
    rc = _lib().rf_gpu_dispatch_gemv_residual(_ptr(weights), ctypes.byref(m), _ptr(input), _ptr(residual),
                                              _ptr(output), in_dim, out_dim, _ptr(stream), ctypes.byref(done))
    _check(rc, "gpu_dispatch_gemv_residual_on_stream", meta)
    return bool(done.value)


def gpu_dispatch_fused_gate_up_on_stream(w_gate, gate_meta: WeightMeta, w_up, up_meta: WeightMeta, input, output,
                                         ff_size: int, h: int, stream=None) -> None:
    g, u = _cmeta(gate_meta), _cmeta(up_meta)
    rc = _lib().rf_gpu_dispatch_fused_gate_up(_ptr(w_gate), ctypes.byref(g), _ptr(w_up), ctypes.byref(u),
                                              _ptr(input), _ptr(output), ff_size, h, _ptr(stream))
    _check(rc, "gpu_dispatch_fused_gate_up_on_stream", gate_meta)


def gpu_dispatch_fused_qkv_on_stream(w_q, q_meta: WeightMeta, q_bias, w_k, k_meta: WeightMeta, k_bias, w_v,
                                     v_meta: WeightMeta, v_bias, input, out_q, out_k, out_v, q_size: int,
                                     kv_size: int, h: int, stream=None) -> None:
    """Biases may be None.  Three Q4_K tensors go to one fused launch; other
    type mixes to three GEMV dispatches (NotInLibrary if a bias is given)."""
    q, k, v = _cmeta(q_meta), _cmeta(k_meta), _cmeta(v_meta)
    rc = _lib().rf_gpu_dispatch_fused_qkv(_ptr(w_q), ctypes.byref(q), _ptr(q_bias), _ptr(w_k), ctypes.byref(k),
                                          _ptr(k_bias), _ptr(w_v), ctypes.byref(v), _ptr(v_bias), _ptr(input),
                                          _ptr(out_q), _ptr(out_k), _ptr(out_v), q_size, kv_size, h, _ptr(stream))
    _check(rc, "gpu_dispatch_fused_qkv_on_stream", q_meta)


def gpu_dispatch_gemm(weights, meta: WeightMeta, input, output, out_dim: int, in_dim: int, seq_len: int) -> None:
    """Null stream, as the reference.  For the GEMM arm the input and output
    buffers must hold round_up(seq_len, 64) rows, the extra rows zero."""
    m = _cmeta(meta)
    rc = _lib().rf_gpu_dispatch_gemm(_ptr(weights), ctypes.byref(m), _ptr(input), _ptr(output), out_dim, in_dim,
                                     seq_len)
    _check(rc, "gpu_dispatch_gemm", meta)


def refresh_runtime_env_flags() -> None:
    _lib().rf_dispatch_refresh_flags()


def parse_env_flag(value, default: bool) -> bool:
    v = None if value is None else str(value).encode()
    return bool(_lib().rf_dispatch_parse_env_flag(v, int(default)))
