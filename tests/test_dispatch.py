"""Host routing (rf_gpu_dispatch_*, include/rocmforge_cdna4.h) checked on the
CPU: recording stand-ins replace the launchers, so every arm of the routing
restated from src/gpu/ops.rs runs without a GPU.  Expected call sequences
come from ops.rs:387-446 (GEMV), :666-695 (residual), :1316-1355 (fused
gate+up), :748-853 (fused QKV), :1591-1963 (GEMM) and safety.rs (flags)."""
import ctypes
import os

import pytest

from rocmforge_amd import ops
from rocmforge_amd.ops import GgmlType, WeightMeta

HIP_OK, HIP_INVALID = 0, 1
_vp, _i = ctypes.c_void_p, ctypes.c_int
GEMV = ctypes.CFUNCTYPE(_i, _vp, _vp, _vp, _i, _i, _vp)
RES = ctypes.CFUNCTYPE(_i, _vp, _vp, _vp, _vp, _i, _i, _vp)
FUSED = ctypes.CFUNCTYPE(_i, _vp, _vp, _vp, _vp, _i, _i, _vp)
GEMM = ctypes.CFUNCTYPE(_i, _vp, _vp, _vp, _i, _i, _i, _vp)
QKV = ctypes.CFUNCTYPE(_i, *([_vp] * 10), _i, _i, _i, _vp)
NAMES = [("gemv_q4_k_q8_inline", GEMV), ("gemv_q4_k_q8_inline_residual", RES), ("gemv_gate_up_q4_k_q8_inline", FUSED),
         ("gemv_q4_k_f32", GEMV), ("gemv_q4_k_f32_residual", RES), ("gemv_gate_up_q4_k_f32", FUSED),
         ("gemv_q6_k_f32", GEMV), ("wmma_gemm_q4_k", GEMM), ("wmma_gemm_q6_k", GEMM),
         ("gemv_qkv_q4_k_q8_inline", QKV)]


class Table(ctypes.Structure):
    _fields_ = [(n, t) for n, t in NAMES]


class Recorder:
    """Installs stand-in launchers; records (name, args) and returns the
    code configured for that launcher (default hipSuccess)."""

    def __init__(self, lib):
        self.lib, self.calls, self.codes = lib, [], {}
        self._keep = []
        tab = Table()
        for name, proto in NAMES:
            def fn(*args, _n=name):
                self.calls.append((_n, [a if a is not None else 0 for a in args]))
                return self.codes.get(_n, HIP_OK)
            cb = proto(fn)
            self._keep.append(cb)
            setattr(tab, name, cb)
        self.table = tab
        lib.rf_dispatch_set_launchers(ctypes.byref(tab))

    def names(self):
        return [c[0] for c in self.calls]

    def close(self):
        self.lib.rf_dispatch_set_launchers(None)


@pytest.fixture
def rec(rf):
    ops._lib()
    r = Recorder(rf)
    yield r
    r.close()
    for k in ("ROCMFORGE_GPU_SAFE_MODE", "ROCMFORGE_ENABLE_EXPERIMENTAL_Q8_ACTIVATION_FASTPATH",
              "ROCMFORGE_DISABLE_WMMA_PREFILL"):
        os.environ.pop(k, None)
    ops.refresh_runtime_env_flags()


def setenv(k, v):
    os.environ[k] = v
    ops.refresh_runtime_env_flags()


W, X, Y, R = 0x1000, 0x2000, 0x3000, 0x4000


def q4k(out, inn):
    return WeightMeta(GgmlType.Q4_K, [inn, out])


def test_parse_env_flag_matches_reference(rf):
    # safety.rs:268-285
    assert not ops.parse_env_flag(None, False) and ops.parse_env_flag(None, True)
    for v in ["1", "true", "On", " yes ", "TRUE"]:
        assert ops.parse_env_flag(v, False), v
    for v in ["0", "false", "no", "", "enabled", "1 1"]:
        assert not ops.parse_env_flag(v, True), v


def test_q4k_gemv_prefers_q8_inline(rec):
    ops.gpu_dispatch_gemv_on_stream(W, q4k(4096, 4096), X, Y, 4096, 4096, 0x77)
    assert rec.calls == [("gemv_q4_k_q8_inline", [W, X, Y, 4096, 4096, 0x77])]


def test_q4k_gemv_falls_back_on_q8_error(rec):
    rec.codes["gemv_q4_k_q8_inline"] = HIP_INVALID
    ops.gpu_dispatch_gemv(W, q4k(64, 4096), X, Y, 64, 4096)
    assert rec.names() == ["gemv_q4_k_q8_inline", "gemv_q4_k_f32"]
    assert rec.calls[1][1] == [W, X, Y, 4096, 64, 0]


def test_q4k_gemv_skips_q8_when_lds_misfits(rec):
    # (K/32)*34 > 32768 from K = 30976 on (q4_k_q8_inline_fits)
    ops.gpu_dispatch_gemv(W, q4k(64, 30976), X, Y, 64, 30976)
    assert rec.names() == ["gemv_q4_k_f32"]
    rec.calls.clear()
    ops.gpu_dispatch_gemv(W, q4k(64, 30720), X, Y, 64, 30720)
    assert rec.names() == ["gemv_q4_k_q8_inline"]


@pytest.mark.parametrize("env", [("ROCMFORGE_ENABLE_EXPERIMENTAL_Q8_ACTIVATION_FASTPATH", "0"),
                                 ("ROCMFORGE_GPU_SAFE_MODE", "1")])
def test_q8_fastpath_flags(rec, env):
    setenv(*env)
    ops.gpu_dispatch_gemv(W, q4k(64, 4096), X, Y, 64, 4096)
    assert rec.names() == ["gemv_q4_k_f32"]


def test_final_launcher_error_is_hip_api_error(rec):
    rec.codes["gemv_q4_k_q8_inline"] = HIP_INVALID
    rec.codes["gemv_q4_k_f32"] = HIP_INVALID
    with pytest.raises(ops.HipApiError) as e:
        ops.gpu_dispatch_gemv(W, q4k(64, 4096), X, Y, 64, 4096)
    assert e.value.code == HIP_INVALID


def test_q6k_gemv(rec):
    ops.gpu_dispatch_gemv(W, WeightMeta(GgmlType.Q6_K, [14336, 4096]), X, Y, 4096, 14336)
    assert rec.calls == [("gemv_q6_k_f32", [W, X, Y, 14336, 4096, 0])]


def test_layout_validation(rec):
    # dims may come in either order (validate_gemv_layout, ops.rs:92-94)
    ops.gpu_dispatch_gemv(W, WeightMeta(GgmlType.Q4_K, [64, 4096]), X, Y, 64, 4096)
    for dims in ([4096, 128], [4096], []):
        with pytest.raises(ops.InvalidWeightLayout):
            ops.gpu_dispatch_gemv(W, WeightMeta(GgmlType.Q4_K, dims), X, Y, 64, 4096)
    assert rec.names() == ["gemv_q4_k_q8_inline"]


def test_type_support(rec):
    with pytest.raises(ops.UnsupportedWeightType):
        ops.gpu_dispatch_gemv(W, WeightMeta(GgmlType.F16, [4096, 64]), X, Y, 64, 4096)
    for t in (GgmlType.Q4_0, GgmlType.Q4_1, GgmlType.Q8_0, GgmlType.Q5_K):
        with pytest.raises(ops.NotInLibrary):
            ops.gpu_dispatch_gemv(W, WeightMeta(t, [4096, 64]), X, Y, 64, 4096)
    assert rec.calls == []


def test_residual_arms(rec):
    assert ops.gpu_dispatch_gemv_residual_on_stream(W, q4k(4096, 4096), X, R, Y, 4096, 4096, 0x5)
    assert rec.calls == [("gemv_q4_k_q8_inline_residual", [W, X, R, Y, 4096, 4096, 0x5])]
    rec.calls.clear()
    rec.codes["gemv_q4_k_q8_inline_residual"] = HIP_INVALID
    assert ops.gpu_dispatch_gemv_residual_on_stream(W, q4k(4096, 4096), X, R, Y, 4096, 4096)
    assert rec.names() == ["gemv_q4_k_q8_inline_residual", "gemv_q4_k_f32_residual"]
    rec.calls.clear()
    # other types: Ok(false), nothing launched (ops.rs:695)
    assert not ops.gpu_dispatch_gemv_residual_on_stream(W, WeightMeta(GgmlType.Q6_K, [4096, 4096]), X, R, Y, 4096,
                                                        4096)
    assert rec.calls == []


def test_fused_gate_up(rec):
    ops.gpu_dispatch_fused_gate_up_on_stream(W, q4k(14336, 4096), W + 8, q4k(14336, 4096), X, Y, 14336, 4096, 0x9)
    assert rec.calls == [("gemv_gate_up_q4_k_q8_inline", [W, W + 8, X, Y, 4096, 14336, 0x9])]
    rec.calls.clear()
    setenv("ROCMFORGE_ENABLE_EXPERIMENTAL_Q8_ACTIVATION_FASTPATH", "off")
    ops.gpu_dispatch_fused_gate_up_on_stream(W, q4k(14336, 4096), W + 8, q4k(14336, 4096), X, Y, 14336, 4096)
    assert rec.names() == ["gemv_gate_up_q4_k_f32"]
    with pytest.raises(ops.InvalidWeightLayout):
        ops.gpu_dispatch_fused_gate_up_on_stream(W, q4k(14336, 4096), W, q4k(14000, 4096), X, Y, 14336, 4096)
    with pytest.raises(ops.NotInLibrary):
        ops.gpu_dispatch_fused_gate_up_on_stream(W, WeightMeta(GgmlType.Q4_0, [4096, 14336]), W,
                                                 WeightMeta(GgmlType.Q4_0, [4096, 14336]), X, Y, 14336, 4096)


def test_gemm_decode_row_is_gemv(rec):
    ops.gpu_dispatch_gemm(W, q4k(4096, 4096), X, Y, 4096, 4096, 1)
    assert rec.names() == ["gemv_q4_k_q8_inline"]


@pytest.mark.parametrize("seq,padded", [(64, 64), (65, 128), (100, 128), (2, 64), (512, 512)])
def test_gemm_pads_m_to_64(rec, seq, padded):
    ops.gpu_dispatch_gemm(W, q4k(14336, 4096), X, Y, 14336, 4096, seq)
    assert rec.calls == [("wmma_gemm_q4_k", [X, W, Y, padded, 14336, 4096, 0])]
    rec.calls.clear()
    ops.gpu_dispatch_gemm(W, WeightMeta(GgmlType.Q6_K, [14336, 4096]), X, Y, 4096, 14336, seq)
    assert rec.calls == [("wmma_gemm_q6_k", [X, W, Y, padded, 4096, 14336, 0])]


def test_gemm_fallbacks(rec):
    # WMMA off, seq_len <= 8: one GEMV per row (ops.rs:1884-1891)
    setenv("ROCMFORGE_DISABLE_WMMA_PREFILL", "1")
    ops.gpu_dispatch_gemm(W, q4k(4096, 4096), X, Y, 4096, 4096, 3)
    assert rec.names() == ["gemv_q4_k_q8_inline"] * 3
    assert [c[1][1] for c in rec.calls] == [X, X + 4096 * 4, X + 2 * 4096 * 4]
    assert [c[1][2] for c in rec.calls] == [Y, Y + 4096 * 4, Y + 2 * 4096 * 4]
    rec.calls.clear()
    # Q6_K, longer sequences: the Q6_K GEMV loop (ops.rs:1935-1963)
    ops.gpu_dispatch_gemm(W, WeightMeta(GgmlType.Q6_K, [256, 128]), X, Y, 128, 256, 20)
    assert rec.names() == ["gemv_q6_k_f32"] * 20
    rec.calls.clear()
    # Q4_K longer sequences: the reference's scalar GEMM, not in this library
    with pytest.raises(ops.NotInLibrary):
        ops.gpu_dispatch_gemm(W, q4k(4096, 4096), X, Y, 4096, 4096, 20)
    assert rec.calls == []


def test_gemm_wmma_failure_falls_through(rec):
    rec.codes["wmma_gemm_q6_k"] = HIP_INVALID
    ops.gpu_dispatch_gemm(W, WeightMeta(GgmlType.Q6_K, [4096, 128]), X, Y, 128, 4096, 10)
    assert rec.names() == ["wmma_gemm_q6_k"] + ["gemv_q6_k_f32"] * 10
    rec.calls.clear()
    # shapes off the WMMA grid (N % 64 != 0) skip it
    ops.gpu_dispatch_gemm(W, WeightMeta(GgmlType.Q6_K, [4096, 96]), X, Y, 96, 4096, 4)
    assert rec.names() == ["gemv_q6_k_f32"] * 4


WQ, WK, WV, BQ, OQ, OK, OV = 0x5000, 0x6000, 0x7000, 0x8000, 0x9000, 0xA000, 0xB000


def test_fused_qkv_q4k_one_launch(rec):
    ops.gpu_dispatch_fused_qkv_on_stream(WQ, q4k(4096, 4096), BQ, WK, q4k(1024, 4096), None, WV, q4k(1024, 4096),
                                         None, X, OQ, OK, OV, 4096, 1024, 4096, 0x77)
    assert rec.calls == [("gemv_qkv_q4_k_q8_inline", [WQ, WK, WV, BQ, 0, 0, X, OQ, OK, OV, 4096, 4096, 1024, 0x77])]


def test_fused_qkv_mixed_types_individual_gemvs(rec):
    # Q4_K_M keeps some attn_v tensors in Q6_K: three GEMV dispatches
    q6 = WeightMeta(GgmlType.Q6_K, [4096, 1024])
    ops.gpu_dispatch_fused_qkv_on_stream(WQ, q4k(4096, 4096), None, WK, q4k(1024, 4096), None, WV, q6, None, X, OQ,
                                         OK, OV, 4096, 1024, 4096)
    assert rec.names() == ["gemv_q4_k_q8_inline", "gemv_q4_k_q8_inline", "gemv_q6_k_f32"]
    assert rec.calls[2][1] == [WV, X, OV, 4096, 1024, 0]


def test_fused_qkv_falls_back_without_fast_path(rec):
    setenv("ROCMFORGE_ENABLE_EXPERIMENTAL_Q8_ACTIVATION_FASTPATH", "0")
    ops.gpu_dispatch_fused_qkv_on_stream(WQ, q4k(4096, 4096), None, WK, q4k(1024, 4096), None, WV, q4k(1024, 4096),
                                         None, X, OQ, OK, OV, 4096, 1024, 4096)
    assert rec.names() == ["gemv_q4_k_f32"] * 3


def test_fused_qkv_bias_outside_fused_arm_not_in_library(rec):
    rec.codes["gemv_qkv_q4_k_q8_inline"] = HIP_INVALID
    with pytest.raises(ops.NotInLibrary):
        ops.gpu_dispatch_fused_qkv_on_stream(WQ, q4k(4096, 4096), BQ, WK, q4k(1024, 4096), None, WV,
                                             q4k(1024, 4096), None, X, OQ, OK, OV, 4096, 1024, 4096)
    assert rec.names() == ["gemv_qkv_q4_k_q8_inline"]
