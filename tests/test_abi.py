"""C-ABI checks that need no GPU: the library loads, exports every symbol
include/rocmforge_cdna4.h declares, and rejects the shapes/pointers the
reference launchers reject (their validation runs before any HIP call)."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HIP_ERROR_INVALID_VALUE = 1


def header_symbols():
    text = (ROOT / "include" / "rocmforge_cdna4.h").read_text()
    return sorted(set(re.findall(r"^(?:hipError_t|const char\*|int|void|size_t)\s+(\w+)\(", text, re.M)))


def test_header_declares_reference_launchers():
    syms = header_symbols()
    for s in ["gemv_q4_k_f32_q8_inline_launch", "gemv_q4_k_f32_q8_inline_residual_launch",
              "gemv_gate_up_swiglu_q4_k_f32_q8_inline_launch", "gemv_q4_k_f32_launch",
              "gemv_q4_k_f32_residual_launch", "gemv_gate_up_swiglu_q4_k_f32_launch",
              "gemv_q6_k_f32_launch", "wmma_gemm_q4_k_launch", "wmma_gemm_q6_k_launch"]:
        assert s in syms


def test_library_exports_every_header_symbol(rf):
    for s in header_symbols():
        assert hasattr(rf, s), f"missing export {s}"
    assert b"gfx950" in rf.rf_library_version()


P = ctypes.c_void_p(0x100000)      # never dereferenced: validation rejects first
NUL = None


@pytest.mark.parametrize("k,n", [(0, 64), (256, 0), (-256, 64), (300, 64), (30976, 64)])
def test_q8_inline_rejects_shapes(rf, k, n):
    assert rf.gemv_q4_k_f32_q8_inline_launch(P, P, P, k, n, NUL) == HIP_ERROR_INVALID_VALUE
    assert rf.gemv_q4_k_f32_q8_inline_residual_launch(P, P, P, P, k, n, NUL) == HIP_ERROR_INVALID_VALUE
    assert rf.gemv_gate_up_swiglu_q4_k_f32_q8_inline_launch(P, P, P, P, k, n, NUL) == HIP_ERROR_INVALID_VALUE


def test_null_and_alignment_rejections(rf):
    # residual null (q4_k_q8_inline.hip:413), gate/up null (:440)
    assert rf.gemv_q4_k_f32_q8_inline_residual_launch(P, P, NUL, P, 256, 64, NUL) == HIP_ERROR_INVALID_VALUE
    assert rf.gemv_gate_up_swiglu_q4_k_f32_q8_inline_launch(NUL, P, P, P, 256, 64, NUL) == HIP_ERROR_INVALID_VALUE
    assert rf.gemv_gate_up_swiglu_q4_k_f32_launch(P, NUL, P, P, 256, 64, NUL) == HIP_ERROR_INVALID_VALUE
    assert rf.gemv_q4_k_f32_residual_launch(P, P, NUL, P, 256, 64, NUL) == HIP_ERROR_INVALID_VALUE
    odd = ctypes.c_void_p(0x100001)
    assert rf.gemv_q4_k_f32_q8_inline_launch(ctypes.c_void_p(0x100008), P, P, 256, 64, NUL) == HIP_ERROR_INVALID_VALUE
    assert rf.gemv_q6_k_f32_launch(odd, P, P, 256, 64, NUL) == HIP_ERROR_INVALID_VALUE


@pytest.mark.parametrize("k,n", [(0, 64), (256, 0), (200, 64)])
def test_fp32_and_q6_reject_shapes(rf, k, n):
    assert rf.gemv_q4_k_f32_launch(P, P, P, k, n, NUL) == HIP_ERROR_INVALID_VALUE
    assert rf.gemv_q6_k_f32_launch(P, P, P, k, n, NUL) == HIP_ERROR_INVALID_VALUE


@pytest.mark.parametrize("m,n,k", [(0, 64, 256), (65, 64, 256), (64, 96, 256), (64, 64, 320), (64, 64, 0)])
def test_gemm_rejects_shapes(rf, m, n, k):
    # wmma_gemm_q4_k.hip:207-210: M % 64, N % 64, K % 256
    assert rf.wmma_gemm_q4_k_launch(P, P, P, m, n, k, NUL) == HIP_ERROR_INVALID_VALUE
    assert rf.wmma_gemm_q6_k_launch(P, P, P, m, n, k, NUL) == HIP_ERROR_INVALID_VALUE


@pytest.mark.parametrize("k", [0, 1024, 3072, 6144, 16384, 300])
def test_qkv_q6v_rejects_shapes(rf, k):
    # K in {2048, 4096, 8192}: whole Q6_K teams of K / 2048 waves in a workgroup
    assert rf.rf_gemv_qkv_q4_k_q6_k_v_rmsnorm_launch(P, P, P, NUL, NUL, NUL, P, P, 1e-6, P, P, P, k, 64, 16,
                                                     NUL) == HIP_ERROR_INVALID_VALUE


def test_qkv_q6v_rejects_pointers(rf):
    f = rf.rf_gemv_qkv_q4_k_q6_k_v_rmsnorm_launch
    assert f(P, P, NUL, NUL, NUL, NUL, P, P, 1e-6, P, P, P, 4096, 64, 16, NUL) == HIP_ERROR_INVALID_VALUE
    assert f(P, P, P, NUL, NUL, NUL, P, NUL, 1e-6, P, P, P, 4096, 64, 16, NUL) == HIP_ERROR_INVALID_VALUE
    assert f(P, P, P, NUL, NUL, NUL, P, P, 1e-6, P, P, NUL, 4096, 64, 16, NUL) == HIP_ERROR_INVALID_VALUE
    assert f(P, P, ctypes.c_void_p(0x100002), NUL, NUL, NUL, P, P, 1e-6, P, P, P, 4096, 64, 16,
             NUL) == HIP_ERROR_INVALID_VALUE
    assert f(P, P, P, NUL, NUL, NUL, P, P, 1e-6, P, P, P, 4096, 0, 16, NUL) == HIP_ERROR_INVALID_VALUE


def test_accumulate_rmsnorm_rejections(rf):
    # validation before any HIP call: null pointers, shapes, alignment, overlap
    f4, f6 = rf.rf_gemm_q4_k_f16_accumulate_rmsnorm_launch, rf.rf_gemm_q6_k_f16_accumulate_rmsnorm_launch
    eps = ctypes.c_float(1e-6)
    o = ctypes.c_void_p(0x200000)
    for f in (f4, f6):
        assert f(P, P, P, NUL, eps, o, 64, 4096, 4096, NUL) == HIP_ERROR_INVALID_VALUE     # no norm weights
        assert f(P, P, P, P, eps, NUL, 64, 4096, 4096, NUL) == HIP_ERROR_INVALID_VALUE     # no output
        assert f(P, P, P, P, eps, o, 96, 4096, 4096, NUL) == HIP_ERROR_INVALID_VALUE       # M % 64
        assert f(P, P, P, P, eps, o, 64, 4000, 4096, NUL) == HIP_ERROR_INVALID_VALUE       # N % 64
        assert f(P, P, P, P, eps, ctypes.c_void_p(0x200002), 64, 4096, 4096, NUL) == HIP_ERROR_INVALID_VALUE
        assert f(P, P, P, P, eps, ctypes.c_void_p(0x100000 + 4096), 64, 4096, 4096, NUL) == HIP_ERROR_INVALID_VALUE
    assert f6(P, P, P, P, eps, o, 64, 4096, 1024, NUL) == HIP_ERROR_INVALID_VALUE           # Q6_K K % 2048
