"""ctypes binding of librocmforge_cdna4.so (the C ABI in include/rocmforge_cdna4.h).

The library is the product: nothing here falls back to another
implementation.  If the shared object is missing, loading raises.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "librocmforge_cdna4.so"

_vp = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float
_sz = ctypes.c_size_t

# name -> argtypes (all return hipError_t as int)
SIGNATURES = {
    "gemv_q4_k_f32_q8_inline_launch": [_vp, _vp, _vp, _i, _i, _vp],
    "gemv_q4_k_f32_q8_inline_residual_launch": [_vp, _vp, _vp, _vp, _i, _i, _vp],
    "gemv_gate_up_swiglu_q4_k_f32_q8_inline_launch": [_vp, _vp, _vp, _vp, _i, _i, _vp],
    "gemv_q4_k_f32_launch": [_vp, _vp, _vp, _i, _i, _vp],
    "gemv_q4_k_f32_residual_launch": [_vp, _vp, _vp, _vp, _i, _i, _vp],
    "gemv_gate_up_swiglu_q4_k_f32_launch": [_vp, _vp, _vp, _vp, _i, _i, _vp],
    "gemv_qkv_q4_k_f32_q8_inline_launch": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _vp],
    "gemv_q6_k_f32_launch": [_vp, _vp, _vp, _i, _i, _vp],
    "gemv_q6_k_f32_residual_launch": [_vp, _vp, _vp, _vp, _i, _i, _vp],
    "wmma_gemm_q4_k_launch": [_vp, _vp, _vp, _i, _i, _i, _vp],
    "wmma_gemm_q6_k_launch": [_vp, _vp, _vp, _i, _i, _i, _vp],
    "rf_gemm_q4_k_f16_launch": [_vp, _vp, _vp, _i, _i, _i, _vp],
    "rf_gemm_q6_k_f16_launch": [_vp, _vp, _vp, _i, _i, _i, _vp],
    "rf_gemm_q6_k_f16_accumulate_launch": [_vp, _vp, _vp, _i, _i, _i, _vp],
    "rf_gemm_q4_k_f16_accumulate_launch": [_vp, _vp, _vp, _i, _i, _i, _vp],
    "rf_gemm_q4_k_f16_accumulate_rmsnorm_launch": [_vp, _vp, _vp, _vp, _f, _vp, _i, _i, _i, _vp],
    "rf_gemm_q6_k_f16_accumulate_rmsnorm_launch": [_vp, _vp, _vp, _vp, _f, _vp, _i, _i, _i, _vp],
    "rf_gemm_qk_f16_segments_launch": [_vp, _vp, _vp, _vp, _i, _i, _i, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp],
    "rf_gemm_q4_k_f16_swiglu_launch": [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp],
    "rf_gemm_q4_k_f16_swiglu_up_launch": [_vp, _vp, _vp, _vp, _i, _i, _i, _vp],
    "rf_gemm_q4_k_segments_launch": [_vp] * 7 + [_i] * 5 + [_vp],
    "rf_gemm_q6_k_segments_launch": [_vp] * 7 + [_i] * 5 + [_vp],
    "rf_gemm_q4_k_accumulate_launch": [_vp, _vp, _vp, _i, _i, _i, _vp],
    "rf_gemm_q6_k_accumulate_launch": [_vp, _vp, _vp, _i, _i, _i, _vp],
    "rf_gemm_q4_k_swiglu_launch": [_vp, _vp, _vp, _vp, _i, _i, _i, _vp],
    "rf_gemm_q6_k_swiglu_launch": [_vp, _vp, _vp, _vp, _i, _i, _i, _vp],
    "rf_gemm_q4_k_swiglu_f16_launch": [_vp, _vp, _vp, _vp, _i, _i, _i, _vp],
    "rf_gemm_q6_k_swiglu_f16_launch": [_vp, _vp, _vp, _vp, _i, _i, _i, _vp],
    "rf_gemv_q4_k_q8_rmsnorm_launch": [_vp, _vp, _vp, _f, _vp, _i, _i, _vp],
    "rf_gemv_gate_up_q4_k_q8_rmsnorm_launch": [_vp, _vp, _vp, _vp, _f, _vp, _i, _i, _vp],
    "rf_gemv_qkv_q4_k_q8_rmsnorm_launch": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _f, _vp, _vp, _vp, _i, _i, _i,
                                           _vp],
    "rf_gemv_q6_k_rmsnorm_launch": [_vp, _vp, _vp, _f, _vp, _i, _i, _vp],
    "rf_gemv_qkv_q4_k_q6_k_v_rmsnorm_launch": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _f, _vp, _vp, _vp, _i, _i,
                                               _i, _vp],
    "gpu_rms_norm": [_vp, _vp, _vp, _i, _f, _vp],
    "gpu_rms_norm_batched": [_vp, _vp, _vp, _i, _f, _i],
    "gpu_rms_norm_batched_on_stream": [_vp, _vp, _vp, _i, _f, _i, _vp],
    "rf_rms_norm_batched_f16_on_stream": [_vp, _vp, _vp, _i, _f, _i, _vp],
    "gpu_rope_heads": [_vp, _i, _i, _i, _f, _i, _vp],
    "gpu_rope_heads_scaled": [_vp, _i, _i, _i, _f, _i, _vp, _vp],
    "gpu_rope_heads_state": [_vp, _vp, _i, _i, _f, _i, _vp],
    "gpu_rope_heads_state_scaled": [_vp, _vp, _i, _i, _f, _i, _vp, _vp],
    "gpu_rope_heads_batched": [_vp, _i, _i, _i, _f, _i, _i],
    "gpu_rope_heads_batched_scaled": [_vp, _i, _i, _i, _f, _i, _i, _vp],
    "rf_rope_heads_batched_on_stream": [_vp, _i, _i, _i, _f, _i, _i, _vp, _vp],
    "gpu_kv_write_rope": [_vp, _vp, _vp, _vp, _i, _i, _i, _f, _i, _vp],
    "gpu_kv_write_rope_scaled": [_vp, _vp, _vp, _vp, _i, _i, _i, _f, _i, _vp, _vp],
    "gpu_kv_write_rope_state": [_vp, _vp, _vp, _vp, _vp, _i, _i, _f, _i, _vp],
    "gpu_kv_write_rope_state_scaled": [_vp, _vp, _vp, _vp, _vp, _i, _i, _f, _i, _vp, _vp],
    "gpu_kv_write_batched": [_vp, _vp, _vp, _vp, _i, _i, _i, _i],
    "rf_kv_write_batched_on_stream": [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp],
    "rf_qk_norm_rope_kv_write_rows": [_vp] * 8 + [_i] * 7 + [_f, _f, _i, _vp, _vp, _vp, _vp],
    "rf_qk_norm_rope_kv_write_state": [_vp] * 8 + [_i, _i, _i, _f, _f, _i, _vp, _vp, _vp, _vp],
    "rf_rope_theta_table": [_vp, _i, _f, _vp],
    "rf_rope_cos_sin_table": [_vp, _i, _i, _f, _vp, _vp, _vp],
    "gpu_flash_attn_decode_strided_multi_head": [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _f, _vp],
    "gpu_flash_attn_decode_strided_multi_head_state": [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _f, _vp],
    "rf_flash_attn_decode_ws": [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _f, _vp, _sz, _vp],
    "rf_flash_attn_decode_state_ws": [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _f, _vp, _sz, _vp],
    "rf_flash_attn_decode_state_bounded": [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _f, _i, _vp, _sz, _vp],
    "rf_attn_decode_qk_norm_rope_state_bounded": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _f, _f,
                                                  _i, _vp, _vp, _vp, _f, _i, _vp, _sz, _vp],
    "rf_flash_attn_decode_state_noalloc": [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _f, _vp],
    "gpu_argmax_f32_on_stream": [_vp, _vp, _vp, _vp, _i, _vp],
    "gpu_argmax_f32": [_vp, _vp, _vp, _vp, _i],
    "rf_argmax_f32_advance_state_on_stream": [_vp, _vp, _vp, _vp, _i, _vp, _vp],
    "rf_attn_decode_qk_norm_rope_state": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _f, _f, _i, _vp,
                                          _vp, _vp, _f, _vp, _sz, _vp],
    "gpu_embed_q4_k_token": [_vp, _vp, _i, _i, _i, _vp],
    "gpu_embed_q4_k_batch": [_vp, _vp, _vp, _i, _i, _i, _vp],
    "gpu_add": [_vp, _vp, _vp, _i, _vp],
    "gpu_mul_on_stream": [_vp, _vp, _vp, _i, _vp],
    "gpu_silu_on_stream": [_vp, _vp, _i, _vp],
    "rf_silu_mul_on_stream": [_vp, _vp, _vp, _i, _vp],
    "rf_silu_mul_f16_on_stream": [_vp, _vp, _vp, _i, _vp],
    "gpu_increment_decode_state_on_stream": [_vp, _vp],
    "convert_f32_to_f16": [_vp, _vp, _i, _vp],
    "wmma_attention_prefill_gqa_causal_launch": [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _f, _vp],
    "rf_attention_prefill_gqa_causal_f16_launch": [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _f, _vp],
    "rf_q8_0_quantize_launch": [_vp, _vp, _vp, _vp, _i, _vp],
    "rf_q4_k_q8_int_dots_launch": [_vp, _vp, _vp, _i, _i, _vp],
    "rf_mfma_peak_launch": [_vp, _vp, _i, _i, _vp],
}

_LIB = None


class LibraryMissing(RuntimeError):
    pass


def load() -> ctypes.CDLL:
    """Load the HIP library once; raise LibraryMissing if it was never built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise LibraryMissing(
            f"{LIB_PATH} not found: build it with `python -m rocmforge_amd.build` "
            "(there is no fallback implementation)")
    lib = ctypes.CDLL(os.fspath(LIB_PATH), mode=ctypes.RTLD_LOCAL)
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name, None)
        if fn is None:
            continue
        fn.argtypes = argtypes
        fn.restype = ctypes.c_int
    lib.rf_library_version.restype = ctypes.c_char_p
    lib.rf_flash_attn_decode_workspace_bytes.argtypes = [_i, _i]
    lib.rf_flash_attn_decode_workspace_bytes.restype = _sz
    _LIB = lib
    return lib
