// dispatch.cpp -- host-side routing of the Q4_K / Q6_K matmul arms, the
// C++ counterpart of ROCmForge's src/gpu/ops.rs dispatch functions:
//   rf_gpu_dispatch_gemv           <- gpu_dispatch_gemv_on_stream (ops.rs:484)
//                                     + dispatch_gemv_impl (ops.rs:270)
//   rf_gpu_dispatch_gemv_residual  <- gpu_dispatch_gemv_residual_on_stream (ops.rs:509)
//   rf_gpu_dispatch_fused_gate_up  <- the Q4_K arm of
//                                     gpu_dispatch_fused_gate_up_with_scratch_on_stream (ops.rs:1316-1355)
//   rf_gpu_dispatch_fused_qkv      <- gpu_dispatch_fused_qkv_on_stream (ops.rs:748), with a Q4_K
//                                     fused arm in place of its Q4_0 one
//   rf_gpu_dispatch_gemm           <- gpu_dispatch_gemm (ops.rs:1591)
// with the layout check validate_gemv_layout (ops.rs:82) and the runtime
// flags of src/gpu/safety.rs (cached environment flags, refreshable).
//
// Only the arms whose kernels this library implements are routed here
// (Q4_K and Q6_K).  Arms that the reference serves with kernels outside
// this library (Q4_0 / Q4_1 / Q8_0 / Q5_K GEMVs, the vulkan-style
// experimental GEMVs, the scalar Q4_K GEMM, the unfused gate/up fallback)
// return RF_DISPATCH_NOT_IN_LIBRARY so the caller keeps its own route.
//
// The launchers are called through a table (default: this library's own
// extern "C" launchers) so the routing can be exercised without a GPU.
#include <ctype.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>

#include "../../include/rocmforge_cdna4.h"

namespace {

// ── runtime flags (safety.rs:50-115) ────────────────────────────────────
// "1", "true", "yes", "on" (any case, surrounding blanks ignored) enable a
// flag; any other value disables it; an unset variable takes the default.
bool parse_env_flag(const char* value, bool dflt) {
    if (value == nullptr) return dflt;
    const char* b = value;
    while (*b && isspace((unsigned char)*b)) ++b;
    const char* e = b + strlen(b);
    while (e > b && isspace((unsigned char)e[-1])) --e;
    const size_t n = (size_t)(e - b);
    if (n > 4) return false;   // longer than any truthy word
    char buf[5];
    for (size_t i = 0; i < n; ++i) buf[i] = (char)tolower((unsigned char)b[i]);
    buf[n] = '\0';
    return !strcmp(buf, "1") || !strcmp(buf, "true") || !strcmp(buf, "yes") || !strcmp(buf, "on");
}

struct CachedEnvFlag {
    const char* name;
    bool dflt;
    std::atomic<int> state{-1};   // -1 unknown, 0 disabled, 1 enabled
    bool enabled() {
        int s = state.load(std::memory_order_relaxed);
        if (s < 0) {
            s = parse_env_flag(getenv(name), dflt) ? 1 : 0;
            state.store(s, std::memory_order_relaxed);
        }
        return s == 1;
    }
    void reset() { state.store(-1, std::memory_order_relaxed); }
};

CachedEnvFlag g_safe_mode{"ROCMFORGE_GPU_SAFE_MODE", false};                                    // safety.rs:81
CachedEnvFlag g_q8_fastpath{"ROCMFORGE_ENABLE_EXPERIMENTAL_Q8_ACTIVATION_FASTPATH", true};      // safety.rs:77
CachedEnvFlag g_disable_wmma_prefill{"ROCMFORGE_DISABLE_WMMA_PREFILL", false};                  // safety.rs:98

// safety.rs:172 (the reference's runtime auto-disable of this path is only
// ever triggered from its Q4_0 arm, which is not routed here)
bool q8_fastpath_enabled() { return !g_safe_mode.enabled() && g_q8_fastpath.enabled(); }
bool wmma_prefill_enabled() { return !g_safe_mode.enabled() && !g_disable_wmma_prefill.enabled(); }   // safety.rs:215

// ── launcher table ───────────────────────────────────────────────────────
rf_launchers g_default = {
    gemv_q4_k_f32_q8_inline_launch,
    gemv_q4_k_f32_q8_inline_residual_launch,
    gemv_gate_up_swiglu_q4_k_f32_q8_inline_launch,
    gemv_q4_k_f32_launch,
    gemv_q4_k_f32_residual_launch,
    gemv_gate_up_swiglu_q4_k_f32_launch,
    gemv_q6_k_f32_launch,
    wmma_gemm_q4_k_launch,
    wmma_gemm_q6_k_launch,
    gemv_qkv_q4_k_f32_q8_inline_launch,
};
rf_launchers g_table = g_default;

// q4_k_q8_inline_fits (kernels/quant.rs:3412): (K/32) * 34 <= 32 KB
bool q4_k_q8_inline_fits(size_t in_dim) { return (in_dim / 32) * 34 <= 32768; }

// supports_gemv_type (ops.rs:42)
bool supports_gemv_type(int32_t t) {
    return t == RF_GGML_Q4_0 || t == RF_GGML_Q4_1 || t == RF_GGML_Q8_0 || t == RF_GGML_Q4_K || t == RF_GGML_Q5_K ||
           t == RF_GGML_Q6_K;
}

// validate_gemv_layout (ops.rs:82-105): a 2-D matrix whose dims are
// (in, out) or (out, in)
bool layout_ok(const rf_weight_meta* m, size_t out_dim, size_t in_dim) {
    if (m == nullptr || m->n_dims < 2) return false;
    const uint64_t d0 = m->dims[0], d1 = m->dims[1];
    return (d0 == in_dim && d1 == out_dim) || (d0 == out_dim && d1 == in_dim);
}

bool fits_int(size_t v) { return v <= (size_t)0x7FFFFFFF; }

// dispatch_gemv_impl, Q4_K and Q6_K arms (ops.rs:387-446)
int gemv_impl(const void* w, const rf_weight_meta* meta, const float* x, float* y, size_t out_dim, size_t in_dim,
              hipStream_t stream) {
    if (!fits_int(out_dim) || !fits_int(in_dim)) return hipErrorInvalidValue;
    const int k = (int)in_dim, n = (int)out_dim;
    switch (meta->wtype) {
    case RF_GGML_Q4_K:
        // Q8-inline activation path first, when enabled and its LDS image
        // fits; any error falls through to the next arm
        if (q8_fastpath_enabled() && q4_k_q8_inline_fits(in_dim)) {
            if (g_table.gemv_q4_k_q8_inline(w, x, y, k, n, stream) == hipSuccess) return RF_DISPATCH_OK;
        }
        // (the reference's opt-in vulkan-style GEMV, ops.rs:413-427, lives
        // outside this library and is not routed here)
        return (int)g_table.gemv_q4_k_f32(w, x, y, k, n, stream);
    case RF_GGML_Q6_K:
        return (int)g_table.gemv_q6_k_f32(w, x, y, k, n, stream);
    default:
        return RF_DISPATCH_NOT_IN_LIBRARY;
    }
}

}  // namespace

extern "C" {

void rf_dispatch_refresh_flags(void) {   // refresh_runtime_env_flags (safety.rs:123)
    g_safe_mode.reset();
    g_q8_fastpath.reset();
    g_disable_wmma_prefill.reset();
}

int rf_dispatch_parse_env_flag(const char* value, int dflt) { return parse_env_flag(value, dflt != 0) ? 1 : 0; }

void rf_dispatch_set_launchers(const rf_launchers* table) { g_table = table ? *table : g_default; }

int rf_gpu_dispatch_gemv(const void* weights, const rf_weight_meta* meta, const float* input, float* output,
                         size_t out_dim, size_t in_dim, hipStream_t stream) {
    if (!layout_ok(meta, out_dim, in_dim)) return RF_DISPATCH_INVALID_LAYOUT;
    if (!supports_gemv_type(meta->wtype)) return RF_DISPATCH_UNSUPPORTED_TYPE;
    return gemv_impl(weights, meta, input, output, out_dim, in_dim, stream);
}

int rf_gpu_dispatch_gemv_residual(const void* weights, const rf_weight_meta* meta, const float* input,
                                  const float* residual, float* output, size_t in_dim, size_t out_dim,
                                  hipStream_t stream, int* dispatched) {
    if (dispatched) *dispatched = 0;
    if (meta == nullptr) return RF_DISPATCH_INVALID_LAYOUT;
    if (!fits_int(out_dim) || !fits_int(in_dim)) return hipErrorInvalidValue;
    const int k = (int)in_dim, n = (int)out_dim;
    switch (meta->wtype) {
    case RF_GGML_Q4_K: {   // ops.rs:666-695
        if (q8_fastpath_enabled() && q4_k_q8_inline_fits(in_dim)) {
            if (g_table.gemv_q4_k_q8_inline_residual(weights, input, residual, output, k, n, stream) == hipSuccess) {
                if (dispatched) *dispatched = 1;
                return RF_DISPATCH_OK;
            }
        }
        const int rc = (int)g_table.gemv_q4_k_f32_residual(weights, input, residual, output, k, n, stream);
        if (rc == hipSuccess && dispatched) *dispatched = 1;
        return rc;
    }
    case RF_GGML_Q4_0:
    case RF_GGML_Q4_1:
        return RF_DISPATCH_NOT_IN_LIBRARY;   // residual kernels of other formats
    default:
        return RF_DISPATCH_OK;               // Ok(false): the caller falls back to GEMV + add
    }
}

int rf_gpu_dispatch_fused_gate_up(const void* w_gate, const rf_weight_meta* gate_meta, const void* w_up,
                                  const rf_weight_meta* up_meta, const float* input, float* output, size_t ff_size,
                                  size_t h, hipStream_t stream) {
    if (gate_meta == nullptr || up_meta == nullptr) return RF_DISPATCH_INVALID_LAYOUT;
    if (gate_meta->wtype != RF_GGML_Q4_K || up_meta->wtype != RF_GGML_Q4_K) return RF_DISPATCH_NOT_IN_LIBRARY;
    if (!layout_ok(gate_meta, ff_size, h) || !layout_ok(up_meta, ff_size, h)) return RF_DISPATCH_INVALID_LAYOUT;
    if (!fits_int(ff_size) || !fits_int(h)) return hipErrorInvalidValue;
    const int k = (int)h, n = (int)ff_size;
    if (q8_fastpath_enabled() && q4_k_q8_inline_fits(h)) {
        if (g_table.gemv_gate_up_q4_k_q8_inline(w_gate, w_up, input, output, k, n, stream) == hipSuccess)
            return RF_DISPATCH_OK;
    }
    return (int)g_table.gemv_gate_up_q4_k_f32(w_gate, w_up, input, output, k, n, stream);
}

int rf_gpu_dispatch_fused_qkv(const void* w_q, const rf_weight_meta* q_meta, const float* q_bias, const void* w_k,
                              const rf_weight_meta* k_meta, const float* k_bias, const void* w_v,
                              const rf_weight_meta* v_meta, const float* v_bias, const float* input, float* out_q,
                              float* out_k, float* out_v, size_t q_size, size_t kv_size, size_t h,
                              hipStream_t stream) {
    if (q_meta == nullptr || k_meta == nullptr || v_meta == nullptr) return RF_DISPATCH_INVALID_LAYOUT;
    if (!fits_int(q_size) || !fits_int(kv_size) || !fits_int(h) || !fits_int(q_size + 2 * kv_size))
        return hipErrorInvalidValue;
    // fused arm (the reference's is Q4_0-only, ops.rs:768-847; this library
    // fuses Q4_K): all three Q4_K, Q8 fast path on, LDS image fits
    if (q_meta->wtype == RF_GGML_Q4_K && k_meta->wtype == RF_GGML_Q4_K && v_meta->wtype == RF_GGML_Q4_K &&
        q8_fastpath_enabled() && q4_k_q8_inline_fits(h) && layout_ok(q_meta, q_size, h) &&
        layout_ok(k_meta, kv_size, h) && layout_ok(v_meta, kv_size, h)) {
        if (g_table.gemv_qkv_q4_k_q8_inline(w_q, w_k, w_v, q_bias, k_bias, v_bias, input, out_q, out_k, out_v, (int)h,
                                            (int)q_size, (int)kv_size, stream) == hipSuccess)
            return RF_DISPATCH_OK;
    }
    // individual dispatches (ops.rs:851-853); the reference then adds the
    // biases with an elementwise kernel that is not part of this library
    if (q_bias != nullptr || k_bias != nullptr || v_bias != nullptr) return RF_DISPATCH_NOT_IN_LIBRARY;
    int rc = rf_gpu_dispatch_gemv(w_q, q_meta, input, out_q, q_size, h, stream);
    if (rc != RF_DISPATCH_OK) return rc;
    rc = rf_gpu_dispatch_gemv(w_k, k_meta, input, out_k, kv_size, h, stream);
    if (rc != RF_DISPATCH_OK) return rc;
    return rf_gpu_dispatch_gemv(w_v, v_meta, input, out_v, kv_size, h, stream);
}

int rf_gpu_dispatch_gemm(const void* weights, const rf_weight_meta* meta, const float* input, float* output,
                         size_t out_dim, size_t in_dim, size_t seq_len) {
    if (meta == nullptr) return RF_DISPATCH_INVALID_LAYOUT;
    hipStream_t null_stream = nullptr;   // gpu_dispatch_gemm launches on the null stream
    // decode: one row is a GEMV (ops.rs:1601-1611)
    if (seq_len == 1 && supports_gemv_type(meta->wtype))
        return rf_gpu_dispatch_gemv(weights, meta, input, output, out_dim, in_dim, null_stream);
    if (!fits_int(out_dim) || !fits_int(in_dim) || !fits_int(seq_len + 63)) return hipErrorInvalidValue;
    // WMMA prefill arms (ops.rs:1665-1755): M padded up to a multiple of 64;
    // the prefill scratch is sized and zeroed for the padded rows
    // (cache.rs:781-834).  A failure falls through to the next arm.
    if (seq_len >= 1 && (meta->wtype == RF_GGML_Q4_K || meta->wtype == RF_GGML_Q6_K) && out_dim % 64 == 0 &&
        in_dim % 256 == 0 && wmma_prefill_enabled()) {
        const int padded_m = (int)((seq_len + 63) / 64 * 64);
        const hipError_t rc = meta->wtype == RF_GGML_Q4_K
                                  ? g_table.wmma_gemm_q4_k(input, weights, output, padded_m, (int)out_dim, (int)in_dim,
                                                           null_stream)
                                  : g_table.wmma_gemm_q6_k(input, weights, output, padded_m, (int)out_dim, (int)in_dim,
                                                           null_stream);
        if (rc == hipSuccess) return RF_DISPATCH_OK;
    }
    // small batches: one GEMV per row (ops.rs:1884-1891)
    if (seq_len <= 8 && supports_gemv_type(meta->wtype)) {
        for (size_t r = 0; r < seq_len; ++r) {
            const int rc = rf_gpu_dispatch_gemv(weights, meta, input + r * in_dim, output + r * out_dim, out_dim,
                                                in_dim, null_stream);
            if (rc != RF_DISPATCH_OK) return rc;
        }
        return RF_DISPATCH_OK;
    }
    switch (meta->wtype) {
    case RF_GGML_Q6_K:   // Q6_K GEMV loop (ops.rs:1935-1963)
        for (size_t r = 0; r < seq_len; ++r) {
            const int rc = (int)g_table.gemv_q6_k_f32(weights, input + r * in_dim, output + r * out_dim, (int)in_dim,
                                                      (int)out_dim, null_stream);
            if (rc != hipSuccess) return rc;
        }
        return RF_DISPATCH_OK;
    case RF_GGML_Q4_0:
    case RF_GGML_Q4_1:
    case RF_GGML_Q8_0:
    case RF_GGML_Q4_K:   // scalar gemm_q4_k_f32 (ops.rs:1924)
    case RF_GGML_Q5_K:
        return RF_DISPATCH_NOT_IN_LIBRARY;
    default:
        return RF_DISPATCH_UNSUPPORTED_TYPE;
    }
}

}  // extern "C"
