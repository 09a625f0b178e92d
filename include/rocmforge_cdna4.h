/*
 * rocmforge_cdna4.h -- C ABI of librocmforge_cdna4.so, the MI355X (gfx950)
 * implementation of ROCmForge's Q4_K / Q6_K matmul hot path.
 *
 * The launcher symbols, argument order/meaning and error codes are those the
 * ROCmForge Rust host already binds (src/gpu/kernels/quant.rs:2115-2196 and
 * src/gpu/kernels/wmma.rs:65-83), so the library is link-compatible with it.
 *
 * Conventions shared by every launcher:
 *   - n_rows = K = input length (multiple of 256), ncols_dst = N = output rows.
 *   - Weights are raw GGUF bytes, row-major: row n owns K/256 consecutive
 *     super-blocks (144 B for Q4_K, 210 B for Q6_K).
 *   - All pointers are caller-owned device memory.  Launchers enqueue on
 *     `stream`, never allocate, free or synchronise (safe under hipGraph
 *     stream capture), and return hipErrorInvalidValue on a rejected shape
 *     or pointer, otherwise hipGetLastError() after the launch.
 *   - Alignment (an addition to the reference checks, returned as
 *     hipErrorInvalidValue): Q4_K weights 16-byte aligned, Q6_K weights
 *     2-byte aligned, fp32 vectors/matrices 16-byte aligned.  hipMalloc
 *     buffers satisfy all of these.
 */
#ifndef ROCMFORGE_CDNA4_H
#define ROCMFORGE_CDNA4_H

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- Q4_K decode GEMV, activations quantised inline to Q8_0 -------------
 * Replaces hip_kernels/quant/q4_k_q8_inline.hip:380 (Rust decl
 * src/gpu/kernels/quant.rs:2115-2196).  y[n] = sum_k W[n,k] * x[k] with x
 * quantised per 32 elements to Q8_0 (bit-exact to the reference quantiser)
 * and integer nibble x int8 dots.  Rejects K with (K/32)*34 > 32768 like the
 * reference (q4_k_q8_inline.hip:374-378). */
hipError_t gemv_q4_k_f32_q8_inline_launch(const void* weights_q4_k, const float* input, float* output,
                                          int n_rows, int ncols_dst, hipStream_t stream);

/* q4_k_q8_inline.hip:404 -- output[n] = y[n] + residual[n]; output may alias
 * residual (in-place residual add); residual must be non-null. */
hipError_t gemv_q4_k_f32_q8_inline_residual_launch(const void* weights_q4_k, const float* input,
                                                   const float* residual, float* output, int n_rows,
                                                   int ncols_dst, hipStream_t stream);

/* q4_k_q8_inline.hip:429 -- swiglu_out[n] = silu(gate[n]) * up[n] with gate
 * and up the two Q4_K GEMVs of one shared Q8 activation vector;
 * silu(g) = g / (1 + exp(-g)).  swiglu_out must not alias the inputs. */
hipError_t gemv_gate_up_swiglu_q4_k_f32_q8_inline_launch(const void* weights_gate_q4_k,
                                                         const void* weights_up_q4_k, const float* input,
                                                         float* swiglu_out, int n_rows, int ncols_dst,
                                                         hipStream_t stream);

/* ---- Q4_K decode GEMV, fp32 activations (fallback family) --------------
 * hip_kernels/quant/q4_k_gemv.hip:517 / :548 / :480 -- same outputs as the
 * three launchers above but with fp32 x (no activation quantisation); no
 * LDS-fit limit on K. */
hipError_t gemv_q4_k_f32_launch(const void* weights_q4_k, const float* input, float* output, int n_rows,
                                int ncols_dst, hipStream_t stream);
hipError_t gemv_q4_k_f32_residual_launch(const void* weights_q4_k, const float* input, const float* residual,
                                         float* output, int n_rows, int ncols_dst, hipStream_t stream);
hipError_t gemv_gate_up_swiglu_q4_k_f32_launch(const void* weights_gate_q4_k, const void* weights_up_q4_k,
                                               const float* input, float* swiglu_out, int n_rows,
                                               int ncols_dst, hipStream_t stream);

/* ---- Q6_K decode GEMV, fp32 activations --------------------------------
 * hip_kernels/quant/q6_k_gemv.hip:276 (Rust decl quant.rs:2115-2196,
 * wrapper gemv_q6_k_f32_on_stream quant.rs:3737). */
hipError_t gemv_q6_k_f32_launch(const void* weights_q6_k, const float* input, float* output, int n_rows,
                                int ncols_dst, hipStream_t stream);

/* ---- Prefill GEMM, dequant-in-register, fp16 MFMA, fp32 accumulate ------
 * hip_kernels/wmma/wmma_gemm_q4_k.hip:506 and wmma_gemm_q6_k.hip:212 (Rust
 * decl src/gpu/kernels/wmma.rs:65-83).  NOTE the argument order: input
 * first.  D[M x N] = fp16(A[M x K]) * fp16(dequant W[N x K])^T, fp32 out.
 * M % 64 == 0, N % 64 == 0, K % 256 == 0 (callers pad M to 64 rows). */
hipError_t wmma_gemm_q4_k_launch(const float* input, const void* weights_q4_k, float* output, int M, int N, int K,
                                 hipStream_t stream);
hipError_t wmma_gemm_q6_k_launch(const float* input, const void* weights_q6_k, float* output, int M, int N, int K,
                                 hipStream_t stream);

/* ---- Parity probes (no reference counterpart) ---------------------------
 * Expose the intermediate integers of the Q8-inline path so tests can check
 * them bit-exactly.  They run the same device code as the GEMV. */

/* Q8_0 quantisation of input[n] (n % 32 == 0): d_out[n/32] fp16 bits,
 * qs_out[n] int8, sum_out[n/32] = sum of each block's 32 int8. */
hipError_t rf_q8_0_quantize_launch(const float* input, uint16_t* d_out, int8_t* qs_out, int32_t* sum_out, int n,
                                   hipStream_t stream);

/* int_dot[n*(K/32) + j] = sum_i nib(W[n], 32j+i) * q8(x)[32j+i] for every
 * output row n and 32-element sub-block j. */
hipError_t rf_q4_k_q8_int_dots_launch(const void* weights_q4_k, const float* input, int32_t* int_dot, int n_rows,
                                      int ncols_dst, hipStream_t stream);

/* Library identification string. */
const char* rf_library_version(void);

#ifdef __cplusplus
}
#endif

#endif /* ROCMFORGE_CDNA4_H */
