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
#include <stddef.h>
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

/* Fused Q/K/V projection over three Q4_K matrices sharing one quantised
 * activation vector: out_q[i] = Wq[i,:]·x + bias_q[i] (i < n_q), likewise
 * out_k / out_v over n_kv rows; each bias may be null.  No Q4_K counterpart
 * in the reference (its Q4_K_M attention input is three GEMV launches,
 * src/gpu/ops.rs:851-853); signature and bias semantics follow its Q4_0
 * fused launcher gemv_qkv_q4_0_f32_launch (hip_kernels/quant/
 * q4_0_fused.hip:674).  Same K limits and alignment as the launcher above. */
hipError_t gemv_qkv_q4_k_f32_q8_inline_launch(const void* w_q, const void* w_k, const void* w_v,
                                              const float* bias_q, const float* bias_k, const float* bias_v,
                                              const float* input, float* out_q, float* out_k, float* out_v,
                                              int n_rows, int n_q, int n_kv, hipStream_t stream);

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

/* output[n] = y[n] + residual[n] for the Q6_K GEMV above; output may alias
 * residual.  No counterpart in the reference (its Q6_K ffn_down runs a GEMV
 * and a separate add: gpu_dispatch_gemv_residual_on_stream returns
 * Ok(false) for Q6_K, src/gpu/ops.rs:666-695); arguments and checks follow
 * gemv_q4_k_f32_q8_inline_residual_launch. */
hipError_t gemv_q6_k_f32_residual_launch(const void* weights_q6_k, const float* input, const float* residual,
                                         float* output, int n_rows, int ncols_dst, hipStream_t stream);

/* ---- Prefill GEMM, dequant-in-register, fp16 MFMA, fp32 accumulate ------
 * hip_kernels/wmma/wmma_gemm_q4_k.hip:201 and wmma_gemm_q6_k.hip:212 (Rust
 * decl src/gpu/kernels/wmma.rs:65-83).  NOTE the argument order: input
 * first.  D[M x N] = fp16(A[M x K]) * fp16(dequant W[N x K])^T, fp32 out.
 * M % 64 == 0, N % 64 == 0, K % 256 == 0 (callers pad M to 64 rows).
 * A is rounded to fp16 (__float2half's value) by a pass of its own into
 * library-owned device memory (a file-scope array: 4 slots of 56 MB per GPU,
 * one per stream, claimed on a stream's first launch) and the fp16
 * tiles of rf_gemm_q*_k_f16_launch run on it; small launches split K over
 * workgroups and add the partial tiles in a fixed order, so every output is
 * the same sum on every run.  Launches on one stream share its slot (stream
 * order); a stream without one takes a free slot or, outside stream
 * capture, the slot of an idle stream (hipStreamQuery), else the
 * fp32-activation tiles run (same values up to summation order).  A stream
 * that will be captured should launch a GEMM once before its capture, so
 * that it holds a slot.  Q6_K takes the fp16 tiles when
 * K % 2048 == 0 and the weights are 16-byte aligned. */
hipError_t wmma_gemm_q4_k_launch(const float* input, const void* weights_q4_k, float* output, int M, int N, int K,
                                 hipStream_t stream);
hipError_t wmma_gemm_q6_k_launch(const float* input, const void* weights_q6_k, float* output, int M, int N, int K,
                                 hipStream_t stream);

/* No counterpart (the reference converts A with __float2half inside its
 * GEMM, wmma_gemm_q4_k.hip:80-87): the Q4_K GEMM on fp16 activations, for a
 * caller whose producing kernel already rounded A to fp16 (bit patterns as
 * uint16_t, row-major [M][K]).  Same operand values as
 * wmma_gemm_q4_k_launch(fp32 A), so the same products; A is read at half
 * the bytes and not converted.  256 x 128 tiles where they fill three
 * quarters of the CUs (M = 512 at N = 14336; they need N % 128 == 0), else
 * 64- or 128-row x 64-column tiles with K split over the waves of a
 * workgroup, and over workgroups (partials in the stream's slot, added in
 * split order) when the tiles leave half the CUs idle.  M % 64 == 0,
 * N % 64 == 0, K % 256 == 0, input and weights 16-byte aligned. */
hipError_t rf_gemm_q4_k_f16_launch(const uint16_t* input_f16, const void* weights_q4_k, float* output, int M, int N,
                                   int K, hipStream_t stream);

/* No counterpart (the reference converts A with __float2half inside its
 * GEMM, wmma_gemm_q6_k.hip:93-100): the Q6_K GEMM on fp16 activations, same
 * contract as rf_gemm_q4_k_f16_launch -- the operand values of
 * wmma_gemm_q6_k_launch(fp32 A).  128 x 64 tiles with K split over the
 * waves of a workgroup (one tile per CU at M = 512, N = 4096), and over
 * workgroups as rf_gemm_q4_k_f16_launch when the tiles leave half the CUs
 * idle.  M % 64 == 0, N % 64 == 0, K % 2048 == 0, input, weights and output
 * 16-byte aligned. */
hipError_t rf_gemm_q6_k_f16_launch(const uint16_t* input_f16, const void* weights_q6_k, float* output, int M, int N,
                                   int K, hipStream_t stream);
/* No counterpart: inout[M x N] += the product of rf_gemm_q4_k_f16_launch, each
 * output read and written once after its fp32 sum (inout + that product bit
 * for bit).  M % 64 == 0, N % 64 == 0, K % 256 == 0, input and weights 16-byte
 * aligned.  Used for the O and FFN-down projections of a prefill. */
hipError_t rf_gemm_q4_k_f16_accumulate_launch(const uint16_t* input_f16, const void* weights_q4_k, float* inout,
                                              int M, int N, int K, hipStream_t stream);
/* Up to three weight matrices over one fp16 input as column segments of one
 * launch, each Q4_K (type 12) or Q6_K (type 14, GGML type ids):
 * out_s[M x n_s] = the product of rf_gemm_q4_k_f16_launch /
 * rf_gemm_q6_k_f16_launch on K-sliced 64-column tiles of 128 or 256 rows
 * (each output written once, the bits of those launchers).  The
 * prefill Q/K/V of a layer of any type mix (the reference runs three GEMMs,
 * src/gpu/forward.rs:2327).  M % 64, n_s % 64 (n1, n2 may be 0), K % 256
 * (K % 2048 with a Q6_K segment); input, weights and outputs 16-byte aligned. */
hipError_t rf_gemm_qk_f16_segments_launch(const uint16_t* input_f16, const void* w0, const void* w1, const void* w2,
                                          int type0, int type1, int type2, float* out0, float* out1, float* out2,
                                          int M, int n0, int n1, int n2, int K, hipStream_t stream);
/* Gate and up on fp16 activations in one launch, SwiGLU in the epilogue:
 * out[M x N] = silu(A Wg^T) * (A Wu^T) as fp32, or rounded to fp16 when
 * out_f16 != 0 -- the values of two rf_gemm_q4_k_f16_launch calls followed
 * by rf_silu_mul(_f16)_on_stream.  The reference runs two GEMMs and a SwiGLU
 * kernel (src/gpu/forward.rs:2327).  M % 64, N % 64, K % 256; input and
 * weights 16-byte aligned. */
hipError_t rf_gemm_q4_k_f16_swiglu_launch(const uint16_t* input_f16, const void* w_gate, const void* w_up, void* out,
                                          int out_f16, int M, int N, int K, hipStream_t stream);
/* The up projection of a SwiGLU on fp16 activations with the gate product
 * gate[M x N] (fp32, e.g. from rf_gemm_q4_k_f16_launch on the gate weights)
 * already computed: out_f16[M x N] = fp16(silu(gate) * (A Wu^T)), the
 * values of rf_gemm_q4_k_f16_launch on w_up followed by
 * rf_silu_mul_f16_on_stream, with the SwiGLU in the GEMM's store (the
 * reference runs the GEMM and a SwiGLU kernel, src/gpu/forward.rs:2327).
 * Shapes as rf_gemm_q4_k_f16_launch; gate and out_f16 16-byte aligned and
 * not overlapping. */
hipError_t rf_gemm_q4_k_f16_swiglu_up_launch(const uint16_t* input_f16, const void* w_up, const float* gate,
                                             uint16_t* out_f16, int M, int N, int K, hipStream_t stream);
/* No counterpart: inout[M x N] += the product of rf_gemm_q6_k_f16_launch (the
 * reference's prefill adds residuals with gpu_add).  Each output is read and
 * written once after its fp32 sum, so the result is inout + that launch's
 * output bit for bit.  Same shape rules.  Used for the FFN down projection of
 * a prefill, into the residual stream. */
hipError_t rf_gemm_q6_k_f16_accumulate_launch(const uint16_t* input_f16, const void* weights_q6_k, float* inout,
                                              int M, int N, int K, hipStream_t stream);
/* No counterpart (the reference's prefill adds the residual with gpu_add and
 * normalises the next layer's input in its own kernel).  The accumulate
 * launchers above, then rf_rms_norm_batched_f16_on_stream of inout (rows of
 * N, weights norm_w, eps) into out_f16 [M x N]: inout and out_f16 have the
 * bits of those two calls.  When the GEMM splits over K the norm is taken in
 * the split reduction's pass over the rows (N % 2048 == 0, N <= 8192).  Same
 * shape rules as the accumulate launchers; norm_w and out_f16 16-byte aligned,
 * out_f16 not overlapping inout.  Used for the FFN down projection of a
 * prefill layer followed by the next layer's attention norm. */
hipError_t rf_gemm_q4_k_f16_accumulate_rmsnorm_launch(const uint16_t* input_f16, const void* weights_q4_k,
                                                      float* inout, const float* norm_w, float eps, uint16_t* out_f16,
                                                      int M, int N, int K, hipStream_t stream);
hipError_t rf_gemm_q6_k_f16_accumulate_rmsnorm_launch(const uint16_t* input_f16, const void* weights_q6_k,
                                                      float* inout, const float* norm_w, float eps, uint16_t* out_f16,
                                                      int M, int N, int K, hipStream_t stream);

/* No counterpart in the reference (its prefill issues one GEMM per weight
 * and adds residuals with gpu_add).  Several weight matrices that share the
 * input and K in one launch: out_i[M x n_i] = fp16(A) * fp16(dequant W_i)^T
 * for i = 0..2, each output row-major with width n_i (n1 = 0 and n2 = 0
 * drop segments; all n_i % 256 == 0).  The per-element arithmetic is the
 * single GEMM's.  K % 512 == 0 (Q6_K: K % 2048 == 0), M % 64 == 0, A and
 * outputs 16-byte aligned.  A is staged as fp16 as for wmma_gemm_q4_k_launch
 * and rf_gemm_qk_f16_segments_launch runs on it.  Used for the Q/K/V
 * projections of a prefill. */
hipError_t rf_gemm_q4_k_segments_launch(const float* input, const void* w0, const void* w1, const void* w2,
                                        float* out0, float* out1, float* out2, int M, int n0, int n1, int n2, int K,
                                        hipStream_t stream);
hipError_t rf_gemm_q6_k_segments_launch(const float* input, const void* w0, const void* w1, const void* w2,
                                        float* out0, float* out1, float* out2, int M, int n0, int n1, int n2, int K,
                                        hipStream_t stream);
/* No counterpart in the reference.  inout[M x N] += fp16(A) * fp16(dequant
 * W)^T: the O and FFN-down projections of a prefill add straight into the
 * residual stream.  N % 256 == 0, other rules as the segment launchers. */
hipError_t rf_gemm_q4_k_accumulate_launch(const float* input, const void* weights_q4_k, float* inout, int M, int N,
                                          int K, hipStream_t stream);
hipError_t rf_gemm_q6_k_accumulate_launch(const float* input, const void* weights_q6_k, float* inout, int M, int N,
                                          int K, hipStream_t stream);
/* No counterpart in the reference (its prefill runs the gate and up GEMMs
 * and then a SwiGLU kernel).  out[M x N] = silu(fp16(A) fp16(Wg)^T) *
 * (fp16(A) fp16(Wu)^T), silu(g) = g / (1 + exp(-g)), with both products
 * summed in one launch (no K split).  N % 128 == 0, other rules as the
 * segment launchers. */
hipError_t rf_gemm_q4_k_swiglu_launch(const float* input, const void* w_gate, const void* w_up, float* out, int M,
                                      int N, int K, hipStream_t stream);
hipError_t rf_gemm_q6_k_swiglu_launch(const float* input, const void* w_gate, const void* w_up, float* out, int M,
                                      int N, int K, hipStream_t stream);
/* The same paired launches with the output rounded to fp16 (round to nearest
 * even, bit patterns as uint16_t): out_f16[M x N] = __float2half(silu(gate) *
 * up) of the fp32 launchers' values -- the operand values the reference's
 * down-projection GEMM makes from fp32 with __float2half, ready for
 * rf_gemm_q6_k_f16_accumulate_launch. */
hipError_t rf_gemm_q4_k_swiglu_f16_launch(const float* input, const void* w_gate, const void* w_up, uint16_t* out_f16,
                                          int M, int N, int K, hipStream_t stream);
hipError_t rf_gemm_q6_k_swiglu_f16_launch(const float* input, const void* w_gate, const void* w_up, uint16_t* out_f16,
                                          int M, int N, int K, hipStream_t stream);

/* ---- Host dispatch (routing of the arms above) --------------------------
 * C counterparts of ROCmForge's src/gpu/ops.rs routing for the Q4_K / Q6_K
 * arms: which launcher a GGUF weight tensor goes to, in which order the
 * paths are tried, and the shape checks made before any launch.  They call
 * the launchers above and allocate nothing.
 *
 * Return value: RF_DISPATCH_OK (0) on success; a hipError_t (> 0) from the
 * last launcher tried; or one of the negative codes below:
 *   RF_DISPATCH_INVALID_LAYOUT   -- GpuError::InvalidWeightLayout
 *                                   (validate_gemv_layout, ops.rs:82-105)
 *   RF_DISPATCH_UNSUPPORTED_TYPE -- GpuError::UnsupportedWeightType
 *   RF_DISPATCH_NOT_IN_LIBRARY   -- an arm the reference serves with a
 *                                   kernel outside this library (Q4_0, Q4_1,
 *                                   Q8_0, Q5_K, the scalar Q4_K GEMM, the
 *                                   unfused gate/up path): the caller keeps
 *                                   its own route for it.
 * Runtime flags (read once, cached; rf_dispatch_refresh_flags re-reads
 * them, as refresh_runtime_env_flags, safety.rs:123):
 *   ROCMFORGE_GPU_SAFE_MODE (default off) disables both fast paths,
 *   ROCMFORGE_ENABLE_EXPERIMENTAL_Q8_ACTIVATION_FASTPATH (default on),
 *   ROCMFORGE_DISABLE_WMMA_PREFILL (default off).
 * Values "1", "true", "yes", "on" (any case) enable a flag. */
enum {
    RF_GGML_F32 = 0, RF_GGML_F16 = 1, RF_GGML_Q4_0 = 2, RF_GGML_Q4_1 = 3, RF_GGML_Q5_0 = 6, RF_GGML_Q5_1 = 7,
    RF_GGML_Q8_0 = 8, RF_GGML_Q2_K = 10, RF_GGML_Q3_K = 11, RF_GGML_Q4_K = 12, RF_GGML_Q5_K = 13, RF_GGML_Q6_K = 14
};  /* GgmlType codes (src/loader/ggml_type.rs:6-19) */

enum { RF_DISPATCH_OK = 0, RF_DISPATCH_INVALID_LAYOUT = -1001, RF_DISPATCH_UNSUPPORTED_TYPE = -1002,
       RF_DISPATCH_NOT_IN_LIBRARY = -1003 };

/* WeightMeta (src/gpu/weights.rs:29-40): GGUF type code and dims (innermost
 * first); role 0 generic, 1 lm_head, 2 tied lm_head. */
typedef struct rf_weight_meta {
    int32_t wtype;
    int32_t n_dims;
    uint64_t dims[4];
    int32_t role;
} rf_weight_meta;

/* gpu_dispatch_gemv_on_stream (ops.rs:484) + dispatch_gemv_impl (ops.rs:270):
 * Q4_K -> Q8-inline GEMV when the fast path is on and (K/32)*34 <= 32 KB, on
 * any error the fp32-activation GEMV; Q6_K -> gemv_q6_k_f32_launch. */
int rf_gpu_dispatch_gemv(const void* weights, const rf_weight_meta* meta, const float* input, float* output,
                         size_t out_dim, size_t in_dim, hipStream_t stream);

/* gpu_dispatch_gemv_residual_on_stream (ops.rs:509, note the argument
 * order: in_dim before out_dim).  *dispatched = 1 when a residual kernel ran
 * (Q4_K: Q8-inline first, then fp32); 0 with RF_DISPATCH_OK for types
 * without a residual kernel (the reference's Ok(false): GEMV + add). */
int rf_gpu_dispatch_gemv_residual(const void* weights, const rf_weight_meta* meta, const float* input,
                                  const float* residual, float* output, size_t in_dim, size_t out_dim,
                                  hipStream_t stream, int* dispatched);

/* The Q4_K arm of gpu_dispatch_fused_gate_up_with_scratch_on_stream
 * (ops.rs:1316-1355): both layouts validated, Q8-inline fused kernel first,
 * then the fp32 fused kernel. */
int rf_gpu_dispatch_fused_gate_up(const void* w_gate, const rf_weight_meta* gate_meta, const void* w_up,
                                  const rf_weight_meta* up_meta, const float* input, float* output, size_t ff_size,
                                  size_t h, hipStream_t stream);

/* gpu_dispatch_fused_qkv_on_stream (ops.rs:748): three Q4_K matrices with
 * the Q8 fast path on and (h/32)*34 <= 32 KB -> one fused launch
 * (gemv_qkv_q4_k_f32_q8_inline_launch, biases folded in; the reference
 * fuses only Q4_0 here); otherwise, or on its error, three
 * rf_gpu_dispatch_gemv calls (ops.rs:851-853) -- with a non-null bias that
 * route returns RF_DISPATCH_NOT_IN_LIBRARY (its bias add is an elementwise
 * kernel outside this library). */
int rf_gpu_dispatch_fused_qkv(const void* w_q, const rf_weight_meta* q_meta, const float* q_bias, const void* w_k,
                              const rf_weight_meta* k_meta, const float* k_bias, const void* w_v,
                              const rf_weight_meta* v_meta, const float* v_bias, const float* input, float* out_q,
                              float* out_k, float* out_v, size_t q_size, size_t kv_size, size_t h,
                              hipStream_t stream);

/* gpu_dispatch_gemm (ops.rs:1591), null stream as in the reference:
 * seq_len == 1 -> GEMV; Q4_K / Q6_K with out_dim % 64 == 0, in_dim % 256 == 0
 * -> WMMA-equivalent GEMM at padded_m = round_up(seq_len, 64) (input and
 * output must hold padded_m rows, the extra ones zero); on failure
 * seq_len <= 8 -> one GEMV per row; Q6_K -> one Q6_K GEMV per row. */
int rf_gpu_dispatch_gemm(const void* weights, const rf_weight_meta* meta, const float* input, float* output,
                         size_t out_dim, size_t in_dim, size_t seq_len);

/* Re-read the cached runtime flags. */
void rf_dispatch_refresh_flags(void);

/* The flag parser itself (1 = enabled), for tests. */
int rf_dispatch_parse_env_flag(const char* value, int dflt);

/* Launcher table used by the dispatch functions (default: this library's
 * launchers).  Passing NULL restores the default.  Tests install recording
 * stand-ins to check the routing without a GPU; not thread-safe against
 * concurrent dispatch. */
typedef struct rf_launchers {
    hipError_t (*gemv_q4_k_q8_inline)(const void*, const float*, float*, int, int, hipStream_t);
    hipError_t (*gemv_q4_k_q8_inline_residual)(const void*, const float*, const float*, float*, int, int,
                                               hipStream_t);
    hipError_t (*gemv_gate_up_q4_k_q8_inline)(const void*, const void*, const float*, float*, int, int, hipStream_t);
    hipError_t (*gemv_q4_k_f32)(const void*, const float*, float*, int, int, hipStream_t);
    hipError_t (*gemv_q4_k_f32_residual)(const void*, const float*, const float*, float*, int, int, hipStream_t);
    hipError_t (*gemv_gate_up_q4_k_f32)(const void*, const void*, const float*, float*, int, int, hipStream_t);
    hipError_t (*gemv_q6_k_f32)(const void*, const float*, float*, int, int, hipStream_t);
    hipError_t (*wmma_gemm_q4_k)(const float*, const void*, float*, int, int, int, hipStream_t);
    hipError_t (*wmma_gemm_q6_k)(const float*, const void*, float*, int, int, int, hipStream_t);
    hipError_t (*gemv_qkv_q4_k_q8_inline)(const void*, const void*, const void*, const float*, const float*,
                                          const float*, const float*, float*, float*, float*, int, int, int,
                                          hipStream_t);
} rf_launchers;
void rf_dispatch_set_launchers(const rf_launchers* table);

/* ---- Layer operations around the matmuls (model_ops.hip) ---------------
 * Same names, argument order and meaning as the reference's launchers;
 * KV caches are fp16 [max_seq][num_kv_heads * head_dim] per layer.  The
 * *_state variants read the position / sequence length from device memory
 * (decode state int[2] = {pos, seq_len}), so a captured graph replays them. */

/* hip_kernels/norm.hip:154 -- out = x * rsqrt(mean(x^2) + eps) * w; out may alias x. */
hipError_t gpu_rms_norm(const float* d_x, const float* d_weight, float* d_out, const int n, const float eps,
                        hipStream_t stream);
/* hip_kernels/norm.hip:173, :184 -- seq_len rows of n (also the per-head Q/K norms). */
hipError_t gpu_rms_norm_batched(const float* d_x, const float* d_weight, float* d_out, const int n, const float eps,
                                const int seq_len);
hipError_t gpu_rms_norm_batched_on_stream(const float* d_x, const float* d_weight, float* d_out, const int n,
                                          const float eps, const int seq_len, hipStream_t stream);
/* No counterpart: the batched norm with its output rounded to fp16 (round to
 * nearest even, bit patterns as uint16_t) -- the operand values a prefill
 * GEMM on fp16 activations (rf_gemm_q4_k_f16_launch) reads, identical to the
 * fp32 GEMM's own __float2half of gpu_rms_norm_batched_on_stream's output. */
hipError_t rf_rms_norm_batched_f16_on_stream(const float* d_x, const float* d_weight, uint16_t* d_out_f16,
                                             const int n, const float eps, const int seq_len, hipStream_t stream);

/* hip_kernels/rope.hip:293-420 -- RoPE over [num_heads][head_dim] in place;
 * neox != 0: pairs (i, i + d/2), else (2i, 2i + 1); freq_scale divides theta_i. */
hipError_t gpu_rope_heads(float* d_x, const int pos, const int num_heads, const int head_dim, const float theta_base,
                          const int neox, hipStream_t stream);
hipError_t gpu_rope_heads_scaled(float* d_x, const int pos, const int num_heads, const int head_dim,
                                 const float theta_base, const int neox, const float* d_freq_scale,
                                 hipStream_t stream);
hipError_t gpu_rope_heads_state(float* d_x, const int* d_pos, const int num_heads, const int head_dim,
                                const float theta_base, const int neox, hipStream_t stream);
hipError_t gpu_rope_heads_state_scaled(float* d_x, const int* d_pos, const int num_heads, const int head_dim,
                                       const float theta_base, const int neox, const float* d_freq_scale,
                                       hipStream_t stream);
/* rows s = 0..seq_len-1 of [seq_len][num_heads * head_dim] at positions start_pos + s (null stream). */
hipError_t gpu_rope_heads_batched(float* d_x, const int start_pos, const int num_heads, const int head_dim,
                                  const float theta_base, const int seq_len, const int neox);
hipError_t gpu_rope_heads_batched_scaled(float* d_x, const int start_pos, const int num_heads, const int head_dim,
                                         const float theta_base, const int seq_len, const int neox,
                                         const float* d_freq_scale);
/* No counterpart: gpu_rope_heads_batched_scaled on a caller's stream. */
hipError_t rf_rope_heads_batched_on_stream(float* d_x, const int start_pos, const int num_heads, const int head_dim,
                                           const float theta_base, const int seq_len, const int neox,
                                           const float* d_freq_scale, hipStream_t stream);

/* hip_kernels/attention.hip:1627-1665 -- V[pos] = fp16(v), K[pos] = fp16(rope(k, pos)). */
hipError_t gpu_kv_write_rope(uint16_t* d_k_cache, uint16_t* d_v_cache, const float* d_k, const float* d_v, const int pos,
                             const int num_kv_heads, const int head_dim, const float theta_base, const int neox,
                             hipStream_t stream);
hipError_t gpu_kv_write_rope_scaled(uint16_t* d_k_cache, uint16_t* d_v_cache, const float* d_k, const float* d_v,
                                    const int pos, const int num_kv_heads, const int head_dim,
                                    const float theta_base, const int neox, const float* d_freq_scale,
                                    hipStream_t stream);
hipError_t gpu_kv_write_rope_state(uint16_t* d_k_cache, uint16_t* d_v_cache, const float* d_k, const float* d_v,
                                   const int* d_pos, const int num_kv_heads, const int head_dim,
                                   const float theta_base, const int neox, hipStream_t stream);
hipError_t gpu_kv_write_rope_state_scaled(uint16_t* d_k_cache, uint16_t* d_v_cache, const float* d_k, const float* d_v,
                                          const int* d_pos, const int num_kv_heads, const int head_dim,
                                          const float theta_base, const int neox, const float* d_freq_scale,
                                          hipStream_t stream);
/* hip_kernels/attention.hip:1667 -- rows [start_pos, start_pos + seq_len) of both caches (null stream);
 * start_pos + seq_len > max_seq is rejected. */
hipError_t gpu_kv_write_batched(uint16_t* d_k_cache, uint16_t* d_v_cache, const float* d_k, const float* d_v,
                                const int start_pos, const int kv_size, const int max_seq, const int seq_len);
/* No counterpart: gpu_kv_write_batched on a caller's stream. */
hipError_t rf_kv_write_batched_on_stream(uint16_t* d_k_cache, uint16_t* d_v_cache, const float* d_k, const float* d_v,
                                         const int start_pos, const int kv_size, const int max_seq,
                                         const int seq_len, hipStream_t stream);

/* No counterpart (the reference takes gpu_rms_norm_batched_on_stream twice,
 * gpu_rope_heads_state_scaled and gpu_kv_write_rope_state_scaled,
 * src/gpu/forward.rs:2384-2430): per-head RMSNorm of q (d_q_norm) and k
 * (d_k_norm; either may be null to skip), RoPE of both at *d_pos, q written
 * back in place, fp16 k and v written to the caches at *d_pos.  head_dim 64, 128 or 256. */
hipError_t rf_qk_norm_rope_kv_write_state(float* d_q, const float* d_k, const float* d_v, const float* d_q_norm,
                                          const float* d_k_norm, uint16_t* d_k_cache, uint16_t* d_v_cache, const int* d_pos,
                                          const int num_heads, const int num_kv_heads, const int head_dim,
                                          const float eps, const float theta_base, const int neox,
                                          const float* d_freq_scale, const float* d_theta, const float* d_cos_sin,
                                          hipStream_t stream);
/* No counterpart (the reference's prefill takes gpu_rms_norm_batched twice,
 * gpu_rope_heads_batched twice, gpu_kv_write_batched and the fp16
 * conversions, src/gpu/forward.rs prefill path): the same step over the rows
 * of a prompt, row r at position start_pos + r.  Query rows [0, rows_q) are
 * written as fp16 to d_q16 ([row][num_heads * head_dim]); key/value rows
 * [0, rows_kv) go to the caches at start_pos + r (start_pos + rows_kv <=
 * max_seq).  d_q, d_k, d_v and d_q16 16-byte aligned; rows_q <= 65535.
 * With d_cos_sin (below) start_pos + rows_q <= max_seq as well. */
hipError_t rf_qk_norm_rope_kv_write_rows(const float* d_q, const float* d_k, const float* d_v, const float* d_q_norm,
                                         const float* d_k_norm, uint16_t* d_q16, uint16_t* d_k_cache,
                                         uint16_t* d_v_cache, const int start_pos, const int rows_q, const int rows_kv,
                                         const int num_heads, const int num_kv_heads, const int head_dim,
                                         const int max_seq, const float eps, const float theta_base, const int neox,
                                         const float* d_freq_scale, const float* d_theta, const float* d_cos_sin,
                                         hipStream_t stream);

/* hip_kernels/attention.hip:950, :972 -- one query token over seq_len cached
 * positions (fp16 bits): out[h] = softmax(q[h] . K[0..seq_len) * scale) V, GQA head h / (nh / nkv).
 * head_dim 64, 128 or 256.  Like the reference these take no workspace; they
 * run one workgroup per query head (the _ws launchers below split the
 * positions over many workgroups). */
hipError_t gpu_flash_attn_decode_strided_multi_head(float* d_out, const float* d_q, const uint16_t* d_k_cache,
                                                    const uint16_t* d_v_cache, const int seq_len, const int num_heads,
                                                    const int num_kv_heads, const int head_dim, const float scale,
                                                    hipStream_t stream);
hipError_t gpu_flash_attn_decode_strided_multi_head_state(float* d_out, const float* d_q, const uint16_t* d_k_cache,
                                                          const uint16_t* d_v_cache, const int* d_seq_len,
                                                          const int num_heads, const int num_kv_heads,
                                                          const int head_dim, const float scale, hipStream_t stream);

/* No counterpart: the decode attention with its positions split over up to
 * 64 workgroups per kv head (all of a GQA group's query heads, <= 8, in one
 * workgroup) and the partial softmax states merged by a second kernel, in
 * the caller's workspace d_workspace of workspace_bytes >=
 * rf_flash_attn_decode_workspace_bytes(num_heads, head_dim) bytes (a smaller
 * one is rejected).  Same results as the launchers above within fp32
 * rounding; GQA groups larger than 8 take the one-workgroup path.  Launches
 * that share a workspace must be stream-ordered. */
size_t rf_flash_attn_decode_workspace_bytes(const int num_heads, const int head_dim);
hipError_t rf_flash_attn_decode_ws(float* d_out, const float* d_q, const uint16_t* d_k_cache, const uint16_t* d_v_cache,
                                   const int seq_len, const int num_heads, const int num_kv_heads, const int head_dim,
                                   const float scale, float* d_workspace, const size_t workspace_bytes,
                                   hipStream_t stream);
hipError_t rf_flash_attn_decode_state_ws(float* d_out, const float* d_q, const uint16_t* d_k_cache,
                                         const uint16_t* d_v_cache, const int* d_seq_len, const int num_heads,
                                         const int num_kv_heads, const int head_dim, const float scale,
                                         float* d_workspace, const size_t workspace_bytes, hipStream_t stream);

/* No counterpart in the reference: rf_flash_attn_decode_state_ws for callers
 * that cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  The workspace is a file-scope device
 * array of 4,259,840 bytes held by each GPU the library runs on until the
 * process ends (its address is looked up once per device); calls with
 * num_heads * (head_dim + 4) > 16640 are rejected with hipErrorInvalidValue.
 * The launcher calls no hipMalloc/hipFree.  All calls on one GPU share the
 * array: calls that overlap on a GPU (other streams or threads) race;
 * stream-ordered calls do not.  Same results as rf_flash_attn_decode_state_ws. */
hipError_t rf_flash_attn_decode_state_noalloc(float* d_out, const float* d_q, const uint16_t* d_k_cache,
                                              const uint16_t* d_v_cache, const int* d_seq_len, const int num_heads,
                                              const int num_kv_heads, const int head_dim, const float scale,
                                              hipStream_t stream);

/* No counterpart (the reference computes theta_i in each RoPE launch): fills
 * the caller's d_theta[head_dim / 2] with theta_i = 1 / base^((float)(2i) /
 * (float)head_dim) (double pow, rounded once), the values every RoPE here
 * uses.  The fused launchers' d_theta argument takes such a table (or null:
 * they then evaluate theta in the kernel, same bits). */
hipError_t rf_rope_theta_table(float* d_theta, const int head_dim, const float theta_base, hipStream_t stream);

/* No counterpart (the reference evaluates cosf / sinf in each RoPE launch):
 * fills the caller's d_cos_sin[positions][head_dim / 2][2] with the cosine
 * and sine of pos * theta_i, theta_i as the fused launchers take it (from
 * d_theta when given, else evaluated; divided by d_freq_scale[i] when given).
 * The fused launchers' d_cos_sin argument (16-byte aligned, or null) takes
 * such a table, built with their theta_base / d_theta / d_freq_scale and
 * covering every position they are called at, in place of evaluating cosf /
 * sinf: the same values, so the same bits. */
hipError_t rf_rope_cos_sin_table(float* d_cos_sin, const int positions, const int head_dim, const float theta_base,
                                 const float* d_theta, const float* d_freq_scale, hipStream_t stream);

/* No counterpart (the reference launches the per-head norms, the q RoPE and
 * the KV write before gpu_flash_attn_decode_strided_multi_head_state,
 * src/gpu/forward.rs:2384-2440): the same step folded into the decode
 * attention.  d_q, d_k, d_v are the raw projections (d_q is not modified);
 * the K/V row at pos = d_state[0] is written, then attention runs over
 * d_state[1] positions.  Same bits as rf_qk_norm_rope_kv_write_state followed
 * by gpu_flash_attn_decode_strided_multi_head_state.  GQA group <= 8. */
hipError_t rf_attn_decode_qk_norm_rope_state(float* d_out, const float* d_q, const float* d_k, const float* d_v,
                                             const float* d_q_norm, const float* d_k_norm, uint16_t* d_k_cache,
                                             uint16_t* d_v_cache, const int* d_state, const int num_heads,
                                             const int num_kv_heads, const int head_dim, const float eps,
                                             const float theta_base, const int neox, const float* d_freq_scale,
                                             const float* d_theta, const float* d_cos_sin, const float scale,
                                             float* d_workspace,
                                             const size_t workspace_bytes, hipStream_t stream);

/* No counterpart (the reference's decode attention,
 * hip_kernels/attention.hip:950, has no bound on the sequence): the two
 * launchers above for a caller that bounds it, seq <= max_seq (e.g. the KV
 * cache length).  With max_seq <= 2048 one workgroup per query head runs
 * (16 waves split the positions and merge their partials through LDS in wave
 * order): no workspace (d_workspace may then be null), one launch instead of
 * the split kernel and its merge, any GQA group.  Beyond 2048 the split path
 * with the workspace as above.  Results within fp32 rounding of the
 * unbounded launchers (another summation order). */
hipError_t rf_flash_attn_decode_state_bounded(float* d_out, const float* d_q, const uint16_t* d_k_cache,
                                              const uint16_t* d_v_cache, const int* d_seq_len, const int num_heads,
                                              const int num_kv_heads, const int head_dim, const float scale,
                                              const int max_seq, float* d_workspace, const size_t workspace_bytes,
                                              hipStream_t stream);
hipError_t rf_attn_decode_qk_norm_rope_state_bounded(float* d_out, const float* d_q, const float* d_k,
                                                     const float* d_v, const float* d_q_norm, const float* d_k_norm,
                                                     uint16_t* d_k_cache, uint16_t* d_v_cache, const int* d_state,
                                                     const int num_heads, const int num_kv_heads, const int head_dim,
                                                     const float eps, const float theta_base, const int neox,
                                                     const float* d_freq_scale, const float* d_theta,
                                                     const float* d_cos_sin, const float scale, const int max_seq,
                                                     float* d_workspace, const size_t workspace_bytes,
                                                     hipStream_t stream);

/* hip_kernels/elementwise.hip:615, :651 -- index of the maximum of d_input[n]
 * (ties: the larger index; NaN never wins); partial buffers hold ceil(n / 1024). */
hipError_t gpu_argmax_f32_on_stream(const float* d_input, float* d_partial_values, int* d_partial_indices,
                                    int* d_output_index, const int n, hipStream_t stream);
hipError_t gpu_argmax_f32(const float* d_input, float* d_partial_values, int* d_partial_indices,
                          int* d_output_index, const int n);
/* No counterpart (the reference follows the argmax with
 * gpu_increment_decode_state_on_stream): the argmax, then d_state[0..1] += 1. */
hipError_t rf_argmax_f32_advance_state_on_stream(const float* d_input, float* d_partial_values,
                                                 int* d_partial_indices, int* d_output_index, const int n,
                                                 int* d_state, hipStream_t stream);

/* hip_kernels/elementwise.hip:780, :804 -- Q4_K rows of a [vocab][hidden]
 * embedding dequantised to fp32; ids outside [0, vocab) leave their row untouched. */
hipError_t gpu_embed_q4_k_token(const uint8_t* d_embedding, float* d_out, const int hidden_size,
                                const int vocab_size, const int token_id, hipStream_t stream);
hipError_t gpu_embed_q4_k_batch(const uint8_t* d_embedding, const int* d_token_ids, float* d_out,
                                const int hidden_size, const int vocab_size, const int seq_len, hipStream_t stream);

/* hip_kernels/elementwise.hip:450-750 and quant/dequant_q4_0_to_f16.hip:103. */
hipError_t gpu_add(const float* d_x, const float* d_y, float* d_out, const int n, hipStream_t stream);
hipError_t gpu_mul_on_stream(const float* d_x, const float* d_y, float* d_out, const int n, hipStream_t stream);
hipError_t gpu_silu_on_stream(const float* d_x, float* d_out, const int n, hipStream_t stream);
hipError_t gpu_increment_decode_state_on_stream(int* d_state, hipStream_t stream);
hipError_t convert_f32_to_f16(const float* input, void* output, int n, hipStream_t stream);
/* No counterpart (the reference takes gpu_silu_on_stream then gpu_mul_on_stream,
 * src/gpu/forward.rs:1133-1143): out = silu(gate) * up. */
hipError_t rf_silu_mul_on_stream(const float* d_gate, const float* d_up, float* d_out, const int n,
                                 hipStream_t stream);
/* No counterpart: the same with the result rounded to fp16 (nearest even). */
hipError_t rf_silu_mul_f16_on_stream(const float* d_gate, const float* d_up, uint16_t* d_out_f16, const int n,
                                     hipStream_t stream);

/* hip_kernels/wmma/wmma_attention_prefill.hip:711 -- causal (or full) GQA
 * attention over seq_len % 64 == 0 rows: Q [seq][nq*128], K, V [seq][nkv*128]
 * fp16 bits, 16-byte aligned; O [seq][nq*128] fp32.  The reference's
 * rounding: fp32 S, 64-key tiles, P rounded to fp16 per tile, fp32 O. */
hipError_t wmma_attention_prefill_gqa_causal_launch(const void* Q, const void* K, const void* V, float* O,
                                                    int seq_len, int num_q_heads, int num_kv_heads, int causal,
                                                    float scale, hipStream_t stream);
/* No counterpart: the same attention with O rounded to fp16 (round to nearest
 * even, bits as uint16_t) -- the operand an O projection on fp16 activations
 * (rf_gemm_q4_k_f16_accumulate_launch) reads, __float2half of the fp32
 * launcher's output. */
hipError_t rf_attention_prefill_gqa_causal_f16_launch(const void* Q, const void* K, const void* V, uint16_t* O_f16,
                                                      int seq_len, int num_q_heads, int num_kv_heads, int causal,
                                                      float scale, hipStream_t stream);

/* ---- GEMVs with the RMSNorm of their input fused in (no counterpart) ----
 * out = W * rmsnorm(input, norm_w, eps), bit-identical to gpu_rms_norm into a
 * buffer followed by the plain launcher; one launch instead of two (the
 * reference normalises with a separate launch before the QKV, gate/up and
 * LM-head GEMVs, src/gpu/forward.rs:2349-2359, :2454-2464, :329-376).
 * input and norm_w 16-byte aligned; otherwise the plain launchers' rules
 * (the Q6_K one: K / 256 % 8 == 0, K <= 16384, 16-byte aligned weights). */
hipError_t rf_gemv_q4_k_q8_rmsnorm_launch(const void* weights_q4_k, const float* input, const float* norm_w,
                                          float eps, float* output, int n_rows, int ncols_dst, hipStream_t stream);
hipError_t rf_gemv_gate_up_q4_k_q8_rmsnorm_launch(const void* weights_gate_q4_k, const void* weights_up_q4_k,
                                                  const float* input, const float* norm_w, float eps,
                                                  float* swiglu_out, int n_rows, int ncols_dst, hipStream_t stream);
hipError_t rf_gemv_qkv_q4_k_q8_rmsnorm_launch(const void* w_q, const void* w_k, const void* w_v, const float* bias_q,
                                              const float* bias_k, const float* bias_v, const float* input,
                                              const float* norm_w, float eps, float* out_q, float* out_k,
                                              float* out_v, int n_rows, int n_q, int n_kv, hipStream_t stream);
hipError_t rf_gemv_q6_k_rmsnorm_launch(const void* weights_q6_k, const float* input, const float* norm_w, float eps,
                                       float* output, int n_rows, int ncols_dst, hipStream_t stream);
/* Q4_K Q and K with a Q6_K V (Q4_K_M layers whose attn_v is Q6_K), the
 * RMSNorm folded in, one launch: out_q / out_k as rf_gemv_q4_k_q8_rmsnorm_launch
 * and out_v as rf_gemv_q6_k_rmsnorm_launch would give them (same bits), plus
 * the optional biases.  The reference runs a norm and three GEMVs
 * (src/gpu/ops.rs:851-853, src/gpu/forward.rs:2349-2359).  K (n_rows) in
 * {2048, 4096, 8192}; weights, input and norm_w 16-byte aligned. */
hipError_t rf_gemv_qkv_q4_k_q6_k_v_rmsnorm_launch(const void* w_q, const void* w_k, const void* w_v_q6_k,
                                                  const float* bias_q, const float* bias_k, const float* bias_v,
                                                  const float* input, const float* norm_w, float eps, float* out_q,
                                                  float* out_k, float* out_v, int n_rows, int n_q, int n_kv,
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

/* ---- Measurement (no reference counterpart) -----------------------------
 * MFMA peak microbenchmark: grid workgroups of 256 threads, each wave issuing
 * iters x 8 independent v_mfma_f32_32x32x16_f16 on operands read from
 * a[0 .. 4096) (fp16 bit patterns: the data decides the switching activity
 * and with it the clock); out[block * 256 + thread] receives a checksum of
 * the accumulators.  FLOPs = grid * 4 * iters * 8 * 32768. */
hipError_t rf_mfma_peak_launch(const uint16_t* a, float* out, int grid, int iters, hipStream_t stream);

/* Library identification string. */
const char* rf_library_version(void);

#ifdef __cplusplus
}
#endif

#endif /* ROCMFORGE_CDNA4_H */
