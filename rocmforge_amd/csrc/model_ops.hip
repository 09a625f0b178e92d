// model_ops.hip -- the decode/prefill operations around the quantised
// matmuls of a llama/qwen-style layer, on CDNA4 (gfx950, wave64).
//
// Drop-in for the reference's launchers of the same names (argument order,
// meaning and error returns kept):
//   gpu_rms_norm / gpu_rms_norm_batched(_on_stream)   hip_kernels/norm.hip:154-199
//   gpu_rope_heads(_state)(_scaled), gpu_rope_heads_batched(_scaled)
//                                                     hip_kernels/rope.hip:238-420
//   gpu_kv_write_rope(_state)(_scaled), gpu_kv_write_batched
//                                                     hip_kernels/attention.hip:1627-1670
//   gpu_flash_attn_decode_strided_multi_head(_state)  hip_kernels/attention.hip:950-993
//   gpu_argmax_f32(_on_stream)                        hip_kernels/elementwise.hip:615-666
//   gpu_embed_q4_k_token / gpu_embed_q4_k_batch       hip_kernels/elementwise.hip:780-827
//   gpu_add, gpu_mul_on_stream, gpu_silu_on_stream, gpu_increment_decode_state_on_stream
//                                                     hip_kernels/elementwise.hip:450-750
//   convert_f32_to_f16                                hip_kernels/quant/dequant_q4_0_to_f16.hip:103
// plus entry points without a counterpart (declared as such in the header):
// stream variants of the null-stream batched launchers, a fused SwiGLU, and
// rf_qk_norm_rope_kv_write_state, which does a Qwen3 decode step's per-head
// Q/K RMSNorm, both RoPEs and the fp16 KV write in one launch (the reference
// takes four).
//
// RoPE frequencies: theta_i = 1 / base^(e_i) with e_i = (float)(2i) / (float)d
// as the reference, evaluated in double and rounded once to float (the
// reference's 1.0f / powf(..) is within an ulp of this), then divided by
// freq_scale[i] when given; angle = (float)pos * theta_i in fp32.  The
// reference-named launchers evaluate theta_i in the kernel; the fused
// launchers take an optional caller-owned table of the same values
// (rf_rope_theta_table fills one), which saves the double-precision pow in
// every lane.  No launcher allocates, frees or synchronises.
#include <hip/hip_fp16.h>

#include <mutex>


#include <type_traits>

#include "qk_common.h"

namespace rf {

constexpr float kNegMax = -3.402823466e+38f;

__device__ __forceinline__ float wave_max(float v) {
    // butterfly over the 64 lanes: every lane ends with the maximum
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

__device__ __forceinline__ float wave_sum_all(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// theta_i = 1 / base^((float)(2i) / (float)d), evaluated in double and
// rounded once to float
__device__ __forceinline__ float theta_exact(int i, int d, float base) {
    const float e = (float)(2 * i) / (float)d;
    return (float)(1.0 / pow((double)base, (double)e));
}

// theta_i from the caller's table when given (the same values), else
// evaluated here; divided by freq_scale[i] when given
__device__ __forceinline__ float rope_theta(int i, int d, float base, const float* __restrict__ tab,
                                            const float* freq_scale) {
    float t = tab != nullptr ? tab[i] : theta_exact(i, d, base);
    if (freq_scale != nullptr) t /= freq_scale[i];
    return t;
}

__global__ void rf_theta_fill_kernel(float* tab, int d, float base) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < d / 2) tab[i] = theta_exact(i, d, base);
}

// (x0, x1) rotated by the angle with cosine c and sine s.  The roundings
// are spelled out (one product rounded, the other fused) so that every
// kernel here rotates to the same bits, whatever contraction the compiler
// would pick where c and s come from
__device__ __forceinline__ void rope_cs(float& x0, float& x1, float c, float s) {
    const float y0 = __fmaf_rn(x0, c, -__fmul_rn(x1, s));
    const float y1 = __fmaf_rn(x0, s, __fmul_rn(x1, c));
    x0 = y0;
    x1 = y1;
}

// (x0, x1) rotated by angle pos * theta
__device__ __forceinline__ void rope_pair(float& x0, float& x1, int pos, float theta) {
    const float a = (float)pos * theta;
    rope_cs(x0, x1, cosf(a), sinf(a));
}

// cs[pos][i] = (cos, sin) of pos * theta_i, theta_i as rope_theta (from the
// table when given, divided by freq_scale[i] when given): the values rope_pair evaluates, so a kernel
// that reads them rotates to the same bits without cosf / sinf
__global__ void rf_rope_cos_sin_kernel(float2* __restrict__ cs, int positions, int d, float base,
                                       const float* __restrict__ tab, const float* __restrict__ freq_scale) {
    const int half = d / 2;
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long)positions * half) return;
    const int pos = (int)(idx / half), i = (int)(idx % half);
    const float a = (float)pos * rope_theta(i, d, base, tab, freq_scale);
    cs[idx] = make_float2(cosf(a), sinf(a));
}

// element indices of pair p of a head: NeoX pairs (p, p + d/2), classic (2p, 2p + 1)
__device__ __forceinline__ void pair_idx(int p, int d, int neox, int* i0, int* i1) {
    if (neox) {
        *i0 = p;
        *i1 = p + d / 2;
    } else {
        *i0 = 2 * p;
        *i1 = 2 * p + 1;
    }
}

// ---- RMSNorm ------------------------------------------------------------------
// out = x * rsqrt(mean(x^2) + eps) * w, rows of n; out may alias x.
// Single vectors and long rows: one 256-thread workgroup per row.  Short
// batched rows (n <= 512, the per-head norms): one wave per row, four rows
// per workgroup.
// OUT = float, or __half (the fp32 value rounded to nearest even: the
// operand a GEMM on fp16 activations reads)
template <typename OUT>
__global__ __launch_bounds__(256) void rf_rms_norm_long_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                               OUT* out, int n, float eps, int rows) {
    __shared__ float red[4];
    const int r = blockIdx.x;
    if (r >= rows) return;
    const float* xr = x + (size_t)r * n;
    OUT* orow = out + (size_t)r * n;
    // the canonical summation order (rms_inv_canonical) whenever the row is
    // float4-addressable: the GEMVs with a fused norm use the same order
    const bool v4 = (n & 7) == 0 && ((reinterpret_cast<uintptr_t>(xr) | reinterpret_cast<uintptr_t>(orow) |
                                      reinterpret_cast<uintptr_t>(w)) & 15u) == 0;
    float inv;
    if (v4) {
        inv = rms_inv_canonical(xr, n, eps, red);
    } else {
        float ss = 0.0f;
        for (int i = threadIdx.x; i < n; i += blockDim.x) ss = __fmaf_rn(xr[i], xr[i], ss);
        ss = xor_sum64(ss);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
        inv = rms_inv_finish(red, n, eps);
    }
    if (v4) {
        for (int i = threadIdx.x; i < n / 4; i += blockDim.x) {
            const float4 a = reinterpret_cast<const float4*>(xr)[i];
            const float4 g = reinterpret_cast<const float4*>(w)[i];
            const float4 o = make_float4((a.x * inv) * g.x, (a.y * inv) * g.y, (a.z * inv) * g.z, (a.w * inv) * g.w);
            if constexpr (std::is_same<OUT, float>::value) {
                reinterpret_cast<float4*>(orow)[i] = o;
            } else {
                uint16_t* o16 = reinterpret_cast<uint16_t*>(orow);
                o16[4 * i] = f16_bits_rn(o.x);
                o16[4 * i + 1] = f16_bits_rn(o.y);
                o16[4 * i + 2] = f16_bits_rn(o.z);
                o16[4 * i + 3] = f16_bits_rn(o.w);
            }
        }
    } else {
        for (int i = threadIdx.x; i < n; i += blockDim.x) {
            const float o = (xr[i] * inv) * w[i];
            if constexpr (std::is_same<OUT, float>::value)
                orow[i] = o;
            else
                reinterpret_cast<uint16_t*>(orow)[i] = f16_bits_rn(o);
        }
    }
}

__global__ __launch_bounds__(256) void rf_rms_norm_short_kernel(const float* __restrict__ x,
                                                                const float* __restrict__ w, float* out, int n,
                                                                float eps, int rows) {
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    const float* xr = x + (size_t)r * n;
    float v[8];
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int i = lane + 64 * k;
        v[k] = i < n ? xr[i] : 0.0f;
        ss += v[k] * v[k];
    }
    ss = wave_sum_all(ss);
    const float inv = rsqrtf(ss / (float)n + eps);
    float* orow = out + (size_t)r * n;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int i = lane + 64 * k;
        if (i < n) orow[i] = v[k] * inv * w[i];
    }
}

static hipError_t rms_rows(const float* x, const float* w, float* out, int n, float eps, int rows, hipStream_t st) {
    if (x == nullptr || w == nullptr || out == nullptr || n <= 0 || rows <= 0) return hipErrorInvalidValue;
    if (n <= 512 && rows > 1)
        hipLaunchKernelGGL(rf_rms_norm_short_kernel, dim3((rows + 3) / 4), dim3(256), 0, st, x, w, out, n, eps, rows);
    else
        hipLaunchKernelGGL(rf_rms_norm_long_kernel<float>, dim3(rows), dim3(256), 0, st, x, w, out, n, eps, rows);
    return hipGetLastError();
}

// ---- RoPE over heads (in place) ---------------------------------------------------
__global__ void rf_rope_heads_kernel(float* x, const int* __restrict__ pos_ptr, int pos0, int nh, int d,
                                     float base, int neox, const float* __restrict__ freq_scale, int seq_len) {
    const int half = d / 2;
    const int p = blockIdx.x * blockDim.x + threadIdx.x;
    const int s = blockIdx.y;
    if (p >= nh * half || s >= seq_len) return;
    const int pos = (pos_ptr ? *pos_ptr : pos0) + s;
    const int head = p / half, i = p % half;
    float* row = x + (size_t)s * nh * d + (size_t)head * d;
    int i0, i1;
    pair_idx(i, d, neox, &i0, &i1);
    float x0 = row[i0], x1 = row[i1];
    rope_pair(x0, x1, pos, rope_theta(i, d, base, nullptr, freq_scale));
    row[i0] = x0;
    row[i1] = x1;
}

static hipError_t rope_heads(float* x, const int* pos_ptr, int pos, int nh, int d, float base, int neox,
                             const float* fs, int seq_len, hipStream_t st) {
    if (x == nullptr || nh <= 0 || d <= 0 || (d & 1) || seq_len <= 0) return hipErrorInvalidValue;
    const int pairs = nh * (d / 2);
    hipLaunchKernelGGL(rf_rope_heads_kernel, dim3((pairs + 255) / 256, seq_len), dim3(256), 0, st, x, pos_ptr, pos, nh,
                       d, base, neox, fs, seq_len);
    return hipGetLastError();
}

// ---- KV cache writes ------------------------------------------------------------------
// Cache layout [max_seq][n_kv * d] fp16 per layer; V copied, K rotated.
__global__ void rf_kv_write_rope_kernel(__half* kc, __half* vc, const float* __restrict__ k,
                                        const float* __restrict__ v, const int* __restrict__ pos_ptr, int pos0,
                                        int nkv, int d, float base, int neox,
                                        const float* __restrict__ freq_scale) {
    const int half = d / 2;
    const int p = blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= nkv * half) return;
    const int pos = pos_ptr ? *pos_ptr : pos0;
    const int head = p / half, i = p % half;
    int i0, i1;
    pair_idx(i, d, neox, &i0, &i1);
    const size_t base_in = (size_t)head * d;
    const size_t base_c = (size_t)pos * nkv * d + base_in;
    float x0 = k[base_in + i0], x1 = k[base_in + i1];
    rope_pair(x0, x1, pos, rope_theta(i, d, base, nullptr, freq_scale));
    kc[base_c + i0] = __float2half(x0);
    kc[base_c + i1] = __float2half(x1);
    vc[base_c + i0] = __float2half(v[base_in + i0]);
    vc[base_c + i1] = __float2half(v[base_in + i1]);
}

__global__ void rf_kv_write_batched_kernel(__half* kc, __half* vc, const float* __restrict__ k,
                                           const float* __restrict__ v, int start_pos, int kv_size, int seq_len) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const int s = blockIdx.y;
    if (i >= kv_size || s >= seq_len) return;
    const size_t c = (size_t)(start_pos + s) * kv_size + i, in = (size_t)s * kv_size + i;
    kc[c] = __float2half(k[in]);
    vc[c] = __float2half(v[in]);
}

// ---- fused Qwen3 decode step: Q/K RMSNorm, RoPE, KV write ----------------------------
// Per-head layout shared with the decode attention: a head of D = 8 LPP
// values is held by LPP consecutive lanes, 8 consecutive dims per lane.
// The per-head RMSNorm sums each lane's 8 squares (fma chain) and adds the
// LPP lanes by an xor butterfly; NeoX pairs (i, i + D/2) sit in lanes sub
// and sub + LPP/2 (one xor shuffle), classic pairs (2i, 2i+1) in one lane.
// Both the standalone step and the attention with the step folded in use
// head_norm_rope below, so they produce the same bits.
// RoPE angles: a head's D / 2 pairs all turn by pos * theta_i, the same for
// every head of a position, so each wave takes the cos / sin of the D / 2
// angles once into its own LDS slice (lane l: pairs l, l + 64) and every
// lane reads its pairs from there.  The values are cosf / sinf of the angle
// rope_pair takes (theta_i from the caller's table when given, divided by
// freq_scale[i] when given), or the same values from a rf_rope_cos_sin_kernel
// table row: the rotations match the per-element RoPE launchers bit for bit.
// In two halves for a caller that issues other loads in between: the lane's
// (cos, sin) values (from the table row, or evaluated), then their LDS
// store.  N = pairs per lane (D / 2 over 64 lanes, at least 1).
template <int LPP>
struct CsLane {
    static constexpr int N = (4 * LPP + 63) / 64;
    float2 c[N];
};
template <int LPP>
__device__ __forceinline__ CsLane<LPP> wave_cos_sin_get(const float2* __restrict__ cs_row,
                                                       const float* __restrict__ tab, float base,
                                                       const float* __restrict__ freq_scale, int pos, int lane) {
    constexpr int H = 4 * LPP;   // D / 2
    CsLane<LPP> r;
#pragma unroll
    for (int k = 0; k < CsLane<LPP>::N; ++k) {
        const int i = lane + 64 * k;
        if (i >= H) break;
        if (cs_row != nullptr) {
            r.c[k] = cs_row[i];
        } else {
            const float a = (float)pos * rope_theta(i, 8 * LPP, base, tab, freq_scale);
            r.c[k] = make_float2(cosf(a), sinf(a));
        }
    }
    return r;
}
template <int LPP>
__device__ __forceinline__ void wave_cos_sin_put(float2* w, const CsLane<LPP>& r, int lane) {
    constexpr int H = 4 * LPP;
#pragma unroll
    for (int k = 0; k < CsLane<LPP>::N; ++k) {
        const int i = lane + 64 * k;
        if (i >= H) break;
        w[i] = r.c[k];
    }
    // the slice is the wave's own: a wave-scope fence orders the writes
    // before the other lanes' reads
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}
template <int LPP>
__device__ __forceinline__ void wave_cos_sin(float2* w, const float2* __restrict__ cs_row,
                                             const float* __restrict__ tab, float base,
                                             const float* __restrict__ freq_scale, int pos, int lane) {
    wave_cos_sin_put<LPP>(w, wave_cos_sin_get<LPP>(cs_row, tab, base, freq_scale, pos, lane), lane);
}

// The lane's (cos, sin) pairs from a wave_cos_sin slice: NeoX pairs (i,
// i + D/2) for i in [p0, p0 + 8), p0 = 8 sub mod D/2 (lanes sub and
// sub + LPP/2 hold the two halves); classic pairs (2i, 2i+1) for i in
// [4 sub, 4 sub + 4)
template <int LPP>
__device__ __forceinline__ void cs8(const float2* w, int sub, int neox, float2 c[8]) {
    constexpr int D = 8 * LPP;
    const int p0 = neox ? (sub < LPP / 2 ? 8 * sub : 8 * sub - D / 2) : 4 * sub;
    const float4* r = reinterpret_cast<const float4*>(w + p0);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        if (neox || k < 2) {
            const float4 a = r[k];
            c[2 * k] = make_float2(a.x, a.y);
            c[2 * k + 1] = make_float2(a.z, a.w);
        }
    }
}

// norm: the head is normalised with the weights gv (the lane's 8, loaded by
// the caller together with its other operands: a load here would wait for
// every load issued before it); then rotated by the lane's cos / sin pairs c
template <int LPP>
__device__ __forceinline__ void head_norm_rope(float v[8], int sub, bool norm, const float gv[8], float eps,
                                               const float2 c[8], int neox) {
    constexpr int D = 8 * LPP;
    if (norm) {
        float ss = v[0] * v[0];
#pragma unroll
        for (int i = 1; i < 8; ++i) ss = __fmaf_rn(v[i], v[i], ss);
#pragma unroll
        for (int o = 1; o < LPP; o <<= 1) ss += __shfl_xor(ss, o);
        const float inv = rsqrtf(ss / (float)D + eps);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = (v[i] * inv) * gv[i];
    }
    if (neox) {
        const bool lo = sub < LPP / 2;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float other = __shfl_xor(v[i], LPP / 2);
            float x0 = lo ? v[i] : other, x1 = lo ? other : v[i];
            rope_cs(x0, x1, c[i].x, c[i].y);
            v[i] = lo ? x0 : x1;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; i += 2) rope_cs(v[i], v[i + 1], c[i / 2].x, c[i / 2].y);
    }
}

__device__ __forceinline__ void load8(const float* p, float v[8]) {
    const float4 a = *reinterpret_cast<const float4*>(p), b = *reinterpret_cast<const float4*>(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

__device__ __forceinline__ void store8_f16(__half* p, const float v[8]) {
    typedef _Float16 hv8 __attribute__((ext_vector_type(8)));
    hv8 h;
#pragma unroll
    for (int i = 0; i < 8; ++i) h[i] = (_Float16)v[i];
    *reinterpret_cast<hv8*>(p) = h;
}

// Heads [0, nh) are query heads (normalised with q_norm when given,
// rotated, written back in place), heads [nh, nh + nkv) key heads
// (normalised with k_norm, rotated, written to the K cache at *pos as fp16;
// the matching V head is copied to the V cache).  64 / LPP heads per wave.
template <int LPP>
__global__ __launch_bounds__(256) void rf_qk_norm_rope_kv_kernel(
    float* q, const float* __restrict__ k, const float* __restrict__ v, const float* __restrict__ q_norm,
    const float* __restrict__ k_norm, __half* kc, __half* vc, const int* __restrict__ pos_ptr, int nh, int nkv,
    float eps, const float* __restrict__ tab, float base, int neox, const float* __restrict__ freq_scale,
    const float2* __restrict__ cs) {
    constexpr int D = 8 * LPP;
    __shared__ __align__(16) float2 lcs[4][D / 2];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int hidx = (blockIdx.x * 4 + wave) * (64 / LPP) + lane / LPP;
    const int sub = lane % LPP;
    const bool live = hidx < nh + nkv;
    const bool is_q = hidx < nh;
    const int head = is_q ? hidx : hidx - nh;
    // every load first (one memory round trip): the head, its norm weights,
    // the V head to copy and the position; the wave's cos / sin meanwhile
    const int pos = *pos_ptr;
    const float* g = is_q ? q_norm : k_norm;
    float x[8], gv[8], vv[8];
    float2 cv[8];
    if (live) {
        load8((is_q ? q : k) + (size_t)head * D + 8 * sub, x);
        if (g != nullptr) load8(g + 8 * sub, gv);
        if (!is_q) load8(v + (size_t)head * D + 8 * sub, vv);
    }
    wave_cos_sin<LPP>(lcs[wave], cs != nullptr ? cs + (size_t)pos * (D / 2) : nullptr, tab, base, freq_scale, pos,
                      lane);
    if (!live) return;                       // whole LPP-lane groups leave together
    cs8<LPP>(lcs[wave], sub, neox, cv);
    head_norm_rope<LPP>(x, sub, g != nullptr, gv, eps, cv, neox);
    if (is_q) {
        float* dst = q + (size_t)head * D + 8 * sub;
        *reinterpret_cast<float4*>(dst) = make_float4(x[0], x[1], x[2], x[3]);
        *reinterpret_cast<float4*>(dst + 4) = make_float4(x[4], x[5], x[6], x[7]);
    } else {
        const size_t c = (size_t)pos * nkv * D + (size_t)head * D + 8 * sub;
        store8_f16(kc + c, x);
        store8_f16(vc + c, vv);
    }
}

// The same step over rows of a prompt (row r at position pos0 + r): query
// rows [0, rows_q) are normalised, rotated and written as fp16 to q16 (the
// prefill attention's operand); key rows [0, rows_kv) go to the caches, with
// their V rows, as in the single-position kernel.  grid.y = rows_q.
template <int LPP>
__global__ __launch_bounds__(256) void rf_qk_norm_rope_kv_rows_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ q_norm, const float* __restrict__ k_norm, __half* __restrict__ q16, __half* kc,
    __half* vc, int pos0, int rows_kv, int nh, int nkv, float eps, const float* __restrict__ tab, float base, int neox,
    const float* __restrict__ freq_scale, const float2* __restrict__ cs) {
    constexpr int D = 8 * LPP;
    __shared__ __align__(16) float2 lcs[4][D / 2];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int hidx = (blockIdx.x * 4 + wave) * (64 / LPP) + lane / LPP;
    const int sub = lane % LPP;
    const int row = blockIdx.y;
    const bool is_q = hidx < nh;
    const bool live = hidx < nh + nkv && (is_q || row < rows_kv);
    const int head = is_q ? hidx : hidx - nh;
    const int pos = pos0 + row;
    const size_t src = (size_t)row * (is_q ? nh : nkv) * D + (size_t)head * D + 8 * sub;
    const float* g = is_q ? q_norm : k_norm;
    float x[8], gv[8], vv[8];
    float2 cv[8];
    if (live) {
        load8((is_q ? q : k) + src, x);
        if (g != nullptr) load8(g + 8 * sub, gv);
        if (!is_q) load8(v + src, vv);
    }
    wave_cos_sin<LPP>(lcs[wave], cs != nullptr ? cs + (size_t)pos * (D / 2) : nullptr, tab, base, freq_scale, pos,
                      lane);
    if (!live) return;                       // whole LPP-lane groups leave together
    cs8<LPP>(lcs[wave], sub, neox, cv);
    head_norm_rope<LPP>(x, sub, g != nullptr, gv, eps, cv, neox);
    if (is_q) {
        store8_f16(q16 + src, x);
    } else {
        const size_t c = (size_t)pos * nkv * D + (size_t)head * D + 8 * sub;
        store8_f16(kc + c, x);
        store8_f16(vc + c, vv);
    }
}

// ---- decode attention -----------------------------------------------------------------
// Single-workgroup path (GQA groups larger than 8): one workgroup (4 waves) per query head.  Scores: LPP lanes per position
// (8 fp16 of K per lane, one 16-byte load), so a wave-instruction covers
// 64 / LPP positions with coalesced K rows; the partial dots are reduced
// across the LPP lanes with shuffles.  Scores go to LDS in chunks of
// kAttnChunk positions; each chunk's max/exp/sum and its pass over V
// (lane pairs of output dims, positions split over the waves) update a
// running (m, l, acc) exactly as an online softmax over chunks.
constexpr int kAttnChunk = 4096;

template <int LPP>
__global__ __launch_bounds__(256) void rf_attn_decode_kernel(float* __restrict__ out, const float* __restrict__ q,
                                                             const __half* __restrict__ kc,
                                                             const __half* __restrict__ vc,
                                                             const int* __restrict__ len_ptr, int len0, int nh,
                                                             int nkv, float scale) {
    constexpr int D = LPP * 8;
    constexpr int PPW = 64 / LPP;                 // positions per wave-instruction
    constexpr int DPL = (D + 127) / 128;          // output dim pairs per lane in the V pass
    __shared__ float sc[kAttnChunk];
    __shared__ float red[4][D];
    __shared__ float wred[8];
    const int seq = len_ptr ? *len_ptr : len0;
    const int head = blockIdx.x;
    const int kvh = head / (nh / nkv);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const size_t row = (size_t)nkv * D;
    const __half* kh = kc + (size_t)kvh * D;
    const __half* vh = vc + (size_t)kvh * D;
    // this lane's 8 query values (dims 8 (lane % LPP) ..)
    float qv[8];
    {
        const float* qh = q + (size_t)head * D + 8 * (lane % LPP);
        const float4 a = *reinterpret_cast<const float4*>(qh), b = *reinterpret_cast<const float4*>(qh + 4);
        qv[0] = a.x; qv[1] = a.y; qv[2] = a.z; qv[3] = a.w; qv[4] = b.x; qv[5] = b.y; qv[6] = b.z; qv[7] = b.w;
    }
    float m_run = kNegMax, l_run = 0.0f;
    float acc[DPL * 2];
#pragma unroll
    for (int i = 0; i < DPL * 2; ++i) acc[i] = 0.0f;

    for (int c0 = 0; c0 < seq; c0 += kAttnChunk) {
        const int cn = min(kAttnChunk, seq - c0);
        // scores
        for (int p0 = wave * PPW; p0 < cn; p0 += 4 * PPW) {
            const int p = p0 + lane / LPP;
            float s = 0.0f;
            if (p < cn) {
                const u32x4 kk = *reinterpret_cast<const u32x4*>(kh + (size_t)(c0 + p) * row + 8 * (lane % LPP));
                const uint32_t w4[4] = {kk.x, kk.y, kk.z, kk.w};
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const __half2 h2 = __builtin_bit_cast(__half2, w4[t]);
                    const float2 f = __half22float2(h2);
                    s += qv[2 * t] * f.x + qv[2 * t + 1] * f.y;
                }
            }
#pragma unroll
            for (int o = LPP / 2; o > 0; o >>= 1) s += __shfl_xor(s, o);
            if (p < cn && lane % LPP == 0) sc[p] = s * scale;
        }
        __syncthreads();
        // chunk max
        float mx = kNegMax;
        for (int i = threadIdx.x; i < cn; i += 256) mx = fmaxf(mx, sc[i]);
        mx = wave_max(mx);
        if (lane == 0) wred[wave] = mx;
        __syncthreads();
        mx = fmaxf(fmaxf(wred[0], wred[1]), fmaxf(wred[2], wred[3]));
        const float m_new = fmaxf(m_run, mx);
        float ls = 0.0f;
        for (int i = threadIdx.x; i < cn; i += 256) {
            const float e = expf(sc[i] - m_new);
            sc[i] = e;
            ls += e;
        }
        ls = wave_sum_all(ls);
        __syncthreads();   // wred reads done, exps published
        if (lane == 0) wred[4 + wave] = ls;
        __syncthreads();
        const float alpha = expf(m_run - m_new);
        l_run = l_run * alpha + ((wred[4] + wred[5]) + (wred[6] + wred[7]));
        m_run = m_new;
#pragma unroll
        for (int i = 0; i < DPL * 2; ++i) acc[i] *= alpha;
        // V pass: wave w takes positions w, w + 4, ...; lane holds dims 2 (lane + 64 j) .. + 1
        for (int p = wave; p < cn; p += 4) {
            const float e = sc[p];
            const __half* vr = vh + (size_t)(c0 + p) * row;
#pragma unroll
            for (int j = 0; j < DPL; ++j) {
                const int dd = 2 * (lane + 64 * j);
                if (dd < D) {
                    const float2 f = __half22float2(*reinterpret_cast<const __half2*>(vr + dd));
                    acc[2 * j] += e * f.x;
                    acc[2 * j + 1] += e * f.y;
                }
            }
        }
        __syncthreads();   // sc reused by the next chunk
    }
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
        const int dd = 2 * (lane + 64 * j);
        if (dd < D) {
            red[wave][dd] = acc[2 * j];
            red[wave][dd + 1] = acc[2 * j + 1];
        }
    }
    __syncthreads();
    const float inv_l = 1.0f / l_run;
    for (int dd = threadIdx.x; dd < D; dd += 256)
        out[(size_t)head * D + dd] = ((red[0][dd] + red[1][dd]) + (red[2][dd] + red[3][dd])) * inv_l;
}

// Split decode attention (the path used when the GQA group is at most 8
// query heads).  Grid = (kv head, split); a workgroup has one wave per
// query head of the kv head's group, so the group's K/V rows are read once
// per workgroup (the other waves hit L1).  Positions go out in chunks of
// kSplitChunk, chunk c to split c mod S, each wave keeping an online
// (m, l, acc) over its chunks.  Within a chunk a wave issues all its K and
// V loads (LPP lanes x 16 bytes per position, 64 / LPP positions per
// instruction) before the first use, so the loads overlap.  The partial
// (m, l, acc) of every (head, split) goes to a workspace and a second
// kernel merges the S partials of each head (rows of D + 4 floats: acc, m, l):
//   out = sum_s e^(m_s - M) acc_s / sum_s e^(m_s - M) l_s,  M = max_s m_s.
constexpr int kSplitChunk = 32;

// QK: the decode step's per-head Q/K norm, RoPE and KV write are folded in
// (qk.*): q, k, v are the raw projections; every wave normalises and
// rotates its query head in registers, and the workgroup whose chunk holds
// the new position (seq - 1) writes that K/V row first -- no other
// workgroup reads it.
struct QkStep {
    const float* k;
    const float* v;
    const float* q_norm;
    const float* k_norm;
    __half* kc;
    __half* vc;
    float eps;
    const float* tab;
    float base;
    int neox;
    const float* freq_scale;
    const float2* cs;      // cos / sin table (rf_rope_cos_sin_kernel), or null
};

template <int LPP, bool QK>
__global__ __launch_bounds__(512) void rf_attn_split_kernel(const float* __restrict__ q,
                                                            const __half* kc,    // not restrict: QK writes a row
                                                            const __half* vc,
                                                            const int* __restrict__ len_ptr, int len0, int nh,
                                                            int nkv, float scale, float* __restrict__ ws, int S,
                                                            QkStep qk) {
    constexpr int D = LPP * 8;
    constexpr int PPW = 64 / LPP;
    constexpr int NI = kSplitChunk / PPW;       // load instructions per chunk (K and V each)
    __shared__ u32x4 new_kv[2][LPP];            // QK: the new position's fp16 K and V row of this kv head
    __shared__ __align__(16) float2 lcs[QK ? 8 : 1][QK ? D / 2 : 2];   // QK: each wave's cos / sin
    const int seq = len_ptr ? *len_ptr : len0;
    const int kvh = blockIdx.x, split = blockIdx.y;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int head = kvh * (nh / nkv) + wave;
    const size_t row = (size_t)nkv * D;
    const int sub = lane % LPP, grp = lane / LPP;
    if (split * kSplitChunk >= seq) {       // no positions: an empty partial (l = 0) for the merge
        if (lane == 0) {
            float* dst = ws + ((size_t)head * S + split) * (D + 4);
            dst[D] = kNegMax;
            dst[D + 1] = 0.0f;
        }
        return;
    }
    const __half* kh = kc + (size_t)kvh * D + 8 * sub;
    const __half* vh = vc + (size_t)kvh * D + 8 * sub;
    const int pos = seq - 1;
    const bool owner = QK && split == (pos / kSplitChunk) % S;   // workgroup-uniform
    // loads in the order they are needed: q, (owner) the raw k / v, then the first chunk
    float qv[8], kx[8], vx[8], gq[8], gk[8];
    float2 cv[8];
    CsLane<LPP> csl;
    load8(q + (size_t)head * D + 8 * sub, qv);
    if constexpr (QK) {
        if (qk.q_norm != nullptr) load8(qk.q_norm + 8 * sub, gq);
        // the cos / sin values now, their LDS slice after the first chunk's
        // K / V loads are issued (the slice waits for this load only)
        csl = wave_cos_sin_get<LPP>(qk.cs != nullptr ? qk.cs + (size_t)pos * (D / 2) : nullptr, qk.tab, qk.base,
                                    qk.freq_scale, pos, lane);
    }
    if (owner && wave == 0) {
        load8(qk.k + (size_t)kvh * D + 8 * sub, kx);
        load8(qk.v + (size_t)kvh * D + 8 * sub, vx);
        if (qk.k_norm != nullptr) load8(qk.k_norm + 8 * sub, gk);
    }
    float m = kNegMax, l = 0.0f, acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
    for (int c0 = split * kSplitChunk; c0 < seq; c0 += S * kSplitChunk) {
        u32x4 kk[NI], vv[NI];
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int p = c0 + i * PPW + grp;
            const bool ok = p < seq;
            kk[i] = ok ? *reinterpret_cast<const u32x4*>(kh + (size_t)p * row) : u32x4{0, 0, 0, 0};
            vv[i] = ok ? *reinterpret_cast<const u32x4*>(vh + (size_t)p * row) : u32x4{0, 0, 0, 0};
        }
        if constexpr (QK) {
            if (c0 == split * kSplitChunk) {     // first chunk: the per-head step, while the loads fly
                wave_cos_sin_put<LPP>(lcs[wave], csl, lane);
                cs8<LPP>(lcs[wave], sub, qk.neox, cv);
                head_norm_rope<LPP>(qv, sub, qk.q_norm != nullptr, gq, qk.eps, cv, qk.neox);
                if (owner) {
                    if (wave == 0) {
                        head_norm_rope<LPP>(kx, sub, qk.k_norm != nullptr, gk, qk.eps, cv, qk.neox);
                        if (grp == 0) {
                            const size_t c = (size_t)pos * row + (size_t)kvh * D + 8 * sub;
                            store8_f16(qk.kc + c, kx);
                            store8_f16(qk.vc + c, vx);
                            typedef _Float16 hv8 __attribute__((ext_vector_type(8)));
                            hv8 hk, hvv;
#pragma unroll
                            for (int i = 0; i < 8; ++i) {
                                hk[i] = (_Float16)kx[i];
                                hvv[i] = (_Float16)vx[i];
                            }
                            new_kv[0][sub] = __builtin_bit_cast(u32x4, hk);
                            new_kv[1][sub] = __builtin_bit_cast(u32x4, hvv);
                        }
                    }
                    __syncthreads();
                }
            }
            if (owner && pos >= c0 && pos < c0 + kSplitChunk) {
                // the row at pos was loaded before it was written: take it from LDS
#pragma unroll
                for (int i = 0; i < NI; ++i)
                    if (c0 + i * PPW + grp == pos) {
                        kk[i] = new_kv[0][sub];
                        vv[i] = new_kv[1][sub];
                    }
            }
        }
        float sc[NI];
        float cm = kNegMax;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const uint32_t w4[4] = {kk[i].x, kk[i].y, kk[i].z, kk[i].w};
            float t = 0.0f;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float2 f = __half22float2(__builtin_bit_cast(__half2, w4[u]));
                t += qv[2 * u] * f.x + qv[2 * u + 1] * f.y;
            }
#pragma unroll
            for (int o = LPP / 2; o > 0; o >>= 1) t += __shfl_xor(t, o);
            sc[i] = (c0 + i * PPW + grp < seq) ? t * scale : kNegMax;
            cm = fmaxf(cm, sc[i]);
        }
#pragma unroll
        for (int o = LPP; o < 64; o <<= 1) cm = fmaxf(cm, __shfl_xor(cm, o));
        const float m_new = fmaxf(m, cm);
        const float alpha = expf(m - m_new);
        float ls = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] *= alpha;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const float e = (c0 + i * PPW + grp < seq) ? expf(sc[i] - m_new) : 0.0f;
            ls += e;
            const uint32_t w4[4] = {vv[i].x, vv[i].y, vv[i].z, vv[i].w};
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float2 f = __half22float2(__builtin_bit_cast(__half2, w4[u]));
                acc[2 * u] += e * f.x;
                acc[2 * u + 1] += e * f.y;
            }
        }
#pragma unroll
        for (int o = LPP; o < 64; o <<= 1) ls += __shfl_xor(ls, o);
        l = l * alpha + ls;
        m = m_new;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int o = LPP; o < 64; o <<= 1) acc[j] += __shfl_xor(acc[j], o);
    float* dst = ws + ((size_t)head * S + split) * (D + 4);
    if (grp == 0) {
        *reinterpret_cast<float4*>(dst + 8 * sub) = make_float4(acc[0], acc[1], acc[2], acc[3]);
        *reinterpret_cast<float4*>(dst + 8 * sub + 4) = make_float4(acc[4], acc[5], acc[6], acc[7]);
    }
    if (lane == 0) {
        dst[D] = m;
        dst[D + 1] = l;
    }
}

// One workgroup per head: thread t takes float4 dim-chunk t % (D / 4) of
// the splits congruent to t / (D / 4); the first wave takes the (m, l) of
// split = lane.  Every load is issued before the first use (one round trip):
// the accumulators of empty splits are loaded too (their slots hold
// whatever the workspace held) and weighted by 0 through a select.  The
// split groups are added in LDS.
constexpr int kMergeSplitsPerThread = 8;    // kMaxSplits / (256 / (D / 4)) for D = 128
__global__ __launch_bounds__(256) void rf_attn_merge_kernel(const float* __restrict__ ws, float* __restrict__ out,
                                                            int nh, int D, int S) {
    __shared__ float fs[64];
    __shared__ float4 part[256];
    __shared__ float lt_s;
    const int head = blockIdx.x;
    const int t = threadIdx.x;
    const float* base = ws + (size_t)head * S * (D + 4);
    const int nch = D / 4;                  // 16, 32 or 64 dim-chunks
    const int ngr = 256 / nch;              // split groups
    const int ch = t % nch, gr = t / nch;
    float mv = kNegMax, lv = 0.0f;
    if (t < 64 && t < S) {
        mv = base[(size_t)t * (D + 4) + D];
        lv = base[(size_t)t * (D + 4) + D + 1];
    }
    constexpr int U = kMergeSplitsPerThread;
    float4 v[U];
    auto load = [&](int s0) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int s = s0 + u * ngr;
            v[u] = s < S ? *reinterpret_cast<const float4*>(base + (size_t)s * (D + 4) + 4 * ch)
                         : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
    auto add = [&](int s0) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int s = s0 + u * ngr;
            const float f = s < S ? fs[s] : 0.0f;
            // an empty split's slots are zeroed by a select (they may hold
            // anything), then one fma per element
            const float4 w = f > 0.0f ? v[u] : make_float4(0.f, 0.f, 0.f, 0.f);
            a.x = __builtin_fmaf(f, w.x, a.x);
            a.y = __builtin_fmaf(f, w.y, a.y);
            a.z = __builtin_fmaf(f, w.z, a.z);
            a.w = __builtin_fmaf(f, w.w, a.w);
        }
    };
    load(gr);                               // in flight with the (m, l) loads
    if (t < 64) {
        float M = mv;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o));
        const float f = lv > 0.0f ? expf(mv - M) : 0.0f;   // splits without positions count 0
        fs[t] = f;
        float lt = f * lv;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) lt += __shfl_xor(lt, o);
        if (t == 0) lt_s = lt;
    }
    __syncthreads();
    add(gr);
    for (int s0 = gr + U * ngr; s0 < S; s0 += U * ngr) {   // D = 256 with more than 32 splits
        load(s0);
        add(s0);
    }
    part[t] = a;
    __syncthreads();
    if (t < nch) {
        float4 r = part[t];
        for (int g = 1; g < ngr; ++g) {
            const float4 b = part[g * nch + t];
            r.x += b.x; r.y += b.y; r.z += b.z; r.w += b.w;
        }
        const float inv = 1.0f / lt_s;
        *reinterpret_cast<float4*>(out + (size_t)head * D + 4 * t) = make_float4(r.x * inv, r.y * inv, r.z * inv,
                                                                                r.w * inv);
    }
}

// One workgroup per query head (the path for caches of up to
// kHeadPathMaxSeq positions): kHeadWaves waves split the positions, each
// keeping an online (m, l, acc) over its own slots, and the workgroup merges
// the wave partials through LDS in wave order -- no workspace, no second
// launch.  Slot s = positions [PPW s, PPW s + PPW) (one load instruction of
// K and one of V) goes to wave s mod kHeadWaves; a wave issues the K and V
// loads of kHeadBatch slots before the first use.  The query heads of a KV
// group read the same K/V rows (L2 hits after the first).
// QK: the decode step folded in, as in rf_attn_split_kernel: every wave
// normalises and rotates its query head in registers; the wave whose slot
// holds the new position (seq - 1) normalises and rotates the new K row
// itself and uses it (and the new V row) from registers in place of the
// cache, and in the workgroup of the group's first query head it writes
// both rows to the caches (no workgroup reads them from memory here).
constexpr int kHeadWaves = 16;
constexpr int kHeadBatch = 4;       // 16 waves of 1024 threads: <= 128 VGPRs, no spills at 4 slots per batch
constexpr int kHeadPathMaxSeq = 2048;

// The arithmetic is spelled out (__fmaf_rn, __fmul_rn) so that the QK and
// plain instantiations, and every kernel built from this code, contract
// the same way and give the same bits.
template <int LPP, bool QK>
__global__ __launch_bounds__(64 * kHeadWaves) void rf_attn_head_kernel(const float* __restrict__ q,
                                                                       const __half* kc, const __half* vc,
                                                                       const int* __restrict__ len_ptr, int len0,
                                                                       int nh, int nkv, float scale, QkStep qk,
                                                                       float* __restrict__ out) {
    constexpr int D = LPP * 8;
    constexpr int PPW = 64 / LPP;
    __shared__ __align__(16) float2 lcs[QK ? kHeadWaves : 1][QK ? D / 2 : 2];
    __shared__ __align__(16) float wacc[kHeadWaves][D];
    __shared__ float wm[kHeadWaves], wl[kHeadWaves];
    const int seq = len_ptr ? *len_ptr : len0;
    const int group = nh / nkv;
    // workgroup b runs on XCD b % 8: the query heads of one KV head go to one
    // XCD (its L2 then serves their common K/V rows) when nkv % 8 == 0
    const int b = blockIdx.x;
    const int head = nkv % 8 == 0 ? ((b % 8) + 8 * ((b / 8) / group)) * group + (b / 8) % group : b;
    const int kvh = head / group;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane % LPP, grp = lane / LPP;
    const size_t row = (size_t)nkv * D;
    const __half* kh = kc + (size_t)kvh * D + 8 * sub;
    const __half* vh = vc + (size_t)kvh * D + 8 * sub;
    const int nslots = (seq + PPW - 1) / PPW;
    const int pos = seq - 1;
    const bool pos_wave = QK && (pos / PPW) % kHeadWaves == wave;      // wave-uniform
    float qv[8], kx[8], vx[8], gq[8], gk[8];
    float2 cv[8];
    load8(q + (size_t)head * D + 8 * sub, qv);
    if constexpr (QK) {
        if (qk.q_norm != nullptr) load8(qk.q_norm + 8 * sub, gq);
        if (pos_wave) {
            load8(qk.k + (size_t)kvh * D + 8 * sub, kx);
            load8(qk.v + (size_t)kvh * D + 8 * sub, vx);
            if (qk.k_norm != nullptr) load8(qk.k_norm + 8 * sub, gk);
        }
        wave_cos_sin<LPP>(lcs[wave], qk.cs != nullptr ? qk.cs + (size_t)pos * (D / 2) : nullptr, qk.tab, qk.base,
                          qk.freq_scale, pos, lane);
        cs8<LPP>(lcs[wave], sub, qk.neox, cv);
    }
    float m = kNegMax, l = 0.0f, acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
    u32x4 knew{0, 0, 0, 0}, vnew{0, 0, 0, 0};
    bool first = true;
    for (int b0 = wave; b0 < nslots; b0 += kHeadWaves * kHeadBatch) {
        u32x4 kk[kHeadBatch], vv[kHeadBatch];
#pragma unroll
        for (int i = 0; i < kHeadBatch; ++i) {
            const int p = (b0 + kHeadWaves * i) * PPW + grp;
            const bool ok = p < seq;
            kk[i] = ok ? *reinterpret_cast<const u32x4*>(kh + (size_t)p * row) : u32x4{0, 0, 0, 0};
            vv[i] = ok ? *reinterpret_cast<const u32x4*>(vh + (size_t)p * row) : u32x4{0, 0, 0, 0};
        }
        if constexpr (QK) {
            if (first) {      // the per-head step while the first loads fly
                head_norm_rope<LPP>(qv, sub, qk.q_norm != nullptr, gq, qk.eps, cv, qk.neox);
                if (pos_wave) {
                    head_norm_rope<LPP>(kx, sub, qk.k_norm != nullptr, gk, qk.eps, cv, qk.neox);
                    typedef _Float16 hv8 __attribute__((ext_vector_type(8)));
                    hv8 hk, hvv;
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        hk[i] = (_Float16)kx[i];
                        hvv[i] = (_Float16)vx[i];
                    }
                    knew = __builtin_bit_cast(u32x4, hk);
                    vnew = __builtin_bit_cast(u32x4, hvv);
                    if (head % group == 0 && grp == 0) {
                        const size_t c = (size_t)pos * row + (size_t)kvh * D + 8 * sub;
                        *reinterpret_cast<u32x4*>(qk.kc + c) = knew;
                        *reinterpret_cast<u32x4*>(qk.vc + c) = vnew;
                    }
                }
                first = false;
            }
            if (pos_wave) {
#pragma unroll
                for (int i = 0; i < kHeadBatch; ++i)
                    if ((b0 + kHeadWaves * i) * PPW + grp == pos) {
                        kk[i] = knew;
                        vv[i] = vnew;
                    }
            }
        }
        float sc[kHeadBatch];
        float cm = kNegMax;
#pragma unroll
        for (int i = 0; i < kHeadBatch; ++i) {
            const uint32_t w4[4] = {kk[i].x, kk[i].y, kk[i].z, kk[i].w};
            float t = 0.0f;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float2 f = __half22float2(__builtin_bit_cast(__half2, w4[u]));
                t = __fmaf_rn(qv[2 * u], f.x, t);
                t = __fmaf_rn(qv[2 * u + 1], f.y, t);
            }
#pragma unroll
            for (int o = LPP / 2; o > 0; o >>= 1) t += __shfl_xor(t, o);
            sc[i] = ((b0 + kHeadWaves * i) * PPW + grp < seq) ? __fmul_rn(t, scale) : kNegMax;
            cm = fmaxf(cm, sc[i]);
        }
#pragma unroll
        for (int o = LPP; o < 64; o <<= 1) cm = fmaxf(cm, __shfl_xor(cm, o));
        const float m_new = fmaxf(m, cm);
        const float alpha = expf(m - m_new);
        float ls = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = __fmul_rn(acc[j], alpha);
#pragma unroll
        for (int i = 0; i < kHeadBatch; ++i) {
            const float e = ((b0 + kHeadWaves * i) * PPW + grp < seq) ? expf(sc[i] - m_new) : 0.0f;
            ls += e;
            const uint32_t w4[4] = {vv[i].x, vv[i].y, vv[i].z, vv[i].w};
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float2 f = __half22float2(__builtin_bit_cast(__half2, w4[u]));
                acc[2 * u] = __fmaf_rn(e, f.x, acc[2 * u]);
                acc[2 * u + 1] = __fmaf_rn(e, f.y, acc[2 * u + 1]);
            }
        }
#pragma unroll
        for (int o = LPP; o < 64; o <<= 1) ls += __shfl_xor(ls, o);
        l = __fmaf_rn(l, alpha, ls);
        m = m_new;
    }
    // (the wave holding the new position always has that slot, so the step
    // above ran; waves without positions leave m = kNegMax, l = 0)
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int o = LPP; o < 64; o <<= 1) acc[j] += __shfl_xor(acc[j], o);
    if (grp == 0) {
        *reinterpret_cast<float4*>(&wacc[wave][8 * sub]) = make_float4(acc[0], acc[1], acc[2], acc[3]);
        *reinterpret_cast<float4*>(&wacc[wave][8 * sub + 4]) = make_float4(acc[4], acc[5], acc[6], acc[7]);
    }
    if (lane == 0) {
        wm[wave] = m;
        wl[wave] = l;
    }
    __syncthreads();
    // out = sum_w e^(m_w - M) acc_w / sum_w e^(m_w - M) l_w in wave order
    // (waves without positions have l = 0 and count 0)
    for (int d = threadIdx.x; d < D; d += 64 * kHeadWaves) {
        float M = kNegMax;
#pragma unroll
        for (int w = 0; w < kHeadWaves; ++w) M = fmaxf(M, wm[w]);
        float lt = 0.0f, a = 0.0f;
#pragma unroll
        for (int w = 0; w < kHeadWaves; ++w) {
            const float f = wl[w] > 0.0f ? expf(wm[w] - M) : 0.0f;
            lt = __fmaf_rn(f, wl[w], lt);
            a = __fmaf_rn(f, wacc[w][d], a);
        }
        out[(size_t)head * D + d] = a * (1.0f / lt);
    }
}

// Workspace of the split path: the (m, l, acc) partials of every head and
// split, (D + 4) floats each, for at most kMaxSplits splits.  It is the
// caller's memory (rf_flash_attn_decode_workspace_bytes gives the size);
// launches that share one workspace must be stream-ordered.
constexpr int kMaxSplits = 64;
static size_t attn_ws_bytes(int nh, int d) { return (size_t)nh * kMaxSplits * (d + 4) * sizeof(float); }

static hipError_t attn_decode(float* out, const float* q, const __half* kc, const __half* vc, const int* len_ptr,
                              int len, int nh, int nkv, int d, float scale, float* ws, size_t ws_bytes,
                              hipStream_t st, const QkStep* qk = nullptr, int max_seq = 0) {
    if (out == nullptr || q == nullptr || kc == nullptr || vc == nullptr) return hipErrorInvalidValue;
    if (nh <= 0 || nkv <= 0 || nh % nkv != 0 || (len_ptr == nullptr && len <= 0)) return hipErrorInvalidValue;
    if (d != 64 && d != 128 && d != 256) return hipErrorInvalidValue;
    const int group = nh / nkv;
    if (max_seq > 0 && max_seq <= kHeadPathMaxSeq) {
        // one workgroup per query head (the sequence is at most max_seq long)
        const QkStep a = qk ? *qk : QkStep{};
#define RF_HEAD(LPP)                                                                                                   \
    if (qk)                                                                                                            \
        hipLaunchKernelGGL((rf_attn_head_kernel<LPP, true>), dim3(nh), dim3(64 * kHeadWaves), 0, st, q, kc, vc,        \
                           len_ptr, len, nh, nkv, scale, a, out);                                                      \
    else                                                                                                               \
        hipLaunchKernelGGL((rf_attn_head_kernel<LPP, false>), dim3(nh), dim3(64 * kHeadWaves), 0, st, q, kc, vc,       \
                           len_ptr, len, nh, nkv, scale, a, out)
        switch (d) {
        case 64: RF_HEAD(8); break;
        case 128: RF_HEAD(16); break;
        default: RF_HEAD(32); break;
        }
#undef RF_HEAD
        return hipGetLastError();
    }
    if (ws != nullptr && ws_bytes < attn_ws_bytes(nh, d)) return hipErrorInvalidValue;
    if (ws != nullptr && group <= 8) {
        int S = (2 * device_cu_count() + nkv - 1) / nkv;
        S = S < 1 ? 1 : (S > kMaxSplits ? kMaxSplits : S);
        if (len_ptr == nullptr) {
            const int chunks = (len + kSplitChunk - 1) / kSplitChunk;
            S = chunks < S ? chunks : S;
        }
        const dim3 grid(nkv, S), blk(64 * group);
        const QkStep a = qk ? *qk : QkStep{};
#define RF_SPLIT(LPP)                                                                                                  \
    if (qk)                                                                                                            \
        hipLaunchKernelGGL((rf_attn_split_kernel<LPP, true>), grid, blk, 0, st, q, kc, vc, len_ptr, len, nh, nkv,      \
                           scale, ws, S, a);                                                                           \
    else                                                                                                               \
        hipLaunchKernelGGL((rf_attn_split_kernel<LPP, false>), grid, blk, 0, st, q, kc, vc, len_ptr, len, nh, nkv,     \
                           scale, ws, S, a)
        switch (d) {
        case 64: RF_SPLIT(8); break;
        case 128: RF_SPLIT(16); break;
        default: RF_SPLIT(32); break;
        }
#undef RF_SPLIT
        hipLaunchKernelGGL(rf_attn_merge_kernel, dim3(nh), dim3(256), 0, st, ws, out, nh, d, S);
        return hipGetLastError();
    }
    if (qk) return hipErrorInvalidValue;      // the folded step needs the split path (workspace, GQA group <= 8)
    switch (d) {
    case 64: hipLaunchKernelGGL(rf_attn_decode_kernel<8>, dim3(nh), dim3(256), 0, st, out, q, kc, vc, len_ptr, len, nh,
                                nkv, scale); break;
    case 128: hipLaunchKernelGGL(rf_attn_decode_kernel<16>, dim3(nh), dim3(256), 0, st, out, q, kc, vc, len_ptr, len,
                                 nh, nkv, scale); break;
    default: hipLaunchKernelGGL(rf_attn_decode_kernel<32>, dim3(nh), dim3(256), 0, st, out, q, kc, vc, len_ptr, len,
                                nh, nkv, scale); break;
    }
    return hipGetLastError();
}

// ---- argmax (ties: the larger index) -----------------------------------------------------
constexpr int kArgmaxItems = 1024;   // per partial (the caller sizes partials as ceil(n / 1024))

__device__ __forceinline__ void amax_take(float v, int i, float& bv, int& bi) {
    if (v > bv || (v == bv && i > bi)) {
        bv = v;
        bi = i;
    }
}

__device__ __forceinline__ void amax_block(float& bv, int& bi, float* sv, int* si) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) amax_take(__shfl_xor(bv, o), __shfl_xor(bi, o), bv, bi);
    if ((threadIdx.x & 63) == 0) {
        sv[threadIdx.x >> 6] = bv;
        si[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    bv = sv[0];
    bi = si[0];
    for (int w = 1; w < 4; ++w) amax_take(sv[w], si[w], bv, bi);
}

__global__ __launch_bounds__(256) void rf_argmax_stage1_kernel(const float* __restrict__ x, float* pv, int* pi, int n) {
    __shared__ float sv[4];
    __shared__ int si[4];
    float bv = kNegMax;
    int bi = 0;
    const int base = blockIdx.x * kArgmaxItems;
#pragma unroll
    for (int t = 0; t < kArgmaxItems / 256; ++t) {
        const int i = base + threadIdx.x + 256 * t;
        if (i < n) amax_take(x[i], i, bv, bi);
    }
    amax_block(bv, bi, sv, si);
    if (threadIdx.x == 0) {
        pv[blockIdx.x] = bv;
        pi[blockIdx.x] = bi;
    }
}

__global__ __launch_bounds__(256) void rf_argmax_final_kernel(const float* __restrict__ pv, const int* __restrict__ pi,
                                                              int* out, int np, int* state) {
    __shared__ float sv[4];
    __shared__ int si[4];
    float bv = kNegMax;
    int bi = 0;
    for (int i = threadIdx.x; i < np; i += 256) amax_take(pv[i], pi[i], bv, bi);
    amax_block(bv, bi, sv, si);
    if (threadIdx.x == 0) {
        *out = bi;
        if (state != nullptr) {          // decode state {pos, seq_len} advanced with the token
            const int a = state[0], b = state[1];
            state[0] = a + 1;
            state[1] = b + 1;
        }
    }
}

// ---- Q4_K embedding rows ---------------------------------------------------------------
// One 256-thread workgroup per (super-block, token): thread t dequantises
// element t.  Tokens outside [0, vocab) leave their row untouched.
__global__ __launch_bounds__(256) void rf_embed_q4k_kernel(const uint8_t* __restrict__ emb,
                                                           const int* __restrict__ ids, int id0, float* out,
                                                           int hidden, int vocab) {
    const int s = blockIdx.y;
    const int tok = ids ? ids[s] : id0;
    if (tok < 0 || tok >= vocab) return;
    const int nb = hidden / kQK;
    const uint8_t* blk = emb + ((size_t)tok * nb + blockIdx.x) * kQ4KBytes;
    const int t = threadIdx.x;
    const int j = t / 32;                 // sub-block
    const uint8_t* sc = blk + 4;
    int scl, mn;
    if (j < 4) {
        scl = sc[j] & 63;
        mn = sc[j + 4] & 63;
    } else {
        scl = (sc[j + 4] & 0x0F) | ((sc[j - 4] >> 6) << 4);
        mn = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4);
    }
    const float d = half_bits_to_float(blk[0] | (blk[1] << 8));
    const float dmin = half_bits_to_float(blk[2] | (blk[3] << 8));
    const uint8_t qb = blk[16 + 32 * (j >> 1) + (t & 31)];
    const int nib = (j & 1) ? (qb >> 4) : (qb & 15);
    out[(size_t)s * hidden + blockIdx.x * kQK + t] = d * (float)scl * (float)nib - dmin * (float)mn;
}

// ---- elementwise ----------------------------------------------------------------------------
__global__ void rf_add_kernel(const float* __restrict__ x, const float* __restrict__ y, float* out, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = x[i] + y[i];
}
__global__ void rf_mul_kernel(const float* __restrict__ x, const float* __restrict__ y, float* out, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = x[i] * y[i];
}
__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }
__global__ void rf_silu_kernel(const float* __restrict__ x, float* out, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = silu_f(x[i]);
}
__global__ void rf_silu_mul_kernel(const float* __restrict__ g, const float* __restrict__ u, float* out, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = silu_f(g[i]) * u[i];
}
__global__ void rf_silu_mul_f16_kernel(const float* __restrict__ g, const float* __restrict__ u, __half* out, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) reinterpret_cast<uint16_t*>(out)[i] = f16_bits_rn(silu_f(g[i]) * u[i]);
}
__global__ void rf_f32_to_f16_kernel(const float* __restrict__ x, __half* out, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = __float2half(x[i]);
}
__global__ void rf_inc_state_kernel(int* st) {
    // vector stores only (one lane)
    if (threadIdx.x == 0) {
        const int a = st[0], b = st[1];
        st[0] = a + 1;
        st[1] = b + 1;
    }
}

static inline dim3 grid1(int n) { return dim3((unsigned)((n + 255) / 256)); }

}  // namespace rf

using namespace rf;

// ---- RMSNorm ----
extern "C" hipError_t gpu_rms_norm(const float* d_x, const float* d_weight, float* d_out, const int n, const float eps,
                                   hipStream_t stream) {
    return rms_rows(d_x, d_weight, d_out, n, eps, 1, stream);
}
extern "C" hipError_t gpu_rms_norm_batched_on_stream(const float* d_x, const float* d_weight, float* d_out, const int n,
                                                     const float eps, const int seq_len, hipStream_t stream) {
    return rms_rows(d_x, d_weight, d_out, n, eps, seq_len, stream);
}
extern "C" hipError_t gpu_rms_norm_batched(const float* d_x, const float* d_weight, float* d_out, const int n,
                                           const float eps, const int seq_len) {
    return rms_rows(d_x, d_weight, d_out, n, eps, seq_len, nullptr);
}
// fp16 output: __float2half of gpu_rms_norm_batched_on_stream's values
extern "C" hipError_t rf_rms_norm_batched_f16_on_stream(const float* d_x, const float* d_weight, uint16_t* d_out_f16,
                                                        const int n, const float eps, const int seq_len,
                                                        hipStream_t stream) {
    if (d_x == nullptr || d_weight == nullptr || d_out_f16 == nullptr || n <= 0 || seq_len <= 0)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(rf_rms_norm_long_kernel<__half>, dim3(seq_len), dim3(256), 0, stream, d_x, d_weight,
                       reinterpret_cast<__half*>(d_out_f16), n, eps, seq_len);
    return hipGetLastError();
}

// ---- RoPE ----
extern "C" hipError_t gpu_rope_heads_scaled(float* d_x, const int pos, const int num_heads, const int head_dim,
                                            const float theta_base, const int neox, const float* d_freq_scale,
                                            hipStream_t stream) {
    return rope_heads(d_x, nullptr, pos, num_heads, head_dim, theta_base, neox, d_freq_scale, 1, stream);
}
extern "C" hipError_t gpu_rope_heads(float* d_x, const int pos, const int num_heads, const int head_dim,
                                     const float theta_base, const int neox, hipStream_t stream) {
    return rope_heads(d_x, nullptr, pos, num_heads, head_dim, theta_base, neox, nullptr, 1, stream);
}
extern "C" hipError_t gpu_rope_heads_state_scaled(float* d_x, const int* d_pos, const int num_heads,
                                                  const int head_dim, const float theta_base, const int neox,
                                                  const float* d_freq_scale, hipStream_t stream) {
    if (d_pos == nullptr) return hipErrorInvalidValue;
    return rope_heads(d_x, d_pos, 0, num_heads, head_dim, theta_base, neox, d_freq_scale, 1, stream);
}
extern "C" hipError_t gpu_rope_heads_state(float* d_x, const int* d_pos, const int num_heads, const int head_dim,
                                           const float theta_base, const int neox, hipStream_t stream) {
    if (d_pos == nullptr) return hipErrorInvalidValue;
    return rope_heads(d_x, d_pos, 0, num_heads, head_dim, theta_base, neox, nullptr, 1, stream);
}
extern "C" hipError_t gpu_rope_heads_batched_scaled(float* d_x, const int start_pos, const int num_heads,
                                                    const int head_dim, const float theta_base, const int seq_len,
                                                    const int neox, const float* d_freq_scale) {
    return rope_heads(d_x, nullptr, start_pos, num_heads, head_dim, theta_base, neox, d_freq_scale, seq_len, nullptr);
}
extern "C" hipError_t gpu_rope_heads_batched(float* d_x, const int start_pos, const int num_heads, const int head_dim,
                                             const float theta_base, const int seq_len, const int neox) {
    return rope_heads(d_x, nullptr, start_pos, num_heads, head_dim, theta_base, neox, nullptr, seq_len, nullptr);
}
extern "C" hipError_t rf_rope_heads_batched_on_stream(float* d_x, const int start_pos, const int num_heads,
                                                      const int head_dim, const float theta_base, const int seq_len,
                                                      const int neox, const float* d_freq_scale, hipStream_t stream) {
    return rope_heads(d_x, nullptr, start_pos, num_heads, head_dim, theta_base, neox, d_freq_scale, seq_len, stream);
}

// ---- KV writes ----
static hipError_t kv_write_rope(uint16_t* kc, uint16_t* vc, const float* k, const float* v, const int* pos_ptr, int pos,
                                int nkv, int d, float base, int neox, const float* fs, hipStream_t st) {
    if (kc == nullptr || vc == nullptr || k == nullptr || v == nullptr || nkv <= 0 || d <= 0 || (d & 1))
        return hipErrorInvalidValue;
    const int pairs = nkv * (d / 2);
    hipLaunchKernelGGL(rf_kv_write_rope_kernel, grid1(pairs), dim3(256), 0, st, reinterpret_cast<__half*>(kc),
                       reinterpret_cast<__half*>(vc), k, v, pos_ptr, pos, nkv, d, base, neox, fs);
    return hipGetLastError();
}
extern "C" hipError_t gpu_kv_write_rope_scaled(uint16_t* d_k_cache, uint16_t* d_v_cache, const float* d_k, const float* d_v,
                                               const int pos, const int num_kv_heads, const int head_dim,
                                               const float theta_base, const int neox, const float* d_freq_scale,
                                               hipStream_t stream) {
    return kv_write_rope(d_k_cache, d_v_cache, d_k, d_v, nullptr, pos, num_kv_heads, head_dim, theta_base, neox,
                         d_freq_scale, stream);
}
extern "C" hipError_t gpu_kv_write_rope(uint16_t* d_k_cache, uint16_t* d_v_cache, const float* d_k, const float* d_v,
                                        const int pos, const int num_kv_heads, const int head_dim,
                                        const float theta_base, const int neox, hipStream_t stream) {
    return kv_write_rope(d_k_cache, d_v_cache, d_k, d_v, nullptr, pos, num_kv_heads, head_dim, theta_base, neox,
                         nullptr, stream);
}
extern "C" hipError_t gpu_kv_write_rope_state_scaled(uint16_t* d_k_cache, uint16_t* d_v_cache, const float* d_k,
                                                     const float* d_v, const int* d_pos, const int num_kv_heads,
                                                     const int head_dim, const float theta_base, const int neox,
                                                     const float* d_freq_scale, hipStream_t stream) {
    if (d_pos == nullptr) return hipErrorInvalidValue;
    return kv_write_rope(d_k_cache, d_v_cache, d_k, d_v, d_pos, 0, num_kv_heads, head_dim, theta_base, neox,
                         d_freq_scale, stream);
}
extern "C" hipError_t gpu_kv_write_rope_state(uint16_t* d_k_cache, uint16_t* d_v_cache, const float* d_k, const float* d_v,
                                              const int* d_pos, const int num_kv_heads, const int head_dim,
                                              const float theta_base, const int neox, hipStream_t stream) {
    if (d_pos == nullptr) return hipErrorInvalidValue;
    return kv_write_rope(d_k_cache, d_v_cache, d_k, d_v, d_pos, 0, num_kv_heads, head_dim, theta_base, neox, nullptr,
                         stream);
}
extern "C" hipError_t rf_kv_write_batched_on_stream(uint16_t* d_k_cache, uint16_t* d_v_cache, const float* d_k,
                                                    const float* d_v, const int start_pos, const int kv_size,
                                                    const int max_seq, const int seq_len, hipStream_t stream) {
    if (d_k_cache == nullptr || d_v_cache == nullptr || d_k == nullptr || d_v == nullptr || kv_size <= 0 ||
        seq_len <= 0 || start_pos < 0 || start_pos + seq_len > max_seq)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(rf_kv_write_batched_kernel, dim3((kv_size + 255) / 256, seq_len), dim3(256), 0, stream,
                       reinterpret_cast<__half*>(d_k_cache), reinterpret_cast<__half*>(d_v_cache), d_k, d_v, start_pos,
                       kv_size, seq_len);
    return hipGetLastError();
}
extern "C" hipError_t gpu_kv_write_batched(uint16_t* d_k_cache, uint16_t* d_v_cache, const float* d_k, const float* d_v,
                                           const int start_pos, const int kv_size, const int max_seq,
                                           const int seq_len) {
    return rf_kv_write_batched_on_stream(d_k_cache, d_v_cache, d_k, d_v, start_pos, kv_size, max_seq, seq_len,
                                         nullptr);
}

extern "C" hipError_t rf_qk_norm_rope_kv_write_state(float* d_q, const float* d_k, const float* d_v,
                                                     const float* d_q_norm, const float* d_k_norm, uint16_t* d_k_cache,
                                                     uint16_t* d_v_cache, const int* d_pos, const int num_heads,
                                                     const int num_kv_heads, const int head_dim, const float eps,
                                                     const float theta_base, const int neox,
                                                     const float* d_freq_scale, const float* d_theta,
                                                     const float* d_cos_sin, hipStream_t stream) {
    if (d_q == nullptr || d_k == nullptr || d_v == nullptr || d_k_cache == nullptr || d_v_cache == nullptr ||
        d_pos == nullptr || num_heads <= 0 || num_kv_heads <= 0)
        return hipErrorInvalidValue;
    if (reinterpret_cast<uintptr_t>(d_cos_sin) & 15u) return hipErrorInvalidValue;
    // 8-element vector loads of q/k/v and 16-byte fp16 stores into the caches
    for (const void* p : {(const void*)d_q, (const void*)d_k, (const void*)d_v, (const void*)d_k_cache,
                          (const void*)d_v_cache})
        if (reinterpret_cast<uintptr_t>(p) & 15u) return hipErrorInvalidValue;
    const int heads = num_heads + num_kv_heads;
    __half* kc = reinterpret_cast<__half*>(d_k_cache);
    __half* vc = reinterpret_cast<__half*>(d_v_cache);
#define RF_QKR(LPP)                                                                                                    \
    hipLaunchKernelGGL(rf_qk_norm_rope_kv_kernel<LPP>, dim3((heads + 4 * (64 / LPP) - 1) / (4 * (64 / LPP))),      \
                       dim3(256), 0, stream, d_q, d_k, d_v, d_q_norm, d_k_norm, kc, vc, d_pos, num_heads,         \
                       num_kv_heads, eps, d_theta, theta_base, neox, d_freq_scale,                              \
                       reinterpret_cast<const float2*>(d_cos_sin))
    switch (head_dim) {
    case 64: RF_QKR(8); break;
    case 128: RF_QKR(16); break;
    case 256: RF_QKR(32); break;
    default: return hipErrorInvalidValue;
    }
#undef RF_QKR
    return hipGetLastError();
}

extern "C" hipError_t rf_qk_norm_rope_kv_write_rows(const float* d_q, const float* d_k, const float* d_v,
                                                    const float* d_q_norm, const float* d_k_norm, uint16_t* d_q16,
                                                    uint16_t* d_k_cache, uint16_t* d_v_cache, const int start_pos,
                                                    const int rows_q, const int rows_kv, const int num_heads,
                                                    const int num_kv_heads, const int head_dim, const int max_seq,
                                                    const float eps, const float theta_base, const int neox,
                                                    const float* d_freq_scale, const float* d_theta,
                                                    const float* d_cos_sin, hipStream_t stream) {
    if (d_q == nullptr || d_k == nullptr || d_v == nullptr || d_q16 == nullptr || d_k_cache == nullptr ||
        d_v_cache == nullptr || num_heads <= 0 || num_kv_heads <= 0 || start_pos < 0 || rows_q <= 0 ||
        rows_kv < 0 || rows_kv > rows_q || rows_q > 65535 || start_pos + rows_kv > max_seq)
        return hipErrorInvalidValue;
    // the cos / sin table holds max_seq positions
    if (d_cos_sin != nullptr && ((reinterpret_cast<uintptr_t>(d_cos_sin) & 15u) || start_pos + rows_q > max_seq))
        return hipErrorInvalidValue;
    for (const void* p : {(const void*)d_q, (const void*)d_k, (const void*)d_v, (const void*)d_q16,
                          (const void*)d_k_cache, (const void*)d_v_cache})
        if (reinterpret_cast<uintptr_t>(p) & 15u) return hipErrorInvalidValue;
    const int heads = num_heads + num_kv_heads;
    __half* kc = reinterpret_cast<__half*>(d_k_cache);
    __half* vc = reinterpret_cast<__half*>(d_v_cache);
    __half* q16 = reinterpret_cast<__half*>(d_q16);
#define RF_QKR(LPP)                                                                                                    \
    hipLaunchKernelGGL(rf_qk_norm_rope_kv_rows_kernel<LPP>,                                                            \
                       dim3((heads + 4 * (64 / LPP) - 1) / (4 * (64 / LPP)), rows_q), dim3(256), 0, stream, d_q, d_k, \
                       d_v, d_q_norm, d_k_norm, q16, kc, vc, start_pos, rows_kv, num_heads, num_kv_heads, eps,        \
                       d_theta, theta_base, neox, d_freq_scale, reinterpret_cast<const float2*>(d_cos_sin))
    switch (head_dim) {
    case 64: RF_QKR(8); break;
    case 128: RF_QKR(16); break;
    case 256: RF_QKR(32); break;
    default: return hipErrorInvalidValue;
    }
#undef RF_QKR
    return hipGetLastError();
}

// ---- decode attention ----
// The reference-named launchers take no workspace: they run the
// one-workgroup-per-head kernel.  The _ws launchers run the split path in
// the caller's workspace.
extern "C" hipError_t gpu_flash_attn_decode_strided_multi_head(float* d_out, const float* d_q, const uint16_t* d_k_cache,
                                                               const uint16_t* d_v_cache, const int seq_len,
                                                               const int num_heads, const int num_kv_heads,
                                                               const int head_dim, const float scale,
                                                               hipStream_t stream) {
    return attn_decode(d_out, d_q, reinterpret_cast<const __half*>(d_k_cache),
                       reinterpret_cast<const __half*>(d_v_cache), nullptr, seq_len, num_heads, num_kv_heads, head_dim,
                       scale, nullptr, 0, stream);
}
extern "C" hipError_t gpu_flash_attn_decode_strided_multi_head_state(float* d_out, const float* d_q,
                                                                     const uint16_t* d_k_cache, const uint16_t* d_v_cache,
                                                                     const int* d_seq_len, const int num_heads,
                                                                     const int num_kv_heads, const int head_dim,
                                                                     const float scale, hipStream_t stream) {
    if (d_seq_len == nullptr) return hipErrorInvalidValue;
    return attn_decode(d_out, d_q, reinterpret_cast<const __half*>(d_k_cache),
                       reinterpret_cast<const __half*>(d_v_cache), d_seq_len, 0, num_heads, num_kv_heads, head_dim,
                       scale, nullptr, 0, stream);
}

extern "C" size_t rf_flash_attn_decode_workspace_bytes(const int num_heads, const int head_dim) {
    if (num_heads <= 0 || head_dim <= 0) return 0;
    return attn_ws_bytes(num_heads, head_dim);
}

extern "C" hipError_t rf_flash_attn_decode_ws(float* d_out, const float* d_q, const uint16_t* d_k_cache,
                                              const uint16_t* d_v_cache, const int seq_len, const int num_heads,
                                              const int num_kv_heads, const int head_dim, const float scale,
                                              float* d_workspace, const size_t workspace_bytes, hipStream_t stream) {
    if (d_workspace == nullptr) return hipErrorInvalidValue;
    return attn_decode(d_out, d_q, reinterpret_cast<const __half*>(d_k_cache),
                       reinterpret_cast<const __half*>(d_v_cache), nullptr, seq_len, num_heads, num_kv_heads, head_dim,
                       scale, d_workspace, workspace_bytes, stream);
}

extern "C" hipError_t rf_flash_attn_decode_state_ws(float* d_out, const float* d_q, const uint16_t* d_k_cache,
                                                    const uint16_t* d_v_cache, const int* d_seq_len,
                                                    const int num_heads, const int num_kv_heads, const int head_dim,
                                                    const float scale, float* d_workspace,
                                                    const size_t workspace_bytes, hipStream_t stream) {
    if (d_seq_len == nullptr || d_workspace == nullptr) return hipErrorInvalidValue;
    return attn_decode(d_out, d_q, reinterpret_cast<const __half*>(d_k_cache),
                       reinterpret_cast<const __half*>(d_v_cache), d_seq_len, 0, num_heads, num_kv_heads, head_dim,
                       scale, d_workspace, workspace_bytes, stream);
}

extern "C" hipError_t rf_attn_decode_qk_norm_rope_state(float* d_out, const float* d_q, const float* d_k,
                                                        const float* d_v, const float* d_q_norm,
                                                        const float* d_k_norm, uint16_t* d_k_cache, uint16_t* d_v_cache,
                                                        const int* d_state, const int num_heads,
                                                        const int num_kv_heads, const int head_dim, const float eps,
                                                        const float theta_base, const int neox,
                                                        const float* d_freq_scale, const float* d_theta,
                                                        const float* d_cos_sin, const float scale, float* d_workspace,
                                                        const size_t workspace_bytes, hipStream_t stream) {
    if (d_k == nullptr || d_v == nullptr || d_state == nullptr || d_workspace == nullptr) return hipErrorInvalidValue;
    if (reinterpret_cast<uintptr_t>(d_cos_sin) & 15u) return hipErrorInvalidValue;
    QkStep qk{d_k, d_v, d_q_norm, d_k_norm, reinterpret_cast<__half*>(d_k_cache), reinterpret_cast<__half*>(d_v_cache),
              eps, d_theta, theta_base, neox, d_freq_scale, reinterpret_cast<const float2*>(d_cos_sin)};
    return attn_decode(d_out, d_q, reinterpret_cast<const __half*>(d_k_cache),
                       reinterpret_cast<const __half*>(d_v_cache), d_state + 1, 0, num_heads, num_kv_heads, head_dim,
                       scale, d_workspace, workspace_bytes, stream, &qk);
}

// The same two launches for a caller that bounds the sequence: with
// max_seq <= kHeadPathMaxSeq (the caller guarantees seq <= max_seq) one
// workgroup per query head runs instead of the split kernel and its merge
// (rf_attn_head_kernel: no workspace, which may then be null); beyond it the
// split path and its workspace as above.
extern "C" hipError_t rf_flash_attn_decode_state_bounded(float* d_out, const float* d_q, const uint16_t* d_k_cache,
                                                         const uint16_t* d_v_cache, const int* d_seq_len,
                                                         const int num_heads, const int num_kv_heads,
                                                         const int head_dim, const float scale, const int max_seq,
                                                         float* d_workspace, const size_t workspace_bytes,
                                                         hipStream_t stream) {
    if (d_seq_len == nullptr || max_seq <= 0) return hipErrorInvalidValue;
    if (max_seq > kHeadPathMaxSeq && d_workspace == nullptr) return hipErrorInvalidValue;
    return attn_decode(d_out, d_q, reinterpret_cast<const __half*>(d_k_cache),
                       reinterpret_cast<const __half*>(d_v_cache), d_seq_len, 0, num_heads, num_kv_heads, head_dim,
                       scale, d_workspace, workspace_bytes, stream, nullptr, max_seq);
}

extern "C" hipError_t rf_attn_decode_qk_norm_rope_state_bounded(
    float* d_out, const float* d_q, const float* d_k, const float* d_v, const float* d_q_norm, const float* d_k_norm,
    uint16_t* d_k_cache, uint16_t* d_v_cache, const int* d_state, const int num_heads, const int num_kv_heads,
    const int head_dim, const float eps, const float theta_base, const int neox, const float* d_freq_scale,
    const float* d_theta, const float* d_cos_sin, const float scale, const int max_seq, float* d_workspace,
    const size_t workspace_bytes, hipStream_t stream) {
    if (d_k == nullptr || d_v == nullptr || d_state == nullptr || max_seq <= 0) return hipErrorInvalidValue;
    if (max_seq > kHeadPathMaxSeq && d_workspace == nullptr) return hipErrorInvalidValue;
    if (reinterpret_cast<uintptr_t>(d_cos_sin) & 15u) return hipErrorInvalidValue;
    QkStep qk{d_k, d_v, d_q_norm, d_k_norm, reinterpret_cast<__half*>(d_k_cache), reinterpret_cast<__half*>(d_v_cache),
              eps, d_theta, theta_base, neox, d_freq_scale, reinterpret_cast<const float2*>(d_cos_sin)};
    return attn_decode(d_out, d_q, reinterpret_cast<const __half*>(d_k_cache),
                       reinterpret_cast<const __half*>(d_v_cache), d_state + 1, 0, num_heads, num_kv_heads, head_dim,
                       scale, d_workspace, workspace_bytes, stream, &qk, max_seq);
}

// ---- decode attention without any allocation ----
// The split path's workspace as a file-scope device array: for callers that
// cannot allocate (hipMalloc is not allowed under stream capture, in tight
// serving loops or in harnesses that forbid it).  Each GPU holds its own copy
// from the first call on that device until the process ends.  In host code
// the array's name is only a stand-in: its device address is taken once per
// device with hipGetSymbolAddress and that address is what the kernels get.
// Every call on one GPU shares the array, so calls that overlap on a GPU
// (other streams, other threads) race; stream-ordered calls do not.  Nothing
// in it must start at zero: every split writes its partial (m, l) and the
// merge reads the accumulators of non-empty splits only.
constexpr size_t kNoAllocScratchBytes = (size_t)64 * kMaxSplits * (256 + 4) * sizeof(float);   // 4,259,840
static __device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];
constexpr int kMaxDevices = 64;
static float* g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mutex;

static hipError_t scratch_ptr(float** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (p == nullptr) return hipErrorInvalidSymbol;
        g_scratch_ptr[dev] = static_cast<float*>(p);
    }
    *out = g_scratch_ptr[dev];
    return hipSuccess;
}

extern "C" hipError_t rf_flash_attn_decode_state_noalloc(float* d_out, const float* d_q, const uint16_t* d_k_cache,
                                                         const uint16_t* d_v_cache, const int* d_seq_len,
                                                         const int num_heads, const int num_kv_heads,
                                                         const int head_dim, const float scale, hipStream_t stream) {
    if (d_seq_len == nullptr || num_heads <= 0 || head_dim <= 0) return hipErrorInvalidValue;
    const size_t need = attn_ws_bytes(num_heads, head_dim);
    if (need > kNoAllocScratchBytes) return hipErrorInvalidValue;    // beyond the array: num_heads * (head_dim + 4) > 16640
    float* ws = nullptr;
    const hipError_t e = scratch_ptr(&ws);
    if (e != hipSuccess) return e;
    return attn_decode(d_out, d_q, reinterpret_cast<const __half*>(d_k_cache),
                       reinterpret_cast<const __half*>(d_v_cache), d_seq_len, 0, num_heads, num_kv_heads, head_dim,
                       scale, ws, kNoAllocScratchBytes, stream);
}

// Caller-owned RoPE table: d_theta[i] = theta_i for i < head_dim / 2 (the
// values every launcher here uses), for the fused launchers' d_theta.
extern "C" hipError_t rf_rope_theta_table(float* d_theta, const int head_dim, const float theta_base,
                                          hipStream_t stream) {
    if (d_theta == nullptr || head_dim <= 0 || (head_dim & 1)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rf_theta_fill_kernel, dim3((head_dim / 2 + 255) / 256), dim3(256), 0, stream, d_theta,
                       head_dim, theta_base);
    return hipGetLastError();
}

// Caller-owned RoPE cos / sin table: d_cos_sin[2 * (pos * head_dim / 2 + i)
// + {0, 1}] = cos / sin of pos * theta_i for pos < positions, theta_i as the
// fused launchers evaluate it (d_theta when given, divided by d_freq_scale[i]
// when given).  The fused launchers' d_cos_sin takes it in place of cosf /
// sinf: the same values, so the same results.
extern "C" hipError_t rf_rope_cos_sin_table(float* d_cos_sin, const int positions, const int head_dim,
                                            const float theta_base, const float* d_theta, const float* d_freq_scale,
                                            hipStream_t stream) {
    if (d_cos_sin == nullptr || positions <= 0 || head_dim <= 0 || (head_dim & 1)) return hipErrorInvalidValue;
    const long n = (long)positions * (head_dim / 2);
    if (n > (1L << 30)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rf_rope_cos_sin_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                       reinterpret_cast<float2*>(d_cos_sin), positions, head_dim, theta_base, d_theta, d_freq_scale);
    return hipGetLastError();
}

// ---- argmax ----
extern "C" hipError_t gpu_argmax_f32_on_stream(const float* d_input, float* d_partial_values, int* d_partial_indices,
                                               int* d_output_index, const int n, hipStream_t stream) {
    if (d_input == nullptr || d_partial_values == nullptr || d_partial_indices == nullptr ||
        d_output_index == nullptr || n <= 0)
        return hipErrorInvalidValue;
    const int np = (n + kArgmaxItems - 1) / kArgmaxItems;
    hipLaunchKernelGGL(rf_argmax_stage1_kernel, dim3(np), dim3(256), 0, stream, d_input, d_partial_values,
                       d_partial_indices, n);
    hipLaunchKernelGGL(rf_argmax_final_kernel, dim3(1), dim3(256), 0, stream, d_partial_values, d_partial_indices,
                       d_output_index, np, nullptr);
    return hipGetLastError();
}
extern "C" hipError_t rf_argmax_f32_advance_state_on_stream(const float* d_input, float* d_partial_values,
                                                            int* d_partial_indices, int* d_output_index, const int n,
                                                            int* d_state, hipStream_t stream) {
    if (d_input == nullptr || d_partial_values == nullptr || d_partial_indices == nullptr ||
        d_output_index == nullptr || d_state == nullptr || n <= 0)
        return hipErrorInvalidValue;
    const int np = (n + kArgmaxItems - 1) / kArgmaxItems;
    hipLaunchKernelGGL(rf_argmax_stage1_kernel, dim3(np), dim3(256), 0, stream, d_input, d_partial_values,
                       d_partial_indices, n);
    hipLaunchKernelGGL(rf_argmax_final_kernel, dim3(1), dim3(256), 0, stream, d_partial_values, d_partial_indices,
                       d_output_index, np, d_state);
    return hipGetLastError();
}
extern "C" hipError_t gpu_argmax_f32(const float* d_input, float* d_partial_values, int* d_partial_indices,
                                     int* d_output_index, const int n) {
    return gpu_argmax_f32_on_stream(d_input, d_partial_values, d_partial_indices, d_output_index, n, nullptr);
}

// ---- embeddings ----
extern "C" hipError_t gpu_embed_q4_k_token(const uint8_t* d_embedding, float* d_out, const int hidden_size,
                                           const int vocab_size, const int token_id, hipStream_t stream) {
    if (d_embedding == nullptr || d_out == nullptr || hidden_size <= 0 || vocab_size <= 0 || token_id < 0 ||
        token_id >= vocab_size || hidden_size % kQK != 0)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(rf_embed_q4k_kernel, dim3(hidden_size / kQK, 1), dim3(256), 0, stream, d_embedding, nullptr,
                       token_id, d_out, hidden_size, vocab_size);
    return hipGetLastError();
}
extern "C" hipError_t gpu_embed_q4_k_batch(const uint8_t* d_embedding, const int* d_token_ids, float* d_out,
                                           const int hidden_size, const int vocab_size, const int seq_len,
                                           hipStream_t stream) {
    if (d_embedding == nullptr || d_token_ids == nullptr || d_out == nullptr || hidden_size <= 0 || vocab_size <= 0 ||
        seq_len <= 0 || hidden_size % kQK != 0)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(rf_embed_q4k_kernel, dim3(hidden_size / kQK, seq_len), dim3(256), 0, stream, d_embedding,
                       d_token_ids, 0, d_out, hidden_size, vocab_size);
    return hipGetLastError();
}

// ---- elementwise ----
extern "C" hipError_t gpu_add(const float* d_x, const float* d_y, float* d_out, const int n, hipStream_t stream) {
    if (n <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rf_add_kernel, grid1(n), dim3(256), 0, stream, d_x, d_y, d_out, n);
    return hipGetLastError();
}
extern "C" hipError_t gpu_mul_on_stream(const float* d_x, const float* d_y, float* d_out, const int n,
                                        hipStream_t stream) {
    if (n <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rf_mul_kernel, grid1(n), dim3(256), 0, stream, d_x, d_y, d_out, n);
    return hipGetLastError();
}
extern "C" hipError_t gpu_silu_on_stream(const float* d_x, float* d_out, const int n, hipStream_t stream) {
    if (n <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rf_silu_kernel, grid1(n), dim3(256), 0, stream, d_x, d_out, n);
    return hipGetLastError();
}
extern "C" hipError_t rf_silu_mul_on_stream(const float* d_gate, const float* d_up, float* d_out, const int n,
                                            hipStream_t stream) {
    if (d_gate == nullptr || d_up == nullptr || d_out == nullptr || n <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rf_silu_mul_kernel, grid1(n), dim3(256), 0, stream, d_gate, d_up, d_out, n);
    return hipGetLastError();
}
// fp16 output: __float2half of rf_silu_mul_on_stream's values
extern "C" hipError_t rf_silu_mul_f16_on_stream(const float* d_gate, const float* d_up, uint16_t* d_out_f16,
                                                const int n, hipStream_t stream) {
    if (d_gate == nullptr || d_up == nullptr || d_out_f16 == nullptr || n <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rf_silu_mul_f16_kernel, grid1(n), dim3(256), 0, stream, d_gate, d_up,
                       reinterpret_cast<__half*>(d_out_f16), n);
    return hipGetLastError();
}
extern "C" hipError_t convert_f32_to_f16(const float* input, void* output, int n, hipStream_t stream) {
    if (input == nullptr || output == nullptr || n <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rf_f32_to_f16_kernel, grid1(n), dim3(256), 0, stream, input, static_cast<__half*>(output), n);
    return hipGetLastError();
}
extern "C" hipError_t gpu_increment_decode_state_on_stream(int* d_state, hipStream_t stream) {
    if (d_state == nullptr) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rf_inc_state_kernel, dim3(1), dim3(64), 0, stream, d_state);
    return hipGetLastError();
}

// ---- prefill attention (causal, GQA), fp16 operands on MFMA ---------------------------
// Drop-in for wmma_attention_prefill_gqa_causal_launch
// (hip_kernels/wmma/wmma_attention_prefill.hip:711-750): Q [seq][nq*128],
// K, V [seq][nkv*128] fp16, O [seq][nq*128] fp32, seq % 64 == 0.  Same
// arithmetic as the reference: S = Q K^T accumulated in fp32 and scaled;
// keys in tiles of 64 with a running row max m; P = fp16(exp(S - m_new))
// for the tile, l = l * alpha + sum of the unrounded exps, O = O * alpha +
// P V (fp32 accumulate), out = O / l.
//
// Workgroup: 4 waves over 128 queries of one head (wave w: queries
// q0 + 32w ..), sharing the head's K tile ([key][dim]) and transposed V
// tile ([dim][key]) in LDS.  Each wave computes S^T = K Q^T (two 32x32
// blocks of v_mfma_f32_32x32x16_f16, Q^T from registers), so a lane owns
// one query column: the row max / sum are in-lane plus one exchange with
// lane ^ 32, alpha is a per-lane scale of the O^T accumulators, and the
// accumulator values of P feed the B operand of O^T = V^T P^T directly --
// the key order they come in is matched by the order the V^T operand is
// read in.  exp(x - m) is evaluated as 2^(x log2 e - m log2 e) (one
// v_exp_f32; within a few fp32 ulps of expf, P is rounded to fp16 anyway),
// the causal mask is applied only on the tiles that reach past a wave's
// first query, and O is rescaled only when some lane's maximum moved.  The
// next K / V tile is loaded into registers while the current one is used;
// V is written transposed as 32-bit key pairs, its keys permuted (bits 2
// and 3 swapped) so that the 8 keys of an operand are one 16-byte read, and
// XOR-swizzled by 8 ((dim / 8) % 8) so that the 16 threads writing one key
// pair (rows 8 apart) hit different banks.  Measured at 512 positions, 32
// heads, fp32 output: 26.5 us before these changes (and one wave per SIMD,
// the mask on diagonal tiles only), 17.4 after, the same bits.
namespace rf {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));

constexpr int kAttD = 128;
constexpr int kKStr = kAttD + 8;     // K tile row stride (halves)
constexpr int kVStr = 64 + 8;        // V^T tile row stride (halves)

// OUT = float, or uint16_t: fp16 bits of the fp32 output (round to nearest
// even), the operand a GEMM on fp16 activations reads
// One wave per SIMD (waves_per_eu 1): the whole register file for the
// accumulators and the prefetched tile (measured 22.8 against 26.5 us at 512
// positions, 32 heads).
template <int NWQ, typename OUT>
__global__ __launch_bounds__(64 * NWQ) __attribute__((amdgpu_waves_per_eu(1, 1))) void rf_attn_prefill_kernel(const _Float16* __restrict__ Q,
                                                              const _Float16* __restrict__ K,
                                                              const _Float16* __restrict__ V, OUT* __restrict__ O,
                                                              int seq, int nq, int nkv, int causal, float scale) {
    __shared__ __align__(16) _Float16 ks[64 * kKStr];
    __shared__ __align__(16) _Float16 vt[kAttD * kVStr];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int head = blockIdx.y;
    const int kvh = head / (nq / nkv);
    const int qb = blockIdx.x * 32 * NWQ;
    const int q0 = qb + 32 * wave;
    const int hi = lane >> 5, col = lane & 31;
    const size_t qrow = (size_t)nq * kAttD, kvrow = (size_t)nkv * kAttD;
    const bool active = q0 < seq;

    // Q^T operands of this lane's query: dims 16 ks + 8 hi .. + 7
    h8 qf[8];
#pragma unroll
    for (int ks_ = 0; ks_ < 8; ++ks_) {
        if (active)
            qf[ks_] = *reinterpret_cast<const h8*>(Q + (size_t)(q0 + col) * qrow + (size_t)head * kAttD + 16 * ks_ +
                                                   8 * hi);
        else
            qf[ks_] = h8{};
    }
    f16v o[4];
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[b][e] = 0.0f;
    float m = kNegMax, l = 0.0f;
    const int query = q0 + col;
    const float scale2 = scale * 1.4426950408889634f;   // log2 e

    const int wg_last_q = min(qb + 32 * NWQ - 1, seq - 1);
    const int ntiles = causal ? wg_last_q / 64 + 1 : seq / 64;
    const int wave_tiles = causal ? (q0 + 31) / 64 + 1 : seq / 64;
    // K / V tiles: thread chunk i = key c >> 4, dims (c & 15) * 8, c = tid +
    // 64 NWQ i; tile t + 1 is loaded into registers while tile t is used
    // (V: chunks 2 p, 2 p + 1 are keys 2 (tid / 16 + 4 NWQ p) and the next, so
    // the transposed tile takes them as one 32-bit key pair per dim)
    constexpr int NCH = 16 / NWQ;
    auto vkey = [&](int i) { return 2 * ((tid >> 4) + 4 * NWQ * (i >> 1)) + (i & 1); };
    auto vpos = [](int k) { return (k & ~12) | ((k & 4) << 1) | ((k & 8) >> 1); };
    h8 kr[NCH], vr[NCH];
    auto tile_load = [&](int t0) {
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
            const int c = tid + 64 * NWQ * i;
            const int key = c >> 4, d8 = (c & 15) * 8;
            kr[i] = *reinterpret_cast<const h8*>(K + (size_t)(t0 + key) * kvrow + (size_t)kvh * kAttD + d8);
            vr[i] = *reinterpret_cast<const h8*>(V + (size_t)(t0 + vkey(i)) * kvrow + (size_t)kvh * kAttD + d8);
        }
    };
    if (ntiles > 0) tile_load(0);
    for (int t = 0; t < ntiles; ++t) {
        const int t0 = 64 * t;
        __syncthreads();   // previous tile's reads done
        // K tile: 64 keys x 128 dims, 16-byte chunks; V tile transposed
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
            const int c = tid + 64 * NWQ * i;     // 0..1023
            const int key = c >> 4, d8 = (c & 15) * 8;
            const h8 kv = kr[i];
            *reinterpret_cast<h8*>(&ks[key * kKStr + d8]) = kv;
        }
        // V transposed: key k of a row at position vpos(k) ^ 8 ((d / 8) % 8),
        // vpos swapping bits 2 and 3 of the key (so the 8 keys an MFMA operand
        // takes, k .. k + 3 and k + 8 .. k + 11 for k % 8 = 0 or 4, are one
        // aligned 16-byte run), the XOR spreading the 16 threads of a key pair,
        // whose rows are 8 apart, over the banks
#pragma unroll
        for (int pi = 0; pi < NCH / 2; ++pi) {
            const int d8 = (tid & 15) * 8, k0 = vkey(2 * pi);
            const int sw = 8 * (tid & 7);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                typedef _Float16 h2 __attribute__((ext_vector_type(2)));
                const h2 pr = {vr[2 * pi][j], vr[2 * pi + 1][j]};
                *reinterpret_cast<h2*>(&vt[(d8 + j) * kVStr + (vpos(k0) ^ sw)]) = pr;
            }
        }
        if (t + 1 < ntiles) tile_load(t0 + 64);
        __syncthreads();
        if (!active || t >= wave_tiles) continue;

        // S^T = K Q^T: blocks b = keys 32 b .. + 31
        f16v s[2];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
#pragma unroll
            for (int e = 0; e < 16; ++e) s[b][e] = 0.0f;
#pragma unroll
            for (int ks_ = 0; ks_ < 8; ++ks_) {
                const h8 a = *reinterpret_cast<const h8*>(&ks[(32 * b + col) * kKStr + 16 * ks_ + 8 * hi]);
                s[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[ks_], s[b], 0, 0, 0);
            }
        }
        // scale (in the log2 domain: exp(x - m) = 2^(x log2 e - m log2 e), one
        // v_exp_f32 each), mask (only a tile that reaches past the wave's first
        // query holds keys to mask: a branch of its own, so the other tiles
        // carry no compare and select per element), tile max
        float tmax = kNegMax;
        const bool diag = causal && t0 + 63 > q0;
        if (diag) {
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    float v = s[b][e] * scale2;
                    const int key = t0 + 32 * b + 8 * (e >> 2) + 4 * hi + (e & 3);
                    if (key > query) v = kNegMax;
                    s[b][e] = v;
                    tmax = fmaxf(tmax, v);
                }
        } else {
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const float v = s[b][e] * scale2;
                    s[b][e] = v;
                    tmax = fmaxf(tmax, v);
                }
        }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
        const float m_new = fmaxf(m, tmax);
        const float alpha = __builtin_amdgcn_exp2f(m - m_new);
        float rs = 0.0f;
        h8 p[4];   // B operands, k-step j = (block j / 2, keys 16 (j % 2) ..)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const float ex = __builtin_amdgcn_exp2f(s[b][e] - m_new);
                rs += ex;
                p[2 * b + (e >> 3)][e & 7] = (_Float16)ex;
            }
        rs += __shfl_xor(rs, 32);
        l = l * alpha + rs;
        m = m_new;
        // rescale O only where some lane's maximum moved (alpha == 1 elsewhere:
        // multiplying by it changes nothing)
        if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {
#pragma unroll
            for (int b = 0; b < 4; ++b)
#pragma unroll
                for (int e = 0; e < 16; ++e) o[b][e] *= alpha;
        }
        // O^T += V^T P^T: A operand lane (dim = 32 bd + col) keys of k-step j in
        // the accumulator order: 32 (j/2) + 16 (j%2) + 4 hi + {0..3, 8..11}
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int kb = 32 * (j >> 1) + 16 * (j & 1) + 4 * hi;
#pragma unroll
            for (int bd = 0; bd < 4; ++bd) {
                // row d = 32 bd + col, keys kb .. kb + 3 and kb + 8 .. kb + 11: the
                // 16-byte run at vpos(kb) under the row's swizzle 8 ((d / 8) % 8)
                const int sw = 8 * ((4 * bd + (col >> 3)) & 7);
                const _Float16* vrow = &vt[(32 * bd + col) * kVStr];
                const h8 a = *reinterpret_cast<const h8*>(vrow + (vpos(kb) ^ sw));
                o[bd] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, p[j], o[bd], 0, 0, 0);
            }
        }
    }
    if (!active) return;
    const float inv_l = l > 0.0f ? 1.0f / l : 0.0f;
    OUT* orow = O + (size_t)query * qrow + (size_t)head * kAttD;
#pragma unroll
    for (int bd = 0; bd < 4; ++bd)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const float r = o[bd][e] * inv_l;
            if constexpr (std::is_same<OUT, float>::value)
                orow[32 * bd + 8 * (e >> 2) + 4 * hi + (e & 3)] = r;
            else
                orow[32 * bd + 8 * (e >> 2) + 4 * hi + (e & 3)] = f16_bits_rn(r);
        }
}

}  // namespace rf

template <typename OUT>
static hipError_t attn_prefill(const void* Q, const void* K, const void* V, OUT* O, int seq_len, int num_q_heads,
                               int num_kv_heads, int causal, float scale, hipStream_t stream) {
    if (Q == nullptr || K == nullptr || V == nullptr || O == nullptr) return hipErrorInvalidValue;
    if (num_q_heads <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads != 0) return hipErrorInvalidValue;
    if (seq_len <= 0 || seq_len % 64 != 0) return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(Q) | reinterpret_cast<uintptr_t>(K) | reinterpret_cast<uintptr_t>(V)) & 15u)
        return hipErrorInvalidValue;
    // four waves (128 queries) per workgroup: measured faster than two
    hipLaunchKernelGGL((rf::rf_attn_prefill_kernel<4, OUT>), dim3((seq_len + 127) / 128, num_q_heads), dim3(256), 0,
                       stream, static_cast<const _Float16*>(Q), static_cast<const _Float16*>(K),
                       static_cast<const _Float16*>(V), O, seq_len, num_q_heads, num_kv_heads, causal, scale);
    return hipGetLastError();
}

extern "C" hipError_t wmma_attention_prefill_gqa_causal_launch(const void* Q, const void* K, const void* V, float* O,
                                                               int seq_len, int num_q_heads, int num_kv_heads,
                                                               int causal, float scale, hipStream_t stream) {
    return attn_prefill(Q, K, V, O, seq_len, num_q_heads, num_kv_heads, causal, scale, stream);
}

// The same with the output rounded to fp16 (bits as uint16_t): the operand of
// an O projection on fp16 activations, __float2half of the fp32 launcher's.
extern "C" hipError_t rf_attention_prefill_gqa_causal_f16_launch(const void* Q, const void* K, const void* V,
                                                                 uint16_t* O_f16, int seq_len, int num_q_heads,
                                                                 int num_kv_heads, int causal, float scale,
                                                                 hipStream_t stream) {
    return attn_prefill(Q, K, V, O_f16, seq_len, num_q_heads, num_kv_heads, causal, scale, stream);
}
