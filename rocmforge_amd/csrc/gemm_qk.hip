// gemm_qk.hip -- Q4_K / Q6_K prefill GEMM on CDNA4 MFMA (gfx950).
//
// Drop-in for hip_kernels/wmma/wmma_gemm_q4_k.hip (wmma_gemm_q4_k_launch) and
// wmma_gemm_q6_k.hip (wmma_gemm_q6_k_launch):
//   D[M x N] (fp32) = fp16(A[M x K] fp32) * fp16(dequant W[N x K])^T,
// fp32 accumulation; M % 64 == 0, N % 64 == 0, K % 256 == 0.  The operand
// rounding is the reference's: A via __float2half (wmma_gemm_q4_k.hip:86),
// W via __float2half of the fp32 dequant value (:137, q6: :148).
//
// Design (wave64 MFMA, not the gfx12 WMMA tiling):
//  * Workgroup = 4 wave64s in a 2x2 grid over a BM x BN output tile; each
//    wave owns a (BM/2) x (BN/2) sub-tile built from 32x32 blocks of
//    v_mfma_f32_32x32x16_f16 (fp32 accumulators stay in registers).
//  * K advances in chunks of 64 (= one Q4_K nibble pair / half of a Q6_K
//    half-block).  Each chunk: A is read as fp32 and rounded to fp16, W is
//    dequantised in registers (2 threads per weight row, 16 bytes of packed
//    quants each) and both land in LDS as [row][k] fp16 with a padded row
//    stride; the next chunk's global loads are in flight while the MFMAs of
//    the current chunk run (register double buffering, two LDS buffers).
#include "qk_common.h"

namespace rf {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kGemmThreads = 256;
constexpr int kKC = 64;               // K per LDS stage
constexpr int kLdsStride = kKC + 8;   // halves per LDS row (16-byte pad against bank conflicts)

// ---- per-thread staged quant bytes for one chunk of one weight row --------
struct Q4Stage {
    u32x4 hdr;  // d, dmin, scales
    u32x4 qs;   // 16 bytes of the chunk's nibble pair (half h of 32)
};
struct Q6Stage {
    u32x4 lo, hi, qh;  // ql[64n+16h..], ql[64n+32+16h..], qh[32n+16h..]
    uint32_t sc;       // bytes: sc[8n+4t+h], sc[8n+4t+2+h] in the low 16 bits
    uint32_t d;
};

// Chunk c of a row covers k in [64c, 64c+64).  For Q4_K: super-block c/4,
// nibble pair p = c%4 (sub-blocks 2p -> k 0..31, 2p+1 -> k 32..63).
__device__ __forceinline__ Q4Stage q4_stage_load(const uint8_t* row, int c, int h) {
    const uint8_t* blk = row + (size_t)(c >> 2) * kQ4KBytes;
    Q4Stage s;
    s.hdr = *reinterpret_cast<const u32x4*>(blk);
    s.qs = *reinterpret_cast<const u32x4*>(blk + 16 + 32 * (c & 3) + 16 * h);
    return s;
}

// Dequantise to 2 x 16 halves: out0 = k (16h .. 16h+15), out1 = k (32+16h ..).
// value = fp16(d*sc*nib - dmin*m) evaluated in fp32 as the reference does.
__device__ __forceinline__ void q4_stage_dequant(const Q4Stage& s, int c, f16x8 out0[2], f16x8 out1[2]) {
    const int p = c & 3;
    int sc0, m0, sc1, m1;
    q4k_scale_min_pair(s.hdr.y, s.hdr.z, s.hdr.w, p, &sc0, &m0, &sc1, &m1);
    const float d = half_bits_to_float(s.hdr.x), dmin = half_bits_to_float(s.hdr.x >> 16);
    const float ds0 = d * (float)sc0, dm0 = dmin * (float)m0;
    const float ds1 = d * (float)sc1, dm1 = dmin * (float)m1;
    const uint32_t w[4] = {s.qs.x, s.qs.y, s.qs.z, s.qs.w};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const uint32_t byte = (w[t] >> (8 * b)) & 0xFFu;
            const int i = 4 * t + b;
            out0[i >> 3][i & 7] = (_Float16)(ds0 * (float)(byte & 15u) - dm0);
            out1[i >> 3][i & 7] = (_Float16)(ds1 * (float)(byte >> 4) - dm1);
        }
    }
}

// Q6_K chunk c: half n = (c%4)>>1, t = c&1 -> quarters q = 2t (k 0..31) and
// 2t+1 (k 32..63); thread h covers l in [16h, 16h+16).
__device__ __forceinline__ Q6Stage q6_stage_load(const uint8_t* row, int c, int h) {
    const uint8_t* blk = row + (size_t)(c >> 2) * kQ6KBytes;
    const int n = (c & 3) >> 1, t = c & 1;
    Q6Stage s;
    s.lo = ld16(blk + 64 * n + 16 * h);
    s.hi = ld16(blk + 64 * n + 32 + 16 * h);
    s.qh = ld16(blk + 128 + 32 * n + 16 * h);
    const uint32_t a = blk[192 + 8 * n + 4 * t + h];
    const uint32_t b = blk[192 + 8 * n + 4 * t + 2 + h];
    s.sc = a | (b << 8);
    s.d = ld_u16(blk + 208);
    return s;
}

__device__ __forceinline__ void q6_stage_dequant(const Q6Stage& s, int c, f16x8 out0[2], f16x8 out1[2]) {
    const int t = c & 1;
    const float d = half_bits_to_float(s.d);
    const float s0 = d * (float)(int8_t)(s.sc & 0xFFu);
    const float s1 = d * (float)(int8_t)((s.sc >> 8) & 0xFFu);
    const uint32_t L[4] = {s.lo.x, s.lo.y, s.lo.z, s.lo.w};
    const uint32_t H[4] = {s.hi.x, s.hi.y, s.hi.z, s.hi.w};
    const uint32_t Q[4] = {s.qh.x, s.qh.y, s.qh.z, s.qh.w};
    const uint32_t nsh = 4u * (uint32_t)t;          // low nibble for q<2, high for q>=2
    const uint32_t qsh0 = 2u * (uint32_t)(2 * t);   // qh shift for q = 2t
    const uint32_t qsh1 = qsh0 + 2u;                // q = 2t+1
#pragma unroll
    for (int w = 0; w < 4; ++w) {
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int i = 4 * w + b;
            const uint32_t sb = 8u * (uint32_t)b;
            const uint32_t qb = (Q[w] >> sb) & 0xFFu;
            const int q0 = (int)((((L[w] >> sb) >> nsh) & 15u) | (((qb >> qsh0) & 3u) << 4)) - 32;
            const int q1 = (int)((((H[w] >> sb) >> nsh) & 15u) | (((qb >> qsh1) & 3u) << 4)) - 32;
            out0[i >> 3][i & 7] = (_Float16)(s0 * (float)q0);
            out1[i >> 3][i & 7] = (_Float16)(s1 * (float)q1);
        }
    }
}

template <bool IS_Q6>
struct WStage;
template <>
struct WStage<false> { Q4Stage v; };
template <>
struct WStage<true> { Q6Stage v; };

// BM x BN workgroup tile, 2x2 waves, wave tile (BM/2) x (BN/2) of 32x32 MFMA blocks.
template <bool IS_Q6, int BM, int BN>
__global__ __launch_bounds__(kGemmThreads) void rf_gemm_qk_kernel(const float* __restrict__ A,
                                                                   const uint8_t* __restrict__ W,
                                                                   float* __restrict__ D, int M, int N, int K) {
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int FM = WM / 32, FN = WN / 32;
    constexpr int A_ROWS_PER_PASS = kGemmThreads / 2;   // 2 threads per A row (32 floats each)
    constexpr int A_PASSES = BM / A_ROWS_PER_PASS > 0 ? BM / A_ROWS_PER_PASS : 1;
    constexpr int W_PASSES = BN / (kGemmThreads / 2) > 0 ? BN / (kGemmThreads / 2) : 1;
    static_assert(BM % 64 == 0 && BN % 64 == 0, "tile");

    __shared__ __align__(16) _Float16 lds_a[2][BM * kLdsStride];
    __shared__ __align__(16) _Float16 lds_w[2][BN * kLdsStride];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int nchunks = K / kKC;
    const size_t row_bytes = (size_t)(K / kQK) * (IS_Q6 ? kQ6KBytes : kQ4KBytes);

    // staging assignment: thread -> (row, half)
    const int sr = tid >> 1, sh = tid & 1;
    const bool a_active = sr < BM || A_PASSES > 1;
    const bool w_active = sr < BN || W_PASSES > 1;

    float4 a_reg[A_PASSES][8];
    WStage<IS_Q6> w_reg[W_PASSES];

    auto load_chunk = [&](int c) {
#pragma unroll
        for (int ps = 0; ps < A_PASSES; ++ps) {
            const int r = sr + ps * A_ROWS_PER_PASS;
            if (r < BM) {
                const float4* src = reinterpret_cast<const float4*>(A + (size_t)(m0 + r) * K + c * kKC + 32 * sh);
#pragma unroll
                for (int i = 0; i < 8; ++i) a_reg[ps][i] = src[i];
            }
        }
#pragma unroll
        for (int ps = 0; ps < W_PASSES; ++ps) {
            const int r = sr + ps * (kGemmThreads / 2);
            if (r < BN) {
                const uint8_t* row = W + (size_t)(n0 + r) * row_bytes;
                if constexpr (IS_Q6) w_reg[ps].v = q6_stage_load(row, c, sh);
                else w_reg[ps].v = q4_stage_load(row, c, sh);
            }
        }
    };

    auto store_chunk = [&](int c, int buf) {
#pragma unroll
        for (int ps = 0; ps < A_PASSES; ++ps) {
            const int r = sr + ps * A_ROWS_PER_PASS;
            if (r < BM) {
                f16x8 h[4];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    h[i >> 1][4 * (i & 1) + 0] = (_Float16)a_reg[ps][i].x;
                    h[i >> 1][4 * (i & 1) + 1] = (_Float16)a_reg[ps][i].y;
                    h[i >> 1][4 * (i & 1) + 2] = (_Float16)a_reg[ps][i].z;
                    h[i >> 1][4 * (i & 1) + 3] = (_Float16)a_reg[ps][i].w;
                }
                f16x8* dst = reinterpret_cast<f16x8*>(&lds_a[buf][r * kLdsStride + 32 * sh]);
#pragma unroll
                for (int i = 0; i < 4; ++i) dst[i] = h[i];
            }
        }
#pragma unroll
        for (int ps = 0; ps < W_PASSES; ++ps) {
            const int r = sr + ps * (kGemmThreads / 2);
            if (r < BN) {
                f16x8 o0[2], o1[2];
                if constexpr (IS_Q6) q6_stage_dequant(w_reg[ps].v, c, o0, o1);
                else q4_stage_dequant(w_reg[ps].v, c, o0, o1);
                f16x8* d0 = reinterpret_cast<f16x8*>(&lds_w[buf][r * kLdsStride + 16 * sh]);
                f16x8* d1 = reinterpret_cast<f16x8*>(&lds_w[buf][r * kLdsStride + 32 + 16 * sh]);
                d0[0] = o0[0];
                d0[1] = o0[1];
                d1[0] = o1[0];
                d1[1] = o1[1];
            }
        }
    };
    (void)a_active;
    (void)w_active;

    f32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    load_chunk(0);
    store_chunk(0, 0);
    __syncthreads();

    const int frag_row = lane & 31;        // A row / W row (= output column) inside a 32-block
    const int frag_k = (lane >> 5) * 8;    // 8 consecutive k per lane
    for (int c = 0; c < nchunks; ++c) {
        const int buf = c & 1;
        if (c + 1 < nchunks) load_chunk(c + 1);
        const _Float16* la = lds_a[buf];
        const _Float16* lw = lds_w[buf];
#pragma unroll
        for (int kk = 0; kk < kKC; kk += 16) {
            f16x8 af[FM], bf[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i)
                af[i] = *reinterpret_cast<const f16x8*>(&la[(wm * WM + 32 * i + frag_row) * kLdsStride + kk + frag_k]);
#pragma unroll
            for (int j = 0; j < FN; ++j)
                bf[j] = *reinterpret_cast<const f16x8*>(&lw[(wn * WN + 32 * j + frag_row) * kLdsStride + kk + frag_k]);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if (c + 1 < nchunks) store_chunk(c + 1, buf ^ 1);
        __syncthreads();
    }

    // 32x32 accumulator layout: lane holds column (lane & 31), rows
    // 8*(e/4) + 4*(lane/32) + (e%4) for e = 0..15.
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int col = n0 + wn * WN + 32 * j + (lane & 31);
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = m0 + wm * WM + 32 * i + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                if (row < M) D[(size_t)row * N + col] = acc[i][j][e];
            }
        }
}

template <bool IS_Q6>
static hipError_t launch_gemm(const float* A, const void* W, float* D, int M, int N, int K, hipStream_t st) {
    const uint8_t* w = static_cast<const uint8_t*>(W);
    if (M % 128 == 0 && N % 128 == 0 && (size_t)(M / 128) * (N / 128) >= (size_t)device_cu_count()) {
        hipLaunchKernelGGL((rf_gemm_qk_kernel<IS_Q6, 128, 128>), dim3(N / 128, M / 128), dim3(kGemmThreads), 0, st,
                           A, w, D, M, N, K);
    } else {
        hipLaunchKernelGGL((rf_gemm_qk_kernel<IS_Q6, 64, 64>), dim3(N / 64, M / 64), dim3(kGemmThreads), 0, st, A,
                           w, D, M, N, K);
    }
    return hipGetLastError();
}

}  // namespace rf

using namespace rf;

// Validation as wmma_gemm_q4_k.hip:513-516 / wmma_gemm_q6_k.hip:220-223,
// plus 16-byte alignment of A (read as float4) and of Q4_K weights.
extern "C" hipError_t wmma_gemm_q4_k_launch(const float* input, const void* weights_q4_k, float* output, int M, int N,
                                            int K, hipStream_t stream) {
    if (M <= 0 || N <= 0 || K <= 0) return hipErrorInvalidValue;
    if ((M % 64) != 0 || (N % 64) != 0 || (K % kQK) != 0) return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(input) & 15u) || (reinterpret_cast<uintptr_t>(weights_q4_k) & 15u))
        return hipErrorInvalidValue;
    return launch_gemm<false>(input, weights_q4_k, output, M, N, K, stream);
}

extern "C" hipError_t wmma_gemm_q6_k_launch(const float* input, const void* weights_q6_k, float* output, int M, int N,
                                            int K, hipStream_t stream) {
    if (M <= 0 || N <= 0 || K <= 0) return hipErrorInvalidValue;
    if ((M % 64) != 0 || (N % 64) != 0 || (K % kQK) != 0) return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(input) & 15u) || (reinterpret_cast<uintptr_t>(weights_q6_k) & 1u))
        return hipErrorInvalidValue;
    return launch_gemm<true>(input, weights_q6_k, output, M, N, K, stream);
}
