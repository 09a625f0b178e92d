// gemm_qk.hip -- Q4_K / Q6_K prefill GEMM on CDNA4 MFMA (gfx950).
//
// Drop-in for hip_kernels/wmma/wmma_gemm_q4_k.hip (wmma_gemm_q4_k_launch) and
// wmma_gemm_q6_k.hip (wmma_gemm_q6_k_launch):
//   D[M x N] (fp32) = fp16(A[M x K] fp32) * fp16(dequant W[N x K])^T,
// fp32 accumulation; M % 64 == 0, N % 64 == 0, K % 256 == 0.  The operand
// rounding is the reference's: A via __float2half (wmma_gemm_q4_k.hip:86),
// W via __float2half of the fp32 dequant value (:137, q6: :148).
//
// Routing.  The fp32-activation launchers (the two above, and the segments /
// accumulate / SwiGLU launchers below) round A to fp16 in a pass of their
// own into library-owned device memory (the same values the reference's
// __float2half gives) and run the fp16-activation tiles:
//  * rf_gemm_q4k_f16a_kernel (Q4_K where 256 x 128 tiles fill at least 3/4
//    of the CUs): 4 waves, each weight dequantised once per 256 rows of A,
//    A and the weight ring by LDS DMA.
//  * rf_gemm_q4k_f16s_kernel (Q4_K otherwise) and rf_gemm_q6k_f16a_kernel
//    (Q6_K, K % 2048 == 0): 8 waves over 64- or 128-row x 64-column tiles, K
//    sliced over waves and added through LDS; when the tiles leave at least
//    half the CUs idle, K is also split over workgroups whose partial tiles
//    rf_gemm_split_reduce_kernel adds in split order.
// Every output is one fixed-order sum: no float atomics, the same bits on
// every run.  When no staging memory is free for the stream (or Q6_K rows are
// not 16-byte aligned) the fp32-activation kernels run, one workgroup per
// tile:
//  * rf_gemm_qk_sq_kernel (N % 256 == 0, K % 512 == 0, and 256 x 256 or
//    128 x 128 tiles that come to about one workgroup per CU): 2 x 2 waves,
//    each weight dequantised once per workgroup into an LDS B tile shared by
//    the two waves that use it.
//  * rf_gemm_qk_v7_kernel (otherwise when N % 256 == 0, K % 512 == 0 and,
//    for Q6_K, K % 2048 == 0): 256-thread workgroups, one wave per SIMD,
//    over a BM x 256 tile; weights stage through an LDS ring with coalesced
//    loads, each wave dequantises its own B operands (the next chunk's,
//    double buffered) in hand-scheduled slots between its MFMAs; XCD-aware
//    tile order.
//  * rf_gemm_qk_v4_kernel: 8 waves, weights loaded per lane (Q6_K with
//    K % 2048 != 0, whose rows are not 16-byte aligned for the ring).
//  * rf_gemm_qk_kernel (any M % 64 == 0, N % 64 == 0, K % 256 == 0): the
//    general fallback.  4 wave64s in a 2x2 grid over a BM x BN tile of 32x32
//    blocks of v_mfma_f32_32x32x16_f16; each 64-wide K chunk of A (fp32 ->
//    fp16) and of W (dequantised in registers, 2 threads per weight row)
//    lands in LDS as [row][k] fp16 with a padded stride, double buffered.
// Launchers with no reference counterpart: several weight matrices over one
// input as column segments of a single launch (rf_gemm_q*_k_segments_launch,
// rf_gemm_qk_f16_segments_launch), D += product (*_accumulate_launch) and
// gate/up pairs with SwiGLU in the epilogue (*_swiglu_launch).
#include <algorithm>
#include <mutex>
#include <type_traits>

#include "qk_common.h"


namespace rf {

// Row-block band of the v7 tile order (measured best at the Llama-3.1-8B
// FFN shapes).
constexpr int kGemmBand = 2;

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// fp16 (round to nearest even) of two fp32 values as an instruction of its
// own.  The reference rounds the fp32 dequant value with __float2half
// (wmma_gemm_q4_k.hip:137): two roundings, exact value -> fp32 -> fp16.  Left
// to itself the compiler merges an FMA and its fp16 conversion into one
// v_fma_mix with an fp16 result, which rounds the exact value once; for Q4_K
// (d sc q - dmin m) the two differ in about one weight in 10^7.  Q6_K values
// d sc (q - 32) are exact in fp32, so there one rounding is the same.
__device__ __forceinline__ uint32_t cvt_pk_f16(float lo, float hi) {
    uint32_t r;
    asm("v_cvt_pk_f16_f32 %0, %1, %2" : "=v"(r) : "v"(lo), "v"(hi));
    return r;
}

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
            const uint32_t h = cvt_pk_f16(ds0 * (float)(byte & 15u) - dm0, ds1 * (float)(byte >> 4) - dm1);
            out0[i >> 3][i & 7] = __builtin_bit_cast(_Float16, (unsigned short)(h & 0xFFFFu));
            out1[i >> 3][i & 7] = __builtin_bit_cast(_Float16, (unsigned short)(h >> 16));
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

// ── v4: 8 waves, two per SIMD; A through LDS, W dequantised per lane ──────
// Workgroup = 512 threads = 8 wave64s.  Wave w owns output columns
// [n0 + 64*(w&3), +64) (two 32-column MFMA blocks) for all BM = 32*FM rows
// of the tile, and the K half kh = w>>2 of every 64-wide chunk: waves w and
// w+4 (same SIMD) compute partial sums of the same outputs over disjoint k,
// which are added through LDS at the end.  With two waves per SIMD one
// wave's MFMAs run while the other dequantises or waits on memory.  Every
// weight is dequantised exactly once per M tile, in the register of the lane
// whose MFMA B operand needs it; A is rounded to fp16 once per tile into LDS.
//
// K order inside a chunk.  A dot product does not depend on the order of its
// terms, so the MFMA k index may be any permutation of the chunk's physical k
// as long as A and B use the same one.  Wave half kh, k16 step s2 (0..1),
// lane half h = lane >> 5, slot e (0..7):
//     physical k = 32*kh + 16*h + 8*s2 + e
// so a lane's B operands for its half chunk come from ONE 16 B run of quant
// bytes per row, and its A operand for step s2 is LDS row m, columns
// [32kh + 16h + 8s2, +8).
//   Q4_K chunk CQ (nibble pair CQ): k < 32 -> low nibble of qs byte 32CQ + k,
//   k >= 32 -> high nibble of qs byte 32CQ + k - 32; both halves read qs bytes
//   [32CQ + 16h, +16): byte j -> step j>>3, slot j&7, low nibble for kh = 0,
//   high nibble for kh = 1.
//   Q6_K chunk CQ (half nh = CQ>>1, t = CQ&1): quarter q = 2t + kh,
//   l = k % 32 = 16h + j; ql byte 64nh + 32kh + l (high nibble iff t = 1),
//   qh byte 32nh + l (bits 2q), scale sc[8nh + 2q + h] = byte (2kh + h) of
//   scale word CQ (sc bytes [4CQ, 4CQ+4)).
struct Q4Hdr {
    u32x4 v;   // d, dmin, scales[12]
};
struct Q4Qs {
    u32x4 q;   // qs bytes [32CQ + 16h, +16)
};
struct Q6Hdr {
    uint32_t d;  // fp16 bits of d (bytes 208..209 in the low half)
};
struct Q6Qs {
    u32x4 ql;      // ql [64nh + 32kh + 16h, +16)
    u32x4 qh;      // qh [32nh + 16h, +16)
    uint32_t sc;   // scales [4CQ, 4CQ+4)
};

__device__ __forceinline__ void put4(f16x8& dst, int half, float a, float b, float c, float d) {
    dst[4 * half + 0] = (_Float16)a;
    dst[4 * half + 1] = (_Float16)b;
    dst[4 * half + 2] = (_Float16)c;
    dst[4 * half + 3] = (_Float16)d;
}
// the same with the fp32 values rounded as the reference rounds them (Q4_K)
__device__ __forceinline__ void put4_rn(f16x8& dst, int half, float a, float b, float c, float d) {
    u32x4 v = __builtin_bit_cast(u32x4, dst);
    v[2 * half] = cvt_pk_f16(a, b);
    v[2 * half + 1] = cvt_pk_f16(c, d);
    dst = __builtin_bit_cast(f16x8, v);
}
__device__ __forceinline__ float byte_f(uint32_t w, int i) { return (float)((w >> (8 * i)) & 0xFFu); }

// Q4_K: B operands of one column for the wave's two k16 steps.  Nibbles are
// converted with byte converts on masked words: low nibbles via
// w & 0x0F0F0F0F, high nibbles via w & 0xF0F0F0F0 (= 16 * nibble) with the
// scale divided by 16 -- a power of two, so (ds/16) * (16 n) == ds * n
// exactly and the fp32 value ds*n - dm (and its fp16 rounding) is the
// reference's.
struct Q4Ops {
    using Hdr = Q4Hdr;
    using Qs = Q4Qs;
    static constexpr int kBytes = kQ4KBytes;
    static constexpr bool kHdrPerBlock = true;
    static __device__ __forceinline__ Hdr hdr(const uint8_t* row, int sb) {
        return Hdr{*reinterpret_cast<const u32x4*>(row + (size_t)sb * kQ4KBytes)};
    }
    template <int CQ>
    static __device__ __forceinline__ Qs qs(const uint8_t* row, int sb, int h, int /*kh*/) {
        return Qs{*reinterpret_cast<const u32x4*>(row + (size_t)sb * kQ4KBytes + 16 + 32 * CQ + 16 * h)};
    }
    template <int CQ, int KH>
    static __device__ __forceinline__ void dequant_k(const Hdr& hd, const Qs& r, int /*h*/, f16x8 (&b)[2]) {
        int sc0, m0, sc1, m1;
        q4k_scale_min_pair(hd.v.y, hd.v.z, hd.v.w, CQ, &sc0, &m0, &sc1, &m1);
        const float d = half_bits_to_float(hd.v.x), dmin = half_bits_to_float(hd.v.x >> 16);
        const float ds = KH ? d * (float)sc1 * 0.0625f : d * (float)sc0;
        const float dm = KH ? dmin * (float)m1 : dmin * (float)m0;
        constexpr uint32_t mask = KH ? 0xF0F0F0F0u : 0x0F0F0F0Fu;
        const uint32_t w[4] = {r.q.x & mask, r.q.y & mask, r.q.z & mask, r.q.w & mask};
#pragma unroll
        for (int j = 0; j < 4; ++j)
            put4_rn(b[j >> 1], j & 1, ds * byte_f(w[j], 0) - dm, ds * byte_f(w[j], 1) - dm,
                    ds * byte_f(w[j], 2) - dm, ds * byte_f(w[j], 3) - dm);
    }
    template <int CQ>
    static __device__ __forceinline__ void dequant(const Hdr& hd, const Qs& r, int h, int kh, f16x8 (&b)[2]) {
        int sc0, m0, sc1, m1;
        q4k_scale_min_pair(hd.v.y, hd.v.z, hd.v.w, CQ, &sc0, &m0, &sc1, &m1);
        const float d = half_bits_to_float(hd.v.x), dmin = half_bits_to_float(hd.v.x >> 16);
        const float ds = kh ? d * (float)sc1 * 0.0625f : d * (float)sc0;
        const float dm = kh ? dmin * (float)m1 : dmin * (float)m0;
        const uint32_t mask = kh ? 0xF0F0F0F0u : 0x0F0F0F0Fu;
        const uint32_t w[4] = {r.q.x & mask, r.q.y & mask, r.q.z & mask, r.q.w & mask};
#pragma unroll
        for (int j = 0; j < 4; ++j)   // word j = bytes 4j..4j+3: step j>>1, slots 4*(j&1) + [0,4)
            put4_rn(b[j >> 1], j & 1, ds * byte_f(w[j], 0) - dm, ds * byte_f(w[j], 1) - dm,
                    ds * byte_f(w[j], 2) - dm, ds * byte_f(w[j], 3) - dm);
    }
};

// Q6_K: q = (ql nibble | qh bits << 4) in 0..63, value = s * (q - 32)
// evaluated as s*q - 32s: s*q, 32s and their difference s*(q-32) are all
// exact in fp32 (|s| has at most 19 significant bits, q at most 6), so the
// fp32 value is the reference's d * sc * (q - 32).
struct Q6Ops {
    using Hdr = Q6Hdr;
    using Qs = Q6Qs;
    static constexpr int kBytes = kQ6KBytes;
    static constexpr bool kHdrPerBlock = true;
    static __device__ __forceinline__ Hdr hdr(const uint8_t* row, int sb) {
        return Hdr{ld_u16(row + (size_t)sb * kQ6KBytes + 208)};
    }
    template <int CQ>
    static __device__ __forceinline__ Qs qs(const uint8_t* row, int sb, int h, int kh) {
        constexpr int nh = CQ >> 1;
        const uint8_t* blk = row + (size_t)sb * kQ6KBytes;
        return Qs{ld16(blk + 64 * nh + 32 * kh + 16 * h), ld16(blk + 128 + 32 * nh + 16 * h), ld4(blk + 192 + 4 * CQ)};
    }
    template <int CQ, int KH>
    static __device__ __forceinline__ void dequant_k(const Hdr& hd, const Qs& r, int h, f16x8 (&b)[2]) {
        dequant<CQ>(hd, r, h, KH, b);
    }
    template <int CQ>
    static __device__ __forceinline__ void dequant(const Hdr& hd, const Qs& r, int h, int kh, f16x8 (&b)[2]) {
        constexpr int t = CQ & 1;
        const float d = half_bits_to_float(hd.d);
        const float s = d * (float)(int8_t)((r.sc >> (8 * (2 * kh + h))) & 0xFFu);
        const float o = 32.0f * s;
        constexpr uint32_t nsh = 4u * t;                   // low nibble for q < 2, high for q >= 2
        const uint32_t qsh = 4u * t + 2u * (uint32_t)kh;   // qh shift 2q
        const uint32_t L[4] = {r.ql.x, r.ql.y, r.ql.z, r.ql.w};
        const uint32_t QH[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t q = ((L[j] >> nsh) & 0x0F0F0F0Fu) | (((QH[j] >> qsh) & 0x03030303u) << 4);
            put4(b[j >> 1], j & 1, s * byte_f(q, 0) - o, s * byte_f(q, 1) - o, s * byte_f(q, 2) - o,
                 s * byte_f(q, 3) - o);
        }
    }
};

constexpr int kV4Threads = 512;
constexpr int kV4LdsBytes = 65536;

// Chunk pipeline (K advances 64 per chunk; this workgroup's chunks are
// [c_begin, c_last], c_begin and the count multiples of 8):
//   iteration c:  (1) A(c+1) registers -> fp16 -> LDS buffer (c+1)&1
//                 (2) W(c) quant registers (+ super-block header) -> B operands
//                 (3) issue global loads of A(c+3) and W(c+2) (+ the header of
//                     the super-block W(c+2) starts, if it starts one)
//                 (4) 2 k16 steps x FM x 2 MFMAs from LDS buffer c&1
//                 (5) LDS-only barrier (outstanding global loads stay in flight)
// A and W loads have two iterations to land.  Register sets are indexed by
// chunk parity (A staging, quant bytes) and super-block parity (headers); the
// loop is unrolled over 8 chunks so every index is static.  Loads past c_last
// re-read the chunk four back (same position in its super-block).
// The grid is tiles x splits, split s covering an equal run of chunks; the
// launchers use one split (chunks_per_split = K / 64).
template <typename T, int FM>
__global__ __launch_bounds__(kV4Threads) void rf_gemm_qk_v4_kernel(const float* __restrict__ A,
                                                                    const uint8_t* __restrict__ W,
                                                                    float* __restrict__ D, int M, int N, int K,
                                                                    int tiles, int chunks_per_split) {
    constexpr int BM = 32 * FM;
    constexpr int BN = 256;
    constexpr int A_F4 = BM * kKC / 4 / kV4Threads;   // float4 per thread per chunk
    constexpr int A_BUF = BM * kLdsStride;             // halves per A buffer
    static_assert(2 * A_BUF * 2 <= kV4LdsBytes, "A buffers");
    static_assert(4 * (FM / 2) * 2 * 16 * 64 * 4 <= kV4LdsBytes, "reduction buffer");
    __shared__ __align__(16) uint8_t lds[kV4LdsBytes];
    _Float16* lds_a = reinterpret_cast<_Float16*>(lds);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = wave & 3, kh = wave >> 2;
    const int h = lane >> 5;
    const int tile = blockIdx.x % tiles;
    const int split = blockIdx.x / tiles;
    const int ntiles = N / BN;
    const int m0 = (tile / ntiles) * BM;
    const int n0 = (tile % ntiles) * BN + wn * 64;
    const int c_begin = split * chunks_per_split;
    const int c_last = c_begin + chunks_per_split - 1;
    const size_t row_bytes = (size_t)(K / kQK) * T::kBytes;
    const uint8_t* wrow0 = W + (size_t)(n0 + (lane & 31)) * row_bytes;
    const uint8_t* wrow1 = wrow0 + 32 * row_bytes;

    // A staging, coalesced: float4 f = i*512 + tid of the BM x 64 chunk is
    // row f/16, columns 4*(f%16) .. +3 (a wave instruction covers 4 rows).
    const int a_row = tid >> 4;
    const int a_col = 4 * (tid & 15);
    const float* a_base = A + (size_t)(m0 + a_row) * K + a_col;
    float4 a_reg[2][A_F4];
    typename T::Hdr hdr[2][2];   // [super-block parity][row]
    typename T::Qs qsr[2][2];    // [chunk parity][row]

    auto a_load = [&](float4 (&r)[A_F4], int c) {
        const float* src = a_base + (size_t)min(c, c_last) * kKC;
#pragma unroll
        for (int i = 0; i < A_F4; ++i) r[i] = *reinterpret_cast<const float4*>(src + (size_t)(32 * i) * K);
    };
    auto a_store = [&](const float4 (&r)[A_F4], int buf) {
        _Float16* dst = lds_a + buf * A_BUF + a_row * kLdsStride + a_col;
#pragma unroll
        for (int i = 0; i < A_F4; ++i) {
            f16x4 hv;
            hv[0] = (_Float16)r[i].x; hv[1] = (_Float16)r[i].y;
            hv[2] = (_Float16)r[i].z; hv[3] = (_Float16)r[i].w;
            *reinterpret_cast<f16x4*>(dst + 32 * i * kLdsStride) = hv;
        }
    };
    // W(c) with c = c8 + J (J static, c8 a multiple of 8)
    auto w_load = [&](auto jj, int c8) {
        constexpr int J = decltype(jj)::value;
        constexpr int JQ = J & 3;
        int sb = c8 / 4 + (J >> 2);
        if (c8 + J > c_last) --sb;
        if constexpr (JQ == 0) {
            hdr[(J >> 2) & 1][0] = T::hdr(wrow0, sb);
            hdr[(J >> 2) & 1][1] = T::hdr(wrow1, sb);
        }
        qsr[J & 1][0] = T::template qs<JQ>(wrow0, sb, h, kh);
        qsr[J & 1][1] = T::template qs<JQ>(wrow1, sb, h, kh);
    };

    f32x16 acc[FM][2];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    const int frag = (lane & 31) * kLdsStride + 32 * kh + 16 * h;
    // iteration I of the 8-chunk group starting at chunk c8
    auto iteration = [&](auto it, int c8) {
        constexpr int I = decltype(it)::value;
        constexpr int P = I & 1;
        const int c = c8 + I;
        __builtin_amdgcn_sched_barrier(0);
        a_store(a_reg[P ^ 1], P ^ 1);
        f16x8 bq[2][2];
        T::template dequant<I & 3>(hdr[(I >> 2) & 1][0], qsr[P][0], h, kh, bq[0]);
        T::template dequant<I & 3>(hdr[(I >> 2) & 1][1], qsr[P][1], h, kh, bq[1]);
        a_load(a_reg[P ^ 1], c + 3);
        w_load(std::integral_constant<int, I + 2>{}, c8);
        const _Float16* la = lds_a + P * A_BUF + frag;
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
            f16x8 af[FM];
#pragma unroll
            for (int i = 0; i < FM; ++i) af[i] = *reinterpret_cast<const f16x8*>(la + 32 * i * kLdsStride + 8 * s2);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bq[j][s2], acc[i][j], 0, 0, 0);
        }
        lds_barrier();
    };

    // prologue: A(c0) -> LDS 0; A(c0+1), A(c0+2), W(c0), W(c0+1) in flight
    a_load(a_reg[0], c_begin);
    w_load(std::integral_constant<int, 0>{}, c_begin);
    a_load(a_reg[1], c_begin + 1);
    w_load(std::integral_constant<int, 1>{}, c_begin);
    a_store(a_reg[0], 0);
    a_load(a_reg[0], c_begin + 2);
    lds_barrier();

    for (int c8 = c_begin; c8 <= c_last; c8 += 8) {
        iteration(std::integral_constant<int, 0>{}, c8);
        iteration(std::integral_constant<int, 1>{}, c8);
        iteration(std::integral_constant<int, 2>{}, c8);
        iteration(std::integral_constant<int, 3>{}, c8);
        iteration(std::integral_constant<int, 4>{}, c8);
        iteration(std::integral_constant<int, 5>{}, c8);
        iteration(std::integral_constant<int, 6>{}, c8);
        iteration(std::integral_constant<int, 7>{}, c8);
    }

    // Add the two K halves through LDS and store: round 0, the kh = 1 wave
    // hands its rows i < FM/2 to its kh = 0 partner, which adds and stores
    // them; round 1 the other way round for rows i >= FM/2.
    float* red = reinterpret_cast<float*>(lds) + wn * (FM / 2) * 2 * 16 * 64 + lane;
    auto store = [&](int i, int j, const f32x16& v) {
        const int col = n0 + 32 * j + (lane & 31);
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int row = m0 + 32 * i + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
            D[(size_t)row * N + col] = v[e];
        }
    };
#pragma unroll
    for (int round = 0; round < 2; ++round) {
        const int giver = round == 0 ? 1 : 0;
        if (kh == giver) {
#pragma unroll
            for (int ii = 0; ii < FM / 2; ++ii)
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int e = 0; e < 16; ++e) red[((ii * 2 + j) * 16 + e) * 64] = acc[round * (FM / 2) + ii][j][e];
        }
        __syncthreads();
        if (kh != giver) {
#pragma unroll
            for (int ii = 0; ii < FM / 2; ++ii)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    f32x16 v = acc[round * (FM / 2) + ii][j];
#pragma unroll
                    for (int e = 0; e < 16; ++e) v[e] += red[((ii * 2 + j) * 16 + e) * 64];
                    store(round * (FM / 2) + ii, j, v);
                }
        }
        __syncthreads();
    }
}

// Workgroups are dispatched round-robin over the XCDs (b -> XCD b % 8).
// Returns the virtual index of workgroup b such that XCD x processes the
// contiguous virtual range [start_x, start_x + count_x): a bijection of
// [0, total).
constexpr int kXcds = 8;
__device__ __forceinline__ int xcd_remap(int b, int total) {
    const int x = b % kXcds, local = b / kXcds;
    const int per = total / kXcds, rem = total % kXcds;
    const int start = x < rem ? x * (per + 1) : rem * (per + 1) + (x - rem) * per;
    return start + local;
}

// ── v7: 4 waves (one per SIMD), full K chunk per wave, MFMA/VALU interleave
// Workgroup = 256 threads over a BM x 256 tile (BM = 32 FM); wave w owns
// output columns [n0 + 64 w, +64) for all BM rows and both K halves of every
// chunk, so no cross-wave reduction is needed and each wave has the whole
// register file of its SIMD (accumulators in AGPRs).  Weights stage through
// an LDS ring (below); B operands are double buffered so chunk c + 1 is
// dequantised while the MFMAs of chunk c run, with scheduling hints placing
// a few VALU operations after every MFMA (the matrix core executes an MFMA
// for many cycles while the SIMD issues the independent VALU work).
constexpr int kV7Threads = 256;

// Weight ring.  Per-lane weight loads (32 rows per instruction, 16 B each)
// saturate the vector L1 long before the MFMAs do.  Here the workgroup loads each
// super-block of its 256 weight rows with coalesced 16-byte loads (a wave
// instruction covers 1 KB of consecutive pieces of ~8 rows: whole cache
// lines), parks them in registers for two chunk iterations, writes them to
// a ring of kStages LDS stages, and each lane reads its operand bytes from
// LDS.  (Plain loads + ds_write rather than LDS DMA: a DMA mixed with the A
// loads leaves the compiler unable to count outstanding loads, and it then
// waits for all of them.)
//   Stage layout: row r of the tile at r * kRS.  Q4_K: the 144-byte block
//   (9 pieces).  Q6_K (blocks are only 2-byte aligned): the 16-byte aligned
//   window of 14 pieces starting at floor16(block), then one padding piece
//   (a second copy of piece 13) so that the row stride, 240 bytes, is
//   bank-conflict free; block byte b sits at r * 240 + shift + b with
//   shift = block offset mod 16 = 2 * (sb mod 8) (row starts are 16-byte
//   aligned because K % 2048 == 0).
//   Loads: every wave issues kNI 16-byte loads per super-block; instruction
//   g = wave * kNI + t moves stage pieces [64 g, 64 g + 64) (lane-linear).
//   The stage holds kGroups such groups; g >= kGroups repeats group
//   g - kGroups (the same bytes to the same place).
//   Schedule: the loads of super-block sb + kDepth are issued in the first
//   chunk iteration of sb and written to LDS in its third; the slot they
//   overwrite belonged to sb - 1, finished one barrier earlier.
//
// Weight ring of the 256-row tile: one super-block of every row per stage
// (Q4_K: 144-byte blocks; Q6_K: the 16-byte aligned 240-byte window around
// the 2-byte aligned block), two stages.  A stage is kGroups KB; each of
// the 4 waves moves kNI of them.
template <bool IS_Q6>
struct RingGeom7 {
    static constexpr int kRS = IS_Q6 ? 240 : 144, kNPR = IS_Q6 ? 15 : 9;
    static constexpr int kStages = 2;
    static constexpr int kGroups = 256 * kRS / 1024;
    static constexpr int kNI = kGroups / 4;
};

// Output routing of one v7 launch.  The N columns fall into up to three
// segments, each with its own weight rows and output matrix: [0, n1) -> (W,
// D), [n1, n2) -> (w1, d1), [n2, N) -> (w2, d2), every boundary a multiple
// of the 256-column tile (a single GEMM has n1 = n2 = N).  Each segment's
// output is row-major with its own width.  accum != 0 adds the product to
// the output's contents instead of storing it (the split-K path always
// adds).  pair != 0 (one segment, no K split): the N columns are N/2 gate
// rows (W) and N/2 up rows (w1) taken 128 at a time -- tile j covers gate
// rows [128j, +128) on waves 0-1 and the same up rows on waves 2-3 -- and
// D[M x N/2] = silu(gate) * up; pair == 2 stores that fp32 value rounded to
// fp16 (round to nearest even) into D read as an array of halves.
struct GemmSegs {
    const uint8_t* w1;
    const uint8_t* w2;
    float* d1;
    float* d2;
    int n1, n2;
    int accum;
    int pair;
};

template <typename T, bool IS_Q6, int FM>
__global__ __launch_bounds__(kV7Threads) void rf_gemm_qk_v7_kernel(const float* __restrict__ A,
                                                                    const uint8_t* __restrict__ W,
                                                                    float* __restrict__ D, int M, int N, int K,
                                                                    int tiles, int chunks_per_split, int mg_arg,
                                                                    GemmSegs segs) {
    using G = RingGeom7<IS_Q6>;
    constexpr int FN = 2;                               // 32-column blocks per wave
    constexpr int BM = 32 * FM;
    constexpr int BN = 128 * FN;
    constexpr int A_RPP = kV7Threads / 16;              // A rows per staging pass
    constexpr int A_F4 = BM * kKC / 4 / kV7Threads;     // float4 per thread per chunk
    constexpr int kStageBytes = BN * G::kRS;
    constexpr int kDepth = G::kStages - 1;
    constexpr int NS = 4 * FM * FN;                     // MFMA slots per iteration
    static_assert(G::kGroups * 1024 == kStageBytes && 4 * G::kNI == G::kGroups, "load groups cover the stage");
    static_assert(A_F4 <= 8, "A register double buffer");
    __shared__ __align__(16) uint8_t w_ring[G::kStages * kStageBytes];
    // A_PF (where LDS allows): four A buffers, chunk c + 2 stored during
    // iteration c, so the first A fragments of chunk c + 1 are read before
    // the end of iteration c (no LDS latency exposed after the per-chunk
    // barrier).  Otherwise two buffers, chunk c + 1 stored in iteration c.
    constexpr bool A_PF = G::kStages * kStageBytes + 4 * BM * kLdsStride * 2 <= 160 * 1024;
    __shared__ __align__(16) _Float16 lds_a[A_PF ? 4 : 2][BM * kLdsStride];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5;
    // XCD-aware order: workgroup b runs on XCD b % 8; give each XCD one
    // contiguous run of the (M-major) tile order so the workgroups sharing an
    // M tile -- the same rows of A -- share that XCD's L2.
    const int vidx = xcd_remap((int)blockIdx.x, (int)gridDim.x);
    const int splits = (int)gridDim.x / tiles;
    const int tile = vidx / splits;
    const int split = vidx % splits;
    const int ntiles = N / BN;
    // tiles ordered in bands of MG row blocks (column-major inside a band),
    // so an XCD's contiguous run covers MG row blocks x (run / MG) column
    // blocks: each weight column block is streamed by M/(BM MG) XCDs
    // instead of M/BM (the A rows an XCD touches grow by MG)
    const int mtiles = M / BM;
    const int MG = (mg_arg > 1 && mtiles % mg_arg == 0) ? mg_arg : 1;
    const int band = tile / (MG * ntiles), rb = tile % (MG * ntiles);
    const int m0 = (band * MG + rb % MG) * BM;
    const int nt0 = (rb / MG) * BN;
    const int n0 = nt0 + wave * 32 * FN;
    const int c_begin = split * chunks_per_split;
    const int c_last = c_begin + chunks_per_split - 1;
    const int sb_begin = c_begin / 4, sb_last = c_last / 4;
    const size_t row_bytes = (size_t)(K / kQK) * T::kBytes;
    // the column segment of this tile (selects, not an indexed argument array)
    const int sgi = nt0 >= segs.n2 ? 2 : (nt0 >= segs.n1 ? 1 : 0);
    const int nbase = sgi == 2 ? segs.n2 : (sgi == 1 ? segs.n1 : 0);
    const int ldd = (sgi == 2 ? N : (sgi == 1 ? segs.n2 : segs.n1)) - nbase;
    const uint8_t* wseg = sgi == 2 ? segs.w2 : (sgi == 1 ? segs.w1 : W);
    float* dseg = sgi == 2 ? segs.d2 : (sgi == 1 ? segs.d1 : D);
    // pair mode: waves 0-1 stream gate rows, waves 2-3 the same up rows
    const bool up_wave = segs.pair && wave >= 2;
    const uint8_t* wtile = segs.pair ? (up_wave ? segs.w1 : W) + (size_t)(nt0 / 2) * row_bytes
                                     : wseg + (size_t)(nt0 - nbase) * row_bytes;

    uint32_t goff[G::kNI];
    uint32_t gdst[G::kNI];
#pragma unroll
    for (int t = 0; t < G::kNI; ++t) {
        const int g = wave * G::kNI + t;
        const int pc = 64 * g + lane;
        gdst[t] = 16u * (uint32_t)pc;
        // a wave's load groups lie in ring rows [128 (w >> 1), +128): up waves
        // address their rows from the up matrix's tile base
        const int row = pc / G::kNPR - (up_wave ? 128 : 0);
        int piece = pc % G::kNPR;
        if (IS_Q6 && piece == 14) piece = 13;
        goff[t] = (uint32_t)((size_t)row * row_bytes) + 16u * (uint32_t)piece;
    }
    u32x4 wst[G::kNI];
    const __amdgpu_buffer_rsrc_t w_rsrc = make_rsrc(wtile);
    auto w_soff = [&](int sb) -> uint32_t {
        sb = min(sb, sb_last);
        return IS_Q6 ? (((uint32_t)sb * kQ6KBytes) & ~15u) : (uint32_t)sb * kQ4KBytes;
    };
    auto w_gload = [&](int sb) {
        const uint32_t so = w_soff(sb);
#pragma unroll
        for (int t = 0; t < G::kNI; ++t) wst[t] = __builtin_amdgcn_raw_buffer_load_b128(w_rsrc, goff[t], so, 0);
    };
    auto w_lstore = [&](int slot) {
        uint8_t* dst = w_ring + slot * kStageBytes;
#pragma unroll
        for (int t = 0; t < G::kNI; ++t) *reinterpret_cast<u32x4*>(dst + gdst[t]) = wst[t];
    };

    const int a_row = tid >> 4;
    const int a_col = 4 * (tid & 15);
    // A float4 i of chunk c: buffer load with the workgroup-uniform part of
    // the offset in a scalar register and the lane's part in a vector one,
    // so the load costs no per-lane address arithmetic
    const __amdgpu_buffer_rsrc_t a_rsrc = make_rsrc(A + (size_t)m0 * K);
    const uint32_t a_voff = (uint32_t)(a_row * K + a_col) * 4u;
    auto a_ld = [&](int c, int i) -> float4 {
        const uint32_t so = (uint32_t)(A_RPP * i * K + min(c, c_last) * kKC) * 4u;
        return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(a_rsrc, a_voff, so, 0));
    };
    float4 a_reg[2][A_F4];
    auto a_load = [&](float4 (&r)[A_F4], int c) {
#pragma unroll
        for (int i = 0; i < A_F4; ++i) r[i] = a_ld(c, i);
    };
    auto a_store = [&](const float4 (&r)[A_F4], int buf) {
        _Float16* dst = &lds_a[buf][a_row * kLdsStride + a_col];
#pragma unroll
        for (int i = 0; i < A_F4; ++i) {
            f16x4 hv;
            hv[0] = (_Float16)r[i].x; hv[1] = (_Float16)r[i].y;
            hv[2] = (_Float16)r[i].z; hv[3] = (_Float16)r[i].w;
            *reinterpret_cast<f16x4*>(dst + A_RPP * i * kLdsStride) = hv;
        }
    };

    f32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    const int frag = (lane & 31) * kLdsStride + 16 * h;
    const int row_lds0 = (wave * 32 * FN + (lane & 31)) * G::kRS;

    // bq[buffer][k half][column block][k16 step]
    f16x8 bq[2][2][FN][2];
    // Raw operand bytes of chunk c + 1 for the lane's two weight rows, read
    // from the ring at the start of iteration c, and the per-(row, k half)
    // scale terms: Q4_K value = a * byte - b (a = d*sc, or d*sc/16 for the
    // high-nibble half read as 16*nibble; b = dmin*m); Q6_K value = a * q - b
    // (a = d*sc, b = 32a).
    u32x4 wq[FN][2];     // Q4: [row][0] = header, [1] = qs bytes; Q6: [row][0] = ql (kh 0), [1] = ql (kh 1)
    u32x4 wqh[FN];       // Q6: qh bytes per row
    uint32_t wsc[FN];    // Q6: scale word per row
    uint32_t wd[FN];     // Q6: d per row
    float pa[FN][2], pb[FN][2];
    auto w_read = [&](auto jj, int sb, int slot) {
        constexpr int CQ = decltype(jj)::value & 3;
        const uint8_t* st = w_ring + slot * kStageBytes;
#pragma unroll
        for (int r = 0; r < FN; ++r) {
            if constexpr (IS_Q6) {
                constexpr int nh = CQ >> 1;
                const uint8_t* rb = st + row_lds0 + 32 * r * G::kRS + 2 * (sb & 7);
                wq[r][0] = ld16(rb + 64 * nh + 16 * h);
                wq[r][1] = ld16(rb + 64 * nh + 32 + 16 * h);
                wqh[r] = ld16(rb + 128 + 32 * nh + 16 * h);
                wsc[r] = ld4(rb + 192 + 4 * CQ);
                wd[r] = ld_u16(rb + 208);
            } else {
                const uint8_t* rb = st + row_lds0 + 32 * r * G::kRS;
                wq[r][0] = *reinterpret_cast<const u32x4*>(rb);
                wq[r][1] = *reinterpret_cast<const u32x4*>(rb + 16 + 32 * CQ + 16 * h);
            }
        }
    };
    auto w_prep = [&](auto jj, int r) {
        constexpr int CQ = decltype(jj)::value & 3;
        if constexpr (IS_Q6) {
            const float d = half_bits_to_float(wd[r]);
#pragma unroll
            for (int kh = 0; kh < 2; ++kh) {
                pa[r][kh] = d * (float)(int8_t)((wsc[r] >> (8 * (2 * kh + h))) & 0xFFu);
                pb[r][kh] = 32.0f * pa[r][kh];
            }
        } else {
            int sc0, m0, sc1, m1;
            q4k_scale_min_pair(wq[r][0].y, wq[r][0].z, wq[r][0].w, CQ, &sc0, &m0, &sc1, &m1);
            const float d = half_bits_to_float(wq[r][0].x), dmin = half_bits_to_float(wq[r][0].x >> 16);
            pa[r][0] = d * (float)sc0;
            pb[r][0] = dmin * (float)m0;
            pa[r][1] = d * (float)sc1 * 0.0625f;
            pb[r][1] = dmin * (float)m1;
        }
    };
    // piece (r, kh, word j) of the dequantisation into bq[buf]: 4 weights
    auto w_piece = [&](auto jj, int buf, int r, int kh, int j) {
        constexpr int CQ = decltype(jj)::value & 3;
        uint32_t q;
        if constexpr (IS_Q6) {
            constexpr uint32_t nsh = 4u * (CQ & 1);
            const uint32_t qsh = 4u * (CQ & 1) + 2u * (uint32_t)kh;
            q = ((wq[r][kh][j] >> nsh) & 0x0F0F0F0Fu) | (((wqh[r][j] >> qsh) & 0x03030303u) << 4);
        } else {
            q = wq[r][1][j] & (kh ? 0xF0F0F0F0u : 0x0F0F0F0Fu);
        }
        // opaque to the optimiser: otherwise it folds the mask into per-byte
        // bit-field extracts and converts byte 0, two instructions per weight
        // instead of one v_cvt_f32_ubyteN
        asm("" : "+v"(q));
        const float a = pa[r][kh], b = pb[r][kh];
        if constexpr (IS_Q6)
            put4(bq[buf][kh][r][j >> 1], j & 1, a * byte_f(q, 0) - b, a * byte_f(q, 1) - b, a * byte_f(q, 2) - b,
                 a * byte_f(q, 3) - b);
        else
            put4_rn(bq[buf][kh][r][j >> 1], j & 1, a * byte_f(q, 0) - b, a * byte_f(q, 1) - b, a * byte_f(q, 2) - b,
                    a * byte_f(q, 3) - b);
    };
    auto w_dequant_all = [&](auto jj, int buf) {
#pragma unroll
        for (int r = 0; r < FN; ++r) {
            w_prep(jj, r);
#pragma unroll
            for (int kh = 0; kh < 2; ++kh)
#pragma unroll
                for (int j = 0; j < 4; ++j) w_piece(jj, buf, r, kh, j);
        }
    };
    auto a_store1 = [&](const float4& v, int buf, int i) {
        f16x4 hv;
        hv[0] = (_Float16)v.x; hv[1] = (_Float16)v.y;
        hv[2] = (_Float16)v.z; hv[3] = (_Float16)v.w;
        *reinterpret_cast<f16x4*>(&lds_a[buf][a_row * kLdsStride + a_col] + A_RPP * i * kLdsStride) = hv;
    };

    // Iteration I of the 8-chunk group at c8.  Hand-scheduled in 16 slots
    // separated by scheduling fences: slot t = 4*step + i issues the MFMA
    // pair (acc[i][0], acc[i][1]) of k16 step `step` (independent of the
    // previous pair) and one slice of the side work -- a piece of the next
    // chunk's dequantisation, one A float4 to LDS, one global load, one ring
    // store -- so the VALU work runs while the matrix core executes.
    f16x8 af[2][FM];
    auto iteration = [&](auto it, int c8, int slot0, int slot1, int slot2, int sd0, int sd1) {
        constexpr int I = decltype(it)::value;
        constexpr int P = I & 1, CQ = I & 3;
        constexpr int IN = (I + 1) & 7;            // in-group index of chunk c + 1
        using JN = std::integral_constant<int, IN>;
        const int c = c8 + I;
        const int sb = c8 / 4 + (I >> 2);
        const int sbn = I == 7 ? sb + 1 : c8 / 4 + ((I + 1) >> 2);
        const int slotn = I == 7 ? slot2 : (((I + 1) >> 2) ? slot1 : slot0);
        const _Float16* la = lds_a[A_PF ? (I & 3) : P] + frag;
        // with A_PF the first MFMAs need no fresh LDS data, so the
        // dequantisation starts two slots later, behind the ring reads
        constexpr int DQ0 = A_PF ? 2 : 0;
        __builtin_amdgcn_sched_barrier(0);
        w_read(JN{}, sbn, slotn);
        if constexpr (!A_PF) {
#pragma unroll
            for (int i = 0; i < FM; ++i) af[0][i] = *reinterpret_cast<const f16x8*>(la + 32 * i * kLdsStride);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int step = 0; step < 4; ++step) {
            const int kh = step >> 1, s2 = step & 1;
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    // slot t: one MFMA, then ~7 VALU operations of side work
                    // (the MFMA occupies the matrix core for 32 cycles, the
                    // time the SIMD needs to issue about 8 VALU operations)
                    const int t = (step * FM + i) * FN + j;   // 0 .. NS-1
                    if (i == 0 && j == 0 && step < 3) {
                        const int nk = (step + 1) >> 1, ns = (step + 1) & 1;
#pragma unroll
                        for (int ii = 0; ii < FM; ++ii)
                            af[(step + 1) & 1][ii] =
                                *reinterpret_cast<const f16x8*>(la + 32 * ii * kLdsStride + 32 * nk + 8 * ns);
                    }
                    if constexpr (A_PF) {
                        // first fragments of chunk c + 1 (stored during
                        // iteration c - 1, behind the last barrier)
                        if (i == 0 && j == 0 && step == 3) {
                            const _Float16* ln = lds_a[(I + 1) & 3] + frag;
#pragma unroll
                            for (int ii = 0; ii < FM; ++ii)
                                af[0][ii] = *reinterpret_cast<const f16x8*>(ln + 32 * ii * kLdsStride);
                        }
                    }
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[step & 1][i], bq[P][kh][j][s2], acc[i][j],
                                                                       0, 0, 0);
                    // dequantisation of chunk c + 1: prep row r at slot
                    // DQ0 + 9r, its 8 pieces at the next 8 slots (packed
                    // into 16 slots when NS = 16)
                    if constexpr (NS >= 9 * FN + DQ0) {
#pragma unroll
                        for (int r = 0; r < FN; ++r) {
                            if (t == DQ0 + 9 * r) w_prep(JN{}, r);
                            if (t >= DQ0 + 9 * r + 1 && t <= DQ0 + 9 * r + 8)
                                w_piece(JN{}, P ^ 1, r, (t - DQ0 - 9 * r - 1) >> 2, (t - DQ0 - 9 * r - 1) & 3);
                        }
                    } else {
                        static_assert(NS == 16, "packed dequantisation schedule");
                        if (t == 0) {
                            w_prep(JN{}, 0);
                            w_prep(JN{}, 1);
                        }
                        if (t < 16) w_piece(JN{}, P ^ 1, t >> 3, (t >> 2) & 1, t & 3);
                    }
                    {
                        // A: store float4 k of chunk c + 1 (A_PF: c + 2) at
                        // slot NS-14+k, reload the register with chunk c + 3
                        // (A_PF: c + 4) six slots later
                        constexpr int RB = A_PF ? P : P ^ 1;
                        constexpr int LB = A_PF ? ((I + 2) & 3) : (P ^ 1);
                        if (t >= NS - 14 && t < NS - 14 + A_F4)
                            a_store1(a_reg[RB][t - (NS - 14)], LB, t - (NS - 14));
                        if (t >= NS - 8 && t < NS - 8 + A_F4) {
                            const int k = t - (NS - 8);
                            a_reg[RB][k] = a_ld(c + (A_PF ? 4 : 3), k);
                        }
                    }
                    if constexpr (CQ == 0) {
                        if (t < G::kNI)
                            wst[t] = __builtin_amdgcn_raw_buffer_load_b128(w_rsrc, goff[t], w_soff(sb + kDepth), 0);
                    }
                    if constexpr (CQ == 2) {
                        if (t < G::kNI) {
                            uint8_t* dst = w_ring + ((I >> 2) ? sd1 : sd0) * kStageBytes;
                            *reinterpret_cast<u32x4*>(dst + gdst[t]) = wst[t];
                        }
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
        }
        static_assert(NS >= 16 && NS >= G::kNI && NS >= 14, "side work fits the slots");
        lds_barrier();
    };

#pragma unroll
    for (int d = 0; d < kDepth; ++d) {
        w_gload(sb_begin + d);
        w_lstore(d);
    }
    if constexpr (A_PF) {
        a_load(a_reg[0], c_begin);
        a_load(a_reg[1], c_begin + 1);
        a_store(a_reg[0], 0);
        a_store(a_reg[1], 1);
        a_load(a_reg[0], c_begin + 2);
        a_load(a_reg[1], c_begin + 3);
    } else {
        a_load(a_reg[0], c_begin);
        a_load(a_reg[1], c_begin + 1);
        a_store(a_reg[0], 0);
        a_load(a_reg[0], c_begin + 2);
    }
    lds_barrier();
    w_read(std::integral_constant<int, 0>{}, sb_begin, 0);
    w_dequant_all(std::integral_constant<int, 0>{}, 0);
    if constexpr (A_PF) {
#pragma unroll
        for (int i = 0; i < FM; ++i) af[0][i] = *reinterpret_cast<const f16x8*>(lds_a[0] + frag + 32 * i * kLdsStride);
    }

    int slot0 = 0;
    for (int c8 = c_begin; c8 <= c_last; c8 += 8) {
        const int slot1 = slot0 + 1 == G::kStages ? 0 : slot0 + 1;
        const int sd0 = slot0 + kDepth >= G::kStages ? slot0 + kDepth - G::kStages : slot0 + kDepth;
        const int sd1 = sd0 + 1 == G::kStages ? 0 : sd0 + 1;
        const int slot2 = slot1 + 1 == G::kStages ? 0 : slot1 + 1;
        iteration(std::integral_constant<int, 0>{}, c8, slot0, slot1, slot2, sd0, sd1);
        iteration(std::integral_constant<int, 1>{}, c8, slot0, slot1, slot2, sd0, sd1);
        iteration(std::integral_constant<int, 2>{}, c8, slot0, slot1, slot2, sd0, sd1);
        iteration(std::integral_constant<int, 3>{}, c8, slot0, slot1, slot2, sd0, sd1);
        iteration(std::integral_constant<int, 4>{}, c8, slot0, slot1, slot2, sd0, sd1);
        iteration(std::integral_constant<int, 5>{}, c8, slot0, slot1, slot2, sd0, sd1);
        iteration(std::integral_constant<int, 6>{}, c8, slot0, slot1, slot2, sd0, sd1);
        iteration(std::integral_constant<int, 7>{}, c8, slot0, slot1, slot2, sd0, sd1);
        slot0 = slot2;
    }

    if (segs.pair) {
        // up waves hand their accumulators to the gate waves through the
        // (now idle) weight ring, lane-fastest so each access is one
        // contiguous 256-byte run
        constexpr int NE = FM * FN * 16;
        static_assert(2 * NE * 64 * 4 <= G::kStages * kStageBytes, "exchange fits the ring");
        float* xch = reinterpret_cast<float*>(w_ring);
        __syncthreads();
        if (wave >= 2) {
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int e = 0; e < 16; ++e)
                        xch[((wave - 2) * NE + (i * FN + j) * 16 + e) * 64 + lane] = acc[i][j][e];
        }
        __syncthreads();
        if (wave < 2) {
            const int ldo = N / 2;
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    const int col = nt0 / 2 + 64 * wave + 32 * j + (lane & 31);
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        const int row = m0 + 32 * i + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                        const float g = acc[i][j][e];
                        const float u = xch[(wave * NE + (i * FN + j) * 16 + e) * 64 + lane];
                        const float v = g / (1.0f + expf(-g)) * u;
                        if (segs.pair == 2)
                            reinterpret_cast<uint16_t*>(D)[(size_t)row * ldo + col] = f16_bits_rn(v);
                        else
                            D[(size_t)row * ldo + col] = v;
                    }
                }
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int col = n0 - nbase + 32 * j + (lane & 31);
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = m0 + 32 * i + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                float* o = dseg + (size_t)row * ldd + col;
                *o = segs.accum ? *o + acc[i][j][e] : acc[i][j][e];
            }
        }
}

// ── sq: BM x BN tiles, 2 x 2 waves, dequantised B shared through LDS ─────
// Workgroup = 256 threads over a BM x BN tile (BM, BN in {128, 256}); wave
// (wm, wn) owns [m0 + (BM/2) wm, +BM/2) x [n0 + (BN/2) wn, +BN/2) as
// FMW x FNW blocks of v_mfma_f32_32x32x16_f16 (FMW = BM/64, FNW = BN/64;
// accumulators in AGPRs).  Per 64-wide K chunk both operands sit in LDS as
// [row][k] fp16 with the padded stride: A (fp32 -> fp16) and B, which the
// workgroup dequantises once (256/BN threads per weight row) -- one
// dequantisation per weight per BM rows of A, shared by the two waves that
// use it.  The next chunk's A store, B dequantisation and global loads run
// in hand-scheduled slots between the MFMAs of the current chunk (both LDS
// operands double buffered, one barrier per chunk, placed before the last
// k16 step so the next chunk's first fragments load behind it).  Launched
// only where its tiles need no K split.
constexpr int kSqThreads = 256;

// Raw quant bytes of one chunk of one weight row (thread-private); with two
// threads per row, thread half kh covers k [32 kh, 32 kh + 32) of the chunk.
template <bool IS_Q6, int TPR>
struct SqRaw;
template <int TPR>
struct SqRaw<false, TPR> {
    u32x4 hdr;              // d, dmin, scales[12]
    u32x4 q[2];             // qs [32CQ, 32CQ + 32) (both nibble halves)
};
template <int TPR>
struct SqRaw<true, TPR> {
    u32x4 ql[4 / TPR];      // ql [64nh, 64nh + 64), or its half [64nh + 32kh, +32)
    u32x4 qh[2];            // qh [32nh, 32nh + 32)
    uint32_t sc;            // scales [4CQ, 4CQ + 4)
    uint32_t d;             // fp16 bits of d
};

template <bool IS_Q6, int BM, int BN>
__global__ __launch_bounds__(kSqThreads) void rf_gemm_qk_sq_kernel(const float* __restrict__ A,
                                                                    const uint8_t* __restrict__ W,
                                                                    float* __restrict__ D, int M, int N, int K,
                                                                    int accum) {
    constexpr int FMW = BM / 64, FNW = BN / 64;          // MFMA blocks per wave along M, N
    constexpr int TPR = kSqThreads / BN;                 // threads per weight row
    constexpr int NP = 16 / TPR;                         // 4-weight pieces per thread per chunk
    constexpr int SPS = FMW * FNW;                       // MFMA slots per k16 step
    constexpr int NS = 4 * SPS;                          // slots per chunk
    constexpr int BAR = 3 * SPS;                         // barrier slot (start of step 3)
    constexpr int A_RPP = kSqThreads / 16;               // A rows per staging pass
    constexpr int A_F4 = BM * kKC / 4 / kSqThreads;      // float4 per thread per chunk
    constexpr int A0 = NS >= 64 ? 28 : 1;                // first A store slot
    constexpr int WLD = NS >= 64 ? 20 : 2 + NP;          // slot of the next-but-one chunk's weight loads
    static_assert(A0 + A_F4 <= BAR && 2 + NP <= BAR && WLD < BAR, "side work before the barrier");
    using Raw = SqRaw<IS_Q6, TPR>;
    constexpr int kBytes = IS_Q6 ? kQ6KBytes : kQ4KBytes;
    __shared__ __align__(16) _Float16 lds_a[2][BM * kLdsStride];
    __shared__ __align__(16) _Float16 lds_b[2][BN * kLdsStride];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int h = lane >> 5;
    const int tile = xcd_remap((int)blockIdx.x, (int)gridDim.x);
    const int ntiles = N / BN;
    const int m0 = (tile / ntiles) * BM;
    const int n0 = (tile % ntiles) * BN;
    const int c_last = K / kKC - 1;
    const uint32_t row_bytes = (uint32_t)(K / kQK) * kBytes;

    // ---- A: A_F4 float4 per thread per chunk, buffer loads ---------------
    const int a_row = tid >> 4;
    const int a_col = 4 * (tid & 15);
    const __amdgpu_buffer_rsrc_t a_rsrc = make_rsrc(A + (size_t)m0 * K);
    const uint32_t a_voff = (uint32_t)(a_row * K + a_col) * 4u;
    auto a_ld = [&](int c, int i) -> float4 {
        const uint32_t so = (uint32_t)(A_RPP * i * K + min(c, c_last) * kKC) * 4u;
        return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(a_rsrc, a_voff, so, 0));
    };
    auto a_st = [&](const float4& v, int buf, int i) {
        f16x4 hv;
        hv[0] = (_Float16)v.x; hv[1] = (_Float16)v.y;
        hv[2] = (_Float16)v.z; hv[3] = (_Float16)v.w;
        *reinterpret_cast<f16x4*>(&lds_a[buf][(a_row + A_RPP * i) * kLdsStride + a_col]) = hv;
    };
    float4 a_reg[A_F4];

    // ---- W: thread tid dequantises k half wkh of weight row n0 + wrow ----
    const int wrow = tid / TPR;
    const int wkh = TPR == 2 ? (tid & 1) : 0;
    const __amdgpu_buffer_rsrc_t w_rsrc = make_rsrc(W + (size_t)n0 * row_bytes);
    const uint32_t w_voff = (uint32_t)wrow * row_bytes;
    Raw wr[2];
    auto w_ld = [&](auto cq, Raw& r, int c) {
        constexpr int CQ = decltype(cq)::value;
        const uint32_t blk = (uint32_t)(min(c, c_last) >> 2) * kBytes;
        if constexpr (IS_Q6) {
            constexpr int nh = CQ >> 1;
            const uint32_t qlo = blk + 64 * nh + (TPR == 2 ? 32u * (uint32_t)wkh : 0u);
#pragma unroll
            for (int i = 0; i < 4 / TPR; ++i)
                r.ql[i] = __builtin_amdgcn_raw_buffer_load_b128(w_rsrc, w_voff, qlo + 16 * i, 0);
#pragma unroll
            for (int i = 0; i < 2; ++i)
                r.qh[i] = __builtin_amdgcn_raw_buffer_load_b128(w_rsrc, w_voff, blk + 128 + 32 * nh + 16 * i, 0);
            r.sc = __builtin_amdgcn_raw_buffer_load_b32(w_rsrc, w_voff, blk + 192 + 4 * CQ, 0);
            r.d = __builtin_amdgcn_raw_buffer_load_b16(w_rsrc, w_voff, blk + 208, 0);
        } else {
            r.hdr = __builtin_amdgcn_raw_buffer_load_b128(w_rsrc, w_voff, blk, 0);
            r.q[0] = __builtin_amdgcn_raw_buffer_load_b128(w_rsrc, w_voff, blk + 16 + 32 * CQ, 0);
            r.q[1] = __builtin_amdgcn_raw_buffer_load_b128(w_rsrc, w_voff, blk + 32 + 32 * CQ, 0);
        }
    };
    // Scale terms: Q4_K value = pa[kh] * byte - pb[kh] (kh 0: low nibbles,
    // k 0..31; kh 1: high nibbles read as 16 * nibble, k 32..63); Q6_K
    // value = ps[g] * q - 32 ps[g] for the 16-wide group g = k / 16.
    float pa[2], pb[2], ps[4];
    auto w_prep = [&](auto cq, const Raw& r) {
        constexpr int CQ = decltype(cq)::value;
        if constexpr (IS_Q6) {
            const float d = half_bits_to_float(r.d);
#pragma unroll
            for (int g = 0; g < 4; ++g) ps[g] = d * (float)(int8_t)((r.sc >> (8 * g)) & 0xFFu);
        } else {
            int sc0, mn0, sc1, mn1;
            q4k_scale_min_pair(r.hdr.y, r.hdr.z, r.hdr.w, CQ, &sc0, &mn0, &sc1, &mn1);
            const float d = half_bits_to_float(r.hdr.x), dmin = half_bits_to_float(r.hdr.x >> 16);
            pa[0] = d * (float)sc0;
            pb[0] = dmin * (float)mn0;
            pa[1] = d * (float)sc1 * 0.0625f;
            pb[1] = dmin * (float)mn1;
        }
    };
    // piece p (0..NP-1) = 4 weights k = 32 kh + 4 j .. + 3 (kh = p >> 3, or
    // the thread's half with two threads per row; j = p & 7); the pair
    // (p - 1, p) for odd p completes 8 weights, stored to LDS
    f16x8 wout;
    auto w_piece = [&](auto cq, const Raw& r, int buf, int p) {
        constexpr int CQ = decltype(cq)::value;
        const int kh = TPR == 2 ? wkh : (p >> 3);
        const int j = p & 7;
        uint32_t q;
        float a, b;
        if constexpr (IS_Q6) {
            constexpr uint32_t t4 = 4u * (CQ & 1);
            const int li = TPR == 2 ? j : 8 * kh + j;
            q = ((r.ql[li >> 2][li & 3] >> t4) & 0x0F0F0F0Fu) |
                (((r.qh[j >> 2][j & 3] >> (t4 + 2u * (uint32_t)kh)) & 0x03030303u) << 4);
            const int g = 2 * kh + (j >> 2);
            a = g == 0 ? ps[0] : (g == 1 ? ps[1] : (g == 2 ? ps[2] : ps[3]));
            b = 32.0f * a;
        } else {
            q = r.q[j >> 2][j & 3] & (kh ? 0xF0F0F0F0u : 0x0F0F0F0Fu);
            a = kh ? pa[1] : pa[0];
            b = kh ? pb[1] : pb[0];
        }
        // opaque to the optimiser: otherwise it folds the mask into per-byte
        // bit-field extracts instead of one v_cvt_f32_ubyteN per weight
        asm("" : "+v"(q));
        if constexpr (IS_Q6)
            put4(wout, j & 1, a * byte_f(q, 0) - b, a * byte_f(q, 1) - b, a * byte_f(q, 2) - b, a * byte_f(q, 3) - b);
        else
            put4_rn(wout, j & 1, a * byte_f(q, 0) - b, a * byte_f(q, 1) - b, a * byte_f(q, 2) - b,
                    a * byte_f(q, 3) - b);
        if (p & 1)
            *reinterpret_cast<f16x8*>(&lds_b[buf][wrow * kLdsStride + 32 * kh + 8 * (j >> 1)]) = wout;
    };

    f32x16 acc[FMW][FNW];
#pragma unroll
    for (int i = 0; i < FMW; ++i)
#pragma unroll
        for (int j = 0; j < FNW; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    const int fa = ((BM / 2) * wm + (lane & 31)) * kLdsStride + 8 * h;
    const int fb = ((BN / 2) * wn + (lane & 31)) * kLdsStride + 8 * h;
    f16x8 af[2][FMW], bf[2][FNW];
    auto frag_ld = [&](int buf, int step, int slot) {
#pragma unroll
        for (int i = 0; i < FMW; ++i)
            af[slot][i] = *reinterpret_cast<const f16x8*>(&lds_a[buf][fa + 32 * i * kLdsStride + 16 * step]);
#pragma unroll
        for (int j = 0; j < FNW; ++j)
            bf[slot][j] = *reinterpret_cast<const f16x8*>(&lds_b[buf][fb + 32 * j * kLdsStride + 16 * step]);
    };

    // Iteration I of the 8-chunk group at c8: NS slots separated by
    // scheduling fences, slot t = SPS step + FNW i + j issuing MFMA (i, j)
    // of k16 step `step` plus one slice of side work for chunk c + 1 (B
    // dequantisation into LDS, A store) or c + 2 (weight loads).  The one
    // barrier per chunk sits before step 3: by then every wave has written
    // its share of chunk c + 1 and issued its last read of chunk c's
    // buffers (step 3's fragments are read during step 2), so step 0 of
    // chunk c + 1 is read during step 3 and the next iteration starts with
    // its operands in registers.
    auto iteration = [&](auto it, int c8) {
        constexpr int I = decltype(it)::value;
        constexpr int P = I & 1;
        using CQN = std::integral_constant<int, (I + 1) & 3>;
        using CQ2 = std::integral_constant<int, (I + 2) & 3>;
        const int c = c8 + I;
#pragma unroll
        for (int step = 0; step < 4; ++step)
#pragma unroll
            for (int i = 0; i < FMW; ++i)
#pragma unroll
                for (int j = 0; j < FNW; ++j) {
                    const int t = SPS * step + FNW * i + j;
                    if (t == BAR) lds_barrier();
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[step & 1][i], bf[step & 1][j], acc[i][j],
                                                                       0, 0, 0);
                    if (t % SPS == 0 && step < 3) frag_ld(P, step + 1, (step + 1) & 1);
                    if (t == BAR) frag_ld(P ^ 1, 0, 0);
                    if (t == 1) w_prep(CQN{}, wr[P ^ 1]);
                    if (t >= 2 && t < 2 + NP) w_piece(CQN{}, wr[P ^ 1], P ^ 1, t - 2);
                    if (t == WLD) w_ld(CQ2{}, wr[P], c + 2);
                    if (t >= A0 && t < A0 + A_F4) {
                        a_st(a_reg[t - A0], P ^ 1, t - A0);
                        a_reg[t - A0] = a_ld(c + 2, t - A0);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
    };

    w_ld(std::integral_constant<int, 0>{}, wr[0], 0);
    w_ld(std::integral_constant<int, 1>{}, wr[1], 1);
#pragma unroll
    for (int i = 0; i < A_F4; ++i) a_reg[i] = a_ld(0, i);
#pragma unroll
    for (int i = 0; i < A_F4; ++i) {
        a_st(a_reg[i], 0, i);
        a_reg[i] = a_ld(1, i);
    }
    w_prep(std::integral_constant<int, 0>{}, wr[0]);
#pragma unroll
    for (int p = 0; p < NP; ++p) w_piece(std::integral_constant<int, 0>{}, wr[0], 0, p);
    lds_barrier();
    frag_ld(0, 0, 0);

    for (int c8 = 0; c8 <= c_last; c8 += 8) {
        iteration(std::integral_constant<int, 0>{}, c8);
        iteration(std::integral_constant<int, 1>{}, c8);
        iteration(std::integral_constant<int, 2>{}, c8);
        iteration(std::integral_constant<int, 3>{}, c8);
        iteration(std::integral_constant<int, 4>{}, c8);
        iteration(std::integral_constant<int, 5>{}, c8);
        iteration(std::integral_constant<int, 6>{}, c8);
        iteration(std::integral_constant<int, 7>{}, c8);
    }

#pragma unroll
    for (int i = 0; i < FMW; ++i)
#pragma unroll
        for (int j = 0; j < FNW; ++j) {
            const int col = n0 + (BN / 2) * wn + 32 * j + (lane & 31);
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = m0 + (BM / 2) * wm + 32 * i + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                float* o = D + (size_t)row * N + col;
                *o = accum ? *o + acc[i][j][e] : acc[i][j][e];
            }
        }
}

// ── f16a: Q4_K GEMM on fp16 activations, 256 x 128 tiles, K halves on wave
// pairs (rf_gemm_q4_k_f16_launch) ─────────────────────────────────────────
// Workgroup = 256 threads over a 256 (M) x 128 (N) tile.  Wave w owns the
// 64 output columns [n0 + 64 (w >> 1), +64) for all 256 rows, over the K
// half kh = w & 1 of every 64-wide chunk; the two halves are added through
// LDS at the end.  Each wave issues 32 MFMAs per chunk against 16
// dequantised weights per lane, so every weight is dequantised once per 256
// rows of A (the fp32-activation kernels: once per 128) and the
// accumulators fill the 256 AGPRs.
//
// Memory.  A (fp16, as the caller rounded it) and the weight ring arrive by
// LDS DMA (global_load_lds_dwordx4: no registers, no LDS store
// instructions), three A chunk buffers and two ring stages.  The DMAs are
// inline asm the compiler does not see, so the kernel waits for them itself
// (s_waitcnt vmcnt before the per-chunk barrier).  A's 128-byte rows are
// XOR-swizzled by 16-byte piece: position p of row r holds k piece
// p ^ g(r), g(r) = (r & 7) ^ ((r >> 3) & 1), so 16 consecutive rows of a
// fragment read fall on 16 different bank groups.
//
// K order.  Chunk c of a Q4_K row = super-block c / 4, nibble pair p = c % 4:
// qs byte i of [32p, 32p + 32) holds chunk elements i (low nibble) and
// 32 + i (high nibble).  Wave half kh, lane half h take the bytes
// [16 kh + 8 h, +8): k16 step 0 is their 8 low nibbles (k = 16 kh + 8 h + j),
// step 1 their 8 high nibbles (k = 32 + 16 kh + 8 h + j).
//
// Dequantisation.  A 16-bit half 0x000q is the fp16 subnormal q * 2^-24 and
// 0x00q0 is q * 2^-20, both exact; v_fma_mix takes such a half as its fp16
// source, so the fp32 value D q - M = fma(half, D * 2^24, -M) (or D * 2^20
// for the high nibbles; D q is exact): per word of 4 bytes one shift and
// four masks for its 8 weights, one fma_mix per weight and one
// v_cvt_pk_f16_f32 per two, the reference's rounding of the fp32 value
// (D = d * sc, M = dmin * m).  The per-sub-block terms (D * 2^24 or 2^20,
// -M) of a super-block are computed once per workgroup into an LDS table.
constexpr int kF16aThreads = 256;
constexpr int kF16aBM = 256, kF16aBN = 128;
constexpr int kF16aStage = kF16aBN * kQ4KBytes;     // one super-block of the tile's 128 rows (18 KB)
constexpr int kF16aGroups = kF16aStage / 1024;      // 16-byte lane loads: 18 groups of 64 per stage
constexpr int kF16aNI = (kF16aGroups + 3) / 4;      // per wave (the last wave repeats groups 0, 1)
constexpr int kF16aABufs = 3;
constexpr int kF16aANI = 8;                         // A DMA instructions per wave per chunk (1 KB each)
constexpr int kF16aABuf = kF16aBM * kKC * 2;        // bytes of one A chunk buffer
constexpr int kTabRow = 80;                         // 8 float pairs + pad: 16 rows on distinct bank groups
constexpr int kTabBytes = kF16aBN * kTabRow;
constexpr int kF16aLds = 2 * kF16aStage + kF16aABufs * kF16aABuf + 2 * kTabBytes;   // 152 KB

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
// The four weights of the bytes b0..b3 of w under nibble mask m (low
// 0x000F000F, high 0x00F000F0), in k order: (w & m) holds (b0, b2) and
// ((w >> 8) & m) holds (b1, b3) as fp16 subnormals; each goes through
// v_fma_mix (fp16 source, fp32 value) and the pairs (b0, b1), (b2, b3) are
// rounded to fp16 together.
__device__ __forceinline__ uint2 f16a_dq4(uint32_t w, uint32_t m, float D, float nM) {
    const f16x2 e = __builtin_bit_cast(f16x2, w & m);
    const f16x2 o = __builtin_bit_cast(f16x2, (w >> 8) & m);
    const float v0 = __builtin_fmaf((float)e[0], D, nM), v2 = __builtin_fmaf((float)e[1], D, nM);
    const float v1 = __builtin_fmaf((float)o[0], D, nM), v3 = __builtin_fmaf((float)o[1], D, nM);
    return make_uint2(cvt_pk_f16(v0, v1), cvt_pk_f16(v2, v3));
}


// K split of the fp16-activation tiles (rf_gemm_q4k_f16a_kernel, q6a_wg, q4s_wg): with S > 1 the
// launch holds S x tiles workgroups, tile v of split s at s * tiles + v (the
// workgroups of one split neighbours, so one XCD mostly reads one K range of
// A), split s covers super-blocks [s nsb / S, (s + 1) nsb / S) of every row
// and stores its partial tile to part + s * M * N (row-major M x N, plain
// stores); rf_gemm_split_reduce_kernel adds the S partials in split order.
struct KSplit {
    int S;
    float* part;
};

// PAIR (gate and up in one tile, SwiGLU in the epilogue): the tile's 128
// weight rows are gate rows [n0, n0 + 64) of W (waves 0-1) and the same up
// rows of W1 (waves 2-3), n0 = 64 per column tile; after the K halves are
// added the gate waves hand their sums to the up waves through LDS, which
// store silu(gate) * up into D[M x N] (N = the gate/up row count) as fp32
// (PAIR 1) or rounded to fp16 (PAIR 2, D read as halves).  PAIR 3: a plain
// tile whose store is the up projection of a SwiGLU, fp16 silu(G) * sum
// with the gate product G [M x N] read back.  sp: K split (plain tiles,
// PAIR_ARG 0, only).
template <int PAIR_ARG>
__global__ __launch_bounds__(kF16aThreads) void rf_gemm_q4k_f16a_kernel(const uint16_t* __restrict__ A,
                                                                         const uint8_t* __restrict__ W,
                                                                         const uint8_t* __restrict__ W1,
                                                                         float* __restrict__ D, int M, int N, int K,
                                                                         const float* __restrict__ G, KSplit sp) {
    constexpr int PAIR = PAIR_ARG == 3 ? 0 : PAIR_ARG;      // 3: a plain tile, gated store
    // one LDS block: ring (2 stages), A (3 buffers), scale tables (2); after
    // the loop its first 128 KB carry the K-half exchange
    __shared__ __align__(16) uint8_t lds[kF16aLds];
    uint8_t* ring = lds;
    uint8_t* abuf0 = lds + 2 * kF16aStage;
    uint8_t* tab0 = abuf0 + kF16aABufs * kF16aABuf;
    const uint32_t ring_lds0 = (uint32_t)(size_t)(__attribute__((address_space(3))) uint8_t*)(ring);
    const uint32_t a_lds0 = (uint32_t)(size_t)(__attribute__((address_space(3))) uint8_t*)(abuf0);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kh = wave & 1, wn = wave >> 1;
    const int h = lane >> 5, col = lane & 31;
    const int mtiles = (M + kF16aBM - 1) / kF16aBM;
    int v = xcd_remap((int)blockIdx.x, (int)gridDim.x);
    const int nsb_row = K / kQK;
    int sb0 = 0, nsb = nsb_row;                // this workgroup's super-blocks [sb0, sb0 + nsb) of each row
    if (PAIR_ARG == 0 && sp.S > 1) {
        const int per = mtiles * (N / kF16aBN);
        const int s = v / per;
        v -= s * per;
        sb0 = __builtin_amdgcn_readfirstlane(s * nsb_row / sp.S);
        nsb = __builtin_amdgcn_readfirstlane((s + 1) * nsb_row / sp.S - sb0);
        D = sp.part + (size_t)s * M * N;
    }
    const int m0 = __builtin_amdgcn_readfirstlane((v % mtiles) * kF16aBM);   // the M tiles of one column tile are neighbours
    const int n0 = __builtin_amdgcn_readfirstlane((v / mtiles) * (PAIR ? kF16aBN / 2 : kF16aBN));
    const int nchunks = 4 * nsb;
    const uint32_t row_bytes = (uint32_t)nsb_row * kQ4KBytes;

    // ---- weight ring: stage = super-block sb of the tile's 128 rows; group
    // g of 64 lanes moves 16-byte pieces [64 g, 64 g + 64) (row pc / 9; with
    // PAIR groups 0-8 hold the 64 gate rows, 9-17 the 64 up rows) -------------
    const uint8_t* w_tile = W + (size_t)n0 * row_bytes;
    const uint8_t* w1_tile = PAIR ? W1 + (size_t)n0 * row_bytes : w_tile;
    uint32_t goff[kF16aNI], gdst[kF16aNI];
    bool gup[kF16aNI];
#pragma unroll
    for (int t = 0; t < kF16aNI; ++t) {
        const int g = (wave * kF16aNI + t) % kF16aGroups;
        const int pc = 64 * g + lane;
        gdst[t] = 1024u * (uint32_t)g;
        gup[t] = PAIR && g >= kF16aGroups / 2;
        goff[t] = (uint32_t)(pc / 9 - (gup[t] ? kF16aBN / 2 : 0)) * row_bytes + 16u * (uint32_t)(pc % 9);
    }
    auto w_dma1 = [&](int t, int sb, int slot) {
        lds_dma16(__builtin_amdgcn_readfirstlane(ring_lds0 + (uint32_t)slot * kF16aStage + gdst[t]), goff[t],
                  (gup[t] ? w1_tile : w_tile) + (size_t)(sb0 + min(sb, nsb - 1)) * kQ4KBytes);
    };

    // ---- A: instruction gi = 8 wave + g covers rows 8 gi + L / 8 of the chunk,
    // position L % 8 (k piece (L % 8) ^ g(row)); rows past M read row M - 1 --
    const uint8_t* a_tile = reinterpret_cast<const uint8_t*>(A) + ((size_t)m0 * K + (size_t)sb0 * kQK) * 2;
    uint32_t dma_voff[kF16aANI];
#pragma unroll
    for (int g = 0; g < kF16aANI; ++g) {
        const int r = 8 * (8 * wave + g) + (lane >> 3);
        const int rc = min(r, M - 1 - m0);
        dma_voff[g] = (uint32_t)(rc * K + 8 * ((lane & 7) ^ (r & 7) ^ ((r >> 3) & 1))) * 2u;
    }
    auto a_dma1 = [&](int g, int c, int buf) {
        lds_dma16(a_lds0 + (uint32_t)(buf * kF16aABuf + (8 * wave + g) * 1024), dma_voff[g],
                  a_tile + (size_t)min(c, nchunks - 1) * kKC * 2);
    };

    // ---- B: the lane's two weight rows (columns), 8 qs bytes each per chunk,
    // double buffered by chunk parity R (chunk c + 1 is dequantised while the
    // bytes of chunk c + 2 arrive) ---------------------------------------------
    const int brow0 = 64 * wn + col;                  // rows brow0 and brow0 + 32 of the tile
    u32x2 bqs[2][2];
    auto b_read = [&](auto cq, int slot, int R) {
        constexpr int p = decltype(cq)::value;
        const uint8_t* st = ring + slot * kF16aStage;
#pragma unroll
        for (int j = 0; j < 2; ++j)
            bqs[R][j] = *reinterpret_cast<const u32x2*>(st + (brow0 + 32 * j) * kQ4KBytes + 16 + 32 * p + 16 * kh +
                                                        8 * h);
    };
    // scale table of super-block slot ts: thread tid writes row tid / 2,
    // sub-blocks 4 (tid & 1) .. + 3 as (D * 2^24 or D * 2^20, -M) pairs
    auto tab_build = [&](int ring_slot, int ts) {
        const int r = tid >> 1, hf = tid & 1;
        const u32x4 hd = *reinterpret_cast<const u32x4*>(ring + ring_slot * kF16aStage + r * kQ4KBytes);
        const float d = half_bits_to_float(hd.x), dmin = half_bits_to_float(hd.x >> 16);
        // the 6-bit scales and mins of sub-blocks 4 hf .. 4 hf + 3, one per
        // byte (get_scale_min_k4's layout, word-wide and without branches)
        const uint32_t sc_lo = hd.y & 0x3F3F3F3Fu, mn_lo = hd.z & 0x3F3F3F3Fu;
        const uint32_t sc_hi = (hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u);
        const uint32_t mn_hi = ((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u);
        const uint32_t scw = hf ? sc_hi : sc_lo, mnw = hf ? mn_hi : mn_lo;
        float e[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {      // sub-block 4 hf + i: even -> low nibbles (2^24), odd -> high (2^20)
            e[2 * i] = d * byte_f(scw, i) * ((i & 1) ? 1048576.0f : 16777216.0f);
            e[2 * i + 1] = -(dmin * byte_f(mnw, i));
        }
        float4* dst = reinterpret_cast<float4*>(tab0 + ts * kTabBytes + r * kTabRow + 32 * hf);
        dst[0] = make_float4(e[0], e[1], e[2], e[3]);
        dst[1] = make_float4(e[4], e[5], e[6], e[7]);
    };
    float sD[2][2], sM[2][2];                         // [col block][step]
    auto tab_read = [&](int ts, int p, int j) {
        const float4 t = *reinterpret_cast<const float4*>(tab0 + ts * kTabBytes + (brow0 + 32 * j) * kTabRow + 16 * p);
        sD[j][0] = t.x;
        sM[j][0] = t.y;
        sD[j][1] = t.z;
        sM[j][1] = t.w;
    };
    // bq[buffer][step][col block] = the 8 fp16 weights of one MFMA B operand;
    // word wi (bytes 4 wi .. 4 wi + 3) of column block j fills registers
    // 2 wi, 2 wi + 1 of both steps
    u32x4 bq[2][2][2];
    auto b_piece = [&](int buf, int j, int wi, int R) {
        const uint32_t w = wi ? bqs[R][j].y : bqs[R][j].x;
        const uint2 lo = f16a_dq4(w, 0x000F000Fu, sD[j][0], sM[j][0]);
        const uint2 hi = f16a_dq4(w, 0x00F000F0u, sD[j][1], sM[j][1]);
        bq[buf][0][j][2 * wi] = lo.x;
        bq[buf][0][j][2 * wi + 1] = lo.y;
        bq[buf][1][j][2 * wi] = hi.x;
        bq[buf][1][j][2 * wi + 1] = hi.y;
    };

    f32x16 acc[8][2];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    // fragment of row block i, step s: row 32 i + col, k piece 4 s + 2 kh + h,
    // at position (4 s + 2 kh + h) ^ g(col) of its row (g(32 i + col) = g(col))
    const int gcol = (col & 7) ^ ((col >> 3) & 1);
    f16x8 af[2][8];
    auto frag_ld = [&](int set, int buf, int s, int i) {
        af[set][i] = *reinterpret_cast<const f16x8*>(abuf0 + buf * kF16aABuf + (32 * i + col) * 128 +
                                                     16 * ((4 * s + 2 * kh + h) ^ gcol));
    };

    // ---- prologue: ring stage 0 and A chunks 0, 1; table 0; chunk 0's B ----
#pragma unroll
    for (int t = 0; t < kF16aNI; ++t) w_dma1(t, 0, 0);
#pragma unroll
    for (int g = 0; g < kF16aANI; ++g) a_dma1(g, 0, 0);
#pragma unroll
    for (int g = 0; g < kF16aANI; ++g) a_dma1(g, 1, 1);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    lds_barrier();
    b_read(std::integral_constant<int, 0>{}, 0, 0);
    tab_build(0, 0);
    lds_barrier();
    tab_read(0, 0, 0);
    tab_read(0, 0, 1);
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < 2; ++q) b_piece(0, j, q, 0);
    b_read(std::integral_constant<int, 1>{}, 0, 1);
#pragma unroll
    for (int i = 0; i < 8; ++i) frag_ld(0, 0, 0, i);

    // Chunk c = 4 sb + CQ, A buffer c % 3, ring slot sb % 2.  32 slots, one
    // MFMA each (slot t = 16 step + 2 i + j), separated by scheduling fences,
    // each followed by a slice of the side work: the A fragments of the next
    // step (for step 1: chunk c + 1's first, from a buffer complete since the
    // last barrier); A chunk c + 2 by DMA into the buffer chunk c - 1 used;
    // the B operands of chunk c + 1 (raw bytes read one chunk ago, scale
    // terms from its super-block's table) and the raw bytes of chunk c + 2;
    // in CQ 0 the ring DMA of super-block sb + 1 (complete after CQ 1's
    // barrier) and in CQ 2 its scale table.
    auto iteration = [&](auto cqc, int sb, int ab) {
        constexpr int CQ = decltype(cqc)::value;
        constexpr int P = CQ & 1;                           // bq buffer of this chunk
        const int c = 4 * sb + CQ;
        const int slot = sb & 1;
        const int abn = ab == 2 ? 0 : ab + 1;               // chunk c + 1
        const int abs2 = abn == 2 ? 0 : abn + 1;            // chunk c + 2
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const f16x8 b0 = __builtin_bit_cast(f16x8, bq[P][s][0]);
            const f16x8 b1 = __builtin_bit_cast(f16x8, bq[P][s][1]);
#pragma unroll
            for (int i = 0; i < 8; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int t = 16 * s + 2 * i + j;
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[s][i], j ? b1 : b0, acc[i][j], 0, 0, 0);
                    if (j == 0) frag_ld(s ^ 1, s ? abn : ab, s ^ 1, i);
                    if (t < 2 * kF16aANI && (t & 1) == 0) a_dma1(t >> 1, c + 2, abs2);
                    if (t == 1 || t == 14) tab_read(CQ == 3 ? slot ^ 1 : slot, (CQ + 1) & 3, t == 14);
                    if (t == 5 || t == 10) b_piece(P ^ 1, 0, t == 10, P ^ 1);
                    if (t == 20 || t == 25) b_piece(P ^ 1, 1, t == 25, P ^ 1);
                    if constexpr (CQ == 2) {
                        if (t == 3) tab_build(slot ^ 1, slot ^ 1);
                    }
                    if (t == 17) b_read(std::integral_constant<int, (CQ + 2) & 3>{}, CQ < 2 ? slot : slot ^ 1, P);
                    if constexpr (CQ == 0) {
                        // into the slot super-block sb - 1 used (last read in its CQ 1)
                        if (t >= 18 && t < 18 + 2 * kF16aNI && (t & 1) == 0) w_dma1((t - 18) >> 1, sb + 1, slot ^ 1);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
        }
        // this chunk's A DMA (chunk c + 2) is complete before the barrier; the
        // ring DMA issued after it (CQ 0) may stay in flight one more chunk
        if constexpr (CQ == 0)
            asm volatile("s_waitcnt vmcnt(%0)" :: "n"(kF16aNI) : "memory");
        else
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        // every LDS access of the chunk except the last 8 fragment reads (of
        // chunk c + 1, whose buffer is not written before the next barrier) is
        // complete -- LDS operations complete in order
        asm volatile("s_waitcnt lgkmcnt(8)\n\ts_barrier" ::: "memory");
    };
    int ab = 0;                                     // (4 sb) % 3
    for (int sb = 0; sb < nsb; ++sb) {
        iteration(std::integral_constant<int, 0>{}, sb, ab);
        iteration(std::integral_constant<int, 1>{}, sb, ab == 2 ? 0 : ab + 1);
        iteration(std::integral_constant<int, 2>{}, sb, ab == 0 ? 2 : ab - 1);
        iteration(std::integral_constant<int, 3>{}, sb, ab);
        ab = ab == 2 ? 0 : ab + 1;
    }

    // ---- K halves: wave kh = 1 hands row blocks 0-3 to kh = 0, kh = 0 hands
    // row blocks 4-7 to kh = 1; each then adds and stores its four blocks.
    // [wave][block i][col block j][e / 4][lane] of float4: each access is one
    // contiguous 1 KB per wave (4 waves x 4 x 2 x 4 KB = 128 KB) -------------
    // (acc indexed by compile-time constants only: one branch per wave half,
    // the barrier between the halves outside them)
    __syncthreads();
    float4* xch = reinterpret_cast<float4*>(lds);
    auto give_half = [&](auto khc) {
        constexpr int give = decltype(khc)::value ? 0 : 4;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    xch[(((wave * 4 + i) * 2 + j) * 4 + q) * 64 + lane] =
                        make_float4(acc[give + i][j][4 * q], acc[give + i][j][4 * q + 1],
                                    acc[give + i][j][4 * q + 2], acc[give + i][j][4 * q + 3]);
    };
    auto keep_half = [&](auto khc, auto fullc) {
        constexpr int KH = decltype(khc)::value;
        constexpr bool FULL = decltype(fullc)::value;     // all 256 rows of the tile below M
        constexpr int keep = KH ? 4 : 0;
        const int partner = wave ^ 1;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int ncol = n0 + 64 * wn + 32 * j + col;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float4 o4 = xch[(((partner * 4 + i) * 2 + j) * 4 + q) * 64 + lane];
                    const float o[4] = {o4.x, o4.y, o4.z, o4.w};
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const int row = m0 + 32 * (keep + i) + 8 * q + 4 * h + u;
                        if (!FULL && row >= M) continue;
                        // kh 0 + kh 1 in a fixed order (either wave forms the same sum)
                        const float a = acc[keep + i][j][4 * q + u];
                        const float sum = KH ? o[u] + a : a + o[u];
                        const size_t e = (size_t)row * N + ncol;
                        if constexpr (PAIR_ARG == 3) {      // up projection of a SwiGLU: fp16 silu(gate) * up
                            const float gg = G[e];
                            reinterpret_cast<uint16_t*>(D)[e] = f16_bits_rn(gg / (1.0f + expf(-gg)) * sum);
                        } else {
                            D[e] = sum;
                        }
                    }
                }
            }
    };
    if (kh)
        give_half(std::integral_constant<int, 1>{});
    else
        give_half(std::integral_constant<int, 0>{});
    __syncthreads();
    const bool full = m0 + kF16aBM <= M;
    if constexpr (PAIR) {
        // per wave half (its own code path to the end, so the accumulators
        // are never merged across branches): the K halves added into acc
        // (kh 0 + kh 1, the order above), the gate waves' sums to LDS at
        // [kh][block i][j][q][lane], the up waves store silu(gate) * up
        auto pair_tail = [&](auto khc) {
            constexpr int KH = decltype(khc)::value;
            constexpr int keep = KH ? 4 : 0;
            const int partner = wave ^ 1;
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const float4 o4 = xch[(((partner * 4 + i) * 2 + j) * 4 + q) * 64 + lane];
                        const float o[4] = {o4.x, o4.y, o4.z, o4.w};
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            const float a = acc[keep + i][j][4 * q + u];
                            acc[keep + i][j][4 * q + u] = KH ? o[u] + a : a + o[u];
                        }
                    }
            __syncthreads();
            if (wn == 0) {
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
#pragma unroll
                        for (int q = 0; q < 4; ++q)
                            xch[(((KH * 4 + i) * 2 + j) * 4 + q) * 64 + lane] =
                                make_float4(acc[keep + i][j][4 * q], acc[keep + i][j][4 * q + 1],
                                            acc[keep + i][j][4 * q + 2], acc[keep + i][j][4 * q + 3]);
            }
            __syncthreads();
            if (wn == 0) return;
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int ncol = n0 + 32 * j + col;
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const float4 g4 = xch[(((KH * 4 + i) * 2 + j) * 4 + q) * 64 + lane];
                        const float gv[4] = {g4.x, g4.y, g4.z, g4.w};
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            const int row = m0 + 32 * (keep + i) + 8 * q + 4 * h + u;
                            if (row >= M) continue;
                            const float gg = gv[u];
                            const float r = gg / (1.0f + expf(-gg)) * acc[keep + i][j][4 * q + u];
                            if constexpr (PAIR == 2)
                                reinterpret_cast<uint16_t*>(D)[(size_t)row * N + ncol] = f16_bits_rn(r);
                            else
                                D[(size_t)row * N + ncol] = r;
                        }
                    }
                }
        };
        if (kh)
            pair_tail(std::integral_constant<int, 1>{});
        else
            pair_tail(std::integral_constant<int, 0>{});
        return;
    }
    if (kh) {
        if (full)
            keep_half(std::integral_constant<int, 1>{}, std::true_type{});
        else
            keep_half(std::integral_constant<int, 1>{}, std::false_type{});
    } else {
        if (full)
            keep_half(std::integral_constant<int, 0>{}, std::true_type{});
        else
            keep_half(std::integral_constant<int, 0>{}, std::false_type{});
    }
}

// ── q6a: Q6_K GEMM on fp16 activations, 128 x 64 tiles, K slices on waves
// (rf_gemm_q6_k_f16_launch) ───────────────────────────────────────────────
// Workgroup = 512 threads (two waves per SIMD) over a 128 (M) x 64 (N) tile:
// at the Llama-3.1-8B down projection (N = 4096) and M = 512 that is 256
// workgroups, one per CU, with no split of K across workgroups.  Wave
// w = 4 cg + ks takes k [16 ks, 16 ks + 16) of every 64-wide chunk for the
// 128 rows and the 32 columns [32 cg, +32) of the tile (4 MFMAs per chunk),
// so each weight is dequantised once per workgroup; the four K-slice
// partials of a column group are added through LDS at the end, in ks order.
// The second wave on each SIMD issues its dequantisation while the first
// one's MFMAs run.
//
// K order.  Chunk c of a Q6_K row covers k [64 c, 64 c + 64) of super-block
// c / 4; its 16-group g = 4 (c % 4) + ks holds the elements 128 n + 32 q + l,
// n = g >> 3, q = (g >> 1) & 3, l in [16 (g & 1), +16): low 4 bits in ql byte
// 64 n + 32 (q & 1) + l (low nibble for q < 2, high for q >= 2), high 2 bits
// at bit 2 q of qh byte 32 n + l, sub-block scale sc[g].  Lane half h takes
// l + 8 h .. l + 8 h + 7: 8 ql bytes and 8 qh bytes of its weight row, the
// same bytes for chunks 2 n and 2 n + 1 of a super-block.
//
// Weights.  Q6_K blocks (210 bytes) start 2-byte aligned.  The ring stage of
// super-block sb holds, per tile row, the 224-byte 16-byte aligned window
// that starts at floor16(sb * 210) (the block at byte 2 sb % 16 of it), in a
// 240-byte LDS row (60 dwords: the 32 rows of a read fall on 8 banks, 4-way),
// loaded by 16-byte LDS DMA (16 instructions per stage: the DMA costs per
// instruction, not per byte).  Three stages: super-block
// sb + 2 loads while sb is used.  K % 2048 == 0 keeps the last window of a
// row inside it.  A arrives as in rf_gemm_q4k_f16a_kernel
// (16-byte LDS DMA, XOR-swizzled 128-byte rows), seven chunk buffers deep:
// a DMA gets four chunks to land.
//
// Dequantisation.  The 6-bit values of four weights are assembled in the
// bytes of a word (the qh field moved to bits 4-5 by one rotate), spread to
// fp16 subnormal halves q * 2^-24 by v_perm, and fma_mix(q * 2^-24,
// s * 2^24, -32 s) = s (q - 32) is exact in fp32 (s = d sc has at most 19
// significant bits), so its fp16 rounding in the same instruction is the
// reference's value __float2half(d * sc * (q - 32)).
//
// Tall tiles (FMR = 8: 256 x 64, Q6aGeom<8>): each wave takes 8 row blocks
// (8 MFMAs per chunk against the same dequantised B operand, so each weight
// is dequantised once per 256 rows of A: half the dequantisation per MFMA of
// the 128-row tiles).  LDS then holds four 32 KB A buffers (a DMA lands
// within one chunk of slack) and two ring stages; the K-slice partials are
// exchanged in two rounds of four row blocks.
constexpr int kQ6aThreads = 512;
constexpr int kQ6aBM = 128, kQ6aBN = 64;
constexpr int kQ6aRowB = 240;                         // ring bytes per weight row (14 pieces + 1 padding)
constexpr int kQ6aRingInstr = 16;                     // 16-byte DMAs per stage
constexpr int kQ6aStage = kQ6aRingInstr * 1024;       // 16384 B
constexpr int kQ6aLdsXch = 8 * 3 * 4096;              // 98,304 B: three row blocks of each wave's partial

// DMAs a wave may leave in flight at the end of chunk c = 4 sb + CQ of the
// K-sliced tiles (q6a_wg, q4s_wg), whose waves issue apw A DMAs per chunk
// and, in CQ 0, rpw ring DMAs for super-block sb + rs - 1.  In flight: the
// DMAs of the last `lag` chunks (an A DMA issued in chunk c lands by the end
// of chunk c + lag, before its buffer's first read in c + lag + 1); with two
// ring stages the stage loaded in chunk 4 sb is read in chunk 4 sb + 3, so
// at the end of CQ 2 the window starts after chunk 4 sb.  vmcnt counts in
// issue order, so completing the oldest DMA completes every older one.
constexpr int ksplit_dma_out(int cq, int apw, int rpw, int lag, int rs) {
    const int win = (rs == 2 && cq >= 2 && cq < lag) ? cq : lag;    // chunks in the window, ending at c
    const int ring_in = win >= 4 ? 1 : (cq < win ? 1 : 0);         // the window holds a CQ 0 chunk
    return apw * win + rpw * ring_in;
}

// Tile geometry: FMR = 2 (64 rows, M <= 64) is lean -- two ring stages and
// six A buffers, 80 KB of LDS, so two workgroups share a CU -- and its K
// split spreads over twice the CUs (measured on MI355X, 4096 x 14336 at
// M = 64: 27.3 us against 31.0 for 128-row tiles one per CU; the same
// geometry for the Q4_K 64-row tiles was slower, 24.0 against 21.0).
template <int FMR>
struct Q6aGeom {
    static constexpr int kBM = 32 * FMR;
    static constexpr int kRS = FMR == 4 ? 3 : 2;      // ring stages: super-block sb + kRS - 1 loads while sb is used
    static constexpr int kABufs = FMR == 4 ? 7 : (FMR == 2 ? 6 : 4);   // DMA of chunk c + kABufs - 1 in chunk c
    static constexpr int kLag = kABufs - 3;           // chunks a DMA may stay in flight
    static constexpr int kABuf = kBM * kKC * 2;       // 8, 16 or 32 KB
    static constexpr int kAPW = FMR / 2;              // A DMAs per wave per chunk (1 KB each)
    static constexpr int kXB = FMR < 4 ? FMR : 4;     // row blocks per exchange round of the K-slice partials
    static constexpr int kRounds = FMR / kXB;
    static constexpr int kLdsLoop = kRS * kQ6aStage + kABufs * kABuf;   // 81,920 B (FMR 2) or 163,840 B
    static constexpr int kLdsXch = 8 * kXB * 4096;    // every wave's partial blocks of one round
    static constexpr int kLds = kLdsLoop > kLdsXch ? kLdsLoop : kLdsXch;
};
constexpr int kQ6aLds = Q6aGeom<4>::kLds;

// The 4 fp16 weights s (q - 32) of the 6-bit values in the bytes of qb, in
// byte order, as two packed words.
__device__ __forceinline__ u32x2 q6a_dq4(uint32_t qb, float S24, float nO) {
    const f16x2 e = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(qb, qb, 0x0C020C00u));
    const f16x2 o = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(qb, qb, 0x0C030C01u));
    f16x2 lo, hi;
    lo[0] = (_Float16)__builtin_fmaf((float)e[0], S24, nO);
    lo[1] = (_Float16)__builtin_fmaf((float)o[0], S24, nO);
    hi[0] = (_Float16)__builtin_fmaf((float)e[1], S24, nO);
    hi[1] = (_Float16)__builtin_fmaf((float)o[1], S24, nO);
    return u32x2{__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
}

// Tile v of the launch (after the XCD remap); lds: the kLds-byte LDS block.

template <bool ACC, int FMR = 4>
__device__ __forceinline__ void q6a_wg(const uint16_t* __restrict__ A, const uint8_t* __restrict__ W,
                                       float* __restrict__ D, int M, int N, int K, int v, uint8_t* lds,
                                       KSplit sp = KSplit{1, nullptr}) {
    using G = Q6aGeom<FMR>;
    uint8_t* ring = lds;
    uint8_t* abuf0 = lds + G::kRS * kQ6aStage;
    const uint32_t ring_lds0 = (uint32_t)(size_t)(__attribute__((address_space(3))) uint8_t*)(ring);
    const uint32_t a_lds0 = (uint32_t)(size_t)(__attribute__((address_space(3))) uint8_t*)(abuf0);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ks = wave & 3, cg = wave >> 2;
    const int h = lane >> 5, col = lane & 31;
    const int mtiles = (M + G::kBM - 1) / G::kBM;
    const int nsb_row = K / kQK;
    int sb0 = 0, nsb = nsb_row;                // this workgroup's super-blocks [sb0, sb0 + nsb) of each row
    if (sp.S > 1) {
        const int per = mtiles * (N / kQ6aBN);
        const int s = v / per;
        v -= s * per;
        sb0 = s * nsb_row / sp.S;
        nsb = (s + 1) * nsb_row / sp.S - sb0;
        D = sp.part + (size_t)s * M * N;
    }
    const int m0 = (v % mtiles) * G::kBM;      // the M tiles of one column tile are neighbours
    const int n0 = (v / mtiles) * kQ6aBN;
    const int nchunks = 4 * nsb;
    const uint32_t row_bytes = (uint32_t)nsb_row * kQ6KBytes;

    // ---- weight ring: DMA instruction ii = wave + 8 t moves the 16-byte
    // pieces [64 ii, 64 ii + 64) of the stage (row i / 15, piece i % 15 of the
    // row's window; piece 14 and the last 64 pieces are padding and repeat
    // piece 13) ----------------------------------------------------------------
    const uint8_t* w_tile = W + (size_t)n0 * row_bytes;
    constexpr int kRPW = kQ6aRingInstr / 8;   // 2 per wave per super-block
    uint32_t roff[kRPW];
#pragma unroll
    for (int t = 0; t < kRPW; ++t) {
        const int i = 64 * (wave + 8 * t) + lane;
        const int r = min(i / 15, 63), pc = i < 960 ? min(i % 15, 13) : 13;
        roff[t] = (uint32_t)r * row_bytes + 16u * (uint32_t)pc;
    }
    auto w_dma1 = [&](int t, int sb, int slot) {
        const int s = sb0 + min(sb, nsb - 1);
        lds_dma16(ring_lds0 + (uint32_t)slot * kQ6aStage + 1024u * (uint32_t)(wave + 8 * t), roff[t],
                  w_tile + (size_t)((s * kQ6KBytes) & ~15));
    };

    // ---- A: instruction gi = kAPW wave + g covers rows 8 gi + L / 8 of the
    // chunk, position L % 8 (k piece (L % 8) ^ g(row)); rows past M read row
    // M - 1 --------------------------------------------------------------------
    const uint8_t* a_tile = reinterpret_cast<const uint8_t*>(A) + ((size_t)m0 * K + (size_t)sb0 * kQK) * 2;
    uint32_t dma_voff[G::kAPW];
#pragma unroll
    for (int g = 0; g < G::kAPW; ++g) {
        const int r = 8 * (G::kAPW * wave + g) + (lane >> 3);
        const int rc = min(r, M - 1 - m0);
        dma_voff[g] = (uint32_t)(rc * K + 8 * ((lane & 7) ^ (r & 7) ^ ((r >> 3) & 1))) * 2u;
    }
    auto a_dma1 = [&](int g, int c, int buf) {
        lds_dma16(a_lds0 + (uint32_t)(buf * G::kABuf + (G::kAPW * wave + g) * 1024), dma_voff[g],
                  a_tile + (size_t)min(c, nchunks - 1) * kKC * 2);
    };

    // ---- B: the lane's weight row (column 32 cg + col) in the ring stage of
    // its super-block (block at byte 2 sb % 16 of the row): raw ql / qh words
    // of half n (dword reads, shifted into place for odd super-blocks), the
    // per-super-block factors d * 2^24 and -32 d, and the chunk's sub-block
    // scale -------------------------------------------------------------------
    const int brow = 32 * cg + col;
    uint32_t rql[2], rqh[2];
    auto raw_read = [&](int n, int sb) {
        const int off = (2 * (sb0 + sb)) & 15;
        const uint8_t* rowp = ring + (sb % G::kRS) * kQ6aStage + brow * kQ6aRowB;
        const int oql = off + 64 * n + 16 * ks + 8 * h;
        const int oqh = off + 128 + 32 * n + 16 * (ks & 1) + 8 * h;
        const uint32_t* pl = reinterpret_cast<const uint32_t*>(rowp + (oql & ~3));
        const uint32_t* ph = reinterpret_cast<const uint32_t*>(rowp + (oqh & ~3));
        if ((sb0 + sb) & 1) {
            const uint32_t l0 = pl[0], l1 = pl[1], l2 = pl[2];
            const uint32_t h0 = ph[0], h1 = ph[1], h2 = ph[2];
            rql[0] = __builtin_amdgcn_alignbit(l1, l0, 16);
            rql[1] = __builtin_amdgcn_alignbit(l2, l1, 16);
            rqh[0] = __builtin_amdgcn_alignbit(h1, h0, 16);
            rqh[1] = __builtin_amdgcn_alignbit(h2, h1, 16);
        } else {
            rql[0] = pl[0];
            rql[1] = pl[1];
            rqh[0] = ph[0];
            rqh[1] = ph[1];
        }
    };
    float d24 = 0.0f, dm32 = 0.0f;
    int scb = 0;
    auto d_read = [&](int sb) {
        const int off = (2 * (sb0 + sb)) & 15;
        const float d = half_bits_to_float(
            *reinterpret_cast<const uint16_t*>(ring + (sb % G::kRS) * kQ6aStage + brow * kQ6aRowB + off + 208));
        d24 = d * 16777216.0f;
        dm32 = -32.0f * d;
    };
    auto sc_read = [&](int cq, int sb) {
        const int off = (2 * (sb0 + sb)) & 15;
        scb = *reinterpret_cast<const int8_t*>(ring + (sb % G::kRS) * kQ6aStage + brow * kQ6aRowB + off + 192 +
                                               4 * cq + ks);
    };
    // qh field 2q of each byte to bits 4-5: rotate right by (2q - 4) mod 32
    const uint32_t rot0 = (uint32_t)(2 * (ks >> 1) + 28) & 31u;   // q = ks >> 1 (chunks 0, 2)
    const uint32_t rot1 = (uint32_t)(2 * (ks >> 1)) & 31u;        // q = 2 + (ks >> 1) (chunks 1, 3)
    u32x4 bq[2];                          // [chunk parity]
    auto b_dequant = [&](int t, int P) {
        const float sc = (float)scb;
        const float S24 = d24 * sc, nO = dm32 * sc;
        const uint32_t rot = t ? rot1 : rot0;
        u32x2 r[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t lo = t ? (rql[i] >> 4) : rql[i];
            const uint32_t qb = (lo & 0x0F0F0F0Fu) | (__builtin_amdgcn_alignbit(rqh[i], rqh[i], rot) & 0x30303030u);
            r[i] = q6a_dq4(qb, S24, nO);
        }
        bq[P] = u32x4{r[0].x, r[0].y, r[1].x, r[1].y};
    };

    f32x16 acc[FMR];
#pragma unroll
    for (int i = 0; i < FMR; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][e] = 0.0f;

    // fragment of row block i: row 32 i + col, k piece 2 ks + h at position
    // (2 ks + h) ^ g(col) of its row
    const int gcol = (col & 7) ^ ((col >> 3) & 1);
    f16x8 af[2][FMR];
    auto frag_ld = [&](int set, int buf, int i) {
        af[set][i] = *reinterpret_cast<const f16x8*>(abuf0 + buf * G::kABuf + (32 * i + col) * 128 +
                                                     16 * ((2 * ks + h) ^ gcol));
    };

    // ---- prologue: ring stages 0 .. kRS - 2; A chunks 0 .. kABufs - 2; chunk
    // 0's operands -------------------------------------------------------------
#pragma unroll
    for (int st = 0; st < G::kRS - 1; ++st)
#pragma unroll
        for (int t = 0; t < kRPW; ++t) w_dma1(t, st, st);
#pragma unroll
    for (int c = 0; c < G::kABufs - 1; ++c)
#pragma unroll
        for (int g = 0; g < G::kAPW; ++g) a_dma1(g, c, c);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    lds_barrier();
    raw_read(0, 0);
    d_read(0);
    sc_read(0, 0);
    b_dequant(0, 0);
#pragma unroll
    for (int i = 0; i < FMR; ++i) frag_ld(0, 0, i);

    // Chunk c = 4 sb + CQ uses A buffer c % kABufs and ring stage sb % kRS.
    // Its FMR MFMA slots carry: the A fragments of chunk c + 1, the A DMA of
    // chunk c + kABufs - 1 (into the buffer chunk c - 1 used), in CQ 0 the
    // ring DMA of super-block sb + kRS - 1 (into the stage sb - 1 used), and
    // the B operands of chunk c + 1 (raw bytes of half n read in the chunk
    // before 2 n).  At the end every DMA issued up to chunk c - kLag is
    // complete (vmcnt = the A DMAs of the last kLag chunks and the ring DMAs
    // among them), then one barrier.  A ring stage is first read in the last
    // chunk of the super-block before it: kRS = 3 (128-row tiles): the DMA
    // issued in chunk 4 sb lands by the end of chunk 4 sb + 4, before the
    // read in chunk 4 sb + 7; kRS = 2 (256 rows): it lands by the end of
    // chunk 4 sb + 1, before the read in chunk 4 sb + 3.
    int ab = 0;                                     // c % kABufs
    auto iteration = [&](auto cqc, int sb) {
        constexpr int CQ = decltype(cqc)::value;
        constexpr int P = CQ & 1;
        constexpr int NQ = (CQ + 1) & 3;            // chunk c + 1 within its super-block
        // ring DMAs (issued in CQ 0) among the DMAs of the last kLag chunks
        constexpr int kOut = ksplit_dma_out(CQ, G::kAPW, kRPW, G::kLag, G::kRS);
        const int c = 4 * sb + CQ;
        const int sbn = CQ == 3 ? sb + 1 : sb;
        const int abn = ab == G::kABufs - 1 ? 0 : ab + 1;       // chunk c + 1
        const int abp = ab == 0 ? G::kABufs - 1 : ab - 1;       // chunk c - 1 (= c + kABufs - 1)
#pragma unroll
        for (int i = 0; i < FMR; ++i) {
            acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[P][i], __builtin_bit_cast(f16x8, bq[P]), acc[i], 0, 0,
                                                            0);
            if (i == 0) {
                // every LDS read of chunk c + 1 right after the first MFMA
                if constexpr ((NQ & 1) == 0) raw_read(NQ >> 1, sbn);
                if constexpr (NQ == 0) d_read(sbn);
                sc_read(NQ, sbn);
#pragma unroll
                for (int r = 0; r < FMR; ++r) frag_ld(P ^ 1, abn, r);
            }
            if (i < G::kAPW) a_dma1(i, c + G::kABufs - 1, abp);
            if constexpr (CQ == 0) {
                if (i < kRPW) w_dma1(i, sb + G::kRS - 1, (sb + G::kRS - 1) % G::kRS);
            }
            if (i == FMR - 1) b_dequant(NQ & 1, P ^ 1);
            __builtin_amdgcn_sched_barrier(0);
        }
        asm volatile("s_waitcnt vmcnt(%0)" :: "n"(kOut) : "memory");
        lds_barrier();
        ab = abn;
    };
    for (int sb = 0; sb < nsb; ++sb) {
        iteration(std::integral_constant<int, 0>{}, sb);
        iteration(std::integral_constant<int, 1>{}, sb);
        iteration(std::integral_constant<int, 2>{}, sb);
        iteration(std::integral_constant<int, 3>{}, sb);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    // ---- K slices, in rounds of kXB row blocks: every wave parks the round's
    // blocks in LDS ([wave][block][e / 4][lane] of float4: each access one
    // contiguous 1 KB per wave); wave (ks, cg), ks < kXB, adds block
    // kXB rd + ks of column group cg over ks' = 0..3 in that order (acc
    // indexed by compile-time constants: the round loop is unrolled) ---------
    float4* xch = reinterpret_cast<float4*>(lds);
    const int ncol = n0 + 32 * cg + col;
#pragma unroll
    for (int rd = 0; rd < G::kRounds; ++rd) {
        __syncthreads();
#pragma unroll
        for (int i = 0; i < G::kXB; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                xch[((wave * G::kXB + i) * 4 + q) * 64 + lane] =
                    make_float4(acc[G::kXB * rd + i][4 * q], acc[G::kXB * rd + i][4 * q + 1],
                                acc[G::kXB * rd + i][4 * q + 2], acc[G::kXB * rd + i][4 * q + 3]);
        __syncthreads();
        if (ks < G::kXB) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float s4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int src = 0; src < 4; ++src) {
                    const float4 p = xch[(((4 * cg + src) * G::kXB + ks) * 4 + q) * 64 + lane];
                    s4[0] += p.x;
                    s4[1] += p.y;
                    s4[2] += p.z;
                    s4[3] += p.w;
                }
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int row = m0 + 32 * (G::kXB * rd + ks) + 8 * q + 4 * h + u;
                    if (row < M) {
                        float* o = D + (size_t)row * N + ncol;
                        *o = ACC ? *o + s4[u] : s4[u];
                    }
                }
            }
        }
    }
}

template <bool ACC, int FMR>
__global__ __launch_bounds__(kQ6aThreads) void rf_gemm_q6k_f16a_kernel(const uint16_t* __restrict__ A,
                                                                        const uint8_t* __restrict__ W,
                                                                        float* __restrict__ D, int M, int N, int K,
                                                                        KSplit sp) {
    __shared__ __align__(16) uint8_t lds[Q6aGeom<FMR>::kLds];
    q6a_wg<ACC, FMR>(A, W, D, M, N, K, xcd_remap((int)blockIdx.x, (int)gridDim.x), lds, sp);
}

// ── q4s: Q4_K GEMM on fp16 activations, 32 FMR x 64 tiles, K slices on waves
// (rf_gemm_q4_k_f16_launch where the 256 x 128 tiles leave CUs idle) ───────
// The layout of rf_gemm_q6k_f16a_kernel for Q4_K weights: eight waves, wave
// w = 4 cg + ks takes k [16 ks, +16) of every 64-wide chunk for the tile's
// rows (FMR row blocks of 32) and the 32 columns of group cg; the four
// K-slice partials of an output block are added through LDS in ks order,
// each output written once.  Chunk c covers nibble pair p = c % 4 of
// super-block c / 4: slice ks holds the low (ks < 2) or high nibbles of qs
// bytes 32 p + 16 (ks & 1) .. + 15, lane half h bytes + 8 h .. + 7, of
// sub-block 2 p + (ks >> 1).  The ring stage of a super-block holds its
// 144-byte blocks of the tile's 64 weight rows (16-byte aligned: plain
// LDS DMA, 16 instructions of which 9 carry the stage); each lane takes its
// row's four (d sc 2^24 or 2^20, -dmin m) pairs from the header once per
// super-block and dequantises as rf_gemm_q4k_f16a_kernel does (nibbles as
// fp16 subnormals into v_fma_mix, the fp32 value rounded to fp16 after).
constexpr int kQ4sThreads = 512;
constexpr int kQ4sBN = 64;
constexpr int kQ4sStage = 16 * 1024;                  // 64 rows x 144 B (+ padding DMAs)

// FMR = 8 (256 x 64 tiles): each weight dequantised once per 256 rows of A;
// LDS then holds two ring stages and four 32 KB A buffers (one chunk of DMA
// slack), as in the tall Q6_K tiles, and the K-slice partials go through
// LDS in rounds of four row blocks.
template <int FMR>
struct Q4sGeom {
    static constexpr int kBM = 32 * FMR;
    static constexpr int kRS = FMR == 8 ? 2 : 3;      // ring stages
    static constexpr int kABufs = FMR == 8 ? 4 : 7;   // DMA of chunk c + kABufs - 1 issued in chunk c
    static constexpr int kLag = kABufs - 3;           // chunks a DMA may stay in flight
    static constexpr int kABuf = kBM * kKC * 2;       // FMR x 4 KB
    static constexpr int kAPW = FMR / 2;              // A DMAs per wave per chunk (1 KB each)
    static constexpr int kRounds = FMR == 8 ? 2 : 1;  // exchange rounds of the K-slice partials
    static constexpr int kXB = FMR / kRounds;         // row blocks per round
    // a ring stage DMA'd in chunk 4 sb (super-block sb + kRS - 1) is first
    // read in chunk 4 (sb + kRS - 1) - 1, so it must land within kLag chunks
    static_assert(FMR == 8 || kLag <= 4 * (kRS - 1) - 2, "ring stage read before its DMA lands");
    static constexpr int kLdsLoop = kRS * kQ4sStage + kABufs * kABuf;
    static constexpr int kLdsXch = 8 * kXB * 4096;    // every wave's partial blocks of one round
    static constexpr int kLds = kLdsLoop > kLdsXch ? kLdsLoop : kLdsXch;
};

// Tile v of the launch (after the XCD remap); lds: the kLds-byte LDS block.
template <int FMR, bool ACC>
__device__ __forceinline__ void q4s_wg(const uint16_t* __restrict__ A, const uint8_t* __restrict__ W,
                                       float* __restrict__ D, int M, int N, int K, int v, uint8_t* lds,
                                       const float* __restrict__ gate = nullptr, KSplit sp = KSplit{1, nullptr}) {
    using G = Q4sGeom<FMR>;
    uint8_t* ring = lds;
    uint8_t* abuf0 = lds + G::kRS * kQ4sStage;
    const uint32_t ring_lds0 = (uint32_t)(size_t)(__attribute__((address_space(3))) uint8_t*)(ring);
    const uint32_t a_lds0 = (uint32_t)(size_t)(__attribute__((address_space(3))) uint8_t*)(abuf0);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ks = wave & 3, cg = wave >> 2;
    const int h = lane >> 5, col = lane & 31;
    const int mtiles = (M + G::kBM - 1) / G::kBM;
    const int nsb_row = K / kQK;
    int sb0 = 0, nsb = nsb_row;                // this workgroup's super-blocks [sb0, sb0 + nsb) of each row
    if (sp.S > 1) {
        const int per = mtiles * (N / kQ4sBN);
        const int s = v / per;
        v -= s * per;
        sb0 = s * nsb_row / sp.S;
        nsb = (s + 1) * nsb_row / sp.S - sb0;
        D = sp.part + (size_t)s * M * N;
        gate = nullptr;
    }
    const int m0 = (v % mtiles) * G::kBM;      // the M tiles of one column tile are neighbours
    const int n0 = (v / mtiles) * kQ4sBN;
    const int nchunks = 4 * nsb;
    const uint32_t row_bytes = (uint32_t)nsb_row * kQ4KBytes;

    // ---- weight ring: DMA instruction ii = wave + 8 t moves 16-byte pieces
    // [64 ii, 64 ii + 64) of the stage (row i / 9, piece i % 9; pieces past
    // the 576 of the stage repeat the last one) ------------------------------
    const uint8_t* w_tile = W + (size_t)n0 * row_bytes + (size_t)sb0 * kQ4KBytes;
    uint32_t roff[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int i = 64 * (wave + 8 * t) + lane;
        roff[t] = i < 576 ? (uint32_t)(i / 9) * row_bytes + 16u * (uint32_t)(i % 9) : 63u * row_bytes + 128u;
    }
    auto w_dma1 = [&](int t, int sb, int slot) {
        lds_dma16(ring_lds0 + (uint32_t)slot * kQ4sStage + 1024u * (uint32_t)(wave + 8 * t), roff[t],
                  w_tile + (size_t)min(sb, nsb - 1) * kQ4KBytes);
    };

    // ---- A: instruction gi = kAPW wave + g covers rows 8 gi + L / 8 of the
    // chunk, position L % 8 (k piece (L % 8) ^ g(row)); rows past M read row
    // M - 1 ---------------------------------------------------------------------
    const uint8_t* a_tile = reinterpret_cast<const uint8_t*>(A) + ((size_t)m0 * K + (size_t)sb0 * kQK) * 2;
    uint32_t dma_voff[G::kAPW];
#pragma unroll
    for (int g = 0; g < G::kAPW; ++g) {
        const int r = 8 * (G::kAPW * wave + g) + (lane >> 3);
        const int rc = min(r, M - 1 - m0);
        dma_voff[g] = (uint32_t)(rc * K + 8 * ((lane & 7) ^ (r & 7) ^ ((r >> 3) & 1))) * 2u;
    }
    auto a_dma1 = [&](int g, int c, int buf) {
        lds_dma16(a_lds0 + (uint32_t)(buf * G::kABuf + (G::kAPW * wave + g) * 1024), dma_voff[g],
                  a_tile + (size_t)min(c, nchunks - 1) * kKC * 2);
    };

    // ---- B: the lane's weight row (column 32 cg + col) in the ring stage ------
    const int brow = 32 * cg + col;
    const int hf = ks >> 1;                     // high nibbles (odd sub-block) for ks >= 2
    const uint32_t nmask = hf ? 0x00F000F0u : 0x000F000Fu;
    const float nfac = hf ? 1048576.0f : 16777216.0f;
    float sD[4], sM[4];                         // per chunk p of the super-block: (d sc 2^x, -dmin m)
    auto hdr_read = [&](int sb) {
        const u32x4 hd = *reinterpret_cast<const u32x4*>(ring + (sb % G::kRS) * kQ4sStage + brow * kQ4KBytes);
        const float d = half_bits_to_float(hd.x) * nfac, dmin = half_bits_to_float(hd.x >> 16);
        // get_scale_min_k4 for sub-blocks hf, 2 + hf (bytes of the low words)
        // and 4 + hf, 6 + hf (high words), word-wide without branches
        const uint32_t sc_lo = hd.y & 0x3F3F3F3Fu, mn_lo = hd.z & 0x3F3F3F3Fu;
        const uint32_t sc_hi = (hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u);
        const uint32_t mn_hi = ((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u);
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const uint32_t scw = p < 2 ? sc_lo : sc_hi, mnw = p < 2 ? mn_lo : mn_hi;
            const int byte = 2 * (p & 1) + hf;
            sD[p] = d * (float)((scw >> (8 * byte)) & 0xFFu);
            sM[p] = -(dmin * (float)((mnw >> (8 * byte)) & 0xFFu));
        }
    };
    u32x2 rqs;
    auto qs_read = [&](int p, int sb) {
        rqs = *reinterpret_cast<const u32x2*>(ring + (sb % G::kRS) * kQ4sStage + brow * kQ4KBytes + 16 + 32 * p +
                                               16 * (ks & 1) + 8 * h);
    };
    u32x4 bq[2];                          // [chunk parity]
    auto b_dequant = [&](int p, int P) {
        // hdr_read folded 2^24 (low nibbles) or 2^20 (high: 16 q) into d
        const uint2 a = f16a_dq4(rqs.x, nmask, sD[p], sM[p]);
        const uint2 b = f16a_dq4(rqs.y, nmask, sD[p], sM[p]);
        bq[P] = u32x4{a.x, a.y, b.x, b.y};
    };

    f32x16 acc[FMR];
#pragma unroll
    for (int i = 0; i < FMR; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][e] = 0.0f;

    const int gcol = (col & 7) ^ ((col >> 3) & 1);
    f16x8 af[2][FMR];
    auto frag_ld = [&](int set, int buf, int i) {
        af[set][i] = *reinterpret_cast<const f16x8*>(abuf0 + buf * G::kABuf + (32 * i + col) * 128 +
                                                     16 * ((2 * ks + h) ^ gcol));
    };

    // ---- prologue: ring stages 0 .. kRS - 2; A chunks 0 .. kABufs - 2;
    // chunk 0's operands --------------------------------------------------------
#pragma unroll
    for (int st = 0; st < G::kRS - 1; ++st)
#pragma unroll
        for (int t = 0; t < 2; ++t) w_dma1(t, st, st);
#pragma unroll
    for (int c = 0; c < G::kABufs - 1; ++c)
#pragma unroll
        for (int g = 0; g < G::kAPW; ++g) a_dma1(g, c, c);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    lds_barrier();
    hdr_read(0);
    qs_read(0, 0);
    b_dequant(0, 0);
#pragma unroll
    for (int i = 0; i < FMR; ++i) frag_ld(0, 0, i);

    // Chunk c = 4 sb + CQ: A buffer c % kABufs, ring stage sb % kRS.  After
    // the first MFMA every LDS read of chunk c + 1 (its fragments, qs bytes
    // and, entering a new super-block, its header); the A DMA of chunk
    // c + kABufs - 1; in CQ 0 the ring DMA of super-block sb + kRS - 1; the B
    // operands of chunk c + 1 after the last MFMA.  At the end every DMA
    // issued up to chunk c - kLag is complete (the ring DMA of chunk 4 sb
    // counted among the last kLag chunks' DMAs), then one barrier.  A ring
    // stage is first read in the last chunk of the super-block before it:
    // with kRS = 3 its DMA (chunk 4 sb) lands by the end of 4 sb + 4, before
    // the read in 4 sb + 7; with kRS = 2 by the end of 4 sb + 1, before the
    // read in 4 sb + 3.
    int ab = 0;
    auto iteration = [&](auto cqc, int sb) {
        constexpr int CQ = decltype(cqc)::value;
        constexpr int P = CQ & 1;
        constexpr int NQ = (CQ + 1) & 3;
        constexpr int kOut = ksplit_dma_out(CQ, G::kAPW, 2, G::kLag, G::kRS);
        const int c = 4 * sb + CQ;
        const int sbn = CQ == 3 ? sb + 1 : sb;
        const int abn = ab == G::kABufs - 1 ? 0 : ab + 1;
        const int abp = ab == 0 ? G::kABufs - 1 : ab - 1;
#pragma unroll
        for (int i = 0; i < FMR; ++i) {
            acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[P][i], __builtin_bit_cast(f16x8, bq[P]), acc[i], 0, 0,
                                                            0);
            if (i == 0) {
                if constexpr (NQ == 0) hdr_read(sbn);
                qs_read(NQ, sbn);
#pragma unroll
                for (int r = 0; r < FMR; ++r) frag_ld(P ^ 1, abn, r);
            }
            if (i < G::kAPW) a_dma1(i, c + G::kABufs - 1, abp);
            if constexpr (CQ == 0) {
                if (i < 2) w_dma1(i, sb + G::kRS - 1, (sb + G::kRS - 1) % G::kRS);
            }
            if (i == FMR - 1) b_dequant(NQ, P ^ 1);
            __builtin_amdgcn_sched_barrier(0);
        }
        asm volatile("s_waitcnt vmcnt(%0)" :: "n"(kOut) : "memory");
        lds_barrier();
        ab = abn;
    };
    for (int sb = 0; sb < nsb; ++sb) {
        iteration(std::integral_constant<int, 0>{}, sb);
        iteration(std::integral_constant<int, 1>{}, sb);
        iteration(std::integral_constant<int, 2>{}, sb);
        iteration(std::integral_constant<int, 3>{}, sb);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    // ---- K slices, in rounds of kXB row blocks: every wave parks the round's
    // blocks in LDS ([wave][block][e / 4][lane] of float4); wave (ks, cg),
    // ks < kXB, adds block kXB rd + ks of column group cg over ks' = 0..3 in
    // that order (acc indexed by compile-time constants: the round loop is
    // unrolled) --------------------------------------------------------------
    float4* xch = reinterpret_cast<float4*>(lds);
    const int ncol = n0 + 32 * cg + col;
#pragma unroll
    for (int rd = 0; rd < G::kRounds; ++rd) {
        __syncthreads();
#pragma unroll
        for (int i = 0; i < G::kXB; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                xch[((wave * G::kXB + i) * 4 + q) * 64 + lane] =
                    make_float4(acc[G::kXB * rd + i][4 * q], acc[G::kXB * rd + i][4 * q + 1],
                                acc[G::kXB * rd + i][4 * q + 2], acc[G::kXB * rd + i][4 * q + 3]);
        __syncthreads();
        if (ks < G::kXB) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float s4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int src = 0; src < 4; ++src) {
                    const float4 p = xch[(((4 * cg + src) * G::kXB + ks) * 4 + q) * 64 + lane];
                    s4[0] += p.x;
                    s4[1] += p.y;
                    s4[2] += p.z;
                    s4[3] += p.w;
                }
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int row = m0 + 32 * (G::kXB * rd + ks) + 8 * q + 4 * h + u;
                    if (row < M) {
                        const size_t e = (size_t)row * N + ncol;
                        if (!ACC && gate != nullptr) {   // up projection of a SwiGLU: fp16 silu(gate) * up
                            const float gg = gate[e];
                            reinterpret_cast<uint16_t*>(D)[e] = f16_bits_rn(gg / (1.0f + expf(-gg)) * s4[u]);
                        } else {
                            float* o = D + e;
                            *o = ACC ? *o + s4[u] : s4[u];
                        }
                    }
                }
            }
        }
    }
}

template <int FMR, bool ACC>
__global__ __launch_bounds__(kQ4sThreads) void rf_gemm_q4k_f16s_kernel(const uint16_t* __restrict__ A,
                                                                        const uint8_t* __restrict__ W,
                                                                        float* __restrict__ D, int M, int N, int K,
                                                                        const float* __restrict__ G, KSplit sp) {
    __shared__ __align__(16) uint8_t lds[Q4sGeom<FMR>::kLds];
    q4s_wg<FMR, ACC>(A, W, D, M, N, K, xcd_remap((int)blockIdx.x, (int)gridDim.x), lds, G, sp);
}

// Column segments on fp16 activations: up to three weight matrices (each
// Q4_K or Q6_K) over one input, each with its own output, in one launch of
// 128 x 64 tiles -- the K-sliced Q4_K tiles (q4s_wg) and the Q6_K tiles
// (q6a_wg) share the tile shape, the 512 threads and the LDS size.  Tile v
// (after the XCD remap) belongs to the segment whose tile range holds it;
// each output is written once (no K split).
struct F16Segs {
    const uint8_t* w[3];
    float* d[3];
    int n[3];
    int q6[3];         // 1: Q6_K on the launch's tiles; 2: Q6_K on 128-row tiles in a 256-row launch
    int tiles[3];      // M tiles x column tiles of each segment
};
static_assert(kQ6aBN == kQ4sBN && kQ6aThreads == kQ4sThreads, "q6a and q4s tiles differ");
template <int FMR>
struct F16SegGeom {
    static constexpr int kLds = Q6aGeom<FMR>::kLds > Q4sGeom<FMR>::kLds ? Q6aGeom<FMR>::kLds : Q4sGeom<FMR>::kLds;
};

// FMR = 4 (128-row tiles) or 8 (256-row tiles, each weight dequantised once
// per 256 rows of A; a Q6_K segment of such a launch runs 128-row tiles)
template <int FMR>
__global__ __launch_bounds__(kQ4sThreads) void rf_gemm_f16_segs_kernel(const uint16_t* __restrict__ A, int M, int K,
                                                                        F16Segs sg) {
    __shared__ __align__(16) uint8_t lds[F16SegGeom<FMR>::kLds];
    int v = xcd_remap((int)blockIdx.x, (int)gridDim.x);
    // segment selection by selects (no runtime index into the argument)
    const int s = v < sg.tiles[0] ? 0 : (v < sg.tiles[0] + sg.tiles[1] ? 1 : 2);
    v -= s == 0 ? 0 : (s == 1 ? sg.tiles[0] : sg.tiles[0] + sg.tiles[1]);
    const uint8_t* w = s == 0 ? sg.w[0] : (s == 1 ? sg.w[1] : sg.w[2]);
    float* d = s == 0 ? sg.d[0] : (s == 1 ? sg.d[1] : sg.d[2]);
    const int n = s == 0 ? sg.n[0] : (s == 1 ? sg.n[1] : sg.n[2]);
    const int q6 = s == 0 ? sg.q6[0] : (s == 1 ? sg.q6[1] : sg.q6[2]);
    static_assert(Q6aGeom<4>::kLds <= F16SegGeom<8>::kLds, "128-row Q6_K tiles fit the 256-row launch's LDS");
    if (FMR == 8 && q6 == 2)
        q6a_wg<false, 4>(A, w, d, M, n, K, v, lds);
    else if (q6)
        q6a_wg<false, FMR>(A, w, d, M, n, K, v, lds);
    else
        q4s_wg<FMR, false>(A, w, d, M, n, K, v, lds);
}

static GemmSegs single_seg(int N) {
    GemmSegs g{};
    g.n1 = g.n2 = N;
    return g;
}

// The fp32-activation ring / register-weight kernels, one workgroup per
// tile and no K split: every output is written once, after its whole sum.
template <bool IS_Q6, int FM>
static void launch_v4(const float* A, const uint8_t* w, float* D, int M, int N, int K, hipStream_t st,
                      const GemmSegs& sg) {
    // column segments, accumulation and gate/up pairs exist only in v7
    const bool plain = sg.n1 == N && sg.n2 == N && !sg.accum && !sg.pair;
    using T = typename std::conditional<IS_Q6, Q6Ops, Q4Ops>::type;
    const int tiles = (M / (32 * FM)) * (N / 256);
    const int nchunks = K / kKC;
    // v7 (LDS weight ring); Q6_K needs 16-byte aligned rows (K % 2048 == 0) for the ring
    const bool v7 = !plain || !IS_Q6 || K % 2048 == 0;
    if (v7)
        hipLaunchKernelGGL((rf_gemm_qk_v7_kernel<T, IS_Q6, FM>), dim3(tiles), dim3(kV7Threads), 0, st, A, w,
                           D, M, N, K, tiles, nchunks, kGemmBand, sg);
    else
        hipLaunchKernelGGL((rf_gemm_qk_v4_kernel<T, FM>), dim3(tiles), dim3(kV4Threads), 0, st, A, w, D, M,
                           N, K, tiles, nchunks);
}

// Shared-dequantisation tiles without a K split; the caller checks that
// they fill the CUs (split-K adds float atomics on M x N outputs, which cost
// more than the tile shape saves).
template <bool IS_Q6, int BM, int BN>
static void launch_sq(const float* A, const uint8_t* w, float* D, int M, int N, int K, hipStream_t st, int accum) {
    const int tiles = (M / BM) * (N / BN);
    hipLaunchKernelGGL((rf_gemm_qk_sq_kernel<IS_Q6, BM, BN>), dim3(tiles), dim3(kSqThreads), 0, st, A, w, D, M, N, K,
                       accum);
}

// sg routes column segments / accumulation (v7 and sq only: the callers of
// a non-trivial sg have checked N % 256 == 0, K % 512 == 0 and, for Q6_K,
// K % 2048 == 0, and segments never reach sq)
template <bool IS_Q6>
static hipError_t launch_gemm(const float* A, const void* W, float* D, int M, int N, int K, hipStream_t st,
                              const GemmSegs& sg) {
    const uint8_t* w = static_cast<const uint8_t*>(W);
    if (N % 256 == 0 && K % 512 == 0) {
        // shared-dequantisation tiles where they come to about one
        // workgroup per CU without a K split: 256 x 256 (M >= 1024 at the
        // Llama FFN shapes, 10 % faster than v7), else 128 x 128 at up to
        // 9/8 workgroups per CU (M = 256: 59.4 vs 63.0 us; with more tiles
        // -- M = 512 -- v7 is faster: 78.6 vs 94.6 us)
        const long cus = device_cu_count();
        const long sq_tiles = (long)(M / 256) * (N / 256);
        const long sq128_tiles = (long)(M / 128) * (N / 128);
        const bool sq_ok = sg.n1 == N && sg.n2 == N && !sg.pair;
        if (sq_ok && M % 256 == 0 && 8 * sq_tiles >= 7 * cus)
            launch_sq<IS_Q6, 256, 256>(A, w, D, M, N, K, st, sg.accum);
        else if (sq_ok && M % 128 == 0 && 8 * sq128_tiles >= 7 * cus && 8 * sq128_tiles <= 9 * cus)
            launch_sq<IS_Q6, 128, 128>(A, w, D, M, N, K, st, sg.accum);
        // 128-row tiles where they come to at least 7/8 of the CUs, or fit
        // in one round of CUs where 64-row tiles would take two (M = 512 at
        // N = 12288: 192 vs 384 tiles on 256 CUs), and always for Q6_K
        // (its heavier dequantisation favours fewer, taller tiles); else
        // 64-row tiles
        else if (M % 128 == 0 && (IS_Q6 || 8L * (M / 128) * (N / 256) >= 7L * cus ||
                                  (2L * (M / 128) * (N / 256) > cus && (long)(M / 128) * (N / 256) <= cus)))
            launch_v4<IS_Q6, 4>(A, w, D, M, N, K, st, sg);
        else
            launch_v4<IS_Q6, 2>(A, w, D, M, N, K, st, sg);
        return hipGetLastError();
    }
    if (M % 128 == 0 && N % 128 == 0 && (size_t)(M / 128) * (N / 128) >= (size_t)device_cu_count()) {
        hipLaunchKernelGGL((rf_gemm_qk_kernel<IS_Q6, 128, 128>), dim3(N / 128, M / 128), dim3(kGemmThreads), 0, st,
                           A, w, D, M, N, K);
    } else {
        hipLaunchKernelGGL((rf_gemm_qk_kernel<IS_Q6, 64, 64>), dim3(N / 64, M / 64), dim3(kGemmThreads), 0, st, A,
                           w, D, M, N, K);
    }
    return hipGetLastError();
}

// ── fp16 staging of fp32 activations, deterministic K split ──────────────
// The fp32-activation launchers round A to fp16 exactly as the reference
// does (__float2half, wmma_gemm_q4_k.hip:86) in a pass of their own, into
// library-owned device memory, and then run the fp16-activation tiles: the
// operand values are the same, and the tiles read half the bytes of A.  Small
// launches split K over workgroups; the partial tiles land in the same
// memory and one more pass adds them in split order, so every output is the
// same sum on every run (no float atomics anywhere).

// Adds the S partial tiles (part + s * n, s = 0 .. S - 1, n = n4 * 4 floats)
// in split order and stores the sum (MODE 0), adds it to D (MODE 1: D + sum),
// or stores fp16 silu(gate) * sum into D read as halves (MODE 2), the
// epilogues of the unsplit tiles.  All pointers 16-byte aligned.
template <int MODE>
__global__ __launch_bounds__(256) void rf_gemm_split_reduce_kernel(const float4* __restrict__ part, int S, size_t n4,
                                                                    float* __restrict__ D,
                                                                    const float4* __restrict__ gate) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (size_t)gridDim.x * blockDim.x) {
        float4 t = part[i];
        for (int k = 1; k < S; ++k) {
            const float4 p = part[(size_t)k * n4 + i];
            t.x += p.x;
            t.y += p.y;
            t.z += p.z;
            t.w += p.w;
        }
        if constexpr (MODE == 0) {
            reinterpret_cast<float4*>(D)[i] = t;
        } else if constexpr (MODE == 1) {
            float4 d = reinterpret_cast<float4*>(D)[i];
            d.x = d.x + t.x;
            d.y = d.y + t.y;
            d.z = d.z + t.z;
            d.w = d.w + t.w;
            reinterpret_cast<float4*>(D)[i] = d;
        } else {
            const float4 g = gate[i];
            const float r0 = g.x / (1.0f + expf(-g.x)) * t.x, r1 = g.y / (1.0f + expf(-g.y)) * t.y;
            const float r2 = g.z / (1.0f + expf(-g.z)) * t.z, r3 = g.w / (1.0f + expf(-g.w)) * t.w;
            reinterpret_cast<uint2*>(D)[i] =
                make_uint2((uint32_t)f16_bits_rn(r0) | ((uint32_t)f16_bits_rn(r1) << 16),
                           (uint32_t)f16_bits_rn(r2) | ((uint32_t)f16_bits_rn(r3) << 16));
        }
    }
}

// out[i] = fp16(a[i]) (round to nearest even, the value of __float2half) for
// n4 * 4 elements; both 16-byte aligned.
__global__ __launch_bounds__(256) void rf_f32_to_f16_kernel(const float4* __restrict__ a, uint2* __restrict__ out,
                                                             size_t n4) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (size_t)gridDim.x * blockDim.x) {
        const float4 v = a[i];
        out[i] = make_uint2(cvt_pk_f16(v.x, v.y), cvt_pk_f16(v.z, v.w));
    }
}

static unsigned stream_grid(size_t n4) { return (unsigned)std::min<size_t>((n4 + 255) / 256, 4096); }

// Library-owned scratch: kGemmSlots slots per GPU in a file-scope device
// array (allocated when the library's code object loads on that GPU, held
// until the process ends; the launchers never allocate).  A slot serves one
// stream at a time: on the fp32-activation launchers its first bytes hold
// the fp16 copy of A (up to kSlotABytes) and the K-split partials follow it;
// on the fp16-activation launchers the whole slot takes partials.  Launches on one stream are ordered, so they share
// its slot safely.  A stream without a slot takes a free one, else (outside
// stream capture) one whose stream is idle (hipStreamQuery: a host-side
// query, nothing enqueued), else runs the unstaged fp32 kernels.  A slot
// claimed under stream capture stays with the capturing stream (the graph
// holds its address; replaying that graph concurrently with other GEMM work
// of the same stream races), and so does the slot of a stream that has been
// destroyed.  The hand-over assumes one host thread launching on a GPU at a
// time (the reference's contract): a slot taken from an idle stream whose
// own thread is between claiming and enqueuing would be shared.  In host
// code the array's name is only a stand-in; its device address is taken
// once per GPU with hipGetSymbolAddress.
constexpr int kGemmSlots = 4;
constexpr size_t kSlotABytes = (size_t)32 << 20;
constexpr size_t kSlotPartBytes = (size_t)24 << 20;
constexpr size_t kSlotBytes = kSlotABytes + kSlotPartBytes;
static __device__ __align__(256) uint8_t gemm_scratch[kGemmSlots * kSlotBytes];
constexpr int kGemmMaxDevices = 64;

struct GemmSlot {
    uint16_t* a;        // the slot's kSlotBytes
};

// Room for K-split partials: the whole slot on the fp16-activation
// launchers, the part after the staged rows of A on the fp32 ones (at least
// kSlotPartBytes).
struct PartBuf {
    float* p;
    size_t bytes;
};
static PartBuf slot_parts(const GemmSlot& slot, size_t a_bytes) {
    const size_t off = (a_bytes + 255) & ~(size_t)255;
    return PartBuf{reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(slot.a) + off), kSlotBytes - off};
}

struct SlotState {
    hipStream_t owner;
    bool taken;
    bool captured;      // claimed under stream capture: never handed on
};
static std::mutex g_slot_mutex;
static uint8_t* g_slot_base[kGemmMaxDevices];
static SlotState g_slots[kGemmMaxDevices][kGemmSlots];

// The slot of `st` on the current device: its own, a free one, or (outside
// stream capture, where stream queries are not allowed) one whose stream is
// idle; false when none is available.
static bool gemm_slot(hipStream_t st, GemmSlot* out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kGemmMaxDevices) return false;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    const bool capturing = hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone;
    std::lock_guard<std::mutex> lock(g_slot_mutex);
    if (g_slot_base[dev] == nullptr) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(gemm_scratch)) != hipSuccess || p == nullptr) return false;
        g_slot_base[dev] = static_cast<uint8_t*>(p);
    }
    SlotState* sl = g_slots[dev];
    int k = -1;
    for (int i = 0; i < kGemmSlots && k < 0; ++i)
        if (sl[i].taken && sl[i].owner == st) k = i;
    for (int i = 0; i < kGemmSlots && k < 0; ++i)
        if (!sl[i].taken) k = i;
    for (int i = 0; i < kGemmSlots && k < 0 && !capturing; ++i)
        if (!sl[i].captured && hipStreamQuery(sl[i].owner) == hipSuccess) k = i;
    if (k < 0) return false;
    sl[k].taken = true;
    sl[k].owner = st;
    sl[k].captured = sl[k].captured || capturing;
    uint8_t* b = g_slot_base[dev] + (size_t)k * kSlotBytes;
    out->a = reinterpret_cast<uint16_t*>(b);
    return true;
}

// K split for `tiles` workgroups over nsb super-blocks per row, `per_cu`
// of which fit a CU at once: the largest S <= 8 with tiles * S <= per_cu
// CUs whose M x N partials fit part (part.p == nullptr: no split).
static int ksplit_count(long tiles, int nsb, int M, int N, const PartBuf& part, int per_cu = 1) {
    if (part.p == nullptr) return 1;
    const long cap = (long)per_cu * device_cu_count();
    int S = 1;
    for (int s = 2; s <= 8 && s <= nsb; ++s)
        if (tiles * s <= cap && (size_t)s * M * N * sizeof(float) <= part.bytes) S = s;
    return S;
}

// The split reduction into the residual stream with the RMSNorm of the
// result in the same pass (the next layer's input norm of a prefill): one
// workgroup per row of N = 2048 NG.  Row r: h = D + (p_0 + .. + p_{S-1}) in
// rf_gemm_split_reduce_kernel<1>'s order, stored to D; thread t holds the
// elements 8 t + 2048 g .. + 7 (g < NG) and takes their squares in
// rms_inv_canonical's order, so out = fp16((h * inv) * w) has the bits of
// rf_rms_norm_batched_f16_on_stream run on the stored h.
template <int NG>
__global__ __launch_bounds__(256) void rf_split_reduce_rmsnorm_kernel(const float* __restrict__ part, int S, int M,
                                                                      int N, float* __restrict__ D,
                                                                      const float* __restrict__ w, float eps,
                                                                      uint16_t* __restrict__ out) {
    __shared__ float red[4];
    const int r = blockIdx.x;
    const size_t mn = (size_t)M * N;
    const size_t row = (size_t)r * N;
    float4 h[NG][2];
#pragma unroll
    for (int g = 0; g < NG; ++g)
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const size_t e = row + 8 * threadIdx.x + 2048 * g + 4 * q;
            float4 t = *reinterpret_cast<const float4*>(part + e);
            for (int k = 1; k < S; ++k) {
                const float4 p = *reinterpret_cast<const float4*>(part + (size_t)k * mn + e);
                t.x += p.x;
                t.y += p.y;
                t.z += p.z;
                t.w += p.w;
            }
            float4 d = *reinterpret_cast<const float4*>(D + e);
            d.x = d.x + t.x;
            d.y = d.y + t.y;
            d.z = d.z + t.z;
            d.w = d.w + t.w;
            *reinterpret_cast<float4*>(D + e) = d;
            h[g][q] = d;
        }
    float ss = 0.0f;
#pragma unroll
    for (int g = 0; g < NG; ++g) ss += sq8(h[g][0], h[g][1]);
    ss = xor_sum64(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    const float inv = rms_inv_finish(red, N, eps);
#pragma unroll
    for (int g = 0; g < NG; ++g)
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int c = 8 * threadIdx.x + 2048 * g + 4 * q;
            const float4 a = h[g][q];
            const float4 gw = *reinterpret_cast<const float4*>(w + c);
            const uint32_t lo =
                (uint32_t)f16_bits_rn((a.x * inv) * gw.x) | ((uint32_t)f16_bits_rn((a.y * inv) * gw.y) << 16);
            const uint32_t hi =
                (uint32_t)f16_bits_rn((a.z * inv) * gw.z) | ((uint32_t)f16_bits_rn((a.w * inv) * gw.w) << 16);
            *reinterpret_cast<uint2*>(out + row + c) = make_uint2(lo, hi);
        }
}

// An RMSNorm of the accumulated rows (weights w, fp16 output) that a split
// reduction may fold in; fused is set when it did.
struct RowNorm {
    const float* w;
    float eps;
    uint16_t* out;
    bool* fused;
    bool fits(int N) const { return N % 2048 == 0 && N <= 8192; }
};

template <int MODE>
static void launch_reduce(const float* part, int S, int M, int N, float* D, const float* G, hipStream_t st) {
    const size_t n4 = (size_t)M * N / 4;
    hipLaunchKernelGGL(rf_gemm_split_reduce_kernel<MODE>, dim3(stream_grid(n4)), dim3(256), 0, st,
                       reinterpret_cast<const float4*>(part), S, n4, D, reinterpret_cast<const float4*>(G));
}

static void reduce_for(bool acc, const float* G, const float* part, int S, int M, int N, float* D, hipStream_t st,
                       const RowNorm* rn = nullptr) {
    if (acc && rn != nullptr && rn->fits(N)) {
        auto go = [&](auto ngc) {
            hipLaunchKernelGGL((rf_split_reduce_rmsnorm_kernel<decltype(ngc)::value>), dim3((unsigned)M), dim3(256), 0,
                               st, part, S, M, N, D, rn->w, rn->eps, rn->out);
        };
        switch (N / 2048) {
        case 1: go(std::integral_constant<int, 1>{}); break;
        case 2: go(std::integral_constant<int, 2>{}); break;
        case 3: go(std::integral_constant<int, 3>{}); break;
        default: go(std::integral_constant<int, 4>{}); break;
        }
        *rn->fused = true;
    } else if (acc)
        launch_reduce<1>(part, S, M, N, D, nullptr, st);
    else if (G != nullptr)
        launch_reduce<2>(part, S, M, N, D, G, st);
    else
        launch_reduce<0>(part, S, M, N, D, nullptr, st);
}

// Q4_K on fp16 activations: 256 x 128 tiles (rf_gemm_q4k_f16a_kernel) where
// they fill at least three quarters of the CUs, else the eight-wave
// K-sliced tiles (rf_gemm_q4k_f16s_kernel) of 256 rows (from M =
// kQ4TallMinM: each weight dequantised once per 256 rows), 64 rows (M <= 64,
// or when they come to at most one round of CUs) or 128, split over K when
// they leave at least half the CUs idle and `part` is given.
// G: when given, D receives fp16 silu(G) * (A W^T) (the up projection of a
// SwiGLU whose gate product G [M x N] is already computed)
#ifndef RF_Q4_TALL_MIN_M
#define RF_Q4_TALL_MIN_M 256
#endif
constexpr int kQ4TallMinM = RF_Q4_TALL_MIN_M;


template <bool ACC, int FMR>
static void q4_f16_tiles(const uint16_t* A, const uint8_t* w, float* D, int M, int N, int K, hipStream_t st,
                         const float* G, const PartBuf& part, const RowNorm* rn = nullptr) {
    const long tiles = (long)((M + 32 * FMR - 1) / (32 * FMR)) * (N / kQ4sBN);
    const int S = 2 * tiles <= (long)device_cu_count() ? ksplit_count(tiles, K / kQK, M, N, part) : 1;
    if (S > 1) {
        hipLaunchKernelGGL((rf_gemm_q4k_f16s_kernel<FMR, false>), dim3((unsigned)(tiles * S)), dim3(kQ4sThreads), 0,
                           st, A, w, nullptr, M, N, K, nullptr, KSplit{S, part.p});
        reduce_for(ACC, G, part.p, S, M, N, D, st, rn);
    } else {
        hipLaunchKernelGGL((rf_gemm_q4k_f16s_kernel<FMR, ACC>), dim3((unsigned)tiles), dim3(kQ4sThreads), 0, st, A, w,
                           D, M, N, K, G, KSplit{1, nullptr});
    }
}

// rn (ACC only): an RMSNorm of the accumulated rows the split reduction
// may fold in (the caller runs it itself when rn->fused stays false).
template <bool ACC>
static hipError_t gemm_q4_f16(const uint16_t* A, const void* W, float* D, int M, int N, int K, hipStream_t st,
                              const float* G, const PartBuf& part, const RowNorm* rn = nullptr) {
    const uint8_t* w = static_cast<const uint8_t*>(W);
    const long big = (long)((M + kF16aBM - 1) / kF16aBM) * (N % kF16aBN == 0 ? N / kF16aBN : 0);
    if (!ACC && 4 * big >= 3L * device_cu_count()) {
        if (G != nullptr)
            hipLaunchKernelGGL(rf_gemm_q4k_f16a_kernel<3>, dim3((unsigned)big), dim3(kF16aThreads), 0, st, A, w, w, D,
                               M, N, K, G, KSplit{1, nullptr});
        else
            hipLaunchKernelGGL(rf_gemm_q4k_f16a_kernel<0>, dim3((unsigned)big), dim3(kF16aThreads), 0, st, A, w, w, D,
                               M, N, K, nullptr, KSplit{1, nullptr});
        return hipGetLastError();
    }
    if (M >= kQ4TallMinM && big > 0) {
        // 256 x 128 tiles split over K where the split brings them to at
        // least three quarters of the CUs and leaves each split >= 12
        // super-blocks (measured on MI355X, fp16 A: 4096 x 12288 at M = 512
        // split in 4, 60.9 against 68.3 us for the 256 x 64 tiles split in
        // 2; with 8 super-blocks per split, 14336 x 4096 at M = 256, 45.0
        // against 43.5; with 4, 4096 x 4096 at M = 512, 34.8 against 27.9)
        const long cus = device_cu_count();
        const int nsb = K / kQK;
        const int S = ksplit_count(big, nsb, M, N, part);
        if (S > 1 && 4 * big * S >= 3 * cus && nsb / S >= 12) {
            hipLaunchKernelGGL(rf_gemm_q4k_f16a_kernel<0>, dim3((unsigned)(big * S)), dim3(kF16aThreads), 0, st, A, w,
                               w, nullptr, M, N, K, nullptr, KSplit{S, part.p});
            reduce_for(ACC, G, part.p, S, M, N, D, st, rn);
            return hipGetLastError();
        }
    }
    if (M >= kQ4TallMinM) {
        // 256-row tiles where they fill 3/4 of the CUs unsplit, or where their
        // K split leaves each workgroup at least 24 super-blocks (measured on
        // MI355X: 14336 x 4096 at M = 256 43.3 against 53.1 us, 4096 x 12288
        // at M = 512 68.3 against 72.2; but 4096 x 4096 at M = 512, split in
        // two, 33.2 against 27.9 for 128-row tiles)
        const long cus = device_cu_count();
        const long t8 = (long)((M + 255) / 256) * (N / kQ4sBN);
        const int s8 = 2 * t8 <= cus ? ksplit_count(t8, K / kQK, M, N, part) : 1;
        if (4 * t8 >= 3 * cus || (s8 > 1 && (K / kQK) / s8 >= 24)) {
            q4_f16_tiles<ACC, 8>(A, w, D, M, N, K, st, G, part, rn);
            return hipGetLastError();
        }
    }
    // 64-row K-sliced tiles also when twice as many of them still fit one
    // round of CUs (measured on MI355X, N = 4096: M = 256 22.3 against 24.7 us
    // at K = 4096, 58.4 against 63.1 at K = 12288)
    const bool rows64 = M <= 64 || 2L * ((M + 127) / 128) * (N / kQ4sBN) <= (long)device_cu_count();
    if (rows64)
        q4_f16_tiles<ACC, 2>(A, w, D, M, N, K, st, G, part, rn);
    else
        q4_f16_tiles<ACC, 4>(A, w, D, M, N, K, st, G, part, rn);
    return hipGetLastError();
}

// Q6_K on fp16 activations (rf_gemm_q6k_f16a_kernel): 256 x 64 tiles from
// M = kQ6TallMinM rows (each weight dequantised once per 256 rows), else
// 128 x 64, split over K as gemm_q4_f16 does.  The caller has checked
// M % 64, N % 64, K % 2048 and 16-byte alignment of A and W.
#ifndef RF_Q6_TALL_MIN_M
#define RF_Q6_TALL_MIN_M 256
#endif
constexpr int kQ6TallMinM = RF_Q6_TALL_MIN_M;
constexpr int kQ6LeanMaxM = 64;      // 64-row tiles up to this M (at M = 128: 40.0 against 33.0 us)

template <bool ACC, int FMR>
static void q6_f16_tiles(const uint16_t* A, const uint8_t* w, float* D, int M, int N, int K, hipStream_t st,
                         const PartBuf& part, const RowNorm* rn = nullptr) {
    const long tiles = (long)((M + 32 * FMR - 1) / (32 * FMR)) * (N / kQ6aBN);
    const int per_cu = FMR == 2 ? 2 : 1;      // the lean 64-row tiles: two workgroups per CU
    const int S = 2 * tiles <= (long)per_cu * device_cu_count() ? ksplit_count(tiles, K / kQK, M, N, part, per_cu)
                                                                  : 1;
    if (S > 1) {
        hipLaunchKernelGGL((rf_gemm_q6k_f16a_kernel<false, FMR>), dim3((unsigned)(tiles * S)), dim3(kQ6aThreads), 0,
                           st, A, w, nullptr, M, N, K, KSplit{S, part.p});
        reduce_for(ACC, nullptr, part.p, S, M, N, D, st, rn);
    } else {
        hipLaunchKernelGGL((rf_gemm_q6k_f16a_kernel<ACC, FMR>), dim3((unsigned)tiles), dim3(kQ6aThreads), 0, st, A, w,
                           D, M, N, K, KSplit{1, nullptr});
    }
}

template <bool ACC>
static hipError_t gemm_q6_f16(const uint16_t* A, const void* W, float* D, int M, int N, int K, hipStream_t st,
                              const PartBuf& part, const RowNorm* rn = nullptr) {
    const uint8_t* w = static_cast<const uint8_t*>(W);
    if (M >= kQ6TallMinM)
        q6_f16_tiles<ACC, 8>(A, w, D, M, N, K, st, part, rn);
    else if (M <= kQ6LeanMaxM)
        q6_f16_tiles<ACC, 2>(A, w, D, M, N, K, st, part, rn);
    else
        q6_f16_tiles<ACC, 4>(A, w, D, M, N, K, st, part, rn);
    return hipGetLastError();
}

// Stages A (fp32, M x K, 16-byte aligned) as fp16 in the slot, in runs of
// whole 64-row blocks that fit kSlotABytes, and calls fn(a16, m0, rows) for
// each run in order (stream-ordered: a run's conversion waits for the
// previous run's GEMM).  The caller has checked that 64 rows fit.
template <class F>
static hipError_t staged_rows(const float* A, int M, int K, const GemmSlot& slot, hipStream_t st, F&& fn) {
    const int run = (int)std::min<size_t>((size_t)M, kSlotABytes / ((size_t)K * 2) / 64 * 64);
    for (int m0 = 0; m0 < M; m0 += run) {
        const int rows = std::min(run, M - m0);
        const size_t n4 = (size_t)rows * K / 4;
        hipLaunchKernelGGL(rf_f32_to_f16_kernel, dim3(stream_grid(n4)), dim3(256), 0, st,
                           reinterpret_cast<const float4*>(A + (size_t)m0 * K), reinterpret_cast<uint2*>(slot.a), n4);
        const hipError_t e = fn(slot.a, m0, rows, slot_parts(slot, (size_t)rows * K * 2));
        if (e != hipSuccess) return e;
    }
    return hipGetLastError();
}

// The stream's slot when A (K fp16 per row) can be staged in runs of 64 rows.
static bool staging_slot(hipStream_t st, int K, GemmSlot* slot) {
    return (size_t)K * 2 * 64 <= kSlotABytes && gemm_slot(st, slot);
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Column segments on fp16 activations (rf_gemm_f16_segs_kernel): up to three
// weight matrices over one input, each Q4_K or Q6_K with its own output.
// The caller has checked the shapes and alignment.
#ifndef RF_SEG_TALL_MIN_M
#define RF_SEG_TALL_MIN_M 256
#endif
static hipError_t f16_segments(const uint16_t* A, const void* const ws[3], const int q6[3], float* const ds[3],
                               const int ns[3], int M, int K, hipStream_t st) {
    F16Segs sg{};
    // 256-row tiles from M = RF_SEG_TALL_MIN_M, else 128-row tiles (measured on
    // MI355X: the Qwen3-8B prefill of 512 tokens, Q/K/V of 4096 + 1024 + 1024
    // rows: 11.38 against 11.78 ms -- 192 tiles, one round of CUs, against 384)
    const bool tall = M >= RF_SEG_TALL_MIN_M;
    const int mtiles = tall ? (M + 255) / 256 : (M + 127) / 128;
    long total = 0;
    for (int i = 0; i < 3; ++i) {
        if (ns[i] == 0) continue;
        sg.w[i] = static_cast<const uint8_t*>(ws[i]);
        sg.d[i] = ds[i];
        sg.n[i] = ns[i];
        sg.q6[i] = q6[i];
        sg.tiles[i] = mtiles * (ns[i] / kQ4sBN);
        if (tall && q6[i]) {
            // a Q6_K segment on 128-row tiles: the 256-row Q6_K tiles take
            // longer than the Q4_K ones and set the launch's time (measured on
            // MI355X, Qwen3-8B Q/K/V with a Q6_K V: M = 512 42.5-44.8 against
            // 45.8-50.5 us, M = 256 36.8-37.7 against 41.7-42.2; same bits)
            sg.q6[i] = 2;
            sg.tiles[i] = ((M + 127) / 128) * (ns[i] / kQ4sBN);
        }
        total += sg.tiles[i];
    }
    if (total > 0x7FFFFFFFL) return hipErrorInvalidValue;
    if (tall)
        hipLaunchKernelGGL(rf_gemm_f16_segs_kernel<8>, dim3((unsigned)total), dim3(kQ4sThreads), 0, st, A, M, K, sg);
    else
        hipLaunchKernelGGL(rf_gemm_f16_segs_kernel<4>, dim3((unsigned)total), dim3(kQ4sThreads), 0, st, A, M, K, sg);
    return hipGetLastError();
}

}  // namespace rf

using namespace rf;

// Validation as wmma_gemm_q4_k.hip:207-210 / wmma_gemm_q6_k.hip:220-223,
// plus 16-byte alignment of A (read as float4) and of Q4_K weights.  A is
// staged as fp16 (the reference's own rounding of it) and the fp16 tiles
// run; with no slot for the stream, the fp32 tiles (no K split).
extern "C" hipError_t wmma_gemm_q4_k_launch(const float* input, const void* weights_q4_k, float* output, int M, int N,
                                            int K, hipStream_t stream) {
    if (M <= 0 || N <= 0 || K <= 0) return hipErrorInvalidValue;
    if ((M % 64) != 0 || (N % 64) != 0 || (K % kQK) != 0) return hipErrorInvalidValue;
    if (!aligned16(input) || !aligned16(weights_q4_k)) return hipErrorInvalidValue;
    GemmSlot slot;
    if (staging_slot(stream, K, &slot))
        return staged_rows(input, M, K, slot, stream, [&](const uint16_t* a16, int m0, int rows, const PartBuf& pb) {
            return gemm_q4_f16<false>(a16, weights_q4_k, output + (size_t)m0 * N, rows, N, K, stream, nullptr,
                                      pb);
        });
    return launch_gemm<false>(input, weights_q4_k, output, M, N, K, stream, single_seg(N));
}

extern "C" hipError_t wmma_gemm_q6_k_launch(const float* input, const void* weights_q6_k, float* output, int M, int N,
                                            int K, hipStream_t stream) {
    if (M <= 0 || N <= 0 || K <= 0) return hipErrorInvalidValue;
    if ((M % 64) != 0 || (N % 64) != 0 || (K % kQK) != 0) return hipErrorInvalidValue;
    if (!aligned16(input) || (reinterpret_cast<uintptr_t>(weights_q6_k) & 1u)) return hipErrorInvalidValue;
    GemmSlot slot;
    // the fp16 tiles read 16-byte aligned weight rows (K % 2048)
    if (K % 2048 == 0 && aligned16(weights_q6_k) && staging_slot(stream, K, &slot))
        return staged_rows(input, M, K, slot, stream, [&](const uint16_t* a16, int m0, int rows, const PartBuf& pb) {
            return gemm_q6_f16<false>(a16, weights_q6_k, output + (size_t)m0 * N, rows, N, K, stream, pb);
        });
    return launch_gemm<true>(input, weights_q6_k, output, M, N, K, stream, single_seg(N));
}

// fp16 activations (the caller's rounding of A, e.g. in the kernel that
// produced them): the same operand values as wmma_gemm_q4_k_launch on fp32
// A, read at half the bytes and without the conversion pass.  M % 64,
// N % 64, K % 256 (the 256 x 128 tiles only when N % 128 == 0); M need not
// fill the 256-row tiles.
extern "C" hipError_t rf_gemm_q4_k_f16_launch(const uint16_t* input_f16, const void* weights_q4_k, float* output,
                                              int M, int N, int K, hipStream_t stream) {
    if (input_f16 == nullptr || weights_q4_k == nullptr || output == nullptr) return hipErrorInvalidValue;
    if (M <= 0 || N <= 0 || K <= 0 || (M % 64) != 0 || (N % kQ4sBN) != 0 || (K % kQK) != 0)
        return hipErrorInvalidValue;
    if (!aligned16(input_f16) || !aligned16(weights_q4_k)) return hipErrorInvalidValue;
    GemmSlot slot;
    const PartBuf part = gemm_slot(stream, &slot) ? slot_parts(slot, 0) : PartBuf{nullptr, 0};
    return gemm_q4_f16<false>(input_f16, weights_q4_k, output, M, N, K, stream, nullptr, part);
}

// Gate and up on fp16 activations in one launch, SwiGLU in the epilogue
// (rf_gemm_q4k_f16a_kernel<1 or 2>: 256 x 128 tiles of 64 gate and the same
// 64 up rows): out[M x N] = silu(A Wg^T) * (A Wu^T), fp32 or rounded to fp16
// (out_f16), the values of rf_gemm_q4_k_f16_launch twice and
// rf_silu_mul(_f16)_on_stream.  M % 64, N % 64, K % 256; input and weights
// 16-byte aligned.
static hipError_t q4_f16_swiglu(const uint16_t* input_f16, const void* w_gate, const void* w_up, void* out,
                                int out_f16, int M, int N, int K, hipStream_t stream) {
    const unsigned tiles = (unsigned)(((M + kF16aBM - 1) / kF16aBM) * (N / 64));
    const uint8_t* wg = static_cast<const uint8_t*>(w_gate);
    const uint8_t* wu = static_cast<const uint8_t*>(w_up);
    if (out_f16)
        hipLaunchKernelGGL(rf_gemm_q4k_f16a_kernel<2>, dim3(tiles), dim3(kF16aThreads), 0, stream, input_f16, wg, wu,
                           static_cast<float*>(out), M, N, K, nullptr, KSplit{1, nullptr});
    else
        hipLaunchKernelGGL(rf_gemm_q4k_f16a_kernel<1>, dim3(tiles), dim3(kF16aThreads), 0, stream, input_f16, wg, wu,
                           static_cast<float*>(out), M, N, K, nullptr, KSplit{1, nullptr});
    return hipGetLastError();
}

extern "C" hipError_t rf_gemm_q4_k_f16_swiglu_launch(const uint16_t* input_f16, const void* w_gate, const void* w_up,
                                                     void* out, int out_f16, int M, int N, int K, hipStream_t stream) {
    if (input_f16 == nullptr || w_gate == nullptr || w_up == nullptr || out == nullptr) return hipErrorInvalidValue;
    if (M <= 0 || N <= 0 || K <= 0 || (M % 64) != 0 || (N % 64) != 0 || (K % kQK) != 0) return hipErrorInvalidValue;
    if (!aligned16(input_f16) || !aligned16(w_gate) || !aligned16(w_up)) return hipErrorInvalidValue;
    return q4_f16_swiglu(input_f16, w_gate, w_up, out, out_f16, M, N, K, stream);
}

// The up projection of a SwiGLU on fp16 activations, the gate product
// already computed: out_f16[M x N] = fp16(silu(gate) * (A Wu^T)), the values
// of rf_gemm_q4_k_f16_launch on w_up followed by rf_silu_mul_f16_on_stream
// (same tiles, the SwiGLU in their epilogue or in the split reduction).
// Shapes as rf_gemm_q4_k_f16_launch; gate [M x N] fp32, 16-byte aligned,
// must not overlap out_f16.
extern "C" hipError_t rf_gemm_q4_k_f16_swiglu_up_launch(const uint16_t* input_f16, const void* w_up,
                                                        const float* gate, uint16_t* out_f16, int M, int N, int K,
                                                        hipStream_t stream) {
    if (input_f16 == nullptr || w_up == nullptr || gate == nullptr || out_f16 == nullptr) return hipErrorInvalidValue;
    if (M <= 0 || N <= 0 || K <= 0 || (M % 64) != 0 || (N % kQ4sBN) != 0 || (K % kQK) != 0)
        return hipErrorInvalidValue;
    if (!aligned16(input_f16) || !aligned16(w_up) || !aligned16(gate) || !aligned16(out_f16))
        return hipErrorInvalidValue;
    const size_t n = (size_t)M * N;
    const uintptr_t g0 = reinterpret_cast<uintptr_t>(gate), o0 = reinterpret_cast<uintptr_t>(out_f16);
    if (g0 < o0 + 2 * n && o0 < g0 + 4 * n) return hipErrorInvalidValue;   // overlapping buffers
    GemmSlot slot;
    const PartBuf part = gemm_slot(stream, &slot) ? slot_parts(slot, 0) : PartBuf{nullptr, 0};
    return gemm_q4_f16<false>(input_f16, w_up, reinterpret_cast<float*>(out_f16), M, N, K, stream, gate, part);
}

// Q6_K on fp16 activations (rf_gemm_q6k_f16a_kernel): M % 64, N % 64,
// K % 2048 (weight rows 16-byte aligned); A and the weights 16-byte aligned.
template <bool ACC>
static hipError_t q6_f16_checked(const uint16_t* input_f16, const void* weights_q6_k, float* output, int M, int N,
                                 int K, hipStream_t stream) {
    if (input_f16 == nullptr || weights_q6_k == nullptr || output == nullptr) return hipErrorInvalidValue;
    if (M <= 0 || N <= 0 || K <= 0 || (M % 64) != 0 || (N % kQ6aBN) != 0 || (K % 2048) != 0)
        return hipErrorInvalidValue;
    if (!aligned16(input_f16) || !aligned16(weights_q6_k) || !aligned16(output)) return hipErrorInvalidValue;
    GemmSlot slot;
    const PartBuf part = gemm_slot(stream, &slot) ? slot_parts(slot, 0) : PartBuf{nullptr, 0};
    return gemm_q6_f16<ACC>(input_f16, weights_q6_k, output, M, N, K, stream, part);
}

extern "C" hipError_t rf_gemm_q6_k_f16_launch(const uint16_t* input_f16, const void* weights_q6_k, float* output,
                                              int M, int N, int K, hipStream_t stream) {
    return q6_f16_checked<false>(input_f16, weights_q6_k, output, M, N, K, stream);
}

// inout[M x N] += fp16(A) * fp16(dequant W)^T: each output read and written
// once, after its fp32 sum (reproducible bit for bit).
extern "C" hipError_t rf_gemm_q6_k_f16_accumulate_launch(const uint16_t* input_f16, const void* weights_q6_k,
                                                         float* inout, int M, int N, int K, hipStream_t stream) {
    return q6_f16_checked<true>(input_f16, weights_q6_k, inout, M, N, K, stream);
}

// inout[M x N] += the product of rf_gemm_q4_k_f16_launch, on the K-sliced
// tiles (each output read and written once after its fp32 sum).
extern "C" hipError_t rf_gemm_q4_k_f16_accumulate_launch(const uint16_t* input_f16, const void* weights_q4_k,
                                                         float* inout, int M, int N, int K, hipStream_t stream) {
    if (input_f16 == nullptr || weights_q4_k == nullptr || inout == nullptr) return hipErrorInvalidValue;
    if (M <= 0 || N <= 0 || K <= 0 || (M % 64) != 0 || (N % kQ4sBN) != 0 || (K % kQK) != 0)
        return hipErrorInvalidValue;
    if (!aligned16(input_f16) || !aligned16(weights_q4_k) || !aligned16(inout)) return hipErrorInvalidValue;
    GemmSlot slot;
    const PartBuf part = gemm_slot(stream, &slot) ? slot_parts(slot, 0) : PartBuf{nullptr, 0};
    return gemm_q4_f16<true>(input_f16, weights_q4_k, inout, M, N, K, stream, nullptr, part);
}

extern "C" hipError_t rf_rms_norm_batched_f16_on_stream(const float* d_x, const float* d_weight, uint16_t* d_out_f16,
                                                        const int n, const float eps, const int seq_len,
                                                        hipStream_t stream);

// The accumulate launchers above followed by rf_rms_norm_batched_f16_on_stream
// of inout (rows of N, weights norm_w) into out_f16, with the norm folded into
// the split-K reduction when the GEMM splits (N % 2048 == 0, N <= 8192);
// both outputs have the bits of the two calls.  norm_w and out_f16 16-byte
// aligned; out_f16 must not overlap inout or the input.
template <bool IS_Q6>
static hipError_t accumulate_rmsnorm(const uint16_t* input_f16, const void* weights, float* inout,
                                     const float* norm_w, float eps, uint16_t* out_f16, int M, int N, int K,
                                     hipStream_t stream) {
    if (input_f16 == nullptr || weights == nullptr || inout == nullptr || norm_w == nullptr || out_f16 == nullptr)
        return hipErrorInvalidValue;
    if (M <= 0 || N <= 0 || K <= 0 || (M % 64) != 0 || (N % 64) != 0 || (K % (IS_Q6 ? 2048 : kQK)) != 0)
        return hipErrorInvalidValue;
    if (!aligned16(input_f16) || !aligned16(weights) || !aligned16(inout) || !aligned16(norm_w) || !aligned16(out_f16))
        return hipErrorInvalidValue;
    const size_t n = (size_t)M * N;
    const uintptr_t d0 = reinterpret_cast<uintptr_t>(inout), o0 = reinterpret_cast<uintptr_t>(out_f16);
    if (d0 < o0 + 2 * n && o0 < d0 + 4 * n) return hipErrorInvalidValue;   // overlapping buffers
    GemmSlot slot;
    const PartBuf part = gemm_slot(stream, &slot) ? slot_parts(slot, 0) : PartBuf{nullptr, 0};
    bool fused = false;
    const RowNorm rn{norm_w, eps, out_f16, &fused};
    const hipError_t e = IS_Q6 ? gemm_q6_f16<true>(input_f16, weights, inout, M, N, K, stream, part, &rn)
                               : gemm_q4_f16<true>(input_f16, weights, inout, M, N, K, stream, nullptr, part, &rn);
    if (e != hipSuccess || fused) return e;
    return rf_rms_norm_batched_f16_on_stream(inout, norm_w, out_f16, N, eps, M, stream);
}

extern "C" hipError_t rf_gemm_q4_k_f16_accumulate_rmsnorm_launch(const uint16_t* input_f16, const void* weights_q4_k,
                                                                 float* inout, const float* norm_w, float eps,
                                                                 uint16_t* out_f16, int M, int N, int K,
                                                                 hipStream_t stream) {
    return accumulate_rmsnorm<false>(input_f16, weights_q4_k, inout, norm_w, eps, out_f16, M, N, K, stream);
}

extern "C" hipError_t rf_gemm_q6_k_f16_accumulate_rmsnorm_launch(const uint16_t* input_f16, const void* weights_q6_k,
                                                                 float* inout, const float* norm_w, float eps,
                                                                 uint16_t* out_f16, int M, int N, int K,
                                                                 hipStream_t stream) {
    return accumulate_rmsnorm<true>(input_f16, weights_q6_k, inout, norm_w, eps, out_f16, M, N, K, stream);
}

// Shapes the segmented / accumulating launches take: whole 256-column tiles,
// K in 512 steps (Q6_K: 2048, for the 16-byte aligned weight ring), the
// GEMM launchers' M/K rules, 16-byte aligned A and outputs.
template <bool IS_Q6>
static bool seg_shape_ok(const float* A, int M, int K) {
    if (M <= 0 || K <= 0 || M % 64 || K % (IS_Q6 ? 2048 : 512)) return false;
    return aligned16(A);
}

// Staged fp16 column segments; the fp32 v7 segments when the stream has
// no slot (or a Q6_K weight matrix is only 2-byte aligned).
template <bool IS_Q6>
static hipError_t gemm_segments(const float* A, const void* w0, const void* w1, const void* w2, float* d0,
                                float* d1, float* d2, int M, int n0, int n1, int n2, int K, hipStream_t st) {
    if (!seg_shape_ok<IS_Q6>(A, M, K) || !w0 || !d0 || n0 <= 0 || n1 < 0 || n2 < 0) return hipErrorInvalidValue;
    if (n0 % 256 || n1 % 256 || n2 % 256 || (n1 == 0 && n2 > 0)) return hipErrorInvalidValue;
    if ((n1 && (!w1 || !d1)) || (n2 && (!w2 || !d2))) return hipErrorInvalidValue;
    const uintptr_t wal = IS_Q6 ? 1u : 15u;
    bool w_al16 = true;
    for (const void* w : {w0, w1, w2}) {
        if (w && (reinterpret_cast<uintptr_t>(w) & wal)) return hipErrorInvalidValue;
        if (w && !aligned16(w)) w_al16 = false;
    }
    for (const float* d : {d0, d1, d2})
        if (d && !aligned16(d)) return hipErrorInvalidValue;
    GemmSlot slot;
    if (w_al16 && staging_slot(st, K, &slot)) {
        const void* ws[3] = {w0, n1 ? w1 : nullptr, n2 ? w2 : nullptr};
        const int q6[3] = {IS_Q6, IS_Q6, IS_Q6};
        const int ns[3] = {n0, n1, n2};
        return staged_rows(A, M, K, slot, st, [&](const uint16_t* a16, int m0, int rows, const PartBuf& pb) {
            float* ds[3] = {d0 + (size_t)m0 * n0, n1 ? d1 + (size_t)m0 * n1 : nullptr,
                            n2 ? d2 + (size_t)m0 * n2 : nullptr};
            return f16_segments(a16, ws, q6, ds, ns, rows, K, st);
        });
    }
    GemmSegs sg{};
    sg.w1 = static_cast<const uint8_t*>(w1);
    sg.w2 = static_cast<const uint8_t*>(w2);
    sg.d1 = d1;
    sg.d2 = d2;
    sg.n1 = n0;
    sg.n2 = n0 + n1;
    return launch_gemm<IS_Q6>(A, w0, d0, M, n0 + n1 + n2, K, st, sg);
}

template <bool IS_Q6>
static hipError_t gemm_accumulate(const float* A, const void* w, float* D, int M, int N, int K, hipStream_t st) {
    if (!seg_shape_ok<IS_Q6>(A, M, K) || !w || !D || N <= 0 || N % 256 || !aligned16(D)) return hipErrorInvalidValue;
    if (reinterpret_cast<uintptr_t>(w) & (IS_Q6 ? 1u : 15u)) return hipErrorInvalidValue;
    GemmSlot slot;
    if (aligned16(w) && staging_slot(st, K, &slot))
        return staged_rows(A, M, K, slot, st, [&](const uint16_t* a16, int m0, int rows, const PartBuf& pb) {
            float* d = D + (size_t)m0 * N;
            return IS_Q6 ? gemm_q6_f16<true>(a16, w, d, rows, N, K, st, pb)
                         : gemm_q4_f16<true>(a16, w, d, rows, N, K, st, nullptr, pb);
        });
    GemmSegs sg = single_seg(N);
    sg.accum = 1;
    return launch_gemm<IS_Q6>(A, w, D, M, N, K, st, sg);
}

extern "C" hipError_t rf_gemm_q4_k_segments_launch(const float* input, const void* w0, const void* w1, const void* w2,
                                                   float* out0, float* out1, float* out2, int M, int n0, int n1,
                                                   int n2, int K, hipStream_t stream) {
    return gemm_segments<false>(input, w0, w1, w2, out0, out1, out2, M, n0, n1, n2, K, stream);
}

extern "C" hipError_t rf_gemm_q6_k_segments_launch(const float* input, const void* w0, const void* w1, const void* w2,
                                                   float* out0, float* out1, float* out2, int M, int n0, int n1,
                                                   int n2, int K, hipStream_t stream) {
    return gemm_segments<true>(input, w0, w1, w2, out0, out1, out2, M, n0, n1, n2, K, stream);
}

// Up to three weight matrices over one fp16 input as column segments of one
// launch (rf_gemm_f16_segs_kernel), each Q4_K (type 12) or Q6_K (type 14):
// out_s[M x n_s] = fp16(A) * fp16(dequant W_s)^T, the products of
// rf_gemm_q4_k_f16_launch / rf_gemm_q6_k_f16_launch on K-sliced 64-column
// tiles of 128 or 256 rows.  The
// prefill Q/K/V of a layer whatever its type mix.  M % 64, n_s % 64 (n1, n2
// may be 0: fewer segments), K % 256 (K % 2048 with a Q6_K segment); input,
// weights and outputs 16-byte aligned.
extern "C" hipError_t rf_gemm_qk_f16_segments_launch(const uint16_t* input_f16, const void* w0, const void* w1,
                                                     const void* w2, int type0, int type1, int type2, float* out0,
                                                     float* out1, float* out2, int M, int n0, int n1, int n2, int K,
                                                     hipStream_t stream) {
    constexpr int kQ4KType = 12, kQ6KType = 14;
    if (input_f16 == nullptr || !aligned16(input_f16) || M <= 0 || M % 64 || K <= 0 || K % kQK)
        return hipErrorInvalidValue;
    if (n0 <= 0 || n1 < 0 || n2 < 0 || (n1 == 0 && n2 > 0)) return hipErrorInvalidValue;
    const void* ws[3] = {w0, w1, w2};
    float* ds[3] = {out0, out1, out2};
    const int ns[3] = {n0, n1, n2}, ts[3] = {type0, type1, type2};
    int q6[3] = {0, 0, 0};
    for (int i = 0; i < 3; ++i) {
        if (ns[i] == 0) continue;
        if (ns[i] % kQ4sBN || ws[i] == nullptr || ds[i] == nullptr || !aligned16(ws[i]) || !aligned16(ds[i]))
            return hipErrorInvalidValue;
        if (ts[i] != kQ4KType && ts[i] != kQ6KType) return hipErrorInvalidValue;
        if (ts[i] == kQ6KType && K % 2048) return hipErrorInvalidValue;
        q6[i] = ts[i] == kQ6KType;
    }
    return f16_segments(input_f16, ws, q6, ds, ns, M, K, stream);
}

extern "C" hipError_t rf_gemm_q4_k_accumulate_launch(const float* input, const void* weights_q4_k, float* inout,
                                                     int M, int N, int K, hipStream_t stream) {
    return gemm_accumulate<false>(input, weights_q4_k, inout, M, N, K, stream);
}

extern "C" hipError_t rf_gemm_q6_k_accumulate_launch(const float* input, const void* weights_q6_k, float* inout,
                                                     int M, int N, int K, hipStream_t stream) {
    return gemm_accumulate<true>(input, weights_q6_k, inout, M, N, K, stream);
}

// Gate/up pairs with SwiGLU in the epilogue: Q4_K staged as fp16 through the
// paired 256 x 128 tiles (rf_gemm_q4k_f16a_kernel<1, 2>); Q6_K (and Q4_K
// without a slot) on the fp32 v7 pair tiles.
template <bool IS_Q6>
static hipError_t gemm_swiglu(const float* A, const void* wg, const void* wu, void* D, int M, int N, int K,
                              hipStream_t st, bool f16_out) {
    if (!seg_shape_ok<IS_Q6>(A, M, K) || !wg || !wu || !D || N <= 0 || N % 128 || !aligned16(D))
        return hipErrorInvalidValue;
    const uintptr_t wal = IS_Q6 ? 1u : 15u;
    if ((reinterpret_cast<uintptr_t>(wg) & wal) || (reinterpret_cast<uintptr_t>(wu) & wal)) return hipErrorInvalidValue;
    GemmSlot slot;
    if (!IS_Q6 && staging_slot(st, K, &slot)) {
        const size_t esz = f16_out ? 2 : 4;
        return staged_rows(A, M, K, slot, st, [&](const uint16_t* a16, int m0, int rows, const PartBuf& pb) {
            return q4_f16_swiglu(a16, wg, wu, static_cast<uint8_t*>(D) + (size_t)m0 * N * esz, f16_out, rows, N, K,
                                 st);
        });
    }
    GemmSegs sg = single_seg(2 * N);
    sg.w1 = static_cast<const uint8_t*>(wu);
    sg.pair = f16_out ? 2 : 1;
    return launch_gemm<IS_Q6>(A, wg, static_cast<float*>(D), M, 2 * N, K, st, sg);
}

extern "C" hipError_t rf_gemm_q4_k_swiglu_launch(const float* input, const void* w_gate, const void* w_up, float* out,
                                                 int M, int N, int K, hipStream_t stream) {
    return gemm_swiglu<false>(input, w_gate, w_up, out, M, N, K, stream, false);
}

extern "C" hipError_t rf_gemm_q6_k_swiglu_launch(const float* input, const void* w_gate, const void* w_up, float* out,
                                                 int M, int N, int K, hipStream_t stream) {
    return gemm_swiglu<true>(input, w_gate, w_up, out, M, N, K, stream, false);
}

// The paired gate/up GEMM with its SwiGLU output rounded to fp16 (the
// operand the next GEMM's fp16 path reads): out_f16[M x N] holds
// __float2half(silu(gate) * up) of the fp32 launcher's values.
extern "C" hipError_t rf_gemm_q4_k_swiglu_f16_launch(const float* input, const void* w_gate, const void* w_up,
                                                     uint16_t* out_f16, int M, int N, int K, hipStream_t stream) {
    return gemm_swiglu<false>(input, w_gate, w_up, out_f16, M, N, K, stream, true);
}

extern "C" hipError_t rf_gemm_q6_k_swiglu_f16_launch(const float* input, const void* w_gate, const void* w_up,
                                                     uint16_t* out_f16, int M, int N, int K, hipStream_t stream) {
    return gemm_swiglu<true>(input, w_gate, w_up, out_f16, M, N, K, stream, true);
}
