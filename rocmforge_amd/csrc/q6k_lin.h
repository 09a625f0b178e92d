// q6k_lin.h -- the K-split Q6_K GEMV body shared by the Q6_K launchers
// (gemv_q6k.hip) and the mixed Q4_K/Q6_K fused QKV launch (gemv_q4k.hip).
#pragma once

#include "qk_common.h"

namespace rf {

constexpr int kQ6Ring = 3;   // register ring depth (rows in flight + 1) of the K-split GEMV (measured best)

// (m & a) | (~m & b) in one v_bfi_b32 (the compiler forms and/or pairs
// from the equivalent C expression)
__device__ __forceinline__ uint32_t bfi(uint32_t m, uint32_t a, uint32_t b) {
    uint32_t d;
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(d) : "s"(m), "v"(a), "v"(b));
    return d;
}

// 16 weights of one scale group (four dwords of 6-bit values) against 16 x,
// the x held pre-scaled by 2^24 (exact), for each of a lane's two runs.  Each 6-bit value is spread into a
// 16-bit half, where it reads as the fp16 subnormal q * 2^-24 (exact), and
// v_fma_mix takes that half as its fp16 operand: fma(q * 2^-24, x * 2^24, t)
// has the product q * x and the rounding of fma((float)q, x, t), so one
// instruction per weight does what a byte convert and an FMA did.
// The two runs of a lane (v0 against x0, v1 against x1) as two chains
// advanced alternately: a v_fma_mix that reads the previous one's result
// waits a cycle, the other chain's instruction fills it.
__device__ __forceinline__ void q6_dot16x2(const uint32_t v0[4], const float* x0, const uint32_t v1[4],
                                           const float* x1, float& t0, float& t1) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    t0 = 0.0f;
    t1 = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        // v_perm_b32 selector bytes: 0-3 pick a byte of v, 0x0C a zero
        const h2 e0 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0u, v0[k], 0x0C020C00u));   // bytes 0, 2
        const h2 o0 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0u, v0[k], 0x0C030C01u));   // bytes 1, 3
        const h2 e1 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0u, v1[k], 0x0C020C00u));
        const h2 o1 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0u, v1[k], 0x0C030C01u));
        t0 = __builtin_fmaf((float)e0[0], x0[4 * k + 0], t0);
        t1 = __builtin_fmaf((float)e1[0], x1[4 * k + 0], t1);
        t0 = __builtin_fmaf((float)o0[0], x0[4 * k + 1], t0);
        t1 = __builtin_fmaf((float)o1[0], x1[4 * k + 1], t1);
        t0 = __builtin_fmaf((float)e0[1], x0[4 * k + 2], t0);
        t1 = __builtin_fmaf((float)e1[1], x1[4 * k + 2], t1);
        t0 = __builtin_fmaf((float)o0[1], x0[4 * k + 3], t0);
        t1 = __builtin_fmaf((float)o1[1], x1[4 * k + 3], t1);
    }
}

// x sums of the two runs (before scaling), then x * 2^24 for q6_dot16x2
__device__ __forceinline__ void q6_x_prep(float (&xr)[2][16], float (&xs)[2]) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        float t = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) t += xr[r][i];
        xs[r] = t;
#pragma unroll
        for (int i = 0; i < 16; ++i) xr[r][i] *= 16777216.0f;
    }
}

// ── K-split Q6_K GEMV, lane-linear loads restaged through LDS ────────────
// A team of nwk = K / 2048 waves computes rows g, g + G, .. (< N) of y = W x
// (+ residual): team wave tw takes super-blocks [8 tw, 8 tw + 8) of every
// row with x held in registers (normalised first when norm_w is given:
// (x * inv) * norm_w, inv computed by the caller).  The weights are read the
// way the memory system streams best: a wave's 1680-byte part of a row
// (16-byte aligned when the matrix is and K/256 % 8 == 0) arrives as two
// lane-linear dwordx4 loads (lane L: bytes 16L and 16(64+L)), with two rows
// in flight.  Per row the wave writes the 1680 bytes to its own 2 KB LDS
// stage and each lane reads its ql / qh / scale bytes back (LDS accesses of
// one wave complete in order, so no barrier is needed).  Measured on MI355X
// for the 4096x14336 ffn_down layout: pure reads with this pattern run at
// ~7.7 TB/s against ~4 TB/s with per-lane 16-byte loads at 2-byte aligned
// block offsets.
//
// Row j's sum is the team's 4 nwk partial sums (16-lane row sums, in
// team-wave order) added in that order, whatever the grid.  Every thread of
// the workgroup calls this once (one barrier before the final sums); part
// holds nrows * nwk * 4 floats of this team.
struct Q6Seg {
    u32x4 a, b;
};

template <int NB>
__device__ __forceinline__ void q6_lin_team(const uint8_t* __restrict__ w, const float* __restrict__ x,
                                            const float* residual, float* y, int K, int N,
                                            const float* __restrict__ norm_w, float inv, int g, int G, int tw,
                                            int nwk, uint8_t* stage, float* part) {
    const int lane = threadIdx.x & (kWave - 1);
    const int nsb = K / kQK;
    const size_t row_bytes = (size_t)nsb * kQ6KBytes;
    const int blk = lane >> 3;
    const int sb = 8 * tw + blk;
    const int p = lane & 7;
    const int n = p >> 2;
    const int hq = (p & 3) >> 1;
    const int is = p & 1;
    const int nrows = g < N ? (N - 1 - g) / G + 1 : 0;

    float xr[2][16];
    {
        const size_t xo = (size_t)sb * kQK + 128 * n + 32 * hq + 16 * is;
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                float4 a = *reinterpret_cast<const float4*>(x + xo + 64 * r + 4 * k);
                if (norm_w) {
                    const float4 gw = *reinterpret_cast<const float4*>(norm_w + xo + 64 * r + 4 * k);
                    a = make_float4((a.x * inv) * gw.x, (a.y * inv) * gw.y, (a.z * inv) * gw.z, (a.w * inv) * gw.w);
                }
                xr[r][4 * k + 0] = a.x; xr[r][4 * k + 1] = a.y; xr[r][4 * k + 2] = a.z; xr[r][4 * k + 3] = a.w;
            }
    }
    float xs[2];
    const uint8_t* wseg = w + (size_t)(8 * tw) * kQ6KBytes;
    const int c1 = min(64 + lane, 104);   // chunks 105..127 re-read chunk 104 (same line), written to the spare area
    auto load = [&](Q6Seg& u, int j) {
        const uint8_t* src = wseg + (size_t)(nrows ? g + min(j, nrows - 1) * G : 0) * row_bytes;
        // nontemporal: each byte is read once; measured 6 % faster than
        // plain loads for the 4096 x 14336 ffn_down (no line is shared
        // between load instructions here, unlike the Q4_K unit loads)
        u.a = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + 16 * lane));
        u.b = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + 16 * c1));
    };
    // Aligned LDS reads.  Block b of the stage starts at byte 210b, which
    // is 0 or 2 past a dword boundary (a3); each 16-byte field is read as the
    // five aligned dwords around it and shifted into place (v_alignbit), and
    // each scale byte / d as the aligned dword holding it.  (Unaligned
    // 16-byte LDS reads at these offsets measured ~4 us slower per launch.)
    const uint32_t* st32 = reinterpret_cast<const uint32_t*>(stage);
    const int blkoff = blk * kQ6KBytes;
    const uint32_t sh = 8u * (uint32_t)(blkoff & 3);
    const int qlw = (blkoff + 16 * p) >> 2;
    const int qhw = (blkoff + 128 + 32 * n + 16 * is) >> 2;
    const int j1 = 192 + 8 * n + 2 * hq + is;        // scale bytes j1 (run 0) and j1 + 4 (run 1)
    const int s0w = (blkoff + j1) >> 2, s1w = (blkoff + j1 + 4) >> 2;
    const uint32_t s0sh = 8u * (uint32_t)((blkoff + j1) & 3), s1sh = 8u * (uint32_t)((blkoff + j1 + 4) & 3);
    const int dww = (blkoff + 208) >> 2;
    const uint32_t qsh = 2u * (uint32_t)hq;
    auto field = [&](int w0, uint32_t s) {
        uint32_t d[5];
#pragma unroll
        for (int t = 0; t < 5; ++t) d[t] = st32[w0 + t];
        return u32x4{__builtin_amdgcn_alignbit(d[1], d[0], s), __builtin_amdgcn_alignbit(d[2], d[1], s),
                     __builtin_amdgcn_alignbit(d[3], d[2], s), __builtin_amdgcn_alignbit(d[4], d[3], s)};
    };
    auto process = [&](const Q6Seg& u, int j) {
        *reinterpret_cast<u32x4*>(stage + 16 * lane) = u.a;
        *reinterpret_cast<u32x4*>(stage + 16 * (64 + lane)) = u.b;
        const u32x4 ql = field(qlw, sh);
        // qh shifted right by a further 2 hq bits in the same funnel shift:
        // only bits 0-1 and 4-5 of each byte are used below, so the bits
        // pulled in from the next dword at the top do not matter
        const u32x4 qh = field(qhw, sh + qsh);
        const float d = half_bits_to_float(st32[dww] >> sh);
        const float s0 = d * (float)(int8_t)((st32[s0w] >> s0sh) & 0xFFu);
        const float s1 = d * (float)(int8_t)((st32[s1w] >> s1sh) & 0xFFu);
        const uint32_t L[4] = {ql.x, ql.y, ql.z, ql.w};
        const uint32_t Q[4] = {qh.x, qh.y, qh.z, qh.w};
        uint32_t v0[4], v1[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            // per byte: q0 = (l & 15) | (h & 3) << 4, q1 = (l >> 4) | ((h >> 4) & 3) << 4,
            // as bit-field selects (v_bfi) of l and h with bits 2-3, 6-7 of h cleared
            const uint32_t hm = Q[t] & 0x33333333u;
            v0[t] = bfi(0x0F0F0F0Fu, L[t], hm << 4);
            v1[t] = bfi(0x0F0F0F0Fu, L[t] >> 4, hm);
        }
        float t0, t1;
        q6_dot16x2(v0, xr[0], v1, xr[1], t0, t1);
        float acc = s0 * (t0 - 32.0f * xs[0]);
        acc += s1 * (t1 - 32.0f * xs[1]);
        // the four 16-lane row sums go to LDS (no cross-row broadcast and
        // no read-lane per row); the final pass adds them in fixed order
        const float r16 = row16_sum(acc);
        if ((lane & 15) == 0) part[(j * nwk + tw) * 4 + (lane >> 4)] = r16;
    };
    Q6Seg ring[NB];
    ring_pipeline<NB>(nrows, ring, load, process, [&]() { q6_x_prep(xr, xs); });
    __syncthreads();
    for (int j = tw * kWave + lane; j < nrows; j += nwk * kWave) {
        float t = 0.0f;
        for (int k = 0; k < 4 * nwk; ++k) t += part[j * nwk * 4 + k];
        y[g + j * G] = t + (residual ? residual[g + j * G] : 0.0f);
    }
}

}  // namespace rf
