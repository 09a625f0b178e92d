// gemv_q6k.hip -- Q6_K decode GEMV for CDNA4 (gfx950, wave64).
//
// Drop-in for hip_kernels/quant/q6_k_gemv.hip (gemv_q6_k_f32_launch):
// fp32 activations (the reference has no Q8 path for Q6_K), same symbol,
// argument meaning and error returns.
//
// Element mapping (docs/q6_k_block_format.md, q6_k_gemv.hip:111-152): for
// half n, quarter q and l < 32 the weight at 128n + 32q + l is
//   q6 = (nibble of ql[64n + 32(q&1) + l], high for q>=2)
//        | ((qh[32n + l] >> 2q) & 3) << 4,   value = d * sc[8n+2q+l/16] * (q6-32).
//
// Tiling: four lanes per 210-byte block (lane p: half n = p>>1, l in
// [16c, 16c+16) with c = p&1), sixteen blocks per wave row step.  Each lane
// reads its 16 B of low-ql, 16 B of high-ql and 16 B of qh with unaligned
// 16-byte loads (blocks are only 2-byte aligned), 8 scale bytes and d, and
// produces 64 products against x held in LDS.
#include "qk_common.h"

namespace rf {

constexpr int kQ6Threads = 256;
constexpr int kQ6Waves = kQ6Threads / kWave;
constexpr int kQ6SbPerStep = 16;

struct Q6Unit {
    u32x4 lo, hi, qh;  // ql[64n+16c..], ql[64n+32+16c..], qh[32n+16c..]
    u32x2 sc;          // scales[8n .. 8n+7]
    uint32_t d;        // fp16 bits
};

__device__ __forceinline__ Q6Unit q6k_load_unit(const uint8_t* blk, int p) {
    const int n = p >> 1, c = p & 1;
    Q6Unit u;
    u.lo = ld16(blk + 64 * n + 16 * c);
    u.hi = ld16(blk + 64 * n + 32 + 16 * c);
    u.qh = ld16(blk + 128 + 32 * n + 16 * c);
    u.sc = ld8(blk + 192 + 8 * n);
    u.d = ld_u16(blk + 208);
    return u;
}

// 16 products of one quarter: packed q6 bytes (4 dwords) against 16 x.
__device__ __forceinline__ float q6_quarter(float acc, float s, const uint32_t q6[4], const float* xq) {
    const float4* xv = reinterpret_cast<const float4*>(xq);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const float4 a = xv[t];
        const uint32_t v = q6[t];
        acc += s * ((float)((v >> 0) & 0xFFu) - 32.0f) * a.x;
        acc += s * ((float)((v >> 8) & 0xFFu) - 32.0f) * a.y;
        acc += s * ((float)((v >> 16) & 0xFFu) - 32.0f) * a.z;
        acc += s * ((float)((v >> 24) & 0xFFu) - 32.0f) * a.w;
    }
    return acc;
}

__device__ __forceinline__ float q6k_unit_dot(const Q6Unit& u, int p, const float* xblk, float acc) {
    const int n = p >> 1, c = p & 1;
    const float d = half_bits_to_float(u.d);
    // scale bytes 8n + 2q + c, q = 0..3: bytes c, c+2 of sc.x and of sc.y
    const uint32_t sh = 8u * (uint32_t)c;
    const float s0 = d * (float)(int8_t)((u.sc.x >> sh) & 0xFFu);
    const float s1 = d * (float)(int8_t)((u.sc.x >> (sh + 16)) & 0xFFu);
    const float s2 = d * (float)(int8_t)((u.sc.y >> sh) & 0xFFu);
    const float s3 = d * (float)(int8_t)((u.sc.y >> (sh + 16)) & 0xFFu);
    const uint32_t L[4] = {u.lo.x, u.lo.y, u.lo.z, u.lo.w};
    const uint32_t H[4] = {u.hi.x, u.hi.y, u.hi.z, u.hi.w};
    const uint32_t Q[4] = {u.qh.x, u.qh.y, u.qh.z, u.qh.w};
    uint32_t q0[4], q1[4], q2[4], q3[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        q0[t] = (L[t] & 0x0F0F0F0Fu) | ((Q[t] & 0x03030303u) << 4);
        q1[t] = (H[t] & 0x0F0F0F0Fu) | (((Q[t] >> 2) & 0x03030303u) << 4);
        q2[t] = ((L[t] >> 4) & 0x0F0F0F0Fu) | (((Q[t] >> 4) & 0x03030303u) << 4);
        q3[t] = ((H[t] >> 4) & 0x0F0F0F0Fu) | (((Q[t] >> 6) & 0x03030303u) << 4);
    }
    const float* xb = xblk + 128 * n + 16 * c;
    acc = q6_quarter(acc, s0, q0, xb);
    acc = q6_quarter(acc, s1, q1, xb + 32);
    acc = q6_quarter(acc, s2, q2, xb + 64);
    acc = q6_quarter(acc, s3, q3, xb + 96);
    return acc;
}

template <int R, bool LDS>
__global__ __launch_bounds__(kQ6Threads) void rf_q6k_gemv_kernel(const uint8_t* __restrict__ w,
                                                                  const float* __restrict__ x, float* __restrict__ y,
                                                                  int K, int N) {
    extern __shared__ __align__(16) uint8_t smem[];
    float* xs = reinterpret_cast<float*>(smem);
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int s = lane >> 2;
    const int p = lane & 3;
    const int nsb = K / kQK;
    const size_t row_bytes = (size_t)nsb * kQ6KBytes;
    int row_begin, row_end;
    wave_row_range(N, blockIdx.x * kQ6Waves + wave, gridDim.x * kQ6Waves, &row_begin, &row_end);

    int row0 = row_begin;
    int sb0 = 0;
    Q6Unit cur[R];
    auto load_step = [&](Q6Unit(&u)[R], int r0, int sbc) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int row = min(r0 + r, row_end - 1);
            u[r] = q6k_load_unit(w + (size_t)row * row_bytes + (size_t)sbc * kQ6KBytes, p);
        }
    };
    if (row0 < row_end) load_step(cur, row0, min(s, nsb - 1));

    if (LDS) {
        stage_f32_to_lds(x, K, xs);
        __syncthreads();
    }
    const float* xv = LDS ? xs : x;

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;

    while (row0 < row_end) {
        int nrow0 = row0, nsb0 = sb0 + kQ6SbPerStep;
        if (nsb0 >= nsb) {
            nsb0 = 0;
            nrow0 += R;
        }
        Q6Unit nxt[R];
        if (nrow0 < row_end) load_step(nxt, nrow0, min(nsb0 + s, nsb - 1));

        const int sb = sb0 + s;
        if (sb < nsb) {
            const float* xblk = xv + sb * kQK;
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r] = q6k_unit_dot(cur[r], p, xblk, acc[r]);
        }
        if (nsb0 == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float g = wave_sum(acc[r]);
                if (lane == r && row0 + r < row_end) y[row0 + r] = g;
                acc[r] = 0.0f;
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) cur[r] = nxt[r];
        row0 = nrow0;
        sb0 = nsb0;
    }
}

}  // namespace rf

using namespace rf;

// Validation as q6_k_gemv.hip:284-285 (K > 0, N > 0, K % 256 == 0), plus
// 2-byte weight alignment (the fp16 d field is read as one 16-bit word).
extern "C" hipError_t gemv_q6_k_f32_launch(const void* weights_q6_k, const float* input, float* output, int n_rows,
                                           int ncols_dst, hipStream_t stream) {
    if (n_rows <= 0 || ncols_dst <= 0) return hipErrorInvalidValue;
    if (n_rows % kQK != 0) return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(weights_q6_k) & 1u) != 0) return hipErrorInvalidValue;
    constexpr int R = 2;
    const int need = (ncols_dst + kQ6Waves - 1) / kQ6Waves;
    const int cap = device_cu_count() * gemv_wg_per_cu();
    const int grid = need < cap ? need : cap;
    const size_t lds = (size_t)n_rows * sizeof(float);
    const uint8_t* w = static_cast<const uint8_t*>(weights_q6_k);
    if (lds <= 65536) {
        hipLaunchKernelGGL((rf_q6k_gemv_kernel<R, true>), dim3(grid), dim3(kQ6Threads), lds, stream, w, input, output,
                           n_rows, ncols_dst);
    } else {
        hipLaunchKernelGGL((rf_q6k_gemv_kernel<R, false>), dim3(grid), dim3(kQ6Threads), 0, stream, w, input, output,
                           n_rows, ncols_dst);
    }
    return hipGetLastError();
}
