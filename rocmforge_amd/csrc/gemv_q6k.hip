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
// Kernels (the launcher picks the first that applies):
//  * rf_q6k_gemv_lin_kernel: K <= 16384, K/256 % 8 == 0, 16-byte aligned
//    matrix.  K split across the waves of a workgroup (8 super-blocks per
//    wave), x held in registers, weights read with lane-linear aligned
//    16-byte loads and restaged per wave through LDS.
//  * rf_q6k_gemv_xreg_kernel: K <= 16384 otherwise.  Same K split and x
//    registers, each lane loading its block fields directly (16-byte loads
//    at the 2-byte aligned block offsets).
//  * rf_q6k_gemv_kernel: larger K.  One row per wave step, four lanes per
//    block, x in L2 (K*4 > 64 KB).
#include "q6k_lin.h"


namespace rf {


constexpr int kQ6SbPerStep = 16;

struct Q6Unit {
    u32x4 lo, hi, qh;  // ql[64n+16c..], ql[64n+32+16c..], qh[32n+16c..]
    u32x2 sc;          // scales[8n .. 8n+7]
    uint32_t d;        // bytes 206..209: scales[14], scales[15], d (fp16 in the high half)
};

__device__ __forceinline__ Q6Unit q6k_load_unit(const uint8_t* blk, int p) {
    const int n = p >> 1, c = p & 1;
    Q6Unit u;
    u.lo = ld16(blk + 64 * n + 16 * c);
    u.hi = ld16(blk + 64 * n + 32 + 16 * c);
    u.qh = ld16(blk + 128 + 32 * n + 16 * c);
    u.sc = ld8(blk + 192 + 8 * n);
    // d is read as the high half of the in-block dword at 206 (a 16-bit load
    // would be packed with its neighbour by the compiler, forcing an early
    // wait on the prefetch)
    u.d = ld4(blk + 206);
    return u;
}

// One 16-weight scale group: s * sum_i (q6_i - 32) * x_i, evaluated as
// s * (sum_i q6_i * x_i - 32 * sum_i x_i) with sum_i x_i (xsum) precomputed
// once per group of x.  The q6 bytes convert straight to float
// (v_cvt_f32_ubyteN), so a weight costs a convert and an FMA.
__device__ __forceinline__ float q6_group(float acc, float s, const uint32_t q6[4], const float* xq, float xsum) {
    const float4* xv = reinterpret_cast<const float4*>(xq);
    float t = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float4 a = xv[k];
        const uint32_t v = q6[k];
        t += (float)((v >> 0) & 0xFFu) * a.x;
        t += (float)((v >> 8) & 0xFFu) * a.y;
        t += (float)((v >> 16) & 0xFFu) * a.z;
        t += (float)((v >> 24) & 0xFFu) * a.w;
    }
    return acc + s * (t - 32.0f * xsum);
}

// xblk: x of this super-block; in the padded LDS layout (x_pad) its second
// half starts 132 floats in, otherwise 128 (HALF).  xsum16: sums of x over
// the block's 16-element groups.
template <int HALF>
__device__ __forceinline__ float q6k_unit_dot(const Q6Unit& u, int p, const float* xblk, const float* xsum16,
                                              float acc) {
    const int n = p >> 1, c = p & 1;
    const float d = half_bits_to_float(u.d >> 16);
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
    const int g = 8 * n + c;   // 16-element group of quarter 0 inside the block
    const float* xb = xblk + HALF * n + 16 * c;
    acc = q6_group(acc, s0, q0, xb, xsum16[g]);
    acc = q6_group(acc, s1, q1, xb + 32, xsum16[g + 2]);
    acc = q6_group(acc, s2, q2, xb + 64, xsum16[g + 4]);
    acc = q6_group(acc, s3, q3, xb + 96, xsum16[g + 6]);
    return acc;
}

// Per-group sums of the staged x (after a barrier that published xs).
template <bool PADDED>
__device__ __forceinline__ void q6_xsum16(const float* xs, int K, float* xsum16) {
    for (int g = threadIdx.x; g < K / 16; g += blockDim.x) {
        const float4* v = reinterpret_cast<const float4*>(xs + (PADDED ? x_pad(16 * g) : 16 * g));
        float t = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float4 a = v[k];
            t += a.x + a.y + a.z + a.w;
        }
        xsum16[g] = t;
    }
}

template <int R, bool LDS, int NW, int NB>
__global__ __launch_bounds__(NW * 64) void rf_q6k_gemv_kernel(const uint8_t* __restrict__ w,
                                                                  const float* __restrict__ x, const float* residual,
                                                                  float* y, int K, int N) {
    extern __shared__ __align__(16) uint8_t smem[];
    float* xs = reinterpret_cast<float*>(smem);
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // wave-uniform (SGPR)
    const int s = lane >> 2;
    const int p = lane & 3;
    const int nsb = K / kQK;
    const size_t row_bytes = (size_t)nsb * kQ6KBytes;
    const int nwaves = gridDim.x * NW;
    int row_begin, row_end;
    wave_row_range(N, blockIdx.x * NW + wave, nwaves, &row_begin, &row_end);

    // Register-buffer pipeline, as in the Q4_K kernel.
    const int spr = (nsb + kQ6SbPerStep - 1) / kQ6SbPerStep;
    const int nsteps = ((row_end - row_begin + R - 1) / R) * spr;
    auto load = [&](Q6Unit (&u)[R], int i) {
        const int row0 = row_begin + (i / spr) * R;
        const int sbc = min((i % spr) * kQ6SbPerStep + s, nsb - 1);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int row = max(min(row0 + r, row_end - 1), 0);   // waves without rows re-read row 0
            u[r] = q6k_load_unit(w + (size_t)row * row_bytes + (size_t)sbc * kQ6KBytes, p);
        }
    };
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
    const float* xv = LDS ? xs : x;
    // row results parked in LDS, written to HBM after the loop (no global
    // store between the prefetch loads in the in-order memory counter)
    // LDS: [x (padded, LDS mode only)] [x group sums (K/16)] [row results]
    const int max_rows = (N + nwaves - 1) / nwaves;
    float* xsum16 = reinterpret_cast<float*>(smem + (LDS ? (size_t)(x_padded_floats(K) + 4) * 4 : 0));
    float* out_lds = xsum16 + K / 16 + wave * max_rows;
    auto process = [&](const Q6Unit (&u)[R], int i) {
        const int row0 = row_begin + (i / spr) * R;
        const int sb = (i % spr) * kQ6SbPerStep + s;
        if (sb < nsb) {
            const float* xblk = xv + (LDS ? x_pad(sb * kQK) : sb * kQK);
#pragma unroll
            for (int r = 0; r < R; ++r)
                acc[r] = q6k_unit_dot<LDS ? 132 : 128>(u[r], p, xblk, xsum16 + sb * 16, acc[r]);
        }
        if ((i % spr) == spr - 1) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float g = wave_sum(acc[r]);
                if (lane == 0 && row0 + r < row_end) out_lds[row0 + r - row_begin] = g;
                acc[r] = 0.0f;
            }
        }
    };

    struct Step {
        Q6Unit u[R];
    };
    Step ring[NB];
    ring_pipeline<NB>(nsteps, ring, [&](Step& b, int i) { load(b.u, i); },
                      [&](const Step& b, int i) { process(b.u, i); },
                      [&]() {
                          if (LDS) {
                              stage_f32_to_lds_regs(x, K, xs);
                              __syncthreads();
                          }
                          q6_xsum16<LDS>(xv, K, xsum16);
                          __syncthreads();
                      });
    for (int j = lane; j < row_end - row_begin; j += kWave)
        y[row_begin + j] = out_lds[j] + (residual ? residual[row_begin + j] : 0.0f);
}

// ── K-split Q6_K GEMV with x held in registers (other K <= 16384) ───────────────
// A workgroup has one wave per 8-super-block slice of K (NWK = nsb/8
// rounded up, at most 8 waves: K <= 16384).  The 8 lanes p = 0..7 of a
// super-block sb = 8w + l/8 read its bytes with three 16-byte loads each,
// so every load instruction covers whole contiguous runs of the block:
//   A: ql[16p .. 16p+16)              (all 128 B of ql across the 8 lanes)
//   B: qh[32n + 16(p&1) .. +16)       (n = p>>2; lanes p, p^2 share it)
//   C: bytes 192..207 (n = 0) or 194..209 (n = 1): the scales, and d in
//      the top half of the last dword for n = 1 (ds_bpermute hands d to
//      the n = 0 lanes).
// Lane p then owns the 32 weights its ql bytes encode: ql-half n, bytes
// b = 16(p&3) .. b+15, i.e. l = 16(p&1) + i of quarters hq and hq + 2
// (hq = (p&3)>>1): elements 128n + 32q + l.  Its 32 x values and their two
// 16-element sums are loaded into registers once, so the weight stream runs
// with no LDS traffic and no barrier in front of it.  Every wave walks all
// rows of its workgroup (rows g, g + grid, g + 2 grid, ...: the grid
// streams neighbouring rows together), reduces its slice's partial over the
// wave and parks it in LDS; the slices of a row are summed in fixed slice
// order at the end.
struct Q6Lane {
    u32x4 ql, qh, sc;
};

__device__ __forceinline__ Q6Lane q6k_load_lane(const uint8_t* blk, int p) {
    const int n = p >> 2;
    Q6Lane u;
    u.ql = ld16(blk + 16 * p);
    u.qh = ld16(blk + 128 + 32 * n + 16 * (p & 1));
    u.sc = ld16(blk + 192 + 2 * n);
    return u;
}

template <int NB>
__global__ __launch_bounds__(512) void rf_q6k_gemv_xreg_kernel(const uint8_t* __restrict__ w,
                                                                const float* __restrict__ x, const float* residual,
                                                                float* y, int K, int N) {
    extern __shared__ __align__(16) float part[];   // [rows of this workgroup][NWK]
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int nwk = blockDim.x / kWave;
    const int nsb = K / kQK;
    const size_t row_bytes = (size_t)nsb * kQ6KBytes;
    const int sb = 8 * wave + (lane >> 3);
    const bool live = sb < nsb;
    const int sbc = live ? sb : nsb - 1;
    const int p = lane & 7;
    const int n = p >> 2;
    const int hq = (p & 3) >> 1;
    const int is = p & 1;
    const int g = blockIdx.x;
    const int G = gridDim.x;
    const int nrows = g < N ? (N - 1 - g) / G + 1 : 0;

    // x of this lane: run r (quarter hq + 2r) at element sbc*256 + 128n + 32(hq+2r) + 16 is
    float xr[2][16];
    {
        const float* xb = x + (size_t)sbc * kQK + 128 * n + 32 * hq + 16 * is;
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float4 a = *reinterpret_cast<const float4*>(xb + 64 * r + 4 * k);
                xr[r][4 * k + 0] = a.x; xr[r][4 * k + 1] = a.y; xr[r][4 * k + 2] = a.z; xr[r][4 * k + 3] = a.w;
            }
    }
    float xs[2];
    const uint8_t* wl = w + (size_t)sbc * kQ6KBytes;
    auto load = [&](Q6Lane& u, int j) {
        const int row = nrows ? g + min(j, nrows - 1) * G : 0;
        u = q6k_load_lane(wl + (size_t)row * row_bytes, p);
    };
    // scale bytes j1 = 8n + 2hq + is (run 0) and j1 + 4 (run 1) inside C:
    // n = 0: dwords 0 / 1, byte j1; n = 1 (C starts at byte 194): offset
    // o1 = j1 - 2 = 6 + 2hq + is -> dword 1 or 2, and o1 + 4 -> dword 2 or 3.
    const int o1 = n ? 6 + 2 * hq + is : 2 * hq + is;
    const uint32_t ssh = 8u * (uint32_t)(o1 & 3);
    const int dw1 = o1 >> 2;
    const uint32_t qsh = 2u * (uint32_t)hq;       // qh bit pair of run 0 (run 1: +4)
    const int dsrc = 4 * ((lane & ~7) | 4);       // lane holding d (n = 1 lane of the group)
    auto process = [&](const Q6Lane& u, int j) {
        const uint32_t dword3 = (uint32_t)__builtin_amdgcn_ds_bpermute(dsrc, (int)u.sc.w);
        const float d = half_bits_to_float(dword3 >> 16);
        const uint32_t w1 = dw1 == 0 ? u.sc.x : (dw1 == 1 ? u.sc.y : u.sc.z);
        const uint32_t w2 = dw1 == 0 ? u.sc.y : (dw1 == 1 ? u.sc.z : u.sc.w);
        const float s0 = d * (float)(int8_t)((w1 >> ssh) & 0xFFu);
        const float s1 = d * (float)(int8_t)((w2 >> ssh) & 0xFFu);
        const uint32_t L[4] = {u.ql.x, u.ql.y, u.ql.z, u.ql.w};
        const uint32_t Q[4] = {u.qh.x, u.qh.y, u.qh.z, u.qh.w};
        uint32_t v0[4], v1[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            v0[t] = (L[t] & 0x0F0F0F0Fu) | (((Q[t] >> qsh) & 0x03030303u) << 4);
            v1[t] = ((L[t] >> 4) & 0x0F0F0F0Fu) | (((Q[t] >> (qsh + 4)) & 0x03030303u) << 4);
        }
        float t0, t1;
        q6_dot16x2(v0, xr[0], v1, xr[1], t0, t1);
        float acc = s0 * (t0 - 32.0f * xs[0]);
        acc += s1 * (t1 - 32.0f * xs[1]);
        const float tot = wave_sum(live ? acc : 0.0f);
        if (lane == 0) part[j * nwk + wave] = tot;
    };
    Q6Lane ring[NB];
    ring_pipeline<NB>(nrows, ring, load, process, [&]() { q6_x_prep(xr, xs); });
    __syncthreads();
    for (int j = threadIdx.x; j < nrows; j += blockDim.x) {
        float t = 0.0f;
        for (int k = 0; k < nwk; ++k) t += part[j * nwk + k];
        y[g + j * G] = t + (residual ? residual[g + j * G] : 0.0f);
    }
}


// The K-split Q6_K GEMV of q6k_lin.h as a kernel: one team of nwk =
// blockDim / 64 waves per workgroup, rows blockIdx.x, blockIdx.x + gridDim.x, ..
template <int NB>
__global__ __launch_bounds__(512) void rf_q6k_gemv_lin_kernel(const uint8_t* __restrict__ w,
                                                               const float* __restrict__ x, const float* residual,
                                                               float* y, int K, int N,
                                                               const float* __restrict__ norm_w, float eps) {
    __shared__ __align__(16) uint8_t stage_lds[8 * 2048];
    extern __shared__ __align__(16) float part[];   // [rows of this workgroup][NWK][4 lane rows]
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    // optional fused RMSNorm: x -> (x * inv) * norm_w, inv in the canonical
    // order of the standalone norm (same bits)
    __shared__ float red[4];
    const float inv = norm_w ? rms_inv_canonical(x, K, eps, red) : 1.0f;
    q6_lin_team<NB>(w, x, residual, y, K, N, norm_w, inv, blockIdx.x, gridDim.x, wave, blockDim.x / kWave,
                    stage_lds + wave * 2048, part);
}

}  // namespace rf

using namespace rf;

// Validation as q6_k_gemv.hip:284-285 (K > 0, N > 0, K % 256 == 0), plus
// 2-byte weight alignment (the fp16 d field is read as one 16-bit word).
static hipError_t launch_q6(const void* weights_q6_k, const float* input, const float* residual, float* output,
                            int n_rows, int ncols_dst, hipStream_t stream) {
    const uint8_t* w = static_cast<const uint8_t*>(weights_q6_k);
    const int nsb = n_rows / kQK;
    if (nsb <= 64 && nsb % 8 == 0 && (reinterpret_cast<uintptr_t>(w) & 15u) == 0) {
        const int nwk = nsb / 8;
        const int cap = device_cu_count() * (nwk >= 4 ? 1 : 8 / nwk);
        const int grid = ncols_dst < cap ? ncols_dst : cap;
        const size_t lds = (size_t)((ncols_dst + grid - 1) / grid) * nwk * 4 * sizeof(float);
        if (lds <= 64 * 1024) {
            hipLaunchKernelGGL((rf_q6k_gemv_lin_kernel<kQ6Ring>), dim3(grid), dim3(nwk * 64), lds, stream, w, input,
                               residual, output, n_rows, ncols_dst, nullptr, 0.0f);
            return hipGetLastError();
        }
    }
    if (nsb <= 64) {
        const int nwk = (nsb + 7) / 8;
        // about 8 waves per CU: short K (few slices per workgroup) gets
        // several workgroups per CU
        const int cap = device_cu_count() * (nwk >= 4 ? 1 : 8 / nwk);
        const int grid = ncols_dst < cap ? ncols_dst : cap;
        const size_t lds = (size_t)((ncols_dst + grid - 1) / grid) * nwk * sizeof(float);
        if (lds <= 64 * 1024) {
            hipLaunchKernelGGL((rf_q6k_gemv_xreg_kernel<kQ6Ring>), dim3(grid), dim3(nwk * 64), lds, stream, w, input,
                               residual, output, n_rows, ncols_dst);
            return hipGetLastError();
        }
    }
    // one row per wave step, 8 waves per workgroup, one workgroup per CU
    constexpr int nw = 8;
    const int need = (ncols_dst + nw - 1) / nw;
    const int cap = device_cu_count();
    const int grid = need < cap ? need : cap;
    const bool in_lds = (size_t)x_padded_floats(n_rows) * sizeof(float) <= 65536;
    const size_t lds = in_lds ? (size_t)(x_padded_floats(n_rows) + 4) * sizeof(float) : 0;
    const size_t out_bytes = (size_t)nw * ((ncols_dst + (size_t)grid * nw - 1) / ((size_t)grid * nw)) * 4 +
                             (size_t)(n_rows / 16) * 4;   // + x group sums
    if (out_bytes > 64 * 1024) return hipErrorInvalidValue;
    const dim3 blk(nw * 64);
#define RF_Q6_LAUNCH(L) \
    hipLaunchKernelGGL((rf_q6k_gemv_kernel<1, L, nw, 3>), dim3(grid), blk, lds + out_bytes, stream, w, input, \
                       residual, output, n_rows, ncols_dst)
    if (in_lds) RF_Q6_LAUNCH(true); else RF_Q6_LAUNCH(false);
#undef RF_Q6_LAUNCH
    return hipGetLastError();
}

extern "C" hipError_t gemv_q6_k_f32_launch(const void* weights_q6_k, const float* input, float* output, int n_rows,
                                           int ncols_dst, hipStream_t stream) {
    if (n_rows <= 0 || ncols_dst <= 0) return hipErrorInvalidValue;
    if (n_rows % kQK != 0) return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(weights_q6_k) & 1u) != 0) return hipErrorInvalidValue;
    return launch_q6(weights_q6_k, input, nullptr, output, n_rows, ncols_dst, stream);
}

// output[n] = y[n] + residual[n], output may alias residual.  No
// counterpart in the reference, whose Q6_K ffn_down takes a GEMV and a
// separate add (gpu_dispatch_gemv_residual_on_stream returns Ok(false) for
// Q6_K, ops.rs:666-695); the argument order and checks follow the Q4_K
// residual launcher (q4_k_q8_inline.hip:404-415).
extern "C" hipError_t gemv_q6_k_f32_residual_launch(const void* weights_q6_k, const float* input,
                                                    const float* residual, float* output, int n_rows, int ncols_dst,
                                                    hipStream_t stream) {
    if (n_rows <= 0 || ncols_dst <= 0 || residual == nullptr) return hipErrorInvalidValue;
    if (n_rows % kQK != 0) return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(weights_q6_k) & 1u) != 0) return hipErrorInvalidValue;
    return launch_q6(weights_q6_k, input, residual, output, n_rows, ncols_dst, stream);
}

// out = W * rmsnorm(input, norm_w, eps) with the standalone norm's bits
// (gpu_rms_norm then gemv_q6_k_f32_launch), one launch.  No counterpart in
// the reference (its LM head and Q6_K attn_v take a norm launch first,
// src/gpu/forward.rs:329-376, :2349-2359).  Needs K / 256 % 8 == 0,
// K <= 16384 and 16-byte aligned weights, input and norm_w.
extern "C" hipError_t rf_gemv_q6_k_rmsnorm_launch(const void* weights_q6_k, const float* input, const float* norm_w,
                                                  float eps, float* output, int n_rows, int ncols_dst,
                                                  hipStream_t stream) {
    if (n_rows <= 0 || ncols_dst <= 0 || n_rows % kQK != 0 || input == nullptr || norm_w == nullptr)
        return hipErrorInvalidValue;
    const int nsb = n_rows / kQK;
    if (nsb > 64 || nsb % 8 != 0 || ((reinterpret_cast<uintptr_t>(weights_q6_k) | reinterpret_cast<uintptr_t>(input) |
                                      reinterpret_cast<uintptr_t>(norm_w)) & 15u) != 0)
        return hipErrorInvalidValue;
    const int nwk = nsb / 8;
    const int cap = device_cu_count() * (nwk >= 4 ? 1 : 8 / nwk);
    const int grid = ncols_dst < cap ? ncols_dst : cap;
    const size_t lds = (size_t)((ncols_dst + grid - 1) / grid) * nwk * 4 * sizeof(float);
    if (lds > 64 * 1024) return hipErrorInvalidValue;
    hipLaunchKernelGGL((rf_q6k_gemv_lin_kernel<kQ6Ring>), dim3(grid), dim3(nwk * 64), lds, stream,
                       static_cast<const uint8_t*>(weights_q6_k), input, nullptr, output, n_rows, ncols_dst, norm_w,
                       eps);
    return hipGetLastError();
}
