// gemv_q4k.hip -- Q4_K decode GEMVs for CDNA4 (gfx950, wave64).
//
// Drop-in for hip_kernels/quant/q4_k_q8_inline.hip (Q8_0-inline family) and
// hip_kernels/quant/q4_k_gemv.hip (FP32-activation family): same extern "C"
// symbols, argument meaning (n_rows = K = input length, ncols_dst = N =
// output rows) and error returns.
//
// Design (MI355X-first, not a port of the wave32 kernels):
//  * 256-thread workgroups = 4 wave64s.  Each wave owns R output rows at a
//    time; inside a row the 64 lanes split 16 consecutive super-blocks four
//    ways (lane = 4*s + p: super-block s, nibble pair p).  One row step
//    therefore reads 16 x 144 B = 2304 contiguous bytes per row with
//    16-byte loads, instead of one lane per 144-byte block.
//  * The activation vector is quantised to Q8_0 once per workgroup into LDS
//    (qs contiguous, scales and per-block int sums separate) while the
//    first weight loads are already in flight.
//  * Integer dots use v_dot4_i32_i8 (4 nibble x int8 products per op); the
//    fp32 sub-block combine is the reference expression, so the only
//    difference to the reference is the fp32 summation order.
//  * Workgroups stride over row groups; the grid is capped at a multiple of
//    the CU count so a large N re-uses each workgroup's quantised vector.
//  * Long rows (K a multiple of 4096 from 8192: the Qwen3-8B ffn_down) take
//    a K-split kernel instead (rf_q4k_q8_lin_kernel): each wave of a team
//    keeps its K slice's Q8 x in registers and streams every row of its
//    workgroup.
#include <type_traits>

#include "q6k_lin.h"


namespace rf {

constexpr int kRingDepth = 3;   // register ring depth of the one-row-per-step GEMV (measured best)

constexpr int kThreads = 256;
constexpr int kWavesPerWg = kThreads / kWave;
constexpr int kSbPerStep = 16;  // super-blocks per wave row step

enum Q4Mode { kPlain = 0, kResidual = 1, kGateUp = 2, kQkv = 3 };

// kQkv: three matrices (Q, K, V projections) in one launch.  The grid's
// waves are split over the matrices in proportion to their rows (qkv_split),
// so each wave streams rows of one matrix and its weight, output and bias
// pointers are fixed for the whole launch; output = dot + bias (bias may be
// null).
struct QkvArgs {
    const uint8_t* w[3];
    const float* bias[3];
    float* y[3];
    int n_q, n_kv;
    const float* norm_w;   // RMSNorm weights applied to x first (any mode), or null
    float eps;
    int no_v;              // Q and K only (the V projection runs elsewhere)
};

// Waves per matrix: [0, nw[0]) on Q, then nw[1] on K, nw[2] on V (each >= 1;
// nwaves >= 3), or with no_v nw[2] = 0 (nwaves >= 2).  Host and device
// compute the same split.
struct QkvSplit {
    int nw[3];
};
__host__ __device__ inline QkvSplit qkv_split(int nwaves, int n_q, int n_kv, int no_v = 0) {
    const int nm = no_v ? 2 : 3;
    const long n = (long)n_q + (long)(nm - 1) * n_kv;
    int q = (int)(((long)nwaves * n_q + n / 2) / n);
    q = q < 1 ? 1 : (q > nwaves - (nm - 1) ? nwaves - (nm - 1) : q);
    const int k = no_v ? nwaves - q : (nwaves - q) / 2;
    return QkvSplit{{q, k, nwaves - q - k}};
}
// Largest number of rows one wave owns (its LDS result slots).
__host__ __device__ inline int qkv_max_rows(const QkvSplit& sp, int n_q, int n_kv) {
    const int a = (n_q + sp.nw[0] - 1) / sp.nw[0];
    const int b = (n_kv + sp.nw[1] - 1) / sp.nw[1];
    const int c = sp.nw[2] ? (n_kv + sp.nw[2] - 1) / sp.nw[2] : 0;
    return a > b ? (a > c ? a : c) : (b > c ? b : c);
}

// Q8-inline LDS rule of the reference launchers (q4_k_q8_inline.hip:374-378):
// (K/32) * 34 bytes <= 32 KB.  Kept so callers see identical validation.
static inline bool q8_inline_fits(int K) { return (size_t)(K / 32) * 34 <= 32768; }

__host__ __device__ inline size_t q8_lds_bytes(int K) { return (size_t)q8_padded_bytes(K) + (size_t)(K / 32) * 8; }

__device__ __forceinline__ Q8Lds q8_lds_carve(uint8_t* smem, int K) {
    Q8Lds l;
    l.qs = reinterpret_cast<int8_t*>(smem);
    l.xd = reinterpret_cast<float*>(smem + q8_padded_bytes(K));
    l.qsum = reinterpret_cast<int*>(smem + q8_padded_bytes(K) + 4 * (K / 32));
    return l;
}

// One row step of one matrix for one lane: the unit's two sub-blocks
// against the Q8 slab.
__device__ __forceinline__ float q4k_q8_unit_dot(const Q4KUnit& u, int p, const u32x4 xlo[2], const u32x4 xhi[2],
                                                 float xd0, float xd1, int qs0, int qs1, float acc) {
    int dlo, dhi;
    q4k_int_dots(u, xlo, xhi, &dlo, &dhi);
    const float d = half_bits_to_float(u.hdr.x);
    const float dmin = half_bits_to_float(u.hdr.x >> 16);
    int sc0, m0, sc1, m1;
    q4k_scale_min_pair(u.hdr.y, u.hdr.z, u.hdr.w, p, &sc0, &m0, &sc1, &m1);
    acc = q4k_q8_combine(acc, xd0, d, dmin, sc0, m0, dlo, qs0);
    acc = q4k_q8_combine(acc, xd1, d, dmin, sc1, m1, dhi, qs1);
    return acc;
}

// ONE: K <= 4096 (a row group is one pipeline step), so the step -> (row
// group, K slice) split needs no division and every step ends a group.
// Workgroup bid of nblk (the kernel below passes blockIdx.x, gridDim.x);
// smem is the dynamic LDS block.
template <int MODE, int R, int NW, int NB, bool ONE>
__device__ __forceinline__ void q4k_q8_gemv_wg(const uint8_t* __restrict__ w0, const uint8_t* __restrict__ w1,
                                               const float* __restrict__ x, const float* residual, float* y, int K,
                                               int N, const QkvArgs& qkv, int bid, int nblk, uint8_t* smem) {
    const Q8Lds q8 = q8_lds_carve(smem, K);
    constexpr int M = (MODE == kGateUp) ? 2 : 1;

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // wave-uniform (SGPR)
    const int s = lane >> 2;
    const int p = lane & 3;
    const int nsb = K / kQK;
    const size_t row_bytes = (size_t)nsb * kQ4KBytes;
    const int nwaves = nblk * NW;
    // Rows are dealt out round-robin: global wave gw owns rows gw, gw+nwaves,
    // ...  All waves of the grid then stream neighbouring rows at the same
    // time, which keeps the open DRAM pages few (measured: an interleaved
    // read of 64 MB runs ~12% faster than per-wave contiguous stretches).
    const int gw = bid * NW + wave;
    int rstride = nwaves, rfirst = gw, nrows_of = N, max_rows = (N + nwaves - 1) / nwaves;
    const uint8_t* wm = w0;
    float* ym = y;
    const float* bm = nullptr;
    if constexpr (MODE == kQkv) {
        // this wave's matrix and its rank among the waves on that matrix
        const QkvSplit sp = qkv_split(nwaves, qkv.n_q, qkv.n_kv, qkv.no_v);
        // (selects, not indexing: a runtime index into the argument arrays
        // would put them in scratch memory)
        const int m = gw < sp.nw[0] ? 0 : (gw < sp.nw[0] + sp.nw[1] ? 1 : 2);
        const int w_first = m == 0 ? 0 : (m == 1 ? sp.nw[0] : sp.nw[0] + sp.nw[1]);
        rfirst = gw - w_first;
        rstride = m == 0 ? sp.nw[0] : (m == 1 ? sp.nw[1] : sp.nw[2]);
        nrows_of = m == 0 ? qkv.n_q : qkv.n_kv;
        max_rows = qkv_max_rows(sp, qkv.n_q, qkv.n_kv);
        wm = m == 0 ? qkv.w[0] : (m == 1 ? qkv.w[1] : qkv.w[2]);
        ym = m == 0 ? qkv.y[0] : (m == 1 ? qkv.y[1] : qkv.y[2]);
        bm = m == 0 ? qkv.bias[0] : (m == 1 ? qkv.bias[1] : qkv.bias[2]);
    }
    const int nrows = rfirst < nrows_of ? (nrows_of - 1 - rfirst) / rstride + 1 : 0;

    const int spr = ONE ? 1 : (nsb + kSbPerStep - 1) / kSbPerStep;   // steps per row group
    const int nsteps = ((nrows + R - 1) / R) * spr;
    auto row_of = [&](int j) { return nrows ? rfirst + min(j, nrows - 1) * rstride : 0; };
    auto load = [&](Q4KUnit (&u)[M][R], int i) {
        const int sb = min((ONE ? 0 : i % spr) * kSbPerStep + s, nsb - 1);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const size_t off = (size_t)row_of((ONE ? i : i / spr) * R + r) * row_bytes + (size_t)sb * kQ4KBytes;
            u[0][r] = q4k_load_unit(wm + off, p);
            if (M == 2) u[M - 1][r] = q4k_load_unit(w1 + off, p);
        }
    };
    float acc[M][R];
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) acc[m][r] = 0.0f;
    // Row results are parked in this wave's LDS slots and written to HBM
    // after the loop: no global store (or residual load) sits between the
    // prefetch loads in the in-order memory counter.
    // [row][matrix][16-lane row of the wave]
    float* out_lds = reinterpret_cast<float*>(smem + q8_lds_bytes(K)) + wave * max_rows * M * 4;
    auto process = [&](const Q4KUnit (&u)[M][R], int i) {
        const int j0 = (ONE ? i : i / spr) * R;
        const int sb = (ONE ? 0 : i % spr) * kSbPerStep + s;
        const bool live = sb < nsb;
        const int sbc = live ? sb : nsb - 1;
        // Q8 slab for this lane: 64 int8 at element sb*256 + 64p.
        const u32x4* xs = reinterpret_cast<const u32x4*>(q8.qs + q8_pad(sbc * kQK) + 64 * p);
        const u32x4 xlo[2] = {xs[0], xs[1]};
        const u32x4 xhi[2] = {xs[2], xs[3]};
        const int b0 = sbc * 8 + 2 * p;
        const float xd0 = q8.xd[b0], xd1 = q8.xd[b0 + 1];
        const int qs0 = q8.qsum[b0], qs1 = q8.qsum[b0 + 1];
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float a = q4k_q8_unit_dot(u[m][r], p, xlo, xhi, xd0, xd1, qs0, qs1, acc[m][r]);
                acc[m][r] = live ? a : acc[m][r];
            }
        if (ONE || (i % spr) == spr - 1) {  // row group finished: reduce into the wave's LDS slots
#pragma unroll
            for (int r = 0; r < R; ++r) {
                // per-16-lane sums only; the four are added after the loop
                // (same association as wave_sum: (r0 + r1) + (r2 + r3))
                const float g = row16_sum(acc[0][r]);
                const float v = (M == 2) ? row16_sum(acc[M - 1][r]) : 0.0f;
                const int j = j0 + r;
                if ((lane & 15) == 0 && j < nrows) {
                    out_lds[4 * M * j + (lane >> 4)] = g;
                    if (M == 2) out_lds[4 * (M * j + 1) + (lane >> 4)] = v;
                }
#pragma unroll
                for (int m = 0; m < M; ++m) acc[m][r] = 0.0f;
            }
        }
    };

    struct Step {
        Q4KUnit u[M][R];
    };
    // x is loaded before the weight prefetch: loads complete in issue
    // order, so the quantisation then waits only for x, not for the weights
    X8Batch xb, nb;
    q8_prefetch(x, K, xb);
    const float* nw = qkv.norm_w;
    if (nw) q8_prefetch(nw, K, nb);     // norm weights with x, ahead of the weight prefetch
    __shared__ float red[4];
    Step ring[NB];
    ring_pipeline<NB>(nsteps, ring, [&](Step& b, int i) { load(b.u, i); },
                      [&](const Step& b, int i) { process(b.u, i); },
                      [&]() {
                          const float inv = nw ? rms_inv_from_batch(xb, x, K, qkv.eps, red) : 1.0f;
                          q8_quantize_finish(x, K, q8, xb, nw, &nb, inv);
                          __syncthreads();
                      });
    for (int j = lane; j < nrows; j += kWave) {
        const int row = rfirst + j * rstride;
        auto sum4 = [&](int s4) {
            return (out_lds[s4] + out_lds[s4 + 1]) + (out_lds[s4 + 2] + out_lds[s4 + 3]);
        };
        const float g = sum4(4 * M * j);
        if (MODE == kPlain) {
            y[row] = g;
        } else if (MODE == kResidual) {
            y[row] = g + residual[row];
        } else if (MODE == kQkv) {
            ym[row] = g + (bm ? bm[row] : 0.0f);
        } else {
            y[row] = g / (1.0f + expf(-g)) * sum4(4 * (M * j + 1));
        }
    }
}

template <int MODE, int R, int NW, int NB, bool ONE = false>
__global__ __launch_bounds__(NW * 64) void rf_q4k_q8_gemv_kernel(const uint8_t* __restrict__ w0,
                                                                   const uint8_t* __restrict__ w1,
                                                                   const float* __restrict__ x,
                                                                   const float* residual, float* y, int K, int N,
                                                                   QkvArgs qkv) {
    extern __shared__ __align__(16) uint8_t smem[];
    q4k_q8_gemv_wg<MODE, R, NW, NB, ONE>(w0, w1, x, residual, y, K, N, qkv, blockIdx.x, gridDim.x, smem);
}

// Q4_K Q and K with a Q6_K V, RMSNorm folded in, one launch: workgroups
// [0, gv) are teams of the K-split Q6_K GEMV (q6k_lin.h: 4 / nwk teams of
// nwk = K / 2048 waves each, team t of the grid taking V rows t, t + teams,
// ..), the rest run the fused Q8-inline Q/K GEMV over Q and K.  Each output
// has the bits of its own launcher (rf_gemv_q4_k_q8_rmsnorm_launch,
// rf_gemv_q6_k_rmsnorm_launch).  LDS: the larger of the two layouts.
struct Q6VArgs {
    const uint8_t* w;
    const float* bias;
    float* y;
    int n;      // V rows
    int gv;     // workgroups on V
};

template <bool ONE>
__global__ __launch_bounds__(256) void rf_qkv_q4k_q6v_kernel(const float* __restrict__ x, int K, QkvArgs qkv,
                                                             Q6VArgs v) {
    extern __shared__ __align__(16) uint8_t smem[];
    if ((int)blockIdx.x < v.gv) {
        const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
        const int nwk = K / 2048;
        const int tpw = 4 / nwk;                          // teams per workgroup
        const int team = wave / nwk;
        __shared__ float red[4];
        const float inv = rms_inv_canonical(x, K, qkv.eps, red);
        const int G = v.gv * tpw;
        const int g = (int)blockIdx.x * tpw + team;
        const int rows = (v.n + G - 1) / G;
        float* part = reinterpret_cast<float*>(smem + 4 * 2048) + team * rows * nwk * 4;
        q6_lin_team<kQ6Ring>(v.w, x, v.bias, v.y, K, v.n, qkv.norm_w, inv, g, G, wave % nwk, nwk,
                                smem + wave * 2048, part);
        return;
    }
    q4k_q8_gemv_wg<kQkv, 2, 4, 3, ONE>(qkv.w[0], nullptr, x, nullptr, nullptr, K, qkv.n_q + qkv.n_kv, qkv,
                                        (int)blockIdx.x - v.gv, (int)gridDim.x - v.gv, smem);
}

// ── FP32-activation family (q4_k_gemv.hip) ───────────────────────────────
// value = d*sc*nib - dmin*m (fp32, q4_k_gemv.hip:60-71), times x from LDS.
// Same lane tiling as the Q8 kernel; x is staged in LDS as fp32 when it
// fits (K*4 <= 64 KB), otherwise read through L2 directly.
template <bool LDS>
__device__ __forceinline__ float q4k_f32_unit_dot(const Q4KUnit& u, int p, const float* xb, float acc) {
    const float d = half_bits_to_float(u.hdr.x);
    const float dmin = half_bits_to_float(u.hdr.x >> 16);
    int sc0, m0, sc1, m1;
    q4k_scale_min_pair(u.hdr.y, u.hdr.z, u.hdr.w, p, &sc0, &m0, &sc1, &m1);
    const float ds0 = d * (float)sc0, dm0 = dmin * (float)m0;
    const float ds1 = d * (float)sc1, dm1 = dmin * (float)m1;
    const uint32_t w[8] = {u.qa.x, u.qa.y, u.qa.z, u.qa.w, u.qb.x, u.qb.y, u.qb.z, u.qb.w};
    const float4* xl = reinterpret_cast<const float4*>(xb);
    const float4* xh = reinterpret_cast<const float4*>(xb + 32);
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        const float4 a = xl[t];
        const float4 b = xh[t];
        const uint32_t v = w[t];
        acc += (ds0 * (float)((v >> 0) & 15) - dm0) * a.x;
        acc += (ds0 * (float)((v >> 8) & 15) - dm0) * a.y;
        acc += (ds0 * (float)((v >> 16) & 15) - dm0) * a.z;
        acc += (ds0 * (float)((v >> 24) & 15) - dm0) * a.w;
        acc += (ds1 * (float)((v >> 4) & 15) - dm1) * b.x;
        acc += (ds1 * (float)((v >> 12) & 15) - dm1) * b.y;
        acc += (ds1 * (float)((v >> 20) & 15) - dm1) * b.z;
        acc += (ds1 * (float)((v >> 28) & 15) - dm1) * b.w;
    }
    return acc;
}

template <int MODE, int R, bool LDS>
__global__ __launch_bounds__(kThreads) void rf_q4k_f32_gemv_kernel(const uint8_t* __restrict__ w0,
                                                                    const uint8_t* __restrict__ w1,
                                                                    const float* __restrict__ x,
                                                                    const float* residual, float* y, int K, int N) {
    extern __shared__ __align__(16) uint8_t smem[];
    float* xs = reinterpret_cast<float*>(smem);
    constexpr int M = (MODE == kGateUp) ? 2 : 1;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // wave-uniform (SGPR)
    const int s = lane >> 2;
    const int p = lane & 3;
    const int nsb = K / kQK;
    const size_t row_bytes = (size_t)nsb * kQ4KBytes;
    int row_begin, row_end;
    wave_row_range(N, blockIdx.x * kWavesPerWg + wave, gridDim.x * kWavesPerWg, &row_begin, &row_end);

    if (LDS) {
        stage_f32_to_lds(x, K, xs);
        __syncthreads();
    }
    const float* xv = LDS ? xs : x;

    for (int row0 = row_begin; row0 < row_end; row0 += R) {
        float acc[M][R];
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
            for (int r = 0; r < R; ++r) acc[m][r] = 0.0f;
        for (int sb0 = 0; sb0 < nsb; sb0 += kSbPerStep) {
            const int sb = sb0 + s;
            if (sb < nsb) {
                const float* xb = xv + sb * kQK + 64 * p;
                Q4KUnit u[M][R];
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const int row = min(row0 + r, row_end - 1);
                    u[0][r] = q4k_load_unit(w0 + (size_t)row * row_bytes + (size_t)sb * kQ4KBytes, p);
                    if (MODE == kGateUp)
                        u[M - 1][r] = q4k_load_unit(w1 + (size_t)row * row_bytes + (size_t)sb * kQ4KBytes, p);
                }
#pragma unroll
                for (int m = 0; m < M; ++m)
#pragma unroll
                    for (int r = 0; r < R; ++r) acc[m][r] = q4k_f32_unit_dot<LDS>(u[m][r], p, xb, acc[m][r]);
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float g = wave_sum(acc[0][r]);
            const float v = (M == 2) ? wave_sum(acc[M - 1][r]) : 0.0f;
            const int row = row0 + r;
            if (lane == r && row < row_end) {
                if (MODE == kPlain) y[row] = g;
                else if (MODE == kResidual) y[row] = g + residual[row];
                else y[row] = g / (1.0f + expf(-g)) * v;
            }
        }
    }
}

// ── K-split Q4_K Q8-inline GEMV for long rows (K >= 8192, K / 256 % 16 == 0) ──
// A team of nwk = K / 4096 waves per workgroup; team wave tw takes
// super-blocks [16 tw, 16 tw + 16) of every row (lane 4 s + p: super-block
// 16 tw + s, nibble pair p, as in the one-row-per-step kernel) for the rows
// g, g + G, .. (< N) of workgroup g of G.  Each lane owns the 64 elements of
// x its nibble pair meets -- two whole Q8_0 blocks -- and quantises them in
// registers (the quantiser's arithmetic, with no cross-lane step), so the
// weight stream runs with no LDS traffic and no barrier in front of it.  A
// row's sum is the team's 4 nwk 16-lane partial sums added in team-wave
// order after the loop, the same whatever the grid.  norm_w (optional):
// x -> (x * inv) * norm_w first, inv in the canonical order of the
// standalone norm (same bits as gpu_rms_norm then the plain launch).
template <int NB>
__global__ __launch_bounds__(512) void rf_q4k_q8_lin_kernel(const uint8_t* __restrict__ w,
                                                             const float* __restrict__ x, const float* residual,
                                                             float* y, int K, int N,
                                                             const float* __restrict__ norm_w, float eps) {
    extern __shared__ __align__(16) float part[];   // [rows of this workgroup][nwk][4]
    __shared__ float red[4];
    const int lane = threadIdx.x & (kWave - 1);
    const int tw = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int nwk = blockDim.x / kWave;
    const int nsb = K / kQK;
    const size_t row_bytes = (size_t)nsb * kQ4KBytes;
    const int s = lane >> 2, p = lane & 3;
    const int sb = 16 * tw + s;
    const int g = blockIdx.x, G = gridDim.x;
    const int nrows = g < N ? (N - 1 - g) / G + 1 : 0;
    const float inv_rms = norm_w ? rms_inv_canonical(x, K, eps, red) : 1.0f;

    // x: elements sb * 256 + 64 p .. + 63 = Q8_0 blocks 8 sb + 2 p, + 1
    u32x4 xlo[2], xhi[2];
    float xd[2];
    int xq[2];
    {
        const float4* xv = reinterpret_cast<const float4*>(x + (size_t)sb * kQK + 64 * p);
        float4 v[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = xv[i];
        if (norm_w) {
            const float4* gv = reinterpret_cast<const float4*>(norm_w + (size_t)sb * kQK + 64 * p);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float4 gg = gv[i];
                v[i] = make_float4((v[i].x * inv_rms) * gg.x, (v[i].y * inv_rms) * gg.y, (v[i].z * inv_rms) * gg.z,
                                   (v[i].w * inv_rms) * gg.w);
            }
        }
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            float e[32];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                e[4 * i] = v[8 * b + i].x; e[4 * i + 1] = v[8 * b + i].y;
                e[4 * i + 2] = v[8 * b + i].z; e[4 * i + 3] = v[8 * b + i].w;
            }
            float amax = 0.0f;
#pragma unroll
            for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(e[i]));
            const float scale = fmaxf(amax / 127.0f, 1e-30f);
            const float sf = __half2float(__float2half(scale));
            const float inv = 1.0f / sf;
            uint32_t packed[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
            int sum = 0;
#pragma unroll
            for (int i = 0; i < 32; ++i) {
                const int q = (int)fminf(fmaxf(e[i] * inv, -127.0f), 127.0f);
                sum += q;
                packed[i >> 2] |= ((uint32_t)q & 0xFFu) << (8 * (i & 3));
            }
            u32x4* dst = b ? xhi : xlo;
            dst[0] = u32x4{packed[0], packed[1], packed[2], packed[3]};
            dst[1] = u32x4{packed[4], packed[5], packed[6], packed[7]};
            xd[b] = sf;
            xq[b] = sum;
        }
    }
    const uint8_t* wl = w + (size_t)sb * kQ4KBytes;
    auto load = [&](Q4KUnit& u, int j) {
        const int row = nrows ? g + min(j, nrows - 1) * G : 0;
        u = q4k_load_unit(wl + (size_t)row * row_bytes, p);
    };
    auto process = [&](const Q4KUnit& u, int j) {
        const float acc = q4k_q8_unit_dot(u, p, xlo, xhi, xd[0], xd[1], xq[0], xq[1], 0.0f);
        const float r16 = row16_sum(acc);
        if ((lane & 15) == 0) part[(j * nwk + tw) * 4 + (lane >> 4)] = r16;
    };
    Q4KUnit ring[NB];
    ring_pipeline<NB>(nrows, ring, load, process, [&]() {});
    __syncthreads();
    for (int j = tw * kWave + lane; j < nrows; j += nwk * kWave) {
        float t = 0.0f;
        for (int k = 0; k < 4 * nwk; ++k) t += part[j * nwk * 4 + k];
        y[g + j * G] = t + (residual ? residual[g + j * G] : 0.0f);
    }
}

// ── launch helpers ────────────────────────────────────────────────────────
// Grid: a fixed number of workgroups per CU (every wave then streams an
// equal contiguous share of the rows), fewer when N is too small to give each
// wave at least `min_rows` rows.
static inline int gemv_grid(int N, int min_rows) {
    const int cap = device_cu_count() * 2;
    const int need = (N + kWavesPerWg * min_rows - 1) / (kWavesPerWg * min_rows);
    return need < cap ? need : cap;
}

template <int MODE>
static hipError_t launch_q8(const void* w0, const void* w1, const float* x, const float* res, float* y, int K, int N,
                            hipStream_t st, const QkvArgs& qkv = QkvArgs{}) {
    constexpr int M = (MODE == kGateUp) ? 2 : 1;
    // One workgroup of four waves per CU, each lane streaming two weight
    // units per step: two matrices (gate+up) or two rows of one matrix.
    // Measured on MI355X against 2 workgroups per CU / 1 row per step:
    // gate+up 14336x4096 12.9 vs 14.1 us, 6144x4096 5.1 vs 5.45 us,
    // 4096x4096 + residual 4.7 vs 5.1 us, 14336x4096 8.0 vs 8.1 us.
    // a fused RMSNorm needs 256-thread workgroups (its summation order)
    const int r = MODE == kGateUp ? 1 : 2;
    constexpr int nw = 4;
    const int cap = device_cu_count();
    const int need = (N + nw - 1) / nw;
    const int grid = need < cap ? need : cap;
    // result slots per wave: its largest row count
    const size_t wave_rows = MODE == kQkv ? (size_t)qkv_max_rows(qkv_split(grid * nw, qkv.n_q, qkv.n_kv), qkv.n_q,
                                                                  qkv.n_kv)
                                          : (N + (size_t)grid * nw - 1) / ((size_t)grid * nw);
    const size_t out_bytes = (size_t)nw * wave_rows * M * 4 * sizeof(float);
    if (q8_lds_bytes(K) + out_bytes > 160 * 1024) return hipErrorInvalidValue;
    const uint8_t* a = static_cast<const uint8_t*>(w0);
    const uint8_t* b = static_cast<const uint8_t*>(w1);
    const size_t lds = q8_lds_bytes(K) + out_bytes;
    auto go = [&](auto one) {
        constexpr bool ONE = decltype(one)::value;
        if (r == 1)
            hipLaunchKernelGGL((rf_q4k_q8_gemv_kernel<MODE, 1, 4, kRingDepth, ONE>), dim3(grid), dim3(4 * 64), lds, st,
                               a, b, x, res, y, K, N, qkv);
        else
            hipLaunchKernelGGL((rf_q4k_q8_gemv_kernel<MODE, 2, 4, 3, ONE>), dim3(grid), dim3(4 * 64), lds, st, a, b, x,
                               res, y, K, N, qkv);
    };
    // the division-free variant for single matrices only: measured on
    // MI355X it takes QKV 6144x4096 from 5.16 to 4.82 us, but the fused
    // gate+up (two matrices) from 12.6 to 13.0 us
    if (K / kQK <= kSbPerStep && MODE != kGateUp)
        go(std::true_type{});
    else
        go(std::false_type{});
    return hipGetLastError();
}

template <int MODE>
static hipError_t launch_f32(const void* w0, const void* w1, const float* x, const float* res, float* y, int K, int N,
                             hipStream_t st) {
    constexpr int R = (MODE == kGateUp) ? 2 : 4;
    const int grid = gemv_grid(N, 1);
    const size_t lds = (size_t)K * sizeof(float);
    if (lds <= 65536) {
        hipLaunchKernelGGL((rf_q4k_f32_gemv_kernel<MODE, R, true>), dim3(grid), dim3(kThreads), lds, st,
                           static_cast<const uint8_t*>(w0), static_cast<const uint8_t*>(w1), x, res, y, K, N);
    } else {
        hipLaunchKernelGGL((rf_q4k_f32_gemv_kernel<MODE, R, false>), dim3(grid), dim3(kThreads), 0, st,
                           static_cast<const uint8_t*>(w0), static_cast<const uint8_t*>(w1), x, res, y, K, N);
    }
    return hipGetLastError();
}

// ── debug / parity entry points (same device code as the GEMV) ───────────
// Each workgroup quantises a slice of kQuantSlice elements with the GEMV's
// own LDS quantiser and copies the LDS image out.
constexpr int kQuantSlice = 8192;
__global__ __launch_bounds__(kThreads) void rf_q8_0_quantize_kernel(const float* __restrict__ x, int K,
                                                                     uint16_t* __restrict__ d_out,
                                                                     int8_t* __restrict__ qs_out,
                                                                     int* __restrict__ sum_out) {
    __shared__ __align__(16) uint8_t smem[q8_padded_bytes(kQuantSlice) + kQuantSlice / 4];
    const int base = blockIdx.x * kQuantSlice;
    const int len = min(kQuantSlice, K - base);
    const Q8Lds q8 = q8_lds_carve(smem, len);
    q8_0_quantize_to_lds(x + base, len, q8);
    __syncthreads();
    for (int i = threadIdx.x; i < len; i += kThreads) qs_out[base + i] = q8.qs[q8_pad(i)];
    for (int b = threadIdx.x; b < len / 32; b += kThreads) {
        d_out[base / 32 + b] = __half_as_ushort(__float2half(q8.xd[b]));
        sum_out[base / 32 + b] = q8.qsum[b];
    }
}

// int_dot[row*(K/32) + sub-block] for every row and sub-block, computed
// with the GEMV's own load/unpack/dot path.
__global__ __launch_bounds__(kThreads) void rf_q4k_q8_partials_kernel(const uint8_t* __restrict__ w,
                                                                       const float* __restrict__ x,
                                                                       int* __restrict__ int_dot, int K, int N) {
    extern __shared__ __align__(16) uint8_t smem[];
    const Q8Lds q8 = q8_lds_carve(smem, K);
    q8_0_quantize_to_lds(x, K, q8);
    __syncthreads();
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // wave-uniform (SGPR)
    const int s = lane >> 2, p = lane & 3;
    const int nsb = K / kQK;
    for (int row = blockIdx.x * kWavesPerWg + wave; row < N; row += gridDim.x * kWavesPerWg) {
        for (int sb0 = 0; sb0 < nsb; sb0 += kSbPerStep) {
            const int sb = sb0 + s;
            if (sb < nsb) {
                const u32x4* xs = reinterpret_cast<const u32x4*>(q8.qs + q8_pad(sb * kQK) + 64 * p);
                u32x4 xlo[2] = {xs[0], xs[1]};
                u32x4 xhi[2] = {xs[2], xs[3]};
                Q4KUnit u = q4k_load_unit(w + ((size_t)row * nsb + sb) * kQ4KBytes, p);
                int dlo, dhi;
                q4k_int_dots(u, xlo, xhi, &dlo, &dhi);
                int_dot[(size_t)row * (K / 32) + sb * 8 + 2 * p] = dlo;
                int_dot[(size_t)row * (K / 32) + sb * 8 + 2 * p + 1] = dhi;
            }
        }
    }
}

}  // namespace rf

using namespace rf;

static inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Shape/pointer validation of the reference launchers
// (q4_k_q8_inline.hip:388-390, 413-415, 438-443; q4_k_gemv.hip:489-493,
// 525-526, 556-557).  Additionally the weights must be 16-byte aligned: the
// kernels stream them with 16-byte loads (GGUF tensors are uploaded into
// their own hipMalloc buffers, which are 256-byte aligned).
// The K-split kernel for long rows: K a multiple of 4096 from 8192 (the
// launchers' Q8 LDS rule caps K at 30720), 16-byte aligned weights and x.
// One workgroup per CU, three rows in flight per wave (measured on MI355X,
// 4096 x 12288 + residual: 8.4-8.5 us against 9.1-9.4 for the one-row-per-step
// kernel; two workgroups per CU 10.1, two rows in flight 11.1).
constexpr int kQ4LinRing = 4;
static bool q4_lin_ok(const void* w, const float* x, int K) {
    return K >= 8192 && K % 4096 == 0 && ((reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(x)) & 15u) == 0;
}
static hipError_t launch_q4_lin(const void* w, const float* x, const float* res, float* y, int K, int N,
                                hipStream_t st, const float* norm_w = nullptr, float eps = 0.0f) {
    const int nwk = K / 4096;
    const int cap = device_cu_count();
    const int grid = N < cap ? N : cap;
    const size_t lds = (size_t)((N + grid - 1) / grid) * nwk * 4 * sizeof(float);
    if (lds > 64 * 1024) return hipErrorInvalidValue;
    hipLaunchKernelGGL((rf_q4k_q8_lin_kernel<kQ4LinRing>), dim3(grid), dim3(nwk * 64), lds, st,
                       static_cast<const uint8_t*>(w), x, res, y, K, N, norm_w, eps);
    return hipGetLastError();
}

extern "C" hipError_t gemv_q4_k_f32_q8_inline_launch(const void* weights_q4_k, const float* input, float* output,
                                                     int n_rows, int ncols_dst, hipStream_t stream) {
    if (n_rows <= 0 || ncols_dst <= 0) return hipErrorInvalidValue;
    if ((n_rows % kQK) != 0) return hipErrorInvalidValue;
    if (!q8_inline_fits(n_rows)) return hipErrorInvalidValue;
    if (!aligned16(weights_q4_k)) return hipErrorInvalidValue;
    if (q4_lin_ok(weights_q4_k, input, n_rows))
        return launch_q4_lin(weights_q4_k, input, nullptr, output, n_rows, ncols_dst, stream);
    return launch_q8<kPlain>(weights_q4_k, nullptr, input, nullptr, output, n_rows, ncols_dst, stream);
}

extern "C" hipError_t gemv_q4_k_f32_q8_inline_residual_launch(const void* weights_q4_k, const float* input,
                                                              const float* residual, float* output, int n_rows,
                                                              int ncols_dst, hipStream_t stream) {
    if (n_rows <= 0 || ncols_dst <= 0 || residual == nullptr) return hipErrorInvalidValue;
    if ((n_rows % kQK) != 0) return hipErrorInvalidValue;
    if (!q8_inline_fits(n_rows)) return hipErrorInvalidValue;
    if (!aligned16(weights_q4_k)) return hipErrorInvalidValue;
    if (q4_lin_ok(weights_q4_k, input, n_rows))
        return launch_q4_lin(weights_q4_k, input, residual, output, n_rows, ncols_dst, stream);
    return launch_q8<kResidual>(weights_q4_k, nullptr, input, residual, output, n_rows, ncols_dst, stream);
}

extern "C" hipError_t gemv_gate_up_swiglu_q4_k_f32_q8_inline_launch(const void* weights_gate_q4_k,
                                                                    const void* weights_up_q4_k, const float* input,
                                                                    float* swiglu_out, int n_rows, int ncols_dst,
                                                                    hipStream_t stream) {
    if (n_rows <= 0 || ncols_dst <= 0) return hipErrorInvalidValue;
    if ((n_rows % kQK) != 0) return hipErrorInvalidValue;
    if (weights_gate_q4_k == nullptr || weights_up_q4_k == nullptr) return hipErrorInvalidValue;
    if (!q8_inline_fits(n_rows)) return hipErrorInvalidValue;
    if (!aligned16(weights_gate_q4_k) || !aligned16(weights_up_q4_k)) return hipErrorInvalidValue;
    return launch_q8<kGateUp>(weights_gate_q4_k, weights_up_q4_k, input, nullptr, swiglu_out, n_rows, ncols_dst,
                              stream);
}

// Fused Q/K/V projection: one launch over the three Q4_K matrices with the
// Q8 activations quantised once.  No counterpart for Q4_K in the reference:
// its Q4_K_M attention input takes three GEMV launches (ops.rs:851-853).
// The signature, bias handling (out = dot + bias, bias optional) and size
// arguments follow its Q4_0 fused QKV launcher (q4_0_fused.hip:674-680, :80-86).
extern "C" hipError_t gemv_qkv_q4_k_f32_q8_inline_launch(const void* w_q, const void* w_k, const void* w_v,
                                                         const float* bias_q, const float* bias_k, const float* bias_v,
                                                         const float* input, float* out_q, float* out_k, float* out_v,
                                                         int n_rows, int n_q, int n_kv, hipStream_t stream) {
    if (n_rows <= 0 || n_q <= 0 || n_kv <= 0) return hipErrorInvalidValue;
    if ((n_rows % kQK) != 0) return hipErrorInvalidValue;
    if (w_q == nullptr || w_k == nullptr || w_v == nullptr) return hipErrorInvalidValue;
    if (out_q == nullptr || out_k == nullptr || out_v == nullptr) return hipErrorInvalidValue;
    if (!q8_inline_fits(n_rows)) return hipErrorInvalidValue;
    if (!aligned16(w_q) || !aligned16(w_k) || !aligned16(w_v)) return hipErrorInvalidValue;
    if ((long)n_q + 2L * n_kv > 0x7FFFFFFFL) return hipErrorInvalidValue;
    QkvArgs a{};
    a.w[0] = static_cast<const uint8_t*>(w_q);
    a.w[1] = static_cast<const uint8_t*>(w_k);
    a.w[2] = static_cast<const uint8_t*>(w_v);
    a.bias[0] = bias_q;
    a.bias[1] = bias_k;
    a.bias[2] = bias_v;
    a.y[0] = out_q;
    a.y[1] = out_k;
    a.y[2] = out_v;
    a.n_q = n_q;
    a.n_kv = n_kv;
    return launch_q8<kQkv>(w_q, nullptr, input, nullptr, nullptr, n_rows, n_q + 2 * n_kv, stream, a);
}

// ---- RMSNorm fused into the Q8-inline GEMVs (no reference counterpart) ----
// out = W * rmsnorm(input, norm_w, eps): the same bits as gpu_rms_norm into a
// buffer followed by the plain launcher, one launch instead of two (the
// reference runs gpu_dispatch_rms_norm before each of these GEMVs,
// src/gpu/forward.rs:2349-2359, :2454-2464).  input and norm_w 16-byte aligned.
static bool norm_args_ok(const float* x, const float* nw) {
    return x != nullptr && nw != nullptr && aligned16(x) && aligned16(nw);
}

extern "C" hipError_t rf_gemv_q4_k_q8_rmsnorm_launch(const void* weights_q4_k, const float* input,
                                                     const float* norm_w, float eps, float* output, int n_rows,
                                                     int ncols_dst, hipStream_t stream) {
    if (n_rows <= 0 || ncols_dst <= 0 || (n_rows % kQK) != 0 || !q8_inline_fits(n_rows)) return hipErrorInvalidValue;
    if (!aligned16(weights_q4_k) || !norm_args_ok(input, norm_w)) return hipErrorInvalidValue;
    if (q4_lin_ok(weights_q4_k, input, n_rows))
        return launch_q4_lin(weights_q4_k, input, nullptr, output, n_rows, ncols_dst, stream, norm_w, eps);
    QkvArgs a{};
    a.norm_w = norm_w;
    a.eps = eps;
    return launch_q8<kPlain>(weights_q4_k, nullptr, input, nullptr, output, n_rows, ncols_dst, stream, a);
}

extern "C" hipError_t rf_gemv_gate_up_q4_k_q8_rmsnorm_launch(const void* weights_gate_q4_k,
                                                             const void* weights_up_q4_k, const float* input,
                                                             const float* norm_w, float eps, float* swiglu_out,
                                                             int n_rows, int ncols_dst, hipStream_t stream) {
    if (n_rows <= 0 || ncols_dst <= 0 || (n_rows % kQK) != 0 || !q8_inline_fits(n_rows)) return hipErrorInvalidValue;
    if (weights_gate_q4_k == nullptr || weights_up_q4_k == nullptr) return hipErrorInvalidValue;
    if (!aligned16(weights_gate_q4_k) || !aligned16(weights_up_q4_k) || !norm_args_ok(input, norm_w))
        return hipErrorInvalidValue;
    QkvArgs a{};
    a.norm_w = norm_w;
    a.eps = eps;
    return launch_q8<kGateUp>(weights_gate_q4_k, weights_up_q4_k, input, nullptr, swiglu_out, n_rows, ncols_dst,
                              stream, a);
}

extern "C" hipError_t rf_gemv_qkv_q4_k_q8_rmsnorm_launch(const void* w_q, const void* w_k, const void* w_v,
                                                         const float* bias_q, const float* bias_k, const float* bias_v,
                                                         const float* input, const float* norm_w, float eps,
                                                         float* out_q, float* out_k, float* out_v, int n_rows, int n_q,
                                                         int n_kv, hipStream_t stream) {
    if (n_rows <= 0 || n_q <= 0 || n_kv <= 0 || (n_rows % kQK) != 0 || !q8_inline_fits(n_rows))
        return hipErrorInvalidValue;
    if (w_q == nullptr || w_k == nullptr || w_v == nullptr) return hipErrorInvalidValue;
    if (out_q == nullptr || out_k == nullptr || out_v == nullptr) return hipErrorInvalidValue;
    if (!aligned16(w_q) || !aligned16(w_k) || !aligned16(w_v) || !norm_args_ok(input, norm_w))
        return hipErrorInvalidValue;
    if ((long)n_q + 2L * n_kv > 0x7FFFFFFFL) return hipErrorInvalidValue;
    QkvArgs a{};
    a.w[0] = static_cast<const uint8_t*>(w_q);
    a.w[1] = static_cast<const uint8_t*>(w_k);
    a.w[2] = static_cast<const uint8_t*>(w_v);
    a.bias[0] = bias_q;
    a.bias[1] = bias_k;
    a.bias[2] = bias_v;
    a.y[0] = out_q;
    a.y[1] = out_k;
    a.y[2] = out_v;
    a.n_q = n_q;
    a.n_kv = n_kv;
    a.norm_w = norm_w;
    a.eps = eps;
    return launch_q8<kQkv>(w_q, nullptr, input, nullptr, nullptr, n_rows, n_q + 2 * n_kv, stream, a);
}

// Q4_K Q and K with a Q6_K V (the Q4_K_M attention input of the layers
// whose attn_v is Q6_K), RMSNorm folded in, one launch; each output has the
// bits of its own normalising launcher.  No counterpart in the reference
// (three GEMV launches after a norm, src/gpu/ops.rs:851-853).  K (n_rows) in
// {2048, 4096, 8192}; weights, input and norm_w 16-byte aligned.
constexpr int kQkvVRowsPerTeam = 2;     // V rows per Q6_K team

extern "C" hipError_t rf_gemv_qkv_q4_k_q6_k_v_rmsnorm_launch(const void* w_q, const void* w_k, const void* w_v_q6_k,
                                                             const float* bias_q, const float* bias_k,
                                                             const float* bias_v, const float* input,
                                                             const float* norm_w, float eps, float* out_q,
                                                             float* out_k, float* out_v, int n_rows, int n_q,
                                                             int n_kv, hipStream_t stream) {
    if (n_rows <= 0 || n_q <= 0 || n_kv <= 0 || (n_rows % kQK) != 0 || !q8_inline_fits(n_rows))
        return hipErrorInvalidValue;
    const int nsb = n_rows / kQK;
    if (nsb % 8 != 0 || nsb / 8 > 4 || 4 % (nsb / 8) != 0) return hipErrorInvalidValue;
    if (w_q == nullptr || w_k == nullptr || w_v_q6_k == nullptr) return hipErrorInvalidValue;
    if (out_q == nullptr || out_k == nullptr || out_v == nullptr) return hipErrorInvalidValue;
    if (!aligned16(w_q) || !aligned16(w_k) || !aligned16(w_v_q6_k) || !norm_args_ok(input, norm_w))
        return hipErrorInvalidValue;
    if ((long)n_q + (long)n_kv > 0x7FFFFFFFL) return hipErrorInvalidValue;
    QkvArgs a{};
    a.w[0] = static_cast<const uint8_t*>(w_q);
    a.w[1] = static_cast<const uint8_t*>(w_k);
    a.bias[0] = bias_q;
    a.bias[1] = bias_k;
    a.y[0] = out_q;
    a.y[1] = out_k;
    a.n_q = n_q;
    a.n_kv = n_kv;
    a.norm_w = norm_w;
    a.eps = eps;
    a.no_v = 1;
    // Q/K workgroups as launch_q8: four waves, two rows per lane step, at
    // most one workgroup per CU
    const int cap = device_cu_count();
    const int nqk = n_q + n_kv;
    const int gq = (nqk + 3) / 4 < cap ? (nqk + 3) / 4 : cap;
    const size_t wave_rows = (size_t)qkv_max_rows(qkv_split(gq * 4, n_q, n_kv, 1), n_q, n_kv);
    const size_t lds_q = q8_lds_bytes(n_rows) + 4 * wave_rows * 4 * sizeof(float);
    // Q6_K teams of nwk waves, kQkvVRowsPerTeam rows each
    const int nwk = nsb / 8, tpw = 4 / nwk;
    const int teams = (n_kv + kQkvVRowsPerTeam - 1) / kQkvVRowsPerTeam;
    const int gv = (teams + tpw - 1) / tpw;
    const size_t v_rows = (size_t)(n_kv + gv * tpw - 1) / (gv * tpw);
    const size_t lds_v = 4 * 2048 + (size_t)tpw * v_rows * nwk * 4 * sizeof(float);
    const size_t lds = lds_q > lds_v ? lds_q : lds_v;
    if (lds > 64 * 1024) return hipErrorInvalidValue;
    const Q6VArgs v{static_cast<const uint8_t*>(w_v_q6_k), bias_v, out_v, n_kv, gv};
    if (nsb <= kSbPerStep)
        hipLaunchKernelGGL(rf_qkv_q4k_q6v_kernel<true>, dim3(gv + gq), dim3(256), lds, stream, input, n_rows, a, v);
    else
        hipLaunchKernelGGL(rf_qkv_q4k_q6v_kernel<false>, dim3(gv + gq), dim3(256), lds, stream, input, n_rows, a, v);
    return hipGetLastError();
}

extern "C" hipError_t gemv_q4_k_f32_launch(const void* weights_q4_k, const float* input, float* output, int n_rows,
                                           int ncols_dst, hipStream_t stream) {
    if (n_rows <= 0 || ncols_dst <= 0) return hipErrorInvalidValue;
    if ((n_rows % kQK) != 0) return hipErrorInvalidValue;
    if (!aligned16(weights_q4_k)) return hipErrorInvalidValue;
    return launch_f32<kPlain>(weights_q4_k, nullptr, input, nullptr, output, n_rows, ncols_dst, stream);
}

extern "C" hipError_t gemv_q4_k_f32_residual_launch(const void* weights_q4_k, const float* input,
                                                    const float* residual, float* output, int n_rows, int ncols_dst,
                                                    hipStream_t stream) {
    if (n_rows <= 0 || ncols_dst <= 0 || residual == nullptr) return hipErrorInvalidValue;
    if ((n_rows % kQK) != 0) return hipErrorInvalidValue;
    if (!aligned16(weights_q4_k)) return hipErrorInvalidValue;
    return launch_f32<kResidual>(weights_q4_k, nullptr, input, residual, output, n_rows, ncols_dst, stream);
}

extern "C" hipError_t gemv_gate_up_swiglu_q4_k_f32_launch(const void* weights_gate_q4_k, const void* weights_up_q4_k,
                                                          const float* input, float* swiglu_out, int n_rows,
                                                          int ncols_dst, hipStream_t stream) {
    if (n_rows <= 0 || ncols_dst <= 0) return hipErrorInvalidValue;
    if ((n_rows % kQK) != 0) return hipErrorInvalidValue;
    if (weights_gate_q4_k == nullptr || weights_up_q4_k == nullptr) return hipErrorInvalidValue;
    if (!aligned16(weights_gate_q4_k) || !aligned16(weights_up_q4_k)) return hipErrorInvalidValue;
    return launch_f32<kGateUp>(weights_gate_q4_k, weights_up_q4_k, input, nullptr, swiglu_out, n_rows, ncols_dst,
                               stream);
}

// Parity probes: Q8_0 blocks (fp16 bits, int8, int sum) and the per
// sub-block integer dots exactly as the Q8-inline GEMV forms them.
extern "C" hipError_t rf_q8_0_quantize_launch(const float* input, uint16_t* d_out, int8_t* qs_out, int* sum_out,
                                              int n, hipStream_t stream) {
    if (n <= 0 || (n % 32) != 0 || !input || !d_out || !qs_out || !sum_out) return hipErrorInvalidValue;
    const int grid = (n + kQuantSlice - 1) / kQuantSlice;
    hipLaunchKernelGGL(rf_q8_0_quantize_kernel, dim3(grid), dim3(kThreads), 0, stream, input, n, d_out, qs_out,
                       sum_out);
    return hipGetLastError();
}

extern "C" hipError_t rf_q4_k_q8_int_dots_launch(const void* weights_q4_k, const float* input, int* int_dot,
                                                 int n_rows, int ncols_dst, hipStream_t stream) {
    if (n_rows <= 0 || ncols_dst <= 0 || (n_rows % kQK) != 0 || !q8_inline_fits(n_rows)) return hipErrorInvalidValue;
    if (!weights_q4_k || !input || !int_dot || !aligned16(weights_q4_k)) return hipErrorInvalidValue;
    const int grid = gemv_grid(ncols_dst, 1);
    hipLaunchKernelGGL(rf_q4k_q8_partials_kernel, dim3(grid), dim3(kThreads), q8_lds_bytes(n_rows), stream,
                       static_cast<const uint8_t*>(weights_q4_k), input, int_dot, n_rows, ncols_dst);
    return hipGetLastError();
}
