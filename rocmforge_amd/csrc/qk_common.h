// qk_common.h -- device-side building blocks shared by the CDNA4 (gfx950)
// Q4_K / Q6_K GEMV and GEMM kernels.
//
// GGUF block layouts (kept byte-identical to ROCmForge, which uploads raw
// GGUF bytes: src/gpu/weights.rs:415-419):
//   Q4_K  144 B / 256 weights: half d @0, half dmin @2, 12 B packed 6-bit
//         scales/mins @4, 128 B nibbles @16 (pair-interleaved: byte 32k+i
//         holds element 64k+i in its low nibble, 64k+32+i in its high one).
//   Q6_K  210 B / 256 weights: ql[128] @0, qh[64] @128, int8 scales[16]
//         @192, half d @208.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rf {

constexpr int kQK = 256;          // weights per super-block
constexpr int kQ4KBytes = 144;
constexpr int kQ6KBytes = 210;
constexpr int kWave = 64;         // CDNA wavefront

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// 16-byte load with only 2-byte alignment promised.  gfx950 runs with the
// unaligned access mode that ROCm enables, and the backend lowers this to a
// single global_load_dwordx4.
struct __attribute__((packed, aligned(2))) Un16 { u32x4 v; };
struct __attribute__((packed, aligned(2))) Un8 { u32x2 v; };
struct __attribute__((packed, aligned(2))) Un4 { uint32_t v; };

// Buffer resource over [p, p + 4 GiB): raw buffer loads through it take a
// vector byte offset and a scalar byte offset (no per-lane 64-bit address
// arithmetic).  Word 3 is the gfx9 family's raw-buffer format (data format
// 32, no swizzle); no bounds checking is relied on.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, -1, 0x00020000);
}

__device__ __forceinline__ u32x4 ld16(const uint8_t* p) {
    return reinterpret_cast<const Un16*>(p)->v;
}
__device__ __forceinline__ u32x2 ld8(const uint8_t* p) {
    return reinterpret_cast<const Un8*>(p)->v;
}
__device__ __forceinline__ uint32_t ld4(const uint8_t* p) {
    return reinterpret_cast<const Un4*>(p)->v;
}
__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) {
    return *reinterpret_cast<const uint16_t*>(p);
}

__device__ __forceinline__ float half_bits_to_float(uint32_t bits) {
    __half_raw r;
    r.x = (unsigned short)(bits & 0xFFFFu);
    return __half2float(__half(r));
}

// ── cross-lane helpers on DPP (VALU only; no LDS round trips) ───────────
// dpp_ctrl encodings (GFX9): quad_perm(a,b,c,d) = a|b<<2|c<<4|d<<6,
// row_ror:n = 0x120+n, row_bcast:15 = 0x142, row_bcast:31 = 0x143.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
constexpr int kQuadXor1 = 0xB1;  // quad_perm [1,0,3,2]
constexpr int kQuadXor2 = 0x4E;  // quad_perm [2,3,0,1]

// Sum over the 64 lanes of a wave, returned to every lane: rows of 16 are
// reduced with quad permutes and row rotates, rows are combined with
// row_bcast into lane 63, which is read back as a scalar.
// Sum over each 16-lane DPP row: every lane holds its row's sum (the first
// four steps of wave_sum).
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_f<kQuadXor1>(v);
    v += dpp_f<kQuadXor2>(v);
    v += dpp_f<0x124>(v);          // row_ror:4
    v += dpp_f<0x128>(v);          // row_ror:8
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f<kQuadXor1>(v);
    v += dpp_f<kQuadXor2>(v);
    v += dpp_f<0x124>(v);          // row_ror:4
    v += dpp_f<0x128>(v);          // row_ror:8  -> every lane holds its row's sum
    v += dpp_f<0x142, 0xA>(v);     // row_bcast:15 into rows 1, 3
    v += dpp_f<0x143, 0xC>(v);     // row_bcast:31 into rows 2, 3 -> lane 63 holds the total
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Q4_K (scale, min) for sub-blocks 2p and 2p+1, from the three scale words
// (s0 = scales[0..3], s1 = scales[4..7], s2 = scales[8..11]).
// Same bit layout as ggml get_scale_min_k4 (q4_k_q8_inline.hip:49-59):
//   j<4 : sc = s[j]&63,                     m = s[j+4]&63
//   j>=4: sc = (s[j+4]&15) | (s[j-4]>>6)<<4, m = (s[j+4]>>4) | (s[j]>>6)<<4
// With j' = j&3 both cases read byte j' of s0/s1/s2, so the lane-variable
// index turns into shifts and one select instead of a dynamic byte array.
__device__ __forceinline__ void q4k_scale_min_pair(uint32_t s0, uint32_t s1, uint32_t s2, int p,
                                                   int* sc0, int* m0, int* sc1, int* m1) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int jj = (2 * p + h) & 3;
        const uint32_t sh = 8u * (uint32_t)jj;
        const int by = (int)((s0 >> sh) & 0xFFu);
        const int bz = (int)((s1 >> sh) & 0xFFu);
        const int bw = (int)((s2 >> sh) & 0xFFu);
        const bool lo = p < 2;
        const int sc = lo ? (by & 63) : ((bw & 15) | ((by >> 6) << 4));
        const int mn = lo ? (bz & 63) : ((bw >> 4) | ((bz >> 6) << 4));
        if (h == 0) { *sc0 = sc; *m0 = mn; } else { *sc1 = sc; *m1 = mn; }
    }
}

// ── Q8_0 activation quantisation into LDS ────────────────────────────────
// Semantics restated from q4_k_q8_inline.hip:141-161 (bit-exact):
//   amax = max|x| over 32; scale = fmaxf(amax/127, 1e-30); d = half(scale);
//   inv = 1/float(d); q = (int8) trunc(fminf(fmaxf(x*inv, -127), 127)).
// Layout chosen for wave64 consumers: qs[K] int8 contiguous, xd[K/32] as
// float(d), qsum[K/32] = sum of the 32 int8 (exact int; computed once per
// block here instead of once per row as the reference does).
// Each half-wave (32 lanes) owns one 32-element block per step.
struct Q8Lds {
    int8_t* qs;   // padded: element e at byte q8_pad(e)
    float* xd;
    int* qsum;
};

// LDS padding against bank conflicts.  The GEMV lanes of one step read the
// same offsets of 16 consecutive super-blocks; an unpadded layout (256 B of
// Q8 / 1 KB of fp32 x per super-block) puts all of them in the same banks.
// Q8 bytes: 16 extra bytes after every 256; fp32 x: 4 extra floats after
// every 128 elements.
__host__ __device__ constexpr int q8_pad(int e) { return e + 16 * (e >> 8); }
__host__ __device__ constexpr int q8_padded_bytes(int K) { return K + 16 * (K >> 8); }
__host__ __device__ constexpr int x_pad(int e) { return e + 4 * (e >> 7); }
__host__ __device__ constexpr int x_padded_floats(int K) { return K + 4 * (K >> 7); }

// ---- RMSNorm inverse in one fixed order --------------------------------------
// inv = rsqrt(sum(x^2) / n + eps) for x[n] (n % 8 == 0, 16-byte aligned),
// summed in one canonical order shared by every kernel that normalises: 256
// virtual threads, thread v summing the squares of elements
// [2048 u + 8 v, + 8) for u = 0, 1, .. (an explicit fma chain per 8), the 64
// lanes of each virtual wave added by an xor butterfly, the four waves as
// (w0 + w1) + (w2 + w3).  The standalone norm and the norm fused into the
// GEMV prologues therefore produce identical bits.
__device__ __forceinline__ float sq8(const float4& a, const float4& b) {
    float t = a.x * a.x;
    t = __fmaf_rn(a.y, a.y, t);
    t = __fmaf_rn(a.z, a.z, t);
    t = __fmaf_rn(a.w, a.w, t);
    t = __fmaf_rn(b.x, b.x, t);
    t = __fmaf_rn(b.y, b.y, t);
    t = __fmaf_rn(b.z, b.z, t);
    t = __fmaf_rn(b.w, b.w, t);
    return t;
}

// The xor butterfly v += v[lane ^ o], o = 32, 16, .., 1, every lane ending
// with the same sum, on VALU exchanges: v_permlane32_swap / _16_swap for 32
// and 16, DPP row_ror:8 for 8, row_shl:4 / row_shr:4 selected by lane bit 2
// for 4, quad permutes for 2 and 1 -- the sums of the __shfl_xor form bit for
// bit (each step adds the same partner), without its LDS round trips.
__device__ __forceinline__ float xor_sum64(float v) {
    const int lane = threadIdx.x & 63;
    const uint32_t b32 = __float_as_uint(v);
    const auto r32 = __builtin_amdgcn_permlane32_swap(b32, b32, false, false);
    v += __uint_as_float(lane >= 32 ? r32[0] : r32[1]);
    const uint32_t b16 = __float_as_uint(v);
    const auto r16 = __builtin_amdgcn_permlane16_swap(b16, b16, false, false);
    v += __uint_as_float(((lane >> 4) & 1) ? r16[0] : r16[1]);
    v += dpp_f<0x128>(v);                     // row_ror:8
    const float up = dpp_f<0x104>(v), dn = dpp_f<0x114>(v);   // row_shl:4, row_shr:4
    v += (lane & 4) ? dn : up;
    v += dpp_f<kQuadXor2>(v);
    v += dpp_f<kQuadXor1>(v);
    return v;
}

// Combines the four virtual-wave sums (red: LDS float[4], written by lane 0
// of each virtual wave before the barrier inside).
__device__ __forceinline__ float rms_inv_finish(float* red, int n, float eps) {
    __syncthreads();
    const float tot = (red[0] + red[1]) + (red[2] + red[3]);
    return rsqrtf(tot / (float)n + eps);
}

// Any workgroup size that is a multiple of 64 (real threads take virtual
// threads t, t + blockDim, ..).
__device__ __forceinline__ float rms_inv_canonical(const float* __restrict__ x, int n, float eps, float* red) {
    for (int v = threadIdx.x; v < 256; v += blockDim.x) {
        float ss = 0.0f;
        for (int idx = 8 * v; idx < n; idx += 2048)
            ss += sq8(*reinterpret_cast<const float4*>(x + idx), *reinterpret_cast<const float4*>(x + idx + 4));
        ss = xor_sum64(ss);
        if ((v & 63) == 0) red[v >> 6] = ss;
    }
    return rms_inv_finish(red, n, eps);
}

// Whole-vector quantisation by one workgroup.  Each thread quantises 8
// consecutive elements (two float4 loads); four neighbouring lanes form one
// 32-element block and combine amax / int sums with two xor-shuffles.
// Loads are batched four passes at a time.  The first batch can be loaded
// separately (q8_prefetch) so a caller can issue it ahead of its own weight
// loads: the memory counter is in order, so loads issued first are waited
// for first.
struct X8Batch {
    float4 v[4][2];
};

__device__ __forceinline__ void q8_load_batch(const float* __restrict__ x, int K, int base, X8Batch& b) {
    const int per_pass = (int)blockDim.x * 8;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int idx = base + u * per_pass + (int)threadIdx.x * 8;
        const int src = idx < K ? idx : 0;   // out-of-range lanes re-read x[0..7], never stored
        b.v[u][0] = *reinterpret_cast<const float4*>(x + src);
        b.v[u][1] = *reinterpret_cast<const float4*>(x + src + 4);
    }
}

// nb (optional): the matching batch of RMSNorm weights; the quantised
// values are then (x * inv) * w, the standalone norm's arithmetic.
__device__ __forceinline__ void q8_quantize_batch(const X8Batch& b, int K, int base, Q8Lds lds,
                                                  const X8Batch* nb = nullptr, float inv = 1.0f) {
    const int per_pass = (int)blockDim.x * 8;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int idx = base + u * per_pass + (int)threadIdx.x * 8;
        float e[8] = {b.v[u][0].x, b.v[u][0].y, b.v[u][0].z, b.v[u][0].w,
                      b.v[u][1].x, b.v[u][1].y, b.v[u][1].z, b.v[u][1].w};
        if (nb != nullptr) {
            const float g[8] = {nb->v[u][0].x, nb->v[u][0].y, nb->v[u][0].z, nb->v[u][0].w,
                                nb->v[u][1].x, nb->v[u][1].y, nb->v[u][1].z, nb->v[u][1].w};
#pragma unroll
            for (int i = 0; i < 8; ++i) e[i] = (e[i] * inv) * g[i];
        }
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(e[i]));
        amax = fmaxf(amax, dpp_f<kQuadXor1>(amax));   // 4 lanes = one 32-element block
        amax = fmaxf(amax, dpp_f<kQuadXor2>(amax));
        const float scale = fmaxf(amax / 127.0f, 1e-30f);
        const float sf = __half2float(__float2half(scale));
        const float inv = 1.0f / sf;
        uint32_t packed[2] = {0u, 0u};
        int s = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int q = (int)fminf(fmaxf(e[i] * inv, -127.0f), 127.0f);
            s += q;
            packed[i >> 2] |= ((uint32_t)q & 0xFFu) << (8 * (i & 3));
        }
        s += dpp_i<kQuadXor1>(s);
        s += dpp_i<kQuadXor2>(s);
        if (idx < K) {
            *reinterpret_cast<u32x2*>(lds.qs + q8_pad(idx)) = u32x2{packed[0], packed[1]};
            if ((threadIdx.x & 3) == 0) {
                lds.xd[idx >> 5] = sf;
                lds.qsum[idx >> 5] = s;
            }
        }
    }
}

// Quantisation from an fp32 copy of x already in LDS (same arithmetic).
__device__ __forceinline__ void q8_quantize_from_lds(const float* xs, int K, Q8Lds lds) {
    const int per_pass = (int)blockDim.x * 8;
    for (int base = 0; base < K; base += 4 * per_pass) {
        X8Batch b;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int idx = base + u * per_pass + (int)threadIdx.x * 8;
            const int src = idx < K ? idx : 0;
            b.v[u][0] = *reinterpret_cast<const float4*>(xs + src);
            b.v[u][1] = *reinterpret_cast<const float4*>(xs + src + 4);
        }
        q8_quantize_batch(b, K, base, lds);
    }
}

__device__ __forceinline__ void q8_prefetch(const float* __restrict__ x, int K, X8Batch& b0) {
    q8_load_batch(x, K, 0, b0);
}

// Quantise all of x given the already loaded first batch; with nw (RMSNorm
// weights, first batch nb0 already loaded) the values are normalised first.
__device__ __forceinline__ void q8_quantize_finish(const float* __restrict__ x, int K, Q8Lds lds, const X8Batch& b0,
                                                   const float* __restrict__ nw = nullptr,
                                                   const X8Batch* nb0 = nullptr, float inv = 1.0f) {
    const int batch = (int)blockDim.x * 8 * 4;
    q8_quantize_batch(b0, K, 0, lds, nw ? nb0 : nullptr, inv);
    for (int base = batch; base < K; base += batch) {
        X8Batch b, nb;
        q8_load_batch(x, K, base, b);
        if (nw) q8_load_batch(nw, K, base, nb);
        q8_quantize_batch(b, K, base, lds, nw ? &nb : nullptr, inv);
    }
}

// The canonical RMS inverse from the first loaded batch (blockDim == 256:
// the batch holds exactly the canonical elements of each thread), loading
// the rest of x for K > 8192.
__device__ __forceinline__ float rms_inv_from_batch(const X8Batch& b0, const float* __restrict__ x, int K, float eps,
                                                    float* red) {
    float ss = 0.0f;
#pragma unroll
    for (int u = 0; u < 4; ++u)
        if (2048 * u + 8 * (int)threadIdx.x < K) ss += sq8(b0.v[u][0], b0.v[u][1]);
    for (int idx = 8192 + 8 * (int)threadIdx.x; idx < K; idx += 2048)
        ss += sq8(*reinterpret_cast<const float4*>(x + idx), *reinterpret_cast<const float4*>(x + idx + 4));
    ss = xor_sum64(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    return rms_inv_finish(red, K, eps);
}

__device__ __forceinline__ void q8_0_quantize_to_lds(const float* __restrict__ x, int K, Q8Lds lds) {
    X8Batch b0;
    q8_prefetch(x, K, b0);
    q8_quantize_finish(x, K, lds, b0);
}

// fp32 copy of x into LDS through registers, in the padded layout (x_pad):
// eight float4 loads in flight per thread.  Stores are unconditional --
// out-of-range lanes write the spare float4 at xs[x_padded_floats(K)] -- so
// the compiler cannot sink each load into a store branch and serialise them.
// xs must hold x_padded_floats(K) + 4 floats.
__device__ __forceinline__ void stage_f32_to_lds_regs(const float* __restrict__ x, int K, float* xs) {
    const int per_pass = (int)blockDim.x * 4;
    const int spare = x_padded_floats(K);
    for (int base = 0; base < K; base += 8 * per_pass) {
        float4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int idx = base + u * per_pass + (int)threadIdx.x * 4;
            v[u] = *reinterpret_cast<const float4*>(x + (idx < K ? idx : 0));
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int idx = base + u * per_pass + (int)threadIdx.x * 4;
            *reinterpret_cast<float4*>(xs + (idx < K ? x_pad(idx) : spare)) = v[u];
        }
    }
}

// fp32 copy of x into LDS with gfx950's direct HBM->LDS loads
// (global_load_lds_dwordx4: each wave moves 1 KB per instruction without
// staging registers, so every copy of the workgroup is in flight at once).
// K*4 must be a multiple of 1 KB (K % 256 == 0) and xs must point to LDS.
__device__ __forceinline__ void stage_f32_to_lds(const float* __restrict__ x, int K, float* xs) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int nw = (int)blockDim.x / kWave;
    for (int base = wave * 256; base < K; base += nw * 256) {
        __builtin_amdgcn_global_load_lds(static_cast<const void*>(x + base + lane * 4),
                                         (__attribute__((address_space(3))) void*)(xs + base), 16, 0, 0);
    }
}

// Register-ring software pipeline over `nsteps` steps with NB buffers: the
// loads of NB-1 steps are in flight while one is computed.  The loop is
// unrolled by NB so every buffer index is a compile-time constant (the
// buffers live in registers and are never copied); every load is
// unconditional (the step index is clamped, redundant reloads of the last
// step hit the cache) and the loop has a single exit at its latch.  Those
// three properties keep the compiler's in-order wait counting exact, so no
// load is waited for before its own step.  `pre()` runs after the first
// NB-1 steps have been issued (activation staging goes there).
template <int NB, typename Buf, typename Load, typename Process, typename Pre>
__device__ __forceinline__ void ring_pipeline(int nsteps, Buf (&buf)[NB], Load load, Process process, Pre pre) {
#pragma unroll
    for (int j = 0; j < NB - 1; ++j) load(buf[j], min(j, max(nsteps - 1, 0)));
    pre();
    int i = 0;
    for (; i + NB - 1 < nsteps; i += NB) {
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            load(buf[(j + NB - 1) % NB], min(i + j + NB - 1, nsteps - 1));
            process(buf[j], i + j);
        }
    }
#pragma unroll
    for (int j = 0; j < NB - 1; ++j)
        if (i + j < nsteps) process(buf[j], i + j);
}

// Contiguous output-row range of global wave `gw` out of `nw` (balanced to
// within one row): each wave streams one contiguous stretch of the matrix.
__device__ __forceinline__ void wave_row_range(int N, int gw, int nw, int* begin, int* end) {
    *begin = (int)(((long long)N * gw) / nw);
    *end = (int)(((long long)N * (gw + 1)) / nw);
}

// ── Q4_K × Q8_0 per-lane work unit ───────────────────────────────────────
// A lane owns nibble pair p (bytes 32p..32p+31 of qs) of one super-block:
// sub-blocks 2p (low nibbles) and 2p+1 (high nibbles), 64 weights.  Four
// lanes cover a super-block; a wave covers 16 super-blocks per row step.
struct Q4KUnit {
    u32x4 hdr;      // d | dmin<<16, scales[0..11]
    u32x4 qa, qb;   // qs bytes 32p .. 32p+31
};

__device__ __forceinline__ Q4KUnit q4k_load_unit(const uint8_t* blk, int p) {
    Q4KUnit u;
    // (plain loads: nontemporal ones were measured 28% slower here -- they
    // stop the L1 from merging the three loads that share a line)
    u.hdr = *reinterpret_cast<const u32x4*>(blk);
    const u32x4* q = reinterpret_cast<const u32x4*>(blk + 16 + 32 * p);
    u.qa = q[0];
    u.qb = q[1];
    return u;
}

// Integer dots of the lane's 64 nibbles against the matching Q8 bytes
// (x8lo = 32 int8 of sub-block 2p, x8hi = 32 int8 of sub-block 2p+1).
// Exact restatement of q4_k_q8_inline.hip:68-95 (int_dot = Σ nib*q8),
// four products per v_dot4_i32_i8 (nibbles 0..15 are non-negative int8).
__device__ __forceinline__ void q4k_int_dots(const Q4KUnit& u, const u32x4 x8lo[2], const u32x4 x8hi[2],
                                             int* dot_lo, int* dot_hi) {
    int lo = 0, hi = 0;
    const uint32_t w[8] = {u.qa.x, u.qa.y, u.qa.z, u.qa.w, u.qb.x, u.qb.y, u.qb.z, u.qb.w};
    const uint32_t a[8] = {x8lo[0].x, x8lo[0].y, x8lo[0].z, x8lo[0].w, x8lo[1].x, x8lo[1].y, x8lo[1].z, x8lo[1].w};
    const uint32_t b[8] = {x8hi[0].x, x8hi[0].y, x8hi[0].z, x8hi[0].w, x8hi[1].x, x8hi[1].y, x8hi[1].z, x8hi[1].w};
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        lo = __builtin_amdgcn_sdot4((int)(w[t] & 0x0F0F0F0Fu), (int)a[t], lo, false);
        hi = __builtin_amdgcn_sdot4((int)((w[t] >> 4) & 0x0F0F0F0Fu), (int)b[t], hi, false);
    }
    *dot_lo = lo;
    *dot_hi = hi;
}

// Sub-block combine, the reference's fp32 expression
// (q4_k_q8_inline.hip:119-122):
//   acc += x_scale * (d*sc*int_dot - dmin*m*q8_sum)
__device__ __forceinline__ float q4k_q8_combine(float acc, float xd, float d, float dmin, int sc, int mn,
                                                int dot, int qsum) {
    return acc + xd * (d * (float)sc * (float)dot - dmin * (float)mn * (float)qsum);
}

// fp16 bits (round to nearest even) of an fp32 value, as an instruction of
// its own: left to itself the compiler folds a preceding multiply or FMA into
// one v_fma_mix with an fp16 result, which rounds the exact product once
// instead of the fp32 value (a different half for a few values in 10^5).
__device__ __forceinline__ uint16_t f16_bits_rn(float v) {
    uint32_t r;
    asm("v_cvt_f16_f32 %0, %1" : "=v"(r) : "v"(v));
    return (uint16_t)r;
}

// Workgroup barrier that does not wait for outstanding global loads
// (__syncthreads() implies a fence, i.e. vmcnt(0), which would drain the
// loads a pipeline keeps in flight across the barrier).  LDS writes of this
// wave are completed first.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Device CU count, cached per device (host side).
// 16 bytes a lane from global memory straight into LDS at m0 + 16 lane
__device__ __forceinline__ void lds_dma16(uint32_t lds_dst, uint32_t voff, const uint8_t* sbase) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2"
                 :: "s"(lds_dst), "v"(voff), "s"(sbase) : "memory", "m0");
}

int device_cu_count();

}  // namespace rf
