/*
 * cpu_baseline.c -- C port of ROCmForge's CPU path for Q4_K / Q6_K GEMV/GEMM,
 * used ONLY as the timing baseline that bench.py reports beside the GPU
 * figure (cpu_baseline.kind = "port").  Test infrastructure: the product
 * library never links it.
 *
 * Restated algorithms (paths relative to the ROCmForge tree):
 *   cb_quantize_q8_k     src/cpu/kernels/q8.rs:19-40 (256-element Q8_K block,
 *                        d = amax/127 (1.0 if amax <= 1e-7), q = round(x/d)
 *                        clamped to +-127, 16 bsums)
 *   cb_dot_q4k_q8k       src/cpu/kernels/gemm_q4k_q8.rs:90-195 (llama.cpp
 *                        AVX2 maddubs/madd block dot, scale unpack via the
 *                        kmask words, min term through bsums)
 *   cb_gemv_q4k_q8k      gemm_q4k_q8.rs:197-241 (quantize x once, rows in
 *                        parallel -- OpenMP stands in for rayon)
 *   cb_gemm_q4k_q8k      gemm_q4k_q8.rs:243-276 (parallel over batch rows)
 *   cb_gemv_q6k          src/cpu/ops.rs:480-572 (scalar dequant-dot; the
 *                        reference parallelises over batch rows only, so a
 *                        single-token GEMV runs on ONE thread; `threads`>1
 *                        is a separately labelled all-cores variant)
 *   cb_silu_fuse         src/cpu/ops.rs:121-130
 * The numerics of this path (Q8_K, round-to-nearest, f32 scale) differ from
 * the GPU Q8_0 path by design; its results are not a parity reference.
 * The reference's acc_m initialisation (gemm_q4k_q8.rs:132-133) adds dmin
 * once per SIMD lane; that is reproduced because it is part of the timed
 * arithmetic.
 */
#include <immintrin.h>
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

float or_f16_to_f32(uint16_t h);

typedef struct {
    float d;
    int8_t qs[256];
    int16_t bsums[16];
} cb_q8k;

static inline float f16(const uint8_t* p) { return or_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

void cb_quantize_q8_k(const float* x, cb_q8k* out) {
    float amax = 0.0f;
    for (int i = 0; i < 256; ++i) amax = fmaxf(amax, fabsf(x[i]));
    float d = amax > 1e-7f ? amax / 127.0f : 1.0f;
    memset(out->bsums, 0, sizeof(out->bsums));
    for (int i = 0; i < 256; ++i) {
        float q = roundf(x[i] / d);
        if (q > 127.0f) q = 127.0f;
        if (q < -127.0f) q = -127.0f;
        out->qs[i] = (int8_t)q;
        out->bsums[i / 16] += (int16_t)q;
    }
    out->d = d;
}

static inline float hsum8(__m256 v) {
    __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
    float t[4];
    _mm_storeu_ps(t, s);
    return t[0] + t[1] + t[2] + t[3];
}

/* pshufb masks that broadcast the 16-bit scale of sub-block pair j */
static __m256i scale_mask(int j) {
    int8_t m[32];
    for (int i = 0; i < 32; ++i) m[i] = (int8_t)(2 * j + (i & 1));
    return _mm256_loadu_si256((const __m256i*)m);
}

float cb_dot_q4k_q8k(const uint8_t* blk, const cb_q8k* q8) {
    const uint32_t km1 = 0x3f3f3f3fu, km2 = 0x0f0f0f0fu, km3 = 0x03030303u;
    float d = q8->d * f16(blk);
    float dmin = -q8->d * f16(blk + 2);
    uint32_t u[4];
    memcpy(u, blk + 4, 12);
    u[3] = ((u[2] >> 4) & km2) | (((u[1] >> 6) & km3) << 4);
    uint32_t ua = u[1] & km1;
    u[1] = (u[2] & km2) | (((u[0] >> 6) & km3) << 4);
    u[2] = ua;
    u[0] &= km1;
    __m256i ms = _mm256_cvtepu8_epi16(_mm_set_epi32((int)u[3], (int)u[2], (int)u[1], (int)u[0]));
    __m256i q8sums = _mm256_loadu_si256((const __m256i*)q8->bsums);
    __m128i q8s = _mm_hadd_epi16(_mm256_extracti128_si256(q8sums, 0), _mm256_extracti128_si256(q8sums, 1));
    __m128i prod = _mm_madd_epi16(_mm256_extracti128_si256(ms, 1), q8s);
    __m128 acc_m = _mm_set1_ps(dmin);
    acc_m = _mm_fmadd_ps(acc_m, _mm_cvtepi32_ps(prod), acc_m);
    __m128i sc128 = _mm256_extracti128_si256(ms, 0);
    __m256i scales = _mm256_set_m128i(sc128, sc128);
    const __m256i m4 = _mm256_set1_epi8(0xF);
    __m256i sumi = _mm256_setzero_si256();
    const uint8_t* q4 = blk + 16;
    const int8_t* qq = q8->qs;
    for (int j = 0; j < 4; ++j) {
        __m256i sl = _mm256_shuffle_epi8(scales, scale_mask(2 * j));
        __m256i sh = _mm256_shuffle_epi8(scales, scale_mask(2 * j + 1));
        __m256i bits = _mm256_loadu_si256((const __m256i*)q4);
        q4 += 32;
        __m256i lo = _mm256_and_si256(bits, m4);
        __m256i hi = _mm256_and_si256(_mm256_srli_epi16(bits, 4), m4);
        __m256i xl = _mm256_loadu_si256((const __m256i*)qq);
        qq += 32;
        __m256i pl = _mm256_madd_epi16(sl, _mm256_maddubs_epi16(lo, xl));
        __m256i xh = _mm256_loadu_si256((const __m256i*)qq);
        qq += 32;
        __m256i ph = _mm256_madd_epi16(sh, _mm256_maddubs_epi16(hi, xh));
        sumi = _mm256_add_epi32(sumi, _mm256_add_epi32(pl, ph));
    }
    __m256 acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(sumi), _mm256_setzero_ps());
    float t[4];
    _mm_storeu_ps(t, acc_m);
    return hsum8(acc) + t[0];
}

void cb_gemv_q4k_q8k(const uint8_t* w, const float* x, float* y, int N, int K, int threads) {
    int nb = K / 256;
    cb_q8k* xq = (cb_q8k*)malloc(sizeof(cb_q8k) * (size_t)nb);
    for (int b = 0; b < nb; ++b) cb_quantize_q8_k(x + 256 * b, &xq[b]);
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int n = 0; n < N; ++n) {
        const uint8_t* row = w + (size_t)n * nb * 144;
        float acc = 0.0f;
        for (int b = 0; b < nb; ++b) acc += cb_dot_q4k_q8k(row + (size_t)b * 144, &xq[b]);
        y[n] = acc;
    }
    free(xq);
}

void cb_gemm_q4k_q8k(const uint8_t* w, const float* x, float* y, int M, int N, int K, int threads) {
    int nb = K / 256;
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int m = 0; m < M; ++m) {
        cb_q8k* xq = (cb_q8k*)malloc(sizeof(cb_q8k) * (size_t)nb);
        for (int b = 0; b < nb; ++b) cb_quantize_q8_k(x + (size_t)m * K + 256 * b, &xq[b]);
        for (int n = 0; n < N; ++n) {
            const uint8_t* row = w + (size_t)n * nb * 144;
            float acc = 0.0f;
            for (int b = 0; b < nb; ++b) acc += cb_dot_q4k_q8k(row + (size_t)b * 144, &xq[b]);
            y[(size_t)m * N + n] = acc;
        }
        free(xq);
    }
}

static float q6k_row_dot(const uint8_t* roww, const float* x, int nb) {
    float acc = 0.0f;
    for (int b = 0; b < nb; ++b) {
        const uint8_t* blk = roww + (size_t)b * 210;
        const uint8_t* ql = blk;
        const uint8_t* qh = blk + 128;
        const int8_t* sc = (const int8_t*)(blk + 192);
        float d = f16(blk + 208);
        const float* xb = x + 256 * b;
        for (int h = 0; h < 2; ++h) {
            for (int l = 0; l < 32; ++l) {
                int is = l / 16;
                int q1 = (int)(int8_t)((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                int q2 = (int)(int8_t)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                int q3 = (int)(int8_t)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                int q4 = (int)(int8_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                acc += d * (float)sc[is + 0] * (float)q1 * xb[l + 0];
                acc += d * (float)sc[is + 2] * (float)q2 * xb[l + 32];
                acc += d * (float)sc[is + 4] * (float)q3 * xb[l + 64];
                acc += d * (float)sc[is + 6] * (float)q4 * xb[l + 96];
            }
            ql += 64;
            qh += 32;
            sc += 8;
            xb += 128;
        }
    }
    return acc;
}

void cb_gemv_q6k(const uint8_t* w, const float* x, float* y, int N, int K, int threads) {
    int nb = K / 256;
    size_t rb = (size_t)nb * 210;
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int n = 0; n < N; ++n) y[n] = q6k_row_dot(w + (size_t)n * rb, x, nb);
}

void cb_gemm_q6k(const uint8_t* w, const float* x, float* y, int M, int N, int K, int threads) {
    int nb = K / 256;
    size_t rb = (size_t)nb * 210;
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) y[(size_t)m * N + n] = q6k_row_dot(w + (size_t)n * rb, x + (size_t)m * K, nb);
}

void cb_silu_fuse(const float* g, float* u, int N) {
    for (int i = 0; i < N; ++i) u[i] = g[i] / (1.0f + expf(-g[i])) * u[i];
}

/* gate+up+SwiGLU on the CPU: two Q4_K GEMVs then silu_fuse (cpu/forward.rs
 * FFN sequence).  `gate` is caller scratch of N floats. */
void cb_gate_up_swiglu(const uint8_t* wg, const uint8_t* wu, const float* x, float* gate, float* out,
                       int N, int K, int threads) {
    cb_gemv_q4k_q8k(wg, x, gate, N, K, threads);
    cb_gemv_q4k_q8k(wu, x, out, N, K, threads);
    cb_silu_fuse(gate, out, N);
}

int cb_max_threads(void) { return omp_get_max_threads(); }
