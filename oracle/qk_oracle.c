/*
 * qk_oracle.c -- CPU restatement of ROCmForge's Q4_K / Q6_K matmul hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the GPU kernels are
 * compared against.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product library never links it.
 *
 * Every function states the reference file:line it restates (paths are
 * relative to the ROCmForge source tree).  Parity pins (see tests/):
 *   or_f32_to_f16 / or_f16_to_f32   numpy float16 RNE conversion, exhaustive
 *                                   over all 65536 halves + 2^24 float probes
 *   or_q4k_scale_min                golden JSON unpacked_scale_min_per_subblock
 *   or_q4k_dequant_row_*            golden JSON dequantized_first_64/last_8
 *                                   (real Qwen3-8B blocks) + byte-level block
 *   or_q6k_dequant_row_f32          byte-level block of the reference WMMA
 *                                   Q6_K test + independent element-order
 *                                   formula in the test (ggml layout)
 *   or_q8_0_quantize                closed-form invariants, all-zero/huge
 *                                   edge blocks, brute force over every fp16
 *                                   scale on tiny blocks, and the reference
 *                                   GPU kernel itself (oracle/_ref) on GPU
 *   or_q4k_q8_partials              brute-force integer dot on dequant-free
 *                                   nibble matrices; sum identity
 *   or_gemv_*                       float64 brute-force dot over the pinned
 *                                   dequant; reference kernels on GPU
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define QK_K 256
#define Q4K_BYTES 144
#define Q6K_BYTES 210

/* ---- IEEE half conversion (round to nearest even) ----------------------
 * Restates __float2half / __half2float (ROCm hip_fp16.h) and the `half`
 * 2.7.1 crate's f16::from_f32 / to_f32 used by the reference CPU path
 * (src/cpu/quant.rs:100-111).  Both are IEEE binary16 with RNE. */
uint16_t or_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xFFu;
    uint32_t man = x & 0x7FFFFFu;
    if (exp == 0xFFu) {                       /* inf / nan */
        if (man == 0) return (uint16_t)(sign | 0x7C00u);
        return (uint16_t)(sign | 0x7E00u | (man >> 13));
    }
    int32_t e = (int32_t)exp - 127 + 15;      /* rebias */
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);   /* overflow -> inf */
    if (e <= 0) {                             /* subnormal or zero */
        if (e < -10) return (uint16_t)sign;   /* below half of min subnormal */
        uint32_t m = man | 0x800000u;         /* implicit one */
        uint32_t shift = (uint32_t)(14 - e);  /* 24-bit mantissa -> 10-bit at 2^-24 */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);          /* q may carry into exponent 1: correct */
    }
    uint32_t q = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;  /* carry may reach inf: correct */
    return (uint16_t)(sign | q);
}

float or_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t x;
    if (exp == 0) {
        if (man == 0) {
            x = sign;
        } else {                               /* subnormal: normalise */
            int e = -1;
            do { man <<= 1; e++; } while (!(man & 0x400u));
            man &= 0x3FFu;
            x = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 0x1F) {
        x = sign | 0x7F800000u | (man << 13);
    } else {
        x = sign | ((exp - 15 + 127) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

static inline float ld_f16(const uint8_t* p) {
    return or_f16_to_f32((uint16_t)(p[0] | (p[1] << 8)));
}

/* ---- Q8_0 inline activation quantizer ----------------------------------
 * hip_kernels/quant/q4_k_q8_inline.hip:133-162
 *   amax = max|x| over 32; scale = fmaxf(amax/127, 1e-30); d = half(scale);
 *   inv = 1/float(d); q = (int8) trunc(fminf(fmaxf(x*inv, -127), 127)).
 * fmaxf/fminf return the non-NaN operand (IEEE maxNum), so an all-zero
 * block (d == 0, inv == inf, 0*inf == NaN) stores q == -127 everywhere. */
void or_q8_0_quantize(const float* x, int K, uint16_t* d_out, int8_t* qs_out) {
    for (int b = 0; b < K / 32; ++b) {
        const float* xb = x + 32 * b;
        float amax = 0.0f;
        for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(xb[i]));
        volatile float scale = fmaxf(amax / 127.0f, 1e-30f);
        uint16_t dh = or_f32_to_f16(scale);
        float sf = or_f16_to_f32(dh);
        volatile float inv = 1.0f / sf;
        d_out[b] = dh;
        for (int i = 0; i < 32; ++i) {
            volatile float prod = xb[i] * inv;
            float qf = fminf(fmaxf(prod, -127.0f), 127.0f);
            qs_out[32 * b + i] = (int8_t)qf;   /* C cast truncates toward zero */
        }
    }
}

/* ---- Q4_K 6-bit scale/min unpack ---------------------------------------
 * hip_kernels/quant/q4_k_q8_inline.hip:49-59 (= ggml get_scale_min_k4,
 * src/cpu/quant.rs:257-266). */
void or_q4k_scale_min(int j, const uint8_t* s, int* sc, int* m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4);
        *m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

/* ---- Q4_K dequant ------------------------------------------------------
 * src/cpu/quant.rs:243-295 (embed_q4_k) and the test copy
 * tests/wmma_q4_k_correctness.rs:42-82: element 64k+i (i<32) is the low
 * nibble of qs[32k+i] in sub-block 2k, element 64k+32+i the high nibble
 * in sub-block 2k+1; value = d*sc*nib - dmin*m.
 * _f64: exact real value (d*sc*nib and dmin*m are exact in double).
 * _f32: the reference fp32 evaluation (d*sc exact, *nib exact, one
 *       rounding at the subtraction -- FMA contraction cannot change it). */
void or_q4k_dequant_row_f64(const uint8_t* w, int n_blocks, double* out) {
    for (int b = 0; b < n_blocks; ++b) {
        const uint8_t* blk = w + (size_t)b * Q4K_BYTES;
        double d = ld_f16(blk), dmin = ld_f16(blk + 2);
        const uint8_t* qs = blk + 16;
        for (int j = 0; j < 8; ++j) {
            int sc, m;
            or_q4k_scale_min(j, blk + 4, &sc, &m);
            for (int i = 0; i < 32; ++i) {
                uint8_t byte = qs[(j >> 1) * 32 + i];
                int nib = (j & 1) ? (byte >> 4) : (byte & 15);
                out[(size_t)b * QK_K + j * 32 + i] = d * sc * nib - dmin * m;
            }
        }
    }
}

void or_q4k_dequant_row_f32(const uint8_t* w, int n_blocks, float* out) {
    for (int b = 0; b < n_blocks; ++b) {
        const uint8_t* blk = w + (size_t)b * Q4K_BYTES;
        float d = ld_f16(blk), dmin = ld_f16(blk + 2);
        const uint8_t* qs = blk + 16;
        for (int j = 0; j < 8; ++j) {
            int sc, m;
            or_q4k_scale_min(j, blk + 4, &sc, &m);
            float d1 = d * (float)sc, m1 = dmin * (float)m;
            for (int i = 0; i < 32; ++i) {
                uint8_t byte = qs[(j >> 1) * 32 + i];
                int nib = (j & 1) ? (byte >> 4) : (byte & 15);
                volatile float p = d1 * (float)nib;
                out[(size_t)b * QK_K + j * 32 + i] = p - m1;
            }
        }
    }
}

/* ---- Q6_K dequant ------------------------------------------------------
 * src/cpu/quant.rs:316-391 (embed_q6_k), hip_kernels/quant/q6_k_gemv.hip:
 * 111-152, docs/q6_k_block_format.md:85-110.  For half n and l<32:
 *   e = 128n + 32q + l,  ql byte = ql[64n + 32(q&1) + l] (low nibble for
 *   q<2, high for q>=2), qh bits = (qh[32n+l] >> 2q) & 3,
 *   scale = sc[8n + 2q + l/16] (int8), value = d*scale*(q6 - 32).
 * The float result is exact (11+8+6 bit product), so f32 == f64. */
void or_q6k_dequant_row_f32(const uint8_t* w, int n_blocks, float* out) {
    for (int b = 0; b < n_blocks; ++b) {
        const uint8_t* blk = w + (size_t)b * Q6K_BYTES;
        const uint8_t* ql = blk;
        const uint8_t* qh = blk + 128;
        const int8_t* sc = (const int8_t*)(blk + 192);
        float d = ld_f16(blk + 208);
        for (int n = 0; n < 2; ++n) {
            for (int q = 0; q < 4; ++q) {
                for (int l = 0; l < 32; ++l) {
                    uint8_t lb = ql[64 * n + 32 * (q & 1) + l];
                    int nib = (q >= 2) ? (lb >> 4) : (lb & 15);
                    int hb = (qh[32 * n + l] >> (2 * q)) & 3;
                    int q6 = (nib | (hb << 4)) - 32;
                    float s = d * (float)sc[8 * n + 2 * q + l / 16];
                    out[(size_t)b * QK_K + 128 * n + 32 * q + l] = s * (float)q6;
                }
            }
        }
    }
}

/* ---- Q4_K x Q8_0 integer partials --------------------------------------
 * hip_kernels/quant/q4_k_q8_inline.hip:68-95: per sub-block j of each
 * super-block, int_dot = sum nib*q8 and q8_sum = sum q8 over 32 elements.
 * int_dot is written per (row, K/32 sub-block); q8_sum per sub-block. */
void or_q4k_q8_partials(const uint8_t* w, const int8_t* xq, int K, int N,
                        int32_t* int_dot, int32_t* q8_sum) {
    int nsb = K / QK_K;
    for (int b = 0; b < K / 32; ++b) {
        int s = 0;
        for (int i = 0; i < 32; ++i) s += xq[32 * b + i];
        q8_sum[b] = s;
    }
    for (int n = 0; n < N; ++n) {
        for (int sb = 0; sb < nsb; ++sb) {
            const uint8_t* qs = w + ((size_t)n * nsb + sb) * Q4K_BYTES + 16;
            for (int j = 0; j < 8; ++j) {
                int acc = 0;
                for (int i = 0; i < 32; ++i) {
                    uint8_t byte = qs[(j >> 1) * 32 + i];
                    int nib = (j & 1) ? (byte >> 4) : (byte & 15);
                    acc += nib * xq[sb * QK_K + j * 32 + i];
                }
                int_dot[(size_t)n * (K / 32) + sb * 8 + j] = acc;
            }
        }
    }
}

/* ---- GEMV outputs (float64) --------------------------------------------
 * Q4_K x Q8_0 inline: hip_kernels/quant/q4_k_q8_inline.hip:99-125,165-225
 *   y[n] = sum_sb sum_j xd_j * (d*sc_j*int_dot_j - dmin*m_j*q8_sum_j),
 * evaluated in float64 over the exact integer partials. */
void or_gemv_q4k_q8(const uint8_t* w, const float* x, int K, int N, double* y) {
    int nsb = K / QK_K, nb = K / 32;
    uint16_t xd[QK_K * 8];
    int8_t xq_stack[1];
    (void)xq_stack;
    /* K is bounded by the launchers' LDS rule: (K/32)*34 <= 32768 */
    static int8_t xq[65536];
    static int32_t qsum[2048];
    or_q8_0_quantize(x, K, xd, xq);
    for (int b = 0; b < nb; ++b) {
        int s = 0;
        for (int i = 0; i < 32; ++i) s += xq[32 * b + i];
        qsum[b] = s;
    }
    for (int n = 0; n < N; ++n) {
        double acc = 0.0;
        for (int sb = 0; sb < nsb; ++sb) {
            const uint8_t* blk = w + ((size_t)n * nsb + sb) * Q4K_BYTES;
            double d = ld_f16(blk), dmin = ld_f16(blk + 2);
            for (int j = 0; j < 8; ++j) {
                int sc, m, dot = 0;
                or_q4k_scale_min(j, blk + 4, &sc, &m);
                for (int i = 0; i < 32; ++i) {
                    uint8_t byte = blk[16 + (j >> 1) * 32 + i];
                    int nib = (j & 1) ? (byte >> 4) : (byte & 15);
                    dot += nib * xq[sb * QK_K + j * 32 + i];
                }
                int b = sb * 8 + j;
                acc += (double)or_f16_to_f32(xd[b]) *
                       (d * sc * (double)dot - dmin * m * (double)qsum[b]);
            }
        }
        y[n] = acc;
    }
}

/* FP32-activation Q4_K GEMV: hip_kernels/quant/q4_k_gemv.hip:46-75
 *   y[n] = sum (d*sc*nib - dmin*m) * x   (float64 here). */
void or_gemv_q4k_f32(const uint8_t* w, const float* x, int K, int N, double* y) {
    static double row[65536 * 4];
    int nsb = K / QK_K;
    for (int n = 0; n < N; ++n) {
        or_q4k_dequant_row_f64(w + (size_t)n * nsb * Q4K_BYTES, nsb, row);
        double acc = 0.0;
        for (int k = 0; k < K; ++k) acc += row[k] * (double)x[k];
        y[n] = acc;
    }
}

/* Q6_K GEMV: hip_kernels/quant/q6_k_gemv.hip:111-217 (float64 here). */
void or_gemv_q6k(const uint8_t* w, const float* x, int K, int N, double* y) {
    static float row[65536 * 4];
    int nsb = K / QK_K;
    for (int n = 0; n < N; ++n) {
        or_q6k_dequant_row_f32(w + (size_t)n * nsb * Q6K_BYTES, nsb, row);
        double acc = 0.0;
        for (int k = 0; k < K; ++k) acc += (double)row[k] * (double)x[k];
        y[n] = acc;
    }
}

/* SwiGLU epilogue: q4_k_q8_inline.hip:364-366 / src/cpu/ops.rs:121-130
 *   out = g / (1 + exp(-g)) * u   (float64 here). */
void or_swiglu(const double* g, const double* u, int N, double* out) {
    for (int n = 0; n < N; ++n) out[n] = g[n] / (1.0 + exp(-g[n])) * u[n];
}

/* ---- GEMM operand staging ----------------------------------------------
 * hip_kernels/wmma/wmma_gemm_q4_k.hip:78-138 and wmma_gemm_q6_k.hip:78-149:
 * A is converted with __float2half, each weight with
 * __float2half(fp32 dequant value).  The oracle returns the fp16-rounded
 * operands as floats; the float64 product is formed by the caller. */
void or_round_f16(const float* a, size_t n, float* out) {
    for (size_t i = 0; i < n; ++i) out[i] = or_f16_to_f32(or_f32_to_f16(a[i]));
}

void or_q4k_dequant_f16(const uint8_t* w, int N, int K, float* out) {
    int nsb = K / QK_K;
    for (int n = 0; n < N; ++n) {
        float* o = out + (size_t)n * K;
        or_q4k_dequant_row_f32(w + (size_t)n * nsb * Q4K_BYTES, nsb, o);
        for (int k = 0; k < K; ++k) o[k] = or_f16_to_f32(or_f32_to_f16(o[k]));
    }
}

void or_q6k_dequant_f16(const uint8_t* w, int N, int K, float* out) {
    int nsb = K / QK_K;
    for (int n = 0; n < N; ++n) {
        float* o = out + (size_t)n * K;
        or_q6k_dequant_row_f32(w + (size_t)n * nsb * Q6K_BYTES, nsb, o);
        for (int k = 0; k < K; ++k) o[k] = or_f16_to_f32(or_f32_to_f16(o[k]));
    }
}

/* ==== Layer operations around the matmuls ==================================
 * Pins (tests/test_oracle_ops.py): the reference's own op tests
 * (src/cpu/ops_tests.rs: rms_norm on [3, 4], rope at position 0, silu(+-1),
 * the two-position decode attention, argmax), closed forms (unit RMS,
 * scale invariance, rotation by exact angles, pair-norm preservation,
 * classic = interleaved NeoX, uniform / one-hot attention) and brute force
 * (direct softmax over all positions, full causal attention). */

/* src/cpu/ops.rs:33-46 -- out = x / sqrt(mean(x^2) + eps) * w, per row. */
void or_rms_norm(const float* x, const float* w, int n, int rows, float eps, double* out) {
    for (int r = 0; r < rows; ++r) {
        const float* xr = x + (size_t)r * n;
        double ss = 0.0;
        for (int i = 0; i < n; ++i) ss += (double)xr[i] * xr[i];
        const double inv = 1.0 / sqrt(ss / n + (double)eps);
        for (int i = 0; i < n; ++i) out[(size_t)r * n + i] = (double)xr[i] * inv * w[i];
    }
}

/* theta_i of src/cpu/ops.rs:79 / hip_kernels/rope.hip:66-70: exponent in
 * fp32, 1 / base^e evaluated in double and rounded once to float, divided
 * (fp32) by freq_scale[i] when given. */
float or_rope_theta(int i, int d, float base, const float* freq_scale) {
    const float e = (float)(2 * i) / (float)d;
    float t = (float)(1.0 / pow((double)base, (double)e));
    if (freq_scale) t = t / freq_scale[i];
    return t;
}

/* src/cpu/ops.rs:69-98 -- RoPE of rows [seq][nh][d] in place (double
 * values), row s at position pos0 + s, angle = (float)pos * theta in fp32. */
void or_rope(double* x, int seq, int nh, int d, int pos0, float base, int neox, const float* freq_scale) {
    const int half = d / 2;
    for (int s = 0; s < seq; ++s)
        for (int h = 0; h < nh; ++h) {
            double* row = x + ((size_t)s * nh + h) * d;
            for (int i = 0; i < half; ++i) {
                const float a = (float)(pos0 + s) * or_rope_theta(i, d, base, freq_scale);
                const double c = cos((double)a), sn = sin((double)a);
                const int i0 = neox ? i : 2 * i, i1 = neox ? i + half : 2 * i + 1;
                const double x0 = row[i0], x1 = row[i1];
                row[i0] = x0 * c - x1 * sn;
                row[i1] = x0 * sn + x1 * c;
            }
        }
}

/* src/cpu/ops.rs:195-249 -- one query over seq cached positions with the
 * online softmax of :150-172; K/V are fp16 bits [seq][nkv * d]. */
void or_attn_decode(const float* q, const uint16_t* kc, const uint16_t* vc, int seq, int nh, int nkv, int d,
                    float scale, double* out) {
    const int group = nh / nkv;
    double acc[1024];
    for (int h = 0; h < nh; ++h) {
        const int kh = h / group;
        double m = -INFINITY, l = 0.0;
        for (int i = 0; i < d; ++i) acc[i] = 0.0;
        for (int t = 0; t < seq; ++t) {
            const uint16_t* kr = kc + (size_t)t * nkv * d + (size_t)kh * d;
            const uint16_t* vr = vc + (size_t)t * nkv * d + (size_t)kh * d;
            double s = 0.0;
            for (int i = 0; i < d; ++i) s += (double)q[h * d + i] * or_f16_to_f32(kr[i]);
            s *= scale;
            const double mn = s > m ? s : m;
            const double ed = exp(m - mn), es = exp(s - mn);
            for (int i = 0; i < d; ++i) acc[i] = acc[i] * ed + es * or_f16_to_f32(vr[i]);
            l = l * ed + es;
            m = mn;
        }
        for (int i = 0; i < d; ++i) out[h * d + i] = acc[i] / l;
    }
}

/* Causal prefill attention with the rounding of the reference's default
 * prefill path (src/gpu/forward.rs:768-824 ->
 * hip_kernels/wmma/wmma_attention_prefill.hip:386-660): Q, K, V rounded to
 * fp16; S = Q K^T (exact products, wide sum) * scale; keys in tiles of 64
 * with a running row max m; per tile P = fp16(exp(S - m_new)) for
 * unmasked keys, l += sum of the unrounded exp, O = O * exp(m_old - m_new)
 * + P V; out = O / l.  q: [seq][nh * d], k, v: [seq][nkv * d] (fp32). */
void or_attn_prefill_f16(const float* q, const float* k, const float* v, int seq, int nh, int nkv, int d, float scale,
                         double* out) {
    const int group = nh / nkv;
    double acc[1024];
    for (int h = 0; h < nh; ++h) {
        const int kh = h / group;
        for (int r = 0; r < seq; ++r) {
            double m = -3.402823466e+38, l = 0.0;
            for (int i = 0; i < d; ++i) acc[i] = 0.0;
            for (int t0 = 0; t0 <= r; t0 += 64) {
                double s[64];
                double tmax = -3.402823466e+38;
                const int tn = (r - t0 + 1) < 64 ? (r - t0 + 1) : 64;
                for (int j = 0; j < tn; ++j) {
                    double dot = 0.0;
                    for (int i = 0; i < d; ++i)
                        dot += (double)or_f16_to_f32(or_f32_to_f16(q[(size_t)r * nh * d + h * d + i])) *
                               or_f16_to_f32(or_f32_to_f16(k[(size_t)(t0 + j) * nkv * d + kh * d + i]));
                    s[j] = (double)(float)dot * scale;
                    if (s[j] > tmax) tmax = s[j];
                }
                const double mn = tmax > m ? tmax : m;
                const double alpha = exp(m - mn);
                double rs = 0.0;
                for (int i = 0; i < d; ++i) acc[i] *= alpha;
                for (int j = 0; j < tn; ++j) {
                    const double e = exp(s[j] - mn);
                    rs += e;
                    const double p = or_f16_to_f32(or_f32_to_f16((float)e));
                    for (int i = 0; i < d; ++i)
                        acc[i] += p * or_f16_to_f32(or_f32_to_f16(v[(size_t)(t0 + j) * nkv * d + kh * d + i]));
                }
                l = alpha * l + rs;
                m = mn;
            }
            for (int i = 0; i < d; ++i) out[((size_t)r * nh + h) * d + i] = acc[i] / l;
        }
    }
}

/* src/cpu/ops.rs:120-123 -- silu(g) * u. */
void or_silu_mul(const float* g, const float* u, int n, double* out) {
    for (int i = 0; i < n; ++i) out[i] = (double)g[i] / (1.0 + exp(-(double)g[i])) * u[i];
}

/* hip_kernels/elementwise.hip:150-160 -- the maximum; equal values go to
 * the larger index; NaN never replaces the running best. */
int or_argmax(const float* x, int n) {
    float bv = -3.402823466e+38f;
    int bi = 0;
    for (int i = 0; i < n; ++i)
        if (x[i] > bv || (x[i] == bv && i > bi)) {
            bv = x[i];
            bi = i;
        }
    return bi;
}
