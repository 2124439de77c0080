/*
 * CPU oracle for the quantized-weight path -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the arithmetic the reference runs through mlx
 * 0.32.3 / mlx-lm 0.32.0 (pinned at pyproject.toml:32-33 of the reference,
 * not vendored there) and through the reference's own KV8 Metal kernel.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker (or the timed CPU baseline);
 * the product path never calls it.
 *
 * Every entry point works on float32 arrays holding the exact values of the
 * caller's bf16/fp16/fp32 tensors; rounding to the storage dtype happens in
 * oracle/__init__.py with exact bit arithmetic.  Products and sums are done
 * in double so each output is the correctly rounded exact result; that is
 * the bar the HIP kernels are measured against.
 *
 * Built by oracle/Makefile into oracle/liboracle.so (gcc -O3 -fopenmp).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* affine packing                                                            */
/* Element j of a row sits in word j / (32/bits) at bit offset               */
/* (j mod (32/bits)) * bits, little-endian within the word: the reference's  */
/* KV8 kernel reads mlx-packed words exactly this way,                       */
/* src/knurlogic/engine/kvattn.py:128-131 and :140-142.                     */
/* ------------------------------------------------------------------------ */

static inline uint32_t unpack_q(const uint32_t* row, int64_t j, int bits) {
    /* element j at bits [j*bits, j*bits + bits) of the row read as one
       little-endian bit stream; for bits dividing 32 this is word
       j / (32/bits), shift (j % (32/bits)) * bits.  mlx packs its 3, 5 and
       6-bit modes into bytes in the same stream order. */
    const int64_t off = j * bits;
    const int64_t q = off >> 5;
    const int sh = (int)(off & 31);
    const uint32_t mask = (1u << bits) - 1u;
    uint64_t v = row[q] >> sh;
    if (sh + bits > 32) v |= (uint64_t)row[q + 1] << (32 - sh);
    return (uint32_t)v & mask;
}

static inline void pack_q(uint32_t* row, int64_t j, int bits, uint32_t q) {
    const int64_t off = j * bits;
    const int64_t w = off >> 5;
    const int sh = (int)(off & 31);
    row[w] |= q << sh;
    if (sh + bits > 32) row[w + 1] |= q >> (32 - sh);
}

/*
 * mx.quantize(w, group_size, bits, mode="affine") for one matrix
 * [rows, cols], cols % group == 0.  Restates mlx's published affine
 * quantizer (mlx/backend/cpu/quantized.cpp, `quantize`), which callers in
 * the reference reach at src/knurlogic/engine/kvquant.py:46-47 and
 * .../_mlx_vlm/models/switch_layers.py:38-48:
 *   - per group: min and max in float32;
 *   - scale = max((max - min) / (2^bits - 1), 1e-7);
 *   - the edge with the larger magnitude is kept exact: if |min| > |max|
 *     the edge is min and the scale positive, else the edge is max and the
 *     scale negative;
 *   - q0 = rint(edge / scale); if q0 != 0 the scale is snapped to
 *     edge / q0 (so 0 is a code point) and bias = edge, else bias = 0;
 *   - q = clamp(rint((w - bias) / scale), 0, 2^bits - 1), using the float32
 *     scale and bias; scales and biases are then stored in w's dtype.
 * scales/biases are returned in float32 BEFORE that final rounding; the
 * Python side rounds them.
 */
void orc_quantize_affine(const float* w, int64_t rows, int64_t cols, int group,
                         int bits, uint32_t* wq, float* scales, float* biases) {
    const float n_bins = (float)((1u << bits) - 1u);
    const float eps = 1e-7f;
    const int64_t wpr = cols * bits / 32;
    const int64_t gpr = cols / group;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; r++) {
        const float* wr = w + r * cols;
        uint32_t* qr = wq + r * wpr;
        memset(qr, 0, sizeof(uint32_t) * (size_t)wpr);
        for (int64_t g = 0; g < gpr; g++) {
            const float* wg = wr + g * group;
            float w_max = -INFINITY, w_min = INFINITY;
            for (int i = 0; i < group; i++) {
                w_max = fmaxf(w_max, wg[i]);
                w_min = fminf(w_min, wg[i]);
            }
            int neg_edge = fabsf(w_min) > fabsf(w_max);
            float scale = fmaxf((w_max - w_min) / n_bins, eps);
            scale = neg_edge ? scale : -scale;
            float edge = neg_edge ? w_min : w_max;
            float q0 = rintf(edge / scale);
            float bias = 0.0f;
            if (q0 != 0.0f) {
                scale = edge / q0;
                bias = edge;
            }
            for (int i = 0; i < group; i++) {
                float q = rintf((wg[i] - bias) / scale);
                q = fminf(fmaxf(q, 0.0f), n_bins);
                pack_q(qr, g * group + i, bits, (uint32_t)q);
            }
            scales[r * gpr + g] = scale;
            biases[r * gpr + g] = bias;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* rounding helpers for dequantize                                           */
/* ------------------------------------------------------------------------ */

static inline float round_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) { /* NaN stays NaN */
        u |= 0x00400000u;
    } else {
        u += 0x7fffu + ((u >> 16) & 1u);
    }
    u &= 0xffff0000u;
    memcpy(&f, &u, 4);
    return f;
}

/* float -> nearest-even IEEE half, returned as float (exact). */
static inline float round_f16(float f) {
    if (isnan(f) || isinf(f)) return f;
    float a = fabsf(f);
    if (a >= 65520.0f) return copysignf(INFINITY, f);
    if (a < 6.103515625e-05f) { /* subnormal range: spacing 2^-24 */
        float q = rintf(a * 16777216.0f) / 16777216.0f;
        return copysignf(q, f);
    }
    int e;
    frexpf(a, &e);               /* a = m * 2^e, m in [0.5, 1) */
    float ulp = ldexpf(1.0f, e - 11);
    return copysignf(rintf(a / ulp) * ulp, f);
}

static inline float round_to(float f, int dtype) {
    if (dtype == 0) return round_bf16(f);
    if (dtype == 1) return round_f16(f);
    return f;
}

/*
 * mx.dequantize(w, scales, biases, group_size, bits, mode="affine",
 * dtype=...) -- reached in the reference at src/knurlogic/engine/kvquant.py:50-51.
 * The value is scale * q + bias (kvattn.py:142).  The storage rounding is
 * a switch because no frozen mlx vector pins it:
 *   rounding 0: the op-by-op order mlx's CPU fallback takes:
 *               out = T(T(scale * q) + bias)      (two roundings in T)
 *   rounding 1: one rounding of the fused float32 value:
 *               out = T(fmaf(scale, q, bias))
 * dtype: 0 bf16, 1 fp16, 2 fp32 (T).
 */
void orc_dequantize_affine(const uint32_t* wq, const float* scales,
                           const float* biases, int64_t rows, int64_t cols,
                           int group, int bits, int dtype, int rounding,
                           float* out) {
    const int64_t wpr = cols * bits / 32;
    const int64_t gpr = cols / group;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; r++) {
        for (int64_t j = 0; j < cols; j++) {
            float s = scales[r * gpr + j / group];
            float b = biases[r * gpr + j / group];
            float q = (float)unpack_q(wq + r * wpr, j, bits);
            float v;
            if (rounding == 0) {
                v = round_to(round_to(s * q, dtype) + b, dtype);
            } else {
                v = round_to(fmaf(s, q, b), dtype);
            }
            out[r * cols + j] = v;
        }
    }
}

/*
 * mx.quantized_matmul(x, w, scales, biases, transpose, group_size, bits)
 * (nn.QuantizedLinear, swapped in at src/knurlogic/engine/model/load_model.py:124-144;
 * wrapped at src/knurlogic/engine/matmul_padding.py:94-105).
 *   transpose = 1: w is [N, K*bits/32], y[m, n] = sum_k x[m,k] * What[n,k]
 *   transpose = 0: w is [K, N*bits/32], y[m, n] = sum_k x[m,k] * What[k,n]
 * What = scale * q + bias, exact in double; the sum in double.  Each output
 * row depends only on its input row (the row-independence contract of
 * tests/engine/test_per_chip_rounding.py:30-41).
 */
void orc_qmm(const float* x, int64_t M, int64_t K, int64_t N,
             const uint32_t* wq, const float* scales, const float* biases,
             int group, int bits, int transpose, float* y, int nthreads) {
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#else
    (void)nthreads;
#endif
    if (transpose) {
        const int64_t wpr = K * bits / 32, gpr = K / group;
#pragma omp parallel
        {
            double* wrow = (double*)malloc(sizeof(double) * (size_t)K);
#pragma omp for schedule(static)
            for (int64_t n = 0; n < N; n++) {
                const uint32_t* qr = wq + n * wpr;
                for (int64_t k = 0; k < K; k++) {
                    double s = scales[n * gpr + k / group];
                    double b = biases[n * gpr + k / group];
                    wrow[k] = s * (double)unpack_q(qr, k, bits) + b;
                }
                for (int64_t m = 0; m < M; m++) {
                    const float* xr = x + m * K;
                    double acc = 0.0;
                    for (int64_t k = 0; k < K; k++) acc += (double)xr[k] * wrow[k];
                    y[m * N + n] = (float)acc;
                }
            }
            free(wrow);
        }
    } else {
        const int64_t wpr = N * bits / 32, gpr = N / group;
#pragma omp parallel
        {
            double* acc = (double*)malloc(sizeof(double) * (size_t)N);
            double* wrow = (double*)malloc(sizeof(double) * (size_t)N);
#pragma omp for schedule(static)
            for (int64_t m = 0; m < M; m++) {
                memset(acc, 0, sizeof(double) * (size_t)N);
                for (int64_t k = 0; k < K; k++) {
                    const uint32_t* qr = wq + k * wpr;
                    for (int64_t n = 0; n < N; n++) {
                        double s = scales[k * gpr + n / group];
                        double b = biases[k * gpr + n / group];
                        wrow[n] = s * (double)unpack_q(qr, n, bits) + b;
                    }
                    double xv = x[m * K + k];
                    for (int64_t n = 0; n < N; n++) acc[n] += xv * wrow[n];
                }
                for (int64_t n = 0; n < N; n++) y[m * N + n] = (float)acc[n];
            }
            free(acc);
            free(wrow);
        }
    }
}

/*
 * 8-bit-KV decode attention with the semantics of the reference's
 * kvattn.decode_sdpa (src/knurlogic/engine/kvattn.py:256-291, kernels
 * :78-183):
 *   - q [B, H, L, D], K/V packed [B, Hk, N, D*bits/32] with scales and
 *     biases [B, Hk, N, D/group]; query head h reads KV head h / (H/Hk);
 *   - q is pre-multiplied by `scale` (:101);
 *   - score(n) = sum_d (q_d*scale) * (ks*k_d + kb)    (:148-150, exact here)
 *   - softmax over the keys row (b, l) may see (mask [B, L, N], 1 = seen;
 *     NULL = every key), out = sum p * (vs*v + vb)    (:142, :155);
 *   - a row with every key masked returns 0 (:11-12, :182).
 * All arrays contiguous; out [B, H, L, D].
 */
void orc_kv8_decode(const float* q, int64_t B, int64_t H, int64_t L, int64_t D,
                    const uint32_t* kw, const float* ks, const float* kb,
                    const uint32_t* vw, const float* vs, const float* vb,
                    int64_t Hk, int64_t N, int group, int bits, float scale,
                    const uint8_t* mask, float* out, int nthreads) {
    const int64_t wpr = D * bits / 32, gpr = D / group;
    const int64_t rep = H / Hk;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#else
    (void)nthreads;
#endif
    /* one (batch, KV head) per task: its K/V dequantized once, exactly */
#pragma omp parallel for schedule(dynamic, 1) collapse(2)
    for (int64_t b = 0; b < B; b++)
        for (int64_t hk = 0; hk < Hk; hk++) {
            double* kd = (double*)malloc(sizeof(double) * (size_t)(N * D + 1));
            double* vd = (double*)malloc(sizeof(double) * (size_t)(N * D + 1));
            double* sc = (double*)malloc(sizeof(double) * (size_t)(N + 1));
            double* qs = (double*)malloc(sizeof(double) * (size_t)D);
            double* o = (double*)malloc(sizeof(double) * (size_t)D);
            for (int64_t n = 0; n < N; n++) {
                const int64_t row = (b * Hk + hk) * N + n;
                for (int64_t d = 0; d < D; d++) {
                    kd[n * D + d] = (double)ks[row * gpr + d / group] *
                                        (double)unpack_q(kw + row * wpr, d, bits) +
                                    (double)kb[row * gpr + d / group];
                    vd[n * D + d] = (double)vs[row * gpr + d / group] *
                                        (double)unpack_q(vw + row * wpr, d, bits) +
                                    (double)vb[row * gpr + d / group];
                }
            }
            for (int64_t h = hk * rep; h < (hk + 1) * rep; h++)
                for (int64_t l = 0; l < L; l++) {
                    const float* qr = q + ((b * H + h) * L + l) * D;
                    for (int64_t d = 0; d < D; d++) qs[d] = (double)(qr[d] * scale);
                    double mx = -INFINITY;
                    int any = 0;
                    for (int64_t n = 0; n < N; n++) {
                        if (mask && !mask[(b * L + l) * N + n]) {
                            sc[n] = -INFINITY;
                            continue;
                        }
                        double s = 0.0;
                        const double* kr = kd + n * D;
                        for (int64_t d = 0; d < D; d++) s += qs[d] * kr[d];
                        sc[n] = s;
                        any = 1;
                        if (s > mx) mx = s;
                    }
                    float* orow = out + ((b * H + h) * L + l) * D;
                    if (!any) {
                        for (int64_t d = 0; d < D; d++) orow[d] = 0.0f;
                        continue;
                    }
                    double den = 0.0;
                    for (int64_t d = 0; d < D; d++) o[d] = 0.0;
                    for (int64_t n = 0; n < N; n++) {
                        if (sc[n] == -INFINITY) continue;
                        const double p = exp(sc[n] - mx);
                        den += p;
                        const double* vr = vd + n * D;
                        for (int64_t d = 0; d < D; d++) o[d] += p * vr[d];
                    }
                    for (int64_t d = 0; d < D; d++) orow[d] = (float)(o[d] / den);
                }
            free(kd);
            free(vd);
            free(sc);
            free(qs);
            free(o);
        }
}

/*
 * VQ codebook-decode matmul for one expert matrix [OUT, IN]:
 *   What[o, i] = scale[o, i / scale_group] * codebook[code[o, i / dim]][i % dim]
 *   y[m, o]    = sum_i x[m, i] * What[o, i]
 * codes are uint8 (code_bytes 1) or uint16 (code_bytes 2), [OUT, IN/dim];
 * codebook [kc, dim]; scale_group = IN gives one scale per output channel.
 * The decode rule is the one the reference's VQ artifacts declare through
 * their `vq_modules` schema (codes / codebook / vq_scales;
 * tests/engine/test_deepseek_v4_mtp.py:206-233 of the reference).
 */
void orc_vq_matmul(const float* x, int64_t M, int64_t IN, int64_t OUT,
                   const void* codes, int code_bytes, const float* codebook,
                   int64_t kc, int dim, const float* scales, int64_t scale_group,
                   float* y, int nthreads) {
    const int64_t cpr = IN / dim, spr = IN / scale_group;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#else
    (void)nthreads;
#endif
    (void)kc;
#pragma omp parallel
    {
        double* wrow = (double*)malloc(sizeof(double) * (size_t)IN);
#pragma omp for schedule(static)
        for (int64_t o = 0; o < OUT; o++) {
            for (int64_t c = 0; c < cpr; c++) {
                int64_t idx = code_bytes == 1 ? ((const uint8_t*)codes)[o * cpr + c]
                                              : ((const uint16_t*)codes)[o * cpr + c];
                for (int d = 0; d < dim; d++) {
                    int64_t i = c * dim + d;
                    wrow[i] = (double)scales[o * spr + i / scale_group] *
                              (double)codebook[idx * dim + d];
                }
            }
            for (int64_t m = 0; m < M; m++) {
                double acc = 0.0;
                const float* xr = x + m * IN;
                for (int64_t i = 0; i < IN; i++) acc += (double)xr[i] * wrow[i];
                y[m * OUT + o] = (float)acc;
            }
        }
        free(wrow);
    }
}

int orc_abi_version(void) { return 1; }
