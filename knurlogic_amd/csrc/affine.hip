// Affine group quantize / dequantize (mx.quantize / mx.dequantize, mode
// "affine") for gfx950.  One thread per group: a group is at most 128
// elements, read with 16-byte loads; both ops are bandwidth-trivial next to
// the matmuls (weights are quantized offline; the KV cache quantizes one
// new token per layer per step).
#include "common.hpp"
#include "../../include/knurlogic_amd.h"

#include <string.h>
#include <math.h>

namespace kmi {

static thread_local char g_err[512];

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

void clear_error() { g_err[0] = 0; }

// mlx's affine quantizer for one group (restated; the oracle's
// orc_quantize_affine follows the same steps in the same float32 order).
template <typename T, int BITS>
__global__ __launch_bounds__(256) void quantize_kernel(
    const typename T::storage* __restrict__ w, int64_t n_groups, int group,
    uint32_t* __restrict__ wq, typename T::storage* __restrict__ scales,
    typename T::storage* __restrict__ biases) {
    const int64_t gi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gi >= n_groups) return;
    const typename T::storage* wg = w + gi * group;
    const float n_bins = (float)((1u << BITS) - 1u);
    float w_max = -INFINITY, w_min = INFINITY;
    for (int i = 0; i < group; i++) {
        float v = T::load(wg[i]);
        w_max = fmaxf(w_max, v);
        w_min = fminf(w_min, v);
    }
    const bool neg_edge = fabsf(w_min) > fabsf(w_max);
    float scale = fmaxf((w_max - w_min) / n_bins, 1e-7f);
    scale = neg_edge ? scale : -scale;
    const float edge = neg_edge ? w_min : w_max;
    const float q0 = rintf(edge / scale);
    float bias = 0.0f;
    if (q0 != 0.0f) {
        scale = edge / q0;
        bias = edge;
    }
    constexpr int EPW = 32 / BITS;
    uint32_t* qg = wq + gi * (group / EPW);
    for (int wi = 0; wi < group / EPW; wi++) {
        uint32_t word = 0;
#pragma unroll
        for (int e = 0; e < EPW; e++) {
            float q = rintf((T::load(wg[wi * EPW + e]) - bias) / scale);
            q = fminf(fmaxf(q, 0.0f), n_bins);
            word |= ((uint32_t)q) << (e * BITS);
        }
        qg[wi] = word;
    }
    scales[gi] = T::store(scale);
    biases[gi] = T::store(bias);
}

// out = T(T(s*q) + b) (rounding 0) or T(fma(s, q, b)) (rounding 1); one
// thread per packed word.
template <typename TS, typename TO, int BITS>
__global__ __launch_bounds__(256) void dequantize_kernel(
    const uint32_t* __restrict__ wq, const typename TS::storage* __restrict__ scales,
    const typename TS::storage* __restrict__ biases, int64_t n_words, int group,
    int rounding, typename TO::storage* __restrict__ out) {
    const int64_t wi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (wi >= n_words) return;
    constexpr int EPW = 32 / BITS;
    constexpr uint32_t MASK = (1u << BITS) - 1u;
    const int64_t e0 = wi * EPW;
    const int64_t g = e0 / group;
    const float s = TS::load(scales[g]);
    const float b = TS::load(biases[g]);
    const uint32_t word = wq[wi];
#pragma unroll
    for (int e = 0; e < EPW; e++) {
        const float q = (float)((word >> (e * BITS)) & MASK);
        float v;
        if (rounding == 0) {
            v = TO::round(__fadd_rn(TO::round(__fmul_rn(s, q)), b));
        } else {
            v = TO::round(__builtin_fmaf(s, q, b));
        }
        out[e0 + e] = TO::store(v);
    }
}

template <typename T>
static void launch_quantize(const void* w, int64_t n_groups, int group, int bits,
                            uint32_t* wq, void* s, void* b, hipStream_t st) {
    dim3 grid((unsigned)ceil_div(n_groups, 256));
    using S = typename T::storage;
    if (bits == 4)
        quantize_kernel<T, 4><<<grid, 256, 0, st>>>((const S*)w, n_groups, group, wq, (S*)s, (S*)b);
    else if (bits == 8)
        quantize_kernel<T, 8><<<grid, 256, 0, st>>>((const S*)w, n_groups, group, wq, (S*)s, (S*)b);
    else
        quantize_kernel<T, 2><<<grid, 256, 0, st>>>((const S*)w, n_groups, group, wq, (S*)s, (S*)b);
}

template <typename TS, typename TO>
static void launch_dequantize(const uint32_t* wq, const void* s, const void* b,
                              int64_t n_words, int group, int bits, int rounding,
                              void* out, hipStream_t st) {
    dim3 grid((unsigned)ceil_div(n_words, 256));
    using SS = typename TS::storage;
    using SO = typename TO::storage;
    if (bits == 4)
        dequantize_kernel<TS, TO, 4><<<grid, 256, 0, st>>>(wq, (const SS*)s, (const SS*)b, n_words, group, rounding, (SO*)out);
    else if (bits == 8)
        dequantize_kernel<TS, TO, 8><<<grid, 256, 0, st>>>(wq, (const SS*)s, (const SS*)b, n_words, group, rounding, (SO*)out);
    else
        dequantize_kernel<TS, TO, 2><<<grid, 256, 0, st>>>(wq, (const SS*)s, (const SS*)b, n_words, group, rounding, (SO*)out);
}

}  // namespace kmi

using namespace kmi;

extern "C" {

const char* kmi_last_error(void) { return g_err; }

int kmi_abi_version(void) { return KMI_ABI_VERSION; }

int kmi_quantize_affine(const void* w, int dtype, int64_t rows, int64_t cols,
                        int group_size, int bits, uint32_t* wq, void* scales,
                        void* biases, void* stream) {
    clear_error();
    KMI_CHECK_ARG(w && wq && scales && biases, "quantize: null pointer");
    KMI_CHECK_ARG(bits == 2 || bits == 4 || bits == 8, "quantize: bits %d not in {2,4,8}", bits);
    KMI_CHECK_ARG(group_size == 32 || group_size == 64 || group_size == 128,
                  "quantize: group_size %d not in {32,64,128}", group_size);
    KMI_CHECK_ARG(rows >= 0 && cols > 0 && cols % group_size == 0,
                  "quantize: last axis %lld is not a multiple of the group %d", (long long)cols, group_size);
    KMI_CHECK_ARG(dtype >= BF16 && dtype <= F32, "quantize: bad dtype %d", dtype);
    const int64_t n_groups = rows * (cols / group_size);
    if (n_groups == 0) return OK;
    hipStream_t st = (hipStream_t)stream;
    if (dtype == BF16) launch_quantize<TBF16>(w, n_groups, group_size, bits, wq, scales, biases, st);
    else if (dtype == F16) launch_quantize<TF16>(w, n_groups, group_size, bits, wq, scales, biases, st);
    else launch_quantize<TF32>(w, n_groups, group_size, bits, wq, scales, biases, st);
    KMI_CHECK_LAUNCH("quantize");
    return OK;
}

int kmi_dequantize_affine(const uint32_t* wq, const void* scales, const void* biases,
                          int scale_dtype, int64_t rows, int64_t cols, int group_size,
                          int bits, void* out, int out_dtype, int rounding, void* stream) {
    clear_error();
    KMI_CHECK_ARG(wq && scales && biases && out, "dequantize: null pointer (affine needs biases)");
    KMI_CHECK_ARG(bits == 2 || bits == 4 || bits == 8, "dequantize: bits %d not in {2,4,8}", bits);
    KMI_CHECK_ARG(group_size == 32 || group_size == 64 || group_size == 128,
                  "dequantize: group_size %d not in {32,64,128}", group_size);
    KMI_CHECK_ARG(rows >= 0 && cols > 0 && cols % group_size == 0, "dequantize: bad shape");
    KMI_CHECK_ARG(rounding == 0 || rounding == 1, "dequantize: rounding %d not in {0,1}", rounding);
    KMI_CHECK_ARG(scale_dtype >= BF16 && scale_dtype <= F32 && out_dtype >= BF16 && out_dtype <= F32,
                  "dequantize: bad dtype");
    const int64_t n_words = rows * cols * bits / 32;
    if (n_words == 0) return OK;
    hipStream_t st = (hipStream_t)stream;
#define KMI_DQ(TS, TO) launch_dequantize<TS, TO>(wq, scales, biases, n_words, group_size, bits, rounding, out, st)
    if (scale_dtype == BF16) {
        if (out_dtype == BF16) KMI_DQ(TBF16, TBF16);
        else if (out_dtype == F16) KMI_DQ(TBF16, TF16);
        else KMI_DQ(TBF16, TF32);
    } else if (scale_dtype == F16) {
        if (out_dtype == BF16) KMI_DQ(TF16, TBF16);
        else if (out_dtype == F16) KMI_DQ(TF16, TF16);
        else KMI_DQ(TF16, TF32);
    } else {
        if (out_dtype == BF16) KMI_DQ(TF32, TBF16);
        else if (out_dtype == F16) KMI_DQ(TF32, TF16);
        else KMI_DQ(TF32, TF32);
    }
#undef KMI_DQ
    KMI_CHECK_LAUNCH("dequantize");
    return OK;
}

}  // extern "C"
