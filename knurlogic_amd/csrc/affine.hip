// Affine group quantize / dequantize (mx.quantize / mx.dequantize, mode
// "affine") for gfx950, and the KV cache's quantize-on-append.  Quantize:
// GS/8 lanes per group, 8 elements per lane in one 16-byte load, the group's
// min / max exchanged by lane shuffles.  Dequantize: one thread per packed
// word.  All are HBM-bound element passes.
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

// mlx's affine quantizer (restated; the oracle's orc_quantize_affine follows
// the same steps in the same float32 order), one group per GS/8 consecutive
// lanes: each lane loads 8 consecutive elements (one 16-byte load for 16-bit
// types), min / max are exchanged across the group's lanes, every lane
// derives the same scale and bias and quantizes its own 8 elements.  Where
// the packed words and scales go: contiguous (quantize), or KV-cache slab
// slots (append).
struct QuantDst {
    uint32_t* wq;
    void* scales;
    void* biases;
    int64_t wst[3], sst[3];     // append: element strides (b, h, n) of wq and of scales / biases
    int64_t pos, H, S;          // append: first slot, heads, new rows per head
    int kv;                     // 0: contiguous [groups] layout, 1: slab slots
};

template <typename T, int BITS, int GS>
__device__ __forceinline__ void quantize_body(const typename T::storage* __restrict__ w, int64_t n_groups,
                                              int64_t D, const QuantDst& d) {
    constexpr int LPG = GS / 8;                  // lanes per group
    using St = typename T::storage;
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t gi = t / LPG;
    const int sub = (int)(t % LPG);
    const bool live = gi < n_groups;             // whole groups are live or not (LPG divides 64)
    float v[8];
    const St* src = w + (live ? gi : 0) * GS + sub * 8;
    if constexpr (sizeof(St) == 2) {
        const u32x4 r = *(const u32x4*)src;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            v[2 * e] = T::load((St)(r[e] & 0xffffu));
            v[2 * e + 1] = T::load((St)(r[e] >> 16));
        }
    } else {
        const float4 r0 = *(const float4*)src, r1 = *(const float4*)(src + 4);
        v[0] = r0.x; v[1] = r0.y; v[2] = r0.z; v[3] = r0.w;
        v[4] = r1.x; v[5] = r1.y; v[6] = r1.z; v[7] = r1.w;
    }
    float w_max = -INFINITY, w_min = INFINITY;
#pragma unroll
    for (int e = 0; e < 8; e++) {
        w_max = fmaxf(w_max, v[e]);
        w_min = fminf(w_min, v[e]);
    }
#pragma unroll
    for (int o = 1; o < LPG; o <<= 1) {
        w_max = fmaxf(w_max, __shfl_xor(w_max, o, 64));
        w_min = fminf(w_min, __shfl_xor(w_min, o, 64));
    }
    const float n_bins = (float)((1u << BITS) - 1u);
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
    uint64_t bitsv = 0;                          // this lane's 8 codes (8 * BITS bits, low first)
#pragma unroll
    for (int e = 0; e < 8; e++) {
        float q = rintf((v[e] - bias) / scale);
        q = fminf(fmaxf(q, 0.0f), n_bins);
        bitsv |= (uint64_t)q << (e * BITS);
    }
    if (!live) return;
    // destination of this group's words and of its scale / bias
    int64_t wo, so;
    if (d.kv) {
        const int64_t gpr = D / GS;
        const int64_t r = gi / gpr, gs = gi % gpr;
        const int64_t s = r % d.S, bh = r / d.S, h = bh % d.H, b = bh / d.H;
        const int64_t n = d.pos + s;
        wo = b * d.wst[0] + h * d.wst[1] + n * d.wst[2] + gs * (GS * BITS / 32);
        so = b * d.sst[0] + h * d.sst[1] + n * d.sst[2] + gs;
    } else {
        wo = gi * (GS * BITS / 32);
        so = gi;
    }
    if constexpr (BITS == 8) {
        d.wq[wo + 2 * sub] = (uint32_t)bitsv;    // word strides need only be 4-byte multiples
        d.wq[wo + 2 * sub + 1] = (uint32_t)(bitsv >> 32);
    } else if constexpr (BITS == 4) {
        d.wq[wo + sub] = (uint32_t)bitsv;
    } else if constexpr (BITS == 2) {            // two lanes per word
        const uint32_t other = __shfl_xor((uint32_t)bitsv, 1, 64);
        if ((sub & 1) == 0) d.wq[wo + sub / 2] = (uint32_t)bitsv | (other << 16);
    } else {                                     // 3, 5, 6 bits: BITS whole bytes per lane
        unsigned char* dst = (unsigned char*)(d.wq + wo) + sub * BITS;
#pragma unroll
        for (int i = 0; i < BITS; i++) dst[i] = (unsigned char)(bitsv >> (8 * i));
    }
    if (sub == 0) {
        ((St*)d.scales)[so] = T::store(scale);
        ((St*)d.biases)[so] = T::store(bias);
    }
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

template <typename T, int BITS, int GS>
__global__ __launch_bounds__(256) void quantize_kernel(const typename T::storage* __restrict__ w,
                                                       int64_t n_groups, int64_t D, QuantDst d) {
    quantize_body<T, BITS, GS>(w, n_groups, D, d);
}

// K and V of one KV-cache append in one launch: grid y picks the tensor.
template <typename T, int BITS, int GS>
__global__ __launch_bounds__(256) void quantize_kv_kernel(const typename T::storage* __restrict__ k, int64_t nk,
                                                          int64_t Dk, QuantDst dk,
                                                          const typename T::storage* __restrict__ v, int64_t nv,
                                                          int64_t Dv, QuantDst dv) {
    if (blockIdx.y == 0) quantize_body<T, BITS, GS>(k, nk, Dk, dk);
    else quantize_body<T, BITS, GS>(v, nv, Dv, dv);
}

// 3, 5 and 6 bits: one thread per 8 elements (BITS whole bytes of the
// row's bit stream).
template <typename TS, typename TO, int BITS>
__global__ __launch_bounds__(256) void dequantize_bytes_kernel(
    const uint32_t* __restrict__ wq, const typename TS::storage* __restrict__ scales,
    const typename TS::storage* __restrict__ biases, int64_t n_units, int group,
    int rounding, typename TO::storage* __restrict__ out) {
    const int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (u >= n_units) return;
    const unsigned char* src = (const unsigned char*)wq + u * BITS;
    uint64_t v = 0;
#pragma unroll
    for (int i = 0; i < BITS; i++) v |= (uint64_t)src[i] << (8 * i);
    const int64_t e0 = u * 8;
    const int64_t g = e0 / group;
    const float s = TS::load(scales[g]);
    const float b = TS::load(biases[g]);
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const float q = (float)((v >> (BITS * e)) & ((1u << BITS) - 1u));
        const float r = rounding == 0 ? TO::round(__fadd_rn(TO::round(__fmul_rn(s, q)), b))
                                      : TO::round(__builtin_fmaf(s, q, b));
        out[e0 + e] = TO::store(r);
    }
}

// mx.dequantize(mode="mxfp4" / "mxfp8"): E2M1 / E4M3 elements times the
// E8M0 scale (2^(e - 127)) of their group of 32; one thread per packed word.
__device__ __forceinline__ float mx_e8m0(uint32_t e) { return e8m0_to_f32(e); }

__device__ __forceinline__ float mx_elem(uint32_t c, int mode) {
    if (mode == 1) {                              // E2M1
        const uint32_t e = (c >> 1) & 3u, m = c & 1u;
        const float mag = e ? __uint_as_float(((e + 126u) << 23) | (m << 22)) : (m ? 0.5f : 0.0f);
        return (c & 8u) ? -mag : mag;
    }
    const uint32_t e = (c >> 3) & 15u, m = c & 7u;  // E4M3
    float mag;
    if (e == 15u && m == 7u) mag = __uint_as_float(0x7fc00000u);
    else if (e == 0u) mag = (float)m * 0.001953125f;
    else mag = __uint_as_float(((e + 120u) << 23) | (m << 20));
    return (c & 0x80u) ? -mag : mag;
}

// mx.quantize(mode="mxfp4" / "mxfp8"), one thread per group of 32: the
// OCP shared exponent X = floor(log2 max|w|) - emax (2 for E2M1, 8 for
// E4M3) as E8M0 byte X + 127 (an all-zero group: 0), elements w / 2^X to
// the nearest code (rintf: ties to the even code, the codes of a binade
// being consecutive), saturated, the input's sign kept (negative zeros too).
__device__ __forceinline__ uint32_t mx_code(float v, int mode) {
    const uint32_t sign = __float_as_uint(v) >> 31;
    const float a = fabsf(v);
    uint32_t c;
    if (mode == 1) {                                       // E2M1: emin 0, 1 mantissa bit, max 6 = code 7
        if (a >= 6.0f) c = 7;
        else if (a < 1.0f) c = (uint32_t)rintf(a * 2.0f);  // 0, 0.5, 1.0 (code 2)
        else {
            const int e = (int)((__float_as_uint(a) >> 23) & 0xff) - 127;
            c = (uint32_t)(((e + 1) << 1) + (int)rintf((a * __uint_as_float((uint32_t)(127 - e) << 23) - 1.0f) * 2.0f));
        }
        return c > 7 ? 7 | (sign << 3) : c | (sign << 3);
    }
    if (a >= 448.0f) c = 0x7e;                             // E4M3: max 448 = 0x7e
    else if (a < 0.015625f) c = (uint32_t)rintf(a * 512.0f);   // subnormals m * 2^-9 (code 8 = 2^-6)
    else {
        const int e = (int)((__float_as_uint(a) >> 23) & 0xff) - 127;
        c = (uint32_t)(((e + 7) << 3) + (int)rintf((a * __uint_as_float((uint32_t)(127 - e) << 23) - 1.0f) * 8.0f));
    }
    if (c > 0x7e) c = 0x7e;
    return c | (sign << 7);
}

template <typename T>
__global__ __launch_bounds__(256) void quantize_mx_kernel(const typename T::storage* __restrict__ w, int64_t n_groups,
                                                          int mode, uint32_t* __restrict__ wq,
                                                          uint8_t* __restrict__ scales) {
    const int64_t gi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gi >= n_groups) return;
    const typename T::storage* src = w + gi * 32;
    float amax = 0.f;
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(T::load(src[i])));
    const int emax = mode == 1 ? 2 : 8;
    int eb = 0;
    if (amax > 0.f) {
        const int e = (int)((__float_as_uint(amax) >> 23) & 0xff);     // biased exponent (normal range)
        eb = e == 0 ? 0 : e - emax;                                     // X + 127, X = floor(log2 amax) - emax
        eb = eb < 0 ? 0 : eb > 254 ? 254 : eb;
    }
    const float inv = eb >= 1 ? __uint_as_float((uint32_t)(254 - eb) << 23) : __uint_as_float(0x7f000000u);
    const int bits = mode == 1 ? 4 : 8, epw = 32 / bits;
    for (int wd = 0; wd < 32 / epw; wd++) {
        uint32_t word = 0;
        for (int e = 0; e < epw; e++) word |= mx_code(T::load(src[wd * epw + e]) * inv, mode) << (bits * e);
        wq[gi * (32 / epw) + wd] = word;
    }
    scales[gi] = (uint8_t)eb;
}

template <typename TO>
__global__ __launch_bounds__(256) void dequantize_mx_kernel(const uint32_t* __restrict__ wq,
                                                            const uint8_t* __restrict__ scales, int64_t n_words,
                                                            int mode, typename TO::storage* __restrict__ out) {
    const int64_t wi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (wi >= n_words) return;
    const int bits = mode == 1 ? 4 : 8, epw = 32 / bits;
    const int64_t e0 = wi * epw;
    const float s = mx_e8m0(scales[e0 / 32]);
    const uint32_t w = wq[wi];
    for (int e = 0; e < epw; e++)
        out[e0 + e] = TO::store(mx_elem((w >> (bits * e)) & ((1u << bits) - 1u), mode) * s);
}

template <typename T, int BITS>
static void launch_quantize_b(const void* w, int64_t n_groups, int group, int64_t D, const QuantDst& d,
                              hipStream_t st) {
    using S = typename T::storage;
    const int64_t threads = n_groups * (group / 8);
    dim3 grid((unsigned)ceil_div(threads, 256));
    if (group == 32) quantize_kernel<T, BITS, 32><<<grid, 256, 0, st>>>((const S*)w, n_groups, D, d);
    else if (group == 64) quantize_kernel<T, BITS, 64><<<grid, 256, 0, st>>>((const S*)w, n_groups, D, d);
    else quantize_kernel<T, BITS, 128><<<grid, 256, 0, st>>>((const S*)w, n_groups, D, d);
}

template <typename T, int BITS>
static void launch_quantize_kv_b(const void* k, int64_t nk, int64_t Dk, const QuantDst& dk, const void* v,
                                 int64_t nv, int64_t Dv, const QuantDst& dv, int group, hipStream_t st) {
    using S = typename T::storage;
    const int64_t n = nk > nv ? nk : nv;
    dim3 grid((unsigned)ceil_div(n * (group / 8), 256), 2);
#define KMI_QKV(G_) quantize_kv_kernel<T, BITS, G_><<<grid, 256, 0, st>>>((const S*)k, nk, Dk, dk, (const S*)v, nv, Dv, dv)
    if (group == 32) KMI_QKV(32);
    else if (group == 64) KMI_QKV(64);
    else KMI_QKV(128);
#undef KMI_QKV
}

template <typename T>
static void launch_quantize_kv(const void* k, int64_t nk, int64_t Dk, const QuantDst& dk, const void* v,
                               int64_t nv, int64_t Dv, const QuantDst& dv, int group, int bits, hipStream_t st) {
    if (bits == 4) launch_quantize_kv_b<T, 4>(k, nk, Dk, dk, v, nv, Dv, dv, group, st);
    else if (bits == 8) launch_quantize_kv_b<T, 8>(k, nk, Dk, dk, v, nv, Dv, dv, group, st);
    else if (bits == 3) launch_quantize_kv_b<T, 3>(k, nk, Dk, dk, v, nv, Dv, dv, group, st);
    else if (bits == 5) launch_quantize_kv_b<T, 5>(k, nk, Dk, dk, v, nv, Dv, dv, group, st);
    else if (bits == 6) launch_quantize_kv_b<T, 6>(k, nk, Dk, dk, v, nv, Dv, dv, group, st);
    else launch_quantize_kv_b<T, 2>(k, nk, Dk, dk, v, nv, Dv, dv, group, st);
}

template <typename T>
static void launch_quantize(const void* w, int64_t n_groups, int group, int bits, int64_t D,
                            const QuantDst& d, hipStream_t st) {
    if (bits == 4) launch_quantize_b<T, 4>(w, n_groups, group, D, d, st);
    else if (bits == 8) launch_quantize_b<T, 8>(w, n_groups, group, D, d, st);
    else if (bits == 3) launch_quantize_b<T, 3>(w, n_groups, group, D, d, st);
    else if (bits == 5) launch_quantize_b<T, 5>(w, n_groups, group, D, d, st);
    else if (bits == 6) launch_quantize_b<T, 6>(w, n_groups, group, D, d, st);
    else launch_quantize_b<T, 2>(w, n_groups, group, D, d, st);
}

template <typename TS, typename TO>
static void launch_dequantize(const uint32_t* wq, const void* s, const void* b,
                              int64_t n_words, int group, int bits, int rounding,
                              void* out, hipStream_t st) {
    dim3 grid((unsigned)ceil_div(n_words, 256));
    using SS = typename TS::storage;
    using SO = typename TO::storage;
    if (32 % bits) {                   // n_words counts 8-element units here
        if (bits == 3)
            dequantize_bytes_kernel<TS, TO, 3><<<grid, 256, 0, st>>>(wq, (const SS*)s, (const SS*)b, n_words, group, rounding, (SO*)out);
        else if (bits == 5)
            dequantize_bytes_kernel<TS, TO, 5><<<grid, 256, 0, st>>>(wq, (const SS*)s, (const SS*)b, n_words, group, rounding, (SO*)out);
        else
            dequantize_bytes_kernel<TS, TO, 6><<<grid, 256, 0, st>>>(wq, (const SS*)s, (const SS*)b, n_words, group, rounding, (SO*)out);
        return;
    }
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
    KMI_CHECK_ARG(bits >= 2 && bits <= 8 && bits != 7, "quantize: bits %d not in {2,3,4,5,6,8}", bits);
    KMI_CHECK_ARG(group_size == 32 || group_size == 64 || group_size == 128,
                  "quantize: group_size %d not in {32,64,128}", group_size);
    KMI_CHECK_ARG(rows >= 0 && cols > 0 && cols % group_size == 0,
                  "quantize: last axis %lld is not a multiple of the group %d", (long long)cols, group_size);
    KMI_CHECK_ARG(dtype >= BF16 && dtype <= F32, "quantize: bad dtype %d", dtype);
    const int64_t n_groups = rows * (cols / group_size);
    if (n_groups == 0) return OK;
    KMI_CHECK_ARG(((uintptr_t)w & 15) == 0, "quantize: w must be 16-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    QuantDst d = {};
    d.wq = wq; d.scales = scales; d.biases = biases; d.kv = 0;
    if (dtype == BF16) launch_quantize<TBF16>(w, n_groups, group_size, bits, cols, d, st);
    else if (dtype == F16) launch_quantize<TF16>(w, n_groups, group_size, bits, cols, d, st);
    else launch_quantize<TF32>(w, n_groups, group_size, bits, cols, d, st);
    KMI_CHECK_LAUNCH("quantize");
    return OK;
}

int kmi_kv_quantize_append(const void* x, int dtype, int64_t B, int64_t H, int64_t S, int64_t D,
                           int group_size, int bits, uint32_t* wq, void* scales, void* biases,
                           const int64_t* strides, int64_t pos, int64_t capacity, void* stream) {
    clear_error();
    KMI_CHECK_ARG(x && wq && scales && biases && strides, "kv_quantize_append: null pointer");
    KMI_CHECK_ARG(bits >= 2 && bits <= 8 && bits != 7, "kv_quantize_append: bits %d not in {2,3,4,5,6,8}",
                  bits);
    KMI_CHECK_ARG(group_size == 32 || group_size == 64 || group_size == 128,
                  "kv_quantize_append: group_size %d not in {32,64,128}", group_size);
    KMI_CHECK_ARG(B >= 0 && H >= 0 && S >= 0 && D > 0 && D % group_size == 0,
                  "kv_quantize_append: head dim %lld is not a multiple of the group %d", (long long)D,
                  group_size);
    KMI_CHECK_ARG(dtype >= BF16 && dtype <= F32, "kv_quantize_append: bad dtype %d", dtype);
    KMI_CHECK_ARG(pos >= 0 && pos + S <= capacity,
                  "kv_quantize_append: slots %lld..%lld past the slab capacity %lld", (long long)pos,
                  (long long)(pos + S), (long long)capacity);
    QuantDst d = {};
    d.wq = wq; d.scales = scales; d.biases = biases; d.pos = pos; d.H = H; d.S = S; d.kv = 1;
    for (int i = 0; i < 3; i++) {
        KMI_CHECK_ARG(strides[i] >= 0 && strides[3 + i] >= 0, "kv_quantize_append: negative stride");
        d.wst[i] = strides[i];
        d.sst[i] = strides[3 + i];
    }
    const int64_t n_groups = B * H * S * (D / group_size);
    if (n_groups == 0) return OK;
    KMI_CHECK_ARG(((uintptr_t)x & 15) == 0, "kv_quantize_append: x must be 16-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    if (dtype == BF16) launch_quantize<TBF16>(x, n_groups, group_size, bits, D, d, st);
    else if (dtype == F16) launch_quantize<TF16>(x, n_groups, group_size, bits, D, d, st);
    else launch_quantize<TF32>(x, n_groups, group_size, bits, D, d, st);
    KMI_CHECK_LAUNCH("kv_quantize_append");
    return OK;
}

int kmi_kv_quantize_append_kv(const void* k, const void* v, int dtype, int64_t B, int64_t H, int64_t S,
                              int64_t Dk, int64_t Dv, int group_size, int bits, uint32_t* k_wq, void* k_scales,
                              void* k_biases, const int64_t* k_strides, uint32_t* v_wq, void* v_scales,
                              void* v_biases, const int64_t* v_strides, int64_t pos, int64_t capacity,
                              void* stream) {
    clear_error();
    KMI_CHECK_ARG(k && v && k_wq && k_scales && k_biases && k_strides && v_wq && v_scales && v_biases && v_strides,
                  "kv_quantize_append: null pointer");
    KMI_CHECK_ARG(bits >= 2 && bits <= 8 && bits != 7, "kv_quantize_append: bits %d not in {2,3,4,5,6,8}",
                  bits);
    KMI_CHECK_ARG(group_size == 32 || group_size == 64 || group_size == 128,
                  "kv_quantize_append: group_size %d not in {32,64,128}", group_size);
    KMI_CHECK_ARG(B >= 0 && H >= 0 && S >= 0 && Dk > 0 && Dv > 0 && Dk % group_size == 0 && Dv % group_size == 0,
                  "kv_quantize_append: head dims %lld / %lld are not multiples of the group %d", (long long)Dk,
                  (long long)Dv, group_size);
    KMI_CHECK_ARG(dtype >= BF16 && dtype <= F32, "kv_quantize_append: bad dtype %d", dtype);
    KMI_CHECK_ARG(pos >= 0 && pos + S <= capacity,
                  "kv_quantize_append: slots %lld..%lld past the slab capacity %lld", (long long)pos,
                  (long long)(pos + S), (long long)capacity);
    QuantDst dk = {}, dv = {};
    dk.wq = k_wq; dk.scales = k_scales; dk.biases = k_biases;
    dv.wq = v_wq; dv.scales = v_scales; dv.biases = v_biases;
    for (QuantDst* d : {&dk, &dv}) {
        d->pos = pos; d->H = H; d->S = S; d->kv = 1;
    }
    for (int i = 0; i < 3; i++) {
        KMI_CHECK_ARG(k_strides[i] >= 0 && k_strides[3 + i] >= 0 && v_strides[i] >= 0 && v_strides[3 + i] >= 0,
                      "kv_quantize_append: negative stride");
        dk.wst[i] = k_strides[i]; dk.sst[i] = k_strides[3 + i];
        dv.wst[i] = v_strides[i]; dv.sst[i] = v_strides[3 + i];
    }
    const int64_t nk = B * H * S * (Dk / group_size), nv = B * H * S * (Dv / group_size);
    if (nk == 0) return OK;
    KMI_CHECK_ARG(((uintptr_t)k & 15) == 0 && ((uintptr_t)v & 15) == 0,
                  "kv_quantize_append: keys and values must be 16-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    if (dtype == BF16) launch_quantize_kv<TBF16>(k, nk, Dk, dk, v, nv, Dv, dv, group_size, bits, st);
    else if (dtype == F16) launch_quantize_kv<TF16>(k, nk, Dk, dk, v, nv, Dv, dv, group_size, bits, st);
    else launch_quantize_kv<TF32>(k, nk, Dk, dk, v, nv, Dv, dv, group_size, bits, st);
    KMI_CHECK_LAUNCH("kv_quantize_append");
    return OK;
}

int kmi_quantize_mx(const void* w, int dtype, int64_t rows, int64_t cols, int mode, uint32_t* wq,
                    uint8_t* scales, void* stream) {
    clear_error();
    KMI_CHECK_ARG(w && wq && scales, "quantize (mx): null pointer");
    KMI_CHECK_ARG(mode == 1 || mode == 2, "quantize (mx): mode %d (1 mxfp4, 2 mxfp8)", mode);
    KMI_CHECK_ARG(rows >= 0 && cols > 0 && cols % 32 == 0, "quantize (mx): cols %lld not a multiple of 32",
                  (long long)cols);
    KMI_CHECK_ARG(dtype >= BF16 && dtype <= F32, "quantize (mx): bad dtype %d", dtype);
    const int64_t n_groups = rows * cols / 32;
    if (n_groups == 0) return OK;
    const dim3 grid((unsigned)ceil_div(n_groups, 256));
    hipStream_t st = (hipStream_t)stream;
    if (dtype == BF16) quantize_mx_kernel<TBF16><<<grid, 256, 0, st>>>((const uint16_t*)w, n_groups, mode, wq, scales);
    else if (dtype == F16) quantize_mx_kernel<TF16><<<grid, 256, 0, st>>>((const uint16_t*)w, n_groups, mode, wq, scales);
    else quantize_mx_kernel<TF32><<<grid, 256, 0, st>>>((const float*)w, n_groups, mode, wq, scales);
    KMI_CHECK_LAUNCH("quantize (mx)");
    return OK;
}

int kmi_dequantize_mx(const uint32_t* wq, const uint8_t* scales, int64_t rows, int64_t cols, int mode,
                      void* out, int out_dtype, void* stream) {
    clear_error();
    KMI_CHECK_ARG(wq && scales && out, "dequantize (mx): null pointer");
    KMI_CHECK_ARG(mode == 1 || mode == 2, "dequantize (mx): mode %d (1 mxfp4, 2 mxfp8)", mode);
    KMI_CHECK_ARG(rows >= 0 && cols > 0 && cols % 32 == 0, "dequantize (mx): cols %lld not a multiple of 32",
                  (long long)cols);
    KMI_CHECK_ARG(out_dtype >= BF16 && out_dtype <= F32, "dequantize (mx): bad dtype");
    const int64_t n_words = rows * cols * (mode == 1 ? 4 : 8) / 32;
    if (n_words == 0) return OK;
    const dim3 grid((unsigned)ceil_div(n_words, 256));
    hipStream_t st = (hipStream_t)stream;
    if (out_dtype == BF16) dequantize_mx_kernel<TBF16><<<grid, 256, 0, st>>>(wq, scales, n_words, mode, (uint16_t*)out);
    else if (out_dtype == F16) dequantize_mx_kernel<TF16><<<grid, 256, 0, st>>>(wq, scales, n_words, mode, (uint16_t*)out);
    else dequantize_mx_kernel<TF32><<<grid, 256, 0, st>>>(wq, scales, n_words, mode, (float*)out);
    KMI_CHECK_LAUNCH("dequantize (mx)");
    return OK;
}

int kmi_dequantize_affine(const uint32_t* wq, const void* scales, const void* biases,
                          int scale_dtype, int64_t rows, int64_t cols, int group_size,
                          int bits, void* out, int out_dtype, int rounding, void* stream) {
    clear_error();
    KMI_CHECK_ARG(wq && scales && biases && out, "dequantize: null pointer (affine needs biases)");
    KMI_CHECK_ARG(bits >= 2 && bits <= 8 && bits != 7, "dequantize: bits %d not in {2,3,4,5,6,8}", bits);
    KMI_CHECK_ARG(group_size == 32 || group_size == 64 || group_size == 128,
                  "dequantize: group_size %d not in {32,64,128}", group_size);
    KMI_CHECK_ARG(rows >= 0 && cols > 0 && cols % group_size == 0, "dequantize: bad shape");
    KMI_CHECK_ARG(rounding == 0 || rounding == 1, "dequantize: rounding %d not in {0,1}", rounding);
    KMI_CHECK_ARG(scale_dtype >= BF16 && scale_dtype <= F32 && out_dtype >= BF16 && out_dtype <= F32,
                  "dequantize: bad dtype");
    // packed words, or 8-element units for the widths that do not divide 32
    const int64_t n_words = 32 % bits ? rows * cols / 8 : rows * cols * bits / 32;
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
