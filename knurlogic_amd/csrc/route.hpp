// The Qwen3.5-MoE router of one token, computed by the 256 threads of a
// workgroup: the arithmetic of SparseMoeBlock (src/knurlogic/engine/
// families/qwen/architecture/qwen3_5.py:174-179) with one float32 rounding
// per step, in the op order of mlx's CPU softmax:
//   m = max x;  e = exp(x - m) (correctly rounded: float64, rounded once);
//   n = sum e (float64, rounded once);  r = 1 / n;  p = e * r;
//   the k largest p in descending order (equal p: lower expert first);
//   t = sum of the selected p (float64 in slot order, rounded once);
//   score = p / t, rounded to the logits' dtype.
// Quotients and products of two floats are formed in float64 and rounded
// once, which is the correctly rounded float32 result.  Used by the router
// kernel and by the SwitchGLU kernels that route their own token, so both
// give the same experts and scores bit for bit.  mlx forms exp with a SIMD
// polynomial a few float32 ulp from the correctly rounded value, so at
// probabilities that close (and at exact ties, which its argpartition
// breaks in its own order) mlx may select a different expert than this
// rule does: top-k membership there is not pinned to mlx.
#pragma once

#include "common.hpp"

namespace kmi {

constexpr int ROUTE_THREADS = 256;
constexpr int ROUTE_MAX_E = 1024;             // 4 experts per thread
constexpr int ROUTE_MAX_K = 64;

// MAXE: the most experts a kernel routes (sizes the key table)
template <int MAXE = ROUTE_MAX_E>
struct RouteLdsT {
    uint64_t keys[MAXE];
    float red[8];
    double dred[4];
    float sel_p[ROUTE_MAX_K];
    int sel_e[ROUTE_MAX_K];
};
using RouteLds = RouteLdsT<>;

// A float64 result rounded to float32 and kept there (no fused rounding
// with a later one to a narrower type).
__device__ __forceinline__ float route_f32(double v) {
    float f = (float)v;
    asm volatile("" : "+v"(f));
    return f;
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float route_dpp_max(float v) {
    const int ninf = (int)0xff800000u;
    return fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(ninf, __float_as_int(v), CTRL, ROW_MASK, 0xf,
                                                                 false)));
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ double route_dpp_add(double v) {
    const int lo = __builtin_amdgcn_update_dpp(0, __double2loint(v), CTRL, ROW_MASK, 0xf, false);
    const int hi = __builtin_amdgcn_update_dpp(0, __double2hiint(v), CTRL, ROW_MASK, 0xf, false);
    return v + __hiloint2double(hi, lo);
}

// max / sum over the 64 lanes, the result in lane 63
__device__ __forceinline__ float route_wave_max(float v) {
    v = route_dpp_max<0xb1, 0xf>(v);
    v = route_dpp_max<0x4e, 0xf>(v);
    v = route_dpp_max<0x141, 0xf>(v);
    v = route_dpp_max<0x140, 0xf>(v);
    v = route_dpp_max<0x142, 0xa>(v);
    v = route_dpp_max<0x143, 0xc>(v);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ double route_wave_sum(double v) {
    v = route_dpp_add<0xb1, 0xf>(v);
    v = route_dpp_add<0x4e, 0xf>(v);
    v = route_dpp_add<0x141, 0xf>(v);
    v = route_dpp_add<0x140, 0xf>(v);
    v = route_dpp_add<0x142, 0xa>(v);
    v = route_dpp_add<0x143, 0xc>(v);
    const int lo = __builtin_amdgcn_readlane(__double2loint(v), 63);
    const int hi = __builtin_amdgcn_readlane(__double2hiint(v), 63);
    return __hiloint2double(hi, lo);
}

// Route the token whose logits row is `lg` (E values of storage type T):
// afterwards (for every thread of the workgroup) sm.sel_e[0..k) holds the
// experts in descending-probability order and sm.sel_p[0..k) the scores,
// already rounded to T.  Every thread of the 256 must call it (barriers).
// E <= ROUTE_MAX_E, k <= min(E, ROUTE_MAX_K).
// PER: experts per thread (E <= 256 * PER).
// route_token in two parts, so a kernel can issue the logits load early and
// route later: route_load reads this thread's logits, route_from routes them.
template <class T, int PER>
__device__ __forceinline__ void route_load(const typename T::storage* __restrict__ lg, int E, float (&x)[PER]) {
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int i = threadIdx.x + ROUTE_THREADS * j;
        x[j] = i < E ? T::load(lg[i]) : -INFINITY;
    }
}

template <class T, int PER, class SM>
__device__ __forceinline__ void route_from(const float (&x)[PER], int E, int k, SM& sm) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < PER; j++) mx = fmaxf(mx, x[j]);
    mx = route_wave_max(mx);
    if (lane == 0) sm.red[w] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(sm.red[0], sm.red[1]), fmaxf(sm.red[2], sm.red[3]));
    float ex[PER];
    double part = 0.0;
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int i = tid + ROUTE_THREADS * j;
        const float d = x[j] - mx;                     // float32 subtraction
        ex[j] = i < E ? route_f32(exp((double)d)) : 0.f;
        part += (double)ex[j];
    }
    part = route_wave_sum(part);
    if (lane == 0) sm.dred[w] = part;
    __syncthreads();
    const double total = ((sm.dred[0] + sm.dred[1]) + sm.dred[2]) + sm.dred[3];
    const float rn = route_f32(1.0 / (double)route_f32(total));
    float p[PER];
    uint64_t key[PER];
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int i = tid + ROUTE_THREADS * j;
        p[j] = route_f32((double)ex[j] * (double)rn);
        // key orders as the selection does: larger p, then the lower expert
        key[j] = ((uint64_t)__float_as_uint(p[j]) << 32) | (uint32_t)~i;
        // keys past E are 0, below every expert's key (its low word ~i > 0)
        if (i < ((E + 15) & ~15)) sm.keys[i] = i < E ? key[j] : 0ull;
    }
    __syncthreads();
    int rank[PER];
#pragma unroll
    for (int j = 0; j < PER; j++) rank[j] = 0;
    // unrolled, so the broadcast LDS reads of several steps are in flight
    // together (a step per LDS round trip would take microseconds)
    const int Ep = (E + 15) & ~15;
    for (int i = 0; i < Ep; i += 16) {
        uint64_t a[16];
#pragma unroll
        for (int q = 0; q < 16; q++) a[q] = sm.keys[i + q];
#pragma unroll
        for (int q = 0; q < 16; q++)
#pragma unroll
            for (int j = 0; j < PER; j++) rank[j] += (int)(a[q] > key[j]);
    }
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int i = tid + ROUTE_THREADS * j;
        if (i < E && rank[j] < k) {
            sm.sel_p[rank[j]] = p[j];
            sm.sel_e[rank[j]] = i;
        }
    }
    __syncthreads();
    double tsum = 0.0;
#pragma unroll 8
    for (int s = 0; s < k; s++) tsum += (double)sm.sel_p[s];
    const double tt = (double)route_f32(tsum);
    __syncthreads();                                   // every thread has read sel_p
    if (tid < k) sm.sel_p[tid] = T::round(route_f32((double)sm.sel_p[tid] / tt));
    __syncthreads();
}

template <class T, int PER, class SM>
__device__ __forceinline__ void route_token(const typename T::storage* __restrict__ lg, int E, int k, SM& sm) {
    float x[PER];
    route_load<T, PER>(lg, E, x);
    route_from<T, PER>(x, E, k, sm);
}

}  // namespace kmi
