// MoE glue around the expert matmuls, for gfx950: the router (softmax,
// top-k, renormalize), the SwiGLU activation between the gate/up and down
// projections, and the weighted combine of the k expert outputs -- the
// reference's SparseMoeBlock / SwitchGLU arithmetic
// (src/knurlogic/engine/families/qwen/architecture/qwen3_5.py:35-40,108-112,
// 170-192), each rounding step where the reference rounds.
#include <type_traits>

#include "common.hpp"
#include "route.hpp"
#include "../../include/knurlogic_amd.h"

namespace kmi {

template <class T>
__device__ __forceinline__ float ld_dt(const void* p, int64_t i) {
    return T::load(((const typename T::storage*)p)[i]);
}
template <class T>
__device__ __forceinline__ void st_dt(void* p, int64_t i, float v) {
    ((typename T::storage*)p)[i] = T::store(v);
}

// A float64 result rounded to float32 and kept there: the empty asm stops
// the compiler from fusing this rounding with a later one to fp16 into a
// single float64 -> fp16 rounding (the reference rounds twice).
__device__ __forceinline__ float f64_to_f32(double v) {
    float f = (float)v;
    asm volatile("" : "+v"(f));
    return f;
}

// One workgroup per token: the router of route.hpp, then the k experts and
// their scores stored.
template <class T, int PER>
__global__ __launch_bounds__(ROUTE_THREADS) void moe_route_kernel(const void* __restrict__ logits, int E, int k,
                                                                  int32_t* __restrict__ inds,
                                                                  void* __restrict__ scores) {
    __shared__ RouteLds sm;
    const int64_t t = blockIdx.x;
    route_token<T, PER>((const typename T::storage*)logits + t * E, E, k, sm);
    if ((int)threadIdx.x < k) {
        inds[t * k + threadIdx.x] = sm.sel_e[threadIdx.x];
        st_dt<T>(scores, t * k + threadIdx.x, sm.sel_p[threadIdx.x]);
    }
}

// act[r, i] = round(round(silu(gate[r, i])) * up[r, i]), silu in float32
// (evaluated in float64, rounded once; in bf16 by silu_bf16r, the expert
// kernels' epilogue, which gives the same values): _SwiGLU with
// qwen3_5.py's _silu.
template <class T>
__global__ __launch_bounds__(256) void swiglu_kernel(const void* __restrict__ gate, const void* __restrict__ up,
                                                     int64_t ld_in, int64_t rows, int64_t I,
                                                     void* __restrict__ out) {
    const int64_t n = rows * I;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < n;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = idx / I, i = idx % I;
        float s;
        if constexpr (std::is_same<T, TBF16>::value) {
            s = silu_bf16r(ld_dt<T>(gate, r * ld_in + i));    // the expert kernels' epilogue arithmetic
        } else {
            const double g = (double)ld_dt<T>(gate, r * ld_in + i);
            s = T::round(f64_to_f32(g / (1.0 + exp(-g))));
        }
        st_dt<T>(out, idx, s * ld_dt<T>(up, r * ld_in + i));
    }
}

// out[t, h] = round(sum_s round(y[t, s, h] * score[t, s])): each product
// rounded to the dtype, the k products summed (float64, exact for k <= 16
// bf16 values) and rounded once.
template <class T>
__global__ __launch_bounds__(256) void moe_combine_kernel(const void* __restrict__ y, const void* __restrict__ scores,
                                                          int64_t T_, int k, int64_t H, void* __restrict__ out) {
    const int64_t n = T_ * H;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < n;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t t = idx / H, h = idx % H;
        double acc = 0.0;
        for (int s = 0; s < k; s++)
            acc += (double)T::round(ld_dt<T>(y, (t * k + s) * H + h) * ld_dt<T>(scores, t * k + s));
        st_dt<T>(out, idx, f64_to_f32(acc));
    }
}

// The bf16 combine with 8 columns per thread: 16-byte loads of each slot's
// row (a token's slots loaded 8 at a time, before any is summed) and one
// 16-byte store, the same arithmetic per output (each product rounded to
// bf16, summed in float64 in slot order, rounded once).  One wave per
// workgroup; the grid's y dimension walks the tokens.  For H % 8 == 0 and
// 16-byte aligned y and out.
__global__ __launch_bounds__(64) void moe_combine_bf16x8(const uint16_t* __restrict__ y,
                                                         const uint16_t* __restrict__ scores, int64_t T_, int k,
                                                         int64_t H, uint16_t* __restrict__ out) {
    const int64_t c = (int64_t)blockIdx.x * 64 + threadIdx.x;      // 8-column group
    if (c >= H / 8) return;
    for (int64_t t = blockIdx.y; t < T_; t += gridDim.y) {
        double acc[8];
#pragma unroll
        for (int e = 0; e < 8; e++) acc[e] = 0.0;
        for (int s0 = 0; s0 < k; s0 += 8) {
            u32x4 v[8];
            float sc[8];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int s = s0 + j < k ? s0 + j : k - 1;             // past k: a real row, not summed
                sc[j] = bf16_to_f32(scores[t * k + s]);
                v[j] = *(const u32x4*)(y + (t * k + s) * H + c * 8);
            }
#pragma unroll
            for (int j = 0; j < 8; j++) {
                if (s0 + j >= k) break;
                const uint32_t w[4] = {v[j].x, v[j].y, v[j].z, v[j].w};   // scalars before any bit reinterpretation
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const float yv = __uint_as_float(e % 2 ? w[e / 2] & 0xffff0000u : w[e / 2] << 16);
                    acc[e] += (double)TBF16::round(yv * sc[j]);
                }
            }
        }
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 4; e++)
            o[e] = (uint32_t)f32_to_bf16(f64_to_f32(acc[2 * e])) |
                   ((uint32_t)f32_to_bf16(f64_to_f32(acc[2 * e + 1])) << 16);
        *(u32x4*)(out + t * H + c * 8) = u32x4{o[0], o[1], o[2], o[3]};
    }
}

// out[t, h] = round(y[t, h] + round(round(sigmoid_f32(g[t])) * sy[t, h])):
// SparseMoeBlock's shared expert, gated by sigmoid(shared_expert_gate(x))
// and added to the routed experts' combine (qwen3_5.py:184-187).
template <class T>
__global__ __launch_bounds__(256) void moe_shared_add_kernel(const void* __restrict__ y, const void* __restrict__ g,
                                                             const void* __restrict__ sy, int64_t T_, int64_t H,
                                                             void* __restrict__ out) {
    const int64_t n = T_ * H;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < n;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t t = idx / H;
        const double gv = (double)ld_dt<T>(g, t);
        const float sg = T::round(f64_to_f32(1.0 / (1.0 + exp(-gv))));
        const float gated = T::round(sg * ld_dt<T>(sy, idx));
        st_dt<T>(out, idx, ld_dt<T>(y, idx) + gated);
    }
}

static unsigned grid_for(int64_t n) {
    const int64_t g = ceil_div(n, 256);
    return (unsigned)(g < 65536 ? (g > 0 ? g : 1) : 65536);
}

}  // namespace kmi

using namespace kmi;

extern "C" {

int kmi_moe_route(const void* logits, int dtype, int64_t T, int E, int k, int32_t* inds,
                  void* scores, void* stream) {
    clear_error();
    KMI_CHECK_ARG(dtype >= BF16 && dtype <= F32, "moe_route: bad dtype %d", dtype);
    KMI_CHECK_ARG(T >= 0 && E >= 1 && E <= ROUTE_MAX_E, "moe_route: %d experts (1..%d)", E, ROUTE_MAX_E);
    KMI_CHECK_ARG(k >= 1 && k <= E && k <= ROUTE_MAX_K, "moe_route: top-%d of %d experts", k, E);
    if (T == 0) return OK;
    KMI_CHECK_ARG(logits && inds && scores, "moe_route: null pointer");
    KMI_CHECK_ARG(T < 0x7fffffffLL, "moe_route: T=%lld", (long long)T);
    hipStream_t st = (hipStream_t)stream;
    const unsigned grid = (unsigned)T;
    const int per = E <= ROUTE_THREADS ? 1 : E <= 2 * ROUTE_THREADS ? 2 : 4;
#define KMI_ROUTE(TT)                                                                                   \
    if (per == 1) moe_route_kernel<TT, 1><<<grid, ROUTE_THREADS, 0, st>>>(logits, E, k, inds, scores);      \
    else if (per == 2) moe_route_kernel<TT, 2><<<grid, ROUTE_THREADS, 0, st>>>(logits, E, k, inds, scores); \
    else moe_route_kernel<TT, 4><<<grid, ROUTE_THREADS, 0, st>>>(logits, E, k, inds, scores);
    if (dtype == BF16) { KMI_ROUTE(TBF16) }
    else if (dtype == F16) { KMI_ROUTE(TF16) }
    else { KMI_ROUTE(TF32) }
#undef KMI_ROUTE
    KMI_CHECK_LAUNCH("moe_route");
    return OK;
}

int kmi_swiglu(const void* gate, const void* up, int64_t ld, int dtype, int64_t rows, int64_t I,
               void* out, void* stream) {
    clear_error();
    KMI_CHECK_ARG(dtype >= BF16 && dtype <= F32, "swiglu: bad dtype %d", dtype);
    KMI_CHECK_ARG(rows >= 0 && I >= 0 && ld >= I, "swiglu: bad sizes");
    if (rows == 0 || I == 0) return OK;
    KMI_CHECK_ARG(gate && up && out, "swiglu: null pointer");
    hipStream_t st = (hipStream_t)stream;
    const unsigned grid = grid_for(rows * I);
    if (dtype == BF16) swiglu_kernel<TBF16><<<grid, 256, 0, st>>>(gate, up, ld, rows, I, out);
    else if (dtype == F16) swiglu_kernel<TF16><<<grid, 256, 0, st>>>(gate, up, ld, rows, I, out);
    else swiglu_kernel<TF32><<<grid, 256, 0, st>>>(gate, up, ld, rows, I, out);
    KMI_CHECK_LAUNCH("swiglu");
    return OK;
}

int kmi_moe_combine(const void* y, const void* scores, int dtype, int64_t T, int k, int64_t H,
                    void* out, void* stream) {
    clear_error();
    KMI_CHECK_ARG(dtype >= BF16 && dtype <= F32, "moe_combine: bad dtype %d", dtype);
    KMI_CHECK_ARG(T >= 0 && k >= 1 && k <= 64 && H >= 0, "moe_combine: bad sizes");
    if (T == 0 || H == 0) return OK;
    KMI_CHECK_ARG(y && scores && out, "moe_combine: null pointer");
    hipStream_t st = (hipStream_t)stream;
    // the 8-column kernel from 2^20 outputs (prefill sizes); below, the
    // per-element kernel's 8x more waves hide the latency better (256 tokens
    // x 2048: 5.6 vs 6.2 us; 2048 tokens: 32.8 vs 17.2)
    if (dtype == BF16 && H % 8 == 0 && T * H >= (1 << 20) && ((uintptr_t)y | (uintptr_t)out) % 16 == 0) {
        const dim3 g2((unsigned)ceil_div(H / 8, 64), (unsigned)(T < 65535 ? T : 65535));
        moe_combine_bf16x8<<<g2, 64, 0, st>>>((const uint16_t*)y, (const uint16_t*)scores, T, k, H, (uint16_t*)out);
        KMI_CHECK_LAUNCH("moe_combine");
        return OK;
    }
    const unsigned grid = grid_for(T * H);
    if (dtype == BF16) moe_combine_kernel<TBF16><<<grid, 256, 0, st>>>(y, scores, T, k, H, out);
    else if (dtype == F16) moe_combine_kernel<TF16><<<grid, 256, 0, st>>>(y, scores, T, k, H, out);
    else moe_combine_kernel<TF32><<<grid, 256, 0, st>>>(y, scores, T, k, H, out);
    KMI_CHECK_LAUNCH("moe_combine");
    return OK;
}

int kmi_moe_shared_add(const void* y, const void* gate, const void* shared_y, int dtype, int64_t T,
                       int64_t H, void* out, void* stream) {
    clear_error();
    KMI_CHECK_ARG(dtype >= BF16 && dtype <= F32, "moe_shared_add: bad dtype %d", dtype);
    KMI_CHECK_ARG(T >= 0 && H >= 0, "moe_shared_add: bad sizes");
    if (T == 0 || H == 0) return OK;
    KMI_CHECK_ARG(y && gate && shared_y && out, "moe_shared_add: null pointer");
    hipStream_t st = (hipStream_t)stream;
    const unsigned grid = grid_for(T * H);
    if (dtype == BF16) moe_shared_add_kernel<TBF16><<<grid, 256, 0, st>>>(y, gate, shared_y, T, H, out);
    else if (dtype == F16) moe_shared_add_kernel<TF16><<<grid, 256, 0, st>>>(y, gate, shared_y, T, H, out);
    else moe_shared_add_kernel<TF32><<<grid, 256, 0, st>>>(y, gate, shared_y, T, H, out);
    KMI_CHECK_LAUNCH("moe_shared_add");
    return OK;
}

}  // extern "C"
