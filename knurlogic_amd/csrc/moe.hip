// MoE glue around the expert matmuls, for gfx950: the router (softmax,
// top-k, renormalize), the SwiGLU activation between the gate/up and down
// projections, and the weighted combine of the k expert outputs -- the
// reference's SparseMoeBlock / SwitchGLU arithmetic
// (src/knurlogic/engine/families/qwen/architecture/qwen3_5.py:35-40,108-112,
// 170-192), each rounding step where the reference rounds.
#include "common.hpp"
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

constexpr int ROUTE_MAX_E = 1024;            // experts a wave holds (16 per lane)

// One wave per token.  probs = softmax(logits) in float32, one rounding per
// step as mlx's CPU softmax takes them (max m; e = exp(x - m); n = sum e;
// r = 1 / n; p = e * r), with exp correctly rounded (evaluated in float64)
// and the sum exact before its one rounding; the k largest probabilities in
// descending order, equal ones taken lower index first; scores = p / t with
// t the float32 sum of the k selected (again exact, then rounded), rounded
// to the logits' dtype.  Quotients and products of two floats are formed in
// float64 and rounded once, which gives the correctly rounded float32
// result (53 >= 2 * 24 + 2 bits).
//
// Selection is by rank, with no serial rounds: probabilities are >= 0, so
// their float32 bits order like the values, and key = bits << 32 | ~expert
// orders exactly as the selection does (larger p first, then lower expert)
// with no two keys equal.  Each lane counts the wave's keys above its own
// (broadcast LDS reads, one 64-bit compare each); rank < k is selected, at
// slot rank.
template <class T, int ROUTE_PER_LANE>
__global__ __launch_bounds__(256) void moe_route_kernel(const void* __restrict__ logits, int64_t T_, int E,
                                                        int k, int32_t* __restrict__ inds,
                                                        void* __restrict__ scores) {
    constexpr int EP = 64 * ROUTE_PER_LANE;             // keys per wave, padded
    __shared__ uint64_t keys[4][EP];
    __shared__ float selp[4][64];
    __shared__ int sele[4][64];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int64_t t = (int64_t)blockIdx.x * 4 + w;
    const bool live = t < T_;                            // a whole wave is live or not
    float lg[ROUTE_PER_LANE];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < ROUTE_PER_LANE; j++) {
        const int e = lane + 64 * j;
        lg[j] = live && e < E ? ld_dt<T>(logits, t * E + e) : -INFINITY;
        mx = fmaxf(mx, lg[j]);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    float ex[ROUTE_PER_LANE];
    double sum = 0.0;
#pragma unroll
    for (int j = 0; j < ROUTE_PER_LANE; j++) {
        const float d = lg[j] - mx;                      // float32 subtraction, as mlx's kernel
        ex[j] = lane + 64 * j < E ? f64_to_f32(exp((double)d)) : 0.f;
        sum += (double)ex[j];
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) sum += __shfl_xor(sum, o, 64);
    const float rn = f64_to_f32(1.0 / (double)f64_to_f32(sum));
    float p[ROUTE_PER_LANE];
    uint64_t key[ROUTE_PER_LANE];
#pragma unroll
    for (int j = 0; j < ROUTE_PER_LANE; j++) {
        const int e = lane + 64 * j;
        p[j] = e < E ? f64_to_f32((double)ex[j] * (double)rn) : 0.f;
        // padding lanes get key 0, below every expert's key (its low word ~e > 0)
        key[j] = e < E ? ((uint64_t)__float_as_uint(p[j]) << 32) | (uint32_t)~e : 0ull;
        keys[w][e] = key[j];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    int rank[ROUTE_PER_LANE];
#pragma unroll
    for (int j = 0; j < ROUTE_PER_LANE; j++) rank[j] = 0;
    for (int i = 0; i < EP; i += 2) {
        const uint64_t a = keys[w][i], b = keys[w][i + 1];
#pragma unroll
        for (int j = 0; j < ROUTE_PER_LANE; j++) rank[j] += (int)(a > key[j]) + (int)(b > key[j]);
    }
#pragma unroll
    for (int j = 0; j < ROUTE_PER_LANE; j++)
        if (lane + 64 * j < E && rank[j] < k) {
            selp[w][rank[j]] = p[j];
            sele[w][rank[j]] = lane + 64 * j;
        }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    double top_sum = 0.0;
    for (int s2 = 0; s2 < k; s2++) top_sum += (double)selp[w][s2];
    const double tsum = (double)f64_to_f32(top_sum);
    if (live && lane < k) {
        inds[t * k + lane] = sele[w][lane];
        st_dt<T>(scores, t * k + lane, f64_to_f32((double)selp[w][lane] / tsum));
    }
}

// act[r, i] = round(round(silu(gate[r, i])) * up[r, i]), silu in float32
// (evaluated in float64, rounded once): _SwiGLU with qwen3_5.py's _silu.
template <class T>
__global__ __launch_bounds__(256) void swiglu_kernel(const void* __restrict__ gate, const void* __restrict__ up,
                                                     int64_t ld_in, int64_t rows, int64_t I,
                                                     void* __restrict__ out) {
    const int64_t n = rows * I;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < n;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = idx / I, i = idx % I;
        const double g = (double)ld_dt<T>(gate, r * ld_in + i);
        const float s = T::round(f64_to_f32(g / (1.0 + exp(-g))));
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
    KMI_CHECK_ARG(k >= 1 && k <= E && k <= 64, "moe_route: top-%d of %d experts", k, E);
    if (T == 0) return OK;
    KMI_CHECK_ARG(logits && inds && scores, "moe_route: null pointer");
    hipStream_t st = (hipStream_t)stream;
    const unsigned grid = (unsigned)ceil_div(T, 4);
    const int per = E <= 64 ? 1 : E <= 128 ? 2 : E <= 256 ? 4 : E <= 512 ? 8 : 16;
#define KMI_ROUTE(TT, PL) moe_route_kernel<TT, PL><<<grid, 256, 0, st>>>(logits, T, E, k, inds, scores)
#define KMI_ROUTE_T(TT)                                     \
    do {                                                    \
        if (per == 1) KMI_ROUTE(TT, 1);                     \
        else if (per == 2) KMI_ROUTE(TT, 2);                \
        else if (per == 4) KMI_ROUTE(TT, 4);                \
        else if (per == 8) KMI_ROUTE(TT, 8);                \
        else KMI_ROUTE(TT, 16);                             \
    } while (0)
    if (dtype == BF16) KMI_ROUTE_T(TBF16);
    else if (dtype == F16) KMI_ROUTE_T(TF16);
    else KMI_ROUTE_T(TF32);
#undef KMI_ROUTE_T
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
