// Dense (unquantized) linear layers and bias adds for gfx950 -- the layers a
// quantized model keeps in bf16 (the MoE router, the shared-expert gate)
// and the bias of the quantized layers.
//
//   kmi_linear: mlx's nn.Linear, y = x @ w^T, or addmm(bias, x, w^T) with
//     one rounding of acc + bias; fp32 accumulation.  HBM-bound on w at
//     decode sizes: one wave per output column streams that weight row in
//     16-byte loads (lanes 8 elements apart), every row of the tile reuses
//     the load, and the 64 lane partials meet in a butterfly reduction.
//   kmi_add_bias: y + bias (nn.QuantizedLinear / QuantizedSwitchLinear add
//     their bias to the rounded product as a separate op), the bias row
//     picked per output row by an expert index when given.
#include "common.hpp"
#include "../../include/knurlogic_amd.h"

namespace kmi {

constexpr int LIN_TM = 8;         // x rows per wave tile
constexpr int LIN_WAVES = 4;      // output columns per workgroup

template <class T>
__device__ __forceinline__ void unpack8(u32x4 v, float* f) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        f[2 * i] = T::load((uint16_t)(v[i] & 0xffffu));
        f[2 * i + 1] = T::load((uint16_t)(v[i] >> 16));
    }
}

template <class T>
__global__ __launch_bounds__(256) void linear_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                                     const uint16_t* __restrict__ bias, uint16_t* __restrict__ y,
                                                     int64_t M, int64_t K, int64_t N) {
    const int lane = threadIdx.x & 63;
    const int64_t n = (int64_t)blockIdx.x * LIN_WAVES + (threadIdx.x >> 6);
    const int64_t m0 = (int64_t)blockIdx.y * LIN_TM;
    if (n >= N) return;                                  // a whole wave leaves
    const int rows = (int)(M - m0 < LIN_TM ? M - m0 : LIN_TM);
    float acc[LIN_TM];
#pragma unroll
    for (int r = 0; r < LIN_TM; r++) acc[r] = 0.f;
    const uint16_t* wr = w + n * K;
    for (int64_t k = 8 * lane; k < K; k += 512) {
        float wf[8], xf[8];
        unpack8<T>(*(const u32x4*)(wr + k), wf);
#pragma unroll
        for (int r = 0; r < LIN_TM; r++) {
            if (r < rows) {
                unpack8<T>(*(const u32x4*)(x + (m0 + r) * K + k), xf);
                float s = acc[r];
#pragma unroll
                for (int i = 0; i < 8; i++) s = fmaf(xf[i], wf[i], s);
                acc[r] = s;
            }
        }
    }
#pragma unroll
    for (int r = 0; r < LIN_TM; r++)
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) acc[r] += __shfl_xor(acc[r], o, 64);
    if (lane < rows) {
        float v = acc[0];
#pragma unroll
        for (int r = 1; r < LIN_TM; r++)
            if (lane == r) v = acc[r];
        if (bias) v += T::load(bias[n]);
        y[(m0 + lane) * N + n] = T::store(v);
    }
}

// y[r, n] = round(y[r, n] + bias[e, n]), e = idx[r / rows_per_index] (or 0
// without idx); rows whose index is outside [0, E) are left alone.
template <class T>
__global__ __launch_bounds__(256) void add_bias_kernel(uint16_t* __restrict__ y, const uint16_t* __restrict__ bias,
                                                       const int32_t* __restrict__ idx, int64_t rows,
                                                       int64_t rows_per_index, int64_t N, int64_t E) {
    const int64_t total = rows * N;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / N, n = i % N;
        const int64_t e = idx ? (int64_t)idx[r / rows_per_index] : 0;
        if (e < 0 || e >= E) continue;
        y[i] = T::store(T::load(y[i]) + T::load(bias[e * N + n]));
    }
}

}  // namespace kmi

using namespace kmi;

extern "C" {

int kmi_linear(const void* x, int64_t M, int64_t K, const void* w, int64_t N, const void* bias, int dtype,
               void* y, void* stream) {
    clear_error();
    KMI_CHECK_ARG(dtype == BF16 || dtype == F16, "linear: bfloat16 or float16 only (got dtype %d)", dtype);
    KMI_CHECK_ARG(M >= 0 && K > 0 && N > 0, "linear: M=%lld K=%lld N=%lld", (long long)M, (long long)K,
                  (long long)N);
    KMI_CHECK_ARG(K % 8 == 0, "linear: K=%lld must be a multiple of 8 (16-byte rows)", (long long)K);
    if (M == 0) return OK;
    KMI_CHECK_ARG(x && w && y, "linear: null pointer");
    KMI_CHECK_ARG(((uintptr_t)x | (uintptr_t)w) % 16 == 0, "linear: x and w must be 16-byte aligned");
    const int64_t mt = ceil_div(M, LIN_TM);
    KMI_CHECK_ARG(mt < 65536, "linear: M=%lld too large", (long long)M);
    const dim3 grid((unsigned)ceil_div(N, LIN_WAVES), (unsigned)mt);
    hipStream_t st = (hipStream_t)stream;
    if (dtype == BF16)
        linear_kernel<TBF16><<<grid, 64 * LIN_WAVES, 0, st>>>((const uint16_t*)x, (const uint16_t*)w,
                                                              (const uint16_t*)bias, (uint16_t*)y, M, K, N);
    else
        linear_kernel<TF16><<<grid, 64 * LIN_WAVES, 0, st>>>((const uint16_t*)x, (const uint16_t*)w,
                                                             (const uint16_t*)bias, (uint16_t*)y, M, K, N);
    KMI_CHECK_LAUNCH("linear");
    return OK;
}

int kmi_add_bias(void* y, int64_t rows, int64_t N, const void* bias, const int32_t* idx, int64_t rows_per_index,
                 int64_t E, int dtype, void* stream) {
    clear_error();
    KMI_CHECK_ARG(dtype == BF16 || dtype == F16, "add_bias: bfloat16 or float16 only (got dtype %d)", dtype);
    KMI_CHECK_ARG(rows >= 0 && N > 0 && E >= 1 && rows_per_index >= 1, "add_bias: bad sizes");
    if (rows == 0) return OK;
    KMI_CHECK_ARG(y && bias, "add_bias: null pointer");
    const int64_t total = rows * N;
    const int64_t g = ceil_div(total, 256);
    const unsigned grid = (unsigned)(g < 65536 ? g : 65536);
    hipStream_t st = (hipStream_t)stream;
    if (dtype == BF16)
        add_bias_kernel<TBF16><<<grid, 256, 0, st>>>((uint16_t*)y, (const uint16_t*)bias, idx, rows, rows_per_index,
                                                     N, E);
    else
        add_bias_kernel<TF16><<<grid, 256, 0, st>>>((uint16_t*)y, (const uint16_t*)bias, idx, rows, rows_per_index,
                                                    N, E);
    KMI_CHECK_LAUNCH("add_bias");
    return OK;
}

}  // extern "C"
