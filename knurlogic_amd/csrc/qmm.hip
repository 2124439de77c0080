// Prefill-shape quantized matmul (M > 16) for gfx950: LDS-tiled bf16 MFMA.
//
// A workgroup (4 waves) owns a 128 x 128 tile of y and walks K in steps of
// 64.  Per step it stages the x tile (bf16) and the packed weight tile, which
// it dequantizes once to bf16 (What = s*q + b, rounded once) into LDS, so
// the dequantization is shared by all 128 activation rows; each wave then
// runs 4 x 4 v_mfma_f32_16x16x32_bf16 blocks (64 x 64) per 32-deep k step.
// Global loads of step t+1 are issued before step t's MFMAs (register
// double buffering; two LDS buffers).
#include "common.hpp"

namespace kmi {

constexpr int GBM = 128, GBN = 128, GBK = 64;
constexpr int GLDS = GBK + 8;   // bf16 per LDS row (16-byte pad)

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
}

template <int BITS, int GS>
__global__ __launch_bounds__(256) void qmm_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ w,
    const uint16_t* __restrict__ sc, const uint16_t* __restrict__ bi,
    uint16_t* __restrict__ y, int64_t M, int64_t N, int64_t K) {
    constexpr int EPW = 32 / BITS;
    constexpr int WPT = (GBK / EPW) / 2;       // words per thread per k tile (2 threads per row)
    __shared__ __align__(16) uint16_t As[2][GBM * GLDS];
    __shared__ __align__(16) uint16_t Bs[2][GBN * GLDS];

    const int tid = threadIdx.x;
    const int64_t bm = (int64_t)blockIdx.y * GBM, bn = (int64_t)blockIdx.x * GBN;
    const int64_t wpr = K / EPW, gpr = K / GS;
    const int nk = (int)(K / GBK);

    // A staging: 128 rows x 8 chunks of 16 B -> 4 chunks per thread
    // B staging: thread -> (row tid/2, half tid%2): WPT words, k [32*half, +32)
    const int brow = tid >> 1, bhalf = tid & 1;
    const int64_t bn_row = bn + brow;
    const bool b_ok = bn_row < N;
    const uint32_t* wp = w + (b_ok ? bn_row : 0) * wpr + bhalf * WPT;
    const uint16_t* sp = sc + (b_ok ? bn_row : 0) * gpr;
    const uint16_t* bp = bi + (b_ok ? bn_row : 0) * gpr;

    u32x4 ra[4];
    uint32_t rw[WPT];
    float rs[2], rb[2];

    auto load_tile = [&](int kt) {
        const int64_t k0 = (int64_t)kt * GBK;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int c = tid + 256 * i;
            const int r = c >> 3, c8 = c & 7;
            const int64_t row = bm + r;
            if (row < M) ra[i] = *(const u32x4*)(x + row * K + k0 + c8 * 8);
            else ra[i] = u32x4{0u, 0u, 0u, 0u};
        }
        const uint32_t* p = wp + k0 / EPW;
#pragma unroll
        for (int q = 0; q < WPT; q += 4) {
            u32x4 t = *(const u32x4*)(p + q);
            rw[q] = t.x; rw[q + 1] = t.y; rw[q + 2] = t.z; rw[q + 3] = t.w;
        }
        // groups touched by k [k0 + 32*half, +32): one (GS >= 32)
        const int64_t g = (k0 + 32 * bhalf) / GS;
        rs[0] = bf16_to_f32(sp[g]);
        rb[0] = bf16_to_f32(bp[g]);
    };

    auto store_tile = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int c = tid + 256 * i;
            const int r = c >> 3, c8 = c & 7;
            *(u32x4*)(&As[buf][r * GLDS + c8 * 8]) = ra[i];
        }
        // dequantize 32 elements: k = 32*half + e
        uint32_t outw[16];
        const float s = rs[0], b = rb[0];
#pragma unroll
        for (int e = 0; e < 32; e += 2) {
            const int wi0 = e / EPW, sh0 = (e % EPW) * BITS;
            const int wi1 = (e + 1) / EPW, sh1 = ((e + 1) % EPW) * BITS;
            const float q0 = (float)((rw[wi0] >> sh0) & ((1u << BITS) - 1u));
            const float q1 = (float)((rw[wi1] >> sh1) & ((1u << BITS) - 1u));
            outw[e / 2] = pack_bf16x2(__builtin_fmaf(s, q0, b), __builtin_fmaf(s, q1, b));
        }
        uint16_t* dst = &Bs[buf][brow * GLDS + 32 * bhalf];
#pragma unroll
        for (int i = 0; i < 4; i++)
            *(u32x4*)(dst + 8 * i) = u32x4{outw[4 * i], outw[4 * i + 1], outw[4 * i + 2], outw[4 * i + 3]};
    };

    const int lane = tid & 63, wave = tid >> 6;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const int l16 = lane & 15, lk = lane >> 4;

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int jn = 0; jn < 4; jn++) acc[i][jn] = f32x4{0.f, 0.f, 0.f, 0.f};

    load_tile(0);
    store_tile(0);
    __syncthreads();
    for (int kt = 0; kt < nk; kt++) {
        const int buf = kt & 1;
        if (kt + 1 < nk) load_tile(kt + 1);
#pragma unroll
        for (int ks = 0; ks < GBK / 32; ks++) {
            u32x4 af[4], bfr[4];
#pragma unroll
            for (int i = 0; i < 4; i++)
                af[i] = *(const u32x4*)(&As[buf][(wm + 16 * i + l16) * GLDS + ks * 32 + lk * 8]);
#pragma unroll
            for (int jn = 0; jn < 4; jn++)
                bfr[jn] = *(const u32x4*)(&Bs[buf][(wn + 16 * jn + l16) * GLDS + ks * 32 + lk * 8]);
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int jn = 0; jn < 4; jn++) acc[i][jn] = mfma16x16x32(af[i], bfr[jn], acc[i][jn]);
        }
        if (kt + 1 < nk) store_tile(buf ^ 1);
        __syncthreads();
    }

    // D: row = 16*i + 4*lk + r, col = 16*jn + l16
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int jn = 0; jn < 4; jn++) {
            const int64_t col = bn + wn + 16 * jn + l16;
            if (col >= N) continue;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int64_t row = bm + wm + 16 * i + 4 * lk + r;
                if (row < M) y[row * N + col] = f32_to_bf16(acc[i][jn][r]);
            }
        }
}

int qmm_gemm(const void* x, int64_t M, int64_t K, int64_t N, const uint32_t* w,
             const void* scales, const void* biases, int group_size, int bits, void* y,
             hipStream_t st) {
    KMI_CHECK_ARG(K % GBK == 0, "quantized_matmul: K=%lld must be a multiple of 64 for M > 16",
                  (long long)K);
    KMI_CHECK_ARG(group_size >= 32, "quantized_matmul: group_size %d", group_size);
    dim3 grid((unsigned)ceil_div(N, GBN), (unsigned)ceil_div(M, GBM));
    KMI_CHECK_ARG(grid.y < 65536, "quantized_matmul: M too large");
    const uint16_t* xx = (const uint16_t*)x;
    const uint16_t* ss = (const uint16_t*)scales;
    const uint16_t* bb = (const uint16_t*)biases;
    uint16_t* yy = (uint16_t*)y;
#define KMI_QMM(B, G) qmm_kernel<B, G><<<grid, 256, 0, st>>>(xx, w, ss, bb, yy, M, N, K)
    if (bits == 4) {
        if (group_size == 32) KMI_QMM(4, 32);
        else if (group_size == 64) KMI_QMM(4, 64);
        else KMI_QMM(4, 128);
    } else {
        if (group_size == 32) KMI_QMM(8, 32);
        else if (group_size == 64) KMI_QMM(8, 64);
        else KMI_QMM(8, 128);
    }
#undef KMI_QMM
    KMI_CHECK_LAUNCH("qmm");
    return OK;
}

}  // namespace kmi
