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

// =============================================================================
// qmm2: M > 128.  256 x 128 x 64 block tiles; 4 waves, each a 128 x 64 tile
// of y (8 x 4 blocks of v_mfma_f32_16x16x32_bf16), so every 16-byte LDS read
// feeds 4 or 8 MFMAs (44 flop per LDS byte).  The x tile (bf16, mostly L2
// hits) is staged one k-tile ahead through registers; the packed weight tile
// (the only HBM stream, 16 B per thread per k-tile at 4 bits) runs Q2_RING
// k-tiles ahead in a register ring, and is dequantized once per k-tile
// (fp32 s*q + b, rounded to bf16 by v_cvt_pk_bf16_f32) into LDS.  Rows past
// M, columns past N and k-tiles past the split read zeros from their buffer
// views.  When the tiles leave CUs idle, K is split: each split writes fp32
// partials and qmm_split_reduce sums them in split order.
// =============================================================================
constexpr int Q2M = 256, Q2N = 128, Q2K = 64, Q2LDS = Q2K + 8;
constexpr int Q2_RING = 4;

typedef __bf16 q2_bf16x2 __attribute__((ext_vector_type(2)));
typedef float q2_f32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t cvt_pk_bf16(float lo, float hi) {
    const q2_f32x2 v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, q2_bf16x2));
}

struct Qmm2Args {
    const uint16_t* x;          // [M, K] bf16
    const uint32_t* w;          // [N, K*bits/32]
    const uint16_t* s;          // [N, K/gs] bf16
    const uint16_t* b;
    uint16_t* y;                // [M, N] bf16 (one split)
    float* partial;             // [splits, M, N] fp32 (several splits)
    int64_t M, N, K;
    int kt_per_split, splits, n_tiles;
};

template <int BITS, int GS>
__global__ __launch_bounds__(512, 1) void qmm2_kernel(Qmm2Args a) {
    constexpr int EPW = 32 / BITS;
    constexpr int BQ = Q2K / 4 / EPW;           // packed words per thread per k-tile (2 or 4)
    static_assert(GS >= 16, "one scale group per 16-wide quarter row");
    __shared__ __align__(16) uint16_t As[2][Q2M * Q2LDS];
    __shared__ __align__(16) uint16_t Bs[2][Q2N * Q2LDS];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nt = (int)(blockIdx.x % a.n_tiles), mt = (int)(blockIdx.x / a.n_tiles);
    const int64_t bm = (int64_t)mt * Q2M, bn = (int64_t)nt * Q2N;
    const int nk = (int)(a.K / Q2K);
    const int kt0 = (int)blockIdx.y * a.kt_per_split;
    const int kt1 = kt0 + a.kt_per_split < nk ? kt0 + a.kt_per_split : nk;
    const int64_t wpr = a.K / EPW, gpr = a.K / GS;

    // A: thread chunk c = tid + 512 i -> row c / 8, 16-byte piece c % 8
    // B: thread -> weight row tid / 4, k quarter tid % 4 (16 values)
    const int brow = tid >> 2, bq = tid & 3;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x + bm * a.K, (a.M - bm) * a.K * 2);
    const int64_t nrows = a.N - bn;
    const __amdgpu_buffer_rsrc_t rwt = make_rsrc(a.w + bn * wpr, nrows * wpr * 4);
    const __amdgpu_buffer_rsrc_t rwz = make_rsrc(a.w, 0);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.s + bn * gpr, nrows * gpr * 2);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(a.b + bn * gpr, nrows * gpr * 2);
    const uint32_t wrow_off = (uint32_t)(brow * wpr * 4 + bq * BQ * 4);
    const uint32_t srow_off = (uint32_t)(brow * gpr * 2);

    u32x4 ra[4];
    uint32_t rw[Q2_RING][BQ];
    uint32_t rsc[Q2_RING], rbi[Q2_RING];

    auto load_a = [&](int kt) {        // kt past the split: a zero-extent view, no traffic
        const __amdgpu_buffer_rsrc_t r = kt < kt1 ? rx : rwz;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int c = tid + 512 * i;
            const uint32_t off = (uint32_t)(((c >> 3) * a.K + (int64_t)kt * Q2K + (c & 7) * 8) * 2);
            ra[i] = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
        }
    };
    auto load_b = [&](int slot, int kt) {
        const bool live = kt < kt1;
        const __amdgpu_buffer_rsrc_t r = live ? rwt : rwz;
        const uint32_t off = wrow_off + (uint32_t)kt * (Q2K / EPW) * 4u;
        if constexpr (BQ == 2) {
            const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0);
            rw[slot][0] = v.x; rw[slot][1] = v.y;
        } else {
            const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
            rw[slot][0] = v.x; rw[slot][1] = v.y; rw[slot][2] = v.z; rw[slot][3] = v.w;
        }
        const uint32_t g = (uint32_t)(((int64_t)kt * Q2K + 16 * bq) / GS);
        rsc[slot] = __builtin_amdgcn_raw_buffer_load_b16(live ? rs : rwz, (int)(srow_off + 2u * g), 0, 0);
        rbi[slot] = __builtin_amdgcn_raw_buffer_load_b16(live ? rb : rwz, (int)(srow_off + 2u * g), 0, 0);
    };
    auto store = [&](int buf, int slot) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int c = tid + 512 * i;
            *(u32x4*)(&As[buf][(c >> 3) * Q2LDS + (c & 7) * 8]) = ra[i];
        }
        const float sc = bf16_to_f32((uint16_t)rsc[slot]), bi = bf16_to_f32((uint16_t)rbi[slot]);
        uint32_t ow[8];
#pragma unroll
        for (int e = 0; e < 16; e += 2) {
            const uint32_t w0 = rw[slot][e / EPW], w1 = rw[slot][(e + 1) / EPW];
            const float q0 = (float)((w0 >> ((e % EPW) * BITS)) & ((1u << BITS) - 1u));
            const float q1 = (float)((w1 >> (((e + 1) % EPW) * BITS)) & ((1u << BITS) - 1u));
            ow[e / 2] = cvt_pk_bf16(__builtin_fmaf(sc, q0, bi), __builtin_fmaf(sc, q1, bi));
        }
        uint16_t* dst = &Bs[buf][brow * Q2LDS + 16 * bq];
        *(u32x4*)dst = u32x4{ow[0], ow[1], ow[2], ow[3]};
        *(u32x4*)(dst + 8) = u32x4{ow[4], ow[5], ow[6], ow[7]};
    };

    // 8 waves: 4 along M x 2 along N, each a 64 x 64 tile (4 x 4 MFMA blocks)
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const int l16 = lane & 15, lk = lane >> 4;
    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (int r = 0; r < Q2_RING; r++) load_b(r, kt0 + r);
    load_a(kt0);
    store(0, 0);
    __syncthreads();
    load_a(kt0 + 1);
    load_b(0, kt0 + Q2_RING);

    for (int kb = kt0; kb < kt1; kb += Q2_RING) {
#pragma unroll
        for (int u = 0; u < Q2_RING; u++) {
            const int t = kb + u;
            if (t < kt1) {
                const int buf = (t - kt0) & 1;
                const int ns = (u + 1) % Q2_RING;        // ring slot of tile t + 1
#pragma unroll
                for (int ks = 0; ks < Q2K / 32; ks++) {
                    u32x4 af[4], bfr[4];
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        af[i] = *(const u32x4*)(&As[buf][(wm + 16 * i + l16) * Q2LDS + ks * 32 + lk * 8]);
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        bfr[j] = *(const u32x4*)(&Bs[buf][(wn + 16 * j + l16) * Q2LDS + ks * 32 + lk * 8]);
#pragma unroll
                    for (int i = 0; i < 4; i++)
#pragma unroll
                        for (int j = 0; j < 4; j++) acc[i][j] = mfma16x16x32(af[i], bfr[j], acc[i][j]);
                    // the next tile's store (its data arrived a tile ago; buf ^ 1 is free
                    // since the last barrier) runs while these MFMAs execute
                    if (ks == 0 && t + 1 < kt1) store(buf ^ 1, ns);
                }
                __syncthreads();
                // x of tile t + 2 before the ring refill: waiting on it at the next
                // store then leaves the younger ring loads in flight
                load_a(t + 2);
                load_b(ns, t + 1 + Q2_RING);
            }
        }
    }

    // D of block (i, j): row 16 i + 4 lk + r, column 16 j + l16
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int64_t col = bn + wn + 16 * j + l16;
            if (col >= a.N) continue;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int64_t row = bm + wm + 16 * i + 4 * lk + r;
                if (row >= a.M) continue;
                if (a.splits == 1) a.y[row * a.N + col] = f32_to_bf16(acc[i][j][r]);
                else a.partial[((int64_t)blockIdx.y * a.M + row) * a.N + col] = acc[i][j][r];
            }
        }
}

__global__ __launch_bounds__(256) void qmm_split_reduce(const float* __restrict__ partial, int S,
                                                        int64_t count, uint16_t* __restrict__ y) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= count) return;
    float acc = 0.f;
    for (int s = 0; s < S; s++) acc += partial[(int64_t)s * count + i];
    y[i] = f32_to_bf16(acc);
}

struct Qmm2Plan {
    int n_tiles, m_tiles, splits, kt_per_split;
    size_t ws;
};

// K splits while the tiles would fill under half of the CUs (one 110 KB
// workgroup per CU), at least 8 k-tiles per split.
static Qmm2Plan plan_qmm2(int64_t M, int64_t N, int64_t K) {
    Qmm2Plan p;
    p.n_tiles = (int)ceil_div(N, Q2N);
    p.m_tiles = (int)ceil_div(M, Q2M);
    const int tiles = p.n_tiles * p.m_tiles;
    const int nk = (int)(K / Q2K);
    int s = tiles * 2 <= 256 ? 256 / tiles : 1;
    if (s > nk / 8) s = nk / 8 > 0 ? nk / 8 : 1;
    p.kt_per_split = (int)ceil_div(nk, s);
    p.splits = (int)ceil_div(nk, p.kt_per_split);
    p.ws = p.splits > 1 ? (size_t)p.splits * M * N * sizeof(float) : 0;
    return p;
}

size_t qmm_gemm_workspace(int64_t M, int64_t K, int64_t N) {
    if (M <= 128) return 0;
    return plan_qmm2(M, N, K).ws;
}

int qmm_gemm(const void* x, int64_t M, int64_t K, int64_t N, const uint32_t* w,
             const void* scales, const void* biases, int group_size, int bits, void* y,
             void* workspace, size_t workspace_bytes, hipStream_t st) {
    KMI_CHECK_ARG(K % GBK == 0, "quantized_matmul: K=%lld must be a multiple of 64 for M > 16",
                  (long long)K);
    KMI_CHECK_ARG(group_size >= 32, "quantized_matmul: group_size %d", group_size);
    const uint16_t* xx = (const uint16_t*)x;
    const uint16_t* ss = (const uint16_t*)scales;
    const uint16_t* bb = (const uint16_t*)biases;
    uint16_t* yy = (uint16_t*)y;
    if (M > 128) {
        KMI_CHECK_ARG(M * K * 2 < (1LL << 31) && N * K * bits / 8 < (1LL << 31),
                      "quantized_matmul: x or w past 2 GiB");
        const Qmm2Plan p = plan_qmm2(M, N, K);
        if (p.ws > 0 && (!workspace || workspace_bytes < p.ws)) {
            set_error("quantized_matmul: workspace of %zu bytes needed, %zu given", p.ws, workspace_bytes);
            return EWORKSPACE;
        }
        Qmm2Args a = {xx, w, ss, bb, yy, (float*)workspace, M, N, K, p.kt_per_split, p.splits, p.n_tiles};
        const dim3 grid((unsigned)(p.n_tiles * p.m_tiles), (unsigned)p.splits);
#define KMI_QMM2(B, G) qmm2_kernel<B, G><<<grid, 512, 0, st>>>(a)
        if (bits == 4) {
            if (group_size == 32) KMI_QMM2(4, 32);
            else if (group_size == 64) KMI_QMM2(4, 64);
            else KMI_QMM2(4, 128);
        } else {
            if (group_size == 32) KMI_QMM2(8, 32);
            else if (group_size == 64) KMI_QMM2(8, 64);
            else KMI_QMM2(8, 128);
        }
#undef KMI_QMM2
        KMI_CHECK_LAUNCH("qmm2");
        if (p.splits > 1) {
            const int64_t count = M * N;
            qmm_split_reduce<<<(unsigned)ceil_div(count, 256), 256, 0, st>>>((const float*)workspace, p.splits,
                                                                              count, yy);
            KMI_CHECK_LAUNCH("qmm_split_reduce");
        }
        return OK;
    }
    dim3 grid((unsigned)ceil_div(N, GBN), (unsigned)ceil_div(M, GBM));
    KMI_CHECK_ARG(grid.y < 65536, "quantized_matmul: M too large");
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
