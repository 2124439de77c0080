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

struct QgemmArgs {
    const uint16_t* x;          // [M, K] bf16
    const uint32_t* w;          // [N, K*bits/32]
    const uint16_t* s;          // [N, K/gs] bf16
    const uint16_t* b;
    uint16_t* y;                // [M, N] bf16 (one split)
    float* partial;             // [splits, M, N] fp32 (several splits)
    int64_t M, N, K;
    int kt_per_split, splits, n_tiles;
};

// =============================================================================
// qmm5: M > 128.  Block tile 256 (M) x 128 (N) x 64 (K); 8 waves (two per
// SIMD) as 4 (M) x 2 (N), each a 64 x 64 tile of y as 2 x 2 blocks of
// v_mfma_f32_32x32x16_bf16 (64 fp32 accumulators per lane).
//   - x and the dequantized weights are staged through LDS (two buffers),
//     both loaded with 8 lanes per 128-byte row segment.  The weight tile is
//     dequantized once per workgroup (fp32 s*q + b, one bf16 rounding: 16
//     values per thread).
//   - k order: in a k-tile, lane half h reads k in [32h, 32h + 32) and MFMA
//     step s the 8 values 32h + 8s .. +8 of it, for x and w alike (the
//     contraction is unchanged).
//   - Per k-tile a wave reads all 16 of its fragments, then runs 16 MFMAs
//     with tile t+1's dequantization and LDS stores between them; x and
//     weights run Q5_RING k-tiles ahead in register rings (x mostly comes
//     from L2 or the last-level cache, whose latency one tile does not
//     cover).
//   - Global load offsets: the lane part is fixed, the k-tile part is the
//     scalar offset (past the split: 2^31, which reads 0).
//   - Workgroups are numbered so that the m-tiles of one n-tile share an
//     XCD (and its L2).  Rows past M, columns past N and k-tiles past the
//     split read zeros from their buffer views.  When the tiles leave CUs
//     idle, K is split: each split writes fp32 partials and
//     qmm_split_reduce sums them in split order.
// Measured limits on gfx950 that shaped it: a 32x32x16 MFMA occupies the
// matrix core 32 cycles, and stays hidden only while a wave issues about 4
// other instructions per MFMA (an instruction takes ~4.5 cycles to issue),
// so instruction count per MFMA is the budget; LDS serves ~190-210 B/clk per
// CU; loads with one row per lane run at a quarter of the rate of loads with
// 8 lanes per 128-byte row.
// =============================================================================
constexpr int Q5M = 256, Q5N = 128, Q5K = 64, Q5LDS = Q5K + 8;
constexpr int Q5_RING = 4;


__device__ __forceinline__ f32x16 mfma32x32x16(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

// 8 consecutive weights (packed: 4-bit in one word, 8-bit in two) dequantized
// to 4 bf16 pairs.
template <int BITS>
__device__ __forceinline__ u32x4 q5_dequant8(uint32_t w0, uint32_t w1, float sc, float bi) {
    u32x4 o;
    if constexpr (BITS == 4) {
#pragma unroll
        for (int j = 0; j < 4; j++)
            o[j] = cvt_pk_bf16(__builtin_fmaf(sc, (float)((w0 >> (8 * j)) & 15u), bi),
                               __builtin_fmaf(sc, (float)((w0 >> (8 * j + 4)) & 15u), bi));
    } else {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            o[j] = cvt_pk_bf16(__builtin_fmaf(sc, (float)((w0 >> (16 * j)) & 255u), bi),
                               __builtin_fmaf(sc, (float)((w0 >> (16 * j + 8)) & 255u), bi));
            o[2 + j] = cvt_pk_bf16(__builtin_fmaf(sc, (float)((w1 >> (16 * j)) & 255u), bi),
                                   __builtin_fmaf(sc, (float)((w1 >> (16 * j + 8)) & 255u), bi));
        }
    }
    return o;
}

template <int BITS, int GS>
__global__ __launch_bounds__(512, 1) void qmm5_kernel(QgemmArgs a) {
    constexpr int EPW = 32 / BITS;
    constexpr int TB = Q5K * BITS / 8;           // bytes of a weight row per k-tile
    constexpr int QB = 16 * BITS / 8;            // bytes of a thread's 16 weights (8 or 16)
    constexpr uint32_t DEAD = 0x80000000u;       // scalar offset past every extent
    __shared__ __align__(16) uint16_t As[2][Q5M * Q5LDS];
    __shared__ __align__(16) uint16_t Bs[2][Q5N * Q5LDS];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, h = lane >> 5;
    // ids grp*8*mtn + 8*mt + x -> n-tile 8 grp + x, m-tile mt (XCD = id % 8)
    const int mtn = (int)((a.M + Q5M - 1) / Q5M);
    const int id = (int)blockIdx.x, grp = id / (8 * mtn), rem = id % (8 * mtn);
    const int gw = a.n_tiles - 8 * grp < 8 ? a.n_tiles - 8 * grp : 8;
    const int mt = rem / gw, nt = 8 * grp + rem % gw;
    const int64_t bm = (int64_t)mt * Q5M, bn = (int64_t)nt * Q5N;
    const int nk = (int)(a.K / Q5K);
    const int kt0 = (int)blockIdx.y * a.kt_per_split;
    const int kt1 = kt0 + a.kt_per_split < nk ? kt0 + a.kt_per_split : nk;
    const int64_t wpr = a.K / EPW, gpr = a.K / GS;

    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x + bm * a.K, (a.M - bm) * a.K * 2);
    const int64_t nrows = a.N - bn;
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.w + bn * wpr, nrows * wpr * 4);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.s + bn * gpr, nrows * gpr * 2);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(a.b + bn * gpr, nrows * gpr * 2);

    // x: chunk c = tid + 512 i -> row c / 8, 16-byte piece c % 8
    uint32_t xoff[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int c = tid + 512 * i;
        xoff[i] = (uint32_t)(((c >> 3) * a.K + (c & 7) * 8) * 2);
    }
    // weights: thread -> row tid / 4, quarter q = tid % 4 (16 weights)
    const int brow = tid >> 2, bq = tid & 3;
    const uint32_t woff = (uint32_t)(brow * wpr * 4 + bq * QB);
    const uint32_t soff = (uint32_t)(brow * gpr * 2 + 2 * ((16 * bq) / GS));

    u32x4 ra[Q5_RING][4];                         // x ring
    uint32_t rwv[Q5_RING][QB / 4];                // weight ring
    uint32_t rsc[Q5_RING], rbi[Q5_RING];

    auto load_x = [&](int slot, int kt) {
        const uint32_t so = kt < kt1 ? (uint32_t)kt * (Q5K * 2) : DEAD;
#pragma unroll
        for (int i = 0; i < 4; i++)
            ra[slot][i] = __builtin_amdgcn_raw_buffer_load_b128(rx, (int)xoff[i], (int)so, 0);
    };
    auto load_w = [&](int slot, int kt) {
        const bool live = kt < kt1;
        const uint32_t so = live ? (uint32_t)kt * TB : DEAD;
        if constexpr (QB == 8) {
            const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rw, (int)woff, (int)so, 0);
            rwv[slot][0] = v.x; rwv[slot][1] = v.y;
        } else {
            const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rw, (int)woff, (int)so, 0);
            rwv[slot][0] = v.x; rwv[slot][1] = v.y; rwv[slot][2] = v.z; rwv[slot][3] = v.w;
        }
        const uint32_t sg = live ? (uint32_t)(2 * (((int64_t)kt * Q5K) / GS)) : DEAD;
        rsc[slot] = __builtin_amdgcn_raw_buffer_load_b16(rs, (int)soff, (int)sg, 0);
        rbi[slot] = __builtin_amdgcn_raw_buffer_load_b16(rb, (int)soff, (int)sg, 0);
    };
    auto store_x = [&](int buf, int slot) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int c = tid + 512 * i;
            *(u32x4*)(&As[buf][(c >> 3) * Q5LDS + (c & 7) * 8]) = ra[slot][i];
        }
    };
    auto store_w = [&](int buf, int slot) {
        const float sc = bf16_to_f32((uint16_t)rsc[slot]), bi = bf16_to_f32((uint16_t)rbi[slot]);
        uint16_t* dst = &Bs[buf][brow * Q5LDS + 16 * bq];
        if constexpr (BITS == 4) {
            *(u32x4*)dst = q5_dequant8<4>(rwv[slot][0], 0u, sc, bi);
            *(u32x4*)(dst + 8) = q5_dequant8<4>(rwv[slot][1], 0u, sc, bi);
        } else {
            *(u32x4*)dst = q5_dequant8<8>(rwv[slot][0], rwv[slot][1], sc, bi);
            *(u32x4*)(dst + 8) = q5_dequant8<8>(rwv[slot][2], rwv[slot][3], sc, bi);
        }
    };

    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

#pragma unroll
    for (int r = 0; r < Q5_RING; r++) {
        load_x(r, kt0 + r);
        load_w(r, kt0 + r);
    }
    store_x(0, 0);
    store_w(0, 0);
    load_x(0, kt0 + Q5_RING);
    load_w(0, kt0 + Q5_RING);
    __syncthreads();

    for (int kb = kt0; kb < kt1; kb += Q5_RING) {
#pragma unroll
        for (int u = 0; u < Q5_RING; u++) {
            const int t = kb + u;
            if (t < kt1) {
                const int buf = (t - kt0) & 1;
                const int ns = (u + 1) % Q5_RING;        // ring slot of tile t + 1
                u32x4 af[4][2], bf[4][2];
#pragma unroll
                for (int s = 0; s < 4; s++)
#pragma unroll
                    for (int i = 0; i < 2; i++) {
                        af[s][i] = *(const u32x4*)(&As[buf][(wm + 32 * i + l32) * Q5LDS + 32 * h + 8 * s]);
                        bf[s][i] = *(const u32x4*)(&Bs[buf][(wn + 32 * i + l32) * Q5LDS + 32 * h + 8 * s]);
                    }
#pragma unroll
                for (int s = 0; s < 4; s++)
#pragma unroll
                    for (int i = 0; i < 2; i++)
#pragma unroll
                        for (int j = 0; j < 2; j++) acc[i][j] = mfma32x32x16(af[s][i], bf[s][j], acc[i][j]);
                // tile t+1 into the other buffers (past the split: zeros, harmless),
                // then its ring slot refilled, all between the MFMAs
                store_w(buf ^ 1, ns);
                store_x(buf ^ 1, ns);
                load_x(ns, t + 1 + Q5_RING);
                load_w(ns, t + 1 + Q5_RING);
                __builtin_amdgcn_sched_group_barrier(0x100, 16, 0);      // LDS reads
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
                    __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);   // VALU
                    if (i >= 8) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);   // VMEM read
                }
                __syncthreads();
            }
        }
    }

    // D of block (i, j): row 32 i + 8 (r / 4) + 4 h + r % 4, column 32 j + l32.
    // Stored through a buffer view of the output: the lane's column and the
    // wave's first row in the offset register, the rest of the row (the same
    // for the wave) in the scalar offset, so an output costs a conversion
    // and a store.  A row past M lands past the view and is dropped; a
    // column past N takes an offset past every view.  (Rows r and r + 1 of a
    // lane are adjacent rows: one v_cvt_pk_bf16_f32 per pair.)
    const int64_t N = a.N;
    const int64_t row0 = bm + wm + 4 * h;
    if (a.splits == 1) {
        const __amdgpu_buffer_rsrc_t ry = make_rsrc(a.y, a.M * N * 2);
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int64_t col = bn + wn + 32 * j + l32;
            const uint32_t vo = col < N ? (uint32_t)((row0 * N + col) * 2) : DEAD;
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int r = 0; r < 16; r += 2) {
                    const uint32_t so = (uint32_t)((32 * i + 8 * (r / 4) + r % 4) * N * 2);
                    const uint32_t v = cvt_pk_bf16(acc[i][j][r], acc[i][j][r + 1]);
                    __builtin_amdgcn_raw_buffer_store_b16((uint16_t)v, ry, (int)vo, (int)so, 0);
                    __builtin_amdgcn_raw_buffer_store_b16((uint16_t)(v >> 16), ry, (int)vo, (int)(so + N * 2), 0);
                }
        }
    } else {
        const __amdgpu_buffer_rsrc_t rp = make_rsrc(a.partial + (int64_t)blockIdx.y * a.M * N, a.M * N * 4);
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int64_t col = bn + wn + 32 * j + l32;
            const uint32_t vo = col < N ? (uint32_t)((row0 * N + col) * 4) : DEAD;
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const uint32_t so = (uint32_t)((32 * i + 8 * (r / 4) + r % 4) * N * 4);
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc[i][j][r]), rp, (int)vo, (int)so, 0);
                }
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

struct QgemmPlan {
    int n_tiles, m_tiles, splits, kt_per_split;
    size_t ws;
};

// K splits while the tiles would fill under half of the CUs (one workgroup
// per CU), at least 8 k-tiles per split.
static QgemmPlan plan_gemm(int64_t M, int64_t N, int64_t K) {
    QgemmPlan p;
    p.n_tiles = (int)ceil_div(N, Q5N);
    p.m_tiles = (int)ceil_div(M, Q5M);
    const int tiles = p.n_tiles * p.m_tiles;
    const int nk = (int)(K / Q5K);
    int s = tiles * 2 <= 256 ? 256 / tiles : 1;
    if (s > nk / 8) s = nk / 8 > 0 ? nk / 8 : 1;
    p.kt_per_split = (int)ceil_div(nk, s);
    p.splits = (int)ceil_div(nk, p.kt_per_split);
    p.ws = p.splits > 1 ? (size_t)p.splits * M * N * sizeof(float) : 0;
    return p;
}

size_t qmm_gemm_workspace(int64_t M, int64_t K, int64_t N) {
    if (M <= 128) return 0;
    return plan_gemm(M, N, K).ws;
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
        const QgemmPlan p = plan_gemm(M, N, K);
        KMI_CHECK_ARG(M * N * (p.splits > 1 ? 4 : 2) < (1LL << 31), "quantized_matmul: y past 2 GiB");
        if (p.ws > 0 && (!workspace || workspace_bytes < p.ws)) {
            set_error("quantized_matmul: workspace of %zu bytes needed, %zu given", p.ws, workspace_bytes);
            return EWORKSPACE;
        }
        QgemmArgs a = {xx, w, ss, bb, yy, (float*)workspace, M, N, K, p.kt_per_split, p.splits, p.n_tiles};
        const dim3 grid((unsigned)(p.n_tiles * p.m_tiles), (unsigned)p.splits);
#define KMI_QMM5(B, G) qmm5_kernel<B, G><<<grid, 512, 0, st>>>(a)
        if (bits == 4) {
            if (group_size == 32) KMI_QMM5(4, 32);
            else if (group_size == 64) KMI_QMM5(4, 64);
            else KMI_QMM5(4, 128);
        } else {
            if (group_size == 32) KMI_QMM5(8, 32);
            else if (group_size == 64) KMI_QMM5(8, 64);
            else KMI_QMM5(8, 128);
        }
#undef KMI_QMM5
        KMI_CHECK_LAUNCH("qmm5");
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
