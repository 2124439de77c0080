// SwitchGLU's two projections at prefill sizes (src/knurlogic/engine/
// families/glm5/architecture/glm5_next/_mlx_vlm/models/switch_layers.py:
// 172-193 over QuantizedSwitchLinear, :71-86): rows grouped by expert (the
// GPU sort), each expert tile of up to BM rows multiplied by its expert's
// weights as a GEMM on v_mfma_f32_32x32x16_bf16 -- the decode kernels'
// skinny MFMA tiles stop paying once an expert sees more rows than one
// 16-row fragment holds.
//
// The k-tile pipeline is the dense prefill GEMM's (qmm.hip, qmm5): a
// workgroup of 8 waves owns a BM x BN tile of y (BM = 256, BN = 128 as 4 x 2
// waves, or BM = 128, BN = 256 as 2 x 4), each wave 64 x 64 as 2 x 2 MFMA
// blocks; x and the packed weights run MG_RING k-tiles ahead in register
// rings; per k-tile the weight tile is dequantized once (fp32 s * q + b,
// one bf16 rounding) into the second LDS buffer while the first feeds the
// MFMAs.  What is grouped:
//   - A rows are the tile's rows: their x rows (row id / lhs_div) gathered
//     through the sort's row ids, rows past the tile reading zeros;
//   - B rows are the tile's expert's; with the GLU epilogue a wave's two
//     32-column blocks are the gate and the up rows of the same 32 output
//     columns, so a lane holds gate and up of an output in the same
//     accumulator slot and writes act = round(round(silu_f32(round(gate)))
//     * round(up)) -- the roundings of the other SwitchGLU kernels;
//   - outputs go to the row ids' rows.
// Workgroups are numbered so that the column tiles of one expert tile run on
// one XCD (workgroup i runs on XCD i % 8), where its x rows stay in L2.
#include "qgemv.hpp"
#include "../../include/knurlogic_amd.h"

namespace kmi {

namespace {

constexpr int MGK = 64, MGLDS = MGK + 8;   // k per tile; bf16 per LDS row (16-byte pad)
constexpr int MG_RING = 4;                 // k-tiles of raw loads in flight
constexpr uint32_t MG_DEAD = 0x80000000u;  // an offset past every extent: reads 0

__device__ __forceinline__ f32x16 mg_mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

// 8 consecutive weights (4-bit: one word; 8-bit: two) -> 4 bf16 pairs of s * q + b
template <int BITS>
__device__ __forceinline__ u32x4 mg_dequant8(uint32_t w0, uint32_t w1, float sc, float bi) {
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

__device__ __forceinline__ float mg_bf16r(float v) { return bf16_to_f32(f32_to_bf16(v)); }

__device__ __forceinline__ float mg_f32_kept(double v) {
    float f = (float)v;
    asm volatile("" : "+v"(f));   // keep the float32 rounding (no fused f64 -> bf16 rounding)
    return f;
}

}  // namespace

// a.tiles / a.sorted: the sort's expert tiles; a.lhs_div: x row = row id /
// lhs_div; a.erows, a.up_off: rows per expert and the first up row (GLU).
// n_tiles: column tiles per expert tile; slots: tile slots of the grid.
template <int BITS, int GS, int BM, bool GLU>
__global__ __launch_bounds__(512, 1) void moe_gemm_kernel(QgArgs a, int n_tiles, int tile_slots) {
    constexpr int BN = 256 * 128 / BM;            // 128 or 256 columns of B
    constexpr int WN = BN / 64;                   // waves along N (2 or 4)
    constexpr int TPR = 512 / BN;                 // threads per B row (4 or 2)
    constexpr int WPT = MGK / TPR;                // weights per thread per k-tile (16 or 32)
    constexpr int QB = WPT * BITS / 8;            // their bytes (8, 16 or 32)
    constexpr int XC = BM / 64;                   // 16-byte x pieces per thread per k-tile
    constexpr int EPW = 32 / BITS;
    constexpr int TB = MGK * BITS / 8;            // bytes of a weight row per k-tile
    static_assert(GS >= WPT && GS % WPT == 0, "a thread's weights lie in one group");
    __shared__ __align__(16) uint16_t As[2][BM * MGLDS];
    __shared__ __align__(16) uint16_t Bs[2][BN * MGLDS];
    __shared__ int32_t rid_s[BM];                 // row id of tile row m (-1: none)

    // workgroup -> (tile, column tile): the column tiles of a tile share an XCD
    const int id = (int)blockIdx.x, xcd = id & 7, kk = id >> 3;
    const int tile = 8 * (kk / n_tiles) + xcd, nt = kk % n_tiles;
    if (tile >= tile_slots) return;
    const int32_t* tp = a.tiles + 3 * (int64_t)tile;
    const int count = tp[2], expert = tp[0], start = tp[1];
    if (count <= 0 || count > BM || expert < 0 || expert >= a.E) return;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, h = lane >> 5;
    const int K = (int)a.K, nk = K / MGK;
    const int64_t wpr = a.K / EPW, gpr = a.K / GS;

    if (tid < BM) rid_s[tid] = tid < count ? a.sorted[start + tid] : -1;
    __syncthreads();

    // x pieces: piece c = tid + 512 i -> tile row c / 8, 16-byte piece c % 8
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, a.xrows * a.K * 2);
    uint32_t xoff[XC];
#pragma unroll
    for (int i = 0; i < XC; i++) {
        const int c = tid + 512 * i, m = c >> 3;
        const int r = rid_s[m];
        const int64_t xr = r < 0 ? -1 : (int64_t)r / a.lhs_div;
        xoff[i] = xr >= 0 && xr < a.xrows ? (uint32_t)((xr * a.K + (c & 7) * 8) * 2) : MG_DEAD;
    }
    // weights: thread -> B row tid / TPR, its part tid % TPR (WPT weights)
    const int brow = tid / TPR, bpart = tid % TPR;
    int64_t wrow;                                 // the B row's row within the expert (-1: past N)
    if constexpr (GLU) {
        const int wv = brow / 64, j = (brow % 64) / 32, l = brow % 32;
        const int64_t col = (int64_t)nt * (BN / 2) + 32 * wv + l;
        wrow = col < a.N ? (j ? a.up_off : 0) + col : -1;
    } else {
        const int64_t col = (int64_t)nt * BN + brow;
        wrow = col < a.N ? col : -1;
    }
    const int64_t e0 = (int64_t)expert * a.erows;
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.w + e0 * wpr, a.erows * wpr * 4);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.s + e0 * gpr, a.erows * gpr * 2);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(a.b + e0 * gpr, a.erows * gpr * 2);
    const uint32_t woff = wrow < 0 ? MG_DEAD : (uint32_t)(wrow * wpr * 4 + bpart * QB);
    const uint32_t soff = wrow < 0 ? MG_DEAD : (uint32_t)(wrow * gpr * 2 + 2 * ((WPT * bpart) / GS));

    u32x4 ra[MG_RING][XC];                        // x ring
    uint32_t rwv[MG_RING][QB / 4];                // weight ring
    uint32_t rsc[MG_RING], rbi[MG_RING];

    auto load_x = [&](int slot, int kt) {
        const uint32_t so = kt < nk ? (uint32_t)kt * (MGK * 2) : MG_DEAD;
#pragma unroll
        for (int i = 0; i < XC; i++) ra[slot][i] = __builtin_amdgcn_raw_buffer_load_b128(rx, (int)xoff[i], (int)so, 0);
    };
    auto load_w = [&](int slot, int kt) {
        const bool live = kt < nk;
        const uint32_t so = live ? (uint32_t)kt * TB : MG_DEAD;
        if constexpr (QB == 8) {
            const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rw, (int)woff, (int)so, 0);
            rwv[slot][0] = v.x; rwv[slot][1] = v.y;
        } else {
#pragma unroll
            for (int q = 0; q < QB / 16; q++) {
                const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rw, (int)(woff + 16 * q), (int)so, 0);
                rwv[slot][4 * q] = v.x; rwv[slot][4 * q + 1] = v.y;
                rwv[slot][4 * q + 2] = v.z; rwv[slot][4 * q + 3] = v.w;
            }
        }
        const uint32_t sg = live ? (uint32_t)(2 * (((int64_t)kt * MGK) / GS)) : MG_DEAD;
        rsc[slot] = __builtin_amdgcn_raw_buffer_load_b16(rs, (int)soff, (int)sg, 0);
        rbi[slot] = __builtin_amdgcn_raw_buffer_load_b16(rb, (int)soff, (int)sg, 0);
    };
    auto store_x = [&](int buf, int slot) {
#pragma unroll
        for (int i = 0; i < XC; i++) {
            const int c = tid + 512 * i;
            *(u32x4*)(&As[buf][(c >> 3) * MGLDS + (c & 7) * 8]) = ra[slot][i];
        }
    };
    auto store_w = [&](int buf, int slot) {
        const float sc = bf16_to_f32((uint16_t)rsc[slot]), bi = bf16_to_f32((uint16_t)rbi[slot]);
        uint16_t* dst = &Bs[buf][brow * MGLDS + WPT * bpart];
#pragma unroll
        for (int q = 0; q < WPT / 8; q++) {
            if constexpr (BITS == 4) *(u32x4*)(dst + 8 * q) = mg_dequant8<4>(rwv[slot][q], 0u, sc, bi);
            else *(u32x4*)(dst + 8 * q) = mg_dequant8<8>(rwv[slot][2 * q], rwv[slot][2 * q + 1], sc, bi);
        }
    };

    const int wm = (wave / WN) * 64, wn = (wave % WN) * 64;
    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

#pragma unroll
    for (int r = 0; r < MG_RING; r++) {
        load_x(r, r);
        load_w(r, r);
    }
    store_x(0, 0);
    store_w(0, 0);
    load_x(0, MG_RING);
    load_w(0, MG_RING);
    __syncthreads();

    for (int kb = 0; kb < nk; kb += MG_RING) {
#pragma unroll
        for (int u = 0; u < MG_RING; u++) {
            const int t = kb + u;
            if (t < nk) {
                const int buf = t & 1;
                const int ns = (u + 1) % MG_RING;        // ring slot of tile t + 1
                u32x4 af[4][2], bf[4][2];
#pragma unroll
                for (int s = 0; s < 4; s++)
#pragma unroll
                    for (int i = 0; i < 2; i++) {
                        af[s][i] = *(const u32x4*)(&As[buf][(wm + 32 * i + l32) * MGLDS + 32 * h + 8 * s]);
                        bf[s][i] = *(const u32x4*)(&Bs[buf][(wn + 32 * i + l32) * MGLDS + 32 * h + 8 * s]);
                    }
#pragma unroll
                for (int s = 0; s < 4; s++)
#pragma unroll
                    for (int i = 0; i < 2; i++)
#pragma unroll
                        for (int j = 0; j < 2; j++) acc[i][j] = mg_mfma(af[s][i], bf[s][j], acc[i][j]);
                // tile t + 1 into the other buffers (past the last: zeros,
                // never read), then its ring slot refilled, between the MFMAs
                store_w(buf ^ 1, ns);
                store_x(buf ^ 1, ns);
                load_x(ns, t + 1 + MG_RING);
                load_w(ns, t + 1 + MG_RING);
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

    // D of block (i, j): tile row 32 i + 8 (r / 4) + 4 h + r % 4, B row 32 j + l32.
    // Stored through a buffer view of y: a row's offset from its row id in
    // 32 bits, and a row past the tile (row id -1) or a column past N at an
    // offset past the view, so no branch; one v_cvt_pk_bf16_f32 per two rows
    // (tile rows m and m + 1 of a lane).
    const __amdgpu_buffer_rsrc_t ry = make_rsrc(a.y, a.rows * a.N * 2);
    const uint32_t rowb = (uint32_t)a.N * 2;
    auto off = [&](int m, bool col_ok, int64_t col) -> uint32_t {
        const int rid = rid_s[m];
        return col_ok && rid >= 0 ? (uint32_t)rid * rowb + (uint32_t)col * 2 : MG_DEAD;
    };
    if constexpr (GLU) {
        const int64_t col = (int64_t)nt * (BN / 2) + wn / 2 + l32;
        const bool cok = col < a.N;
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int r = 0; r < 16; r += 2) {
                const int m = wm + 32 * i + 8 * (r / 4) + 4 * h + (r % 4);
                // act = round(round(silu_f32(round(gate))) * round(up))
                const float p0 = silu_bf16r(mg_bf16r(acc[i][0][r])) * mg_bf16r(acc[i][1][r]);
                const float p1 = silu_bf16r(mg_bf16r(acc[i][0][r + 1])) * mg_bf16r(acc[i][1][r + 1]);
                const uint32_t v = cvt_pk_bf16(p0, p1);
                __builtin_amdgcn_raw_buffer_store_b16((uint16_t)v, ry, (int)off(m, cok, col), 0, 0);
                __builtin_amdgcn_raw_buffer_store_b16((uint16_t)(v >> 16), ry, (int)off(m + 1, cok, col), 0, 0);
            }
    } else {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int64_t col = (int64_t)nt * BN + wn + 32 * j + l32;
            const bool cok = col < a.N;
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int r = 0; r < 16; r += 2) {
                    const int m = wm + 32 * i + 8 * (r / 4) + 4 * h + (r % 4);
                    const uint32_t v = cvt_pk_bf16(acc[i][j][r], acc[i][j][r + 1]);
                    __builtin_amdgcn_raw_buffer_store_b16((uint16_t)v, ry, (int)off(m, cok, col), 0, 0);
                    __builtin_amdgcn_raw_buffer_store_b16((uint16_t)(v >> 16), ry, (int)off(m + 1, cok, col), 0, 0);
                }
        }
    }
}

namespace {

template <int BITS, int GS, int BM>
int launch_mg(const QgArgs& a, bool glu, int64_t tile_slots, hipStream_t st) {
    constexpr int BN = 256 * 128 / BM;
    const int64_t cols = glu ? BN / 2 : BN;
    const int n_tiles = (int)ceil_div(a.N, cols);
    const int64_t wgs = 8 * n_tiles * ceil_div(tile_slots, 8);
    if (wgs >= (1LL << 31)) {
        set_error("moe_gemm: grid of %lld workgroups", (long long)wgs);
        return EINVAL_ARG;
    }
    const dim3 grid((unsigned)wgs);
    if (glu) moe_gemm_kernel<BITS, GS, BM, true><<<grid, 512, 0, st>>>(a, n_tiles, (int)tile_slots);
    else moe_gemm_kernel<BITS, GS, BM, false><<<grid, 512, 0, st>>>(a, n_tiles, (int)tile_slots);
    return OK;
}

template <int BM>
int launch_mg_bm(const QgArgs& a, int bits, int gs, bool glu, int64_t tile_slots, hipStream_t st) {
    if (bits == 4 && gs == 32) return launch_mg<4, 32, BM>(a, glu, tile_slots, st);
    if (bits == 4 && gs == 64) return launch_mg<4, 64, BM>(a, glu, tile_slots, st);
    if (bits == 4 && gs == 128) return launch_mg<4, 128, BM>(a, glu, tile_slots, st);
    if (bits == 8 && gs == 32) return launch_mg<8, 32, BM>(a, glu, tile_slots, st);
    if (bits == 8 && gs == 64) return launch_mg<8, 64, BM>(a, glu, tile_slots, st);
    if (bits == 8 && gs == 128) return launch_mg<8, 128, BM>(a, glu, tile_slots, st);
    set_error("moe_gemm: %d-bit, group %d", bits, gs);
    return EINVAL_ARG;
}

}  // namespace

bool moe_gemm_supported(int64_t H, int64_t I, int bits, int gs, int mx) {
    return !mx && (bits == 4 || bits == 8) && (gs == 32 || gs == 64 || gs == 128) && H % MGK == 0 &&
           I % MGK == 0 && H % gs == 0 && I % gs == 0;
}

int launch_moe_gemm(const QgArgs& a, int bits, int gs, bool glu, int tile_rows, int64_t tile_slots,
                    hipStream_t st) {
    if (!a.tiles || !a.sorted || a.mx || a.K % MGK || a.lhs_div < 1 || (glu && a.up_off <= 0)) {
        set_error("moe_gemm: expert tiles of affine weights, K %% 64 == 0");
        return EINVAL_ARG;
    }
    if (a.xrows * a.K * 2 >= (1LL << 31) || a.erows * (a.K * bits / 8) >= (1LL << 31) ||
        a.rows * a.N * 2 >= (1LL << 31)) {
        set_error("moe_gemm: x, y or an expert's weights past 2 GiB");
        return EINVAL_ARG;
    }
    if (tile_rows == 128) return launch_mg_bm<128>(a, bits, gs, glu, tile_slots, st);
    if (tile_rows == 256) return launch_mg_bm<256>(a, bits, gs, glu, tile_slots, st);
    set_error("moe_gemm: tile rows %d (128 or 256)", tile_rows);
    return EINVAL_ARG;
}

}  // namespace kmi
