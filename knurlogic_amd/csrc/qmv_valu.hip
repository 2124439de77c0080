// Decode-shape quantized GEMV on the VALU (M <= 4 activation rows per
// tile), templated on the launch shape; the host side (qmv.hip) picks the
// shape.  See qmv.hip for the arithmetic.
//
// Decode shapes are latency-bound unless the whole weight stream is in
// flight at once, so each wave issues every load of its rows (S 16-byte
// chunk slots per lane per row: all of K when K fits) right after the small
// L2-resident x and scale/bias loads, and the grid is sized so all waves are
// resident together.  Loads are consumed in issue order, so the math of the
// first chunks overlaps the arrival of the later ones.  All global reads are
// buffer loads: 32-bit offsets (one VGPR per address) and hardware range
// checks (reads past a buffer return 0) instead of clamps or branches --
// a guarded load becomes a branch whose join waits for the load.
#include "qmv_common.hpp"

namespace kmi {

template <int BITS, int MT, int RPW, int S, int WV>
__global__ __launch_bounds__(64 * WV) void qmv_valu_kernel(QmvArgs a) {
    constexpr int NT = 64 * WV;                   // threads per workgroup
    constexpr int CK = 128 / BITS;                // k per 16-byte chunk: 32 or 16
    constexpr int XV = CK / 8;                    // 16-byte x loads per chunk
    constexpr int SR = 4;                         // scale/bias pairs per thread held in registers
    constexpr int ROWS = WV * RPW;                // weight rows per workgroup
    extern __shared__ __align__(16) unsigned char smem[];

    Tile t;
    if (!resolve_tile(a, t)) return;
    const int C = (int)(a.K / CK);                // chunks per row
    const int NB = (C + 64 * S - 1) / (64 * S);   // load batches per row
    const int wpr = (int)(a.K / (32 / BITS));     // packed words per row
    const int gpr = (int)(a.K >> a.gs_shift);     // groups per row
    const int xstride = (int)a.K + 8;             // bf16 per LDS x row
    // x row m in LDS: [piece v8 < XV][chunk c < C] 16-byte slots, so the 64
    // lanes of one ds_read_b128 hit 64 consecutive slots
    uint16_t* xs = (uint16_t*)smem;                                                      // [MT][xstride]
    float* xc = (float*)(smem + (size_t)MT * xstride * 2);                               // [MT][C]
    uint32_t* sbl = (uint32_t*)(smem + (size_t)MT * xstride * 2 + (size_t)MT * C * 4);  // [ROWS][gpr]

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int nwg = (int)blockIdx.x * ROWS;
    const int n0 = nwg + wave * RPW;
    const int64_t eoff = (int64_t)t.expert * a.N;
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.w + eoff * wpr, a.N * (int64_t)wpr * 4);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.s + eoff * gpr, a.N * (int64_t)gpr * 2);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(a.b + eoff * gpr, a.N * (int64_t)gpr * 2);
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, a.Xrows * a.K * 2);
    const int nx = (int)t.count * C;              // x chunks of the tile
    const int nsb = ROWS * gpr;                   // scale/bias pairs of the workgroup

    // byte offset of x chunk (m, c); rows that do not exist get an offset
    // past every buffer, which reads as zeros
    constexpr uint32_t NONE = 0x80000000u;
    auto x_off = [&](int m, int c) -> uint32_t {
        const int64_t xrow = x_row_of(a, t.start + m);
        return (xrow >= 0 && xrow < a.Xrows) ? (uint32_t)((xrow * a.K + (int64_t)c * CK) * 2) : NONE;
    };
    auto stage_x = [&](int idx, const u32x4* v) {
        const int m = idx / C, c = idx - m * C;
        float sum = 0.f;
#pragma unroll
        for (int v8 = 0; v8 < XV; v8++)
            *(u32x4*)(xs + m * xstride + (v8 * C + c) * 8) = permute8<BITS>(v[v8], sum);
        xc[m * C + c] = sum;
    };
    auto sb_pair = [&](int idx) -> uint32_t {      // (scale | bias << 16) of pair idx
        const int rl = idx / gpr, g = idx - rl * gpr;
        const int off = (int)(((uint32_t)(nwg + rl) * (uint32_t)gpr + (uint32_t)g) * 2u);
        const uint32_t sv = __builtin_amdgcn_raw_buffer_load_b16(rs, off, 0, 0);
        const uint32_t bv = __builtin_amdgcn_raw_buffer_load_b16(rb, off, 0, 0);
        return sv | (bv << 16);
    };

    // (0) what will not fit in registers (many x rows, wide groups): plain
    // loops, before any weight load is issued so their waits drain nothing
    for (int idx = tid + NT; idx < nx; idx += NT) {
        const uint32_t off = x_off(idx / C, idx % C);
        u32x4 v[XV];
#pragma unroll
        for (int v8 = 0; v8 < XV; v8++)
            v[v8] = __builtin_amdgcn_raw_buffer_load_b128(rx, (int)(off + 16u * v8), 0, 0);
        stage_x(idx, v);
    }
    for (int idx = tid + NT * SR; idx < nsb; idx += NT) sbl[idx] = sb_pair(idx);

    // (1) this thread's x chunk and (2) scale/bias pairs
    u32x4 xr[XV];
    {
        const uint32_t off = tid < nx ? x_off(tid / C, tid % C) : NONE;
#pragma unroll
        for (int v8 = 0; v8 < XV; v8++)
            xr[v8] = __builtin_amdgcn_raw_buffer_load_b128(rx, (int)(off + 16u * v8), 0, 0);
    }
    uint32_t sr[SR];
#pragma unroll
    for (int j = 0; j < SR; j++) sr[j] = sb_pair(tid + NT * j);

    // (3) every weight load of this wave's rows for the first batch
    u32x4 W[S][RPW];
    auto load = [&](int nb) {
#pragma unroll
        for (int u = 0; u < S; u++) {
            const int c = lane + 64 * (nb * S + u);
#pragma unroll
            for (int r = 0; r < RPW; r++)
                W[u][r] = __builtin_amdgcn_raw_buffer_load_b128(
                    rw, (int)(((uint32_t)(n0 + r) * (uint32_t)wpr + (uint32_t)c * 4u) * 4u), 0, AUX_NT);
        }
    };
    load(0);

    // (4) x and scales/biases -> LDS
    if (tid < nx) stage_x(tid, xr);
#pragma unroll
    for (int j = 0; j < SR; j++)
        if (tid + NT * j < nsb) sbl[tid + NT * j] = sr[j];
    lds_barrier();

    float acc[RPW][MT];
#pragma unroll
    for (int r = 0; r < RPW; r++)
#pragma unroll
        for (int m = 0; m < MT; m++) acc[r][m] = 0.f;

    for (int nb = 0; nb < NB; nb++) {
        if (nb > 0) load(nb);
#pragma unroll
        for (int u = 0; u < S; u++) {
            const int c = lane + 64 * (nb * S + u);
            if (c >= C) continue;
            const int g = (c * CK) >> a.gs_shift;
#pragma unroll
            for (int m = 0; m < MT; m++) {
                if (m >= t.count) continue;
                const uint16_t* xp = xs + m * xstride + c * 8;
                u32x4 xv[XV];
#pragma unroll
                for (int v8 = 0; v8 < XV; v8++) xv[v8] = *(const u32x4*)(xp + v8 * C * 8);
                const float X = xc[m * C + c];
#pragma unroll
                for (int r = 0; r < RPW; r++) {
                    float A0 = 0.f, A1 = 0.f;
                    if constexpr (BITS == 4) {
#pragma unroll
                        for (int wd = 0; wd < 4; wd++) {
                            const u32x4 q = nibbles_to_bf16_magic(W[u][r][wd]);
                            A0 = dot2(xv[wd][0], q[0], A0);
                            A1 = dot2(xv[wd][1], q[1], A1);
                            A0 = dot2(xv[wd][2], q[2], A0);
                            A1 = dot2(xv[wd][3], q[3], A1);
                        }
                    } else {
#pragma unroll
                        for (int wd = 0; wd < 4; wd++) {
                            const uint32_t word = W[u][r][wd];
                            A0 = dot2(xv[wd >> 1][(wd & 1) * 2], bytes_to_bf16x2(word, 0), A0);
                            A1 = dot2(xv[wd >> 1][(wd & 1) * 2 + 1], bytes_to_bf16x2(word, 2), A1);
                        }
                    }
                    const uint32_t sbv = sbl[(wave * RPW + r) * gpr + g];
                    const float sc = bf16_to_f32((uint16_t)(sbv & 0xffffu));
                    const float bi = bf16_to_f32((uint16_t)(sbv >> 16));
                    const float bb = (BITS == 4) ? __builtin_fmaf(-128.f, sc, bi) : bi;
                    acc[r][m] = __builtin_fmaf(sc, A0 + A1, __builtin_fmaf(bb, X, acc[r][m]));
                }
            }
        }
    }

#pragma unroll
    for (int r = 0; r < RPW; r++)
#pragma unroll
        for (int m = 0; m < MT; m++) {
            if (m >= t.count) continue;
            const float v = wave_sum(acc[r][m]);
            if (lane == 0 && n0 + r < a.N) a.y[y_row_of(a, t.start + m) * a.N + n0 + r] = f32_to_bf16(v);
        }
}

template <int BITS, int MT, int RPW, int S>
static bool launch_wv(const ValuShape& v, const QmvArgs& a, dim3 grid, size_t lds, hipStream_t st) {
    if (v.WV == 4) qmv_valu_kernel<BITS, MT, RPW, S, 4><<<grid, 256, lds, st>>>(a);
    else if (v.WV == 8) qmv_valu_kernel<BITS, MT, RPW, S, 8><<<grid, 512, lds, st>>>(a);
    else if (v.WV == 16) qmv_valu_kernel<BITS, MT, RPW, S, 16><<<grid, 1024, lds, st>>>(a);
    else return false;
    return true;
}

template <int BITS, int MT>
static bool launch_shape(const ValuShape& v, const QmvArgs& a, dim3 grid, size_t lds, hipStream_t st) {
    if (v.RPW == 1) {
        if (v.S == 1) return launch_wv<BITS, MT, 1, 1>(v, a, grid, lds, st);
        if (v.S == 2) return launch_wv<BITS, MT, 1, 2>(v, a, grid, lds, st);
        if (v.S == 4) return launch_wv<BITS, MT, 1, 4>(v, a, grid, lds, st);
        if (v.S == 8) return launch_wv<BITS, MT, 1, 8>(v, a, grid, lds, st);
    }
    if constexpr (MT == 1) {
        if (v.RPW == 2) {
            if (v.S == 1) return launch_wv<BITS, MT, 2, 1>(v, a, grid, lds, st);
            if (v.S == 2) return launch_wv<BITS, MT, 2, 2>(v, a, grid, lds, st);
            if (v.S == 4) return launch_wv<BITS, MT, 2, 4>(v, a, grid, lds, st);
        }
        if (v.RPW == 4) {
            if (v.S == 1) return launch_wv<BITS, MT, 4, 1>(v, a, grid, lds, st);
            if (v.S == 2) return launch_wv<BITS, MT, 4, 2>(v, a, grid, lds, st);
        }
    }
    return false;
}

bool launch_qmv_valu(int bits, int mt, const ValuShape& v, const QmvArgs& a, dim3 grid,
                     size_t lds, hipStream_t st) {
    if (bits == 4) {
        if (mt == 1) return launch_shape<4, 1>(v, a, grid, lds, st);
        if (mt == 2) return launch_shape<4, 2>(v, a, grid, lds, st);
        if (mt == 4) return launch_shape<4, 4>(v, a, grid, lds, st);
    } else if (bits == 8) {
        if (mt == 1) return launch_shape<8, 1>(v, a, grid, lds, st);
        if (mt == 2) return launch_shape<8, 2>(v, a, grid, lds, st);
        if (mt == 4) return launch_shape<8, 4>(v, a, grid, lds, st);
    }
    return false;
}

}  // namespace kmi
