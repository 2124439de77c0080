// Decode-shape quantized GEMV on the VALU: one activation row per tile (the
// dense M = 1 call, or one routed row per tile of gather_qmm).  The host side
// (qmv.hip) picks the launch shape.
//
// The work is HBM-bound only if the decode math stays well under the weight
// stream, so the inner loop is built around the fewest VALU operations per
// packed word:
//
//   * codes become fp16 "1024 + q" with one v_and_or_b32 per pair: a low
//     nibble (or a byte) lands in the low mantissa bits of 0x6400 = 1024.0,
//     and a high nibble is left in place, giving 1024 + 16 q, which is also
//     exact (fp16 has 10 mantissa bits).  A 4-bit word costs 1 shift + 4
//     and-or + 4 v_dot2_f32_f16 for 8 weights; an 8-bit word 2 v_perm_b32 +
//     2 v_dot2 for 4 weights.
//   * x is staged in LDS as fp16 with a power-of-two scale per 16-byte chunk
//     of weights (the chunk's largest |x| maps to [2^14, 2^15)), so every
//     bf16 value converts exactly and nothing overflows; the scale, the
//     chunk's x sum and the magic correction 1024 * (sum of x under low
//     codes + sum under high codes / 16) sit beside it in fp32.
//   * per chunk and row:  y += s * (mult * (A_lo + A_hi / 16) - corr) + b * X,
//     which is  s * sum(q x) + b * sum(x)  over the chunk (a chunk lies in
//     one quantization group).
//
// Every load of a wave is issued up front, the x piece first (it gates the
// LDS staging and the barrier; loads complete in issue order), then each
// chunk's weights, scale and bias in the order the loop consumes them.  All
// global reads are raw buffer loads: 32-bit offsets, and an offset past the
// buffer reads 0 with no traffic, which is how absent rows and chunks are
// expressed (no clamps, no branches around loads).
#include "qmv_common.hpp"

namespace kmi {

namespace {
constexpr uint32_t NONE = QV_NONE;
}  // namespace

// GATHER: tiles come from the expert sort (tile z = one routed row); else
// tile z is row z of a dense x, and no pointer-dependent branch delays the
// first loads (each scalar round trip to the kernel arguments costs the
// first wave of a CU most of a microsecond).
// MX: microscaled codes (E2M1 / E4M3 converted exactly to fp16, x staged in
// natural pair order), one E8M0 byte scale per 32 inputs, no bias term.
template <int BITS, int RPW, int S, int WV, bool GATHER, bool MX>
__global__ __launch_bounds__(64 * WV) void qmv_valu_kernel(QmvArgs a) {
    constexpr int NT = 64 * WV;                   // threads per workgroup
    constexpr uint32_t SB = MX ? 1 : 2;           // bytes per scale
    constexpr int CK = 128 / BITS;                // k per 16-byte chunk: 32 or 16
    constexpr int XV = CK / 8;                    // 8-element x pieces per chunk: 4 or 2
    extern __shared__ __align__(16) unsigned char smem[];

    Tile t;
    if constexpr (GATHER) {
        if (!resolve_tile(a, t)) return;
    } else {
        t.expert = 0;
        t.start = blockIdx.z;
        t.count = 1;
    }
    const int C = (int)(a.K / CK);                // chunks per row
    const int NB = (C + 64 * S - 1) / (64 * S);   // load batches per row
    const int wpr = (int)(a.K / (32 / BITS));     // packed words per row
    const int gpr = (int)(a.K >> a.gs_shift);     // groups per row
    const int P = (int)(a.K >> 3);                // x pieces per row
    u32x4* xs = (u32x4*)smem;                                  // [XV][C] fp16 pieces
    float4* xm = (float4*)(smem + (size_t)XV * C * 16);        // [C] {mult, corr, sum, -}

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: scalar offsets
    const int n0 = (int)blockIdx.x * (WV * RPW) + wave * RPW;
    const int64_t eoff = (int64_t)t.expert * a.N;
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.w + eoff * wpr, a.N * (int64_t)wpr * 4);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc((const char*)a.s + eoff * gpr * SB, a.N * (int64_t)gpr * SB);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc((const char*)a.b + eoff * gpr * SB, MX ? 0 : a.N * (int64_t)gpr * 2);
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, a.Xrows * a.K * 2);

    const int64_t xrow = GATHER ? x_row_of(a, t.start) : t.start;
    const bool xok = xrow >= 0 && xrow < a.Xrows;
    // Load offsets: lane-only VGPRs shared by every load of a stream, with
    // the wave-uniform part (x row, weight row, slot) in the scalar offset
    // operand, so issuing a wave's loads costs almost no VALU work (with
    // several waves per SIMD, prologue instructions delay the last wave's
    // loads).  NONE marks a lane with nothing to read.
    const uint32_t xso = xok ? (uint32_t)(xrow * a.K * 2) : 0u;
    auto xvo = [&](int p) -> uint32_t { return (xok && p < P) ? (uint32_t)p * 16u : NONE; };

    auto stage = [&](int p, u32x4 raw) { stage_x16<BITS, MX>(p, raw, P, C, xs, xm); };

    // (0) pieces beyond two per thread (long rows): staged before any
    // weight load is issued, so their waits drain nothing
    if (P > 2 * NT) {
        for (int p = tid + 2 * NT; p - (tid & 3) < P; p += NT) {
            const u32x4 raw = __builtin_amdgcn_raw_buffer_load_b128(rx, (int)xvo(p), (int)xso, 0);
            stage(p, raw);
        }
    }

    // (1) this thread's first two pieces, then every load of batch 0
    const u32x4 xr0 = __builtin_amdgcn_raw_buffer_load_b128(rx, (int)xvo(tid), (int)xso, 0);
    const u32x4 xr1 = __builtin_amdgcn_raw_buffer_load_b128(rx, (int)xvo(tid + NT), (int)xso, 0);

    // slots (64 chunks) with every lane in the row, and the partial one
    const int full = C >> 6;
    const bool in_tail = lane < (C & 63);
    const uint32_t vw = (uint32_t)lane * 16u;
    const uint32_t vg = (uint32_t)((lane * CK) >> a.gs_shift) * SB;
    const uint32_t vwt = in_tail ? vw : NONE, vgt = in_tail ? vg : NONE;
    // rows past N (only in the last wave of the grid) re-read row N-1; their
    // results are never stored
    uint32_t wrow[RPW], srow[RPW];
#pragma unroll
    for (int r = 0; r < RPW; r++) {
        const uint32_t row = (uint32_t)(n0 + r < a.N ? n0 + r : a.N - 1);
        wrow[r] = row * (uint32_t)wpr * 4u;
        srow[r] = row * (uint32_t)gpr * SB;
    }

    u32x4 W[S][RPW];
    uint32_t SC[S][RPW], BI[S][RPW];
    // The small scale/bias loads go first: each chunk-row then waits only
    // for its own weights (the barrier keeps the compiler from moving them
    // behind the weight loads).
    auto load = [&](int nb) {
#pragma unroll
        for (int u = 0; u < S; u++) {
            const int su = nb * S + u;
            const uint32_t vo = su < full ? vg : su == full ? vgt : NONE;
            const uint32_t so = (uint32_t)(((64 * su * CK) >> a.gs_shift) * SB);
#pragma unroll
            for (int r = 0; r < RPW; r++) {
                if constexpr (MX) {
                    SC[u][r] = __builtin_amdgcn_raw_buffer_load_b8(rs, (int)vo, (int)(srow[r] + so), 0);
                    BI[u][r] = 0u;
                } else {
                    SC[u][r] = __builtin_amdgcn_raw_buffer_load_b16(rs, (int)vo, (int)(srow[r] + so), 0);
                    BI[u][r] = __builtin_amdgcn_raw_buffer_load_b16(rb, (int)vo, (int)(srow[r] + so), 0);
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < S; u++) {
            const int su = nb * S + u;
            const uint32_t vo = su < full ? vw : su == full ? vwt : NONE;
#pragma unroll
            for (int r = 0; r < RPW; r++)
                W[u][r] = __builtin_amdgcn_raw_buffer_load_b128(rw, (int)vo, (int)(wrow[r] + (uint32_t)su * 1024u),
                                                                AUX_NT);
        }
    };
    load(0);

    // (2) x -> LDS
    stage(tid, xr0);
    if (P > NT) stage(tid + NT, xr1);
    lds_barrier();

    const Magic16 mk = magic16();
    float acc[RPW];
#pragma unroll
    for (int r = 0; r < RPW; r++) acc[r] = 0.f;

    for (int nb = 0; nb < NB; nb++) {
        if (nb > 0) load(nb);
#pragma unroll
        for (int u = 0; u < S; u++) {
            const int cbase = 64 * (nb * S + u);
            if (cbase >= C) break;                    // wave-uniform
            const int c = lane + cbase;
            const bool cok = c < C;
            const int cc = cok ? c : 0;
            u32x4 xv[XV];
#pragma unroll
            for (int v = 0; v < XV; v++) xv[v] = xs[v * C + cc];
            const float4 m = xm[cc];
#pragma unroll
            for (int r = 0; r < RPW; r++) {
                float nv;
                if constexpr (MX) {
                    nv = __builtin_fmaf(mx_scale(SC[u][r]), chunk_mx<BITS>(W[u][r], xv, m), acc[r]);
                } else {
                    const float q = chunk_qx<BITS>(W[u][r], xv, m, mk);
                    const float sv = __uint_as_float(SC[u][r] << 16), bv = __uint_as_float(BI[u][r] << 16);
                    nv = __builtin_fmaf(sv, q, __builtin_fmaf(bv, m.z, acc[r]));
                }
                acc[r] = cok ? nv : acc[r];
            }
        }
    }

    const int64_t yrow = GATHER ? y_row_of(a, t.start) : t.start;
#pragma unroll
    for (int r = 0; r < RPW; r++) {
        const float v = wave_sum(acc[r]);
        if (lane == 0 && n0 + r < a.N) a.y[yrow * a.N + n0 + r] = f32_to_bf16(v);
    }
}

template <int BITS, int RPW, int S>
static bool launch_wv(const ValuShape& v, const QmvArgs& a, dim3 grid, size_t lds, hipStream_t st) {
    const bool g = a.tiles != nullptr;
    // 16 waves (affine): one row per wave, eight slots per batch (long rows)
    constexpr bool W16 = RPW == 1 && S == 8;
    if (a.mx) {                                   // dense only
        if (g) return false;
        if (v.WV == 4) qmv_valu_kernel<BITS, RPW, S, 4, false, true><<<grid, 256, lds, st>>>(a);
        else if (v.WV == 8) qmv_valu_kernel<BITS, RPW, S, 8, false, true><<<grid, 512, lds, st>>>(a);
        else return false;
        return true;
    }
    if (v.WV == 4) {
        if (g) qmv_valu_kernel<BITS, RPW, S, 4, true, false><<<grid, 256, lds, st>>>(a);
        else qmv_valu_kernel<BITS, RPW, S, 4, false, false><<<grid, 256, lds, st>>>(a);
    } else if (v.WV == 8) {
        if (g) qmv_valu_kernel<BITS, RPW, S, 8, true, false><<<grid, 512, lds, st>>>(a);
        else qmv_valu_kernel<BITS, RPW, S, 8, false, false><<<grid, 512, lds, st>>>(a);
    } else if constexpr (W16) {
        if (v.WV != 16) return false;
        if (g) qmv_valu_kernel<BITS, RPW, S, 16, true, false><<<grid, 1024, lds, st>>>(a);
        else qmv_valu_kernel<BITS, RPW, S, 16, false, false><<<grid, 1024, lds, st>>>(a);
    } else {
        return false;
    }
    return true;
}

template <int BITS>
static bool launch_shape(const ValuShape& v, const QmvArgs& a, dim3 grid, size_t lds, hipStream_t st) {
    if (v.RPW == 1) {
        if (v.S == 1) return launch_wv<BITS, 1, 1>(v, a, grid, lds, st);
        if (v.S == 2) return launch_wv<BITS, 1, 2>(v, a, grid, lds, st);
        if (v.S == 4) return launch_wv<BITS, 1, 4>(v, a, grid, lds, st);
        if (v.S == 8) return launch_wv<BITS, 1, 8>(v, a, grid, lds, st);
    }
    if (v.RPW == 2) {
        if (v.S == 1) return launch_wv<BITS, 2, 1>(v, a, grid, lds, st);
        if (v.S == 2) return launch_wv<BITS, 2, 2>(v, a, grid, lds, st);
        if (v.S == 4) return launch_wv<BITS, 2, 4>(v, a, grid, lds, st);
    }
    if (v.RPW == 4) {
        if (v.S == 1) return launch_wv<BITS, 4, 1>(v, a, grid, lds, st);
        if (v.S == 2) return launch_wv<BITS, 4, 2>(v, a, grid, lds, st);
    }
    return false;
}

bool launch_qmv_valu(int bits, const ValuShape& v, const QmvArgs& a, dim3 grid, size_t lds,
                     hipStream_t st) {
    if (bits == 4) return launch_shape<4>(v, a, grid, lds, st);
    if (bits == 8) return launch_shape<8>(v, a, grid, lds, st);
    return false;
}

}  // namespace kmi
