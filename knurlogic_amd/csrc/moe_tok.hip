// SwitchGLU for decode-size token counts on gfx950, token-major: every
// (token, slot) pair reads its own expert, so no sort is needed, and at
// T = 1 each routed expert's bytes are read exactly once (at a few tokens a
// shared expert is read by a few workgroups that run together; the repeats
// come from the L2 / Infinity Cache).
//
//   moe_glu_tok:  act[p, n] = round(round(silu(round(x_t . Wg[e_p, n]))) *
//                 round(x_t . Wu[e_p, n])) -- the gate and up rows of one
//                 column in the same wave, the _SwiGLU epilogue in registers
//                 (qwen3_5.py:108-112 over switch_layers.py:172-193).
//   moe_down_tok: y[t, s, n] = round(act[t*k+s] . Wd[e_ts, n]) for all k
//                 slots of token t in one workgroup (lanes spread over
//                 (slot, chunk) items, every slot's loads in flight
//                 together), then either the weighted combine
//                 round(sum_s round(y * score)) (qwen3_5.py:181-182) or
//                 y itself.
// Both stream packed 16-byte chunks with raw buffer loads and decode them as
// the decode GEMV does (qmv_common.hpp): codes as fp16 "1024 + q" against x
// staged as fp16 with a power-of-two scale per chunk, v_dot2_f32_f16, and per
// chunk s * sum(q x) + b * sum(x) in fp32.
#include "qmv_common.hpp"
#include "moe_tok.hpp"
#include "route.hpp"

#include "../../include/knurlogic_amd.h"

namespace kmi {


__device__ __forceinline__ float bf16r(float v) { return bf16_to_f32(f32_to_bf16(v)); }

__device__ __forceinline__ float f64_to_f32_kept(double v) {
    float f = (float)v;
    asm volatile("" : "+v"(f));   // keep the float32 rounding (no fused f64 -> bf16 rounding)
    return f;
}

// ---- gate + up + SwiGLU -----------------------------------------------------
// grid (ceil(N / (WV*RPW)), T*k); K = H.  The decode GEMV's streaming scheme
// (qmv_valu.hip) over two row sets: x (one token row) staged as fp16 with a
// power-of-two scale per chunk, codes decoded as fp16 "1024 + q", every load
// of a wave issued up front with the wave-uniform part of its offset in the
// scalar operand, each chunk-row's scale and bias loaded per lane ahead of
// its weights.  S 16-byte chunk slots per lane per row (all of K).
// ROUTE: the pair's expert comes from routing its token's logits in the
// workgroup (route.hpp, the router kernel's arithmetic), after the x loads
// are issued; workgroup 0 of each pair writes the expert and its score.
// MX: OCP microscaled codes (mxfp4 at BITS 4, mxfp8 at 8) with one E8M0
// byte scale per 32 inputs and no biases, in place of the affine decode.
template <int BITS, int RPW, int S, int WV, bool ROUTE, bool MX>
__global__ __launch_bounds__(64 * WV) void moe_glu_tok(MoeTokArgs a) {
    constexpr int NT = 64 * WV, CK = 128 / BITS, XV = CK / 8, ROWS = WV * RPW;
    constexpr uint32_t SB = MX ? 1 : 2;              // bytes per scale
    constexpr uint32_t NONE = QV_NONE;
    extern __shared__ __align__(16) unsigned char smem[];
    const int C = (int)(a.K / CK);
    const int wpr = (int)(a.K / (32 / BITS));
    const int gpr = (int)(a.K >> a.gs_shift);
    const int P = (int)(a.K >> 3);                   // x pieces of the row
    u32x4* xs = (u32x4*)smem;                                  // [XV][C] fp16 pieces
    float4* xm = (float4*)(smem + (size_t)XV * C * 16);        // [C] {scale, correction, sum}

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int p = blockIdx.y;
    const int64_t t = p / a.k;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x + t * a.K, a.K * 2);
    auto xvo = [&](int q) -> uint32_t { return q < P ? (uint32_t)q * 16u : NONE; };
    // x pieces first: independent of the expert, in flight during the routing
    const u32x4 xr0 = __builtin_amdgcn_raw_buffer_load_b128(rx, (int)xvo(tid), 0, 0);
    const u32x4 xr1 = __builtin_amdgcn_raw_buffer_load_b128(rx, (int)xvo(tid + NT), 0, 0);
    int e;
    if constexpr (ROUTE) {
        static_assert(NT == ROUTE_THREADS, "the in-kernel router takes 256 threads");
        __shared__ RouteLds rsm;
        route_token<TBF16, 1>(a.logits + t * a.E, (int)a.E, a.k, rsm);      // E <= 256
        const int s = p - (int)t * a.k;
        e = __builtin_amdgcn_readfirstlane(rsm.sel_e[s]);
        if (blockIdx.x == 0 && tid == 0) {
            a.inds_out[p] = e;
            a.scores_out[p] = f32_to_bf16(rsm.sel_p[s]);
        }
    } else {
        e = a.inds[p];
    }
    const int n0 = (int)blockIdx.x * ROWS + wave * RPW;
    const bool ok_e = e >= 0 && e < a.E;
    const int64_t eoff = (int64_t)(ok_e ? e : 0) * a.erows;
    const int64_t wbytes = ok_e ? a.N * (int64_t)wpr * 4 : 0, sbytes = ok_e ? a.N * (int64_t)gpr * SB : 0;
    const __amdgpu_buffer_rsrc_t rw0 = make_rsrc(a.w0 + eoff * wpr, wbytes);
    const __amdgpu_buffer_rsrc_t rw1 = make_rsrc(a.w1 + eoff * wpr, wbytes);
    const __amdgpu_buffer_rsrc_t rs0 = make_rsrc((const char*)a.s0 + eoff * gpr * SB, sbytes);
    const __amdgpu_buffer_rsrc_t rb0 = make_rsrc((const char*)a.b0 + eoff * gpr * SB, MX ? 0 : sbytes);
    const __amdgpu_buffer_rsrc_t rs1 = make_rsrc((const char*)a.s1 + eoff * gpr * SB, sbytes);
    const __amdgpu_buffer_rsrc_t rb1 = make_rsrc((const char*)a.b1 + eoff * gpr * SB, MX ? 0 : sbytes);

    // (0) x pieces beyond two per thread (long rows), before any weight load
    if (P > 2 * NT) {
        for (int q = tid + 2 * NT; q - (tid & 3) < P; q += NT)
            stage_x16<BITS, MX>(q, __builtin_amdgcn_raw_buffer_load_b128(rx, (int)xvo(q), 0, 0), P, C, xs, xm);
    }
    // (1) scales/biases and weights of both sets
    const int full = C >> 6;
    const bool in_tail = lane < (C & 63);
    const uint32_t vw = (uint32_t)lane * 16u;
    const uint32_t vg = (uint32_t)((lane * CK) >> a.gs_shift) * SB;
    const uint32_t vwt = in_tail ? vw : NONE, vgt = in_tail ? vg : NONE;
    uint32_t wrow[RPW], srow[RPW];
#pragma unroll
    for (int r = 0; r < RPW; r++) {           // rows past N re-read row N-1 (never stored)
        const uint32_t row = (uint32_t)(n0 + r < a.N ? n0 + r : a.N - 1);
        wrow[r] = row * (uint32_t)wpr * 4u;
        srow[r] = row * (uint32_t)gpr * SB;
    }
    u32x4 W0[S][RPW], W1[S][RPW];
    uint32_t S0[S][RPW], B0[S][RPW], S1[S][RPW], B1[S][RPW];
#pragma unroll
    for (int u = 0; u < S; u++) {
        const uint32_t vo = u < full ? vg : u == full ? vgt : NONE;
        const uint32_t so = (uint32_t)(((64 * u * CK) >> a.gs_shift) * SB);
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            if constexpr (MX) {
                S0[u][r] = __builtin_amdgcn_raw_buffer_load_b8(rs0, (int)vo, (int)(srow[r] + so), 0);
                S1[u][r] = __builtin_amdgcn_raw_buffer_load_b8(rs1, (int)vo, (int)(srow[r] + so), 0);
                B0[u][r] = B1[u][r] = 0u;
            } else {
                S0[u][r] = __builtin_amdgcn_raw_buffer_load_b16(rs0, (int)vo, (int)(srow[r] + so), 0);
                B0[u][r] = __builtin_amdgcn_raw_buffer_load_b16(rb0, (int)vo, (int)(srow[r] + so), 0);
                S1[u][r] = __builtin_amdgcn_raw_buffer_load_b16(rs1, (int)vo, (int)(srow[r] + so), 0);
                B1[u][r] = __builtin_amdgcn_raw_buffer_load_b16(rb1, (int)vo, (int)(srow[r] + so), 0);
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < S; u++) {
        const uint32_t vo = u < full ? vw : u == full ? vwt : NONE;
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            W0[u][r] = __builtin_amdgcn_raw_buffer_load_b128(rw0, (int)vo, (int)(wrow[r] + (uint32_t)u * 1024u), AUX_NT);
            W1[u][r] = __builtin_amdgcn_raw_buffer_load_b128(rw1, (int)vo, (int)(wrow[r] + (uint32_t)u * 1024u), AUX_NT);
        }
    }

    // (2) x -> LDS
    stage_x16<BITS, MX>(tid, xr0, P, C, xs, xm);
    if (P > NT) stage_x16<BITS, MX>(tid + NT, xr1, P, C, xs, xm);
    lds_barrier();

    const Magic16 mk = magic16();
    float acc0[RPW], acc1[RPW];
#pragma unroll
    for (int r = 0; r < RPW; r++) acc0[r] = acc1[r] = 0.f;
#pragma unroll
    for (int u = 0; u < S; u++) {
        if (64 * u >= C) break;                       // wave-uniform
        const int c = lane + 64 * u;
        const bool cok = c < C;
        const int cc = cok ? c : 0;
        u32x4 xv[XV];
#pragma unroll
        for (int v = 0; v < XV; v++) xv[v] = xs[v * C + cc];
        const float4 m = xm[cc];
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            float g0, g1;
            if constexpr (MX) {
                g0 = __builtin_fmaf(mx_scale(S0[u][r]), chunk_mx<BITS>(W0[u][r], xv, m), acc0[r]);
                g1 = __builtin_fmaf(mx_scale(S1[u][r]), chunk_mx<BITS>(W1[u][r], xv, m), acc1[r]);
            } else {
                const float q0 = chunk_qx<BITS>(W0[u][r], xv, m, mk);
                const float q1 = chunk_qx<BITS>(W1[u][r], xv, m, mk);
                g0 = __builtin_fmaf(__uint_as_float(S0[u][r] << 16), q0,
                                    __builtin_fmaf(__uint_as_float(B0[u][r] << 16), m.z, acc0[r]));
                g1 = __builtin_fmaf(__uint_as_float(S1[u][r] << 16), q1,
                                    __builtin_fmaf(__uint_as_float(B1[u][r] << 16), m.z, acc1[r]));
            }
            acc0[r] = cok ? g0 : acc0[r];
            acc1[r] = cok ? g1 : acc1[r];
        }
    }
#pragma unroll
    for (int r = 0; r < RPW; r++) {
        const float g = bf16r(wave_sum(acc0[r]));
        const float u = bf16r(wave_sum(acc1[r]));
        if (lane == 0 && n0 + r < a.N) {
            const float s = silu_bf16r(g);
            a.out[(int64_t)p * a.N + n0 + r] = ok_e ? f32_to_bf16(s * u) : (uint16_t)0;
        }
    }
}

// ---- down projection + combine ----------------------------------------------
// grid (ceil(N / (WV*RPW)), T); K = I.  All k slots of token t in one
// workgroup: their act rows staged once (fp16, as in the gate/up kernel),
// lanes spread over (slot, chunk) items (U per lane) so short rows keep every
// lane busy and all k experts' loads are in flight together.  The item's
// expert differs per lane, so the expert part of an offset is per lane and
// the row part (wave-uniform) is in the scalar operand.
template <int BITS, int KMAX, int U, int RPW, int WV, bool MX>
__global__ __launch_bounds__(64 * WV) void moe_down_tok(MoeTokArgs a) {
    constexpr int NT = 64 * WV, CK = 128 / BITS, XV = CK / 8;
    constexpr uint32_t SB = MX ? 1 : 2;              // bytes per scale
    constexpr int XREG = 4;                          // x pieces per thread held in registers
    constexpr uint32_t NONE = QV_NONE;
    extern __shared__ __align__(16) unsigned char smem[];
    const int C = (int)(a.K / CK);
    const int k = a.k;
    const int wpr = (int)(a.K / (32 / BITS));
    const int gpr = (int)(a.K >> a.gs_shift);
    const int P = (int)(a.K >> 3);                   // x pieces per slot row
    const size_t slot_bytes = (size_t)XV * C * 16 + (size_t)C * 16;
    auto xs_of = [&](int s) { return (u32x4*)(smem + s * slot_bytes); };
    auto xm_of = [&](int s) { return (float4*)(smem + s * slot_bytes + (size_t)XV * C * 16); };

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t t = blockIdx.y;
    const int n0 = (int)blockIdx.x * (WV * RPW) + wave * RPW;
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.w0, a.E * a.N * (int64_t)wpr * 4);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.s0, a.E * a.N * (int64_t)gpr * SB);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(a.b0, MX ? 0 : a.E * a.N * (int64_t)gpr * 2);
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x + t * k * a.K, (int64_t)k * a.K * 2);

    // x pieces q = tid + NT j of the k slot rows: slot q / P, piece q % P
    // (P is a multiple of 4, so a chunk's pieces stay in one lane quad)
    auto xq = [&](int q, int& sl, int& pc) {
        sl = q / P;
        pc = q - sl * P;
        if (sl >= k) { sl = 0; pc = P; }              // past the slots: stage nothing
    };
    for (int q = tid + XREG * NT; q - (tid & 3) < k * P; q += NT) {
        int sl, pc;
        xq(q, sl, pc);
        const uint32_t o = pc < P ? (uint32_t)((sl * a.K + pc * 8) * 2) : NONE;
        stage_x16<BITS, MX>(pc, __builtin_amdgcn_raw_buffer_load_b128(rx, (int)o, 0, 0), P, C, xs_of(sl), xm_of(sl));
    }
    u32x4 xr[XREG];
#pragma unroll
    for (int j = 0; j < XREG; j++) {
        int sl, pc;
        xq(tid + j * NT, sl, pc);
        const uint32_t o = pc < P ? (uint32_t)((sl * a.K + pc * 8) * 2) : NONE;
        xr[j] = __builtin_amdgcn_raw_buffer_load_b128(rx, (int)o, 0, 0);
    }

    // this lane's items i = lane + 64 u: slot i / C, chunk i % C; per-lane
    // expert offsets, rows in the scalar offset
    // the k experts by scalar loads (the sort-free caller wrote inds before
    // this launch; uniform reads of a constant address-space view are scalar
    // and do not wait behind the vector loads), then each lane's by select
    typedef const __attribute__((address_space(4))) int32_t* cint_p;
    const cint_p ic = (cint_p)(a.inds + t * k);
    int ex[KMAX];
#pragma unroll
    for (int s = 0; s < KMAX; s++) ex[s] = s < k ? ic[s] : -1;
    int isl[U];
    uint32_t vwo[U], vso[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
        const int i = lane + 64 * u;
        const int sidx = i / C, c = i - sidx * C;
        int e = -1;
#pragma unroll
        for (int s = 0; s < KMAX; s++) e = sidx == s ? ex[s] : e;
        const bool ok = sidx < k && e >= 0 && e < a.E;
        isl[u] = sidx < k ? sidx : -1;
        vwo[u] = ok ? (uint32_t)((((int64_t)e * a.N) * wpr + (int64_t)c * 4) * 4) : NONE;
        vso[u] = ok ? (uint32_t)((((int64_t)e * a.N) * gpr + ((c * CK) >> a.gs_shift)) * SB) : NONE;
    }
    uint32_t wrow[RPW], srow[RPW];
#pragma unroll
    for (int r = 0; r < RPW; r++) {           // rows past N re-read row N-1 (never stored)
        const uint32_t row = (uint32_t)(n0 + r < a.N ? n0 + r : a.N - 1);
        wrow[r] = row * (uint32_t)wpr * 4u;
        srow[r] = row * (uint32_t)gpr * SB;
    }
    u32x4 W[U][RPW];
    uint32_t SC[U][RPW], BI[U][RPW];
#pragma unroll
    for (int u = 0; u < U; u++)
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            if constexpr (MX) {
                SC[u][r] = __builtin_amdgcn_raw_buffer_load_b8(rs, (int)vso[u], (int)srow[r], 0);
                BI[u][r] = 0u;
            } else {
                SC[u][r] = __builtin_amdgcn_raw_buffer_load_b16(rs, (int)vso[u], (int)srow[r], 0);
                BI[u][r] = __builtin_amdgcn_raw_buffer_load_b16(rb, (int)vso[u], (int)srow[r], 0);
            }
        }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < U; u++)
#pragma unroll
        for (int r = 0; r < RPW; r++)
            W[u][r] = __builtin_amdgcn_raw_buffer_load_b128(rw, (int)vwo[u], (int)wrow[r], AUX_NT);

    // x -> LDS
#pragma unroll
    for (int j = 0; j < XREG; j++) {
        if (j * NT >= k * P) break;                   // wave-uniform
        int sl, pc;
        xq(tid + j * NT, sl, pc);
        stage_x16<BITS, MX>(pc, xr[j], P, C, xs_of(sl), xm_of(sl));
    }
    lds_barrier();

    const Magic16 mk = magic16();
    float acc[U][RPW];
#pragma unroll
    for (int u = 0; u < U; u++) {
        const int i = lane + 64 * u;
        const int sl = isl[u] < 0 ? 0 : isl[u];
        const int c = isl[u] < 0 ? 0 : i - sl * C;
        const u32x4* xsp = xs_of(sl);
        u32x4 xv[XV];
#pragma unroll
        for (int v = 0; v < XV; v++) xv[v] = xsp[v * C + c];
        const float4 m = xm_of(sl)[c];
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            float v;
            if constexpr (MX) {
                v = mx_scale(SC[u][r]) * chunk_mx<BITS>(W[u][r], xv, m);
            } else {
                const float q = chunk_qx<BITS>(W[u][r], xv, m, mk);
                v = __builtin_fmaf(__uint_as_float(SC[u][r] << 16), q, __uint_as_float(BI[u][r] << 16) * m.z);
            }
            acc[u][r] = isl[u] < 0 ? 0.f : v;
        }
    }
    // per slot: sum this lane's items of the slot, then over the wave
#pragma unroll
    for (int r = 0; r < RPW; r++) {
        double comb = 0.0;
#pragma unroll
        for (int s = 0; s < KMAX; s++) {
            if (s >= k) break;
            float v = 0.f;
#pragma unroll
            for (int u = 0; u < U; u++) v += isl[u] == s ? acc[u][r] : 0.f;
            const float y = bf16r(wave_sum(v));
            if (a.scores) {
                comb += (double)bf16r(y * bf16_to_f32(a.scores[t * k + s]));
            } else if (lane == 0 && n0 + r < a.N) {
                a.out[(t * k + s) * a.N + n0 + r] = f32_to_bf16(y);
            }
        }
        if (a.scores && lane == 0 && n0 + r < a.N)
            a.out[t * a.N + n0 + r] = f32_to_bf16(f64_to_f32_kept(comb));
    }
}

constexpr int TOK_WV = 4;



}  // namespace kmi

using namespace kmi;

// Launchers shared with the SwitchGLU entry point (moe_glu.hip).
namespace kmi {

int launch_moe_glu_tok(const MoeTokArgs& a, int bits, hipStream_t st) {
    const int64_t CK = 128 / bits, C = a.K / CK;
    const int64_t slots = ceil_div(C, 64);
    const int S = slots <= 1 ? 1 : slots <= 2 ? 2 : slots <= 4 ? 4 : 0;
    if (S == 0) {
        set_error("switch_glu: no gate/up kernel for %lld chunks per row", (long long)C);
        return EINVAL_ARG;
    }
    // rows per wave: as many as keep >= 2048 waves (2 per SIMD) in the grid,
    // within 8 chunk-rows of loads per set
    const int64_t pairs = a.T * a.k;
    int rpw = 1;
    if (S <= 4 && a.N * pairs / 2 >= 2048) rpw = 2;
    if (S <= 2 && a.N * pairs / 4 >= 2048) rpw = 4;
    const dim3 grid((unsigned)ceil_div(a.N, TOK_WV * rpw), (unsigned)pairs);
    const size_t lds = (size_t)a.K * 2 + (size_t)C * 16;
#define KMI_GLU_M(R, SS, RT, M)                                                                 \
    if (bits == 4) moe_glu_tok<4, R, SS, TOK_WV, RT, M><<<grid, 64 * TOK_WV, lds, st>>>(a);     \
    else moe_glu_tok<8, R, SS, TOK_WV, RT, M><<<grid, 64 * TOK_WV, lds, st>>>(a);
#define KMI_GLU_R(R, SS, RT)                                                                    \
    if (a.mx) { KMI_GLU_M(R, SS, RT, true) } else { KMI_GLU_M(R, SS, RT, false) }
#define KMI_GLU(R, SS)                                                                  \
    if (rpw == R && S == SS) {                                                          \
        if (a.logits) { KMI_GLU_R(R, SS, true) } else { KMI_GLU_R(R, SS, false) }       \
        return OK;                                                                      \
    }
    KMI_GLU(1, 1) KMI_GLU(1, 2) KMI_GLU(1, 4) KMI_GLU(2, 1) KMI_GLU(2, 2) KMI_GLU(2, 4) KMI_GLU(4, 1) KMI_GLU(4, 2)
#undef KMI_GLU
#undef KMI_GLU_R
#undef KMI_GLU_M
    set_error("switch_glu: no gate/up kernel for %lld chunks per row", (long long)C);
    return EINVAL_ARG;
}

int launch_moe_down_tok(const MoeTokArgs& a, int bits, hipStream_t st) {
    const int64_t CK = 128 / bits, C = a.K / CK;
    const int U = (int)ceil_div((int64_t)a.k * C, 64);
    // two rows per wave while the grid keeps >= 2048 waves
    const int rpw = U <= 4 && a.N * a.T / 2 >= 2048 ? 2 : 1;
    const dim3 grid((unsigned)ceil_div(a.N, TOK_WV * rpw), (unsigned)a.T);
    const size_t lds = (size_t)a.k * ((size_t)a.K * 2 + (size_t)C * 16);
    if (a.E * a.N * (a.K * bits / 8) >= (1LL << 31)) {
        set_error("switch_glu: down experts past 2 GiB");
        return EINVAL_ARG;
    }
#define KMI_DOWN_M(KM, UU, R, M)                                                                   \
    if (bits == 4) moe_down_tok<4, KM, UU, R, TOK_WV, M><<<grid, 64 * TOK_WV, lds, st>>>(a);       \
    else moe_down_tok<8, KM, UU, R, TOK_WV, M><<<grid, 64 * TOK_WV, lds, st>>>(a);
#define KMI_DOWN(KM, UU, R)                                                                        \
    if (a.k <= KM && U == UU && rpw == R) {                                                        \
        if (a.mx) { KMI_DOWN_M(KM, UU, R, true) } else { KMI_DOWN_M(KM, UU, R, false) }            \
        return OK;                                                                                 \
    }
    KMI_DOWN(8, 1, 1) KMI_DOWN(8, 2, 1) KMI_DOWN(8, 3, 1) KMI_DOWN(8, 4, 1) KMI_DOWN(8, 6, 1) KMI_DOWN(8, 8, 1)
    KMI_DOWN(8, 1, 2) KMI_DOWN(8, 2, 2) KMI_DOWN(8, 3, 2) KMI_DOWN(8, 4, 2)
#undef KMI_DOWN
#undef KMI_DOWN_M
    set_error("switch_glu: no down kernel for k=%d, %lld chunks per row", a.k, (long long)C);
    return EINVAL_ARG;
}

}  // namespace kmi
