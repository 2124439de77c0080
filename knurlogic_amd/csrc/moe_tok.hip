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
// Both stream packed 16-byte chunks with raw buffer loads and use the
// factorized dequant of the decode GEMV: per group, s * sum(q x) +
// (b - 128 s or b) * sum(x), the 4-bit nibbles unpacked to bf16 "128 + q"
// and dotted with v_dot2_f32_bf16.
#include "qmv_common.hpp"
#include "moe_tok.hpp"
#include "../../include/knurlogic_amd.h"

namespace kmi {


__device__ __forceinline__ float bf16r(float v) { return bf16_to_f32(f32_to_bf16(v)); }

__device__ __forceinline__ float f64_to_f32_kept(double v) {
    float f = (float)v;
    asm volatile("" : "+v"(f));   // keep the float32 rounding (no fused f64 -> bf16 rounding)
    return f;
}

// Stage one x row (K bf16) into LDS as [piece][chunk] 16-byte slots with the
// 4-bit unpack permutation, and its per-chunk sums.
template <int BITS>
__device__ __forceinline__ void stage_row(uint16_t* xs, float* xc, const u32x4* v, int c, int C) {
    constexpr int XV = (128 / BITS) / 8;
    float sum = 0.f;
#pragma unroll
    for (int v8 = 0; v8 < XV; v8++) *(u32x4*)(xs + (v8 * C + c) * 8) = permute8<BITS>(v[v8], sum);
    xc[c] = sum;
}

// Partial dot product of one 16-byte weight chunk with the staged x chunk.
template <int BITS>
__device__ __forceinline__ float chunk_dot(const u32x4& W, const u32x4* xv) {
    float A0 = 0.f, A1 = 0.f;
    if constexpr (BITS == 4) {
#pragma unroll
        for (int wd = 0; wd < 4; wd++) {
            const u32x4 q = nibbles_to_bf16_magic(W[wd]);
            A0 = dot2(xv[wd][0], q[0], A0);
            A1 = dot2(xv[wd][1], q[1], A1);
            A0 = dot2(xv[wd][2], q[2], A0);
            A1 = dot2(xv[wd][3], q[3], A1);
        }
    } else {
#pragma unroll
        for (int wd = 0; wd < 4; wd++) {
            A0 = dot2(xv[wd >> 1][(wd & 1) * 2], bytes_to_bf16x2(W[wd], 0), A0);
            A1 = dot2(xv[wd >> 1][(wd & 1) * 2 + 1], bytes_to_bf16x2(W[wd], 2), A1);
        }
    }
    return A0 + A1;
}

// acc += s * dot + b' * xsum  (b' = b - 128 s for the 4-bit "128 + q" unpack)
template <int BITS>
__device__ __forceinline__ float apply_group(float acc, float dot, float xsum, uint32_t sb) {
    const float sc = bf16_to_f32((uint16_t)(sb & 0xffffu));
    const float bi = bf16_to_f32((uint16_t)(sb >> 16));
    const float bb = (BITS == 4) ? __builtin_fmaf(-128.f, sc, bi) : bi;
    return __builtin_fmaf(sc, dot, __builtin_fmaf(bb, xsum, acc));
}

// ---- gate + up + SwiGLU -----------------------------------------------------
// grid (ceil(N / (WV*RPW)), T*k); K = H.  S 16-byte chunks per lane per row.
template <int BITS, int RPW, int S, int WV>
__global__ __launch_bounds__(64 * WV) void moe_glu_tok(MoeTokArgs a) {
    constexpr int CK = 128 / BITS, XV = CK / 8, ROWS = WV * RPW;
    extern __shared__ __align__(16) unsigned char smem[];
    const int C = (int)(a.K / CK);
    const int wpr = (int)(a.K / (32 / BITS));
    const int gpr = (int)(a.K >> a.gs_shift);
    uint16_t* xs = (uint16_t*)smem;                                        // [XV][C] 16-byte slots
    float* xc = (float*)(smem + (size_t)XV * C * 16);                      // [C]
    uint32_t* sbl = (uint32_t*)(xc + C);                                   // [2][ROWS][gpr]

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int p = blockIdx.y;
    const int64_t t = p / a.k;
    const int e = a.inds[p];
    const int nwg = (int)blockIdx.x * ROWS, n0 = nwg + wave * RPW;
    const bool ok_e = e >= 0 && e < a.E;
    const int64_t eoff = (int64_t)(ok_e ? e : 0) * a.erows;
    const int64_t wbytes = ok_e ? a.N * (int64_t)wpr * 4 : 0, sbytes = ok_e ? a.N * (int64_t)gpr * 2 : 0;
    const __amdgpu_buffer_rsrc_t rw0 = make_rsrc(a.w0 + eoff * wpr, wbytes);
    const __amdgpu_buffer_rsrc_t rw1 = make_rsrc(a.w1 + eoff * wpr, wbytes);
    const __amdgpu_buffer_rsrc_t rs0 = make_rsrc(a.s0 + eoff * gpr, sbytes);
    const __amdgpu_buffer_rsrc_t rb0 = make_rsrc(a.b0 + eoff * gpr, sbytes);
    const __amdgpu_buffer_rsrc_t rs1 = make_rsrc(a.s1 + eoff * gpr, sbytes);
    const __amdgpu_buffer_rsrc_t rb1 = make_rsrc(a.b1 + eoff * gpr, sbytes);
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x + t * a.K, a.K * 2);

    // x chunks first (one per thread for C <= 64*WV), then every weight load
    const int NT = 64 * WV;
    u32x4 xr[XV];
#pragma unroll
    for (int v8 = 0; v8 < XV; v8++)
        xr[v8] = __builtin_amdgcn_raw_buffer_load_b128(rx, (int)((tid * CK + v8 * 8) * 2), 0, 0);
    u32x4 W0[S][RPW], W1[S][RPW];
#pragma unroll
    for (int u = 0; u < S; u++) {
        const int c = lane + 64 * u;
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            const int off = (int)(((uint32_t)(n0 + r) * (uint32_t)wpr + (uint32_t)c * 4u) * 4u);
            W0[u][r] = __builtin_amdgcn_raw_buffer_load_b128(rw0, off, 0, AUX_NT);
            W1[u][r] = __builtin_amdgcn_raw_buffer_load_b128(rw1, off, 0, AUX_NT);
        }
    }
    // scales / biases of both row sets -> LDS (rows past N read 0)
    for (int idx = tid; idx < ROWS * gpr; idx += NT) {
        const int rl = idx / gpr, g = idx - rl * gpr;
        const int off = (int)(((uint32_t)(nwg + rl) * (uint32_t)gpr + (uint32_t)g) * 2u);
        sbl[idx] = __builtin_amdgcn_raw_buffer_load_b16(rs0, off, 0, 0) |
                   ((uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rb0, off, 0, 0) << 16);
        sbl[ROWS * gpr + idx] = __builtin_amdgcn_raw_buffer_load_b16(rs1, off, 0, 0) |
                                ((uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rb1, off, 0, 0) << 16);
    }
    if (tid < C) stage_row<BITS>(xs, xc, xr, tid, C);
    for (int c = tid + NT; c < C; c += NT) {           // wide rows: the rest of x
        u32x4 v[XV];
#pragma unroll
        for (int v8 = 0; v8 < XV; v8++)
            v[v8] = __builtin_amdgcn_raw_buffer_load_b128(rx, (int)((c * CK + v8 * 8) * 2), 0, 0);
        stage_row<BITS>(xs, xc, v, c, C);
    }
    lds_barrier();

    float acc0[RPW], acc1[RPW];
#pragma unroll
    for (int r = 0; r < RPW; r++) acc0[r] = acc1[r] = 0.f;
#pragma unroll
    for (int u = 0; u < S; u++) {
        const int c = lane + 64 * u;
        if (c >= C) continue;
        const int g = (c * CK) >> a.gs_shift;
        u32x4 xv[XV];
#pragma unroll
        for (int v8 = 0; v8 < XV; v8++) xv[v8] = *(const u32x4*)(xs + (v8 * C + c) * 8);
        const float X = xc[c];
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            const int rl = wave * RPW + r;
            acc0[r] = apply_group<BITS>(acc0[r], chunk_dot<BITS>(W0[u][r], xv), X, sbl[rl * gpr + g]);
            acc1[r] = apply_group<BITS>(acc1[r], chunk_dot<BITS>(W1[u][r], xv), X,
                                        sbl[(ROWS + rl) * gpr + g]);
        }
    }
#pragma unroll
    for (int r = 0; r < RPW; r++) {
        const float g = bf16r(wave_sum(acc0[r]));
        const float u = bf16r(wave_sum(acc1[r]));
        if (lane == 0 && n0 + r < a.N) {
            const double gd = (double)g;
            const float s = bf16r(f64_to_f32_kept(gd / (1.0 + exp(-gd))));
            a.out[(int64_t)p * a.N + n0 + r] = ok_e ? f32_to_bf16(s * u) : (uint16_t)0;
        }
    }
}

// ---- down projection + combine ----------------------------------------------
// grid (ceil(N / (WV*RPW)), T); K = I.  Lane items (slot, chunk): U per lane.
template <int BITS, int KMAX, int U, int RPW, int WV>
__global__ __launch_bounds__(64 * WV) void moe_down_tok(MoeTokArgs a) {
    constexpr int CK = 128 / BITS, XV = CK / 8, ROWS = WV * RPW;
    extern __shared__ __align__(16) unsigned char smem[];
    const int C = (int)(a.K / CK);
    const int k = a.k;
    const int wpr = (int)(a.K / (32 / BITS));
    const int gpr = (int)(a.K >> a.gs_shift);
    uint16_t* xs = (uint16_t*)smem;                                        // [k][XV][C] slots
    float* xc = (float*)(smem + (size_t)k * XV * C * 16);                  // [k][C]
    uint32_t* sbl = (uint32_t*)(xc + k * C);                               // [k][ROWS][gpr]

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int NT = 64 * WV;
    const int64_t t = blockIdx.y;
    const int nwg = (int)blockIdx.x * ROWS, n0 = nwg + wave * RPW;
    const int64_t wexp = a.N * (int64_t)wpr;                                // words per expert
    const int64_t gexp = a.N * (int64_t)gpr;
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.w0, a.E * wexp * 4);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.s0, a.E * gexp * 2);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(a.b0, a.E * gexp * 2);
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x + t * k * a.K, (int64_t)k * a.K * 2);

    int ex[KMAX];                      // experts of the k slots (an invalid one reads zeros)
#pragma unroll
    for (int s = 0; s < KMAX; s++) {
        const int e = s < k ? a.inds[t * k + s] : -1;
        ex[s] = (e >= 0 && e < a.E) ? e : -1;
    }
    auto ebase = [&](int s) -> uint32_t {  // expert word base, or past the buffer
        return ex[s] >= 0 ? (uint32_t)(ex[s] * wexp) : 0x20000000u;
    };

    // this lane's items: i = lane + 64 u -> slot i / C, chunk i % C
    u32x4 W[U][RPW];
    int sl[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
        const int i = lane + 64 * u;
        const int s = i / C, c = i - (i / C) * C;
        sl[u] = i < k * C ? s : -1;
        uint32_t eb = 0x20000000u;
#pragma unroll
        for (int q = 0; q < KMAX; q++)
            if (q == s) eb = ebase(q);
        if (sl[u] < 0) eb = 0x20000000u;
#pragma unroll
        for (int r = 0; r < RPW; r++)
            W[u][r] = __builtin_amdgcn_raw_buffer_load_b128(
                rw, (int)((eb + (uint32_t)(n0 + r) * (uint32_t)wpr + (uint32_t)c * 4u) * 4u), 0, AUX_NT);
    }
    // x rows of the k slots, scales / biases -> LDS
    for (int idx = tid; idx < k * C; idx += NT) {
        const int s = idx / C, c = idx - s * C;
        u32x4 v[XV];
#pragma unroll
        for (int v8 = 0; v8 < XV; v8++)
            v[v8] = __builtin_amdgcn_raw_buffer_load_b128(rx, (int)(((int64_t)s * a.K + c * CK + v8 * 8) * 2), 0, 0);
        stage_row<BITS>(xs + (size_t)s * XV * C * 8, xc + s * C, v, c, C);
    }
    for (int idx = tid; idx < k * ROWS * gpr; idx += NT) {
        const int s = idx / (ROWS * gpr), rem = idx - s * ROWS * gpr;
        const int rl = rem / gpr, g = rem - rl * gpr;
        int e = -1;
#pragma unroll
        for (int q = 0; q < KMAX; q++)
            if (q == s) e = ex[q];
        const uint32_t off = e >= 0 ? (uint32_t)((e * gexp + (int64_t)(nwg + rl) * gpr + g) * 2) : 0x40000000u;
        const uint32_t sv = __builtin_amdgcn_raw_buffer_load_b16(rs, (int)off, 0, 0);
        const uint32_t bv = __builtin_amdgcn_raw_buffer_load_b16(rb, (int)off, 0, 0);
        sbl[idx] = (nwg + rl < a.N) ? (sv | (bv << 16)) : 0u;
    }
    lds_barrier();

    float acc[U][RPW];
#pragma unroll
    for (int u = 0; u < U; u++) {
        const int i = lane + 64 * u;
        const int s = sl[u] < 0 ? 0 : sl[u], c = i - (i / C) * C;
        u32x4 xv[XV];
#pragma unroll
        for (int v8 = 0; v8 < XV; v8++) xv[v8] = *(const u32x4*)(xs + ((size_t)s * XV * C + v8 * C + c) * 8);
        const float X = xc[s * C + c];
        const int g = (c * CK) >> a.gs_shift;
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            const float v = apply_group<BITS>(0.f, chunk_dot<BITS>(W[u][r], xv), X,
                                              sbl[(s * ROWS + wave * RPW + r) * gpr + g]);
            acc[u][r] = sl[u] < 0 ? 0.f : v;
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
            for (int u = 0; u < U; u++) v += sl[u] == s ? acc[u][r] : 0.f;
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

// Weight rows per wave: 1 while a call has few workgroups' worth of rows,
// else 4 (the staged x row is then shared by 16 rows per workgroup).
static int tok_rpw(int64_t N, int64_t wgs_per_row_tile) {
    return ceil_div(N, TOK_WV) * wgs_per_row_tile >= 2048 ? 4 : 1;
}

static int glu_lds(int64_t K, int bits, int gs, int rpw) {
    const int64_t CK = 128 / bits, C = K / CK;
    return (int)((128 / bits / 8) * C * 16 + C * 4 + 2 * TOK_WV * rpw * (K / gs) * 4);
}

}  // namespace kmi

using namespace kmi;

// Launchers shared with the SwitchGLU entry point (moe_glu.hip).
namespace kmi {

int launch_moe_glu_tok(const MoeTokArgs& a, int bits, hipStream_t st) {
    const int64_t CK = 128 / bits, C = a.K / CK;
    const int S = (int)ceil_div(C, 64);
    const int rpw = tok_rpw(a.N, a.T * a.k);
    const dim3 grid((unsigned)ceil_div(a.N, TOK_WV * rpw), (unsigned)(a.T * a.k));
    const size_t lds = (size_t)glu_lds(a.K, bits, 1 << a.gs_shift, rpw);
#define KMI_GLU(B, R, SS)                                                               \
    if (bits == B && rpw == R && S == SS) {                                             \
        moe_glu_tok<B, R, SS, TOK_WV><<<grid, 64 * TOK_WV, lds, st>>>(a);              \
        return OK;                                                                      \
    }
    KMI_GLU(4, 1, 1) KMI_GLU(4, 1, 2) KMI_GLU(4, 1, 4) KMI_GLU(8, 1, 1) KMI_GLU(8, 1, 2) KMI_GLU(8, 1, 4)
    KMI_GLU(8, 1, 8) KMI_GLU(4, 4, 1) KMI_GLU(4, 4, 2) KMI_GLU(8, 4, 1) KMI_GLU(8, 4, 2)
#undef KMI_GLU
    set_error("switch_glu: no gate/up kernel for %lld chunks per row", (long long)C);
    return EINVAL_ARG;
}

int launch_moe_down_tok(const MoeTokArgs& a, int bits, hipStream_t st) {
    const int64_t CK = 128 / bits, C = a.K / CK;
    const int U = (int)ceil_div((int64_t)a.k * C, 64);
    const int rpw = U <= 4 ? tok_rpw(a.N, a.T) : 1;
    const dim3 grid((unsigned)ceil_div(a.N, TOK_WV * rpw), (unsigned)a.T);
    const size_t lds = (size_t)a.k * ((128 / bits / 8) * C * 16 + C * 4) +
                       (size_t)a.k * TOK_WV * rpw * (a.K >> a.gs_shift) * 4;
#define KMI_DOWN(B, KM, UU, R)                                                          \
    if (bits == B && a.k <= KM && U == UU && rpw == R) {                                \
        moe_down_tok<B, KM, UU, R, TOK_WV><<<grid, 64 * TOK_WV, lds, st>>>(a);         \
        return OK;                                                                      \
    }
    KMI_DOWN(4, 8, 1, 1) KMI_DOWN(4, 8, 2, 1) KMI_DOWN(4, 8, 3, 1) KMI_DOWN(4, 8, 4, 1)
    KMI_DOWN(4, 8, 6, 1) KMI_DOWN(4, 8, 8, 1)
    KMI_DOWN(8, 8, 1, 1) KMI_DOWN(8, 8, 2, 1) KMI_DOWN(8, 8, 3, 1) KMI_DOWN(8, 8, 4, 1)
    KMI_DOWN(8, 8, 6, 1) KMI_DOWN(8, 8, 8, 1)
    KMI_DOWN(4, 8, 1, 4) KMI_DOWN(4, 8, 2, 4) KMI_DOWN(4, 8, 3, 4) KMI_DOWN(4, 8, 4, 4)
    KMI_DOWN(8, 8, 1, 4) KMI_DOWN(8, 8, 2, 4) KMI_DOWN(8, 8, 3, 4) KMI_DOWN(8, 8, 4, 4)
#undef KMI_DOWN
    set_error("switch_glu: no down kernel for k=%d, %lld chunks per row", a.k, (long long)C);
    return EINVAL_ARG;
}

}  // namespace kmi
