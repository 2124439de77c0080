// Dense quantized matmul for 2..16 activation rows on gfx950, with the
// weight, x and scale/bias tiles staged by direct-to-LDS buffer loads
// (buffer_load_dwordx4 ... lds): the decode / MTP-verify shapes of
// mx.quantized_matmul (nn.QuantizedLinear, src/knurlogic/engine/model/
// load_model.py:124-144; the 9..31-row calls of engine/matmul_padding.py:
// 94-105 included).
//
//   y[m, n] = sum_g ( s[n, g] * P[m, n, g] + b[n, g] * X[m, g] )
//   P[m, n, g] = sum_{k in g} x[m, k] q[n, k],   X[m, g] = sum_{k in g} x[m, k]
//
// A workgroup owns 64 weight rows (16 per wave: the n of
// v_mfma_f32_16x16x32_bf16) and walks its share of K in chunks of 512 codes
// (256 where K is not a multiple of 512) through 3 LDS stages, two chunks in
// flight: the loads write LDS directly, so the depth costs no registers, and
// the wait for a chunk is an explicit vmcnt (the DMA loads return nothing to
// registers) followed by a barrier.  A 512-code chunk is two 256-code slices
// worked by two sets of four waves (eight per workgroup, so two per SIMD to
// hide each other's LDS and MFMA latencies), whose sums meet in the
// epilogue; the E8M0 scales of the microscaled modes decode without
// branches (e8m0_to_f32).  The DMA writes a wave's 64 lanes as one contiguous 1 KB block, so
// the bank-conflict swizzles are applied on the global side: lane slot s of
// a weight or x row holds the row's 16-byte piece s ^ (row & 7), and weight
// blocks are padded by 16 bytes.  x is staged in its natural k order, so
// 4-bit codes are decoded in natural order too (two v_perm_b32 + four
// fp8 -> bf16 conversions per 8 codes, exact).  Per chunk every LDS read is
// issued first, then the groups' independent MFMA chains, then the
// per-group scale / bias FMAs.
#include "qgemv_dl.hpp"
#include "../../include/knurlogic_amd.h"

namespace kmi {

template <int BITS, int GS, bool MX, int NS, int KS>
__global__ __launch_bounds__(256 * KS) void qgemv_dl_kernel(QgArgs a) {
    using S_ = DlShape<BITS, GS, MX, KS>;
    constexpr int KC = S_::KC, NW = S_::NW, XPB = S_::XPB, XBR = S_::XBR, XI = S_::XI, MXR = S_::MXR;
    constexpr int MXL = S_::MXL;
    constexpr int SB = S_::SB;
    constexpr int RB = S_::RB, RPI = S_::RPI, WBLK = S_::WBLK, PPR = S_::PPR, W_BYTES = S_::W_BYTES;
    constexpr int X_BYTES = S_::X_BYTES, GPC = S_::GPC, GPS = S_::GPS, DPR = S_::DPR, SBI = S_::SBI;
    constexpr int STAGE = S_::STAGE, GB = S_::GB, LB = S_::LB, NT = S_::NT;
    constexpr int PER_WAVE = S_::PER_WAVE;
    extern __shared__ __align__(16) unsigned char smem[];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rw4 = wave & 3, slice = wave >> 2;         // row block and K slice of this wave
    const int64_t n0 = (int64_t)blockIdx.x * DL_ROWS;
    const int64_t K = a.K, G = K / GS, M = a.rows;
    const uint32_t rowbytes = (uint32_t)(K * BITS / 8);
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.w, a.N * (int64_t)rowbytes);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.s, a.N * G * SB);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(a.b, MX ? 0 : a.N * G * SB);
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, M * K * 2);
    const int chunks = (int)(K / KC);
    const int c0 = (int)blockIdx.y * a.gps;
    const int nc = chunks - c0 < a.gps ? chunks - c0 : a.gps;

    // per-lane parts of the DMA offsets (rows past N / past M read zeros)
    uint32_t wv[WBLK / NW];
#pragma unroll
    for (int j = 0; j < WBLK / NW; j++) {
        const int r = (wave + NW * j) * RPI + lane / PPR, slot = lane % PPR;
        wv[j] = n0 + r < a.N ? (uint32_t)(n0 + r) * rowbytes + 16u * (uint32_t)(slot ^ (r & 7)) : DL_NONE;
    }
    uint32_t xv[XI / NW];
#pragma unroll
    for (int j = 0; j < XI / NW; j++) {
        const int b = wave + NW * j;                     // block b: x row b / XBR (XPB rows per block)
        const int m = XPB * (b / XBR) + lane / (64 / XPB), slot = (b % XBR) * 64 + lane % (64 / XPB);
        xv[j] = m < M ? (uint32_t)(m * K * 2) + 16u * (uint32_t)(slot ^ (m & 7)) : DL_NONE;
    }
    uint32_t sbv[SBI / NW];
    int sbo[SBI / NW], sbw[SBI / NW];
#pragma unroll
    for (int j = 0; j < SBI / NW; j++) {
        if constexpr (MX) {
            const int row = wave * MXR + lane / MXL;
            sbv[j] = lane < 32 && n0 + row < a.N ? (uint32_t)((n0 + row) * G) + 4u * (uint32_t)(lane % MXL)
                                                 : DL_NONE;
            sbo[j] = wave * 256;
            sbw[j] = 0;
        } else {
            const int q = wave + NW * j, which = q / DPR, d = q % DPR;
            const int row = d * (DL_ROWS / DPR) + lane / DPR;
            sbv[j] = n0 + row < a.N ? (uint32_t)((n0 + row) * G * 2) + 4u * (uint32_t)(lane % DPR) : DL_NONE;
            sbo[j] = which * (DL_ROWS * GPC * 2) + d * 256;
            sbw[j] = which;
        }
    }

    // chunk i of this split into stage i % NS; past the split's chunks every
    // load reads zeros into a stage that is never read again
    auto issue = [&](int i) {
        const bool live = i < nc;
        const uint32_t c = (uint32_t)(c0 + (live ? i : 0));
        unsigned char* base = smem + (i % NS) * STAGE;
#pragma unroll
        for (int j = 0; j < WBLK / NW; j++)
            dma16(rw, base + (wave + NW * j) * DL_WBLK_BYTES, live ? wv[j] : DL_NONE, c * RB, 1);
#pragma unroll
        for (int j = 0; j < XI / NW; j++)
            dma16(rx, base + W_BYTES + (wave + NW * j) * 1024, live ? xv[j] : DL_NONE, c * (KC * 2), 0);
#pragma unroll
        for (int j = 0; j < SBI / NW; j++)
            dma4(sbw[j] ? rb : rs, base + W_BYTES + X_BYTES + sbo[j], live ? sbv[j] : DL_NONE, c * (GPC * SB));
    };
#pragma unroll
    for (int i = 0; i < NS - 1; i++) issue(i);

    const int nl = lane & 15, j4 = lane >> 4;
    const int wr = rw4 * 16 + nl;                        // this lane's weight row in the tile
    const int g0 = slice * GPS;                          // this wave's first group of a chunk
    const int sro = MX ? (wr / MXR) * 256 + (wr % MXR) * GPC : wr * GPC;   // row's scales in the stage
    const u32x4 ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int i = 0; i < nc; i++) {
        wait_vmcnt<PER_WAVE * (NS - 2)>();               // this wave's loads of chunk i are in LDS
        __builtin_amdgcn_s_barrier();                    // and every wave's
        const unsigned char* base = smem + (i % NS) * STAGE;
        const unsigned char* wl = base + (wr / RPI) * DL_WBLK_BYTES + (wr % RPI) * RB;
        const unsigned char* xl = base + W_BYTES + nl * (KC * 2);
        const unsigned char* sl = base + W_BYTES + X_BYTES;
        constexpr int GH = GPS < 4 ? GPS : 4;
#pragma unroll
        for (int h = 0; h < GPS; h += GH) {
            u32x4 wd[GH];
            u32x4 A[GH][NT];
            float sc[GH], bi[GH];
#pragma unroll
            for (int g = 0; g < GH; g++) {
                const int gi = g0 + h + g;
                const int off = gi * GB + j4 * LB;
                const unsigned char* p = wl + 16 * ((off / 16) ^ (wr & 7)) + off % 16;
                if constexpr (LB == 4) wd[g] = u32x4{*(const uint32_t*)p, 0u, 0u, 0u};
                else if constexpr (LB == 8) {
                    const u32x2 t = *(const u32x2*)p;
                    wd[g] = u32x4{t.x, t.y, 0u, 0u};
                } else wd[g] = *(const u32x4*)p;
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    const int xp = gi * (GS / 8) + j4 * (GS / 32) + t;
                    A[g][t] = *(const u32x4*)(xl + 16 * (xp ^ (nl & 7)));
                }
                if constexpr (MX) {
                    sc[g] = e8m0_to_f32(sl[sro + gi]);
                    bi[g] = 0.f;
                } else {
                    sc[g] = bf16_to_f32(((const uint16_t*)sl)[sro + gi]);
                    bi[g] = bf16_to_f32(((const uint16_t*)sl)[DL_ROWS * GPC + sro + gi]);
                }
            }
            f32x4 P[GH], X[GH];
#pragma unroll
            for (int g = 0; g < GH; g++) {
                P[g] = f32x4{0.f, 0.f, 0.f, 0.f};
                X[g] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int t = 0; t < NT; t++)
#pragma unroll
                for (int g = 0; g < GH; g++) {
                    u32x4 B;
                    if constexpr (MX && BITS == 4) {
                        const uint32_t w = wd[g][t];
                        B = u32x4{__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.f, 0)),
                                  __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.f, 1)),
                                  __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.f, 2)),
                                  __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.f, 3))};
                    } else if constexpr (MX) {
                        const uint32_t w0 = wd[g][2 * t], w1 = wd[g][2 * t + 1];
                        B = u32x4{__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.f, false)),
                                  __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.f, true)),
                                  __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.f, false)),
                                  __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.f, true))};
                    } else if constexpr (BITS == 4) {
                        B = nib8_natural(wd[g][t]);
                    } else {
                        B = u32x4{bytes_to_bf16x2(wd[g][2 * t], 0), bytes_to_bf16x2(wd[g][2 * t], 2),
                                  bytes_to_bf16x2(wd[g][2 * t + 1], 0), bytes_to_bf16x2(wd[g][2 * t + 1], 2)};
                    }
                    if constexpr (!MX) X[g] = mfma16x16x32(A[g][t], ones, X[g]);
                    P[g] = mfma16x16x32(A[g][t], B, P[g]);
                }
#pragma unroll
            for (int g = 0; g < GH; g++)
#pragma unroll
                for (int e = 0; e < 4; e++)
                    acc[e] = MX ? __builtin_fmaf(sc[g], P[g][e], acc[e])
                                : __builtin_fmaf(sc[g], P[g][e], __builtin_fmaf(bi[g], X[g][e], acc[e]));
        }
        issue(i + NS - 1);
    }
    wait_vmcnt<0>();                                     // no LDS write may land after the workgroup ends

    if constexpr (KS > 1) {
        // slices 1.. hand their sums to slice 0 through LDS (the stages are
        // free once every wave is past its last chunk), added in slice order
        __syncthreads();
        f32x4* red = (f32x4*)smem;
        if (slice > 0) red[((slice - 1) * 4 + rw4) * 64 + lane] = acc;
        __syncthreads();
        if (slice > 0) return;
#pragma unroll
        for (int s = 1; s < KS; s++) {
            const f32x4 v = red[((s - 1) * 4 + rw4) * 64 + lane];
#pragma unroll
            for (int e = 0; e < 4; e++) acc[e] += v[e];
        }
    }

    // D of the MFMA: item e is x row 4 * j4 + e, column nl (weight row wr)
    const int64_t n = n0 + wr;
    if (n < a.N) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int64_t m = 4 * j4 + e;
            if (m < M) {
                if (a.S == 1) a.y[m * a.N + n] = f32_to_bf16(acc[e]);
                else a.partial[((int64_t)blockIdx.y * M + m) * a.N + n] = acc[e];
            }
        }
    }
}

namespace {

template <int BITS, int GS, bool MX, int NS, int KS>
int launch_dl_ns(const QgArgs& a, dim3 grid, hipStream_t st) {
    constexpr size_t lds = (size_t)NS * DlShape<BITS, GS, MX, KS>::STAGE;
    if constexpr (lds > 160 * 1024) {
        set_error("qgemv_dl: %d stages of %d slices exceed the LDS", NS, KS);
        return EINVAL_ARG;
    } else {
        allow_dynamic_lds_once((const void*)qgemv_dl_kernel<BITS, GS, MX, NS, KS>);
        qgemv_dl_kernel<BITS, GS, MX, NS, KS><<<grid, 256 * KS, lds, st>>>(a);
        return OK;
    }
}

// two K slices (8 waves, two per SIMD) wherever K holds whole 512-code chunks;
// three stages (two chunks in flight) fit the LDS at either width
constexpr int DL_NS = 3;

int dl_ks(int64_t K) { return K % (2 * DL_KC) == 0 ? 2 : 1; }

template <int BITS, int GS, bool MX>
int launch_dl(const QgArgs& a, dim3 grid, hipStream_t st) {
    if (dl_ks(a.K) == 2) return launch_dl_ns<BITS, GS, MX, DL_NS, 2>(a, grid, st);
    return launch_dl_ns<BITS, GS, MX, DL_NS, 1>(a, grid, st);
}

}  // namespace

bool qgemv_dl_supported(int64_t M, int64_t K, int bits, int gs) {
    return M >= 1 && M <= 16 && K % DL_KC == 0 && (bits == 4 || bits == 8) && (gs == 32 || gs == 64);
}

// K splits so the grid reaches about one workgroup per CU, each split
// keeping at least 4 chunks
QgPlan plan_qgemv_dl(int64_t N, int64_t K) {
    const int64_t tiles = ceil_div(N, DL_ROWS), chunks = K / (DL_KC * dl_ks(K));
    int64_t S = 1;
    while (tiles * S * 2 <= 256 && chunks / (S * 2) >= 4) S *= 2;
    QgPlan p = {};
    p.gps = (int)ceil_div(chunks, S);
    p.S = (int)ceil_div(chunks, p.gps);     // no split without chunks
    p.mc = 1;
    return p;
}

int launch_qgemv_dl(const QgArgs& a, const QgPlan& p, int bits, int gs, hipStream_t st) {
    const dim3 grid((unsigned)ceil_div(a.N, DL_ROWS), (unsigned)p.S);
    if (a.mx) {
        if (bits == 4 && gs == 32) return launch_dl<4, 32, true>(a, grid, st);
        if (bits == 8 && gs == 32) return launch_dl<8, 32, true>(a, grid, st);
    } else {
        if (bits == 4 && gs == 64) return launch_dl<4, 64, false>(a, grid, st);
        if (bits == 4 && gs == 32) return launch_dl<4, 32, false>(a, grid, st);
        if (bits == 8 && gs == 64) return launch_dl<8, 64, false>(a, grid, st);
        if (bits == 8 && gs == 32) return launch_dl<8, 32, false>(a, grid, st);
    }
    set_error("quantized_matmul: no direct-to-LDS kernel for %d bits, group %d", bits, gs);
    return EINVAL_ARG;
}

}  // namespace kmi
