// Skinny quantized matmul over rows grouped by expert, with the tile's x
// rows staged once: the expert-grouped projections of SwitchGLU (gate|up
// with the _SwiGLU epilogue, and down) at token counts where each routed
// expert sees a handful to a few dozen rows (src/knurlogic/engine/families/
// glm5/architecture/glm5_next/_mlx_vlm/models/switch_layers.py:172-193 over
// QuantizedSwitchLinear, :71-86).
//
//   y[m, n] = sum_g ( s[n, g] * P[m, n, g] + b[n, g] * X[m, g] )
//   P[m, n, g] = sum_{k in g} x[m, k] q[n, k],   X[m, g] = sum_{k in g} x[m, k]
//
// A workgroup owns one tile (expert e, up to XR of its rows) and G
// consecutive 64-row column blocks of e's weight.  Its x rows (K bf16 each,
// every row padded by 16 bytes so the 16 rows of an MFMA fragment read
// different banks) are loaded into LDS once by direct-to-LDS loads; the
// weight and scale/bias chunks (256 codes of 64 rows) of all G blocks then
// stream through NS LDS stages, NS - 1 chunks in flight, one chunk after
// the other across the block boundaries, so a workgroup keeps its pipeline
// full for G * K / 256 chunks instead of refilling it per column block and
// re-staging x each time.  Per chunk a wave (16 weight rows) decodes its
// codes exactly to bf16 (integers < 256; E2M1 / E4M3 in the microscaled
// modes), runs the per-group MFMA chains against the staged x and adds
// s * P; the bias term sum_g b * X of the chunk's groups is one fp32 MFMA
// (v_mfma_f32_16x16x4_f32: X of the tile rows by group, from a table formed
// once per workgroup, against the rows' biases).  4-bit codes decode in
// the order [0,2,4,6,1,3,5,7] of each run of 8 (no byte shuffle), and the
// staged x is put in that order once, while the X table is summed.  After
// a block's last chunk the wave writes the block's outputs (SwiGLU of the
// gate and up sums for GLU) and starts the next block.
#include "qgemv_dl.hpp"
#include "pair_tiles.hpp"
#include "../../include/knurlogic_amd.h"


namespace kmi {

namespace {

template <int BITS, int GS, bool MX, int NSET>
struct XsShape {
    using D = DlShape<BITS, GS, MX, 1>;
    static constexpr int SET = D::W_BYTES + D::SB_BYTES;      // one set's weights + scales of a chunk
    static constexpr int STAGE = NSET * SET;
    static constexpr int PER_WAVE = NSET * (D::WBLK + D::SBI) / D::NW;   // DMA loads per wave per chunk
};

__device__ __forceinline__ float xs_bf16r(float v) { return bf16_to_f32(f32_to_bf16(v)); }

__device__ __forceinline__ float xs_f32_kept(double v) {
    float f = (float)v;
    asm volatile("" : "+v"(f));   // keep the float32 rounding (no fused f64 -> bf16 rounding)
    return f;
}

}  // namespace

// xrow: LDS bytes per staged x row (K * 2 + 16); xbytes: the x region (a
// multiple of 1 KB, at least XR rows); G: column blocks per workgroup.  XR:
// the tile's rows (4, 16, 32 or 64); a 4-row tile feeds the 16-row MFMA
// fragments with its rows repeated (the extra outputs are never written).
// LDS: the x region, NS stages, then (affine) the X table [K / GS][XR] fp32.
template <int BITS, int GS, bool MX, int XR, int NSET, int NS>
__global__ __launch_bounds__(256) void qgemv_xs_kernel(QgArgs a, int G, uint32_t xrow, uint32_t xbytes) {
    using D = DlShape<BITS, GS, MX, 1>;
    using XS = XsShape<BITS, GS, MX, NSET>;
    constexpr int RB = D::RB, RPI = D::RPI, WBLK = D::WBLK, PPR = D::PPR, W_BYTES = D::W_BYTES;
    constexpr int GPC = D::GPC, DPR = D::DPR, SBI = D::SBI, SB = D::SB, MXR = D::MXR, MXL = D::MXL;
    constexpr int GB = D::GB, LB = D::LB, NT = D::NT;
    constexpr int SET = XS::SET, STAGE = XS::STAGE, PER_WAVE = XS::PER_WAVE;
    constexpr int MT = XR, MC = XR < 16 ? 1 : XR / 16;
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ int32_t rid_s[MT];        // output row of tile row m (-1: none)
    __shared__ uint32_t xro_s[MT];       // byte offset of tile row m's x row (DL_NONE: none)

    // the tile: from the sort's list, or formed here from the routed pairs
    // (its working space over the x region, which is filled after the
    // tile's rows are read)
    int count, expert, start = 0;
    if (a.tiles) {
        const int32_t* tp = a.tiles + 3 * (int64_t)blockIdx.z;
        count = tp[2];
        expert = tp[0];
        start = tp[1];
    } else {
        const int pe = pair_tile_load(a.route, (int)a.rows);
        count = pair_tile_from(pe, (int)a.rows, (int)a.E, a.tm, (int)blockIdx.z, *(PairTileLds*)smem, rid_s,
                               expert, start);
        if (a.tiles_out && blockIdx.x == 0)     // the sort's list, for the next launch
            pair_tile_store(a.tiles_out, a.sorted_out, (int)blockIdx.z, expert, start, count, rid_s);
    }
    if (count <= 0 || count > MT || expert < 0 || expert >= a.E) return;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t K = a.K, Gk = K / GS;
    const uint32_t rowbytes = (uint32_t)(K * BITS / 8);
    const int NB = (int)((a.N + 63) / 64);
    const int j0 = (int)blockIdx.x * G;
    const int nblk = NB - j0 < G ? NB - j0 : G;
    const int C = (int)(K / DL_KC);
    const int total = nblk * C;

    __amdgpu_buffer_rsrc_t rw[NSET], rs[NSET], rb[NSET];
#pragma unroll
    for (int set = 0; set < NSET; set++) {
        const int64_t r0 = (int64_t)expert * a.erows + (set ? a.up_off : 0);
        rw[set] = make_rsrc((const char*)a.w + r0 * rowbytes, a.N * (int64_t)rowbytes);
        rs[set] = make_rsrc((const char*)a.s + r0 * Gk * SB, a.N * Gk * SB);
        rb[set] = make_rsrc((const char*)a.b + r0 * Gk * SB, MX ? 0 : a.N * Gk * SB);
    }
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, a.xrows * K * 2);

    // per-lane DMA coordinates within a 64-row block (the same for every block)
    int wr_[WBLK / 4];
    uint32_t wrel[WBLK / 4];
#pragma unroll
    for (int j = 0; j < WBLK / 4; j++) {
        const int r = (wave + 4 * j) * RPI + lane / PPR, slot = lane % PPR;
        wr_[j] = r;
        wrel[j] = (uint32_t)r * rowbytes + 16u * (uint32_t)(slot ^ (r & 7));
    }
    int sr_[SBI / 4];
    uint32_t srel[SBI / 4];
    int sbo[SBI / 4], sbw[SBI / 4];
#pragma unroll
    for (int j = 0; j < SBI / 4; j++) {
        if constexpr (MX) {
            const int row = wave * MXR + lane / MXL;
            sr_[j] = lane < 32 ? row : 1 << 20;
            srel[j] = (uint32_t)(row * Gk) + 4u * (uint32_t)(lane % MXL);
            sbo[j] = wave * 256;
            sbw[j] = 0;
        } else {
            const int q = wave + 4 * j, which = q / DPR, d = q % DPR;
            const int row = d * (DL_ROWS / DPR) + lane / DPR;
            sr_[j] = row;
            srel[j] = (uint32_t)(row * Gk * 2) + 4u * (uint32_t)(lane % DPR);
            sbo[j] = which * (DL_ROWS * GPC * 2) + d * 256;
            sbw[j] = which;
        }
    }

    // chunk i (block j0 + i / C, codes 256 * (i % C) ..) into stage i % NS;
    // past the last chunk every load reads zeros into a stage never read again
    auto issue = [&](int i) {
        const bool live = i < total;
        const int ii = live ? i : 0;
        const int n0 = 64 * (j0 + ii / C), c = ii % C;
        unsigned char* base = smem + xbytes + (i % NS) * STAGE;
#pragma unroll
        for (int set = 0; set < NSET; set++) {
#pragma unroll
            for (int j = 0; j < WBLK / 4; j++) {
                const bool ok = live && n0 + wr_[j] < a.N;
                dma16(rw[set], base + set * SET + (wave + 4 * j) * DL_WBLK_BYTES,
                      ok ? (uint32_t)n0 * rowbytes + wrel[j] : DL_NONE, (uint32_t)c * RB, 1);
            }
#pragma unroll
            for (int j = 0; j < SBI / 4; j++) {
                const bool ok = live && n0 + sr_[j] < a.N;
                const uint32_t rowoff = MX ? (uint32_t)(n0 * Gk) : (uint32_t)(n0 * Gk * 2);
                dma4(sbw[j] ? rb[set] : rs[set], base + set * SET + W_BYTES + sbo[j],
                     ok ? rowoff + srel[j] : DL_NONE, (uint32_t)c * (GPC * SB));
            }
        }
    };
#pragma unroll
    for (int i = 0; i < NS - 1; i++) issue(i);

    // the tile's rows: output row ids and x offsets (rows past count read none)
    if (tid < MT) {
        const int m = tid;
        int32_t rid = -1;
        uint32_t xo = DL_NONE;
        if (m < count) {
            rid = a.tiles ? a.sorted[start + m] : rid_s[m];
            const uint32_t mper = (uint32_t)a.Mper, ldiv = (uint32_t)a.lhs_div, ur = (uint32_t)rid;
            const uint32_t pr = mper == 1 ? ur : ur / mper;
            const uint32_t xb = a.lhs ? (uint32_t)a.lhs[pr] : (ldiv == 1 ? pr : pr / ldiv);
            const uint32_t xr = xb * mper + (ur - pr * mper);
            if (xr < (uint64_t)a.xrows) xo = (uint32_t)((uint64_t)xr * K * 2);
        }
        rid_s[m] = rid;
        xro_s[m] = xo;
    }
    __syncthreads();
    // x rows into LDS: 1 KB blocks of the padded [count][xrow] image
    {
        const uint32_t xb_used = (uint32_t)count * xrow;
        const uint32_t rowb = (uint32_t)K * 2u;
        for (uint32_t b = (uint32_t)wave; b * 1024u < xb_used; b += 4) {
            const uint32_t pos = b * 1024u + 16u * (uint32_t)lane;
            const uint32_t m = pos / xrow, col = pos - m * xrow;
            const uint32_t xo = m < (uint32_t)count && col < rowb ? xro_s[m] : DL_NONE;
            dma16(rx, smem + b * 1024u, xo == DL_NONE ? DL_NONE : xo + col, 0, 0);
        }
    }

    const int nl = lane & 15, j4 = lane >> 4;
    const int wr = wave * 16 + nl;                       // this lane's weight row in a block
    const int sro = MX ? (wr / MXR) * 256 + (wr % MXR) * GPC : wr * GPC;   // row's scales in the stage
    const unsigned char* xl[MC];
#pragma unroll
    for (int cc = 0; cc < MC; cc++) xl[cc] = smem + (uint32_t)(16 * cc + (XR < 16 ? nl % XR : nl)) * xrow;
    f32x4 acc[NSET][MC];
#pragma unroll
    for (int set = 0; set < NSET; set++)
#pragma unroll
        for (int cc = 0; cc < MC; cc++) acc[set][cc] = f32x4{0.f, 0.f, 0.f, 0.f};

    wait_vmcnt<0>();                                     // chunks 0 .. NS - 2 and the x rows
    __builtin_amdgcn_s_barrier();                        // of every wave
    // affine: X[g][m] = the sum of tile row m's x over group g (the bias
    // term's operand), and at 4 bits the staged x put in the decode's order
    float* const xtab = (float*)(smem + xbytes + NS * STAGE);
    if constexpr (!MX) {
        const int Gk = (int)(K / GS);
        for (int it = tid; it < count * Gk; it += 256) {
            const int m = it / Gk, g = it - (it / Gk) * Gk;
            unsigned char* xp = smem + (uint32_t)m * xrow + (uint32_t)g * (GS * 2);
            float sum = 0.f;
#pragma unroll
            for (int q = 0; q < GS / 8; q++) {
                const u32x4 v = *(const u32x4*)(xp + 16 * q);
#pragma unroll
                for (int e = 0; e < 4; e++) sum += __uint_as_float(v[e] << 16) + __uint_as_float(v[e] & 0xffff0000u);
                if constexpr (BITS == 4) *(u32x4*)(xp + 16 * q) = x8_paired(v);
            }
            xtab[g * XR + m] = sum;
        }
        lds_barrier();
    }

    for (int i = 0; i < total; i++) {
        if (i > 0) {
            wait_vmcnt<PER_WAVE * (NS - 2)>();           // this wave's loads of chunk i
            __builtin_amdgcn_s_barrier();                // and every wave's
        }
        const unsigned char* base = smem + xbytes + (i % NS) * STAGE;
        const int c = i % C;
        const uint32_t kb = (uint32_t)c * (DL_KC * 2);    // x byte offset of the chunk
        // affine: the bias term of the chunk's groups, lane (n, j4) holding
        // X[tile row n][group 4 q + j4] and that group's bias of weight row n
        if constexpr (!MX) {
#pragma unroll
            for (int q = 0; q < (GPC + 3) / 4; q++) {
                const int gq = 4 * q + j4;
                const bool ok = gq < GPC;
                float xa[MC];
#pragma unroll
                for (int cc = 0; cc < MC; cc++)
                    xa[cc] = ok ? xtab[(c * GPC + gq) * XR + (XR < 16 ? nl % XR : 16 * cc + nl)] : 0.f;
#pragma unroll
                for (int set = 0; set < NSET; set++) {
                    const uint16_t* sl = (const uint16_t*)(base + set * SET + W_BYTES);
                    const float bv = ok ? bf16_to_f32(sl[DL_ROWS * GPC + sro + gq]) : 0.f;
#pragma unroll
                    for (int cc = 0; cc < MC; cc++)
                        acc[set][cc] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[cc], bv, acc[set][cc], 0, 0, 0);
                }
            }
        }
        // groups whose reads are issued together: fewer at larger tiles, so
        // the fragments of a batch stay within the register budget
        constexpr int GH0 = MC * NSET >= 4 ? 1 : MC * NSET >= 2 ? 2 : 4;
        constexpr int GH = GPC < GH0 ? GPC : GH0;
#pragma unroll
        for (int h = 0; h < GPC; h += GH) {
            u32x4 wd[NSET][GH];
            u32x4 A[MC][GH][NT];
            float sc[NSET][GH];
#pragma unroll
            for (int g = 0; g < GH; g++) {
                const int gi = h + g;
                const int off = gi * GB + j4 * LB;
#pragma unroll
                for (int set = 0; set < NSET; set++) {
                    const unsigned char* wl = base + set * SET + (wr / RPI) * DL_WBLK_BYTES + (wr % RPI) * RB;
                    const unsigned char* p = wl + 16 * ((off / 16) ^ (wr & 7)) + off % 16;
                    if constexpr (LB == 4) wd[set][g] = u32x4{*(const uint32_t*)p, 0u, 0u, 0u};
                    else if constexpr (LB == 8) {
                        const u32x2 t = *(const u32x2*)p;
                        wd[set][g] = u32x4{t.x, t.y, 0u, 0u};
                    } else wd[set][g] = *(const u32x4*)p;
                    const unsigned char* sl = base + set * SET + W_BYTES;
                    if constexpr (MX) sc[set][g] = e8m0_to_f32(sl[sro + gi]);
                    else sc[set][g] = bf16_to_f32(((const uint16_t*)sl)[sro + gi]);
                }
#pragma unroll
                for (int cc = 0; cc < MC; cc++)
#pragma unroll
                    for (int t = 0; t < NT; t++)
                        A[cc][g][t] = *(const u32x4*)(xl[cc] + kb + 2 * (gi * GS + j4 * (GS / 4) + 8 * t));
            }
#pragma unroll
            for (int g = 0; g < GH; g++) {
                u32x4 B[NSET][NT];
#pragma unroll
                for (int set = 0; set < NSET; set++)
#pragma unroll
                    for (int t = 0; t < NT; t++) {
                        if constexpr (MX && BITS == 4) {
                            const uint32_t w = wd[set][g][t];
                            B[set][t] = u32x4{
                                __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.f, 0)),
                                __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.f, 1)),
                                __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.f, 2)),
                                __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.f, 3))};
                        } else if constexpr (MX) {
                            const uint32_t w0 = wd[set][g][2 * t], w1 = wd[set][g][2 * t + 1];
                            B[set][t] = u32x4{
                                __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.f, false)),
                                __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.f, true)),
                                __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.f, false)),
                                __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.f, true))};
                        } else if constexpr (BITS == 4) {
                            B[set][t] = nib8_paired(wd[set][g][t]);
                        } else {
                            B[set][t] = u32x4{bytes_to_bf16x2(wd[set][g][2 * t], 0),
                                              bytes_to_bf16x2(wd[set][g][2 * t], 2),
                                              bytes_to_bf16x2(wd[set][g][2 * t + 1], 0),
                                              bytes_to_bf16x2(wd[set][g][2 * t + 1], 2)};
                        }
                    }
#pragma unroll
                for (int cc = 0; cc < MC; cc++) {
                    f32x4 P[NSET];
#pragma unroll
                    for (int set = 0; set < NSET; set++) P[set] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int t = 0; t < NT; t++)
#pragma unroll
                        for (int set = 0; set < NSET; set++) P[set] = mfma16x16x32(A[cc][g][t], B[set][t], P[set]);
#pragma unroll
                    for (int set = 0; set < NSET; set++)
#pragma unroll
                        for (int e = 0; e < 4; e++) acc[set][cc][e] = __builtin_fmaf(sc[set][g], P[set][e], acc[set][cc][e]);
                }
            }
        }
        issue(i + NS - 1);
        if (c == C - 1) {
            // the block's outputs: D item e of the MFMA is tile row 4 * j4 + e, column nl
            const int64_t n = 64 * (int64_t)(j0 + i / C) + wr;
            if (n < a.N) {
#pragma unroll
                for (int cc = 0; cc < MC; cc++)
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const int m = 16 * cc + 4 * j4 + e;
                        if (m >= count) continue;
                        const int64_t row = rid_s[m];
                        if constexpr (NSET == 2) {
                            // act = round(round(silu_f32(round(gate))) * round(up))
                            const float sl = silu_bf16r(xs_bf16r(acc[0][cc][e]));
                            a.y[row * a.N + n] = f32_to_bf16(sl * xs_bf16r(acc[1][cc][e]));
                        } else {
                            a.y[row * a.N + n] = f32_to_bf16(acc[0][cc][e]);
                        }
                    }
            }
#pragma unroll
            for (int set = 0; set < NSET; set++)
#pragma unroll
                for (int cc = 0; cc < MC; cc++) acc[set][cc] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    }
    wait_vmcnt<0>();                                     // no LDS write may land after the workgroup ends
}

namespace {

// column blocks per workgroup: 4, fewer while the grid (tile slots, empty
// ones included) would have under `floor` workgroups: 1024 for down and
// the microscaled gate|up (mxfp4 at 16 tokens: 84.3 us at 900, 76.7 at
// 1024), 900 for the affine gate|up.  Measured at 128 experts, top-8,
// 2048 -> 768 -> 2048, affine 4-bit, µs per
// call: down flat within 2 µs over 1-8 blocks from 16 to 256 tokens;
// gate|up (12 column blocks) by tokens and blocks --
//   T =  9:  1 60.0   2 63.7   3 63.7   4 72.6
//   T = 12:  1 67.0   2 66.0   3 77.5   4 72.5
//   T = 16:  1 73.6   2 69.8   3 81.4   4 76.4
//   T = 24:  1 84.8   2 90.7   3 88.5   4 100.6
//   T = 32:  1 93.6   2 92.5   3 90.9   4 103.0
// (the floor of 900 picks 1, 1, 2, 2, 2 there).
int xs_blocks_per_wg(int64_t NB, int64_t tiles, bool affine_glu) {
    const int64_t floor = affine_glu ? 900 : 1024;
    int64_t g = NB < 4 ? NB : 4;
    while (g > 1 && ceil_div(NB, g) * tiles < floor) g--;
    return (int)g;
}

constexpr size_t XS_LDS_MAX = 160 * 1024 - 1024;   // the static row tables stay below 1 KB

// the affine kernels' X table: [K / GS][XR] fp32
template <int GS, bool MX, int XR>
size_t xs_xtab_bytes(int64_t K) { return MX ? 0 : (size_t)(K / GS) * XR * 4; }

template <int BITS, int GS, bool MX, int XR, int NSET, int NS>
int launch_xs_one(const QgArgs& a, int64_t ntiles, uint32_t xrow, uint32_t xbytes, hipStream_t st) {
    constexpr size_t stage = XsShape<BITS, GS, MX, NSET>::STAGE;
    const size_t lds = (size_t)xbytes + NS * stage + xs_xtab_bytes<GS, MX, XR>(a.K);
    if (lds > XS_LDS_MAX) return 1;
    allow_dynamic_lds_once((const void*)qgemv_xs_kernel<BITS, GS, MX, XR, NSET, NS>);
    const int64_t NB = (a.N + 63) / 64;
    const int G = xs_blocks_per_wg(NB, ntiles, NSET == 2 && !MX);
    const dim3 grid((unsigned)ceil_div(NB, G), 1, (unsigned)ntiles);
    qgemv_xs_kernel<BITS, GS, MX, XR, NSET, NS><<<grid, 256, lds, st>>>(a, G, xrow, xbytes);
    return 0;
}

// stages: 4 where two workgroups per CU still fit, else 3
template <int BITS, int GS, bool MX, int XR, int NSET>
int launch_xs_mc(const QgArgs& a, int64_t ntiles, uint32_t xrow, uint32_t xbytes, hipStream_t st) {
    constexpr size_t stage = XsShape<BITS, GS, MX, NSET>::STAGE;
    if ((size_t)xbytes + 4 * stage + xs_xtab_bytes<GS, MX, XR>(a.K) <= 78 * 1024)
        return launch_xs_one<BITS, GS, MX, XR, NSET, 4>(a, ntiles, xrow, xbytes, st);
    return launch_xs_one<BITS, GS, MX, XR, NSET, 3>(a, ntiles, xrow, xbytes, st);
}

template <int BITS, int GS, bool MX, int NSET>
int launch_xs_set(const QgArgs& a, int tr, int64_t ntiles, uint32_t xrow, uint32_t xbytes, hipStream_t st) {
    if (tr == 4) return launch_xs_mc<BITS, GS, MX, 4, NSET>(a, ntiles, xrow, xbytes, st);
    if (tr == 16) return launch_xs_mc<BITS, GS, MX, 16, NSET>(a, ntiles, xrow, xbytes, st);
    if (tr == 32) return launch_xs_mc<BITS, GS, MX, 32, NSET>(a, ntiles, xrow, xbytes, st);
    return launch_xs_mc<BITS, GS, MX, 64, NSET>(a, ntiles, xrow, xbytes, st);
}

template <int BITS, int GS, bool MX>
int launch_xs_glu(const QgArgs& a, bool glu, int tr, int64_t ntiles, uint32_t xrow, uint32_t xbytes,
                  hipStream_t st) {
    if (glu) return launch_xs_set<BITS, GS, MX, 2>(a, tr, ntiles, xrow, xbytes, st);
    return launch_xs_set<BITS, GS, MX, 1>(a, tr, ntiles, xrow, xbytes, st);
}

}  // namespace

// 0: launched; 1: this shape does not fit the kernel (the caller takes qgemv)
int launch_qgemv_xs(const QgArgs& a, int bits, int gs, bool glu, int tile_rows, int64_t ntiles, hipStream_t st) {
    const bool formed = !a.tiles && a.route;      // tiles formed in the kernel
    if (!(a.tiles && a.sorted) && !formed) return 1;
    if (a.S != 1 || a.K % DL_KC != 0) return 1;
    const int tr = tile_rows;
    if (!(tr == 4 || tr == 16 || tr == 32 || tr == 64) || !(bits == 4 || bits == 8)) return 1;
    if (formed && (a.tm != tr || !pair_tiles_fit(a.rows, a.E, tr))) return 1;
    if (glu && a.up_off <= 0) return 1;
    const uint32_t xrow = (uint32_t)(a.K * 2 + 16);
    uint64_t xb = ((uint64_t)tr * xrow + 1023) / 1024 * 1024;
    if (formed && xb < (sizeof(PairTileLds) + 1023) / 1024 * 1024) xb = (sizeof(PairTileLds) + 1023) / 1024 * 1024;
    if (xb > XS_LDS_MAX || a.xrows * a.K * 2 >= (1LL << 31)) return 1;
    const uint32_t xbytes = (uint32_t)xb;
    if (a.mx) {
        if (gs != 32) return 1;
        if (bits == 4) return launch_xs_glu<4, 32, true>(a, glu, tr, ntiles, xrow, xbytes, st);
        return launch_xs_glu<8, 32, true>(a, glu, tr, ntiles, xrow, xbytes, st);
    }
    if (bits == 4 && gs == 64) return launch_xs_glu<4, 64, false>(a, glu, tr, ntiles, xrow, xbytes, st);
    if (bits == 4 && gs == 32) return launch_xs_glu<4, 32, false>(a, glu, tr, ntiles, xrow, xbytes, st);
    if (bits == 8 && gs == 64) return launch_xs_glu<8, 64, false>(a, glu, tr, ntiles, xrow, xbytes, st);
    if (bits == 8 && gs == 32) return launch_xs_glu<8, 32, false>(a, glu, tr, ntiles, xrow, xbytes, st);
    return 1;
}

}  // namespace kmi
