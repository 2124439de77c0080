// Batched affine-quantized matmul for gfx950: mx.quantized_matmul with a
// weight that carries batch dimensions broadcast against x's, in both
// orientations --
//   transpose=True:  y = x What^T, What [N, K] (groups along K),
//   transpose=False: y = x What,   What [K, N] (groups along N) --
// and the masked softmax between the two products of mlx-lm's quantized
// scaled-dot-product attention
// (src/knurlogic/engine/families/glm5/architecture/glm5_next/_mlx_vlm/models/base.py:260-302).
// The per-head MLA projection takes the transpose=False product too
// (.../_mlx_vlm/models/mla.py:80-87, called at .../glm5_next/language.py:760).
//
// One kernel serves both orientations.  A workgroup owns a 64x64 output
// tile of one batch entry and walks the reduction axis in 64-wide tiles.
// The weight tile is dequantized (scale * q + bias in fp32) and split into
// two bf16 operands, hi = bf16(v) and lo = bf16(v - hi), which give v to
// 2^-17; both go to LDS k-contiguous per output column, whichever way the
// weight is stored, so both orientations feed the same MFMA loop: four
// waves, each 2x2 blocks of v_mfma_f32_16x16x32_bf16 against hi and then
// lo per 32 k.  The products are those of an fp32 dequantize (the
// precision of mlx's decode-size kernels), so a bf16 rounding of the scores
// downstream lands where the exact product puts it.
// Reductions long enough to leave the grid short (attention over many
// keys) split K across workgroups; the fp32 partials are summed in a fixed
// order by a second kernel, so results do not depend on timing.
#include "common.hpp"
#include "../../include/knurlogic_amd.h"

namespace kmi {

constexpr int QB_T = 64;                 // output rows, columns and reduction per tile
constexpr int QB_LD = 72;                // LDS row stride in bf16 (144 B: rows start 4 banks apart)
constexpr uint32_t QB_DEAD = 0x80000000u;
constexpr int QB_MAXD = 4;               // batch dimensions

struct QbArgs {
    const uint16_t* x;
    const uint32_t* w;
    const uint16_t* s;
    const uint16_t* b;
    uint16_t* y;                 // [P, M, ldy] bf16, when S == 1
    float* partial;              // [S, P, M, N] fp32, when S > 1
    int64_t M, K, N;
    int64_t xr, wr, sr;          // row strides: x in elements, w in words, scales / biases in elements
    int64_t ldy;                 // row stride of y (elements)
    int nd;
    int64_t shape[QB_MAXD], xs[QB_MAXD], ws[QB_MAXD], ss[QB_MAXD];
    int64_t P;                   // batch entries (product of shape)
    int mtiles, S, kts;          // row tiles, K splits, k-tiles per split
    int scale_x;                 // 1: x is staged as bf16(x * x_scale)
    float x_scale;
    // gather form (one batch dimension of P pairs): the weight of pair p is
    // entry widx[p] of nw stacked ones (ws[0] / ss[0] apart; out of range:
    // a zero output), its x entry xidx[p] (xs[0] apart)
    const int32_t* widx;
    const int32_t* xidx;
    int64_t nw, nx;              // stacked weights / x entries (indices past them: zero rows)
};

// OCP microscaling element and scale encodings (mxfp4: E2M1 elements,
// mxfp8: E4M3, both with an E8M0 power-of-two scale per 32 elements), built
// from their bit fields; every value is exact in fp32 (and in bf16).
__device__ __forceinline__ float qb_e8m0(uint32_t e) { return e8m0_to_f32(e); }     // 2^(e - 127)

__device__ __forceinline__ float qb_e2m1(uint32_t c) {
    const uint32_t e = (c >> 1) & 3u, m = c & 1u;
    const float mag = e ? __uint_as_float(((e + 126u) << 23) | (m << 22)) : (m ? 0.5f : 0.0f);
    return (c & 8u) ? -mag : mag;
}

__device__ __forceinline__ float qb_e4m3(uint32_t c) {
    const uint32_t e = (c >> 3) & 15u, m = c & 7u;
    float mag;
    if (e == 15u && m == 7u) mag = __uint_as_float(0x7fc00000u);
    else if (e == 0u) mag = (float)m * 0.001953125f;                         // m * 2^-9
    else mag = __uint_as_float(((e + 120u) << 23) | (m << 20));
    return (c & 0x80u) ? -mag : mag;
}

// MODE 0 affine (integer code), 1 mxfp4, 2 mxfp8: the element value of a code
template <int MODE>
__device__ __forceinline__ float qb_elem(uint32_t c) {
    if constexpr (MODE == 1) return qb_e2m1(c);
    else if constexpr (MODE == 2) return qb_e4m3(c);
    else return (float)c;
}

__device__ __forceinline__ uint32_t qb_pack(float lo, float hi) { return cvt_pk_bf16(lo, hi); }

// two fp32 values -> their bf16 hi parts and lo = bf16(v - hi), packed
__device__ __forceinline__ void qb_split(float v0, float v1, uint32_t& hi, uint32_t& lo) {
    hi = cvt_pk_bf16(v0, v1);
    lo = cvt_pk_bf16(v0 - __uint_as_float(hi << 16), v1 - __uint_as_float(hi & 0xffff0000u));
}

__device__ __forceinline__ uint32_t qb_code(uint32_t word, int i, int bits) {
    return (word >> (bits * i)) & ((1u << bits) - 1u);
}

// MB: 16-row blocks per output tile (1, 2 or 4): a tile is 16 MB rows x 64
// columns; the four waves cover it as WM x WN, each IM x JN MFMA blocks
// (few activation rows -- attention's GQA heads x queries -- take narrow
// tiles, so no MFMA or LDS work goes to rows that do not exist).
template <int BITS, int GS, bool TRANS, int MODE, int MB>
__global__ __launch_bounds__(256) void qmm_batched_kernel(QbArgs a) {
    constexpr int BM = 16 * MB;
    constexpr int WM = MB == 1 ? 1 : 2, WN = 4 / WM, IM = MB / WM, JN = 4 / WN;
    // one LDS stage (27 KB: five workgroups per CU); the next k-tile's
    // global loads are in flight in registers while this one is multiplied
    __shared__ __align__(16) uint16_t As[BM * QB_LD];
    __shared__ __align__(16) uint16_t Bh[QB_T * QB_LD];     // hi parts of the dequantized weight
    // lo parts (the mx modes' values are exact in bf16: no lo part)
    constexpr bool LO = MODE == 0;
    __shared__ __align__(16) uint16_t Bl[LO ? QB_T * QB_LD : 8];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;

    const int64_t p = blockIdx.z;
    const int mt = (int)(blockIdx.y % a.mtiles), split = (int)(blockIdx.y / a.mtiles);
    const int64_t nt = blockIdx.x;
    const int64_t M = a.M, K = a.K, N = a.N;

    // this batch entry's matrices
    int64_t xo = 0, wo = 0, so = 0, rem = p;
    bool w_ok = true, x_ok = true;
    if (a.widx) {
        const int64_t e = a.widx[p];
        w_ok = e >= 0 && e < a.nw;
        wo = (w_ok ? e : 0) * a.ws[0];
        so = (w_ok ? e : 0) * a.ss[0];
        const int64_t xi = a.xidx ? (int64_t)a.xidx[p] : p;
        x_ok = xi >= 0 && xi < a.nx;
        xo = (x_ok ? xi : 0) * a.xs[0];
    } else {
        for (int d = a.nd - 1; d >= 0; d--) {
            const int64_t i = rem % a.shape[d];
            rem /= a.shape[d];
            xo += i * a.xs[d];
            wo += i * a.ws[d];
            so += i * a.ss[d];
        }
    }
    const int64_t wrow_words = (TRANS ? K : N) * BITS / 32;
    const int64_t wrows = TRANS ? N : K;
    const int64_t srow = (TRANS ? K : N) / GS;
    // x rows are read in whole 16-byte runs (a run that crosses the end of
    // the range reads as zeros entirely), so the range ends at the last
    // row's padding to 8 elements; elements past K are zeroed on staging
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x + xo, x_ok ? ((M - 1) * a.xr + ((K + 7) & ~7LL)) * 2 : 0);
    // scales: bf16 (affine) or one E8M0 byte (mx modes); mx modes have no biases
    constexpr int SB = MODE ? 1 : 2;
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.w + wo, w_ok ? ((wrows - 1) * a.wr + wrow_words) * 4 : 0);
    const __amdgpu_buffer_rsrc_t rs =
        make_rsrc((const char*)a.s + so * SB, w_ok ? ((wrows - 1) * a.sr + srow) * SB : 0);
    const __amdgpu_buffer_rsrc_t rb =
        make_rsrc(MODE ? (const void*)a.s : (const void*)(a.b + so), (w_ok && !MODE) ? ((wrows - 1) * a.sr + srow) * 2 : 0);

    const int64_t kt_all = (K + QB_T - 1) / QB_T;
    const int64_t kt0 = (int64_t)split * a.kts;
    int64_t kt1 = kt0 + a.kts;
    if (kt1 > kt_all) kt1 = kt_all;

    // staging coordinates: x row xrow, k run [16 xc, 16 xc + 16) of the tile
    const int xrow = tid >> 2, xc = tid & 3;
    const int64_t m_x = (int64_t)mt * BM + xrow;
    const bool x_row = xrow < BM;                 // this thread stages x (whole waves)
    // weight: TRANS -- row n = wrow_t of the tile, codes [16 xc, +16) of k;
    //         !TRANS -- rows k = 4 kq .. 4 kq + 3, columns n = 4 nq .. 4 nq + 3
    const int kq = tid >> 4, nq = tid & 15;
    const int64_t n_t = nt * QB_T + xrow;

    // staged words: TRANS 16 codes (4 / 8 bits: the words themselves; other
    // widths: four words from the one holding the run's first bit), else 4
    // rows x 4 codes (one word per row, or two for the other widths)
    constexpr bool WORD_ALIGNED = BITS == 4 || BITS == 8;
    constexpr int WV = TRANS ? (BITS == 8 ? 4 : BITS == 4 ? 2 : 4) : (WORD_ALIGNED ? 4 : 8);
    // other widths: the bit offset of a thread's run within its first word
    // is the same on every k-tile / row (tiles hold 64 codes)
    const uint32_t wsh = TRANS ? (uint32_t)((16 * xc * BITS) & 31) : (uint32_t)((4 * nq * BITS) & 31);
    u32x4 rxv[2];
    uint32_t rwv[WV];
    uint32_t rsv[TRANS ? 1 : 4], rbv[TRANS ? 1 : 4];

    auto issue = [&](int64_t kt) {
        const int64_t k0 = kt * QB_T + 16 * xc;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int64_t k = k0 + 8 * h;
            const uint32_t off = (x_row && m_x < M && k < K) ? (uint32_t)((m_x * a.xr + k) * 2) : QB_DEAD;
            rxv[h] = x_row ? __builtin_amdgcn_raw_buffer_load_b128(rx, (int)off, 0, 0) : u32x4{0u, 0u, 0u, 0u};
        }
        if constexpr (TRANS) {
            const bool ok = n_t < N && k0 < K;
            const uint32_t woff = ok ? (uint32_t)((n_t * a.wr + k0 * BITS / 32) * 4) : QB_DEAD;
            if constexpr (BITS == 8) {
                const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rw, (int)woff, 0, 0);
                rwv[0] = v.x; rwv[1] = v.y; rwv[2] = v.z; rwv[3] = v.w;
            } else if constexpr (BITS == 4) {
                const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rw, (int)woff, 0, 0);
                rwv[0] = v.x; rwv[1] = v.y;
            } else {
                // words past the row's end belong to the next row or read
                // as zeros past the range; their bits are never used
#pragma unroll
                for (int q = 0; q < 4; q++)
                    rwv[q] = __builtin_amdgcn_raw_buffer_load_b32(rw, ok ? (int)(woff + 4 * q) : (int)QB_DEAD, 0, 0);
            }
            const uint32_t soff = ok ? (uint32_t)((n_t * a.sr + k0 / GS) * SB) : QB_DEAD;
            if constexpr (MODE) {
                rsv[0] = __builtin_amdgcn_raw_buffer_load_b8(rs, (int)soff, 0, 0);
                rbv[0] = 0;
            } else {
                rsv[0] = __builtin_amdgcn_raw_buffer_load_b16(rs, (int)soff, 0, 0);
                rbv[0] = __builtin_amdgcn_raw_buffer_load_b16(rb, (int)soff, 0, 0);
            }
        } else {
            const int64_t n = nt * QB_T + 4 * nq;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int64_t k = kt * QB_T + 4 * kq + j;
                const bool ok = k < K && n < N;
                if constexpr (BITS == 8) {
                    const uint32_t woff = ok ? (uint32_t)((k * a.wr + n / 4) * 4) : QB_DEAD;
                    rwv[j] = __builtin_amdgcn_raw_buffer_load_b32(rw, (int)woff, 0, 0);
                } else if constexpr (BITS == 4) {
                    const uint32_t woff = ok ? (uint32_t)(k * a.wr * 4 + n / 2) : QB_DEAD;
                    rwv[j] = __builtin_amdgcn_raw_buffer_load_b16(rw, (int)woff, 0, 0);
                } else {
                    const uint32_t woff = ok ? (uint32_t)((k * a.wr + n * BITS / 32) * 4) : QB_DEAD;
                    rwv[2 * j] = __builtin_amdgcn_raw_buffer_load_b32(rw, (int)woff, 0, 0);
                    rwv[2 * j + 1] = __builtin_amdgcn_raw_buffer_load_b32(rw, ok ? (int)(woff + 4) : (int)QB_DEAD, 0, 0);
                }
                const uint32_t soff = ok ? (uint32_t)((k * a.sr + n / GS) * SB) : QB_DEAD;
                if constexpr (MODE) {
                    rsv[j] = __builtin_amdgcn_raw_buffer_load_b8(rs, (int)soff, 0, 0);
                    rbv[j] = 0;
                } else {
                    rsv[j] = __builtin_amdgcn_raw_buffer_load_b16(rs, (int)soff, 0, 0);
                    rbv[j] = __builtin_amdgcn_raw_buffer_load_b16(rb, (int)soff, 0, 0);
                }
            }
        }
    };

    auto store = [&](int64_t kt) {
        // x: zero the elements past K of a run that straddles it, apply the scale
        const int64_t k0 = kt * QB_T + 16 * xc;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            u32x4 v = rxv[h];
            const int64_t k = k0 + 8 * h;
            if (k + 8 > K && k < K) {
#pragma unroll
                for (int e = 0; e < 8; e++)
                    if (k + e >= K) v[e >> 1] &= (e & 1) ? 0x0000ffffu : 0xffff0000u;
            }
            if (a.scale_x) {
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const uint32_t u = v[e];
                    v[e] = qb_pack(bf16_to_f32((uint16_t)(u & 0xffffu)) * a.x_scale,
                                   bf16_to_f32((uint16_t)(u >> 16)) * a.x_scale);
                }
            }
            if (x_row) *(u32x4*)&As[xrow * QB_LD + 16 * xc + 8 * h] = v;
        }
        if constexpr (TRANS) {
            const float sc = MODE ? qb_e8m0(rsv[0] & 0xffu) : bf16_to_f32((uint16_t)rsv[0]);
            const float bi = MODE ? 0.0f : bf16_to_f32((uint16_t)rbv[0]);
            float q[16];
            if constexpr (WORD_ALIGNED) {
                constexpr int CPW = 32 / BITS;
#pragma unroll
                for (int i = 0; i < 16; i++) q[i] = qb_elem<MODE>(qb_code(rwv[i / CPW], i % CPW, BITS));
            } else {
                // the run's bit stream shifted to bit 0, then fields at i * BITS
                const uint32_t r0 = __builtin_amdgcn_alignbit(rwv[1], rwv[0], wsh);
                const uint32_t r1 = __builtin_amdgcn_alignbit(rwv[2], rwv[1], wsh);
                const uint32_t r2 = __builtin_amdgcn_alignbit(rwv[3], rwv[2], wsh);
                const uint32_t r[3] = {r0, r1, r2};
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const int o = i * BITS, w = o >> 5, sh = o & 31;
                    const uint32_t f = sh + BITS <= 32 ? r[w] >> sh : __builtin_amdgcn_alignbit(r[w + 1], r[w], sh);
                    q[i] = (float)(f & ((1u << BITS) - 1u));
                }
            }
            uint32_t oh[8], ol[8];
#pragma unroll
            for (int i = 0; i < 16; i += 2)
                qb_split(__builtin_fmaf(sc, q[i], bi), __builtin_fmaf(sc, q[i + 1], bi), oh[i / 2], ol[i / 2]);
            u32x4* dh = (u32x4*)&Bh[xrow * QB_LD + 16 * xc];
            dh[0] = u32x4{oh[0], oh[1], oh[2], oh[3]};
            dh[1] = u32x4{oh[4], oh[5], oh[6], oh[7]};
            if constexpr (LO) {
                u32x4* dl = (u32x4*)&Bl[xrow * QB_LD + 16 * xc];
                dl[0] = u32x4{ol[0], ol[1], ol[2], ol[3]};
                dl[1] = u32x4{ol[4], ol[5], ol[6], ol[7]};
            }
        } else {
            float v[4][4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float sc = MODE ? qb_e8m0(rsv[j] & 0xffu) : bf16_to_f32((uint16_t)rsv[j]);
                const float bi = MODE ? 0.0f : bf16_to_f32((uint16_t)rbv[j]);
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    float q;
                    if constexpr (WORD_ALIGNED) {
                        q = qb_elem<MODE>(qb_code(rwv[j], c, BITS));
                    } else {
                        const uint32_t r = __builtin_amdgcn_alignbit(rwv[2 * j + 1], rwv[2 * j], wsh);
                        q = (float)((r >> (c * BITS)) & ((1u << BITS) - 1u));
                    }
                    v[j][c] = __builtin_fmaf(sc, q, bi);
                }
            }
#pragma unroll
            for (int c = 0; c < 4; c++) {
                uint32_t h0, l0, h1, l1;
                qb_split(v[0][c], v[1][c], h0, l0);
                qb_split(v[2][c], v[3][c], h1, l1);
                *(u32x2*)&Bh[(4 * nq + c) * QB_LD + 4 * kq] = u32x2{h0, h1};
                if constexpr (LO) *(u32x2*)&Bl[(4 * nq + c) * QB_LD + 4 * kq] = u32x2{l0, l1};
            }
        }
    };

    f32x4 acc[IM][JN];
#pragma unroll
    for (int i = 0; i < IM; i++)
#pragma unroll
        for (int j = 0; j < JN; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int fr = lane & 15, fk = 8 * (lane >> 4);
    auto compute = [&]() {
#pragma unroll
        for (int kk = 0; kk < QB_T; kk += 32) {
            u32x4 A[IM], H[JN], Lo[JN];
#pragma unroll
            for (int i = 0; i < IM; i++)
                A[i] = *(const u32x4*)&As[(16 * IM * wm + 16 * i + fr) * QB_LD + kk + fk];
#pragma unroll
            for (int j = 0; j < JN; j++) {
                H[j] = *(const u32x4*)&Bh[(16 * JN * wn + 16 * j + fr) * QB_LD + kk + fk];
                if constexpr (LO) Lo[j] = *(const u32x4*)&Bl[(16 * JN * wn + 16 * j + fr) * QB_LD + kk + fk];
            }
#pragma unroll
            for (int i = 0; i < IM; i++)
#pragma unroll
                for (int j = 0; j < JN; j++) {
                    if constexpr (LO) acc[i][j] = mfma16x16x32(A[i], Lo[j], acc[i][j]);
                    acc[i][j] = mfma16x16x32(A[i], H[j], acc[i][j]);
                }
        }
    };

    // LDS-only barriers: the loads of the next k-tile stay in flight
    if (kt0 < kt1) issue(kt0);
    for (int64_t kt = kt0; kt < kt1; kt++) {
        store(kt);
        lds_barrier();
        if (kt + 1 < kt1) issue(kt + 1);
        compute();
        lds_barrier();
    }

#pragma unroll
    for (int i = 0; i < IM; i++)
#pragma unroll
        for (int j = 0; j < JN; j++) {
            const int64_t n = nt * QB_T + 16 * JN * wn + 16 * j + fr;
            if (n >= N) continue;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int64_t m = (int64_t)mt * BM + 16 * IM * wm + 16 * i + 4 * (lane >> 4) + e;
                if (m >= M) continue;
                if (a.S == 1)
                    a.y[(p * M + m) * a.ldy + n] = f32_to_bf16(acc[i][j][e]);
                else
                    a.partial[(((int64_t)split * a.P + p) * M + m) * N + n] = acc[i][j][e];
            }
        }
}

// y = bf16(sum over the S splits, in split order)
__global__ __launch_bounds__(256) void qmm_batched_reduce(const float* __restrict__ partial, int S,
                                                          int64_t count, int64_t N, int64_t ldy,
                                                          uint16_t* __restrict__ y) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= count) return;
    // the S loads are issued together, then summed in split order
    float v[8];
    float s = 0.f;
    for (int k0 = 0; k0 < S; k0 += 8) {
#pragma unroll
        for (int k = 0; k < 8; k++) v[k] = k0 + k < S ? partial[(k0 + k) * count + i] : 0.f;
#pragma unroll
        for (int k = 0; k < 8; k++) s += v[k];
    }
    y[(i / N) * ldy + i % N] = f32_to_bf16(s);
}

// ---- masked softmax --------------------------------------------------------------
// mlx-lm's quantized attention between its two products (base.py:285-295):
// a bool mask replaces hidden scores by finfo(bf16).min, an additive mask is
// added (rounded to bf16), "causal" hides key j from query l of L when
// j > N - L + l; then softmax(precise=True): max, exp and sum in fp32, the
// probabilities rounded to bf16.  One workgroup per row.

struct SmArgs {
    const uint16_t* x;
    int64_t ldx;
    uint16_t* out;
    int64_t ldo;
    int64_t N;
    int64_t dims[4];             // row index = ((i0 * d1 + i1) * d2 + i2) * d3 + i3
    const void* mask;
    int kind;                    // KMI_MASK_*
    int64_t ms[4];               // mask element strides of the four row dimensions
};

constexpr float BF16_LOWEST = -3.38953139e38f;      // finfo(bfloat16).min

__device__ __forceinline__ float block_reduce(float v, bool is_max, float* red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float u = __shfl_xor(v, o, 64);
        v = is_max ? fmaxf(v, u) : v + u;
    }
    const int wave = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int w = 1; w < 4; w++) r = is_max ? fmaxf(r, red[w]) : r + red[w];
    return r;
}

constexpr uint32_t BF16_NEG_INF = 0xff80u;

// Eight scores from j0 on, masked: hidden -> finfo(bf16).min, additive mask
// added and rounded, past the row -> -inf (adds nothing to the sum).
__device__ __forceinline__ u32x4 sm_chunk(const SmArgs& a, const uint16_t* xr, const uint8_t* mb,
                                          const uint16_t* ma, int64_t j0, int64_t vis) {
    u32x4 v = *(const u32x4*)(xr + j0);
    if (a.kind == KMI_MASK_NONE && j0 + 8 <= a.N) return v;
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const int64_t j = j0 + e;
        uint32_t h = (v[e >> 1] >> (16 * (e & 1))) & 0xffffu;
        if (j >= a.N) {
            h = BF16_NEG_INF;
        } else if (a.kind == KMI_MASK_BOOL) {
            if (!mb[j]) h = f32_to_bf16(BF16_LOWEST);
        } else if (a.kind == KMI_MASK_ADD) {
            h = f32_to_bf16(bf16_to_f32((uint16_t)h) + bf16_to_f32(ma[j]));
        } else if (a.kind == KMI_MASK_CAUSAL) {
            if (j > vis) h = f32_to_bf16(BF16_LOWEST);
        }
        v[e >> 1] = (e & 1) ? ((v[e >> 1] & 0x0000ffffu) | (h << 16)) : ((v[e >> 1] & 0xffff0000u) | h);
    }
    return v;
}

__device__ __forceinline__ float sm_max8(u32x4 v, float m) {
#pragma unroll
    for (int e = 0; e < 4; e++)
        m = fmaxf(m, fmaxf(__uint_as_float(v[e] << 16), __uint_as_float(v[e] & 0xffff0000u)));
    return m;
}

__device__ __forceinline__ float sm_sum8(u32x4 v, float mx, float s) {
#pragma unroll
    for (int e = 0; e < 4; e++)
        s += expf(__uint_as_float(v[e] << 16) - mx) + expf(__uint_as_float(v[e] & 0xffff0000u) - mx);
    return s;
}

__device__ __forceinline__ u32x4 sm_prob8(u32x4 v, float mx, float sum) {
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; e++)
        o[e] = qb_pack(expf(__uint_as_float(v[e] << 16) - mx) / sum,
                       expf(__uint_as_float(v[e] & 0xffff0000u) - mx) / sum);
    return o;
}

// One workgroup per row, 8 scores per 16-byte load.  CH > 0: the row stays
// in registers (CH chunks of 8 per thread, N <= 2048 CH); CH == 0: any N,
// three passes over the row.
template <int CH>
__global__ __launch_bounds__(256) void masked_softmax_kernel(SmArgs a) {
    __shared__ float red[4];
    const int64_t r = blockIdx.x;
    const int64_t i3 = r % a.dims[3], r2 = r / a.dims[3];
    const int64_t i2 = r2 % a.dims[2], r1 = r2 / a.dims[2];
    const int64_t i1 = r1 % a.dims[1], i0 = r1 / a.dims[1];
    const uint16_t* xr = a.x + r * a.ldx;
    uint16_t* orow = a.out + r * a.ldo;
    const int64_t moff = i0 * a.ms[0] + i1 * a.ms[1] + i2 * a.ms[2] + i3 * a.ms[3];
    const uint8_t* mb = a.kind == KMI_MASK_BOOL ? (const uint8_t*)a.mask + moff : nullptr;
    const uint16_t* ma = a.kind == KMI_MASK_ADD ? (const uint16_t*)a.mask + moff : nullptr;
    const int64_t vis = a.N - a.dims[3] + i3;              // causal: last visible key
    const int64_t nch = (a.N + 7) / 8;
    const int t = threadIdx.x;

    float mx = -INFINITY, sum = 0.f;
    if constexpr (CH > 0) {
        u32x4 v[CH];
#pragma unroll
        for (int c = 0; c < CH; c++) {
            const int64_t j = t + 256 * c;
            v[c] = j < nch ? sm_chunk(a, xr, mb, ma, 8 * j, vis)
                           : u32x4{0xff80ff80u, 0xff80ff80u, 0xff80ff80u, 0xff80ff80u};
            mx = sm_max8(v[c], mx);
        }
        mx = block_reduce(mx, true, red);
#pragma unroll
        for (int c = 0; c < CH; c++) sum = sm_sum8(v[c], mx, sum);
        sum = block_reduce(sum, false, red);
#pragma unroll
        for (int c = 0; c < CH; c++) {
            const int64_t j = t + 256 * c;
            if (j < nch) *(u32x4*)(orow + 8 * j) = sm_prob8(v[c], mx, sum);
        }
    } else {
        for (int64_t j = t; j < nch; j += 256) mx = sm_max8(sm_chunk(a, xr, mb, ma, 8 * j, vis), mx);
        mx = block_reduce(mx, true, red);
        for (int64_t j = t; j < nch; j += 256) sum = sm_sum8(sm_chunk(a, xr, mb, ma, 8 * j, vis), mx, sum);
        sum = block_reduce(sum, false, red);
        for (int64_t j = t; j < nch; j += 256)
            *(u32x4*)(orow + 8 * j) = sm_prob8(sm_chunk(a, xr, mb, ma, 8 * j, vis), mx, sum);
    }
}

// ---- host side ------------------------------------------------------------------

struct QbPlan {
    int64_t P, mtiles, ntiles;
    int S, kts, mb;
};

// narrow: whether 32-row tiles exist for the width (4 and 8 bits)
static QbPlan plan_batched(int64_t P, int64_t M, int64_t K, int64_t N, bool narrow = true) {
    QbPlan q;
    q.P = P;
    q.mb = M <= 16 ? 1 : (M <= 32 && narrow) ? 2 : 4;
    q.mtiles = ceil_div(M, 16 * q.mb);
    q.ntiles = ceil_div(N, QB_T);
    const int64_t kt_all = ceil_div(K, QB_T);
    // the K split depends on 64-row tiles only (so the workspace size does
    // not depend on the tile shape)
    const int64_t tiles = ceil_div(M, QB_T) * q.ntiles * P;
    // split K while the grid is short of four workgroups per CU and each
    // split keeps at least 4 k-tiles
    int64_t S = 1;
    while (tiles * S < 1024 && kt_all / (S * 2) >= 4) S *= 2;
    const int64_t kts = ceil_div(kt_all, S);
    q.kts = (int)kts;
    q.S = (int)ceil_div(kt_all, kts);
    return q;
}

static size_t batched_partial_bytes(const QbPlan& q, int64_t M, int64_t N) {
    return q.S > 1 ? (size_t)q.S * q.P * M * N * 4 : 0;
}

template <int B_, int G_, bool T_, int M_>
static void launch_qb(const QbArgs& a, int mb, dim3 grid, hipStream_t st) {
    if (mb == 1) qmm_batched_kernel<B_, G_, T_, M_, 1><<<grid, 256, 0, st>>>(a);
    else if (mb == 2 && (B_ == 4 || B_ == 8)) qmm_batched_kernel<B_, G_, T_, M_, (B_ == 4 || B_ == 8) ? 2 : 4><<<grid, 256, 0, st>>>(a);
    else qmm_batched_kernel<B_, G_, T_, M_, 4><<<grid, 256, 0, st>>>(a);
}

#define KMI_QB_CASE(B_, G_, T_) \
    if (mode == 0 && bits == B_ && gs == G_ && trans == T_) { launch_qb<B_, G_, T_, 0>(a, mb, grid, st); return OK; }
#define KMI_QB_G(B_, T_) KMI_QB_CASE(B_, 32, T_) KMI_QB_CASE(B_, 64, T_) KMI_QB_CASE(B_, 128, T_)
#define KMI_QB_B(B_) KMI_QB_G(B_, true) KMI_QB_G(B_, false)

static int launch_batched(const QbArgs& a, int mode, int bits, int gs, bool trans, int mb, dim3 grid,
                          hipStream_t st) {
    KMI_QB_B(4) KMI_QB_B(8) KMI_QB_B(2) KMI_QB_B(3) KMI_QB_B(5) KMI_QB_B(6)
    if (mode == 1 && trans) { launch_qb<4, 32, true, 1>(a, mb, grid, st); return OK; }
    if (mode == 1 && !trans) { launch_qb<4, 32, false, 1>(a, mb, grid, st); return OK; }
    if (mode == 2 && trans) { launch_qb<8, 32, true, 2>(a, mb, grid, st); return OK; }
    if (mode == 2 && !trans) { launch_qb<8, 32, false, 2>(a, mb, grid, st); return OK; }
    set_error("quantized_matmul (batched): no kernel for bits=%d gs=%d", bits, gs);
    return EINVAL_ARG;
}

#undef KMI_QB_B
#undef KMI_QB_G
#undef KMI_QB_CASE

static int64_t batch_count(int nd, const int64_t* shape) {
    int64_t P = 1;
    for (int d = 0; d < nd; d++) P *= shape[d];
    return P;
}

}  // namespace kmi

using namespace kmi;

extern "C" {

size_t kmi_qmm_batched_workspace_bytes(int nd, const int64_t* batch_shape, int64_t M, int64_t K, int64_t N) {
    if (nd < 0 || nd > QB_MAXD || (nd > 0 && !batch_shape) || M <= 0 || K <= 0 || N <= 0) return 0;
    const int64_t P = batch_count(nd, batch_shape);
    if (P <= 0) return 0;
    return batched_partial_bytes(plan_batched(P, M, K, N), M, N);
}

int kmi_qmm_batched(const void* x, const int64_t* x_strides, const uint32_t* w, const int64_t* w_strides,
                    const void* scales, const void* biases, const int64_t* s_strides, int nd,
                    const int64_t* batch_shape, int64_t M, int64_t K, int64_t N, int transpose, int dtype,
                    int group_size, int bits, int mode, const int32_t* widx, const int32_t* xidx, int64_t nw,
                    int64_t nx, float x_scale, void* y, int64_t ldy, void* workspace, size_t workspace_bytes,
                    void* stream) {
    clear_error();
    KMI_CHECK_ARG(dtype == BF16, "quantized_matmul (batched): only bfloat16 is supported (got dtype %d)", dtype);
    KMI_CHECK_ARG(mode == 0 || (mode == 1 && bits == 4 && group_size == 32) ||
                      (mode == 2 && bits == 8 && group_size == 32),
                  "quantized_matmul (batched): mode %d with %d bits / group %d (mxfp4: 4 / 32, mxfp8: 8 / 32)",
                  mode, bits, group_size);
    KMI_CHECK_ARG(!(widx || xidx) || (widx && nd == 1 && nw >= 1 && nx >= 1),
                  "quantized_matmul (batched): the gather form takes widx, one batch dimension, nw, nx >= 1");
    KMI_CHECK_ARG(bits >= 2 && bits <= 8 && bits != 7, "quantized_matmul (batched): bits %d not in {2,3,4,5,6,8}",
                  bits);
    KMI_CHECK_ARG(group_size == 32 || group_size == 64 || group_size == 128,
                  "quantized_matmul (batched): group_size %d not in {32, 64, 128}", group_size);
    KMI_CHECK_ARG(nd >= 0 && nd <= QB_MAXD, "quantized_matmul (batched): %d batch dimensions (at most %d)",
                  nd, QB_MAXD);
    KMI_CHECK_ARG(M >= 0 && K > 0 && N > 0, "quantized_matmul (batched): M=%lld K=%lld N=%lld", (long long)M,
                  (long long)K, (long long)N);
    const int64_t grouped = transpose ? K : N;
    KMI_CHECK_ARG(grouped % group_size == 0,
                  "quantized_matmul (batched): the quantized axis (%lld) is not a multiple of the group %d",
                  (long long)grouped, group_size);
    KMI_CHECK_ARG(x_strides && w_strides && s_strides && (nd == 0 || batch_shape),
                  "quantized_matmul (batched): null stride array");
    for (int d = 0; d < nd; d++)
        KMI_CHECK_ARG(batch_shape[d] >= 0 && x_strides[d] >= 0 && w_strides[d] >= 0 && s_strides[d] >= 0,
                      "quantized_matmul (batched): negative batch size or stride (dimension %d)", d);
    const int64_t P = batch_count(nd, batch_shape);
    if (M == 0 || P == 0) return OK;
    KMI_CHECK_ARG(x && w && scales && (biases || mode) && y, "quantized_matmul (batched): null pointer");
    const int64_t xr = x_strides[nd], wr = w_strides[nd], sr = s_strides[nd];
    const int64_t wrow_words = grouped * bits / 32, wrows = transpose ? N : K;
    KMI_CHECK_ARG(xr >= K && xr % 8 == 0 && ((uintptr_t)x & 15) == 0,
                  "quantized_matmul (batched): x rows must be 16-byte aligned (row stride %lld)", (long long)xr);
    KMI_CHECK_ARG(wr >= wrow_words && sr >= grouped / group_size,
                  "quantized_matmul (batched): weight / scale rows overlap");
    for (int d = 0; d < nd; d++)
        KMI_CHECK_ARG(x_strides[d] % 8 == 0, "quantized_matmul (batched): x batch stride %lld not a multiple of 8",
                      (long long)x_strides[d]);
    // 32-bit buffer offsets within one batch entry
    KMI_CHECK_ARG(((M - 1) * xr + ((K + 7) & ~7LL)) * 2 < (1LL << 31) && ((wrows - 1) * wr + wrow_words) * 4 < (1LL << 31) &&
                      ((wrows - 1) * sr + grouped / group_size) * (mode ? 1 : 2) < (1LL << 31),
                  "quantized_matmul (batched): one batch entry exceeds 2 GB");
    if (transpose && (bits == 4 || bits == 8)) {
        // 16-byte (8-bit) / 8-byte (4-bit) weight loads along a row
        bool al = ((uintptr_t)w & 15) == 0 && wr % 4 == 0;
        for (int d = 0; d < nd; d++) al = al && w_strides[d] % 4 == 0;
        KMI_CHECK_ARG(al, "quantized_matmul (batched): weight rows must be 16-byte aligned");
    }
    KMI_CHECK_ARG(ldy >= N, "quantized_matmul (batched): output row stride %lld < N", (long long)ldy);
    const QbPlan q = plan_batched(P, M, K, N, bits == 4 || bits == 8);
    KMI_CHECK_ARG(q.mtiles * q.S < 65536 && P < 65536 && q.ntiles < (1LL << 31),
                  "quantized_matmul (batched): grid too large (M=%lld, batch %lld)", (long long)M, (long long)P);
    const size_t need = batched_partial_bytes(q, M, N);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need)) {
        set_error("quantized_matmul (batched): workspace of %zu bytes needed, %zu given", need, workspace_bytes);
        return EWORKSPACE;
    }
    QbArgs a = {};
    a.x = (const uint16_t*)x; a.w = w; a.s = (const uint16_t*)scales; a.b = (const uint16_t*)biases;
    a.y = (uint16_t*)y; a.partial = (float*)workspace;
    a.M = M; a.K = K; a.N = N; a.xr = xr; a.wr = wr; a.sr = sr; a.ldy = ldy;
    a.nd = nd;
    for (int d = 0; d < nd; d++) {
        a.shape[d] = batch_shape[d];
        a.xs[d] = x_strides[d];
        a.ws[d] = w_strides[d];
        a.ss[d] = s_strides[d];
    }
    a.P = P; a.mtiles = (int)q.mtiles; a.S = q.S; a.kts = q.kts;
    a.scale_x = x_scale != 1.0f;
    a.x_scale = x_scale;
    a.widx = widx; a.xidx = xidx; a.nw = nw; a.nx = nx;
    hipStream_t st = (hipStream_t)stream;
    const dim3 grid((unsigned)q.ntiles, (unsigned)(q.mtiles * q.S), (unsigned)P);
    int rc = launch_batched(a, mode, bits, group_size, transpose != 0, q.mb, grid, st);
    if (rc) return rc;
    KMI_CHECK_LAUNCH("quantized_matmul (batched)");
    if (q.S > 1) {
        const int64_t count = P * M * N;
        qmm_batched_reduce<<<(unsigned)ceil_div(count, 256), 256, 0, st>>>((const float*)workspace, q.S, count,
                                                                          N, ldy, (uint16_t*)y);
        KMI_CHECK_LAUNCH("quantized_matmul (batched) reduce");
    }
    return OK;
}

int kmi_masked_softmax(const void* x, int64_t ldx, int dtype, const int64_t* row_dims, int64_t N,
                       const void* mask, int mask_kind, const int64_t* mask_strides, void* out, int64_t ldo,
                       void* stream) {
    clear_error();
    KMI_CHECK_ARG(dtype == BF16, "masked_softmax: only bfloat16 scores are supported (got dtype %d)", dtype);
    KMI_CHECK_ARG(row_dims && N >= 0 && ldx >= N && ldo >= N, "masked_softmax: bad row shape or strides");
    KMI_CHECK_ARG(mask_kind >= KMI_MASK_NONE && mask_kind <= KMI_MASK_CAUSAL, "masked_softmax: mask kind %d",
                  mask_kind);
    int64_t R = 1;
    for (int d = 0; d < 4; d++) {
        KMI_CHECK_ARG(row_dims[d] >= 0, "masked_softmax: negative row dimension");
        R *= row_dims[d];
    }
    if (R == 0 || N == 0) return OK;
    KMI_CHECK_ARG(x && out, "masked_softmax: null pointer");
    const int64_t Np = (N + 7) & ~7LL;
    KMI_CHECK_ARG(ldx % 8 == 0 && ldo % 8 == 0 && ldx >= Np && ldo >= Np && ((uintptr_t)x & 15) == 0 &&
                      ((uintptr_t)out & 15) == 0,
                  "masked_softmax: rows must be 16-byte aligned and padded to a multiple of 8 (N=%lld, "
                  "ldx=%lld, ldo=%lld)", (long long)N, (long long)ldx, (long long)ldo);
    KMI_CHECK_ARG(R < (1LL << 31), "masked_softmax: %lld rows", (long long)R);
    SmArgs a = {};
    a.x = (const uint16_t*)x; a.ldx = ldx; a.out = (uint16_t*)out; a.ldo = ldo; a.N = N;
    a.kind = mask_kind; a.mask = mask;
    for (int d = 0; d < 4; d++) a.dims[d] = row_dims[d];
    if (mask_kind == KMI_MASK_BOOL || mask_kind == KMI_MASK_ADD) {
        KMI_CHECK_ARG(mask && mask_strides, "masked_softmax: null mask");
        for (int d = 0; d < 4; d++) {
            KMI_CHECK_ARG(mask_strides[d] >= 0, "masked_softmax: negative mask stride");
            a.ms[d] = mask_strides[d];
        }
    }
    const int64_t per_thread = ceil_div(ceil_div(N, 8), 256);
    hipStream_t st = (hipStream_t)stream;
    if (per_thread <= 1) masked_softmax_kernel<1><<<(unsigned)R, 256, 0, st>>>(a);
    else if (per_thread <= 2) masked_softmax_kernel<2><<<(unsigned)R, 256, 0, st>>>(a);
    else if (per_thread <= 4) masked_softmax_kernel<4><<<(unsigned)R, 256, 0, st>>>(a);
    else if (per_thread <= 8) masked_softmax_kernel<8><<<(unsigned)R, 256, 0, st>>>(a);
    else if (per_thread <= 16) masked_softmax_kernel<16><<<(unsigned)R, 256, 0, st>>>(a);
    else masked_softmax_kernel<0><<<(unsigned)R, 256, 0, st>>>(a);
    KMI_CHECK_LAUNCH("masked_softmax");
    return OK;
}

}  // extern "C"
