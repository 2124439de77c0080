// Skinny quantized matmul for gfx950: up to 64 activation rows against an
// affine-quantized weight (mlx layout: packed uint32 codes, per-group bf16
// scales and biases), dense or per routed expert -- the decode / verify /
// grouped-expert shapes of mx.quantized_matmul and mx.gather_qmm
// (called from nn.QuantizedLinear, src/knurlogic/engine/model/load_model.py:124-144,
// and QuantizedSwitchLinear, .../_mlx_vlm/models/switch_layers.py:71-86).
//
//   y[m, n] = sum_g ( s[n, g] * P[m, n, g] + b[n, g] * X[m, g] )
//   P[m, n, g] = sum_{k in g} x[m, k] q[n, k],   X[m, g] = sum_{k in g} x[m, k]
//
// A workgroup owns 64 weight rows (16 per wave: the columns n of
// v_mfma_f32_16x16x32_bf16) and walks K in chunks of 256 codes.  Each chunk
// is staged through LDS with fully coalesced loads (a wave instruction reads
// 4-8 weight rows x 128-256 contiguous bytes, or 2 x rows x 512 bytes), two
// chunks ahead in registers; the waves then read MFMA fragments from LDS.
// (Loading fragments straight from global memory puts 16 rows in every
// instruction and is bound by L1 tag lookups, not by HBM.)
//
// Codes become bf16 without rounding (integers < 256), so P is a plain
// MFMA with fp32 accumulation and the scale one FMA per output per group.
// X is summed while x is staged (bf16 dot products with ones, then across
// the lanes holding a group's pieces) into a small LDS table, and the
// bias term sum_g b[n, g] X[m, g] of a chunk is one fp32 MFMA
// (v_mfma_f32_16x16x4_f32) per 4 groups into the same accumulators.  The
// only rounding is fp32 accumulation and the final bf16.  A row's
// arithmetic is the same at any number of rows.
//
// 4-bit codes decode 8 per 7 instructions into the k order
// [0,2,4,6,1,3,5,7] (low nibbles, then high nibbles, of each byte), and x is
// stored to LDS in that order within each run of 8, so A and B agree.
#include "qgemv.hpp"
#include "../../include/knurlogic_amd.h"

namespace kmi {

constexpr int QG_KC = 256;      // codes per K chunk
constexpr int QG_ROWS = 64;     // weight rows per workgroup

// Eight 4-bit codes (code i in bits 4i..4i+3) -> eight exact bf16 in the
// order [0,2,4,6,1,3,5,7].  A byte q in 0..15 read as fp8 e4m3 is exactly
// q * 2^-9 (bytes 0..7 are the subnormals m * 2^-9, bytes 8..15 the first
// binade (8+m) * 2^-9), and the conversion's power-of-two scale 2^9 is
// exact: bf16(q).
__device__ __forceinline__ u32x4 nib8_exact(uint32_t w) {
    const uint32_t lo = w & 0x0F0F0F0Fu;            // codes 0, 2, 4, 6
    const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;     // codes 1, 3, 5, 7
    u32x4 r;
    r.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 512.f, false));
    r.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 512.f, true));
    r.z = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 512.f, false));
    r.w = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 512.f, true));
    return r;
}

// 8 bf16 of x (k order 0..7) -> the order [0,2,4,6,1,3,5,7]
__device__ __forceinline__ u32x4 x8_to_nibble_order(u32x4 v) {
    return u32x4{__builtin_amdgcn_perm(v.y, v.x, 0x05040100u), __builtin_amdgcn_perm(v.w, v.z, 0x05040100u),
                 __builtin_amdgcn_perm(v.y, v.x, 0x07060302u), __builtin_amdgcn_perm(v.w, v.z, 0x07060302u)};
}

__device__ __forceinline__ float qg_bf16r(float v) { return bf16_to_f32(f32_to_bf16(v)); }

// E8M0 scale byte (held in a 16-bit LDS slot): 2^(e - 127); 255 is NaN
__device__ __forceinline__ float mx_scale_qg(uint32_t e) { return e8m0_to_f32(e); }

__device__ __forceinline__ float qg_f32_kept(double v) {
    float f = (float)v;
    asm volatile("" : "+v"(f));   // keep the float32 rounding (no fused f64 -> bf16 rounding)
    return f;
}

template <int BITS, int NSET, int MC>
struct QgShape {
    static constexpr int MT = 16 * MC;                   // activation rows per tile
    static constexpr int RB = QG_KC * BITS / 8;          // weight bytes per row per chunk
    static constexpr int WST = RB + 16;                  // LDS row stride of the weights
    static constexpr int XST = QG_KC * 2 + 16;           // LDS row stride of x
    static constexpr int WPIECES = RB / 16;              // 16-byte pieces per weight row
    static constexpr int WPASS = QG_ROWS * WPIECES / 256;
    static constexpr int XPASS = MT / 8;                 // 32 pieces per x row, 8 rows per pass
    static constexpr size_t W_BYTES = (size_t)NSET * QG_ROWS * WST;
    static constexpr size_t X_BYTES = (size_t)MT * XST;
};

template <int BITS, int GS, int NSET, int MC>
constexpr size_t qg_lds_bytes() {
    using S = QgShape<BITS, NSET, MC>;
    return 2 * (S::W_BYTES + S::X_BYTES + (size_t)2 * NSET * QG_ROWS * (QG_KC / GS) * 2 +
                (size_t)(QG_KC / GS) * S::MT * 4);
}

// MX: microscaled codes (GS 32): the codes convert to bf16 exactly (E2M1,
// E4M3), natural k order, one E8M0 scale per group and no bias term.
template <int BITS, int GS, int MC, bool GLU, bool MX>
__global__ __launch_bounds__(256) void qgemv_kernel(QgArgs a) {
    constexpr int NSET = GLU ? 2 : 1;
    constexpr int SB = MX ? 1 : 2;                       // bytes per scale
    using S = QgShape<BITS, NSET, MC>;
    constexpr int MT = S::MT, RB = S::RB, WST = S::WST, XST = S::XST;
    constexpr int WPIECES = S::WPIECES, WPASS = S::WPASS, XPASS = S::XPASS;
    constexpr int GPC = QG_KC / GS;                      // groups per chunk
    constexpr int SPT = (QG_ROWS * GPC + 255) / 256;     // scale loads per thread
    constexpr int RUN = GS / 4;                          // codes per lane per group
    constexpr int LB = RUN * BITS / 8;                   // bytes per lane per group
    constexpr int NT = GS / 32;                          // MFMAs per group per chunk and set
    extern __shared__ __align__(16) unsigned char smem[];
    auto Wl = [&](int buf, int set) { return smem + buf * S::W_BYTES + set * (S::W_BYTES / NSET); };
    unsigned char* xbase = smem + 2 * S::W_BYTES;
    auto Xl = [&](int buf) { return xbase + buf * S::X_BYTES; };
    uint16_t* sbase = (uint16_t*)(xbase + 2 * S::X_BYTES);
    auto Sl = [&](int buf, int set, int which) {       // which: 0 scales, 1 biases
        return sbase + ((buf * NSET + set) * 2 + which) * (QG_ROWS * GPC);
    };
    // X[g][m]: the sum of tile row m's x over group g of the chunk (affine)
    float* xtbase = (float*)(sbase + 2 * NSET * 2 * (QG_ROWS * GPC));
    auto Xt = [&](int buf) { return xtbase + buf * (GPC * MT); };

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nl = lane & 15, j4 = lane >> 4;

    int expert = 0;
    int64_t start, count;
    if (a.tiles) {
        const int32_t* tp = a.tiles + 3 * (int64_t)blockIdx.z;
        count = tp[2];
        expert = tp[0];
        start = tp[1];
        if (count <= 0 || expert < 0 || expert >= a.E) return;
    } else {
        start = (int64_t)blockIdx.z * a.tm;
        count = a.rows - start;
        if (count > a.tm) count = a.tm;
        if (count <= 0) return;
    }

    const int64_t K = a.K, G = K / GS;
    const int64_t rowbytes = K * BITS / 8;
    const int64_t n0 = (int64_t)blockIdx.x * QG_ROWS;
    __amdgpu_buffer_rsrc_t rw[NSET], rs[NSET], rb[NSET];
#pragma unroll
    for (int set = 0; set < NSET; set++) {
        const int64_t r0 = (int64_t)expert * a.erows + (set ? a.up_off : 0);
        rw[set] = make_rsrc((const char*)a.w + r0 * rowbytes, a.N * rowbytes);
        rs[set] = make_rsrc((const char*)a.s + r0 * G * SB, a.N * G * SB);
        rb[set] = make_rsrc((const char*)a.b + r0 * G * SB, MX ? 0 : a.N * G * SB);
    }
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, a.xrows * K * 2);
    const __amdgpu_buffer_rsrc_t rz = make_rsrc(a.x, 0);

    // per-thread staging coordinates (rows past N / past the tile read zeros)
    uint32_t woff[WPASS];          // weight row base + piece, chunk 0
#pragma unroll
    for (int p = 0; p < WPASS; p++) {
        const int64_t row = n0 + p * (256 / WPIECES) + tid / WPIECES;
        woff[p] = row < a.N ? (uint32_t)(row * rowbytes) + 16u * (tid % WPIECES) : 0x80000000u;
    }
    const int wk = (tid % WPIECES) * 16 * 8 / BITS;     // first code of this thread's weight piece
    // x row of each staged row (row ids, pairs and x rows all < 2^31, checked
    // on the host, so 32-bit arithmetic; the divisions by one are skipped)
    const uint32_t mper = (uint32_t)a.Mper, ldiv = (uint32_t)a.lhs_div;
    // and the output row id of each tile row (-1 past the tile) into LDS,
    // for the epilogue
    __shared__ int32_t orow_s[XPASS * 8];
    uint32_t xoff[XPASS];
#pragma unroll
    for (int p = 0; p < XPASS; p++) {
        const int r = p * 8 + tid / 32;
        xoff[p] = 0x80000000u;
        if (tid % 32 == 0) orow_s[r] = r < count ? (a.sorted ? a.sorted[start + r] : (int32_t)(start + r)) : -1;
        if (r < count) {
            const uint32_t rid = a.sorted ? (uint32_t)a.sorted[start + r] : (uint32_t)(start + r);
            const uint32_t pr = mper == 1 ? rid : rid / mper;
            const uint32_t xb = a.lhs ? (uint32_t)a.lhs[pr] : (ldiv == 1 ? pr : pr / ldiv);
            const uint32_t xr = xb * mper + (rid - pr * mper);
            if (xr < (uint64_t)a.xrows) xoff[p] = (uint32_t)((uint64_t)xr * K * 2) + 16u * (tid % 32);
        }
    }
    const int xk = (tid % 32) * 8;                       // first k of this thread's x piece

    const int64_t chunks = (K + QG_KC - 1) / QG_KC;
    const int64_t c0 = (int64_t)blockIdx.y * a.gps;
    int64_t c1 = c0 + a.gps;
    if (c1 > chunks) c1 = chunks;
    const int nc = c1 > c0 ? (int)(c1 - c0) : 0;

    // register ring: D chunks of staging loads in flight (4 measured no
    // faster than 2, at twice the registers)
    constexpr int D = 2;
    u32x4 rwv[D][NSET][WPASS], rxv[D][XPASS];
    uint32_t rsv[D][NSET][SPT], rbv[D][NSET][SPT];
    auto issue = [&](int slot, int i) {
        const bool live = i < nc;
        const int64_t kc0 = (c0 + (live ? i : 0)) * QG_KC;     // first code of the chunk
        const bool wk_ok = kc0 + wk < K;
        const bool xk_ok = kc0 + xk < K;
#pragma unroll
        for (int set = 0; set < NSET; set++)
#pragma unroll
            for (int p = 0; p < WPASS; p++)
                rwv[slot][set][p] = __builtin_amdgcn_raw_buffer_load_b128(
                    live ? rw[set] : rz, (int)(wk_ok ? woff[p] + (uint32_t)(kc0 * BITS / 8) : 0x80000000u), 0, 0);
#pragma unroll
        for (int set = 0; set < NSET; set++)
#pragma unroll
            for (int q = 0; q < SPT; q++) {
                const int idx = tid + 256 * q;
                const int64_t row = n0 + idx / GPC, g = kc0 / GS + idx % GPC;
                const bool ok = idx < QG_ROWS * GPC && row < a.N && g < G;
                const int off = ok ? (int)((row * G + g) * SB) : (int)0x80000000u;
                if constexpr (MX) {
                    rsv[slot][set][q] = __builtin_amdgcn_raw_buffer_load_b8(live ? rs[set] : rz, off, 0, 0);
                    rbv[slot][set][q] = 0u;
                } else {
                    rsv[slot][set][q] = __builtin_amdgcn_raw_buffer_load_b16(live ? rs[set] : rz, off, 0, 0);
                    rbv[slot][set][q] = __builtin_amdgcn_raw_buffer_load_b16(live ? rb[set] : rz, off, 0, 0);
                }
            }
#pragma unroll
        for (int p = 0; p < XPASS; p++)
            rxv[slot][p] = __builtin_amdgcn_raw_buffer_load_b128(
                live ? rx : rz, (int)(xk_ok ? xoff[p] + (uint32_t)(kc0 * 2) : 0x80000000u), 0, 0);
    };
    auto store = [&](int slot, int buf) {
#pragma unroll
        for (int set = 0; set < NSET; set++)
#pragma unroll
            for (int p = 0; p < WPASS; p++)
                *(u32x4*)(Wl(buf, set) + (p * (256 / WPIECES) + tid / WPIECES) * WST + 16 * (tid % WPIECES)) =
                    rwv[slot][set][p];
#pragma unroll
        for (int set = 0; set < NSET; set++)
#pragma unroll
            for (int q = 0; q < SPT; q++) {
                const int idx = tid + 256 * q;
                if (idx < QG_ROWS * GPC) {
                    Sl(buf, set, 0)[idx] = (uint16_t)rsv[slot][set][q];
                    Sl(buf, set, 1)[idx] = (uint16_t)rbv[slot][set][q];
                }
            }
#pragma unroll
        for (int p = 0; p < XPASS; p++) {
            u32x4 v = rxv[slot][p];
            if constexpr (!MX) {
                // the piece's 8 values summed (dot products with ones), then
                // over the GS / 8 consecutive lanes holding the group's pieces
                typedef __bf16 qg_bf2 __attribute__((ext_vector_type(2)));
                const qg_bf2 one = __builtin_bit_cast(qg_bf2, 0x3F803F80u);
                // (each element copied to a scalar first: a bit cast of a vector
                // element v[e] reads element 0 in this compiler)
                const uint32_t ve[4] = {v.x, v.y, v.z, v.w};
                float ps = 0.f;
#pragma unroll
                for (int e = 0; e < 4; e++) ps = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(qg_bf2, ve[e]), one, ps, false);
                ps += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(ps), 0xb1, 0xf, 0xf, false));  // lane ^ 1
                ps += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(ps), 0x4e, 0xf, 0xf, false));  // lane ^ 2
                if constexpr (GS >= 64)
                    ps += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(ps), 0x141, 0xf, 0xf, false));  // 8-lane mirror
                if constexpr (GS >= 128)
                    ps += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(ps), 0x140, 0xf, 0xf, false));  // 16-lane mirror
                if (tid % (GS / 8) == 0) Xt(buf)[((tid % 32) / (GS / 8)) * MT + p * 8 + tid / 32] = ps;
            }
            if constexpr (BITS == 4 && !MX) v = x8_to_nibble_order(v);
            *(u32x4*)(Xl(buf) + (p * 8 + tid / 32) * XST + 16 * (tid % 32)) = v;
        }
    };

    f32x4 acc[NSET][MC];
#pragma unroll
    for (int set = 0; set < NSET; set++)
#pragma unroll
        for (int c = 0; c < MC; c++) acc[set][c] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int wr = wave * 16 + nl;                       // this lane's weight row in the tile

    // groups unrolled UF at a time: their LDS reads, decodes and MFMA chains
    // overlap; fully unrolled at larger tiles the scheduler hoists every
    // group's fragments and the register file overflows
    constexpr int UF0 = 4 / (MC * NSET) > 0 ? 4 / (MC * NSET) : 1;
    constexpr int UF = UF0 < GPC ? UF0 : GPC;
    auto compute = [&](int buf) {
        // affine: the chunk's bias term sum_g b * X, one fp32 MFMA per 4
        // groups (lane (n, j4): X of tile row n and the bias of weight row
        // n, at group 4 q + j4)
        if constexpr (!MX) {
#pragma unroll
            for (int q = 0; q < (GPC + 3) / 4; q++) {
                const int gq = 4 * q + j4;
                const bool ok = gq < GPC;
                float xa[MC];
#pragma unroll
                for (int c = 0; c < MC; c++) xa[c] = ok ? Xt(buf)[gq * MT + 16 * c + nl] : 0.f;
#pragma unroll
                for (int set = 0; set < NSET; set++) {
                    const float bv = ok ? bf16_to_f32(Sl(buf, set, 1)[wr * GPC + gq]) : 0.f;
#pragma unroll
                    for (int c = 0; c < MC; c++)
                        acc[set][c] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[c], bv, acc[set][c], 0, 0, 0);
                }
            }
        }
#pragma unroll UF
        for (int gi = 0; gi < GPC; gi++) {
            u32x4 B[NSET][NT];
            float sc[NSET];
#pragma unroll
            for (int set = 0; set < NSET; set++) {
                const unsigned char* wp = Wl(buf, set) + wr * WST + gi * (GS * BITS / 8) + j4 * LB;
                uint32_t wv[LB / 4];
                if constexpr (LB == 4) {
                    wv[0] = *(const uint32_t*)wp;
                } else if constexpr (LB == 8) {
                    const u32x2 t = *(const u32x2*)wp;
                    wv[0] = t.x; wv[1] = t.y;
                } else {
#pragma unroll
                    for (int q = 0; q < LB / 4; q += 4) {
                        const u32x4 t = *(const u32x4*)(wp + 4 * q);
                        wv[q] = t.x; wv[q + 1] = t.y; wv[q + 2] = t.z; wv[q + 3] = t.w;
                    }
                }
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    if constexpr (MX && BITS == 4) {          // 8 E2M1 codes, natural order
                        const uint32_t w = wv[t];
                        B[set][t] = u32x4{
                            __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.f, 0)),
                            __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.f, 1)),
                            __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.f, 2)),
                            __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.f, 3))};
                    } else if constexpr (MX) {                // 8 E4M3 codes
                        const uint32_t w0 = wv[2 * t], w1 = wv[2 * t + 1];
                        B[set][t] = u32x4{
                            __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.f, false)),
                            __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.f, true)),
                            __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.f, false)),
                            __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.f, true))};
                    } else if constexpr (BITS == 4) {
                        B[set][t] = nib8_exact(wv[t]);
                    } else {
                        B[set][t] = u32x4{bytes_to_bf16x2(wv[2 * t], 0), bytes_to_bf16x2(wv[2 * t], 2),
                                          bytes_to_bf16x2(wv[2 * t + 1], 0), bytes_to_bf16x2(wv[2 * t + 1], 2)};
                    }
                }
                if constexpr (MX) sc[set] = mx_scale_qg(Sl(buf, set, 0)[wr * GPC + gi]);
                else sc[set] = bf16_to_f32(Sl(buf, set, 0)[wr * GPC + gi]);
            }
#pragma unroll
            for (int c = 0; c < MC; c++) {
                f32x4 P[NSET];
#pragma unroll
                for (int set = 0; set < NSET; set++) P[set] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    const u32x4 A = *(const u32x4*)(Xl(buf) + (16 * c + nl) * XST + (gi * GS + j4 * RUN + 8 * t) * 2);
#pragma unroll
                    for (int set = 0; set < NSET; set++) P[set] = mfma16x16x32(A, B[set][t], P[set]);
                }
#pragma unroll
                for (int set = 0; set < NSET; set++)
#pragma unroll
                    for (int e = 0; e < 4; e++) acc[set][c][e] = __builtin_fmaf(sc[set], P[set][e], acc[set][c][e]);
            }
        }
    };

    // Chunk j sits in ring slot j % D, then in LDS buffer j % 2.  A step
    // reissues the slot just stored (chunk j + D), computes chunk j, and
    // stores chunk j + 1; steps run D at a time so slots are compile-time.  A
    // chunk past the end reads zeros everywhere and adds nothing.
#pragma unroll
    for (int d = 0; d < D; d++) {
        issue(d, d);
        __builtin_amdgcn_sched_barrier(0);
    }
    store(0, 0);
    lds_barrier();
    for (int i = 0; i < nc; i += D) {
#pragma unroll
        for (int d = 0; d < D; d++) {
            issue(d, i + d + D);
            __builtin_amdgcn_sched_barrier(0);
            compute(d & 1);
            __builtin_amdgcn_sched_barrier(0);
            store((d + 1) % D, (d + 1) & 1);
            lds_barrier();
        }
    }

    // Stored through a buffer view of y (or of this split's partials): 32-bit
    // offsets from the row ids, a row past the tile or a column past N at an
    // offset past the view (no branch); rows e and e + 1 of a lane share one
    // v_cvt_pk_bf16_f32.
    const int64_t n = n0 + wr;
    const bool nok = n < a.N;
    if (GLU || a.S == 1) {
        const __amdgpu_buffer_rsrc_t ry = make_rsrc(a.y, a.rows * a.N * 2);
        const uint32_t rowb = (uint32_t)a.N * 2, colb = (uint32_t)n * 2;
#pragma unroll
        for (int c = 0; c < MC; c++)
#pragma unroll
            for (int e = 0; e < 4; e += 2) {
                float v0, v1;
                if constexpr (GLU) {
                    // act = round(round(silu_f32(round(gate))) * round(up))
                    v0 = silu_bf16r(qg_bf16r(acc[0][c][e])) * qg_bf16r(acc[1][c][e]);
                    v1 = silu_bf16r(qg_bf16r(acc[0][c][e + 1])) * qg_bf16r(acc[1][c][e + 1]);
                } else {
                    v0 = acc[0][c][e];
                    v1 = acc[0][c][e + 1];
                }
                const uint32_t v = cvt_pk_bf16(v0, v1);
                const int32_t r0 = orow_s[16 * c + 4 * j4 + e], r1 = orow_s[16 * c + 4 * j4 + e + 1];
                const uint32_t o0 = nok && r0 >= 0 ? (uint32_t)r0 * rowb + colb : 0x80000000u;
                const uint32_t o1 = nok && r1 >= 0 ? (uint32_t)r1 * rowb + colb : 0x80000000u;
                __builtin_amdgcn_raw_buffer_store_b16((uint16_t)v, ry, (int)o0, 0, 0);
                __builtin_amdgcn_raw_buffer_store_b16((uint16_t)(v >> 16), ry, (int)o1, 0, 0);
            }
    } else {
        const __amdgpu_buffer_rsrc_t rp =
            make_rsrc(a.partial + (int64_t)blockIdx.y * a.rows * a.N, a.rows * a.N * 4);
        const uint32_t rowb = (uint32_t)a.N * 4, colb = (uint32_t)n * 4;
#pragma unroll
        for (int c = 0; c < MC; c++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int32_t r = orow_s[16 * c + 4 * j4 + e];
                const uint32_t o = nok && r >= 0 ? (uint32_t)r * rowb + colb : 0x80000000u;
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc[0][c][e]), rp, (int)o, 0, 0);
            }
    }
}

// ---- host side ----------------------------------------------------------------

QgPlan plan_qgemv(int64_t N, int64_t K, int64_t tiles, int tile_rows, int gs) {
    (void)gs;
    QgPlan p;
    p.mc = tile_rows <= 16 ? 1 : tile_rows <= 32 ? 2 : 4;
    const int64_t chunks = ceil_div(K, QG_KC);
    const int64_t wgs = ceil_div(N, QG_ROWS) * (tiles > 0 ? tiles : 1);
    // K splits only while the grid is short of 2 workgroups per CU and each
    // split keeps >= 8 chunks.  Depends on the shape and tile count only.
    int64_t S = 1;
    while (wgs * S < 512 && chunks / (S * 2) >= 8) S *= 2;
    p.S = (int)S;
    p.gps = (int)ceil_div(chunks, S);
    return p;
}

int qgemv_gather_tile_rows(int64_t avg_rows) {
    // routed rows per expert spread around their mean (roughly binomial), so
    // the tile covers about 1.5x the mean
    return avg_rows <= 10 ? 16 : avg_rows <= 20 ? 32 : 64;
}

QgPlan plan_qgemv_unsplit(int64_t N, int64_t K, int64_t tiles, int tile_rows, int gs) {
    QgPlan p = plan_qgemv(N, K, tiles, tile_rows, gs);
    p.S = 1;
    p.gps = (int)ceil_div(K, QG_KC);
    return p;
}

template <int B_, int G_, int M_, bool L_, bool X_>
static int launch_one(const QgArgs& a, dim3 grid, hipStream_t st) {
    constexpr size_t lds = qg_lds_bytes<B_, G_, L_ ? 2 : 1, M_>();
    static_assert(lds <= 160 * 1024, "qgemv tile exceeds the LDS");
    allow_dynamic_lds_once((const void*)qgemv_kernel<B_, G_, M_, L_, X_>);
    qgemv_kernel<B_, G_, M_, L_, X_><<<grid, 256, lds, st>>>(a);
    return OK;
}

#define KMI_QG_CASE(B_, G_, M_, L_)                                                                   \
    if (!a.mx && bits == B_ && gs == G_ && p.mc == M_ && glu == L_) return launch_one<B_, G_, M_, L_, false>(a, grid, st);
#define KMI_QG_MXC(B_, M_, L_)                                                                        \
    if (a.mx && bits == B_ && gs == 32 && p.mc == M_ && glu == L_) return launch_one<B_, 32, M_, L_, true>(a, grid, st);
#define KMI_QG_M(B_, G_, L_) KMI_QG_CASE(B_, G_, 1, L_) KMI_QG_CASE(B_, G_, 2, L_) KMI_QG_CASE(B_, G_, 4, L_)
#define KMI_QG_G(B_, L_) KMI_QG_M(B_, 32, L_) KMI_QG_M(B_, 64, L_) KMI_QG_M(B_, 128, L_)

int launch_qgemv(const QgArgs& a, const QgPlan& p, int bits, int gs, bool glu, int64_t ntiles,
                 hipStream_t st) {
    if (glu && p.S != 1) {
        set_error("qgemv: the SwiGLU epilogue needs an unsplit K");
        return EINVAL_ARG;
    }
    if (a.rows * a.N * (p.S > 1 ? 4 : 2) >= (1LL << 31)) {
        set_error("qgemv: an output (or a split's partials) past 2 GiB");
        return EINVAL_ARG;
    }
    const dim3 grid((unsigned)ceil_div(a.N, QG_ROWS), (unsigned)p.S, (unsigned)ntiles);
    KMI_QG_G(4, false) KMI_QG_G(8, false) KMI_QG_G(4, true) KMI_QG_G(8, true)
    KMI_QG_MXC(4, 1, false) KMI_QG_MXC(4, 2, false) KMI_QG_MXC(4, 4, false)
    KMI_QG_MXC(4, 1, true) KMI_QG_MXC(4, 2, true) KMI_QG_MXC(4, 4, true)
    KMI_QG_MXC(8, 1, false) KMI_QG_MXC(8, 2, false) KMI_QG_MXC(8, 4, false)
    KMI_QG_MXC(8, 1, true) KMI_QG_MXC(8, 2, true) KMI_QG_MXC(8, 4, true)
    set_error("qgemv: no kernel for bits=%d gs=%d mc=%d", bits, gs, p.mc);
    return EINVAL_ARG;
}

#undef KMI_QG_G
#undef KMI_QG_M
#undef KMI_QG_CASE
#undef KMI_QG_MXC

}  // namespace kmi
