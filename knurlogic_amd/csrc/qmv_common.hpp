// Shared declarations of the decode-shape quantized matmul kernels.
#pragma once

#include "common.hpp"

namespace kmi {

struct QmvArgs {
    const uint16_t* x;        // activations (bf16), [X rows, K]
    const uint32_t* w;        // [E, N, K*bits/32]
    const uint16_t* s;        // [E, N, K/gs]
    const uint16_t* b;        // [E, N, K/gs]
    uint16_t* y;              // [rows, N] (bf16), when S == 1
    float* partial;           // [S, rows, N], when S > 1
    int64_t K, N;
    int64_t rows;             // rows of y
    int64_t KS;               // K slice length (multiple of the group), qmv_mfma only
    int S;                    // number of K slices, qmv_mfma only
    int tile_m;               // rows per dense tile
    int gs_shift;             // log2(group size)
    // gather (all null for a dense call: tile z = rows [tile_m*z, +tile_m))
    const int32_t* tiles;     // [max_tiles][3]: expert, start, count (count 0 = unused)
    const int32_t* sorted;    // [rows] row ids grouped by expert
    const int32_t* lhs;       // [P] x batch index per pair
    int64_t Mper;             // rows per pair (x [X, Mper, K])
    int64_t Xrows;            // X * Mper: rows of x, for bounds
    int mx;                   // 1: OCP microscaled codes (E2M1 at 4 bits, E4M3 at 8), uint8
                              // E8M0 scales per 32 inputs in s, no biases (gs_shift 5)
};

struct Tile {
    int expert;
    int64_t start, count;
};

__device__ __forceinline__ bool resolve_tile(const QmvArgs& a, Tile& t) {
    if (a.tiles) {
        const int32_t* p = a.tiles + 3 * (int64_t)blockIdx.z;
        t.count = p[2];
        if (t.count <= 0) return false;
        t.expert = p[0];
        t.start = p[1];
    } else {
        t.expert = 0;
        t.start = (int64_t)blockIdx.z * a.tile_m;
        t.count = a.rows - t.start;
        if (t.count > a.tile_m) t.count = a.tile_m;
        if (t.count <= 0) return false;
    }
    return true;
}

__device__ __forceinline__ int64_t x_row_of(const QmvArgs& a, int64_t row) {
    if (!a.sorted) return row;
    const int64_t rid = a.sorted[row];
    const int64_t p = rid / a.Mper;
    return (int64_t)a.lhs[p] * a.Mper + (rid - p * a.Mper);
}

__device__ __forceinline__ int64_t y_row_of(const QmvArgs& a, int64_t row) {
    return a.sorted ? (int64_t)a.sorted[row] : row;
}

// Position of element e of an 8-run in LDS so one 16-byte read gives the
// pairs the 4-bit unpack produces: (e, e+4) for e = 0..3.
template <int BITS>
__device__ __forceinline__ int lds_perm(int k) {
    if (BITS == 4) {
        const int e = k & 7;
        return (k & ~7) | ((e & 3) << 1) | (e >> 2);
    }
    return k;
}

// Permute 8 bf16 of x for the unpack order; add their fp32 values to sum.
template <int BITS>
__device__ __forceinline__ u32x4 permute8(u32x4 v, float& sum) {
    uint16_t e[8], o[8];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        e[2 * i] = (uint16_t)(v[i] & 0xffffu);
        e[2 * i + 1] = (uint16_t)(v[i] >> 16);
    }
#pragma unroll
    for (int i = 0; i < 8; i++) {
        o[lds_perm<BITS>(i)] = e[i];
        sum += bf16_to_f32(e[i]);
    }
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; i++) r[i] = (uint32_t)o[2 * i] | ((uint32_t)o[2 * i + 1] << 16);
    return r;
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                           __builtin_bit_cast(bf16x2_t, b), c, false);
}

// Sum over the 64 lanes of a wave with DPP moves (no LDS round trips):
// quad swaps, half-row and row mirrors give every lane its 16-lane row sum,
// then row broadcasts 15 and 31 carry the row sums up to lane 63.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add(float v) {
    return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}

__device__ __forceinline__ float wave_sum(float v) {
    v = dpp_add<0xb1, 0xf>(v);    // quad_perm [1,0,3,2]
    v = dpp_add<0x4e, 0xf>(v);    // quad_perm [2,3,0,1]
    v = dpp_add<0x141, 0xf>(v);   // row_half_mirror
    v = dpp_add<0x140, 0xf>(v);   // row_mirror
    v = dpp_add<0x142, 0xa>(v);   // row_bcast:15 into rows 1 and 3
    v = dpp_add<0x143, 0xc>(v);   // row_bcast:31 into rows 2 and 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}


// ---- fp16 "1024 + q" decode shared by the VALU decode kernels -------------
// A code becomes fp16 1024 + q with one v_and_or_b32 per pair: a low nibble
// (or a byte) lands in the low mantissa bits of 0x6400 = 1024.0, and a high
// nibble is left in place as 1024 + 16 q, also exact (fp16 has 10 mantissa
// bits).  x is staged as fp16 with a power-of-two scale per 16-byte weight
// chunk (the chunk's largest |x| maps to [2^14, 2^15)), exact for every bf16
// value, with the chunk's {scale, correction, sum} beside it, so that
//   chunk_qx = scale * (A_lo + A_hi / 16) - correction = sum(q x) over the chunk.

typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

// A constant kept in a VGPR.  Held in a register (not an instruction
// literal), a mask-and-or pair folds into one v_and_or_b32.
__device__ __forceinline__ uint32_t vconst(uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}

__device__ __forceinline__ float fdot2_f16(uint32_t x, uint32_t w, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, x), __builtin_bit_cast(f16x2_t, w), c, false);
}

__device__ __forceinline__ uint32_t pk_f16(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
}

template <int CTRL>
__device__ __forceinline__ float dpp_max(float v) {
    return fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false)));
}

constexpr uint32_t QV_NONE = 0x80000000u;   // a buffer offset past every buffer: reads 0

// Piece p (x[8p .. 8p+8)) of a row -> xs [XV][C] 16-byte fp16 slots and the
// chunk record xm [C] = {scale, correction, sum}.  Every lane of the wave runs
// this (the quad reductions read neighbours); only pieces p < P store.
// NAT: every dword holds the natural pair (x_2i, x_2i+1) (the microscaled
// decode's order; 8-bit chunks use it anyway), and the correction is 0.
template <int BITS, bool NAT = false>
__device__ __forceinline__ void stage_x16(int p, u32x4 raw, int P, int C, u32x4* xs, float4* xm) {
    constexpr int XV = (128 / BITS) / 8;            // pieces per chunk: 4 or 2
    float f[8];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        f[2 * i] = __uint_as_float(raw[i] << 16);
        f[2 * i + 1] = __uint_as_float(raw[i] & 0xffff0000u);
    }
    float am = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) am = fmaxf(am, fabsf(f[i]));
    am = dpp_max<0xb1>(am);                           // quad_perm [1,0,3,2]
    if constexpr (XV == 4) am = dpp_max<0x4e>(am);    // quad_perm [2,3,0,1]
    int e = (int)((__float_as_uint(am) >> 23) & 0xffu);
    e = e < 15 ? 15 : e;
    const float mult = __uint_as_float((uint32_t)(e - 14) << 23);   // 2^(e-141)
    const float inv = __uint_as_float((uint32_t)(268 - e) << 23);   // 2^(141-e)
    u32x4 o;
    float lo, hi = 0.f;
    if constexpr (BITS == 4 && !NAT) {
        // dword i pairs (x_i, x_{i+4}): the codes one and-or places there
#pragma unroll
        for (int i = 0; i < 4; i++) o[i] = pk_f16(f[i] * inv, f[i + 4] * inv);
        lo = (f[0] + f[2]) + (f[4] + f[6]);           // under low nibbles
        hi = (f[1] + f[3]) + (f[5] + f[7]);           // under high nibbles
    } else {
#pragma unroll
        for (int i = 0; i < 4; i++) o[i] = pk_f16(f[2 * i] * inv, f[2 * i + 1] * inv);
        lo = ((f[0] + f[1]) + (f[2] + f[3])) + ((f[4] + f[5]) + (f[6] + f[7]));
    }
    lo = dpp_add<0xb1, 0xf>(lo);
    if constexpr (XV == 4) lo = dpp_add<0x4e, 0xf>(lo);
    if constexpr (BITS == 4) {
        hi = dpp_add<0xb1, 0xf>(hi);
        hi = dpp_add<0x4e, 0xf>(hi);
    }
    if (p < P) {
        const int c = p / XV, v = p % XV;
        xs[v * C + c] = o;
        if (v == 0) {
            const float corr = NAT ? 0.f : BITS == 4 ? 1024.f * __builtin_fmaf(hi, 0.0625f, lo) : 1024.f * lo;
            xm[c] = make_float4(mult, corr, lo + hi, 0.f);
        }
    }
}

// ---- OCP microscaled chunks (mxfp4: E2M1, mxfp8: E4M3) ---------------------
// A 16-byte chunk is 32 E2M1 or 16 E4M3 codes in mlx's packing (element j
// at bits BITS*j); every element converts to fp16 exactly (the conversion's
// scale is 1.0), and the chunk's dot with its x pieces (staged NAT) is
// v_dot2_f32_f16 on natural pairs.  The E8M0 group scale (per 32 elements)
// is applied by the caller.
template <int BITS>
__device__ __forceinline__ float chunk_mx(const u32x4& W, const u32x4* xv, const float4& m) {
    float A = 0.f, B = 0.f;
    if constexpr (BITS == 4) {
#pragma unroll
        for (int wd = 0; wd < 4; wd++) {
            const uint32_t w = W[wd];
            A = fdot2_f16(xv[wd][0], __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.f, 0)), A);
            B = fdot2_f16(xv[wd][1], __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.f, 1)), B);
            A = fdot2_f16(xv[wd][2], __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.f, 2)), A);
            B = fdot2_f16(xv[wd][3], __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.f, 3)), B);
        }
    } else {
#pragma unroll
        for (int wd = 0; wd < 4; wd++) {
            const uint32_t w = W[wd];
            A = fdot2_f16(xv[wd >> 1][(wd & 1) * 2],
                          __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.f, false)), A);
            B = fdot2_f16(xv[wd >> 1][(wd & 1) * 2 + 1],
                          __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.f, true)), B);
        }
    }
    return m.x * (A + B);
}

// E8M0 scale byte: 2^(e - 127); 255 is NaN
__device__ __forceinline__ float mx_scale(uint32_t e) { return e8m0_to_f32(e); }

// The masks and the 1024.0 pair held in VGPRs (see vconst).
struct Magic16 {
    uint32_t mlo, mhi, e16;
};
__device__ __forceinline__ Magic16 magic16() {
    return Magic16{vconst(0x000F000Fu), vconst(0x00F000F0u), vconst(0x64006400u)};
}

// sum(q x) over one 16-byte chunk of codes W against its staged x pieces xv
// and record m (see stage_x16).
template <int BITS>
__device__ __forceinline__ float chunk_qx(const u32x4& W, const u32x4* xv, const float4& m, const Magic16& k) {
    float A = 0.f, B = 0.f;
    if constexpr (BITS == 4) {
#pragma unroll
        for (int wd = 0; wd < 4; wd++) {
            const uint32_t w = W[wd], w8 = w >> 8;
            A = fdot2_f16(xv[wd][0], (w & k.mlo) | k.e16, A);
            B = fdot2_f16(xv[wd][1], (w & k.mhi) | k.e16, B);
            A = fdot2_f16(xv[wd][2], (w8 & k.mlo) | k.e16, A);
            B = fdot2_f16(xv[wd][3], (w8 & k.mhi) | k.e16, B);
        }
        A = __builtin_fmaf(B, 0.0625f, A);
    } else {
#pragma unroll
        for (int wd = 0; wd < 4; wd++) {
            const uint32_t w = W[wd];
            A = fdot2_f16(xv[wd >> 1][(wd & 1) * 2], __builtin_amdgcn_perm(k.e16, w, 0x05010500u), A);
            B = fdot2_f16(xv[wd >> 1][(wd & 1) * 2 + 1], __builtin_amdgcn_perm(k.e16, w, 0x05030502u), B);
        }
        A += B;
    }
    return __builtin_fmaf(m.x, A, -m.y);
}

// Launch shape of the VALU kernel (qmv_valu.hip): S 16-byte chunk slots per
// lane, RPW weight rows per wave, WV waves per workgroup.
struct ValuShape {
    int S, RPW, WV;
    int64_t groups;   // workgroups along N
};

// Launches qmv_valu_kernel<bits, v.RPW, v.S, v.WV>; returns false for a
// shape that has no instantiation.
bool launch_qmv_valu(int bits, const ValuShape& v, const QmvArgs& a, dim3 grid, size_t lds,
                     hipStream_t st);

}  // namespace kmi
