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
