// VQ codebook-decode expert matmul for gfx950: an expert matrix whose rows
// are runs of 8-element weight vectors, each vector an index into a per-
// layer fp16 codebook, times a per-output-channel (or per-group) fp16 scale:
//   What[o, i] = scale[o, i / sg] * codebook[codes[o, i / 8]][i % 8]
//   y[p, o]    = x[lhs[p]] . What_e[o],  e = rhs[p]
// the decode the VQ artifacts' model.py performs in VQSwitchLinear (class
// named at tests/engine/test_deepseek_v4_mtp.py:249,360; code layout of
// _pack_vq, :206-233), at 8-element vectors and byte / 16-bit indices.
//
// The codebook sits in LDS as fp16 for the whole workgroup (4 KB at 256
// entries, 64 KB at 4096).  A lane owns (output row, K segment): it loads
// its CPS code indices of the row in one contiguous run (the SEG lanes of a
// row cover the row's codes back to back), gathers each code's 16-byte
// entry from LDS, and dots it with the matching 8 x values (staged in LDS
// as fp16; the lanes of a segment read the same address) by v_dot2_f32_f16;
// scale groups are applied to fp32 partials, the SEG lanes of a row are
// summed with cross-lane shuffles, and one lane writes bf16.  With two row
// sets (the gate and up projections) the epilogue is Qwen3.5's _SwiGLU.
//
// x is converted to fp16 for the dot products: exact for activations of
// normal fp16 range (|x| < 65504; tiny values lose precision below 6e-5).
#include "common.hpp"
#include "qgemv.hpp"
#include "vq_mfma.hpp"
#include "pair_tiles.hpp"
#include "route.hpp"
#include "../../include/knurlogic_amd.h"

namespace kmi {

typedef _Float16 vq_f16x2 __attribute__((ext_vector_type(2)));

struct VqArgs {
    const uint16_t* x;          // bf16 [X, K]
    const int32_t* lhs;         // [P] x row per pair, or null: x row = p / lhs_div
    int64_t lhs_div;
    const int32_t* rhs;         // [P] expert per pair
    int64_t P, X;
    const void* codes0;         // [E, erows, K/8] (u8 or u16)
    const uint16_t* sc0;        // [E, erows, K/sg] fp16 ([E, erows] per channel)
    const uint16_t* cb0;        // [kc, 8] fp16
    const void* codes1;         // second row set (GLU: the up rows), or null
    const uint16_t* sc1;
    const uint16_t* cb1;
    int kc;
    uint16_t* y;                // [P, N] bf16
    int64_t E, N, K;
    int64_t erows;              // rows from one expert to the next in codes/scales
    int sg;                     // scale group (elements); K for one scale per channel
};

__device__ __forceinline__ float dot2_f16(uint32_t a, uint32_t b, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(vq_f16x2, a), __builtin_bit_cast(vq_f16x2, b), acc, false);
}

__device__ __forceinline__ float dot8_f16(u32x4 c, u32x4 x, float acc) {
    acc = dot2_f16(c.x, x.x, acc);
    acc = dot2_f16(c.y, x.y, acc);
    acc = dot2_f16(c.z, x.z, acc);
    return dot2_f16(c.w, x.w, acc);
}

__device__ __forceinline__ float vq_bf16r(float v) { return bf16_to_f32(f32_to_bf16(v)); }

__device__ __forceinline__ float vq_f32_kept(double v) {
    float f = (float)v;
    asm volatile("" : "+v"(f));
    return f;
}

template <int CB>
__device__ __forceinline__ uint32_t code_at(const uint32_t* w, int j) {
    if constexpr (CB == 1) return (w[j >> 2] >> (8 * (j & 3))) & 0xffu;
    else return (w[j >> 1] >> (16 * (j & 1))) & 0xffffu;
}

// CB: index bytes; SEG lanes per row; CPS codes per lane; SGC codes per
// scale group (0: one scale per row); NSET row sets (2: gate/up + SwiGLU).
template <int CB, int SEG, int CPS, int SGC, int NSET>
__global__ __launch_bounds__(256) void vq_gemv(VqArgs a) {
    constexpr int RPWG = 256 / SEG;                  // rows per workgroup
    constexpr int NW = CPS * CB / 4;                 // index words per lane
    constexpr int NG = SGC ? CPS / SGC : 1;          // scale groups per lane
    static_assert((CPS * CB) % 4 == 0, "a lane's index run is whole 32-bit words");
    extern __shared__ __align__(16) unsigned char smem[];
    const int tid = threadIdx.x;
    const int64_t p = blockIdx.y;
    const int e = a.rhs[p];
    const bool ok_e = e >= 0 && e < a.E;
    const int64_t xrow = a.lhs ? (int64_t)a.lhs[p] : p / a.lhs_div;
    const bool ok_x = xrow >= 0 && xrow < a.X;
    const bool two_cb = NSET == 2 && a.cb1 != a.cb0;
    uint16_t* cbl0 = (uint16_t*)smem;                                    // [kc][8]
    uint16_t* cbl1 = two_cb ? cbl0 + (size_t)a.kc * 8 : cbl0;            // [kc][8]
    uint16_t* xl = cbl0 + (size_t)a.kc * 8 * (two_cb ? 2 : 1);           // [K] fp16

    const int row = (int)blockIdx.x * RPWG + tid / SEG, seg = tid % SEG;
    const int64_t cpr = a.K / 8;                                         // codes per row
    const int64_t gpr = SGC ? cpr / SGC : 1;                             // scales per row
    const int64_t erow = (int64_t)(ok_e ? e : 0) * a.erows;
    const int64_t cbytes = ok_e ? a.N * cpr * CB : 0;                    // this expert's rows
    const int64_t sbytes = ok_e ? a.N * gpr * 2 : 0;

    // this lane's index words and scales first, so their loads fly during staging
    uint32_t cw[NSET][NW];
    uint16_t sv[NSET][NG];     // fp16 bits, converted at use (not at the load: no early wait)
#pragma unroll
    for (int s = 0; s < NSET; s++) {
        const __amdgpu_buffer_rsrc_t rc = make_rsrc((const char*)(s ? a.codes1 : a.codes0) + erow * cpr * CB, cbytes);
        const __amdgpu_buffer_rsrc_t rsc = make_rsrc((s ? a.sc1 : a.sc0) + erow * gpr, sbytes);
        const uint32_t cbase = (uint32_t)(((int64_t)row * cpr + (int64_t)seg * CPS) * CB);
        if constexpr (NW % 4 == 0) {
#pragma unroll
            for (int q = 0; q < NW; q += 4) {
                const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rc, (int)(cbase + 16u * (q / 4)), 0, AUX_NT);
                cw[s][q] = v.x; cw[s][q + 1] = v.y; cw[s][q + 2] = v.z; cw[s][q + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int q = 0; q < NW; q++)
                cw[s][q] = __builtin_amdgcn_raw_buffer_load_b32(rc, (int)(cbase + 4u * q), 0, AUX_NT);
        }
#pragma unroll
        for (int g = 0; g < NG; g++) {
            const int64_t gi = SGC ? (int64_t)row * gpr + ((int64_t)seg * CPS) / SGC + g : row;
            sv[s][g] = __builtin_amdgcn_raw_buffer_load_b16(rsc, (int)(gi * 2), 0, 0);
        }
    }
    // codebook(s) and the x row -> LDS
    {
        const __amdgpu_buffer_rsrc_t rcb0 = make_rsrc(a.cb0, (int64_t)a.kc * 16);
        for (int i = tid; i < a.kc; i += 256)
            *(u32x4*)(cbl0 + i * 8) = __builtin_amdgcn_raw_buffer_load_b128(rcb0, i * 16, 0, 0);
        if (two_cb) {
            const __amdgpu_buffer_rsrc_t rcb1 = make_rsrc(a.cb1, (int64_t)a.kc * 16);
            for (int i = tid; i < a.kc; i += 256)
                *(u32x4*)(cbl1 + i * 8) = __builtin_amdgcn_raw_buffer_load_b128(rcb1, i * 16, 0, 0);
        }
        const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x + (ok_x ? xrow : 0) * a.K, ok_x ? a.K * 2 : 0);
        for (int i = tid; i < (int)cpr; i += 256) {
            const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rx, i * 16, 0, 0);
            u32x4 o;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const vq_f16x2 h = {(_Float16)bf16_to_f32((uint16_t)(v[q] & 0xffffu)),
                                    (_Float16)bf16_to_f32((uint16_t)(v[q] >> 16))};
                o[q] = __builtin_bit_cast(uint32_t, h);
            }
            *(u32x4*)(xl + i * 8) = o;
        }
    }
    __syncthreads();

    float r[NSET];
#pragma unroll
    for (int s = 0; s < NSET; s++) {
        const uint16_t* cbl = s ? cbl1 : cbl0;
        float acc[NG];
#pragma unroll
        for (int g = 0; g < NG; g++) acc[g] = 0.f;
#pragma unroll
        for (int j = 0; j < CPS; j++) {
            uint32_t c = code_at<CB>(cw[s], j);
            c = __builtin_elementwise_min(c, (uint32_t)(a.kc - 1));
            const u32x4 cv = *(const u32x4*)(cbl + c * 8);
            const u32x4 xv = *(const u32x4*)(xl + (seg * CPS + j) * 8);
            acc[SGC ? j / SGC : 0] = dot8_f16(cv, xv, acc[SGC ? j / SGC : 0]);
        }
        float v = 0.f;
#pragma unroll
        for (int g = 0; g < NG; g++) v = __builtin_fmaf(f16_to_f32(sv[s][g]), acc[g], v);
#pragma unroll
        for (int o = SEG / 2; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
        r[s] = vq_bf16r(v);
    }
    if (seg == 0 && row < a.N) {
        float out = r[0];
        if constexpr (NSET == 2) {     // round(round(silu_f32(gate)) * up)
            out = silu_bf16r(r[0]) * r[1];
        }
        a.y[p * a.N + row] = (ok_e && ok_x) ? f32_to_bf16(out) : (uint16_t)0;
    }
}

// Lanes per row and codes per lane for a row of K elements: the widest SEG in
// {8, 4, 2} whose segments hold whole scale groups and whole 32-bit words,
// widened (up to 64 lanes, a row per wave) while the grid of `rows` rows
// would leave fewer than 1024 workgroups: shorter gather chains per lane.
// Only for small codebooks: every workgroup stages the whole codebook, and
// at 4096 entries (64 KB) fewer rows per workgroup cost more than they save.
static bool vq_shape(int64_t K, int sgc, int code_bytes, int64_t rows, int kc, int& seg, int& cps) {
    const int64_t cpr = K / 8;
    auto valid = [&](int s) {
        if (cpr % s) return false;
        const int64_t c = cpr / s;
        return !(sgc && c % sgc) && (c * code_bytes) % 4 == 0;
    };
    seg = 0;
    for (int s = 8; s >= 2; s >>= 1)
        if (valid(s)) { seg = s; break; }
    if (!seg) return false;
    while (kc <= 256 && seg < 64 && rows / (256 / seg) < 1024 && valid(seg * 2)) seg *= 2;
    cps = (int)(cpr / seg);
    return true;
}

static int launch_vq(const VqArgs& a, int code_bytes, int nset, hipStream_t st) {
    const int sgc = a.sg >= a.K ? 0 : a.sg / 8;
    int seg = 0, cps = 0;
    if (!vq_shape(a.K, sgc, code_bytes, a.N * a.P, a.kc, seg, cps)) {
        set_error("vq: K=%lld with scale group %d has no lane layout", (long long)a.K, a.sg);
        return EINVAL_ARG;
    }
    const bool two_cb = nset == 2 && a.cb1 != a.cb0;
    const size_t lds = (size_t)a.kc * 16 * (two_cb ? 2 : 1) + (size_t)a.K * 2;
    if (lds > 160 * 1024) {
        set_error("vq: codebook(s) of %d entries and K=%lld exceed the 160 KB LDS", a.kc, (long long)a.K);
        return EINVAL_ARG;
    }
    const dim3 grid((unsigned)ceil_div(a.N, 256 / seg), (unsigned)a.P);
#define KMI_VQ(CB_, SEG_, CPS_, SGC_, NS_)                                                        \
    if (code_bytes == CB_ && seg == SEG_ && cps == CPS_ && sgc == SGC_ && nset == NS_) {          \
        static bool attr = false;                                                                 \
        if (!attr) {                                                                              \
            (void)hipFuncSetAttribute((const void*)vq_gemv<CB_, SEG_, CPS_, SGC_, NS_>,           \
                                      hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);    \
            attr = true;                                                                          \
        }                                                                                         \
        vq_gemv<CB_, SEG_, CPS_, SGC_, NS_><<<grid, 256, lds, st>>>(a);                           \
        return OK;                                                                                \
    }
#define KMI_VQ2(CB_, SEG_, CPS_, SGC_) KMI_VQ(CB_, SEG_, CPS_, SGC_, 1) KMI_VQ(CB_, SEG_, CPS_, SGC_, 2)
    // (index bytes, lanes per row, codes per lane, codes per scale group)
    KMI_VQ2(1, 2, 8, 0)   /* K = 128 */
    KMI_VQ2(1, 4, 4, 0)   /* K = 128 */
    KMI_VQ2(1, 2, 8, 8)   /* K = 128 */
    KMI_VQ2(1, 2, 16, 0)   /* K = 256 */
    KMI_VQ2(1, 4, 8, 0)   /* K = 256 */
    KMI_VQ2(1, 8, 4, 0)   /* K = 256 */
    KMI_VQ2(1, 2, 16, 8)   /* K = 256 */
    KMI_VQ2(1, 4, 8, 8)   /* K = 256 */
    KMI_VQ2(1, 2, 32, 0)   /* K = 512 */
    KMI_VQ2(1, 4, 16, 0)   /* K = 512 */
    KMI_VQ2(1, 8, 8, 0)   /* K = 512 */
    KMI_VQ2(1, 16, 4, 0)   /* K = 512 */
    KMI_VQ2(1, 2, 32, 8)   /* K = 512 */
    KMI_VQ2(1, 4, 16, 8)   /* K = 512 */
    KMI_VQ2(1, 8, 8, 8)   /* K = 512 */
    KMI_VQ2(1, 2, 44, 0)   /* K = 704 */
    KMI_VQ2(1, 2, 48, 0)   /* K = 768 */
    KMI_VQ2(1, 4, 24, 0)   /* K = 768 */
    KMI_VQ2(1, 8, 12, 0)   /* K = 768 */
    KMI_VQ2(1, 2, 48, 8)   /* K = 768 */
    KMI_VQ2(1, 4, 24, 8)   /* K = 768 */
    KMI_VQ2(1, 2, 64, 0)   /* K = 1024 */
    KMI_VQ2(1, 4, 32, 0)   /* K = 1024 */
    KMI_VQ2(1, 8, 16, 0)   /* K = 1024 */
    KMI_VQ2(1, 16, 8, 0)   /* K = 1024 */
    KMI_VQ2(1, 32, 4, 0)   /* K = 1024 */
    KMI_VQ2(1, 2, 64, 8)   /* K = 1024 */
    KMI_VQ2(1, 4, 32, 8)   /* K = 1024 */
    KMI_VQ2(1, 8, 16, 8)   /* K = 1024 */
    KMI_VQ2(1, 16, 8, 8)   /* K = 1024 */
    KMI_VQ2(1, 2, 128, 0)   /* K = 2048 */
    KMI_VQ2(1, 4, 64, 0)   /* K = 2048 */
    KMI_VQ2(1, 8, 32, 0)   /* K = 2048 */
    KMI_VQ2(1, 16, 16, 0)   /* K = 2048 */
    KMI_VQ2(1, 32, 8, 0)   /* K = 2048 */
    KMI_VQ2(1, 64, 4, 0)   /* K = 2048 */
    KMI_VQ2(1, 2, 128, 8)   /* K = 2048 */
    KMI_VQ2(1, 4, 64, 8)   /* K = 2048 */
    KMI_VQ2(1, 8, 32, 8)   /* K = 2048 */
    KMI_VQ2(1, 16, 16, 8)   /* K = 2048 */
    KMI_VQ2(1, 32, 8, 8)   /* K = 2048 */
    KMI_VQ2(1, 2, 176, 0)   /* K = 2816 */
    KMI_VQ2(1, 4, 88, 0)   /* K = 2816 */
    KMI_VQ2(1, 8, 44, 0)   /* K = 2816 */
    KMI_VQ2(1, 2, 176, 8)   /* K = 2816 */
    KMI_VQ2(1, 4, 88, 8)   /* K = 2816 */
    KMI_VQ2(1, 2, 256, 0)   /* K = 4096 */
    KMI_VQ2(1, 4, 128, 0)   /* K = 4096 */
    KMI_VQ2(1, 8, 64, 0)   /* K = 4096 */
    KMI_VQ2(1, 16, 32, 0)   /* K = 4096 */
    KMI_VQ2(1, 32, 16, 0)   /* K = 4096 */
    KMI_VQ2(1, 64, 8, 0)   /* K = 4096 */
    KMI_VQ2(1, 2, 256, 8)   /* K = 4096 */
    KMI_VQ2(1, 4, 128, 8)   /* K = 4096 */
    KMI_VQ2(1, 8, 64, 8)   /* K = 4096 */
    KMI_VQ2(1, 16, 32, 8)   /* K = 4096 */
    KMI_VQ2(1, 32, 16, 8)   /* K = 4096 */
    KMI_VQ2(1, 64, 8, 8)   /* K = 4096 */
    KMI_VQ2(2, 2, 8, 0)   /* K = 128 */
    KMI_VQ2(2, 4, 4, 0)   /* K = 128 */
    KMI_VQ2(2, 8, 2, 0)   /* K = 128 */
    KMI_VQ2(2, 2, 8, 8)   /* K = 128 */
    KMI_VQ2(2, 2, 16, 0)   /* K = 256 */
    KMI_VQ2(2, 4, 8, 0)   /* K = 256 */
    KMI_VQ2(2, 8, 4, 0)   /* K = 256 */
    KMI_VQ2(2, 16, 2, 0)   /* K = 256 */
    KMI_VQ2(2, 2, 16, 8)   /* K = 256 */
    KMI_VQ2(2, 4, 8, 8)   /* K = 256 */
    KMI_VQ2(2, 2, 32, 0)   /* K = 512 */
    KMI_VQ2(2, 4, 16, 0)   /* K = 512 */
    KMI_VQ2(2, 8, 8, 0)   /* K = 512 */
    KMI_VQ2(2, 16, 4, 0)   /* K = 512 */
    KMI_VQ2(2, 32, 2, 0)   /* K = 512 */
    KMI_VQ2(2, 2, 32, 8)   /* K = 512 */
    KMI_VQ2(2, 4, 16, 8)   /* K = 512 */
    KMI_VQ2(2, 8, 8, 8)   /* K = 512 */
    KMI_VQ2(2, 2, 44, 0)   /* K = 704 */
    KMI_VQ2(2, 4, 22, 0)   /* K = 704 */
    KMI_VQ2(2, 2, 48, 0)   /* K = 768 */
    KMI_VQ2(2, 4, 24, 0)   /* K = 768 */
    KMI_VQ2(2, 8, 12, 0)   /* K = 768 */
    KMI_VQ2(2, 16, 6, 0)   /* K = 768 */
    KMI_VQ2(2, 2, 48, 8)   /* K = 768 */
    KMI_VQ2(2, 4, 24, 8)   /* K = 768 */
    KMI_VQ2(2, 2, 64, 0)   /* K = 1024 */
    KMI_VQ2(2, 4, 32, 0)   /* K = 1024 */
    KMI_VQ2(2, 8, 16, 0)   /* K = 1024 */
    KMI_VQ2(2, 16, 8, 0)   /* K = 1024 */
    KMI_VQ2(2, 32, 4, 0)   /* K = 1024 */
    KMI_VQ2(2, 64, 2, 0)   /* K = 1024 */
    KMI_VQ2(2, 2, 64, 8)   /* K = 1024 */
    KMI_VQ2(2, 4, 32, 8)   /* K = 1024 */
    KMI_VQ2(2, 8, 16, 8)   /* K = 1024 */
    KMI_VQ2(2, 16, 8, 8)   /* K = 1024 */
    KMI_VQ2(2, 2, 128, 0)   /* K = 2048 */
    KMI_VQ2(2, 4, 64, 0)   /* K = 2048 */
    KMI_VQ2(2, 8, 32, 0)   /* K = 2048 */
    KMI_VQ2(2, 16, 16, 0)   /* K = 2048 */
    KMI_VQ2(2, 32, 8, 0)   /* K = 2048 */
    KMI_VQ2(2, 64, 4, 0)   /* K = 2048 */
    KMI_VQ2(2, 2, 128, 8)   /* K = 2048 */
    KMI_VQ2(2, 4, 64, 8)   /* K = 2048 */
    KMI_VQ2(2, 8, 32, 8)   /* K = 2048 */
    KMI_VQ2(2, 16, 16, 8)   /* K = 2048 */
    KMI_VQ2(2, 32, 8, 8)   /* K = 2048 */
    KMI_VQ2(2, 2, 176, 0)   /* K = 2816 */
    KMI_VQ2(2, 4, 88, 0)   /* K = 2816 */
    KMI_VQ2(2, 8, 44, 0)   /* K = 2816 */
    KMI_VQ2(2, 16, 22, 0)   /* K = 2816 */
    KMI_VQ2(2, 2, 176, 8)   /* K = 2816 */
    KMI_VQ2(2, 4, 88, 8)   /* K = 2816 */
    KMI_VQ2(2, 2, 256, 0)   /* K = 4096 */
    KMI_VQ2(2, 4, 128, 0)   /* K = 4096 */
    KMI_VQ2(2, 8, 64, 0)   /* K = 4096 */
    KMI_VQ2(2, 16, 32, 0)   /* K = 4096 */
    KMI_VQ2(2, 32, 16, 0)   /* K = 4096 */
    KMI_VQ2(2, 64, 8, 0)   /* K = 4096 */
    KMI_VQ2(2, 2, 256, 8)   /* K = 4096 */
    KMI_VQ2(2, 4, 128, 8)   /* K = 4096 */
    KMI_VQ2(2, 8, 64, 8)   /* K = 4096 */
    KMI_VQ2(2, 16, 32, 8)   /* K = 4096 */
    KMI_VQ2(2, 32, 16, 8)   /* K = 4096 */
    KMI_VQ2(2, 64, 8, 8)   /* K = 4096 */
#undef KMI_VQ2
#undef KMI_VQ
    set_error("vq: no kernel for K=%lld (%d lanes x %d codes, scale group %d)", (long long)a.K, seg, cps, a.sg);
    return EINVAL_ARG;
}

static int vq_check(int dtype, int code_bytes, int kc, int dim, int scale_group, int64_t K, int64_t N,
                    int64_t E) {
    KMI_CHECK_ARG(dtype == BF16, "vq: only bfloat16 activations are implemented");
    KMI_CHECK_ARG(code_bytes == 1 || code_bytes == 2, "vq: code_bytes=%d (1 or 2)", code_bytes);
    KMI_CHECK_ARG(dim == 8, "vq: vector length %d (8 is implemented)", dim);
    KMI_CHECK_ARG(kc >= 1 && kc <= (code_bytes == 1 ? 256 : 65536), "vq: %d codebook entries", kc);
    KMI_CHECK_ARG(K > 0 && K % 64 == 0 && N > 0 && E > 0, "vq: K=%lld must be a multiple of 64", (long long)K);
    KMI_CHECK_ARG(scale_group == 0 || (scale_group % 64 == 0 && K % scale_group == 0),
                  "vq: scale group %d (0 = per channel, else a multiple of 64 dividing K)", scale_group);
    KMI_CHECK_ARG(E * N * (K / 8) * code_bytes < (1LL << 31), "vq: codes past 2 GiB");
    return OK;
}

}  // namespace kmi

using namespace kmi;

extern "C" {

int kmi_vq_gather_qmm(const void* x, int64_t X, int64_t K, const void* codes, int code_bytes,
                      const void* codebook, int kc, int dim, const void* scales, int scale_group,
                      int64_t E, int64_t N, const int32_t* lhs, const int32_t* rhs, int64_t P,
                      int dtype, void* y, void* stream) {
    clear_error();
    int rc = vq_check(dtype, code_bytes, kc, dim, scale_group, K, N, E);
    if (rc) return rc;
    KMI_CHECK_ARG(P >= 0 && X >= 1, "vq_gather_qmm: bad sizes");
    if (P == 0) return OK;
    KMI_CHECK_ARG(x && codes && codebook && scales && rhs && y, "vq_gather_qmm: null pointer");
    VqArgs a = {};
    a.x = (const uint16_t*)x; a.lhs = lhs; a.lhs_div = 1; a.rhs = rhs; a.P = P; a.X = X;
    a.codes0 = codes; a.sc0 = (const uint16_t*)scales; a.cb0 = (const uint16_t*)codebook;
    a.codes1 = nullptr; a.sc1 = nullptr; a.cb1 = a.cb0; a.kc = kc;
    a.y = (uint16_t*)y; a.E = E; a.N = N; a.K = K; a.erows = N;
    a.sg = scale_group ? scale_group : (int)K;
    rc = launch_vq(a, code_bytes, 1, (hipStream_t)stream);
    if (rc) return rc;
    KMI_CHECK_LAUNCH("vq_gemv");
    return OK;
}

int kmi_vq_glu(const void* x, int64_t T, int64_t H, int64_t I, int k, const int32_t* inds,
               const void* codes_gate, const void* scales_gate, const void* codebook_gate,
               const void* codes_up, const void* scales_up, const void* codebook_up, int code_bytes,
               int kc, int dim, int scale_group, int64_t E, int dtype, void* act, void* stream) {
    clear_error();
    int rc = vq_check(dtype, code_bytes, kc, dim, scale_group, H, I, E);
    if (rc) return rc;
    KMI_CHECK_ARG(T >= 0 && k >= 1, "vq_glu: bad sizes");
    if (T == 0) return OK;
    KMI_CHECK_ARG(x && inds && codes_gate && scales_gate && codebook_gate && codes_up && scales_up &&
                  codebook_up && act, "vq_glu: null pointer");
    VqArgs a = {};
    a.x = (const uint16_t*)x; a.lhs = nullptr; a.lhs_div = k; a.rhs = inds; a.P = T * k; a.X = T;
    a.codes0 = codes_gate; a.sc0 = (const uint16_t*)scales_gate; a.cb0 = (const uint16_t*)codebook_gate;
    a.codes1 = codes_up; a.sc1 = (const uint16_t*)scales_up; a.cb1 = (const uint16_t*)codebook_up;
    a.kc = kc; a.y = (uint16_t*)act; a.E = E; a.N = I; a.K = H; a.erows = I;
    a.sg = scale_group ? scale_group : (int)H;
    rc = launch_vq(a, code_bytes, 2, (hipStream_t)stream);
    if (rc) return rc;
    KMI_CHECK_LAUNCH("vq_gemv(glu)");
    return OK;
}

// Workspace: act [T*k, I], y [T*k, H] for the combine, then the expert sort
// of the MFMA path (sized for up to 4096 experts).
static size_t vq_act_bytes(int64_t T, int64_t I, int k) { return ((size_t)T * k * I * 2 + 255) & ~(size_t)255; }
static size_t vq_y_bytes(int64_t T, int64_t H, int k) { return ((size_t)T * k * H * 2 + 255) & ~(size_t)255; }

size_t kmi_vq_switch_glu_workspace_bytes(int64_t T, int64_t H, int64_t I, int k) {
    if (T <= 0 || H <= 0 || I <= 0 || k <= 0) return 0;
    return vq_act_bytes(T, I, k) + vq_y_bytes(T, H, k) + sort_index_bytes(T * k, 4096, 1);   // any tile size
}

}  // extern "C"

// The VQ SwitchGLU; with logits (one token, the MFMA gate/up path) its
// pair-mode gate/up kernel routes the token and writes inds / scores, which
// the down kernel then reads.  vq_route_in_kernel says when that applies.
static bool vq_route_in_kernel(int64_t T, int64_t H, int k, int64_t E, int code_bytes, int kc, int scale_group,
                               bool two_cb) {
    return T == 1 && k >= 1 && k <= 8 && E >= k && E <= ROUTE_THREADS && scale_group == 0 &&
           vq_mfma_supported(H, code_bytes, kc, two_cb);
}

static int vq_switch_glu_impl(const void* x, int64_t T, int64_t H, int64_t I, int k, const int32_t* inds,
                              const void* scores, const void* codes_gate, const void* scales_gate,
                              const void* codebook_gate, const void* codes_up, const void* scales_up,
                              const void* codebook_up, const void* codes_down, const void* scales_down,
                              const void* codebook_down, int code_bytes, int kc, int dim, int scale_group,
                              int64_t E, int dtype, void* out, void* workspace, size_t workspace_bytes,
                              void* stream, const void* logits, bool routed = false) {
    int rc = vq_check(dtype, code_bytes, kc, dim, scale_group, H, I, E);
    if (rc) return rc;
    rc = vq_check(dtype, code_bytes, kc, dim, scale_group, I, H, E);
    if (rc) return rc;
    KMI_CHECK_ARG(T >= 0 && k >= 1 && k <= 64, "vq_switch_glu: bad sizes");
    if (T == 0) return OK;
    KMI_CHECK_ARG(x && inds && codes_gate && scales_gate && codebook_gate && codes_up && scales_up &&
                  codebook_up && codes_down && scales_down && codebook_down && out,
                  "vq_switch_glu: null pointer");
    const size_t need = kmi_vq_switch_glu_workspace_bytes(T, H, I, k);
    if (!workspace || workspace_bytes < need) {
        set_error("vq_switch_glu: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
        return EWORKSPACE;
    }
    uint16_t* act = (uint16_t*)workspace;
    hipStream_t st = (hipStream_t)stream;
    const int64_t P = T * k;
    const bool two_cb = codebook_up != codebook_gate;
    // Each projection runs expert-major on MFMA where that kernel covers it
    // (per-channel scales, K a multiple of 128), else per pair on the VALU.
    const bool sortable = scale_group == 0 && E <= 4096 && P < (1LL << 24);
    auto al16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
    const bool m_glu = sortable && vq_mfma_supported(H, code_bytes, kc, two_cb) && al16(codes_gate) &&
                       al16(codes_up);
    const bool m_down = sortable && vq_mfma_supported(I, code_bytes, kc, false) && al16(codes_down);
    if (logits && !(m_glu && T == 1)) {
        set_error("vq_switch_glu: in-kernel routing needs one token on the MFMA gate/up path");
        return EINVAL_ARG;
    }
    uint16_t* y = scores ? (uint16_t*)((char*)workspace + vq_act_bytes(T, I, k)) : (uint16_t*)out;
    // one token: its k pairs are their own tiles (pair mode), no sort
    const bool pair_mode = T == 1;
    // Tile rows: LDS holds a tile's x rows, sized for the largest tile, so
    // few routed rows per expert take 4- or 8-row tiles (more workgroups fit a
    // CU); the sort cuts every expert's rows into tiles of at most this.
    const int64_t avg = ceil_div(P, E < P ? E : P);
    int tile_rows = avg <= 2 ? 4 : avg <= 4 ? 8 : VQM_TILE_ROWS;
    if (tile_rows > P) tile_rows = (int)P;
    if (pair_mode) tile_rows = 1;
    // inds from the router (every expert in range) and few pairs: the MFMA
    // kernels form their tiles themselves, no sort
    const bool formed = routed && !pair_mode && pair_tiles_fit(P, E, tile_rows);
    SortedRows sr = {};
    void* index_ws = (char*)workspace + vq_act_bytes(T, I, k) + vq_y_bytes(T, H, k);
    if ((m_glu || m_down) && !pair_mode && !formed) {
        // the sort zeroes y's rows of out-of-range experts (no tile holds them)
        rc = launch_sort_rows(inds, P, 1, (int)E, tile_rows, index_ws, m_down ? y : nullptr, H, st, &sr);
        if (rc) return rc;
    }
    if (m_glu) {
        VqmArgs g = {};
        g.x = (const uint16_t*)x; g.X = T; g.lhs_magic = k > 1 ? (uint32_t)((0x100000000ULL + k - 1) / k) : 0u;
        g.tiles = pair_mode || formed ? nullptr : sr.tiles; g.sorted = sr.sorted; g.rhs = inds; g.E = E;
        g.pairs = formed ? (int)P : 0;
        if (formed && m_down) {     // the gate/up kernel writes the sort's list for the down kernel
            g.sorted_out = (int32_t*)index_ws;
            g.tiles_out = (int32_t*)index_ws + P;
        }
        g.codes0 = codes_gate; g.sc0 = (const uint16_t*)scales_gate; g.cb0 = (const uint16_t*)codebook_gate;
        g.codes1 = codes_up; g.sc1 = (const uint16_t*)scales_up; g.cb1 = (const uint16_t*)codebook_up;
        g.kc = kc; g.y = act; g.N = I; g.K = H; g.erows = I; g.tile_rows = tile_rows;
        if (logits) {   // pair mode: the kernel routes its token and writes inds / scores
            g.logits = (const uint16_t*)logits;
            g.inds_out = (int32_t*)inds;
            g.scores_out = (uint16_t*)scores;
            g.k = k;
        }
        rc = launch_vq_mfma(g, code_bytes, 2, pair_mode ? P : sort_max_tiles(P, E, tile_rows), st);
        if (rc) return rc;
        KMI_CHECK_LAUNCH("vq_mfma(glu)");
    } else {
        VqArgs g = {};
        g.x = (const uint16_t*)x; g.lhs = nullptr; g.lhs_div = k; g.rhs = inds; g.P = P; g.X = T;
        g.codes0 = codes_gate; g.sc0 = (const uint16_t*)scales_gate; g.cb0 = (const uint16_t*)codebook_gate;
        g.codes1 = codes_up; g.sc1 = (const uint16_t*)scales_up; g.cb1 = (const uint16_t*)codebook_up;
        g.kc = kc; g.y = act; g.E = E; g.N = I; g.K = H; g.erows = I;
        g.sg = scale_group ? scale_group : (int)H;
        rc = launch_vq(g, code_bytes, 2, st);
        if (rc) return rc;
        KMI_CHECK_LAUNCH("vq_gemv(glu)");
    }
    // a few tokens: the down projection token-major, with the combine in its
    // epilogue (the same kernel writes y without scores, so both agree bit
    // for bit)
    if (m_down && P <= 16 && vq_down_tok_supported(I, code_bytes, kc, k)) {
        VqdArgs d = {};
        d.x = act; d.inds = inds; d.codes = codes_down; d.sc = (const uint16_t*)scales_down;
        d.cb = (const uint16_t*)codebook_down; d.scores = (const uint16_t*)scores;
        d.out = scores ? (uint16_t*)out : y;
        d.E = E; d.N = H; d.K = I; d.T = T; d.k = k; d.kc = kc;
        rc = launch_vq_down_tok(d, code_bytes, st);
        if (rc) return rc;
        KMI_CHECK_LAUNCH("vq_down_tok");
        return OK;
    }
    if (m_down) {
        VqmArgs d = {};
        d.x = act; d.X = P; d.lhs_magic = 0;
        d.tiles = pair_mode ? nullptr : sr.tiles; d.sorted = sr.sorted; d.rhs = inds; d.E = E;
        if (formed && m_glu) {      // the list the gate/up kernel wrote
            d.sorted = (const int32_t*)index_ws;
            d.tiles = (const int32_t*)index_ws + P;
        } else if (formed) {
            d.pairs = (int)P;
        }
        d.codes0 = codes_down; d.sc0 = (const uint16_t*)scales_down; d.cb0 = (const uint16_t*)codebook_down;
        d.codes1 = nullptr; d.sc1 = nullptr; d.cb1 = d.cb0;
        d.kc = kc; d.y = y; d.N = H; d.K = I; d.erows = H; d.tile_rows = tile_rows;
        rc = launch_vq_mfma(d, code_bytes, 1, pair_mode ? P : sort_max_tiles(P, E, tile_rows), st);
        if (rc) return rc;
        KMI_CHECK_LAUNCH("vq_mfma(down)");
    } else {
        VqArgs d = {};
        d.x = act; d.lhs = nullptr; d.lhs_div = 1; d.rhs = inds; d.P = P; d.X = P;
        d.codes0 = codes_down; d.sc0 = (const uint16_t*)scales_down; d.cb0 = (const uint16_t*)codebook_down;
        d.codes1 = nullptr; d.sc1 = nullptr; d.cb1 = d.cb0; d.kc = kc;
        d.y = y; d.E = E; d.N = H; d.K = I; d.erows = H;
        d.sg = scale_group ? scale_group : (int)I;
        rc = launch_vq(d, code_bytes, 1, st);
        if (rc) return rc;
        KMI_CHECK_LAUNCH("vq_gemv(down)");
    }
    if (scores) return kmi_moe_combine(y, scores, dtype, T, k, H, out, stream);
    return OK;
}

extern "C" {

int kmi_vq_switch_glu(const void* x, int64_t T, int64_t H, int64_t I, int k, const int32_t* inds,
                      const void* scores, const void* codes_gate, const void* scales_gate,
                      const void* codebook_gate, const void* codes_up, const void* scales_up,
                      const void* codebook_up, const void* codes_down, const void* scales_down,
                      const void* codebook_down, int code_bytes, int kc, int dim, int scale_group,
                      int64_t E, int dtype, void* out, void* workspace, size_t workspace_bytes,
                      void* stream) {
    clear_error();
    return vq_switch_glu_impl(x, T, H, I, k, inds, scores, codes_gate, scales_gate, codebook_gate, codes_up,
                              scales_up, codebook_up, codes_down, scales_down, codebook_down, code_bytes, kc, dim,
                              scale_group, E, dtype, out, workspace, workspace_bytes, stream, nullptr);
}

int kmi_vq_experts(const void* x, const void* logits, int64_t T, int64_t H, int64_t I, int k,
                   const void* codes_gate, const void* scales_gate, const void* codebook_gate,
                   const void* codes_up, const void* scales_up, const void* codebook_up,
                   const void* codes_down, const void* scales_down, const void* codebook_down, int code_bytes,
                   int kc, int dim, int scale_group, int64_t E, int dtype, void* out, int32_t* inds,
                   void* scores, void* workspace, size_t workspace_bytes, void* stream) {
    clear_error();
    KMI_CHECK_ARG(dtype == BF16, "vq_experts: only bfloat16 activations and logits are implemented");
    KMI_CHECK_ARG(E >= 1 && E <= ROUTE_MAX_E && k >= 1 && k <= 8 && k <= E,
                  "vq_experts: top-%d of %lld experts (k <= 8, E <= %d)", k, (long long)E, ROUTE_MAX_E);
    KMI_CHECK_ARG(T >= 0, "vq_experts: T=%lld", (long long)T);
    if (T == 0) return OK;
    KMI_CHECK_ARG(logits && inds && scores, "vq_experts: null pointer");
    const bool two_cb = codebook_up != codebook_gate;
    auto al16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
    if (vq_route_in_kernel(T, H, k, E, code_bytes, kc, scale_group, two_cb) && al16(codes_gate) && al16(codes_up) &&
        vq_check(dtype, code_bytes, kc, dim, scale_group, H, I, E) == OK)
        return vq_switch_glu_impl(x, T, H, I, k, inds, scores, codes_gate, scales_gate, codebook_gate, codes_up,
                                  scales_up, codebook_up, codes_down, scales_down, codebook_down, code_bytes, kc, dim,
                                  scale_group, E, dtype, out, workspace, workspace_bytes, stream, logits);
    clear_error();
    int rc = kmi_moe_route(logits, dtype, T, (int)E, k, inds, scores, stream);
    if (rc) return rc;
    return vq_switch_glu_impl(x, T, H, I, k, inds, scores, codes_gate, scales_gate, codebook_gate, codes_up,
                              scales_up, codebook_up, codes_down, scales_down, codebook_down, code_bytes, kc, dim,
                              scale_group, E, dtype, out, workspace, workspace_bytes, stream, nullptr, true);
}

}  // extern "C"
