// VQ experts in the artifacts' bit-packed layout on MFMA, expert-major:
// the (token, slot) rows are grouped by expert on the GPU (the gather sort
// of qmv.hip) and a tile of up to 16 rows routed to one expert shares every
// field decode and codebook gather.  The packed layout is the one
// vq_packed.hip documents: per output row, ceil(in/dim/32) * PB uint32
// words holding the row's PB-bit codebook indices LSB first, fp16 scales
// per group of `group` inputs (src/knurlogic/engine/families/deepseek/
// heads/deepseek_v4.py:36-44,95-129):
//   What[o, i] = scales[o, i / group] * codebook[code(o, i / dim)][i % dim]
//   y[r, o]    = x[r] . What_e[o]   for the rows r of the tile
//
// v_mfma_f32_16x16x32_f16 over 16 weight rows (n) and the tile's x rows
// (m): per scale group of a row, lane q (= lane / 16) owns the contiguous
// run of group / (4 dim) fields starting at q * group / 4 inputs, so its
// bits are one run of at most 97 bits: one 16-byte load, three funnel
// shifts to bring the run to bit 0, then fields at compile-time offsets.
// MFMA step t of the group takes the 8 inputs q * group / 4 + 8 t .. of
// every lane -- for x (A, fp16 in LDS) and the gathered codebook vectors
// (B) alike -- so each MFMA sums inside one scale group, and the group's
// scale multiplies the fp32 sum once (the per-pair kernel's order).  The
// result is rounded to bf16 per projection; two row sets (gate, up) end in
// Qwen3.5's _SwiGLU with the same roundings.
//
// x is converted to fp16 (exact for |x| < 65504, as in the other VQ
// kernels).  The codebooks are staged through registers.
#include "common.hpp"
#include "vq_packed_mfma.hpp"
#include "pair_tiles.hpp"
#include "../../include/knurlogic_amd.h"


namespace kmi {

namespace {

typedef _Float16 vpm_f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 vpm_f16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f32x4 vpm_mfma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(vpm_f16x8, a),
                                                   __builtin_bit_cast(vpm_f16x8, b), c, 0, 0, 0);
}

__device__ __forceinline__ float vpm_bf16r(float v) { return bf16_to_f32(f32_to_bf16(v)); }

__device__ __forceinline__ float vpm_f32_kept(double v) {
    float f = (float)v;
    asm volatile("" : "+v"(f));
    return f;
}

// 8 bf16 -> 8 fp16
__device__ __forceinline__ u32x4 vpm_bf16x8_to_f16x8(u32x4 v) {
    u32x4 o;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const vpm_f16x2 h = {(_Float16)__uint_as_float(v[q] << 16), (_Float16)__uint_as_float(v[q] & 0xffff0000u)};
        o[q] = __builtin_bit_cast(uint32_t, h);
    }
    return o;
}

constexpr uint32_t VPM_NONE = 0x80000000u;   // an offset past every buffer: reads 0
constexpr int VPM_WG = 256;                   // 4 waves, 16 weight rows each

}  // namespace



// PB bits per field, DIM inputs per code vector, GRP inputs per scale group,
// NSET row sets (2: gate and up, then SwiGLU).
template <int PB, int DIM, int GRP, int NSET>
__global__ __launch_bounds__(VPM_WG) void vq_packed_mfma(VpmArgs a) {
    constexpr int FPL = GRP / (4 * DIM);              // fields per lane per group
    constexpr int SPG = GRP / 32;                      // MFMA steps per group
    constexpr int FPS = 8 / DIM;                       // fields per lane per step
    constexpr int RUN = FPL * PB;                      // bits of a lane's run per group
    static_assert(FPL >= 1 && FPS >= 1 && FPS * SPG == FPL, "group / dim shape");
    static_assert(RUN + 31 <= 128, "a lane's run of fields spans one 16-byte load");
    extern __shared__ __align__(16) unsigned char smem[];

    // the tile: from the sort's list, or formed in the workgroup from
    // a.pairs routed pairs before anything is staged (a slot past the last
    // tile ends here; the working space lies over the x rows, staged later)
    int count = 0, e = 0, start = 0;
    __shared__ int32_t prow_s[VPM_TILE];             // row ids of the tile (sorted or formed here)
    if (a.tiles) {
        const int32_t* tp = a.tiles + 3 * (int64_t)blockIdx.y;
        count = tp[2];
        e = tp[0];
        start = tp[1];
        if (count <= 0 || count > a.tile_rows || e < 0 || e >= a.E) return;
        // the tile's row ids for the stores (LDS, ordered by the staging barrier)
        if ((int)threadIdx.x < count) prow_s[threadIdx.x] = a.sorted[start + threadIdx.x];
    } else {
        const int pe = pair_tile_load(a.rhs, a.pairs);
        const int cbs = (a.kc * DIM * 2 + 15) & ~15;
        const int cbl = cbs * (NSET == 2 && a.cb[1] != a.cb[0] ? 2 : 1);
        count = pair_tile_from(pe, a.pairs, (int)a.E, a.tile_rows, (int)blockIdx.y, *(PairTileLds*)(smem + cbl),
                               prow_s, e, start);
        if (a.tiles_out && blockIdx.x == 0)     // the sort's list, for the next launch
            pair_tile_store(a.tiles_out, a.sorted_out, (int)blockIdx.y, e, start, count, prow_s);
        if (count <= 0 || count > a.tile_rows) return;
    }

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 15, q = lane >> 4;
    const int K = (int)a.K, G = K / GRP;
    const bool two_cb = NSET == 2 && a.cb[1] != a.cb[0];
    const int cbytes = a.kc * DIM * 2;
    const int cbstride = (cbytes + 15) & ~15;
    unsigned char* cbl0 = smem;
    unsigned char* cbl1 = smem + (two_cb ? cbstride : 0);
    const int xstride = K * 2 + 16;                    // bytes per staged x row (rows on distinct banks)
    unsigned char* xs = smem + (size_t)cbstride * (two_cb ? 2 : 1);

    // ---- codebook(s) -> LDS through registers (8 loads per thread in flight)
    {
        const int pieces = cbytes / 16, tail = cbytes - pieces * 16;
        for (int s = 0; s < (two_cb ? 2 : 1); s++) {
            const __amdgpu_buffer_rsrc_t rcb = make_rsrc(a.cb[s], cbytes);
            unsigned char* dst = s ? cbl1 : cbl0;
            for (int p0 = tid; p0 < pieces; p0 += VPM_WG * 8) {
                u32x4 v[8];
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    const int p = p0 + VPM_WG * u;
                    v[u] = __builtin_amdgcn_raw_buffer_load_b128(rcb, p < pieces ? p * 16 : (int)VPM_NONE, 0, 0);
                }
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    const int p = p0 + VPM_WG * u;
                    if (p < pieces) *(u32x4*)(dst + p * 16) = v[u];
                }
            }
            if (tid < tail / 4)
                *(uint32_t*)(dst + pieces * 16 + tid * 4) =
                    __builtin_amdgcn_raw_buffer_load_b32(rcb, pieces * 16 + tid * 4, 0, 0);
        }
    }
    // ---- the tile's x rows -> LDS as fp16 (rows past the tile are not staged)
    {
        const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, a.X * a.K * 2);
        const int P8 = K / 8;                          // 16-byte pieces per row
        for (int m = 0; m < count; m++) {
            const uint32_t rid = (uint32_t)(a.tiles ? a.sorted[start + m] : prow_s[m]);
            const uint32_t xr = a.lhs_div == 1 ? rid : rid / (uint32_t)a.lhs_div;
            const bool ok = xr < (uint64_t)a.X;
            for (int p0 = tid; p0 < P8; p0 += VPM_WG * 4) {
                u32x4 v[4];
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const int p = p0 + VPM_WG * u;
                    v[u] = __builtin_amdgcn_raw_buffer_load_b128(
                        rx, ok && p < P8 ? (int)(((int64_t)xr * K + p * 8) * 2) : (int)VPM_NONE, 0, 0);
                }
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const int p = p0 + VPM_WG * u;
                    if (p < P8) *(u32x4*)(xs + (size_t)m * xstride + p * 16) = vpm_bf16x8_to_f16x8(v[u]);
                }
            }
        }
    }
    __syncthreads();

    // ---- per column block of 64 rows (a.cblk of them share the staging),
    //      per scale group: the lane's field run, the codebook gathers, SPG MFMAs
    const int nbt = (int)((a.N + 63) / 64);
    const int b0 = (int)blockIdx.x * a.cblk;
    const int nb = nbt - b0 < a.cblk ? nbt - b0 : a.cblk;
    const int64_t ebase = (int64_t)e * a.N;
    const int mrow = n < count ? n : count - 1;        // A rows past the tile repeat a real row
    const unsigned char* xa = xs + (size_t)mrow * xstride + (size_t)q * (GRP / 4) * 2;
    // a lane's 16-byte load may run up to 3 words past its row: past the
    // expert's last word the view returns 0 for each word out of range
    __amdgpu_buffer_rsrc_t rc[NSET], rs[NSET];
#pragma unroll
    for (int s = 0; s < NSET; s++) {
        rc[s] = make_rsrc(a.codes[s] + ebase * a.W, a.N * a.W * 4);
        rs[s] = make_rsrc(a.sc[s] + ebase * G, a.N * (int64_t)G * 2);
    }
    const uint32_t kcm1 = (uint32_t)(a.kc - 1);
    // bit of the lane's first field in group g within its row (rows start
    // on word boundaries): field g * GRP / DIM + q * FPL
    auto run_bit = [&](int g) -> uint32_t { return (uint32_t)(g * (GRP / DIM) + q * FPL) * (uint32_t)PB; };
    for (int cbk = 0; cbk < nb; cbk++) {
        const int row = (b0 + cbk) * 64 + wave * 16 + n;
        const int crow = row < a.N ? row : (int)a.N - 1;   // rows past N re-read row N-1, never stored
        const uint32_t rowword = (uint32_t)crow * (uint32_t)a.W;
        f32x4 acc[NSET];
#pragma unroll
        for (int s = 0; s < NSET; s++) acc[s] = f32x4{0.f, 0.f, 0.f, 0.f};
        constexpr int GB = 4;                              // groups whose loads are issued together
        for (int g0 = 0; g0 < G; g0 += GB) {
            u32x4 wv[NSET][GB];
            uint32_t sv[NSET][GB];
#pragma unroll
            for (int s = 0; s < NSET; s++)
#pragma unroll
                for (int j = 0; j < GB; j++) {
                    const int g = g0 + j;
                    const uint32_t w0 = rowword + (run_bit(g < G ? g : G - 1) >> 5);
                    wv[s][j] = __builtin_amdgcn_raw_buffer_load_b128(rc[s], g < G ? (int)(w0 * 4u) : (int)VPM_NONE,
                                                                     0, 0);
                    sv[s][j] = __builtin_amdgcn_raw_buffer_load_b16(
                        rs[s], g < G ? (int)((uint32_t)crow * (uint32_t)G * 2u + (uint32_t)g * 2u) : (int)VPM_NONE, 0, 0);
                }
#pragma unroll
            for (int j = 0; j < GB; j++) {
                // a group past G (the last batch of a row) reads zero codes and a
                // zero scale at the last group's addresses: it adds 0
                const int g = g0 + j < G ? g0 + j : G - 1;
                const uint32_t sh = run_bit(g) & 31u;
                u32x4 A[SPG];
#pragma unroll
                for (int t = 0; t < SPG; t++) A[t] = *(const u32x4*)(xa + (size_t)(g * GRP + 8 * t) * 2);
                // every gather of the group (both row sets, all SPG steps)
                // issued before its first MFMA (the scheduling barrier keeps
                // them there): one LDS round trip per group
                u32x4 B[NSET][SPG];
#pragma unroll
                for (int s = 0; s < NSET; s++) {
                    const u32x4 w = wv[s][j];
                    // the run at bit 0: r0 | r1 << 32 | r2 << 64 (funnel shifts by the run's offset)
                    const uint32_t r0 = __builtin_amdgcn_alignbit(w.y, w.x, sh);
                    const uint32_t r1 = __builtin_amdgcn_alignbit(w.z, w.y, sh);
                    const uint32_t r2 = __builtin_amdgcn_alignbit(w.w, w.z, sh);
                    const unsigned char* cbl = s ? cbl1 : cbl0;
#pragma unroll
                    for (int t = 0; t < SPG; t++) {
                        uint32_t bw[4];
#pragma unroll
                        for (int f = 0; f < FPS; f++) {
                            const int fi = t * FPS + f;            // field of the run
                            const int bo = fi * PB, wi = bo >> 5, bs = bo & 31;
                            const uint32_t lo = wi == 0 ? r0 : wi == 1 ? r1 : r2;
                            const uint32_t hi = wi == 0 ? r1 : wi == 1 ? r2 : 0u;
                            uint32_t c = (bs + PB <= 32) ? (lo >> bs) : __builtin_amdgcn_alignbit(hi, lo, (uint32_t)bs);
                            c = __builtin_elementwise_min(c & ((1u << PB) - 1u), kcm1);
                            if constexpr (DIM == 2) {
                                bw[f] = *(const uint32_t*)(cbl + c * 4);
                            } else if constexpr (DIM == 4) {
                                const u32x2 v = *(const u32x2*)(cbl + c * 8);
                                bw[2 * f] = v.x;
                                bw[2 * f + 1] = v.y;
                            } else {
                                const u32x4 v = *(const u32x4*)(cbl + c * 16);
                                bw[0] = v.x; bw[1] = v.y; bw[2] = v.z; bw[3] = v.w;
                            }
                        }
                        B[s][t] = u32x4{bw[0], bw[1], bw[2], bw[3]};
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int s = 0; s < NSET; s++) {
                    f32x4 P = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int t = 0; t < SPG; t++) P = vpm_mfma(A[t], B[s][t], P);
                    const float scl = f16_to_f32((uint16_t)sv[s][j]);
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[s][i] = __builtin_fmaf(scl, P[i], acc[s][i]);
                }
            }
        }

        // ---- epilogue: lane holds D[m = 4q + i][n]
        if (row < a.N) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = 4 * q + i;
                if (m >= count) continue;
                float out = vpm_bf16r(acc[0][i]);
                if constexpr (NSET == 2) {     // round(round(silu_f32(gate)) * up)
                    const float up = vpm_bf16r(acc[1][i]);
                    out = silu_bf16r(out) * up;
                }
                const int64_t r = prow_s[m];
                a.y[r * a.N + row] = f32_to_bf16(out);
            }
        }
    }
}

namespace {

size_t vpm_lds_bytes(int64_t K, int kc, int dim, bool two_cb, int tile_rows) {
    const size_t cbs = ((size_t)kc * dim * 2 + 15) & ~(size_t)15;
    return cbs * (two_cb ? 2 : 1) + (size_t)tile_rows * (K * 2 + 16);
}

}  // namespace

// the shapes the MFMA kernel covers
bool vpm_supported(int pack_bits, int dim, int group, int64_t K, int kc, bool two_cb) {
    if (!(dim == 2 || dim == 4 || dim == 8)) return false;
    if (!(group == 32 || group == 64 || group == 128)) return false;
    if (K % group || K % (32 * dim)) return false;
    const int fpl = group / (4 * dim);
    if (fpl < 1 || fpl * pack_bits + 31 > 128 || (8 / dim) * (group / 32) != fpl) return false;
    if (!(pack_bits >= 8 && pack_bits <= 12) && pack_bits != 16) return false;
    return vpm_lds_bytes(K, kc, dim, two_cb, VPM_TILE) <= 160 * 1024;
}

namespace {

template <int PB, int DIM, int GRP, int NSET>
int vpm_launch4(const VpmArgs& a, dim3 grid, size_t lds, hipStream_t st) {
    if constexpr (GRP / (4 * DIM) < 1 || (GRP / (4 * DIM)) * PB + 31 > 128) {
        return EINVAL_ARG;
    } else {
        allow_dynamic_lds_once((const void*)vq_packed_mfma<PB, DIM, GRP, NSET>);
        vq_packed_mfma<PB, DIM, GRP, NSET><<<grid, VPM_WG, lds, st>>>(a);
        return OK;
    }
}

template <int PB, int NSET>
int vpm_launch_pb(const VpmArgs& a, int dim, int group, dim3 grid, size_t lds, hipStream_t st) {
#define KMI_VPM_DG(D_, G_) if (dim == D_ && group == G_) return vpm_launch4<PB, D_, G_, NSET>(a, grid, lds, st);
    KMI_VPM_DG(2, 32) KMI_VPM_DG(2, 64) KMI_VPM_DG(2, 128)
    KMI_VPM_DG(4, 32) KMI_VPM_DG(4, 64) KMI_VPM_DG(4, 128)
    KMI_VPM_DG(8, 32) KMI_VPM_DG(8, 64) KMI_VPM_DG(8, 128)
#undef KMI_VPM_DG
    return EINVAL_ARG;
}

// column blocks of 64 rows per workgroup: one
int vpm_cblk(int64_t nbt) { return nbt < 1 ? (int)nbt : 1; }

}  // namespace

// ntiles: grid rows (tiles of the sort)
int launch_vpm(const VpmArgs& a, int pack_bits, int dim, int group, int nset, int64_t ntiles, hipStream_t st) {
    const bool two_cb = nset == 2 && a.cb[1] != a.cb[0];
    if (a.tile_rows < 1 || a.tile_rows > VPM_TILE) {
        set_error("vq (packed, MFMA): tile rows %d (1 .. %d)", a.tile_rows, VPM_TILE);
        return EINVAL_ARG;
    }
    if (!a.tiles && !(a.rhs && pair_tiles_fit(a.pairs, a.E, a.tile_rows))) {
        set_error("vq (packed, MFMA): no tiles, and %d pairs over %lld experts are not formed in the kernel",
                  a.pairs, (long long)a.E);
        return EINVAL_ARG;
    }
    size_t lds = vpm_lds_bytes(a.K, a.kc, dim, two_cb, a.tile_rows);
    const size_t cbl = (((size_t)a.kc * dim * 2 + 15) & ~(size_t)15) * (two_cb ? 2 : 1);
    if (!a.tiles && lds < cbl + sizeof(PairTileLds)) lds = cbl + sizeof(PairTileLds);   // the tile's working space
    const int64_t nbt = ceil_div(a.N, 64);
    VpmArgs b = a;
    b.cblk = vpm_cblk(nbt);
    const dim3 grid((unsigned)ceil_div(nbt, b.cblk), (unsigned)ntiles);
    int rc = EINVAL_ARG;
#define KMI_VPM_PB(PB_)                                                                                 \
    if (pack_bits == PB_)                                                                               \
        rc = nset == 2 ? vpm_launch_pb<PB_, 2>(b, dim, group, grid, lds, st)                            \
                       : vpm_launch_pb<PB_, 1>(b, dim, group, grid, lds, st);
    KMI_VPM_PB(8) KMI_VPM_PB(9) KMI_VPM_PB(10) KMI_VPM_PB(11) KMI_VPM_PB(12) KMI_VPM_PB(16)
#undef KMI_VPM_PB
    if (rc) set_error("vq (packed, MFMA): no kernel for %d-bit fields, dim %d, group %d", pack_bits, dim, group);
    return rc;
}

}  // namespace kmi
