// VQ expert matmul on MFMA for gfx950, expert-major: the (token, expert)
// pairs are grouped by expert on the GPU (the gather sort of qmv.hip), and a
// tile of up to 16 rows routed to one expert shares every code gather.
//
//   What[o, i] = scale[o] * codebook[codes[o, i / 8]][i % 8]   (per channel)
//   y[r, o]    = x[r] . What_e[o]   for the rows r of the tile
//
// v_mfma_f32_16x16x32_f16 takes, per lane, 8 fp16 values along k of one
// row of B: exactly one 8-element codebook vector.  So lane (n = l % 16,
// q = l / 16) gathers codebook[code] from LDS straight into its B operand
// (no decode arithmetic) for weight row n, and A holds the tile's x rows
// (fp16 in LDS) at the same k-run.  Lane q of a row owns the q-th quarter
// of the row's codes, loaded contiguously; MFMA step kb takes code
// q * CPR/4 + kb from every lane (any order of k works with one scale per
// row).  One code per lane per MFMA: a 4-wave workgroup streams 256 codes
// per step.
//
// Scales apply to the fp32 sums; each projection's result is rounded to
// bf16, and two row sets (gate, up) end in Qwen3.5's _SwiGLU with the same
// roundings as the VALU kernel in vq.hip.
//
// x is converted to fp16 (exact for |x| < 65504; tiny values lose precision
// below 6e-5), as in vq.hip.
#include "common.hpp"
#include "vq_mfma.hpp"
#include "pair_tiles.hpp"
#include "route.hpp"


namespace kmi {

namespace {

typedef _Float16 vqm_f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 vqm_f16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f32x4 mfma_f16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(vqm_f16x8, a),
                                                   __builtin_bit_cast(vqm_f16x8, b), c, 0, 0, 0);
}

__device__ __forceinline__ float vqm_bf16r(float v) { return bf16_to_f32(f32_to_bf16(v)); }

__device__ __forceinline__ float vqm_f32_kept(double v) {
    float f = (float)v;
    asm volatile("" : "+v"(f));
    return f;
}

// 8 bf16 -> 8 fp16
__device__ __forceinline__ u32x4 bf16x8_to_f16x8(u32x4 v) {
    u32x4 o;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const vqm_f16x2 h = {(_Float16)__uint_as_float(v[q] << 16), (_Float16)__uint_as_float(v[q] & 0xffff0000u)};
        o[q] = __builtin_bit_cast(uint32_t, h);
    }
    return o;
}

constexpr uint32_t NONE = 0x80000000u;      // an offset past every buffer: reads 0

constexpr int WG = 256;                     // 4 waves
constexpr int TM = VQM_TILE_ROWS;           // tile rows (MFMA M)

}  // namespace

// CB: index bytes (1, 2); NSET: row sets (2: gate, up + SwiGLU); LW: 32-bit
// words of codes per lane; KS: waves sharing a 16-row group, each over
// 1/KS of K (partials summed in LDS), so small grids still fill the chip.
// MB: several column blocks per workgroup (a.cblk), the next block's codes
// loaded into a second register set while a block computes; else one block
// and one register set (fewer registers: more waves to cover the gathers).
// RT (pair mode only): the pair's expert from routing its token's logits in
// the workgroup (E <= 256), not from rhs.
template <int CB, int NSET, int LW, int KS, bool MB, bool RT = false>
__global__ __launch_bounds__(WG) void vq_mfma(VqmArgs a) {
    constexpr int CPL = LW * 4 / CB;                 // codes per lane
    constexpr int RW = 64 / KS;                      // weight rows per workgroup
    extern __shared__ __align__(16) unsigned char smem[];

    // tile: (expert, first sorted row, rows) from the sort; formed in the
    // workgroup from a.pairs routed pairs, before anything is staged (a slot
    // past the last tile ends here; the working space lies over the x rows,
    // staged later); or in pair mode (no tiles) pair blockIdx.y alone, its
    // expert straight from rhs
    int e, start, count;
    __shared__ int32_t prow_s[TM];                   // row ids of the tile (sorted or formed here)
    if (a.tiles) {
        const int32_t* tp = a.tiles + 3 * (int64_t)blockIdx.y;
        count = tp[2];
        if (count <= 0 || count > a.tile_rows) return;   // a tile never exceeds the staged rows
        e = tp[0];
        start = tp[1];
        // the tile's row ids for the stores (LDS, ordered by the staging barrier)
        if ((int)threadIdx.x < count) prow_s[threadIdx.x] = a.sorted[start + threadIdx.x];
    } else if (a.pairs) {
        const int pe = pair_tile_load(a.rhs, a.pairs);
        const size_t cbl = (size_t)((a.kc + 63) / 64) * 1024 * (NSET == 2 && a.cb1 != a.cb0 ? 2 : 1);
        count = pair_tile_from(pe, a.pairs, (int)a.E, a.tile_rows, (int)blockIdx.y, *(PairTileLds*)(smem + cbl),
                               prow_s, e, start);
        if (a.tiles_out && blockIdx.x == 0)     // the sort's list, for the next launch
            pair_tile_store(a.tiles_out, a.sorted_out, (int)blockIdx.y, e, start, count, prow_s);
        if (count <= 0 || count > a.tile_rows) return;
    } else {
        start = (int)blockIdx.y;
        count = 1;
        // RT: the expert is routed below, once the loads that do not need it
        // (codebook, x) are in flight; the logits load goes first
        e = RT ? 0 : a.rhs[start];
    }
    float rlog[1];
    if constexpr (RT) {
        static_assert(WG == ROUTE_THREADS, "the in-kernel router takes 256 threads");
        route_load<TBF16, 1>(a.logits + (int64_t)(start / a.k) * a.E, (int)a.E, rlog);
    }

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rg = wave / KS, kp = wave % KS;        // row group, K part
    const int n = lane & 15, q = lane >> 4;
    const int K = (int)a.K, CPR = K / 8;
    // this workgroup's column blocks of RW weight rows: cblk of them (1 at KS > 1)
    const int nbt = (int)((a.N + RW - 1) / RW);
    const int b0 = (int)blockIdx.x * a.cblk;
    const int nb = MB ? (nbt - b0 < a.cblk ? nbt - b0 : a.cblk) : 1;
    auto row_of = [&](int g) { return (b0 + g) * RW + rg * 16 + n; };

    if (e < 0 || e >= a.E) {                         // pair mode: an out-of-range expert gives 0
        for (int g = 0; g < nb; g++) {
            const int row = row_of(g);
            if (kp == 0 && q == 0 && row < a.N) a.y[(int64_t)start * a.N + row] = 0;
        }
        return;
    }

    const int xstride = K * 2 + 16;                  // bytes per staged x row (padded: rows on distinct banks)
    const bool two_cb = NSET == 2 && a.cb1 != a.cb0;
    const int cbb = (a.kc + 63) / 64;                // 1 KB blocks per codebook
    const int nblk = cbb * (two_cb ? 2 : 1);
    unsigned char* cbl0 = smem;
    unsigned char* cbl1 = smem + (two_cb ? (size_t)cbb * 1024 : 0);
    unsigned char* xs = smem + (size_t)nblk * 1024;
    f32x4* red = (f32x4*)(xs + (size_t)a.tile_rows * xstride);   // [4 waves][NSET][64], KS > 1

    // Sorted row ids of the tile, by scalar loads (tracked apart from the
    // vector loads, so waiting for them drains nothing of the code stream;
    // the sort kernel wrote `sorted` before this launch, and a constant
    // address-space view makes uniform reads scalar).  x row = row id /
    // lhs_div, by multiply-high with the host's magic (exact for the row
    // ids the host admits).
    typedef const __attribute__((address_space(4))) int32_t* cint_p;
    const cint_p srt = (cint_p)(a.tiles ? a.sorted + start : nullptr);
    auto rowid = [&](int m) -> uint32_t {
        return a.tiles ? (uint32_t)srt[m] : a.pairs ? (uint32_t)prow_s[m] : (uint32_t)start;
    };
    auto xrow_of = [&](int m) -> int {
        const uint32_t r = rowid(m);
        return a.lhs_magic ? (int)__umulhi(r, a.lhs_magic) : (int)r;
    };

    // ---- staging, every load issued before any wait:
    //  1. the codebook(s): each wave loads 8 KB blocks of 1 KB at once, then
    //     stores them (entries past kc read 0 and are never gathered: codes
    //     are clamped to kc - 1);
    //  2. the first x pieces of the tile (8 bf16 -> 8 fp16 per piece, at most
    //     XB per thread in flight);
    //  3. this lane's codes and row scales (the HBM stream);
    //  then the x pieces are converted into LDS and the rest of x staged.
    const __amdgpu_buffer_rsrc_t rcb0 = make_rsrc(a.cb0, (int64_t)a.kc * 16);
    const __amdgpu_buffer_rsrc_t rcb1 = make_rsrc(a.cb1, (int64_t)a.kc * 16);
    for (int j0 = wave; j0 < nblk; j0 += 32) {
        u32x4 v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int j = j0 + 4 * u;
            const bool second = j >= cbb;
            const int p = (j - (second ? cbb : 0)) * 64 + lane;
            v[u] = __builtin_amdgcn_raw_buffer_load_b128(second ? rcb1 : rcb0,
                                                         j < nblk && p < a.kc ? p * 16 : (int)NONE, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (j0 + 4 * u < nblk) *(u32x4*)(smem + (size_t)(j0 + 4 * u) * 1024 + lane * 16) = v[u];
    }
    // x pieces: a batch is rows m0 .. m0 + XB - 1 at piece k8 of each (row ids
    // by scalar loads: m is uniform); rows past the tile read 0, unstored
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, a.X * a.K * 2);
    constexpr int XB = 8;
    auto x_batch_load = [&](int m0, int k8, u32x4 (&v)[XB]) {
#pragma unroll
        for (int i = 0; i < XB; i++) {
            const int m = m0 + i;
            uint32_t off = NONE;
            if (m < count && k8 < CPR) {
                const int xr = xrow_of(m);
                if (xr >= 0 && xr < a.X) off = (uint32_t)(((int64_t)xr * K + k8 * 8) * 2);
            }
            v[i] = __builtin_amdgcn_raw_buffer_load_b128(rx, (int)off, 0, 0);
        }
    };
    auto x_batch_store = [&](int m0, int k8, const u32x4 (&v)[XB]) {
#pragma unroll
        for (int i = 0; i < XB; i++)
            if (m0 + i < count && k8 < CPR) *(u32x4*)(xs + (size_t)(m0 + i) * xstride + k8 * 16) = bf16x8_to_f16x8(v[i]);
    };
    u32x4 xv[XB];
    x_batch_load(0, tid, xv);

    if constexpr (RT) {
        __shared__ RouteLdsT<ROUTE_THREADS> rsm;     // E <= 256
        route_from<TBF16, 1>(rlog, (int)a.E, a.k, rsm);
        const int s = start % a.k;
        e = __builtin_amdgcn_readfirstlane(rsm.sel_e[s]);
        if (blockIdx.x == 0 && tid == 0) {
            a.inds_out[start] = e;
            a.scores_out[start] = f32_to_bf16(rsm.sel_p[s]);
        }
    }

    // ---- this lane's codes and row scale of column block g (the HBM
    //      stream), into register set `slot`
    const int64_t ebase = (int64_t)e * a.erows;
    const int cfirst = kp * (CPR / KS) + q * CPL;              // this lane's first code of its row
    uint32_t cw[MB ? 2 : 1][NSET][LW];
    // row scales kept as loaded (fp16 bits) and converted where the epilogue
    // uses them: a conversion at the load makes the compiler wait for that
    // load -- and, loads completing in order, for the block's code loads
    // before it -- right where the next block's codes are prefetched
    uint16_t scl[MB ? 2 : 1][NSET];
    // A block past the workgroup's last (g >= nb) loads nothing: every
    // offset is past its buffer.  So the next block's loads can be issued on
    // every path -- behind a branch, the compiler's vmcnt waits would take the
    // path without them and wait for the prefetch right after issuing it.
    auto load_codes = [&](int g, int slot_) {
        const int slot = MB ? slot_ : 0;
        const int row = row_of(g);
        const int crow = row < a.N ? row : (int)a.N - 1;       // rows past N re-read row N-1, never stored
        const bool live = g < nb;
#pragma unroll
        for (int s = 0; s < NSET; s++) {
            const char* cb = (const char*)(s ? a.codes1 : a.codes0) + ebase * CPR * CB;
            const __amdgpu_buffer_rsrc_t rc = make_rsrc(cb, a.N * CPR * CB);
            const uint32_t lo = live ? (uint32_t)((crow * CPR + cfirst) * CB) : NONE;
            if constexpr (LW % 4 == 0) {
#pragma unroll
                for (int i = 0; i < LW; i += 4) {
                    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rc, (int)(lo + i * 4), 0, AUX_NT);
                    cw[slot][s][i] = v.x; cw[slot][s][i + 1] = v.y; cw[slot][s][i + 2] = v.z; cw[slot][s][i + 3] = v.w;
                }
            } else if constexpr (LW % 2 == 0) {
#pragma unroll
                for (int i = 0; i < LW; i += 2) {
                    const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rc, (int)(lo + i * 4), 0, AUX_NT);
                    cw[slot][s][i] = v.x; cw[slot][s][i + 1] = v.y;
                }
            } else {
#pragma unroll
                for (int i = 0; i < LW; i++)
                    cw[slot][s][i] = __builtin_amdgcn_raw_buffer_load_b32(rc, (int)(lo + i * 4), 0, AUX_NT);
            }
            const __amdgpu_buffer_rsrc_t rsc = make_rsrc((s ? a.sc1 : a.sc0) + ebase, a.N * 2);
            scl[slot][s] = __builtin_amdgcn_raw_buffer_load_b16(rsc, live ? crow * 2 : (int)NONE, 0, 0);
        }
    };
    load_codes(0, 0);

    // ---- x -> LDS (the first batch waits for its own loads only), then
    //      the workgroup
    x_batch_store(0, tid, xv);
    for (int k0 = 0; k0 < CPR; k0 += WG)
        for (int m0 = k0 ? 0 : XB; m0 < count; m0 += XB) {
            x_batch_load(m0, k0 + tid, xv);
            x_batch_store(m0, k0 + tid, xv);
        }
    lds_barrier();

    const int mrow = n < count ? n : count - 1;                 // A rows past the tile repeat a real row
    const unsigned char* xa = xs + (size_t)mrow * xstride + (size_t)cfirst * 16;
    // ---- column block g from register set `slot`: MFMA over the lane's
    //      codes, the K parts summed, the epilogue's values (bf16) into res;
    //      false for the waves whose K part another wave finishes.  The
    //      stores wait for the end of the kernel: a store pending beside the
    //      next block's loads makes the compiler's vmcnt waits drain them all
    //      (loads and stores do not complete in one order).
    auto compute = [&](int g, int slot_, uint16_t (&res)[4]) -> bool {
        const int slot = MB ? slot_ : 0;
        f32x4 acc[NSET];
#pragma unroll
        for (int s = 0; s < NSET; s++) acc[s] = f32x4{0.f, 0.f, 0.f, 0.f};
        // operands of KB codes per group, group j + 1's LDS reads issued
        // before group j's MFMAs (the scheduling barriers keep them there):
        // one LDS round trip per group instead of one per code (left to
        // itself the compiler waits for each gather before its MFMA)
        constexpr int KB = CPL % 4 == 0 ? 4 : CPL % 2 == 0 ? 2 : 1;
        u32x4 av[2][KB], bv[2][NSET][KB];
        auto fetch = [&](int kb0, int buf) {
#pragma unroll
            for (int j = 0; j < KB; j++) {
                const int kb = kb0 + j;
                av[buf][j] = *(const u32x4*)(xa + kb * 16);
#pragma unroll
                for (int s = 0; s < NSET; s++) {
                    uint32_t code;
                    if constexpr (CB == 1) code = (cw[slot][s][kb >> 2] >> (8 * (kb & 3))) & 0xffu;
                    else code = (cw[slot][s][kb >> 1] >> (16 * (kb & 1))) & 0xffffu;
                    code = __builtin_elementwise_min(code, (uint32_t)(a.kc - 1));
                    bv[buf][s][j] = *(const u32x4*)((s ? cbl1 : cbl0) + code * 16);
                }
            }
        };
        fetch(0, 0);
#pragma unroll
        for (int kb0 = 0; kb0 < CPL; kb0 += KB) {
            const int buf = (kb0 / KB) & 1;
            if (kb0 + KB < CPL) fetch(kb0 + KB, buf ^ 1);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < KB; j++)
#pragma unroll
                for (int s = 0; s < NSET; s++) acc[s] = mfma_f16(av[buf][j], bv[buf][s][j], acc[s]);
            __builtin_amdgcn_sched_barrier(0);
        }

        // K parts of a row group summed in LDS, in part order (one column
        // block per workgroup at KS > 1)
        if constexpr (KS > 1) {
#pragma unroll
            for (int s = 0; s < NSET; s++) red[(wave * NSET + s) * 64 + lane] = acc[s];
            lds_barrier();
            if (kp != 0) return false;
#pragma unroll
            for (int s = 0; s < NSET; s++) {
                f32x4 t = red[(wave * NSET + s) * 64 + lane];
#pragma unroll
                for (int j = 1; j < KS; j++) t += red[((wave + j) * NSET + s) * 64 + lane];
                acc[s] = t;
            }
        }

        // epilogue: lane holds D[m = 4q + i][n]
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float out = vqm_bf16r(f16_to_f32(scl[slot][0]) * acc[0][i]);
            if constexpr (NSET == 2) {     // round(round(silu_f32(gate)) * up)
                const float up = vqm_bf16r(f16_to_f32(scl[slot][1]) * acc[1][i]);
                out = silu_bf16r(out) * up;
            }
            res[i] = f32_to_bf16(out);
        }
        return true;
    };
    auto store = [&](int g, const uint16_t (&res)[4]) {
        const int row = row_of(g);
        if (row >= a.N) return;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int m = 4 * q + i;
            if (m >= count) continue;
            const int64_t r = a.tiles || a.pairs ? prow_s[m] : start;
            a.y[r * a.N + row] = res[i];
        }
    };
    if constexpr (MB) {
        // two register sets: block g + 1's codes stream in while block g
        // computes; the loads of a block past nb read nothing, so they are
        // issued on every path (a load behind a branch would leave the
        // compiler's vmcnt count at the path without it, and the next
        // block's prefetch would be waited for right after its issue)
        uint16_t res[VQM_MAX_CBLK][4];
#pragma unroll
        for (int g = 0; g < VQM_MAX_CBLK; g++) {
            load_codes(g + 1, (g + 1) & 1);
            if (g < nb) compute(g, g & 1, res[g]);
        }
#pragma unroll
        for (int g = 0; g < VQM_MAX_CBLK; g++)
            if (g < nb) store(g, res[g]);
    } else {
        uint16_t res[4];
        if (compute(0, 0, res)) store(0, res);
    }
}


size_t vq_mfma_lds(int64_t K, int kc, bool two_cb, int tile_rows, int nset, int ks) {
    return (size_t)((kc + 63) / 64) * 1024 * (two_cb ? 2 : 1) + (size_t)tile_rows * (K * 2 + 16) +
           (ks > 1 ? (size_t)4 * nset * 64 * 16 : 0);
}

// code words per lane at K split KS, or 0 if the lanes' code runs are not
// whole 32-bit words
static int vq_lw(int64_t K, int code_bytes, int ks) {
    const int64_t b = K * code_bytes;
    return b % (128 * ks) ? 0 : (int)(b / (128 * ks));
}

#define KMI_VQM_SHAPES(X)                                                          \
    X(1, 4, 1) X(1, 2, 2) X(1, 1, 4)          /* K = 512, u8 */                     \
    X(1, 6, 1) X(1, 3, 2)                     /* K = 768 */                         \
    X(1, 8, 1) X(1, 4, 2) X(1, 2, 4)          /* K = 1024 */                        \
    X(1, 12, 1) X(1, 6, 2) X(1, 3, 4)         /* K = 1536 */                        \
    X(1, 16, 1) X(1, 8, 2) X(1, 4, 4)         /* K = 2048 */                        \
    X(1, 22, 1) X(1, 11, 2)                   /* K = 2816 */                        \
    X(1, 32, 1) X(1, 16, 2) X(1, 8, 4)        /* K = 4096 */                        \
    X(2, 8, 1) X(2, 4, 2) X(2, 2, 4)          /* K = 512, u16 */                    \
    X(2, 12, 1) X(2, 6, 2) X(2, 3, 4)         /* K = 768 */                         \
    X(2, 16, 1) X(2, 8, 2) X(2, 4, 4)         /* K = 1024 */                        \
    X(2, 24, 1) X(2, 12, 2) X(2, 6, 4)        /* K = 1536 */                        \
    X(2, 32, 1) X(2, 16, 2) X(2, 8, 4)        /* K = 2048 */                        \
    X(2, 22, 2) X(2, 11, 4)                   /* K = 2816 */                        \
    X(2, 32, 2) X(2, 16, 4)                   /* K = 4096 */

static bool vq_has_kernel(int code_bytes, int lw, int ks) {
#define KMI_VQM_HAS(CB_, LW_, KS_) if (code_bytes == CB_ && lw == LW_ && ks == KS_) return true;
    KMI_VQM_SHAPES(KMI_VQM_HAS)
#undef KMI_VQM_HAS
    return false;
}

bool vq_mfma_supported(int64_t K, int code_bytes, int kc, bool two_cb) {
    if (K % 128) return false;
    bool any = false;
    for (int ks = 1; ks <= 4; ks *= 2) any = any || vq_has_kernel(code_bytes, vq_lw(K, code_bytes, ks), ks);
    return any && vq_mfma_lds(K, kc, two_cb, TM, 2, 4) <= 160 * 1024;
}

// column blocks per workgroup for 2-byte codes without a K split:
// VQM_MAX_CBLK (4), so a workgroup's 64 KB codebook staging and x staging
// serve 256 weight rows (measured at 128 experts, 16 tokens, 4096 x 8: 103
// -> 90 us; 2, 3, 6 and 8 blocks were slower); 1-byte codes keep one block
// (4 KB codebooks; the smaller register set runs more waves)
static int vq_cblk(int64_t nbt) { return (int)(VQM_MAX_CBLK < nbt ? VQM_MAX_CBLK : nbt); }

int launch_vq_mfma(const VqmArgs& a_in, int code_bytes, int nset, int64_t ntiles, hipStream_t st) {
    VqmArgs a = a_in;
    const bool two_cb = nset == 2 && a.cb1 != a.cb0;
    if (a.tile_rows < 1 || a.tile_rows > TM || (!a.tiles && !a.pairs && a.tile_rows != 1)) {
        set_error("vq_mfma: tile rows %d", a.tile_rows);
        return EINVAL_ARG;
    }
    if (a.pairs && (a.tiles || a.logits || !pair_tiles_fit(a.pairs, a.E, a.tile_rows))) {
        set_error("vq_mfma: %d pairs over %lld experts: no tiles formed in the kernel", a.pairs, (long long)a.E);
        return EINVAL_ARG;
    }
    // widest K split (up to 4) that the grid needs to reach ~512 workgroups
    const int64_t base = ceil_div(a.N, 64) * ntiles;
    int ks = 0;
    for (int c = 1; c <= 4; c *= 2) {
        if (!vq_has_kernel(code_bytes, vq_lw(a.K, code_bytes, c), c)) continue;
        if (ks == 0 || base * ks < 512) ks = c;
    }
    if (ks == 0) {
        set_error("vq_mfma: no kernel for K=%lld, %d-byte codes", (long long)a.K, code_bytes);
        return EINVAL_ARG;
    }
    const int lw = vq_lw(a.K, code_bytes, ks);
    size_t lds = vq_mfma_lds(a.K, a.kc, two_cb, a.tile_rows, nset, ks);
    const size_t cbl = (size_t)((a.kc + 63) / 64) * 1024 * (two_cb ? 2 : 1);
    if (a.pairs && lds < cbl + sizeof(PairTileLds)) lds = cbl + sizeof(PairTileLds);   // the tile's working space
    const int64_t nbt = ceil_div(a.N, 64 / ks);
    const bool rt = a.logits != nullptr;
    if (rt && (a.tiles || nset != 2 || a.E > ROUTE_THREADS || a.k < 1 || a.k > 8)) {
        set_error("vq_mfma: in-kernel routing is for pair mode, gate/up, E <= %d, k <= 8", ROUTE_THREADS);
        return EINVAL_ARG;
    }
    if (lds + (rt ? sizeof(RouteLdsT<ROUTE_THREADS>) : 0) > 160 * 1024) {   // the router's state is static LDS
        set_error("vq_mfma: %zu bytes of LDS", lds);
        return EINVAL_ARG;
    }
    const bool mb = code_bytes == 2 && ks == 1 && !rt;
    a.cblk = mb ? vq_cblk(nbt) : 1;
    const dim3 grid((unsigned)ceil_div(nbt, a.cblk), (unsigned)ntiles);
#define KMI_VQM_GO(CB_, NS_, LW_, KS_, MB_, RT_)                                                  \
    {                                                                                            \
        allow_dynamic_lds_once((const void*)vq_mfma<CB_, NS_, LW_, KS_, MB_, RT_>);              \
        vq_mfma<CB_, NS_, LW_, KS_, MB_, RT_><<<grid, WG, lds, st>>>(a);                         \
        return OK;                                                                               \
    }
#define KMI_VQM_ONE(CB_, NS_, LW_, KS_)                                                          \
    if (code_bytes == CB_ && nset == NS_ && lw == LW_ && ks == KS_) {                            \
        constexpr bool MB_ = CB_ == 2 && KS_ == 1;                                               \
        if constexpr (NS_ == 2) {                                                                \
            if (rt) KMI_VQM_GO(CB_, NS_, LW_, KS_, false, true)                                  \
        }                                                                                        \
        KMI_VQM_GO(CB_, NS_, LW_, KS_, MB_, false)                                               \
    }
#define KMI_VQM_LAUNCH(CB_, LW_, KS_) KMI_VQM_ONE(CB_, 1, LW_, KS_) KMI_VQM_ONE(CB_, 2, LW_, KS_)
    KMI_VQM_SHAPES(KMI_VQM_LAUNCH)
#undef KMI_VQM_LAUNCH
#undef KMI_VQM_ONE
#undef KMI_VQM_GO
    set_error("vq_mfma: no kernel for K=%lld, %d-byte codes", (long long)a.K, code_bytes);
    return EINVAL_ARG;
}

// =============================================================================
// vq_down_tok: the down projection of a few tokens, token-major.  A
// workgroup owns 16 output rows of one token; wave w takes the token's
// slots w, w + 4, ..  Per slot, lane (n, q) holds its row's q-th quarter of
// the codes and runs one MFMA per code with the slot's act row in every A
// row (so D is the same in every row), gathering the codebook vector from
// LDS as the B operand.  y = round(scale * acc); with scores the slots'
// round(y * score) are summed in slot order in float64 and rounded once, as
// moe_combine does, so the result is the combine of the y this kernel
// writes without scores, bit for bit.  An out-of-range expert gives y = 0.
template <int CB, int LW>
__global__ __launch_bounds__(WG) void vq_down_tok(VqdArgs a) {
    constexpr int CPL = LW * 4 / CB;                 // codes per lane
    extern __shared__ __align__(16) unsigned char smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 15, q = lane >> 4;
    const int t = (int)blockIdx.y;
    const int64_t row0 = (int64_t)blockIdx.x * 16;
    const int64_t row = row0 + n;
    const int K = (int)a.K, CPR = K / 8, k = a.k;
    const int xstride = K * 2 + 16;
    const int cbb = (a.kc + 63) / 64;
    unsigned char* xs = smem + (size_t)cbb * 1024;                      // [k][K] fp16
    float* prod = (float*)(xs + (size_t)k * xstride);                   // [k][16]

    // codebook and the token's k act rows (fp16) by batches of loads
    const __amdgpu_buffer_rsrc_t rcb = make_rsrc(a.cb, (int64_t)a.kc * 16);
    for (int j0 = wave; j0 < cbb; j0 += 16) {
        u32x4 v[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int j = j0 + 4 * u, p = j * 64 + lane;
            v[u] = __builtin_amdgcn_raw_buffer_load_b128(rcb, j < cbb && p < a.kc ? p * 16 : (int)NONE, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < 4; u++)
            if (j0 + 4 * u < cbb) *(u32x4*)(smem + (size_t)(j0 + 4 * u) * 1024 + lane * 16) = v[u];
    }
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x + (int64_t)t * k * K, (int64_t)k * K * 2);
    const int xitems = k * CPR;
    for (int f0 = tid; f0 < xitems; f0 += WG * 4) {
        u32x4 v[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int f = f0 + WG * i;
            v[i] = __builtin_amdgcn_raw_buffer_load_b128(rx, f < xitems ? f * 16 : (int)NONE, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int f = f0 + WG * i;
            if (f < xitems) *(u32x4*)(xs + (size_t)(f / CPR) * xstride + (f % CPR) * 16) = bf16x8_to_f16x8(v[i]);
        }
    }

    // this wave's slots, two at a time: codes and scales of both issued together
    const int crow = (int)(row < a.N ? row : a.N - 1);
    const int cfirst = q * CPL;
    // the scale stays as loaded (fp16 bits) until the epilogue, so the next
    // slots' prefetch is not waited for at its issue
    auto load_slot = [&](int s, uint32_t (&cw)[LW], uint16_t& scl, bool& ok) {
        const int e = s < k ? a.inds[(int64_t)t * k + s] : -1;
        ok = e >= 0 && e < a.E;
        const char* base = (const char*)a.codes + (int64_t)(ok ? e : 0) * a.N * CPR * CB;
        const __amdgpu_buffer_rsrc_t rc = make_rsrc(base, ok ? a.N * CPR * CB : 0);
        const uint32_t lo = (uint32_t)((crow * CPR + cfirst) * CB);
        if constexpr (LW % 4 == 0) {
#pragma unroll
            for (int i = 0; i < LW; i += 4) {
                const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rc, (int)(lo + i * 4), 0, AUX_NT);
                cw[i] = v.x; cw[i + 1] = v.y; cw[i + 2] = v.z; cw[i + 3] = v.w;
            }
        } else if constexpr (LW % 2 == 0) {
#pragma unroll
            for (int i = 0; i < LW; i += 2) {
                const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rc, (int)(lo + i * 4), 0, AUX_NT);
                cw[i] = v.x; cw[i + 1] = v.y;
            }
        } else {
#pragma unroll
            for (int i = 0; i < LW; i++) cw[i] = __builtin_amdgcn_raw_buffer_load_b32(rc, (int)(lo + i * 4), 0, AUX_NT);
        }
        const __amdgpu_buffer_rsrc_t rsc = make_rsrc(a.sc + (int64_t)(ok ? e : 0) * a.N, ok ? a.N * 2 : 0);
        scl = __builtin_amdgcn_raw_buffer_load_b16(rsc, crow * 2, 0, 0);
    };
    const int nslot = (k - wave + 3) / 4;            // slots wave, wave + 4, ..
    uint32_t cw[2][LW];
    uint16_t scl[2];
    bool okk[2];
    load_slot(wave, cw[0], scl[0], okk[0]);
    load_slot(wave + 4, cw[1], scl[1], okk[1]);

    lds_barrier();

    for (int j0 = 0; j0 < nslot; j0 += 2) {
        if (j0 > 0) {
            load_slot(wave + 4 * j0, cw[0], scl[0], okk[0]);
            load_slot(wave + 4 * (j0 + 1), cw[1], scl[1], okk[1]);
        }
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int s = wave + 4 * (j0 + u);
            if (j0 + u >= nslot) continue;
            const unsigned char* xa = xs + (size_t)s * xstride + (size_t)cfirst * 16;
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
            // groups of KB codes, group j + 1's reads issued before group j's MFMAs
            constexpr int KB = CPL % 4 == 0 ? 4 : CPL % 2 == 0 ? 2 : 1;
            u32x4 av[2][KB], bv[2][KB];
            auto fetch = [&](int kb0, int buf) {
#pragma unroll
                for (int j = 0; j < KB; j++) {
                    const int kb = kb0 + j;
                    av[buf][j] = *(const u32x4*)(xa + kb * 16);
                    uint32_t code;
                    if constexpr (CB == 1) code = (cw[u][kb >> 2] >> (8 * (kb & 3))) & 0xffu;
                    else code = (cw[u][kb >> 1] >> (16 * (kb & 1))) & 0xffffu;
                    code = __builtin_elementwise_min(code, (uint32_t)(a.kc - 1));
                    bv[buf][j] = *(const u32x4*)(smem + code * 16);
                }
            };
            fetch(0, 0);
#pragma unroll
            for (int kb0 = 0; kb0 < CPL; kb0 += KB) {
                const int buf = (kb0 / KB) & 1;
                if (kb0 + KB < CPL) fetch(kb0 + KB, buf ^ 1);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int j = 0; j < KB; j++) acc = mfma_f16(av[buf][j], bv[buf][j], acc);
                __builtin_amdgcn_sched_barrier(0);
            }
            // D[m][n] is the same for every m: lanes q = 0 hold it in item 0
            const float y = okk[u] ? vqm_bf16r(f16_to_f32(scl[u]) * acc[0]) : 0.f;
            if (q == 0) {
                if (a.scores) {
                    const float sc = bf16_to_f32(a.scores[(int64_t)t * k + s]);
                    prod[s * 16 + n] = vqm_bf16r(y * sc);
                } else if (row < a.N) {
                    a.out[((int64_t)t * k + s) * a.N + row] = f32_to_bf16(y);
                }
            }
        }
    }
    if (!a.scores) return;
    lds_barrier();
    if (tid < 16 && row0 + tid < a.N) {
        double acc = 0.0;
        for (int s = 0; s < k; s++) acc += (double)prod[s * 16 + tid];
        a.out[(int64_t)t * a.N + row0 + tid] = f32_to_bf16(vqm_f32_kept(acc));
    }
}

#define KMI_VQD_SHAPES(X)                                                        \
    X(1, 1) X(1, 2) X(1, 3) X(1, 4) X(1, 6) X(1, 8) X(1, 12) X(1, 16)            \
    X(2, 2) X(2, 4) X(2, 6) X(2, 8) X(2, 12) X(2, 16) X(2, 24) X(2, 32)

static int vqd_lw(int64_t K, int code_bytes) {
    const int64_t b = K * code_bytes;                // bytes of codes per row, 4 lanes
    return b % 128 ? 0 : (int)(b / 128);
}

bool vq_down_tok_supported(int64_t K, int code_bytes, int kc, int k) {
    const int lw = vqd_lw(K, code_bytes);
    bool has = false;
#define KMI_VQD_HAS(CB_, LW_) has = has || (code_bytes == CB_ && lw == LW_);
    KMI_VQD_SHAPES(KMI_VQD_HAS)
#undef KMI_VQD_HAS
    return has && k >= 1 && k <= 64 && vq_down_tok_lds(K, kc, k) <= 160 * 1024;
}

size_t vq_down_tok_lds(int64_t K, int kc, int k) {
    return (size_t)((kc + 63) / 64) * 1024 + (size_t)k * (K * 2 + 16) + (size_t)k * 16 * 4;
}

int launch_vq_down_tok(const VqdArgs& a, int code_bytes, hipStream_t st) {
    const int lw = vqd_lw(a.K, code_bytes);
    const size_t lds = vq_down_tok_lds(a.K, a.kc, a.k);
    const dim3 grid((unsigned)ceil_div(a.N, 16), (unsigned)a.T);
#define KMI_VQD_ONE(CB_, LW_)                                                                     \
    if (code_bytes == CB_ && lw == LW_) {                                                         \
        allow_dynamic_lds_once((const void*)vq_down_tok<CB_, LW_>);                              \
        vq_down_tok<CB_, LW_><<<grid, WG, lds, st>>>(a);                                          \
        return OK;                                                                                \
    }
    KMI_VQD_SHAPES(KMI_VQD_ONE)
#undef KMI_VQD_ONE
    set_error("vq_down_tok: no kernel for K=%lld, %d-byte codes", (long long)a.K, code_bytes);
    return EINVAL_ARG;
}

}  // namespace kmi
