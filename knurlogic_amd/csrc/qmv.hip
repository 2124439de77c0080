// Decode-shape quantized matmul for gfx950: M <= 16 activation rows per
// weight (dense) or per routed expert (gather_qmm).
//
//   y[m, n] = sum_k x[m, k] * (s[n, g] * q[n, k] + b[n, g])
//           = sum_g ( s[n, g] * P[m, n, g] + b[n, g] * X[m, g] ),
//   P[m, n, g] = sum_{k in g} x[m, k] q[n, k],   X[m, g] = sum_{k in g} x[m, k].
//
// The integer codes go to bf16 in registers without rounding (4-bit codes as
// "128 + q" by OR-ing the nibble into the mantissa of 128.0, 8-bit codes
// through cvt_f32_ubyte), so the only rounding is the fp32 accumulation; the
// per-group scale and bias are applied to fp32 partial sums.  x sits in LDS
// as bf16 (k pre-permuted to the unpack order) with its per-chunk sums.
//
// Two kernels:
//   qmv_valu  (M <= 4 per tile): HBM-bound streaming.  Each lane reads 16
//             contiguous bytes of a weight row per load (a wave reads 1 KB
//             of one row per instruction), dots them with x by
//             v_dot2c_f32_bf16, applies scale/bias per 16-byte chunk, and
//             the row is summed across the wave at the end.  No split-K.
//   qmv_mfma  (5..16 rows per tile): v_mfma_f32_16x16x32_bf16 on 16 weight
//             rows x 16 activation rows; split-K partials when the K slice
//             does not cover K.
//
// gather_qmm: a tile is (expert, <= MT rows routed to it), built on the GPU
// by sort_rows_by_expert, so each routed expert's weights are read once per
// tile.
#include "qmv_common.hpp"
#include "../../include/knurlogic_amd.h"

namespace kmi {
// =========================================================================
// qmv_mfma: <= 16 activation rows, 64 weight rows per workgroup, K slices.
// =========================================================================
constexpr int QM_ROWS_WG = 64;   // 4 waves x 16 weight rows
constexpr int QM_TILE = 16;      // activation rows per tile (MFMA M)
constexpr int QM_UNROLL = 8;     // groups whose loads are in flight per wave

template <int BITS, int GS>
__global__ __launch_bounds__(256) void qmv_mfma_kernel(QmvArgs a) {
    constexpr int EPW = 32 / BITS;
    constexpr int WPG = GS * BITS / 32;   // words of one row per group
    constexpr int WPL = WPG / 4;          // words per lane per group
    constexpr int MF = GS / 32;           // MFMAs per group

    extern __shared__ __align__(16) unsigned char smem[];
    Tile t;
    if (!resolve_tile(a, t)) return;
    const int64_t k0 = (int64_t)blockIdx.y * a.KS;
    int64_t k1 = k0 + a.KS;
    if (k1 > a.K) k1 = a.K;
    const int KSl = (int)(k1 - k0);
    const int ngr = KSl / GS;
    const int lds_stride = (int)a.KS + 8;
    uint16_t* xs = (uint16_t*)smem;                                   // [16][lds_stride]
    float* xg = (float*)(smem + (size_t)QM_TILE * lds_stride * 2);    // [ngr][16]

    const int tid = threadIdx.x;
    const int runs = KSl / 8;
    for (int idx = tid; idx < (int)t.count * runs; idx += blockDim.x) {
        const int m = idx / runs, r = idx - m * runs;
        const int64_t xrow = x_row_of(a, t.start + m);
        u32x4 v = {0u, 0u, 0u, 0u};
        if (xrow >= 0 && xrow < a.Xrows) v = *(const u32x4*)(a.x + xrow * a.K + k0 + (int64_t)r * 8);
        float dummy = 0.f;
        *(u32x4*)(xs + m * lds_stride + r * 8) = permute8<BITS>(v, dummy);
    }
    __syncthreads();
    for (int idx = tid; idx < ngr * QM_TILE; idx += blockDim.x) {
        const int g = idx / QM_TILE, m = idx - g * QM_TILE;
        float sum = 0.f;
        if (m < t.count) {
            const uint16_t* p = xs + m * lds_stride + g * GS;
            for (int i = 0; i < GS; i += 8) {
                const u32x4 v = *(const u32x4*)(p + i);
#pragma unroll
                for (int e = 0; e < 4; e++) sum += bf16_to_f32(v[e] & 0xffffu) + bf16_to_f32(v[e] >> 16);
            }
        }
        xg[idx] = sum;
    }
    __syncthreads();

    const int lane = tid & 63, wave = tid >> 6;
    const int nl = lane & 15, j = lane >> 4;
    const int64_t n = (int64_t)blockIdx.x * QM_ROWS_WG + wave * 16 + nl;
    const bool n_ok = n < a.N;
    const int64_t nn = n_ok ? n : (a.N - 1);
    const int64_t wpr = a.K / EPW, gpr = a.K / GS;
    const uint32_t* wrow = a.w + ((int64_t)t.expert * a.N + nn) * wpr + (k0 / EPW) + j * WPL;
    const uint16_t* srow = a.s + ((int64_t)t.expert * a.N + nn) * gpr + k0 / GS;
    const uint16_t* brow = a.b + ((int64_t)t.expert * a.N + nn) * gpr + k0 / GS;
    const bool a_ok = nl < t.count;
    const uint16_t* xa = xs + nl * lds_stride + j * (GS / 4);

    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int g0 = 0; g0 < ngr; g0 += QM_UNROLL) {
        const int nu = (ngr - g0) < QM_UNROLL ? (ngr - g0) : QM_UNROLL;
        uint32_t wv[QM_UNROLL][WPL];
        float sv[QM_UNROLL], bv[QM_UNROLL];
#pragma unroll
        for (int u = 0; u < QM_UNROLL; u++) {
            if (u < nu) {
                const uint32_t* p = wrow + (int64_t)(g0 + u) * WPG;
                if constexpr (WPL == 1) {
                    wv[u][0] = p[0];
                } else if constexpr (WPL == 2) {
                    u32x2 tt = *(const u32x2*)p;
                    wv[u][0] = tt.x; wv[u][1] = tt.y;
                } else {
#pragma unroll
                    for (int q = 0; q < WPL; q += 4) {
                        u32x4 tt = *(const u32x4*)(p + q);
                        wv[u][q] = tt.x; wv[u][q + 1] = tt.y; wv[u][q + 2] = tt.z; wv[u][q + 3] = tt.w;
                    }
                }
                sv[u] = bf16_to_f32(srow[g0 + u]);
                bv[u] = bf16_to_f32(brow[g0 + u]);
            }
        }
#pragma unroll
        for (int u = 0; u < QM_UNROLL; u++) {
            if (u < nu) {
                const int g = g0 + u;
                f32x4 P = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int tt = 0; tt < MF; tt++) {
                    u32x4 A = {0u, 0u, 0u, 0u};
                    if (a_ok) A = *(const u32x4*)(xa + g * GS + tt * 8);
                    u32x4 B;
                    if constexpr (BITS == 4) {
                        B = nibbles_to_bf16_magic(wv[u][tt]);
                    } else {
                        const uint32_t w0 = wv[u][2 * tt], w1 = wv[u][2 * tt + 1];
                        B.x = bytes_to_bf16x2(w0, 0);
                        B.y = bytes_to_bf16x2(w0, 2);
                        B.z = bytes_to_bf16x2(w1, 0);
                        B.w = bytes_to_bf16x2(w1, 2);
                    }
                    P = mfma16x16x32(A, B, P);
                }
                const float s = sv[u];
                const float bb = (BITS == 4) ? __builtin_fmaf(-128.f, s, bv[u]) : bv[u];
                const f32x4 X = *(const f32x4*)(xg + g * QM_TILE + 4 * j);
#pragma unroll
                for (int i = 0; i < 4; i++) acc[i] = __builtin_fmaf(s, P[i], __builtin_fmaf(bb, X[i], acc[i]));
            }
        }
    }

    if (!n_ok) return;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int m = 4 * j + i;
        if (m >= t.count) continue;
        const int64_t row = y_row_of(a, t.start + m);
        if (a.S == 1) a.y[row * a.N + n] = f32_to_bf16(acc[i]);
        else a.partial[((int64_t)blockIdx.y * a.rows + row) * a.N + n] = acc[i];
    }
}

// y[r, n] = bf16(sum_s partial[s, r, n]), slices summed in order.  Rows of
// pairs with an out-of-range expert (gather) are left alone here: the sort
// kernel zeroed them in y and they have no partials.
__global__ __launch_bounds__(256) void qmv_reduce(const float* __restrict__ partial, int S,
                                                  int64_t count, int64_t N,
                                                  const int32_t* __restrict__ rhs, int64_t Mper,
                                                  int64_t E, uint16_t* __restrict__ y) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= count) return;
    if (rhs) {
        const int e = rhs[i / N / Mper];
        if (e < 0 || e >= E) return;
    }
    float acc = 0.f;
    for (int s = 0; s < S; s++) acc += partial[(int64_t)s * count + i];
    y[i] = f32_to_bf16(acc);
}

// ---- GPU grouping of rows by expert (one workgroup) --------------------------
// Rows r = p*Mper + m of pairs p with expert rhs[p] are listed grouped by
// expert in `sorted`, and each expert's segment is cut into tiles of <= TM
// rows: tiles[t] = (expert, start, count); unused tile slots get count 0.
// Rows of pairs with an out-of-range expert are zeroed in y and never listed
// (the index arrays are not validated on the host).
constexpr int SORT_THREADS = 1024;

__global__ __launch_bounds__(SORT_THREADS) void sort_rows_by_expert(
    const int32_t* __restrict__ rhs, int64_t P, int64_t Mper, int E, int TM,
    int32_t* __restrict__ sorted, int32_t* __restrict__ tiles, int max_tiles,
    int32_t* __restrict__ offsets /* [E+1] */, uint16_t* __restrict__ y, int64_t N) {
    extern __shared__ int32_t sh[];
    int32_t* cnt = sh;            // [E]
    int32_t* base = sh + E;       // [E]  row offset, then cursor
    int32_t* tbase = sh + 2 * E;  // [E]  first tile of the expert
    const int tid = threadIdx.x;
    for (int e = tid; e < E; e += blockDim.x) cnt[e] = 0;
    for (int t = tid; t < max_tiles; t += blockDim.x) {
        tiles[3 * t + 0] = 0; tiles[3 * t + 1] = 0; tiles[3 * t + 2] = 0;
    }
    __syncthreads();
    for (int64_t p = tid; p < P; p += blockDim.x) {
        const int e = rhs[p];
        if (e >= 0 && e < E) atomicAdd(&cnt[e], (int)Mper);
    }
    __syncthreads();
    if (tid == 0) {
        int run = 0, trun = 0;
        for (int e = 0; e < E; e++) {
            base[e] = run;
            tbase[e] = trun;
            offsets[e] = run;
            run += cnt[e];
            trun += (cnt[e] + TM - 1) / TM;
        }
        offsets[E] = run;
    }
    __syncthreads();
    for (int e = tid; e < E; e += blockDim.x) {
        const int c = cnt[e];
        int t = tbase[e];
        for (int s = 0; s < c; s += TM, t++) {
            if (t < max_tiles) {
                tiles[3 * t + 0] = e;
                tiles[3 * t + 1] = base[e] + s;
                tiles[3 * t + 2] = (c - s) < TM ? (c - s) : TM;
            }
        }
    }
    __syncthreads();
    for (int64_t p = tid; p < P; p += blockDim.x) {
        const int e = rhs[p];
        if (e < 0 || e >= E) {
            for (int64_t i = 0; i < Mper * N; i++) y[p * Mper * N + i] = 0;
            continue;
        }
        const int pos = atomicAdd(&base[e], (int)Mper);
        for (int64_t m = 0; m < Mper; m++) sorted[pos + m] = (int32_t)(p * Mper + m);
    }
}

// ---- host side ----------------------------------------------------------------

enum class QmvKind { VALU1, VALU2, VALU4, MFMA };

static int tile_rows(QmvKind k) {
    switch (k) {
        case QmvKind::VALU1: return 1;
        case QmvKind::VALU2: return 2;
        case QmvKind::VALU4: return 4;
        default: return QM_TILE;
    }
}

static size_t valu_lds(int64_t K, int bits, int mt, int gs, const ValuShape& v) {
    const int64_t CK = 128 / bits;
    return (size_t)mt * (K + 8) * 2 + (size_t)mt * (K / CK) * 4 +
           (size_t)v.WV * v.RPW * (K / gs) * 4;
}

// Launch shape of the VALU kernel.  S: chunk slots per lane, all of K up to
// 8 slots (one load batch).  RPW: weight rows per wave, so the grid's waves
// over all tiles stay within what 256 CUs hold at once yet fill them.  WV:
// waves per workgroup, so the weight bytes a workgroup streams are at least
// 4x the x bytes it stages into LDS (x is read from L2 once per workgroup).
static ValuShape valu_shape(int64_t N, int64_t K, int bits, int64_t tiles, int mt) {
    const int64_t C = K / (128 / bits);
    const int64_t slots = ceil_div(C, 64);
    ValuShape v;
    v.S = slots <= 1 ? 1 : slots <= 2 ? 2 : slots <= 4 ? 4 : 8;
    const int64_t T = tiles > 0 ? tiles : 1;
    v.RPW = 1;
    if (mt == 1) {
        if (v.S <= 4 && N * T / 2 >= 4096) v.RPW = 2;
        if (v.S <= 2 && N * T / 4 >= 4096) v.RPW = 4;
    }
    const int64_t rows_target = (int64_t)16 * mt * 4 / bits;   // 16*mt at 4 bits, 8*mt at 8 bits
    const int64_t wv = ceil_div(rows_target, v.RPW);
    v.WV = wv <= 4 ? 4 : wv <= 8 ? 8 : 16;
    // no more waves per workgroup than the rows need
    while (v.WV > 4 && (int64_t)(v.WV / 2) * v.RPW >= N) v.WV /= 2;
    v.groups = ceil_div(N, (int64_t)v.WV * v.RPW);
    return v;
}

// Kernel choice by rows per tile: the VALU kernel while its LDS (x rows of
// the tile, their chunk sums, the workgroup's scales/biases) fits 64 KB at
// the shape it would launch with, else the MFMA kernel.
static QmvKind choose_kind(int64_t rows_per_tile, int64_t K, int64_t N, int64_t total_rows, int bits,
                           int gs) {
    const size_t cap = 64 * 1024;
    const QmvKind kinds[3] = {QmvKind::VALU1, QmvKind::VALU2, QmvKind::VALU4};
    const int mts[3] = {1, 2, 4};
    for (int i = 0; i < 3; i++) {
        if (rows_per_tile > mts[i]) continue;
        const ValuShape v = valu_shape(N, K, bits, ceil_div(total_rows, mts[i]), mts[i]);
        if (valu_lds(K, bits, mts[i], gs, v) <= cap) return kinds[i];
    }
    return QmvKind::MFMA;
}

struct MfmaPlan {
    int64_t KS;
    int S;
    size_t lds;
};

// K slice for the MFMA kernel: about 1024 workgroups over 256 CUs, the x
// tile within ~34 KB of LDS, slices a multiple of the group.
static MfmaPlan plan_mfma(int64_t K, int64_t N, int64_t tiles, int gs) {
    const int64_t nblk = ceil_div(N, QM_ROWS_WG);
    int64_t want_s = ceil_div(1024, nblk * (tiles > 0 ? tiles : 1));
    if (want_s < 1) want_s = 1;
    int64_t KS = ceil_div(K, want_s);
    KS = ceil_div(KS, gs) * gs;
    if (KS > 1024) KS = 1024;
    if (KS < gs) KS = gs;
    if (KS > K) KS = K;
    MfmaPlan p;
    p.KS = KS;
    p.S = (int)ceil_div(K, KS);
    p.lds = (size_t)QM_TILE * (KS + 8) * 2 + (size_t)(KS / gs) * QM_TILE * 4;
    return p;
}

static int launch_qmv(QmvKind k, const QmvArgs& a, int bits, int gs, dim3 grid, size_t lds,
                      hipStream_t st, const ValuShape* v = nullptr) {
    if (k != QmvKind::MFMA) {
        if (!launch_qmv_valu(bits, tile_rows(k), *v, a, grid, lds, st)) {
            set_error("qmv: no kernel for shape S=%d RPW=%d WV=%d", v->S, v->RPW, v->WV);
            return EINVAL_ARG;
        }
        KMI_CHECK_LAUNCH("qmv_valu");
        return OK;
    }
#define KMI_QMV(B, G) qmv_mfma_kernel<B, G><<<grid, 256, lds, st>>>(a)
    if (bits == 4) {
        if (gs == 32) KMI_QMV(4, 32);
        else if (gs == 64) KMI_QMV(4, 64);
        else KMI_QMV(4, 128);
    } else {
        if (gs == 32) KMI_QMV(8, 32);
        else if (gs == 64) KMI_QMV(8, 64);
        else KMI_QMV(8, 128);
    }
#undef KMI_QMV
    KMI_CHECK_LAUNCH("qmv");
    return OK;
}

int qmm_gemm(const void* x, int64_t M, int64_t K, int64_t N, const uint32_t* w,
             const void* scales, const void* biases, int group_size, int bits, void* y,
             void* workspace, size_t workspace_bytes, hipStream_t st);
size_t qmm_gemm_workspace(int64_t M, int64_t K, int64_t N);  // qmm.hip

static int check_common(int64_t K, int64_t N, int dtype, int gs, int bits) {
    KMI_CHECK_ARG(dtype == BF16, "quantized matmul: only bfloat16 activations are supported (got dtype %d)", dtype);
    KMI_CHECK_ARG(bits == 4 || bits == 8, "quantized matmul: bits %d not in {4, 8}", bits);
    KMI_CHECK_ARG(gs == 32 || gs == 64 || gs == 128, "quantized matmul: group_size %d not in {32, 64, 128}", gs);
    KMI_CHECK_ARG(K > 0 && K % gs == 0, "quantized matmul: K=%lld must be a multiple of the group %d",
                  (long long)K, gs);
    KMI_CHECK_ARG(K % 64 == 0, "quantized matmul: K=%lld must be a multiple of 64", (long long)K);
    KMI_CHECK_ARG(N > 0, "quantized matmul: N=%lld", (long long)N);
    // 32-bit buffer offsets: one weight matrix (one expert) under 2 GB
    KMI_CHECK_ARG(N * K * bits / 8 < (1LL << 31), "quantized matmul: a %lld x %lld weight exceeds 2 GB",
                  (long long)N, (long long)K);
    return OK;
}

// Workspace layout for gather_qmm: sorted rows [P*M] | tiles [3*max_tiles] |
// offsets [E+1] | (pad to 256) | partials [S, P*M, N] fp32 (MFMA kernel).
static int64_t gather_max_tiles(int64_t P, int64_t M, int64_t E, int tm) {
    const int64_t R = P * M;
    return (R < E ? R : E) + ceil_div(R, tm);
}

static size_t gather_index_bytes(int64_t P, int64_t M, int64_t E, int tm) {
    size_t b = (size_t)(P * M) * 4 + (size_t)gather_max_tiles(P, M, E, tm) * 12 + (size_t)(E + 1) * 4;
    return (b + 255) & ~(size_t)255;
}

// rows per tile for gather: average routed rows per active expert
static QmvKind gather_kind(int64_t P, int64_t M, int64_t E, int64_t K, int64_t N, int bits, int gs) {
    const int64_t R = P * M;
    const int64_t active = R < E ? R : E;
    const int64_t rpt = ceil_div(R, active);
    return choose_kind(rpt, K, N, R, bits, gs);
}

}  // namespace kmi

using namespace kmi;

extern "C" {

size_t kmi_qmm_workspace_bytes(int64_t M, int64_t K, int64_t N, int group_size, int bits) {
    if (M <= 0 || K <= 0 || N <= 0 || group_size <= 0 || (bits != 4 && bits != 8)) return 0;
    if (M > QM_TILE) return qmm_gemm_workspace(M, K, N);         // GEMM path (split-K partials)
    if (choose_kind(M, K, N, M, bits, group_size) != QmvKind::MFMA) return 0;   // VALU path
    MfmaPlan p = plan_mfma(K, N, 1, group_size);
    return p.S > 1 ? (size_t)p.S * M * N * sizeof(float) : 0;
}

int kmi_qmm(const void* x, int64_t M, int64_t K, int64_t N, const uint32_t* w,
            const void* scales, const void* biases, int dtype, int group_size,
            int bits, void* y, void* workspace, size_t workspace_bytes, void* stream) {
    clear_error();
    int rc = check_common(K, N, dtype, group_size, bits);
    if (rc) return rc;
    KMI_CHECK_ARG(M >= 0, "quantized_matmul: M=%lld", (long long)M);
    KMI_CHECK_ARG(w && scales && biases, "quantized_matmul: null pointer (affine needs biases)");
    if (M == 0) return OK;
    KMI_CHECK_ARG(x && y, "quantized_matmul: null pointer");
    hipStream_t st = (hipStream_t)stream;
    if (M > QM_TILE)
        return qmm_gemm(x, M, K, N, w, scales, biases, group_size, bits, y, workspace, workspace_bytes, st);
    QmvArgs a = {};
    a.x = (const uint16_t*)x; a.w = w; a.s = (const uint16_t*)scales; a.b = (const uint16_t*)biases;
    a.y = (uint16_t*)y; a.K = K; a.N = N; a.rows = M; a.Mper = 1; a.Xrows = M; a.S = 1;
    a.gs_shift = group_size == 32 ? 5 : group_size == 64 ? 6 : 7;
    const QmvKind kind = choose_kind(M, K, N, M, bits, group_size);
    if (kind != QmvKind::MFMA) {
        const int tm = tile_rows(kind);
        a.tile_m = tm;
        const ValuShape v = valu_shape(N, K, bits, ceil_div(M, tm), tm);
        dim3 grid((unsigned)v.groups, 1, (unsigned)ceil_div(M, tm));
        return launch_qmv(kind, a, bits, group_size, grid, valu_lds(K, bits, tm, group_size, v), st, &v);
    }
    MfmaPlan p = plan_mfma(K, N, 1, group_size);
    const size_t need = p.S > 1 ? (size_t)p.S * M * N * sizeof(float) : 0;
    if (need > 0 && (workspace == nullptr || workspace_bytes < need)) {
        set_error("quantized_matmul: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
        return EWORKSPACE;
    }
    a.partial = (float*)workspace; a.KS = p.KS; a.S = p.S; a.tile_m = QM_TILE;
    dim3 grid((unsigned)ceil_div(N, QM_ROWS_WG), (unsigned)p.S, 1);
    rc = launch_qmv(QmvKind::MFMA, a, bits, group_size, grid, p.lds, st);
    if (rc) return rc;
    if (p.S > 1) {
        const int64_t count = M * N;
        qmv_reduce<<<(unsigned)ceil_div(count, 256), 256, 0, st>>>((const float*)workspace, p.S, count, N,
                                                                     nullptr, 1, 0, (uint16_t*)y);
        KMI_CHECK_LAUNCH("qmv_reduce");
    }
    return OK;
}

size_t kmi_gather_qmm_workspace_bytes(int64_t P, int64_t M, int64_t E, int64_t K,
                                      int64_t N, int group_size, int bits) {
    if (P <= 0 || M <= 0 || E <= 0 || K <= 0 || N <= 0 || group_size <= 0 || (bits != 4 && bits != 8))
        return 0;
    const QmvKind kind = gather_kind(P, M, E, K, N, bits, group_size);
    const int tm = tile_rows(kind);
    size_t b = gather_index_bytes(P, M, E, tm);
    if (kind == QmvKind::MFMA) {
        MfmaPlan p = plan_mfma(K, N, gather_max_tiles(P, M, E, tm), group_size);
        if (p.S > 1) b += (size_t)p.S * P * M * N * sizeof(float);
    }
    return b;
}

int kmi_gather_qmm(const void* x, int64_t X, int64_t M, int64_t K, const uint32_t* w,
                   const void* scales, const void* biases, int64_t E, int64_t N,
                   const int32_t* lhs, const int32_t* rhs, int64_t P, int dtype,
                   int group_size, int bits, int sorted_indices, void* y,
                   void* workspace, size_t workspace_bytes, void* stream) {
    (void)sorted_indices;
    clear_error();
    int rc = check_common(K, N, dtype, group_size, bits);
    if (rc) return rc;
    KMI_CHECK_ARG(E > 0 && E <= 4096, "gather_qmm: %lld experts (1..4096 supported)", (long long)E);
    KMI_CHECK_ARG(M >= 1 && P >= 0 && X >= 1, "gather_qmm: bad sizes");
    KMI_CHECK_ARG(P * M < (1LL << 31), "gather_qmm: too many rows");
    if (P == 0) return OK;
    KMI_CHECK_ARG(x && w && scales && biases && y && lhs && rhs, "gather_qmm: null pointer");
    const QmvKind kind = gather_kind(P, M, E, K, N, bits, group_size);
    const int tm = tile_rows(kind);
    const int64_t max_tiles = gather_max_tiles(P, M, E, tm);
    KMI_CHECK_ARG(max_tiles < 65536, "gather_qmm: %lld tiles exceed the grid", (long long)max_tiles);
    const size_t need = kmi_gather_qmm_workspace_bytes(P, M, E, K, N, group_size, bits);
    if (workspace == nullptr || workspace_bytes < need) {
        set_error("gather_qmm: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
        return EWORKSPACE;
    }
    hipStream_t st = (hipStream_t)stream;
    char* ws = (char*)workspace;
    int32_t* sorted = (int32_t*)ws;
    int32_t* tiles = sorted + P * M;
    int32_t* offsets = tiles + 3 * max_tiles;
    float* partial = (float*)(ws + gather_index_bytes(P, M, E, tm));
    sort_rows_by_expert<<<1, SORT_THREADS, (size_t)3 * E * sizeof(int32_t), st>>>(
        rhs, P, M, (int)E, tm, sorted, tiles, (int)max_tiles, offsets, (uint16_t*)y, N);
    KMI_CHECK_LAUNCH("sort_rows_by_expert");
    const int64_t rows = P * M;
    QmvArgs a = {};
    a.x = (const uint16_t*)x; a.w = w; a.s = (const uint16_t*)scales; a.b = (const uint16_t*)biases;
    a.y = (uint16_t*)y; a.partial = partial;
    a.K = K; a.N = N; a.rows = rows; a.S = 1; a.tile_m = tm;
    a.gs_shift = group_size == 32 ? 5 : group_size == 64 ? 6 : 7;
    a.tiles = tiles; a.sorted = sorted; a.lhs = lhs; a.Mper = M; a.Xrows = X * M;
    if (kind != QmvKind::MFMA) {
        const ValuShape v = valu_shape(N, K, bits, ceil_div(P * M, tm), tm);
        dim3 grid((unsigned)v.groups, 1, (unsigned)max_tiles);
        return launch_qmv(kind, a, bits, group_size, grid, valu_lds(K, bits, tm, group_size, v), st, &v);
    }
    MfmaPlan p = plan_mfma(K, N, max_tiles, group_size);
    a.KS = p.KS; a.S = p.S;
    dim3 grid((unsigned)ceil_div(N, QM_ROWS_WG), (unsigned)p.S, (unsigned)max_tiles);
    rc = launch_qmv(QmvKind::MFMA, a, bits, group_size, grid, p.lds, st);
    if (rc) return rc;
    if (p.S > 1) {
        const int64_t count = rows * N;
        qmv_reduce<<<(unsigned)ceil_div(count, 256), 256, 0, st>>>(partial, p.S, count, N, rhs, M, E,
                                                                     (uint16_t*)y);
        KMI_CHECK_LAUNCH("qmv_reduce");
    }
    return OK;
}

}  // extern "C"
