// Decode-shape quantized matmul (M <= 16 rows per expert tile) for gfx950.
//
// y[m, n] = sum_k x[m, k] * (s[n, g] * q[n, k] + b[n, g])
//         = sum_g ( s[n, g] * P[m, n, g] + b[n, g] * X[m, g] ),
//   P[m, n, g] = sum_{k in g} x[m, k] * q[n, k],  X[m, g] = sum_{k in g} x[m, k].
//
// HBM-bound: the packed weights are streamed once, with one vector load per
// lane per group (8 bytes at 4 bits, 16 bytes at 8 bits, group 64).  The
// integer codes go to bf16 in registers (exact: 4-bit codes as "128 + q"
// through the 0x4300 exponent trick, 8-bit codes through cvt_f32_ubyte), and
// P for a 16-row x 16-column block comes from v_mfma_f32_16x16x32_bf16; the
// per-group scale and bias are applied to the fp32 accumulator, so no
// dequantized weight is ever rounded.  x for the workgroup's K slice sits in
// LDS (bf16, k pre-permuted to the unpack order), with its per-group sums.
//
// Work split: a workgroup = 4 waves = 64 weight rows x one K slice x one
// tile of <= 16 activation rows.  More than one K slice writes fp32 partials
// [S][rows][N] that qmv_reduce sums in slice order (deterministic).
//
// The same kernel serves gather_qmm: a tile is (expert, <= 16 rows routed to
// it), built on the GPU by sort_rows_by_expert, so each routed expert's
// weights are read once per call.
#include "common.hpp"
#include "../../include/knurlogic_amd.h"

namespace kmi {

constexpr int QMV_ROWS_PER_WG = 64;   // 4 waves x 16 weight rows
constexpr int QMV_TILE_M = 16;        // activation rows per tile (MFMA M)
constexpr int QMV_UNROLL = 8;         // groups whose loads are in flight per wave

struct QmvArgs {
    const uint16_t* x;        // activations (bf16), [X rows, K]
    const uint32_t* w;        // [E, N, K*bits/32]
    const uint16_t* s;        // [E, N, K/gs]
    const uint16_t* b;        // [E, N, K/gs]
    uint16_t* y;              // [rows, N] (bf16), when S == 1
    float* partial;           // [S, rows, N], when S > 1
    int64_t K, N;
    int64_t rows;             // rows of y
    int64_t KS;               // K slice length (multiple of the group)
    int S;                    // number of K slices
    // gather (all null for a dense call: tile z = rows [16z, 16z+16))
    const int32_t* tiles;     // [max_tiles][3]: expert, start, count (count 0 = unused)
    const int32_t* sorted;    // [rows] row ids grouped by expert
    const int32_t* lhs;       // [P] x batch index per pair
    int64_t Mper;             // rows per pair (x [X, Mper, K])
    int64_t Xrows;            // X * Mper: rows of x, for bounds
};

// Position of k within its 8-run in LDS so one 16-byte read gives the A
// operand in the order the B unpack produces.
template <int BITS>
__device__ __forceinline__ int lds_perm(int k) {
    if (BITS == 4) {
        // unpack order of a 4-bit word: [0,4,1,5,2,6,3,7]; element e of the
        // word lands in slot 2*(e%4) + e/4
        const int e = k & 7;
        return (k & ~7) | ((e & 3) << 1) | (e >> 2);
    }
    return k;
}

template <int BITS, int GS>
__global__ __launch_bounds__(256) void qmv_kernel(QmvArgs a) {
    constexpr int EPW = 32 / BITS;
    constexpr int WPG = GS * BITS / 32;   // words of one row per group
    constexpr int WPL = WPG / 4;          // words per lane per group
    constexpr int MF = GS / 32;           // MFMAs per group
    constexpr int WPM = BITS / 4;         // words per lane per MFMA

    extern __shared__ __align__(16) unsigned char smem[];

    // ---- which tile / slice / rows --------------------------------------
    int expert = 0;
    int64_t tstart, tcount;
    if (a.tiles) {
        const int32_t* t = a.tiles + 3 * (int64_t)blockIdx.z;
        tcount = t[2];
        if (tcount <= 0) return;
        expert = t[0];
        tstart = t[1];
    } else {
        tstart = (int64_t)blockIdx.z * QMV_TILE_M;
        tcount = a.rows - tstart;
        if (tcount > QMV_TILE_M) tcount = QMV_TILE_M;
    }
    const int64_t k0 = (int64_t)blockIdx.y * a.KS;
    int64_t k1 = k0 + a.KS;
    if (k1 > a.K) k1 = a.K;
    const int KSl = (int)(k1 - k0);
    const int ngr = KSl / GS;
    const int lds_stride = (int)a.KS + 8;                 // bf16 elements per x row
    uint16_t* xs = (uint16_t*)smem;                       // [16][lds_stride]
    float* xg = (float*)(smem + (size_t)QMV_TILE_M * lds_stride * 2);  // [ngr_max][16]

    // ---- stage x[tile rows, k0:k1] into LDS (bf16, permuted) -------------
    const int tid = threadIdx.x;
    const int runs = KSl / 8;                             // 16-byte runs per row
    for (int idx = tid; idx < tcount * runs; idx += blockDim.x) {
        const int m = idx / runs, r = idx - m * runs;
        int64_t row = tstart + m;
        int64_t xrow;
        if (a.sorted) {
            const int64_t rid = a.sorted[row];
            const int64_t p = rid / a.Mper;
            xrow = (int64_t)a.lhs[p] * a.Mper + (rid - p * a.Mper);
        } else {
            xrow = row;
        }
        u32x4 v = {0u, 0u, 0u, 0u};
        if (xrow >= 0 && xrow < a.Xrows)
            v = *(const u32x4*)(a.x + xrow * a.K + k0 + (int64_t)r * 8);
        uint16_t e[8];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            e[2 * i] = (uint16_t)(v[i] & 0xffffu);
            e[2 * i + 1] = (uint16_t)(v[i] >> 16);
        }
        uint16_t o[8];
#pragma unroll
        for (int i = 0; i < 8; i++) o[lds_perm<BITS>(i)] = e[i];
        u32x4 pv;
#pragma unroll
        for (int i = 0; i < 4; i++) pv[i] = (uint32_t)o[2 * i] | ((uint32_t)o[2 * i + 1] << 16);
        *(u32x4*)(xs + m * lds_stride + r * 8) = pv;
    }
    __syncthreads();
    // per-group sums of x (over the bf16 values), [group][m]
    for (int idx = tid; idx < ngr * QMV_TILE_M; idx += blockDim.x) {
        const int g = idx / QMV_TILE_M, m = idx - g * QMV_TILE_M;
        float sum = 0.f;
        if (m < tcount) {
            const uint16_t* p = xs + m * lds_stride + g * GS;
            for (int i = 0; i < GS; i++) sum += bf16_to_f32(p[i]);
        }
        xg[idx] = sum;
    }
    __syncthreads();

    // ---- stream the weights ------------------------------------------------
    const int lane = tid & 63, wave = tid >> 6;
    const int nl = lane & 15, j = lane >> 4;
    const int64_t n = (int64_t)blockIdx.x * QMV_ROWS_PER_WG + wave * 16 + nl;
    const bool n_ok = n < a.N;
    const int64_t nn = n_ok ? n : (a.N - 1);              // clamp loads in bounds
    const int64_t wpr = a.K / EPW, gpr = a.K / GS;
    const uint32_t* wrow = a.w + ((int64_t)expert * a.N + nn) * wpr + (k0 / EPW) + j * WPL;
    const uint16_t* srow = a.s + ((int64_t)expert * a.N + nn) * gpr + k0 / GS;
    const uint16_t* brow = a.b + ((int64_t)expert * a.N + nn) * gpr + k0 / GS;
    const bool a_ok = nl < tcount;                        // A row m = nl holds data
    const uint16_t* xa = xs + nl * lds_stride + j * (GS / 4);

    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int g0 = 0; g0 < ngr; g0 += QMV_UNROLL) {
        const int nu = (ngr - g0) < QMV_UNROLL ? (ngr - g0) : QMV_UNROLL;
        uint32_t wv[QMV_UNROLL][WPL];
        float sv[QMV_UNROLL], bv[QMV_UNROLL];
#pragma unroll
        for (int u = 0; u < QMV_UNROLL; u++) {
            if (u < nu) {
                const uint32_t* p = wrow + (int64_t)(g0 + u) * WPG;
                if constexpr (WPL == 1) {
                    wv[u][0] = p[0];
                } else if constexpr (WPL == 2) {
                    u32x2 t = *(const u32x2*)p;
                    wv[u][0] = t.x; wv[u][1] = t.y;
                } else {
#pragma unroll
                    for (int q = 0; q < WPL; q += 4) {
                        u32x4 t = *(const u32x4*)(p + q);
                        wv[u][q] = t.x; wv[u][q + 1] = t.y; wv[u][q + 2] = t.z; wv[u][q + 3] = t.w;
                    }
                }
                sv[u] = bf16_to_f32(srow[g0 + u]);
                bv[u] = bf16_to_f32(brow[g0 + u]);
            }
        }
#pragma unroll
        for (int u = 0; u < QMV_UNROLL; u++) {
            if (u < nu) {
                const int g = g0 + u;
                f32x4 P = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int t = 0; t < MF; t++) {
                    u32x4 A = {0u, 0u, 0u, 0u};
                    if (a_ok) A = *(const u32x4*)(xa + g * GS + t * 8);
                    u32x4 B;
                    if constexpr (BITS == 4) {
                        B = nibbles_to_bf16_magic(wv[u][t]);
                    } else {
                        const uint32_t w0 = wv[u][2 * t], w1 = wv[u][2 * t + 1];
                        B.x = bytes_to_bf16x2(w0, 0);
                        B.y = bytes_to_bf16x2(w0, 2);
                        B.z = bytes_to_bf16x2(w1, 0);
                        B.w = bytes_to_bf16x2(w1, 2);
                    }
                    P = mfma16x16x32(A, B, P);
                }
                // 4-bit codes entered as 128 + q: fold the offset into the bias
                const float s = sv[u];
                const float bb = (BITS == 4) ? __builtin_fmaf(-128.f, s, bv[u]) : bv[u];
                const f32x4 X = *(const f32x4*)(xg + g * QMV_TILE_M + 4 * j);
#pragma unroll
                for (int i = 0; i < 4; i++) acc[i] = __builtin_fmaf(s, P[i], __builtin_fmaf(bb, X[i], acc[i]));
            }
        }
    }

    // ---- write: D row m = 4*j + i, column n --------------------------------
    if (!n_ok) return;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int m = 4 * j + i;
        if (m >= tcount) continue;
        const int64_t row = a.sorted ? (int64_t)a.sorted[tstart + m] : (tstart + m);
        if (a.S == 1) {
            a.y[row * a.N + n] = f32_to_bf16(acc[i]);
        } else {
            a.partial[((int64_t)blockIdx.y * a.rows + row) * a.N + n] = acc[i];
        }
    }
}

// y[r, n] = bf16(sum_s partial[s, r, n]), slices summed in order.
__global__ __launch_bounds__(256) void qmv_reduce(const float* __restrict__ partial, int S,
                                                  int64_t count, uint16_t* __restrict__ y) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= count) return;
    float acc = 0.f;
    for (int s = 0; s < S; s++) acc += partial[(int64_t)s * count + i];
    y[i] = f32_to_bf16(acc);
}

// Rows whose pair has an out-of-range expert are written as zeros (and never
// read weights): the index arrays are not validated on the host.
__global__ __launch_bounds__(256) void zero_rows(uint16_t* __restrict__ y, const int32_t* __restrict__ rhs,
                                                 int64_t P, int64_t Mper, int64_t N, int64_t E) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= P * Mper * N) return;
    const int64_t p = i / (Mper * N);
    const int e = rhs[p];
    if (e < 0 || e >= E) y[i] = 0;
}

// ---- GPU grouping of rows by expert (one workgroup) --------------------------
// rows r = p*Mper + m of pairs p with expert rhs[p] are listed grouped by
// expert in `sorted`, and the expert segments are cut into tiles of <= 16
// rows: tiles[t] = (expert, start, count).  Unused tile slots get count 0.
// LDS: E counters + E tile offsets.
constexpr int SORT_THREADS = 1024;

__global__ __launch_bounds__(SORT_THREADS) void sort_rows_by_expert(
    const int32_t* __restrict__ rhs, int64_t P, int64_t Mper, int E,
    int32_t* __restrict__ sorted, int32_t* __restrict__ tiles, int max_tiles,
    int32_t* __restrict__ offsets /* [E+1] */) {
    extern __shared__ int32_t sh[];
    int32_t* cnt = sh;          // [E]
    int32_t* base = sh + E;     // [E]  row offset, then cursor
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
            trun += (cnt[e] + QMV_TILE_M - 1) / QMV_TILE_M;
        }
        offsets[E] = run;
    }
    __syncthreads();
    for (int e = tid; e < E; e += blockDim.x) {
        const int c = cnt[e];
        int t = tbase[e];
        for (int s = 0; s < c; s += QMV_TILE_M, t++) {
            if (t < max_tiles) {
                tiles[3 * t + 0] = e;
                tiles[3 * t + 1] = base[e] + s;
                tiles[3 * t + 2] = (c - s) < QMV_TILE_M ? (c - s) : QMV_TILE_M;
            }
        }
    }
    __syncthreads();
    for (int64_t p = tid; p < P; p += blockDim.x) {
        const int e = rhs[p];
        if (e < 0 || e >= E) continue;
        const int pos = atomicAdd(&base[e], (int)Mper);
        for (int64_t m = 0; m < Mper; m++) sorted[pos + m] = (int32_t)(p * Mper + m);
    }
}

// ---- host side ----------------------------------------------------------------

struct QmvPlan {
    int64_t KS;
    int S;
    size_t lds;
};

// Pick the K slice: enough workgroups to fill 256 CUs (about 1024), x tile
// within ~34 KB of LDS, slices a multiple of the group.
static QmvPlan plan_qmv(int64_t K, int64_t N, int64_t tiles, int gs) {
    const int64_t nblk = ceil_div(N, QMV_ROWS_PER_WG);
    int64_t want_s = ceil_div(1024, nblk * (tiles > 0 ? tiles : 1));
    if (want_s < 1) want_s = 1;
    int64_t KS = ceil_div(K, want_s);
    KS = ceil_div(KS, gs) * gs;
    const int64_t KS_MAX = 1024;
    if (KS > KS_MAX) KS = KS_MAX;
    if (KS < gs) KS = gs;
    if (KS > K) KS = K;
    QmvPlan p;
    p.KS = KS;
    p.S = (int)ceil_div(K, KS);
    p.lds = (size_t)QMV_TILE_M * (KS + 8) * 2 + (size_t)(KS / gs) * QMV_TILE_M * 4;
    return p;
}

template <int BITS, int GS>
static void launch_qmv_t(const QmvArgs& a, dim3 grid, size_t lds, hipStream_t st) {
    qmv_kernel<BITS, GS><<<grid, 256, lds, st>>>(a);
}

static int launch_qmv(const QmvArgs& a, int bits, int gs, dim3 grid, size_t lds, hipStream_t st) {
    if (bits == 4) {
        if (gs == 32) launch_qmv_t<4, 32>(a, grid, lds, st);
        else if (gs == 64) launch_qmv_t<4, 64>(a, grid, lds, st);
        else launch_qmv_t<4, 128>(a, grid, lds, st);
    } else {
        if (gs == 32) launch_qmv_t<8, 32>(a, grid, lds, st);
        else if (gs == 64) launch_qmv_t<8, 64>(a, grid, lds, st);
        else launch_qmv_t<8, 128>(a, grid, lds, st);
    }
    KMI_CHECK_LAUNCH("qmv");
    return OK;
}

int qmm_gemm(const void* x, int64_t M, int64_t K, int64_t N, const uint32_t* w,
             const void* scales, const void* biases, int group_size, int bits, void* y,
             hipStream_t st);  // qmm.hip

static int check_common(int64_t K, int64_t N, int dtype, int gs, int bits) {
    KMI_CHECK_ARG(dtype == BF16, "quantized matmul: only bfloat16 activations are supported (got dtype %d)", dtype);
    KMI_CHECK_ARG(bits == 4 || bits == 8, "quantized matmul: bits %d not in {4, 8}", bits);
    KMI_CHECK_ARG(gs == 32 || gs == 64 || gs == 128, "quantized matmul: group_size %d not in {32, 64, 128}", gs);
    KMI_CHECK_ARG(K > 0 && K % gs == 0 && K % 8 == 0, "quantized matmul: K=%lld must be a multiple of the group %d",
                  (long long)K, gs);
    KMI_CHECK_ARG(N > 0, "quantized matmul: N=%lld", (long long)N);
    return OK;
}

}  // namespace kmi

using namespace kmi;

extern "C" {

size_t kmi_qmm_workspace_bytes(int64_t M, int64_t K, int64_t N, int group_size, int bits) {
    (void)bits;
    if (M <= 0 || K <= 0 || N <= 0 || group_size <= 0) return 0;
    if (M > QMV_TILE_M) return 0;                      // GEMM path: no workspace
    QmvPlan p = plan_qmv(K, N, ceil_div(M, QMV_TILE_M), group_size);
    return p.S > 1 ? (size_t)p.S * M * N * sizeof(float) : 0;
}

int kmi_qmm(const void* x, int64_t M, int64_t K, int64_t N, const uint32_t* w,
            const void* scales, const void* biases, int dtype, int group_size,
            int bits, void* y, void* workspace, size_t workspace_bytes, void* stream) {
    clear_error();
    int rc = check_common(K, N, dtype, group_size, bits);
    if (rc) return rc;
    KMI_CHECK_ARG(x && w && scales && biases && y, "quantized_matmul: null pointer (affine needs biases)");
    KMI_CHECK_ARG(M >= 0, "quantized_matmul: M=%lld", (long long)M);
    if (M == 0) return OK;
    hipStream_t st = (hipStream_t)stream;
    if (M > QMV_TILE_M) return qmm_gemm(x, M, K, N, w, scales, biases, group_size, bits, y, st);
    QmvPlan p = plan_qmv(K, N, 1, group_size);
    const size_t need = p.S > 1 ? (size_t)p.S * M * N * sizeof(float) : 0;
    if (need > 0 && (workspace == nullptr || workspace_bytes < need)) {
        set_error("quantized_matmul: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
        return EWORKSPACE;
    }
    QmvArgs a = {};
    a.x = (const uint16_t*)x; a.w = w; a.s = (const uint16_t*)scales; a.b = (const uint16_t*)biases;
    a.y = (uint16_t*)y; a.partial = (float*)workspace;
    a.K = K; a.N = N; a.rows = M; a.KS = p.KS; a.S = p.S;
    a.Mper = 1; a.Xrows = M;
    dim3 grid((unsigned)ceil_div(N, QMV_ROWS_PER_WG), (unsigned)p.S, 1);
    rc = launch_qmv(a, bits, group_size, grid, p.lds, st);
    if (rc) return rc;
    if (p.S > 1) {
        const int64_t count = M * N;
        qmv_reduce<<<(unsigned)ceil_div(count, 256), 256, 0, st>>>((const float*)workspace, p.S, count, (uint16_t*)y);
        KMI_CHECK_LAUNCH("qmv_reduce");
    }
    return OK;
}

// Workspace layout for gather_qmm: sorted rows [P*M] | tiles [3*max_tiles] |
// offsets [E+1] | (pad to 256) | partials [S, P*M, N] fp32.
static int64_t gather_max_tiles(int64_t P, int64_t M, int64_t E) {
    const int64_t R = P * M;
    return (R < E ? R : E) + ceil_div(R, QMV_TILE_M);
}

static size_t gather_index_bytes(int64_t P, int64_t M, int64_t E) {
    size_t b = (size_t)(P * M) * 4 + (size_t)gather_max_tiles(P, M, E) * 12 + (size_t)(E + 1) * 4;
    return (b + 255) & ~(size_t)255;
}

size_t kmi_gather_qmm_workspace_bytes(int64_t P, int64_t M, int64_t E, int64_t K,
                                      int64_t N, int group_size, int bits) {
    (void)bits;
    if (P <= 0 || M <= 0 || E <= 0 || K <= 0 || N <= 0 || group_size <= 0) return 0;
    QmvPlan p = plan_qmv(K, N, gather_max_tiles(P, M, E), group_size);
    size_t b = gather_index_bytes(P, M, E);
    if (p.S > 1) b += (size_t)p.S * P * M * N * sizeof(float);
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
    KMI_CHECK_ARG(x && w && scales && biases && y && lhs && rhs, "gather_qmm: null pointer");
    KMI_CHECK_ARG(E > 0 && E <= 4096, "gather_qmm: %lld experts (1..4096 supported)", (long long)E);
    KMI_CHECK_ARG(M >= 1 && P >= 0 && X >= 1, "gather_qmm: bad sizes");
    KMI_CHECK_ARG(P * M < (1LL << 31), "gather_qmm: too many rows");
    if (P == 0) return OK;
    const int64_t max_tiles = gather_max_tiles(P, M, E);
    QmvPlan p = plan_qmv(K, N, max_tiles, group_size);
    const size_t need = kmi_gather_qmm_workspace_bytes(P, M, E, K, N, group_size, bits);
    if (workspace == nullptr || workspace_bytes < need) {
        set_error("gather_qmm: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
        return EWORKSPACE;
    }
    KMI_CHECK_ARG(max_tiles < 65536, "gather_qmm: %lld tiles exceed the grid", (long long)max_tiles);
    hipStream_t st = (hipStream_t)stream;
    char* ws = (char*)workspace;
    int32_t* sorted = (int32_t*)ws;
    int32_t* tiles = sorted + P * M;
    int32_t* offsets = tiles + 3 * max_tiles;
    float* partial = (float*)(ws + gather_index_bytes(P, M, E));
    sort_rows_by_expert<<<1, SORT_THREADS, (size_t)3 * E * sizeof(int32_t), st>>>(
        rhs, P, M, (int)E, sorted, tiles, (int)max_tiles, offsets);
    KMI_CHECK_LAUNCH("sort_rows_by_expert");
    const int64_t rows = P * M;
    QmvArgs a = {};
    a.x = (const uint16_t*)x; a.w = w; a.s = (const uint16_t*)scales; a.b = (const uint16_t*)biases;
    a.y = (uint16_t*)y; a.partial = partial;
    a.K = K; a.N = N; a.rows = rows; a.KS = p.KS; a.S = p.S;
    a.tiles = tiles; a.sorted = sorted; a.lhs = lhs; a.Mper = M; a.Xrows = X * M;
    dim3 grid((unsigned)ceil_div(N, QMV_ROWS_PER_WG), (unsigned)p.S, (unsigned)max_tiles);
    rc = launch_qmv(a, bits, group_size, grid, p.lds, st);
    if (rc) return rc;
    if (p.S > 1) {
        const int64_t count = rows * N;
        qmv_reduce<<<(unsigned)ceil_div(count, 256), 256, 0, st>>>(partial, p.S, count, (uint16_t*)y);
        KMI_CHECK_LAUNCH("qmv_reduce");
    }
    // rows of pairs with an out-of-range expert were never listed: zero them
    zero_rows<<<(unsigned)ceil_div(rows * N, 256), 256, 0, st>>>((uint16_t*)y, rhs, P, M, N, E);
    KMI_CHECK_LAUNCH("zero_rows");
    return OK;
}

}  // extern "C"
