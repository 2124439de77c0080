// Decode-shape quantized matmul for gfx950: the dense entry (kmi_qmm) for
// M <= 64 activation rows and gather_qmm (kmi_gather_qmm) for any number of
// routed rows.
//
//   qmv_valu  (qmv_valu.hip, one row per tile): HBM-bound streaming GEMV.
//   qgemv     (qgemv.hip, up to 64 rows per tile): MFMA on codes decoded in
//             registers, per-group scale/bias on fp32 partials.
//
// gather_qmm: a tile is (expert, <= tile rows routed to it), built on the GPU
// by sort_rows_by_expert, so each routed expert's weights are read once per
// tile.
#include "qmv_common.hpp"
#include "qgemv.hpp"
#include "../../include/knurlogic_amd.h"


namespace kmi {
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
// Rows of pairs with an out-of-range expert are zeroed in y (when y is given)
// and never listed (the index arrays are not validated on the host).  Within
// an expert the order of rows follows atomic arrival; each row's result does
// not depend on its position.
constexpr int SORT_THREADS = 1024;
constexpr int SORT_MAX_E = 4096;

// Exclusive prefix sum over the workgroup's threads (thread order), and the
// total in *total.  `wsum` holds SORT_THREADS / 64 ints of LDS.
__device__ __forceinline__ int block_exclusive_scan(int v, int* wsum, int* total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    int inc = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(inc, o, 64);
        if (lane >= o) inc += t;
    }
    if (lane == 63) wsum[w] = inc;
    __syncthreads();
    if (w == 0) {
        constexpr int NW = SORT_THREADS / 64;
        int x = lane < NW ? wsum[lane] : 0;
#pragma unroll
        for (int o = 1; o < NW; o <<= 1) {
            const int t = __shfl_up(x, o, 64);
            if (lane >= o) x += t;
        }
        if (lane < NW) wsum[lane] = x;            // inclusive wave totals
    }
    __syncthreads();
    const int before = w > 0 ? wsum[w - 1] : 0;
    *total = wsum[SORT_THREADS / 64 - 1];
    __syncthreads();                              // wsum is reused by the next scan
    return before + inc - v;
}

__global__ __launch_bounds__(SORT_THREADS) void sort_rows_by_expert(
    const int32_t* __restrict__ rhs, int64_t P, int64_t Mper, int E, int TM,
    int32_t* __restrict__ sorted, int32_t* __restrict__ tiles, int max_tiles,
    int32_t* __restrict__ offsets /* [E+1] */, uint16_t* __restrict__ y, int64_t N) {
    constexpr int EPT = SORT_MAX_E / SORT_THREADS;     // experts per thread
    __shared__ int cnt[SORT_MAX_E];
    __shared__ int cursor[SORT_MAX_E];
    __shared__ int wsum[SORT_THREADS / 64];
    const int tid = threadIdx.x;
    for (int e = tid; e < E; e += SORT_THREADS) cnt[e] = 0;
    for (int t = tid; t < 3 * max_tiles; t += SORT_THREADS) tiles[t] = 0;
    __syncthreads();
    for (int64_t p = tid; p < P; p += SORT_THREADS) {
        const int e = rhs[p];
        if (e >= 0 && e < E) atomicAdd(&cnt[e], (int)Mper);
    }
    __syncthreads();
    // thread tid owns experts [EPT*tid, EPT*tid + EPT): row and tile offsets by scans
    int c[EPT], rows = 0, ntile = 0;
#pragma unroll
    for (int i = 0; i < EPT; i++) {
        const int e = EPT * tid + i;
        c[i] = e < E ? cnt[e] : 0;
        rows += c[i];
        ntile += (c[i] + TM - 1) / TM;
    }
    int total_rows, total_tiles;
    int rbase = block_exclusive_scan(rows, wsum, &total_rows);
    int tbase = block_exclusive_scan(ntile, wsum, &total_tiles);
#pragma unroll
    for (int i = 0; i < EPT; i++) {
        const int e = EPT * tid + i;
        if (e < E) {
            offsets[e] = rbase;
            cursor[e] = rbase;
            for (int s = 0; s < c[i]; s += TM, tbase++)
                if (tbase < max_tiles) {
                    tiles[3 * tbase + 0] = e;
                    tiles[3 * tbase + 1] = rbase + s;
                    tiles[3 * tbase + 2] = (c[i] - s) < TM ? (c[i] - s) : TM;
                }
            rbase += c[i];
        }
    }
    if (tid == 0) offsets[E] = total_rows;
    __syncthreads();
    for (int64_t p = tid; p < P; p += SORT_THREADS) {
        const int e = rhs[p];
        if (e < 0 || e >= E) {
            if (y)
                for (int64_t i = 0; i < Mper * N; i++) y[p * Mper * N + i] = 0;
            continue;
        }
        const int pos = atomicAdd(&cursor[e], (int)Mper);
        for (int64_t m = 0; m < Mper; m++) sorted[pos + m] = (int32_t)(p * Mper + m);
    }
}

int64_t sort_max_tiles(int64_t rows, int64_t E, int tm) {
    return (rows < E ? rows : E) + ceil_div(rows, tm);
}

size_t sort_index_bytes(int64_t rows, int64_t E, int tm) {
    size_t b = (size_t)rows * 4 + (size_t)sort_max_tiles(rows, E, tm) * 12 + (size_t)(E + 1) * 4;
    return (b + 255) & ~(size_t)255;
}

int launch_sort_rows(const int32_t* rhs, int64_t P, int64_t Mper, int E, int tm, void* index_ws,
                     uint16_t* y, int64_t N, hipStream_t st, SortedRows* out) {
    const int64_t rows = P * Mper;
    const int64_t max_tiles = sort_max_tiles(rows, E, tm);
    if (E > SORT_MAX_E || max_tiles >= 65536 || rows >= (1LL << 31)) {
        set_error("sort: %lld rows over %d experts exceed the sort's limits", (long long)rows, E);
        return EINVAL_ARG;
    }
    out->sorted = (int32_t*)index_ws;
    out->tiles = out->sorted + rows;
    out->offsets = out->tiles + 3 * max_tiles;
    out->max_tiles = max_tiles;
    sort_rows_by_expert<<<1, SORT_THREADS, 0, st>>>(rhs, P, Mper, E, tm, out->sorted, out->tiles,
                                                   (int)max_tiles, out->offsets, y, N);
    KMI_CHECK_LAUNCH("sort_rows_by_expert");
    return OK;
}

// ---- host side ----------------------------------------------------------------

#ifndef KMI_SKINNY_MIN_ROWS
#define KMI_SKINNY_MIN_ROWS 2
#endif

enum class QmvKind { VALU1, SKINNY };

static int tile_rows(QmvKind k) { return k == QmvKind::VALU1 ? 1 : 16; }

// LDS of the VALU kernel: the tile's x row as fp16 (2 bytes per k) and a
// 16-byte {scale, correction, sum} record per 16-byte weight chunk.
static size_t valu_lds(int64_t K, int bits) {
    return (size_t)K * 2 + (size_t)(K / (128 / bits)) * 16;
}

// Launch shape of the VALU kernel.  S: 16-byte chunk slots per lane, all of
// K up to 8 slots (one load batch).  RPW: weight rows per wave, as many as
// keep S * RPW <= 8 loads in registers while the grid still has >= 4096
// waves (4 per SIMD) to spread over the chip; 2 rows from 2048 waves for a
// dense call (one tile), whose every workgroup stages the same x (4-bit
// [4096, 4096]: 4.55 us at 1 row per wave, 4.36 at 2; [14336, 4096] stays
// at 2: 8.0 us, 8.6 at 4).  WV: waves per workgroup, which
// amortizes the x staging over WV * RPW rows.
static ValuShape valu_shape(int64_t N, int64_t K, int bits, int64_t tiles, bool mx = false) {
    const int64_t C = K / (128 / bits);
    const int64_t slots = ceil_div(C, 64);
    ValuShape v;
    v.S = slots <= 1 ? 1 : slots <= 2 ? 2 : slots <= 4 ? 4 : 8;
    const int64_t T = tiles > 0 ? tiles : 1;
    v.RPW = 1;
    if (v.S <= 4 && N * T / 2 >= (tiles <= 1 ? 2048 : 4096)) v.RPW = 2;
    if (v.S <= 2 && N * T / 4 >= 4096) v.RPW = 4;
    // 4 waves while each thread stages at most two x pieces (K <= 4096):
    // smaller workgroups start sooner; longer rows need 8 waves to keep the
    // staging ahead of the weight stream short
    v.WV = K <= 4096 ? 4 : 8;
    // affine rows of more than 8 slots (two batches of loads) and over 1024
    // x pieces: 16 waves, which stage at most two pieces per thread (8-bit
    // [4096, 14336] 13.75 -> 12.9 us; measured slower at 16: rows of one
    // batch, 4-bit 9.55 -> 10.0, and mxfp8 14.35 -> 14.6)
    if (!mx && v.RPW == 1 && v.S == 8 && slots > 8 && K / 8 > 2 * 512) v.WV = 16;
    // no more waves per workgroup than the rows need
    while (v.WV > 4 && (int64_t)(v.WV / 2) * v.RPW >= N) v.WV /= 2;
    v.groups = ceil_div(N, (int64_t)v.WV * v.RPW);
    return v;
}

// Kernel choice by rows per tile: the VALU GEMV for one row per tile while
// its LDS fits 64 KB, else qgemv (MFMA).
static QmvKind choose_kind(int64_t rows_per_tile, int64_t K, int bits) {
    if (rows_per_tile < KMI_SKINNY_MIN_ROWS && rows_per_tile <= 1 && valu_lds(K, bits) <= 64 * 1024)
        return QmvKind::VALU1;
    return QmvKind::SKINNY;
}

static int skinny_tile_rows(int64_t rows_per_tile) {
    return rows_per_tile <= 16 ? 16 : rows_per_tile <= 32 ? 32 : 64;
}

static int launch_valu(const QmvArgs& a, int bits, dim3 grid, size_t lds, hipStream_t st,
                       const ValuShape& v) {
    if (!launch_qmv_valu(bits, v, a, grid, lds, st)) {
        set_error("qmv: no kernel for shape S=%d RPW=%d WV=%d", v.S, v.RPW, v.WV);
        return EINVAL_ARG;
    }
    KMI_CHECK_LAUNCH("qmv_valu");
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

constexpr int64_t SKINNY_MAX_M = 64;     // dense rows handled by qgemv (more: the GEMM)

static size_t skinny_partial_bytes(const QgPlan& p, int64_t rows, int64_t N) {
    return p.S > 1 ? (size_t)p.S * rows * N * sizeof(float) : 0;
}

// qgemv launch plus the in-order reduction of K-split partials
static int run_skinny(QgArgs& a, const QgPlan& p, int bits, int gs, int64_t ntiles, void* partial,
                      const int32_t* rhs, int64_t Mper, bool dl, hipStream_t st) {
    a.S = p.S; a.gps = p.gps; a.partial = (float*)partial;
    int rc;
    if (dl) rc = launch_qgemv_dl(a, p, bits, gs, st);
    else if (a.tiles && p.S == 1 && launch_qgemv_xs(a, bits, gs, false, 16 * p.mc, ntiles, st) == 0) rc = OK;
    else rc = launch_qgemv(a, p, bits, gs, false, ntiles, st);
    if (rc) return rc;
    KMI_CHECK_LAUNCH(dl ? "qgemv_dl" : "qgemv");
    if (p.S > 1) {
        const int64_t count = a.rows * a.N;
        qmv_reduce<<<(unsigned)ceil_div(count, 256), 256, 0, st>>>(a.partial, p.S, count, a.N, rhs, Mper,
                                                                     a.E, a.y);
        KMI_CHECK_LAUNCH("qmv_reduce");
    }
    return OK;
}

// Dense 2..16-row calls take the direct-to-LDS kernel where it has a variant
static bool use_dl(int64_t M, int64_t K, int bits, int gs) {
    return qgemv_dl_supported(M, K, bits, gs);
}

static QgPlan dense_skinny_plan(int64_t M, int64_t K, int64_t N, int bits, int gs) {
    if (use_dl(M, K, bits, gs)) return plan_qgemv_dl(N, K);
    const int tm = skinny_tile_rows(M);
    return plan_qgemv(N, K, ceil_div(M, tm), tm, gs);
}

// rows per tile for gather: average routed rows per active expert
static int64_t gather_rows_per_tile(int64_t P, int64_t M, int64_t E) {
    const int64_t R = P * M;
    const int64_t active = R < E ? R : E;
    return ceil_div(R, active);
}

}  // namespace kmi

using namespace kmi;

extern "C" {

size_t kmi_qmm_workspace_bytes(int64_t M, int64_t K, int64_t N, int group_size, int bits) {
    if (M <= 0 || K <= 0 || N <= 0 || group_size <= 0 || (bits != 4 && bits != 8)) return 0;
    if (M > SKINNY_MAX_M) return qmm_gemm_workspace(M, K, N);       // GEMM path (split-K partials)
    if (choose_kind(M, K, bits) != QmvKind::SKINNY) return 0;   // VALU path
    return skinny_partial_bytes(dense_skinny_plan(M, K, N, bits, group_size), M, N);
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
    KMI_CHECK_ARG(M * K * 2 < (1LL << 31), "quantized_matmul: x of %lld x %lld exceeds 2 GB",
                  (long long)M, (long long)K);
    hipStream_t st = (hipStream_t)stream;
    if (M > SKINNY_MAX_M)
        return qmm_gemm(x, M, K, N, w, scales, biases, group_size, bits, y, workspace, workspace_bytes, st);
    const QmvKind kind = choose_kind(M, K, bits);
    if (kind != QmvKind::SKINNY) {
        QmvArgs a = {};
        a.x = (const uint16_t*)x; a.w = w; a.s = (const uint16_t*)scales; a.b = (const uint16_t*)biases;
        a.y = (uint16_t*)y; a.K = K; a.N = N; a.rows = M; a.Mper = 1; a.Xrows = M; a.S = 1;
        a.gs_shift = group_size == 32 ? 5 : group_size == 64 ? 6 : 7;
        const int tm = tile_rows(kind);
        a.tile_m = tm;
        const ValuShape v = valu_shape(N, K, bits, ceil_div(M, tm));
        dim3 grid((unsigned)v.groups, 1, (unsigned)ceil_div(M, tm));
        return launch_valu(a, bits, grid, valu_lds(K, bits), st, v);
    }
    const int tm = skinny_tile_rows(M);
    const int64_t ntiles = ceil_div(M, tm);
    const bool dl = use_dl(M, K, bits, group_size);
    const QgPlan p = dense_skinny_plan(M, K, N, bits, group_size);
    const size_t need = skinny_partial_bytes(p, M, N);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need)) {
        set_error("quantized_matmul: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
        return EWORKSPACE;
    }
    QgArgs a = {};
    a.x = (const uint16_t*)x; a.xrows = M; a.w = w; a.s = (const uint16_t*)scales;
    a.b = (const uint16_t*)biases; a.E = 1; a.N = N; a.K = K; a.erows = N; a.y = (uint16_t*)y;
    a.rows = M; a.tm = tm; a.lhs_div = 1; a.Mper = 1;
    return run_skinny(a, p, bits, group_size, ntiles, workspace, nullptr, 1, dl, st);
}

// Microscaled dense decode: the decode kernels of kmi_qmm with the E2M1 /
// E4M3 decode and byte scales; more than 64 rows, or K not a multiple of 64,
// take the batched kernel (nd = 0).
static bool mx_decode_shape(int64_t M, int64_t K) { return M <= SKINNY_MAX_M && K % 64 == 0; }

size_t kmi_qmm_mx_workspace_bytes(int64_t M, int64_t K, int64_t N, int mode) {
    if (M <= 0 || K <= 0 || N <= 0 || (mode != 1 && mode != 2)) return 0;
    const int bits = mode == 1 ? 4 : 8;
    if (!mx_decode_shape(M, K)) return kmi_qmm_batched_workspace_bytes(0, nullptr, M, K, N);
    if (choose_kind(M, K, bits) != QmvKind::SKINNY) return 0;
    return skinny_partial_bytes(dense_skinny_plan(M, K, N, bits, 32), M, N);
}

int kmi_qmm_mx(const void* x, int64_t M, int64_t K, int64_t N, const uint32_t* w, const uint8_t* scales,
               int dtype, int mode, void* y, void* workspace, size_t workspace_bytes, void* stream) {
    clear_error();
    KMI_CHECK_ARG(mode == 1 || mode == 2, "quantized_matmul: mode %d is not microscaled (1 mxfp4, 2 mxfp8)", mode);
    const int bits = mode == 1 ? 4 : 8;
    KMI_CHECK_ARG(M >= 0 && K > 0 && K % 32 == 0 && N > 0,
                  "quantized_matmul: M=%lld K=%lld N=%lld (K a multiple of 32)", (long long)M, (long long)K,
                  (long long)N);
    if (!mx_decode_shape(M, K)) {
        const int64_t xs[1] = {K}, ws[1] = {K * bits / 32}, ss[1] = {K / 32};
        return kmi_qmm_batched(x, xs, w, ws, scales, nullptr, ss, 0, nullptr, M, K, N, 1, dtype, 32, bits, mode,
                               nullptr, nullptr, 0, 0, 1.0f, y, N, workspace, workspace_bytes, stream);
    }
    int rc = check_common(K, N, dtype, 32, bits);
    if (rc) return rc;
    KMI_CHECK_ARG(w && scales, "quantized_matmul: null pointer");
    if (M == 0) return OK;
    KMI_CHECK_ARG(x && y, "quantized_matmul: null pointer");
    hipStream_t st = (hipStream_t)stream;
    const QmvKind kind = choose_kind(M, K, bits);
    if (kind != QmvKind::SKINNY) {
        QmvArgs a = {};
        a.x = (const uint16_t*)x; a.w = w; a.s = (const uint16_t*)scales; a.b = nullptr;
        a.y = (uint16_t*)y; a.K = K; a.N = N; a.rows = M; a.Mper = 1; a.Xrows = M; a.S = 1;
        a.gs_shift = 5; a.mx = 1;
        const int tm = tile_rows(kind);
        a.tile_m = tm;
        const ValuShape v = valu_shape(N, K, bits, ceil_div(M, tm), true);
        dim3 grid((unsigned)v.groups, 1, (unsigned)ceil_div(M, tm));
        return launch_valu(a, bits, grid, valu_lds(K, bits), st, v);
    }
    const int tm = skinny_tile_rows(M);
    const int64_t ntiles = ceil_div(M, tm);
    const bool dl = use_dl(M, K, bits, 32);
    const QgPlan p = dense_skinny_plan(M, K, N, bits, 32);
    const size_t need = skinny_partial_bytes(p, M, N);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need)) {
        set_error("quantized_matmul: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
        return EWORKSPACE;
    }
    QgArgs a = {};
    a.x = (const uint16_t*)x; a.xrows = M; a.w = w; a.s = (const uint16_t*)scales; a.b = nullptr;
    a.E = 1; a.N = N; a.K = K; a.erows = N; a.y = (uint16_t*)y;
    a.rows = M; a.tm = tm; a.lhs_div = 1; a.Mper = 1; a.mx = 1;
    return run_skinny(a, p, bits, 32, ntiles, workspace, nullptr, 1, dl, st);
}

size_t kmi_gather_qmm_workspace_bytes(int64_t P, int64_t M, int64_t E, int64_t K,
                                      int64_t N, int group_size, int bits) {
    if (P <= 0 || M <= 0 || E <= 0 || K <= 0 || N <= 0 || group_size <= 0 || (bits != 4 && bits != 8))
        return 0;
    const int64_t rpt = gather_rows_per_tile(P, M, E);
    const QmvKind kind = choose_kind(rpt, K, bits);
    const int tm = kind == QmvKind::SKINNY ? qgemv_gather_tile_rows(rpt) : tile_rows(kind);
    size_t b = sort_index_bytes(P * M, E, tm);
    if (kind == QmvKind::SKINNY)
        b += skinny_partial_bytes(plan_qgemv(N, K, sort_max_tiles(P * M, E, tm), tm, group_size), P * M, N);
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
    KMI_CHECK_ARG(E > 0 && E <= SORT_MAX_E, "gather_qmm: %lld experts (1..%d supported)", (long long)E,
                  SORT_MAX_E);
    KMI_CHECK_ARG(M >= 1 && P >= 0 && X >= 1, "gather_qmm: bad sizes");
    KMI_CHECK_ARG(P * M < (1LL << 31), "gather_qmm: too many rows");
    KMI_CHECK_ARG(X * M * K * 2 < (1LL << 31), "gather_qmm: x exceeds 2 GB");
    if (P == 0) return OK;
    KMI_CHECK_ARG(x && w && scales && biases && y && lhs && rhs, "gather_qmm: null pointer");
    const int64_t rpt = gather_rows_per_tile(P, M, E);
    const QmvKind kind = choose_kind(rpt, K, bits);
    const int tm = kind == QmvKind::SKINNY ? qgemv_gather_tile_rows(rpt) : tile_rows(kind);
    const size_t need = kmi_gather_qmm_workspace_bytes(P, M, E, K, N, group_size, bits);
    if (workspace == nullptr || workspace_bytes < need) {
        set_error("gather_qmm: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
        return EWORKSPACE;
    }
    hipStream_t st = (hipStream_t)stream;
    SortedRows sr;
    rc = launch_sort_rows(rhs, P, M, (int)E, tm, workspace, (uint16_t*)y, N, st, &sr);
    if (rc) return rc;
    void* partial = (char*)workspace + sort_index_bytes(P * M, E, tm);
    const int64_t rows = P * M;
    if (kind != QmvKind::SKINNY) {
        QmvArgs a = {};
        a.x = (const uint16_t*)x; a.w = w; a.s = (const uint16_t*)scales; a.b = (const uint16_t*)biases;
        a.y = (uint16_t*)y; a.K = K; a.N = N; a.rows = rows; a.S = 1; a.tile_m = tm;
        a.gs_shift = group_size == 32 ? 5 : group_size == 64 ? 6 : 7;
        a.tiles = sr.tiles; a.sorted = sr.sorted; a.lhs = lhs; a.Mper = M; a.Xrows = X * M;
        const ValuShape v = valu_shape(N, K, bits, ceil_div(rows, tm));
        dim3 grid((unsigned)v.groups, 1, (unsigned)sr.max_tiles);
        return launch_valu(a, bits, grid, valu_lds(K, bits), st, v);
    }
    const QgPlan p = plan_qgemv(N, K, sr.max_tiles, tm, group_size);
    QgArgs a = {};
    a.x = (const uint16_t*)x; a.xrows = X * M; a.w = w; a.s = (const uint16_t*)scales;
    a.b = (const uint16_t*)biases; a.E = E; a.N = N; a.K = K; a.erows = N; a.y = (uint16_t*)y;
    a.rows = rows; a.tm = tm; a.tiles = sr.tiles; a.sorted = sr.sorted; a.lhs = lhs; a.lhs_div = 1;
    a.Mper = M;
    return run_skinny(a, p, bits, group_size, sr.max_tiles, partial, rhs, M, false, st);
}

}  // extern "C"
