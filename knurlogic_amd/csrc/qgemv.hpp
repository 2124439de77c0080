// Arguments and launcher of the skinny quantized matmul (qgemv.hip): up to
// 64 activation rows per weight (dense) or per routed expert (gather).
#pragma once

#include "common.hpp"

namespace kmi {

struct QgArgs {
    const uint16_t* x;          // activations, bf16 [xrows, K]
    int64_t xrows;
    const uint32_t* w;          // [E, erows, K*bits/32]
    const uint16_t* s;          // [E, erows, K/gs]
    const uint16_t* b;          // [E, erows, K/gs]
    int64_t E, N, K;
    int64_t erows;              // rows from one expert to the next (N; 2I for a stacked gate|up)
    int64_t up_off;             // GLU: row of the first up row within an expert
    uint16_t* y;                // [rows, N] bf16, when S == 1
    float* partial;             // [S, rows, N] fp32, when S > 1
    int64_t rows;               // rows of y
    int S;                      // K splits (grid y)
    int gps;                    // K chunks (256 codes) per split
    // dense: tiles == null, tile z = rows [tm*z, tm*z + tm)
    int tm;
    // gather: tile z = tiles[z] = (expert, start, count) over `sorted`; x row of
    // row id r: p = r / Mper, (lhs ? lhs[p] : p / lhs_div) * Mper + r % Mper
    const int32_t* tiles;
    const int32_t* sorted;
    // qgemv_xs with tiles == null: the expert of each of the `rows` routed
    // pairs (row id = pair), tiles of tm rows formed in the kernel
    // (pair_tiles.hpp); every expert in range.  With tiles_out, column
    // block 0 writes the sort's list of those tiles (tiles_out, sorted_out)
    const int32_t* route;
    int32_t* tiles_out;
    int32_t* sorted_out;
    const int32_t* lhs;
    int64_t lhs_div;
    int64_t Mper;
    // 0: affine (bf16 scales and biases per group); 1: OCP microscaled codes
    // (E2M1 at 4 bits, E4M3 at 8) with one uint8 E8M0 scale per 32 inputs in
    // `s` and no biases (gs 32)
    int mx;
};

// Launch shape: 64 weight rows per workgroup (16 per wave), K in chunks of
// 256 codes, S splits of gps chunks each.
struct QgPlan {
    int mc;        // 16-row activation chunks per tile (1, 2 or 4)
    int S;         // K splits
    int gps;       // chunks per split
};

QgPlan plan_qgemv(int64_t N, int64_t K, int64_t tiles, int tile_rows, int gs);
// tile rows (16, 32, 64) for rows grouped by expert, from the average routed
// rows per active expert: large enough that most experts take one tile
int qgemv_gather_tile_rows(int64_t avg_rows);
// the same plan with K unsplit (the SwiGLU epilogue needs whole sums)
QgPlan plan_qgemv_unsplit(int64_t N, int64_t K, int64_t tiles, int tile_rows, int gs);

// Rows grouped by expert on the GPU (qmv.hip): the index part of a workspace
// holds sorted row ids [rows], tiles [max_tiles][3] (expert, start, count)
// and expert offsets [E+1].
struct SortedRows {
    int32_t* sorted;
    int32_t* tiles;
    int32_t* offsets;
    int64_t max_tiles;
};

int64_t sort_max_tiles(int64_t rows, int64_t E, int tm);
size_t sort_index_bytes(int64_t rows, int64_t E, int tm);     // a multiple of 256
// rows r = p*Mper + m of the P pairs, grouped by expert rhs[p] into tiles of
// <= tm rows; rows of out-of-range experts are zeroed in y ([rows, N]) if y
int launch_sort_rows(const int32_t* rhs, int64_t P, int64_t Mper, int E, int tm, void* index_ws,
                     uint16_t* y, int64_t N, hipStream_t st, SortedRows* out);

// Expert tiles of 128 or 256 rows as a grouped GEMM (moe_gemm.hip): affine
// 4/8-bit weights, group 32/64/128, K % 64 == 0; glu: gate rows at 0, up rows
// at a.up_off, out = SwiGLU(gate, up); x row = row id / a.lhs_div
bool moe_gemm_supported(int64_t H, int64_t I, int bits, int gs, int mx);
int launch_moe_gemm(const QgArgs& a, int bits, int gs, bool glu, int tile_rows, int64_t tile_slots,
                    hipStream_t st);

// glu: gate rows at 0, up rows at a.up_off, out = SwiGLU(gate, up) in bf16
int launch_qgemv(const QgArgs& a, const QgPlan& p, int bits, int gs, bool glu, int64_t ntiles,
                 hipStream_t st);

// Dense calls of 1..16 rows with direct-to-LDS staging (qgemv_dl.hip):
// 4 or 8 bits, groups of 32 or 64, K a multiple of 256.
bool qgemv_dl_supported(int64_t M, int64_t K, int bits, int gs);
QgPlan plan_qgemv_dl(int64_t N, int64_t K);
int launch_qgemv_dl(const QgArgs& a, const QgPlan& p, int bits, int gs, hipStream_t st);

// Rows grouped by expert with the tile's x rows staged once and G column
// blocks per workgroup (qgemv_xs.hip): 0 when launched, 1 when the shape
// does not fit that kernel (K not a multiple of 256, x tile past the LDS).
// tile_rows: rows per tile of the sort (4, 16, 32 or 64).
int launch_qgemv_xs(const QgArgs& a, int bits, int gs, bool glu, int tile_rows, int64_t ntiles, hipStream_t st);

}  // namespace kmi
