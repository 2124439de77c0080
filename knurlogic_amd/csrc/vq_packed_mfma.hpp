// Arguments and launcher of the MFMA VQ expert matmul over the bit-packed
// code layout (vq_packed_mfma.hip).
#pragma once

#include "common.hpp"

namespace kmi {

constexpr int VPM_TILE = 16;   // most rows (tokens or pairs) per expert tile

struct VpmArgs {
    const uint16_t* x;          // bf16 [X, K]
    int64_t X;
    int64_t lhs_div;            // x row = row id / lhs_div
    const int32_t* tiles;       // [ntiles][3] (expert, start, count <= tile_rows) over `sorted`
    const int32_t* sorted;      // row ids grouped by expert
    const int32_t* rhs;         // tiles == null: the tiles (of tile_rows) formed in each
    int pairs;                  // workgroup from rhs[0 .. pairs) (pair_tiles.hpp), every expert
                                // in range; row id = pair
    int32_t* tiles_out;         // if set, column block 0 writes the sort's list of the formed
    int32_t* sorted_out;        // tiles, for the next launch
    int64_t E;
    const uint32_t* codes[2];   // [E, N, W] packed fields (set 1: the up rows)
    const uint16_t* sc[2];      // [E, N, K / group] fp16
    const uint16_t* cb[2];      // [kc, DIM] fp16
    int kc;
    int64_t N, K, W;            // W: words per row
    uint16_t* y;                // [row ids, N] bf16
    int tile_rows;              // largest tile the launch stages (<= 16): sizes the LDS
    int cblk;                   // 64-row column blocks per workgroup (set by launch_vpm)
};

// the shapes the kernel covers: dim 2 / 4 / 8, scale groups of 32 / 64 / 128
// inputs, K a multiple of the group and of 32 * dim, a lane's fields of one
// group inside one 16-byte load, codebooks and 16 x rows inside the LDS
bool vpm_supported(int pack_bits, int dim, int group, int64_t K, int kc, bool two_cb);
// nset 2: gate and up rows + SwiGLU; ntiles: tiles of the sort (grid rows)
int launch_vpm(const VpmArgs& a, int pack_bits, int dim, int group, int nset, int64_t ntiles, hipStream_t st);

}  // namespace kmi
