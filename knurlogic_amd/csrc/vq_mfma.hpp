// Arguments and launcher of the MFMA VQ expert matmul (vq_mfma.hip).
#pragma once

#include "common.hpp"

namespace kmi {

constexpr int VQM_TILE_ROWS = 16;   // rows (tokens or pairs) per expert tile
constexpr int VQM_MAX_CBLK = 4;     // column blocks of 64 rows per workgroup (2-byte codes)

struct VqmArgs {
    const uint16_t* x;          // bf16 [X, K]
    int64_t X;
    uint32_t lhs_magic;         // x row = umulhi(row id, lhs_magic); 0: x row = row id
    const int32_t* tiles;       // [ntiles][3] (expert, start, count <= 16) over `sorted`; null:
                                // pair mode, tile z = row id z alone with expert rhs[z]
    const int32_t* sorted;      // row ids grouped by expert
    const int32_t* rhs;         // pair mode: expert per row id
    int pairs;                  // tiles == null and pairs > 0: the tiles (of tile_rows) formed in
                                // each workgroup from rhs[0 .. pairs) (pair_tiles.hpp), every
                                // expert in range; row id = pair
    int32_t* tiles_out;         // with pairs: if set, column block 0 writes the sort's list of
    int32_t* sorted_out;        // the formed tiles, for the next launch
    int64_t E;
    const void* codes0;         // [E, erows, K/8] (u8 or u16)
    const uint16_t* sc0;        // [E, erows] fp16, one scale per output row
    const uint16_t* cb0;        // [kc, 8] fp16
    const void* codes1;         // second row set (GLU: the up rows), or null
    const uint16_t* sc1;
    const uint16_t* cb1;
    int kc;
    uint16_t* y;                // [row ids, N] bf16
    int64_t N, K, erows;
    int tile_rows;              // largest tile count the launch stages (<= 16): sizes the LDS
    int cblk;                   // column blocks per workgroup (set by launch_vq_mfma)
    // pair mode with router logits: each workgroup routes its pair's token
    // (route.hpp, the router kernel's arithmetic) in place of reading rhs,
    // and column block 0 writes the pair's expert and score
    const uint16_t* logits;     // [X, E] bf16, or null
    int32_t* inds_out;          // [X * k] experts (read by the down kernel)
    uint16_t* scores_out;       // [X * k] bf16 scores
    int k;                      // slots per token (pair = token * k + slot)
};

size_t vq_mfma_lds(int64_t K, int kc, bool two_cb, int tile_rows, int nset, int ks);
// K, index width, codebook size that the MFMA path covers (per-channel scales)
bool vq_mfma_supported(int64_t K, int code_bytes, int kc, bool two_cb);
// ntiles: grid rows (tiles of the sort, or the row ids in pair mode)
int launch_vq_mfma(const VqmArgs& a, int code_bytes, int nset, int64_t ntiles, hipStream_t st);

// Down projection of a few tokens, token-major: every (token, slot) pair's
// expert row block in one workgroup per (16 rows, token), and with scores
// the weighted combine of the token's k slots in the epilogue.
struct VqdArgs {
    const uint16_t* x;          // act [T*k, K] bf16 (pair-major)
    const int32_t* inds;        // [T*k] expert per pair
    const void* codes;          // [E, N, K/8] (u8 or u16)
    const uint16_t* sc;         // [E, N] fp16
    const uint16_t* cb;         // [kc, 8] fp16
    const uint16_t* scores;     // [T*k] bf16, or null: y [T*k, N] is written
    uint16_t* out;              // [T, N] with scores, else [T*k, N]
    int64_t E, N, K, T;
    int k, kc;
};

// the shapes vq_down_tok covers (K a multiple of 128, K / 8 codes per row
// split over 4 lanes in whole 32-bit words)
bool vq_down_tok_supported(int64_t K, int code_bytes, int kc, int k);
size_t vq_down_tok_lds(int64_t K, int kc, int k);
int launch_vq_down_tok(const VqdArgs& a, int code_bytes, hipStream_t st);

}  // namespace kmi
