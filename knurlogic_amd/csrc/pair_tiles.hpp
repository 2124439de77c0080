// Expert tiles of a few routed (token, slot) pairs, formed inside each
// workgroup of an expert-grouped kernel from the pairs' experts, so no sort
// launch runs before it.  The tiles are those of sort_rows_by_expert
// (qmv.hip): experts in ascending order, each expert's rows cut into tiles
// of at most TM; within an expert the rows are in pair order, so every
// workgroup of a launch (and the next launch over the same pairs) agrees
// on tile z.  The grid covers sort_max_tiles(P, E, TM) tile slots, as with
// the sort; slots past the last tile find no tile.  A tile's start is its
// first row's place in the sort's `sorted` list, so a kernel can write the
// sort's list (tiles, sorted) for a later launch over the same pairs.
//
// Bookkeeping in LDS: one bit per pair in its expert's mask, an expert's
// row count a popcount of its mask, tile bases an exclusive scan over the
// experts, and a pair's rank within its expert the popcount of the mask
// bits below it.  One scan gives both the tile bases and the row offsets
// (tiles and rows packed in one int: each sum stays below 2^16).
#pragma once

#include "common.hpp"

namespace kmi {

constexpr int PT_THREADS = 256;                  // the workgroup that forms the tile
constexpr int PT_MAX_PAIRS = PT_THREADS;         // one pair per thread
constexpr int PT_MAX_E = PT_THREADS;             // one expert per thread in the scan
constexpr int PT_MASK_WORDS = 1024;              // E * ceil(P / 32) mask words
constexpr int PT_MAX_TM = 16;

// Working space of pair_tile_from: a kernel may place it over LDS that it
// fills only after the tile is known (its x rows, say).
struct PairTileLds {
    uint32_t mask[PT_MASK_WORDS];    // mask[e * W + w], bit b: pair 32 w + b routed to e
    int32_t wsum[PT_THREADS / 64];
    int32_t sel[4];                  // the tile: expert, first rank, rows, start
};

// Host side: whether P pairs over E experts fit the in-kernel tiles.
inline bool pair_tiles_fit(int64_t P, int64_t E, int tm) {
    return P >= 1 && P <= PT_MAX_PAIRS && E >= 1 && E <= PT_MAX_E && E * ((P + 31) / 32) <= PT_MASK_WORDS &&
           tm >= 1 && tm <= PT_MAX_TM;
}

// This thread's pair's expert as loaded (pair_tile_from range-checks it).
// Issued first, so the loads a kernel issues before pair_tile_from are in
// flight with it (a check here would wait for the load right away).
__device__ __forceinline__ int pair_tile_load(const int32_t* __restrict__ rhs, int P) {
    const int t = threadIdx.x;
    return t < P ? rhs[t] : -1;
}

// Inclusive sum over the 64 lanes of a wave by DPP row shifts and row
// broadcasts (no LDS round trip).
__device__ __forceinline__ int pair_wave_scan(int x) {
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);   // row_shr:1
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);   // row_shr:2
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);   // row_shr:4
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);   // row_shr:8
    x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);   // row_bcast:15
    x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);   // row_bcast:31
    return x;
}

// Tile z from every thread's pair_tile_load result; all PT_THREADS threads
// call it.  Returns the tile's row count (0: slot z holds no tile), its
// expert in `expert` and the place of its first row in the sort's list in
// `start`, all workgroup-uniform, and writes its row ids to rows[0 ..
// count) (LDS, at least TM entries).  Orders LDS only (lds_barrier), so
// global loads in flight stay in flight.
__device__ __forceinline__ int pair_tile_from(int e, int P, int E, int TM, int z, PairTileLds& sm,
                                              int32_t* rows, int& expert, int& start) {
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    if (e < 0 || e >= E) e = -1;
    const int W = (P + 31) >> 5;
    for (int i = t; i < E * W; i += PT_THREADS) sm.mask[i] = 0u;
    if (t == 0) sm.sel[2] = 0;
    lds_barrier();
    if (e >= 0) atomicOr(&sm.mask[e * W + (t >> 5)], 1u << (t & 31));
    lds_barrier();
    int cnt = 0;
    if (t < E)
        for (int i = 0; i < W; i++) cnt += __popc(sm.mask[t * W + i]);
    const int nt = (cnt + TM - 1) / TM;
    // exclusive scan over the threads (expert order) of rows << 16 | tiles
    const int v0 = cnt << 16 | nt;
    const int inc = pair_wave_scan(v0);
    if (lane == 63) sm.wsum[w] = inc;
    lds_barrier();
    int packed = inc - v0;
    for (int i = 0; i < w; i++) packed += sm.wsum[i];
    const int base = packed & 0xffff;
    if (nt > 0 && z >= base && z < base + nt) {
        const int first = (z - base) * TM;
        sm.sel[0] = t;
        sm.sel[1] = first;
        sm.sel[2] = cnt - first < TM ? cnt - first : TM;
        sm.sel[3] = (packed >> 16) + first;
    }
    lds_barrier();
    const int ex = __builtin_amdgcn_readfirstlane(sm.sel[0]);
    const int first = __builtin_amdgcn_readfirstlane(sm.sel[1]);
    const int count = __builtin_amdgcn_readfirstlane(sm.sel[2]);
    start = __builtin_amdgcn_readfirstlane(sm.sel[3]);
    if (count > 0 && e == ex) {
        int rank = __popc(sm.mask[ex * W + (t >> 5)] & ((1u << (t & 31)) - 1u));
        for (int i = 0; i < (t >> 5); i++) rank += __popc(sm.mask[ex * W + i]);
        if (rank >= first && rank < first + count) rows[rank - first] = t;
    }
    lds_barrier();
    expert = ex;
    return count;
}

// The sort's list entry of tile z (a formed tile, or none: count 0), for a
// later launch over the same pairs; written by one workgroup per tile.
__device__ __forceinline__ void pair_tile_store(int32_t* __restrict__ tiles, int32_t* __restrict__ sorted, int z,
                                                int expert, int start, int count, const int32_t* rows) {
    const int t = threadIdx.x;
    if (t < 3) tiles[3 * z + t] = t == 0 ? expert : t == 1 ? start : count;
    if (t < count) sorted[start + t] = rows[t];
}

}  // namespace kmi
