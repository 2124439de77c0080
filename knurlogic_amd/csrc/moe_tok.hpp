// Arguments of the token-major SwitchGLU kernels (moe_tok.hip), shared with
// their entry point (moe_glu.hip).
#pragma once

#include "common.hpp"

namespace kmi {

struct MoeTokArgs {
    const uint16_t* x;          // [T, H] bf16 (gate/up) or act [T*k, I] (down)
    const uint32_t* w0;         // gate/up: gate rows; down: [E, N, K*bits/32]
    const uint16_t* s0;         // affine: bf16 scales; mx: uint8 E8M0 scales (same pointer)
    const uint16_t* b0;
    const uint32_t* w1;         // gate/up: up rows (same layout as the gate rows)
    const uint16_t* s1;
    const uint16_t* b1;
    const int32_t* inds;        // [T, k] (gate/up: unused when logits are given)
    const uint16_t* logits;     // gate/up only: [T, E] bf16 router logits, routed in the kernel, or null
    int32_t* inds_out;          // with logits: [T, k] experts written (for the down kernel and the caller)
    uint16_t* scores_out;       // with logits: [T, k] bf16 scores written
    const uint16_t* scores;     // [T, k] bf16, or null (down: write y, no combine)
    uint16_t* out;              // gate/up: act [T*k, N]; down: [T, N] or y [T*k, N]
    int64_t E, N, K, T;
    int64_t erows;              // rows from one expert to the next in w0/w1/s0/..: 2N for the
                                // stacked [gate | up] weight, N for down
    int k, gs_shift;
    int mx;                     // 0: affine (bf16 scales, biases); 1: OCP microscaled codes (E2M1 at
                                // bits 4, E4M3 at 8) with uint8 E8M0 scales per 32 inputs, no biases
};

int launch_moe_glu_tok(const MoeTokArgs& a, int bits, hipStream_t st);
int launch_moe_down_tok(const MoeTokArgs& a, int bits, hipStream_t st);

}  // namespace kmi
