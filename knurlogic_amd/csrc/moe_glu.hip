// SwitchGLU (+ the weighted combine) as one C-ABI call: the reference's
// SwitchGLU.__call__ (src/knurlogic/engine/families/glm5/architecture/
// glm5_next/_mlx_vlm/models/switch_layers.py:172-193) with Qwen3.5's
// _SwiGLU and SparseMoeBlock combine (src/knurlogic/engine/families/qwen/
// architecture/qwen3_5.py:108-112,181-182).
//
// Up to TOK_MAX_PAIRS (token, slot) pairs run token-major (moe_tok.hip: two
// kernels, no sort); more pairs group rows by expert (gather_qmm for the
// gate|up and down projections, the SwiGLU and combine kernels between).
#include "moe_tok.hpp"
#include "../../include/knurlogic_amd.h"

namespace kmi {



constexpr int64_t TOK_MAX_PAIRS = 256;

__global__ void pair_indices(int32_t* __restrict__ tok, int32_t* __restrict__ pair, int64_t P, int k) {
    const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (p < P) {
        tok[p] = (int32_t)(p / k);
        pair[p] = (int32_t)p;
    }
}

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

struct GluPlan {
    bool tok;
    size_t act, y, gu, idx, g1, g2, total;
};

static GluPlan plan_glu(int64_t T, int64_t H, int64_t I, int k, int64_t E, int gs, int bits) {
    GluPlan p = {};
    const int64_t P = T * k;
    p.tok = P <= TOK_MAX_PAIRS;
    p.act = align256((size_t)P * I * 2);
    if (!p.tok) {
        p.y = align256((size_t)P * H * 2);
        p.gu = align256((size_t)P * 2 * I * 2);
        p.idx = align256((size_t)P * 4 * 2);
        p.g1 = align256(kmi_gather_qmm_workspace_bytes(P, 1, E, H, 2 * I, gs, bits));
        p.g2 = align256(kmi_gather_qmm_workspace_bytes(P, 1, E, I, H, gs, bits));
    }
    p.total = p.act + p.y + p.gu + p.idx + (p.g1 > p.g2 ? p.g1 : p.g2);
    return p;
}

}  // namespace kmi

using namespace kmi;

extern "C" {

size_t kmi_switch_glu_workspace_bytes(int64_t T, int64_t H, int64_t I, int k, int64_t E,
                                      int group_size, int bits) {
    if (T <= 0 || H <= 0 || I <= 0 || k <= 0 || E <= 0) return 0;
    return plan_glu(T, H, I, k, E, group_size, bits).total;
}

int kmi_switch_glu(const void* x, int64_t T, int64_t H, int64_t I, int k, const int32_t* inds,
                   const void* scores, const uint32_t* w_gu, const void* s_gu, const void* b_gu,
                   const uint32_t* w_down, const void* s_down, const void* b_down,
                   int64_t E, int dtype, int group_size, int bits, void* out, void* workspace,
                   size_t workspace_bytes, void* stream) {
    clear_error();
    KMI_CHECK_ARG(dtype == BF16, "switch_glu: only bfloat16 activations are implemented");
    KMI_CHECK_ARG(bits == 4 || bits == 8, "switch_glu: bits=%d (4 or 8)", bits);
    KMI_CHECK_ARG(group_size == 32 || group_size == 64 || group_size == 128,
                  "switch_glu: group_size=%d", group_size);
    KMI_CHECK_ARG(T >= 0 && H > 0 && I > 0 && k >= 1 && k <= 8 && E >= 1,
                  "switch_glu: bad sizes (k at most 8)");
    KMI_CHECK_ARG(H % 64 == 0 && I % 64 == 0 && H % group_size == 0 && I % group_size == 0,
                  "switch_glu: H=%lld, I=%lld must be multiples of 64 and of the group",
                  (long long)H, (long long)I);
    if (T == 0) return OK;
    KMI_CHECK_ARG(x && inds && w_gu && s_gu && b_gu && w_down && s_down && b_down && out,
                  "switch_glu: null pointer");
    const int epw = 32 / bits;
    KMI_CHECK_ARG(E * 2 * I * (H / epw) * 4 < (1LL << 31) && E * H * (I / epw) * 4 < (1LL << 31),
                  "switch_glu: expert weights past 2 GiB");
    const GluPlan p = plan_glu(T, H, I, k, E, group_size, bits);
    if (!workspace || workspace_bytes < p.total) {
        set_error("switch_glu: workspace of %zu bytes needed, %zu given", p.total, workspace_bytes);
        return EWORKSPACE;
    }
    hipStream_t st = (hipStream_t)stream;
    char* ws = (char*)workspace;
    uint16_t* act = (uint16_t*)ws;
    const int64_t P = T * k;
    const int gs_shift = group_size == 32 ? 5 : group_size == 64 ? 6 : 7;
    const int64_t wpr_h = H / epw, gpr_h = H / group_size;
    if (p.tok) {
        MoeTokArgs g = {};
        g.x = (const uint16_t*)x;
        g.w0 = w_gu; g.s0 = (const uint16_t*)s_gu; g.b0 = (const uint16_t*)b_gu;
        g.w1 = w_gu + I * wpr_h; g.s1 = (const uint16_t*)s_gu + I * gpr_h; g.b1 = (const uint16_t*)b_gu + I * gpr_h;
        g.inds = inds; g.out = act;
        g.E = E; g.N = I; g.K = H; g.T = T; g.erows = 2 * I; g.k = k; g.gs_shift = gs_shift;
        int rc = launch_moe_glu_tok(g, bits, st);
        if (rc) return rc;
        KMI_CHECK_LAUNCH("moe_glu_tok");
        MoeTokArgs d = {};
        d.x = act; d.w0 = w_down; d.s0 = (const uint16_t*)s_down; d.b0 = (const uint16_t*)b_down;
        d.inds = inds; d.scores = (const uint16_t*)scores; d.out = (uint16_t*)out;
        d.E = E; d.N = H; d.K = I; d.T = T; d.erows = H; d.k = k; d.gs_shift = gs_shift;
        rc = launch_moe_down_tok(d, bits, st);
        if (rc) return rc;
        KMI_CHECK_LAUNCH("moe_down_tok");
        return OK;
    }
    // grouped by expert: gate|up gather, SwiGLU, down gather, combine
    uint16_t* y = (uint16_t*)(ws + p.act);
    uint16_t* gu = (uint16_t*)(ws + p.act + p.y);                       // [P, 2I]
    int32_t* tok = (int32_t*)(ws + p.act + p.y + p.gu);
    int32_t* pair = tok + P;
    void* gws = ws + p.act + p.y + p.gu + p.idx;
    const size_t gbytes = p.g1 > p.g2 ? p.g1 : p.g2;
    pair_indices<<<(unsigned)ceil_div(P, 256), 256, 0, st>>>(tok, pair, P, k);
    KMI_CHECK_LAUNCH("pair_indices");
    int rc = kmi_gather_qmm(x, T, 1, H, w_gu, s_gu, b_gu, E, 2 * I, tok, inds, P, dtype, group_size,
                            bits, 0, gu, gws, gbytes, stream);
    if (rc) return rc;
    rc = kmi_swiglu(gu, gu + I, 2 * I, dtype, P, I, act, stream);
    if (rc) return rc;
    uint16_t* yd = scores ? y : (uint16_t*)out;
    rc = kmi_gather_qmm(act, P, 1, I, w_down, s_down, b_down, E, H, pair, inds, P, dtype, group_size,
                        bits, 0, yd, gws, gbytes, stream);
    if (rc) return rc;
    if (scores) return kmi_moe_combine(y, scores, dtype, T, k, H, out, stream);
    return OK;
}

}  // extern "C"
