// SwitchGLU (+ the weighted combine) as one C-ABI call: the reference's
// SwitchGLU.__call__ (src/knurlogic/engine/families/glm5/architecture/
// glm5_next/_mlx_vlm/models/switch_layers.py:172-193) with Qwen3.5's
// _SwiGLU and SparseMoeBlock combine (src/knurlogic/engine/families/qwen/
// architecture/qwen3_5.py:108-112,181-182).
//
// Up to TOK_MAX_PAIRS (token, slot) pairs run token-major (moe_tok.hip: two
// kernels, no sort).  More pairs are grouped by expert on the GPU once, and
// both projections run over the same tiles (qgemv.hip), so each routed
// expert's weights are read once per call: gate|up with the SwiGLU
// epilogue, then down, then the weighted combine.

#include "moe_tok.hpp"
#include "pair_tiles.hpp"
#include "qgemv.hpp"
#include "route.hpp"
#include "../../include/knurlogic_amd.h"

namespace kmi {



// Token-major wins up to 64 pairs (Qwen3.5-MoE shape, 4-bit: T = 4 33 vs
// 46 us grouped, T = 8 60 vs 64 us) and loses above (T = 16 105 vs 83 us:
// each pair re-reads its expert).
constexpr int64_t TOK_MAX_PAIRS = 64;

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

struct GluPlan {
    bool tok;
    bool gemm;      // expert tiles of 128 or 256 rows on the grouped GEMM (moe_gemm.hip)
    int tm;
    size_t act, y, idx, total;
};

// Rows per active expert from which both projections run as a grouped GEMM
// (prefill chunks: 64 rows fill four 16-row fragments of the skinny kernels)
constexpr int64_t GEMM_MIN_ROWS = 64;

// rows per tile: the average routed pairs per active expert, in 16-row chunks
// (gemm_ok: the grouped GEMM takes these weights)
static GluPlan plan_glu(int64_t T, int64_t H, int64_t I, int k, int64_t E, bool gemm_ok) {
    GluPlan p = {};
    const int64_t P = T * k;
    p.tok = P <= TOK_MAX_PAIRS;
    p.act = align256((size_t)P * I * 2);
    if (!p.tok) {
        const int64_t active = P < E ? P : E;
        const int64_t rpt = ceil_div(P, active);
        // at one or two rows per active expert, 4-row tiles: both projections
        // then stage their x rows once per workgroup (qgemv_xs) with two
        // workgroups per CU
        const int tm_skinny = rpt <= 2 ? 4 : qgemv_gather_tile_rows(rpt);
        p.gemm = gemm_ok && rpt >= GEMM_MIN_ROWS;
        p.tm = p.gemm ? (rpt <= 128 ? 128 : 256) : tm_skinny;
        p.y = align256((size_t)P * H * 2);
        // sized for either tiling, so the workspace query need not know the mode
        const size_t a = sort_index_bytes(P, E, tm_skinny), b = sort_index_bytes(P, E, p.gemm ? p.tm : tm_skinny);
        p.idx = a > b ? a : b;
    }
    p.total = p.act + p.y + p.idx;
    return p;
}

}  // namespace kmi

using namespace kmi;

extern "C" {

size_t kmi_switch_glu_workspace_bytes(int64_t T, int64_t H, int64_t I, int k, int64_t E,
                                      int group_size, int bits) {
    if (T <= 0 || H <= 0 || I <= 0 || k <= 0 || E <= 0) return 0;
    return plan_glu(T, H, I, k, E, moe_gemm_supported(H, I, bits, group_size, 0)).total;
}

}  // extern "C"

// SwitchGLU + combine; with route_logits (token-major only) the gate/up
// kernel routes each token itself and writes route_inds / route_scores,
// which the down kernel then reads as inds / scores.  routed: inds come
// from the router (every expert in range), so at a few pairs the expert
// kernels form their tiles themselves and no sort runs.
static int switch_glu_impl(const void* x, int64_t T, int64_t H, int64_t I, int k, const int32_t* inds,
                           const void* scores, const uint32_t* w_gu, const void* s_gu, const void* b_gu,
                           const uint32_t* w_down, const void* s_down, const void* b_down,
                           int64_t E, int dtype, int group_size, int bits, void* out, void* workspace,
                           size_t workspace_bytes, void* stream, const void* route_logits,
                           int32_t* route_inds, void* route_scores, int mx = 0, bool routed = false) {
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
    KMI_CHECK_ARG(x && inds && w_gu && s_gu && w_down && s_down && out && (mx || (b_gu && b_down)),
                  "switch_glu: null pointer");
    const int epw = 32 / bits;
    KMI_CHECK_ARG(E * 2 * I * (H / epw) * 4 < (1LL << 31) && E * H * (I / epw) * 4 < (1LL << 31),
                  "switch_glu: expert weights past 2 GiB");
    KMI_CHECK_ARG(E <= 4096, "switch_glu: %lld experts (at most 4096)", (long long)E);
    KMI_CHECK_ARG(T * H * 2 < (1LL << 31) && T * k * (H > I ? H : I) * 2 < (1LL << 31),
                  "switch_glu: activations past 2 GiB");
    const GluPlan p = plan_glu(T, H, I, k, E, moe_gemm_supported(H, I, bits, group_size, mx));
    KMI_CHECK_ARG(!mx || group_size == 32, "switch_glu (mx): group %d (32)", group_size);
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
        g.logits = (const uint16_t*)route_logits;
        g.inds_out = route_inds;
        g.scores_out = (uint16_t*)route_scores;
        g.x = (const uint16_t*)x;
        // scales: bf16 (affine) or one byte (mx); the up rows start I rows in
        const int64_t sbw = mx ? 1 : 2;
        g.w0 = w_gu; g.s0 = (const uint16_t*)s_gu; g.b0 = (const uint16_t*)b_gu;
        g.w1 = w_gu + I * wpr_h; g.s1 = (const uint16_t*)((const char*)s_gu + I * gpr_h * sbw);
        g.b1 = mx ? nullptr : (const uint16_t*)b_gu + I * gpr_h;
        g.inds = inds; g.out = act;
        g.E = E; g.N = I; g.K = H; g.T = T; g.erows = 2 * I; g.k = k; g.gs_shift = gs_shift; g.mx = mx;
        int rc = launch_moe_glu_tok(g, bits, st);
        if (rc) return rc;
        KMI_CHECK_LAUNCH("moe_glu_tok");
        MoeTokArgs d = {};
        d.x = act; d.w0 = w_down; d.s0 = (const uint16_t*)s_down; d.b0 = (const uint16_t*)b_down;
        d.inds = inds; d.scores = (const uint16_t*)scores; d.out = (uint16_t*)out;
        d.E = E; d.N = H; d.K = I; d.T = T; d.erows = H; d.k = k; d.gs_shift = gs_shift; d.mx = mx;
        rc = launch_moe_down_tok(d, bits, st);
        if (rc) return rc;
        KMI_CHECK_LAUNCH("moe_down_tok");
        return OK;
    }
    // grouped by expert: one sort (or, for a few routed pairs, tiles formed
    // in the x-staged kernels), gate|up + SwiGLU, down, combine
    uint16_t* y = scores ? (uint16_t*)(ws + p.act) : (uint16_t*)out;    // [P, H]
    SortedRows sr = {};
    bool have_sort = false;
    auto sort = [&]() -> int {       // once, where a kernel needs the sort's list
        if (have_sort) return OK;
        have_sort = true;
        return launch_sort_rows(inds, P, 1, (int)E, p.tm, ws + p.act + p.y, y, H, st, &sr);
    };
    const bool formed = routed && !p.gemm && p.tm == 4 && pair_tiles_fit(P, E, p.tm);
    int rc = formed ? OK : sort();
    if (rc) return rc;
    const int64_t max_tiles = sort_max_tiles(P, E, p.tm);
    auto take_sort = [&](QgArgs& a) -> int {
        const int r = sort();
        a.tiles = sr.tiles; a.sorted = sr.sorted; a.route = nullptr;
        return r;
    };
    QgArgs g = {};
    g.x = (const uint16_t*)x; g.xrows = T; g.w = w_gu; g.s = (const uint16_t*)s_gu;
    g.b = (const uint16_t*)b_gu; g.E = E; g.N = I; g.K = H; g.erows = 2 * I; g.up_off = I; g.mx = mx;
    g.y = act; g.rows = P; g.tm = p.tm; g.tiles = sr.tiles; g.sorted = sr.sorted; g.lhs = nullptr;
    g.lhs_div = k; g.Mper = 1;
    // formed tiles: the gate|up kernel also writes the sort's list (in the
    // sort's place in the workspace) for the down kernel
    int32_t* const list = (int32_t*)(ws + p.act + p.y);
    if (formed) {
        g.route = inds;
        g.sorted_out = list;
        g.tiles_out = list + P;
    }
    if (p.gemm) {
        rc = launch_moe_gemm(g, bits, group_size, true, p.tm, max_tiles, st);
        if (rc) return rc;
    } else {
        const QgPlan pg = plan_qgemv_unsplit(I, H, max_tiles, p.tm, group_size);
        g.S = 1; g.gps = pg.gps;
        if (p.tm != 4 || launch_qgemv_xs(g, bits, group_size, true, p.tm, max_tiles, st) != 0) {
            if ((rc = take_sort(g)) != OK) return rc;
            rc = launch_qgemv(g, pg, bits, group_size, true, max_tiles, st);
            if (rc) return rc;
        }
    }
    KMI_CHECK_LAUNCH(p.gemm ? "moe_gemm(gate|up)" : "qgemv(gate|up)");
    QgArgs d = {};
    d.x = act; d.xrows = P; d.w = w_down; d.s = (const uint16_t*)s_down; d.b = (const uint16_t*)b_down;
    d.E = E; d.N = H; d.K = I; d.erows = H; d.y = y; d.rows = P; d.tm = p.tm; d.tiles = sr.tiles; d.mx = mx;
    d.sorted = sr.sorted; d.lhs = nullptr; d.lhs_div = 1; d.Mper = 1;
    if (formed && !have_sort) {     // the list the gate|up kernel wrote
        d.sorted = list;
        d.tiles = list + P;
    }
    if (p.gemm) {
        rc = launch_moe_gemm(d, bits, group_size, false, p.tm, max_tiles, st);
        if (rc) return rc;
    } else {
        const QgPlan pd = plan_qgemv_unsplit(H, I, max_tiles, p.tm, group_size);
        d.S = 1; d.gps = pd.gps;
        // the down projection stages each tile's act rows once (qgemv_xs)
        // where they fit
        if (launch_qgemv_xs(d, bits, group_size, false, p.tm, max_tiles, st) != 0) {
            if ((rc = take_sort(d)) != OK) return rc;
            rc = launch_qgemv(d, pd, bits, group_size, false, max_tiles, st);
            if (rc) return rc;
        }
    }
    KMI_CHECK_LAUNCH(p.gemm ? "moe_gemm(down)" : "qgemv(down)");
    if (scores) return kmi_moe_combine(y, scores, dtype, T, k, H, out, stream);
    return OK;
}

extern "C" {

int kmi_switch_glu(const void* x, int64_t T, int64_t H, int64_t I, int k, const int32_t* inds,
                   const void* scores, const uint32_t* w_gu, const void* s_gu, const void* b_gu,
                   const uint32_t* w_down, const void* s_down, const void* b_down,
                   int64_t E, int dtype, int group_size, int bits, void* out, void* workspace,
                   size_t workspace_bytes, void* stream) {
    clear_error();
    return switch_glu_impl(x, T, H, I, k, inds, scores, w_gu, s_gu, b_gu, w_down, s_down, b_down, E, dtype,
                           group_size, bits, out, workspace, workspace_bytes, stream, nullptr, nullptr, nullptr);
}

int kmi_switch_glu_mx(const void* x, int64_t T, int64_t H, int64_t I, int k, const int32_t* inds,
                      const void* scores, const uint32_t* w_gu, const uint8_t* s_gu, const uint32_t* w_down,
                      const uint8_t* s_down, int64_t E, int dtype, int mode, void* out, void* workspace,
                      size_t workspace_bytes, void* stream) {
    clear_error();
    KMI_CHECK_ARG(mode == 1 || mode == 2, "switch_glu (mx): mode %d (1 mxfp4, 2 mxfp8)", mode);
    return switch_glu_impl(x, T, H, I, k, inds, scores, w_gu, s_gu, nullptr, w_down, s_down, nullptr, E, dtype,
                           32, mode == 1 ? 4 : 8, out, workspace, workspace_bytes, stream, nullptr, nullptr,
                           nullptr, 1);
}

int kmi_moe_experts(const void* x, const void* logits, int64_t T, int64_t H, int64_t I, int k, int64_t E,
                    const uint32_t* w_gu, const void* s_gu, const void* b_gu, const uint32_t* w_down,
                    const void* s_down, const void* b_down, int dtype, int group_size, int bits, void* out,
                    int32_t* inds, void* scores, void* workspace, size_t workspace_bytes, void* stream) {
    clear_error();
    KMI_CHECK_ARG(dtype == BF16, "moe_experts: only bfloat16 activations and logits are implemented");
    KMI_CHECK_ARG(E >= 1 && E <= ROUTE_MAX_E && k >= 1 && k <= 8 && k <= E,
                  "moe_experts: top-%d of %lld experts (k <= 8, E <= %d)", k, (long long)E, ROUTE_MAX_E);
    if (T == 0) return OK;
    KMI_CHECK_ARG(logits && inds && scores, "moe_experts: null pointer");
    const GluPlan p = plan_glu(T, H, I, k, E, false);
    if (p.tok && E <= ROUTE_THREADS)   // decode sizes: the gate/up kernel routes its own token
        return switch_glu_impl(x, T, H, I, k, inds, scores, w_gu, s_gu, b_gu, w_down, s_down, b_down, E, dtype,
                               group_size, bits, out, workspace, workspace_bytes, stream, logits, inds, scores);
    int rc = kmi_moe_route(logits, dtype, T, (int)E, k, inds, scores, stream);
    if (rc) return rc;
    return switch_glu_impl(x, T, H, I, k, inds, scores, w_gu, s_gu, b_gu, w_down, s_down, b_down, E, dtype,
                           group_size, bits, out, workspace, workspace_bytes, stream, nullptr, nullptr, nullptr, 0,
                           true);
}

}  // extern "C"
