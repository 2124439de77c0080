// 8-bit-KV decode attention for gfx950: the reference's kvattn.decode_sdpa
// semantics (q pre-scaled, softmax over the keys each row may see, a row
// that sees no key returns 0) read straight from the quantized cache.
//
// Work split: one workgroup = (batch b, KV head hk, a block of keys); its 4
// waves each walk their own quarter of the block in steps of 32 keys,
// keeping an online-softmax state for all R = (H/Hk)*L query rows of the KV
// head -- every K/V byte is read from HBM once per call, whatever R is.
// Per step a wave
//   - loads 32 keys of K and V (16-byte loads, each 8-lane group covering a
//     128-byte key row), dequantizes them in fp32 (scale*q + bias, one fp16
//     rounding) into LDS: K^ as [key][d], V^ transposed as [d][key];
//   - S^T[key, r] = K^ Q^T on v_mfma_f32_16x16x32_f16 (Q pre-scaled, fp16,
//     held in registers for the whole call);
//   - rescales its running sums and accumulates O^T[d, r] += V^T P^T on the
//     same MFMA (P in fp16).
// The 4 waves' states merge in LDS (in wave order: deterministic) into one
// fp32 partial (o, m, l) per workgroup; kv8_combine merges the blocks'
// partials (log-sum-exp) and writes q's dtype.
#include "common.hpp"
#include "../../include/knurlogic_amd.h"

namespace kmi {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

struct Kv8Args {
    const void* q;              // [B, H, L, D] contiguous, dtype qdt
    const uint32_t* kw; const void* ks; const void* kb;
    const uint32_t* vw; const void* vs; const void* vb;
    int64_t st[6][3];           // element strides (b, h, n) of kw, ks, kb, vw, vs, vb
    const uint8_t* mask;        // [B, L, N] (1 = key visible) or null
    float* part;                // [B*Hk][nblk][R][D + 2]
    int qdt, sdt;               // dtypes of q and of scales/biases
    int B, H, Hk, L, N, D, group, R, causal, keys_per_wg, nblk;
    float scale;
};

__device__ __forceinline__ float load_any(const void* p, int64_t i, int dt) {
    if (dt == BF16) return bf16_to_f32(((const uint16_t*)p)[i]);
    if (dt == F16) return f16_to_f32(((const uint16_t*)p)[i]);
    return ((const float*)p)[i];
}

__device__ __forceinline__ uint32_t pack_f16(float lo, float hi) {
    f16x2 v = {(_Float16)lo, (_Float16)hi};
    return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ f32x4 mfma_f16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

__device__ __forceinline__ void wave_lds_sync() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_wave_barrier();
}

constexpr int KV_WAVES = 4;
constexpr int KV_STEP = 32;            // keys per wave step

template <int D>
struct KvLds {
    static constexpr int KSTR = D + 8;          // fp16 per K^ row
    static constexpr int VSTR = KV_STEP + 8;    // fp16 per V^T row
    static constexpr int WAVE = KV_STEP * KSTR + D * VSTR;   // fp16 per wave
};

template <int D, int RT>
__global__ __launch_bounds__(256) void kv8_partial(Kv8Args a) {
    constexpr int KSTEPS = D / 32;   // QK k-steps over d
    constexpr int DT = D / 16;       // PV d-tiles
    constexpr int PIECES = D / 16;   // 16-byte pieces per key row
    constexpr int LOADS = 8 * PIECES / 64;   // (key quad, piece) items per lane per step
    using Lds = KvLds<D>;
    extern __shared__ __align__(16) unsigned char smem[];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int bh = blockIdx.y, blk = blockIdx.x;
    const int b = bh / a.Hk, hk = bh % a.Hk;
    const int rep = a.H / a.Hk;
    const int per_wave = a.keys_per_wg / KV_WAVES;
    const int wkey0 = blk * a.keys_per_wg + wave * per_wave;
    const int steps = per_wave / KV_STEP;
    const int l16 = lane & 15, jg = lane >> 4;

    _Float16* kh = (_Float16*)smem + wave * Lds::WAVE;     // [32][KSTR]
    _Float16* vt = kh + KV_STEP * Lds::KSTR;               // [D][VSTR]

    // ---- Q^T operands (fp16, pre-scaled), lane column r ----------------------
    u32x4 qop[RT][KSTEPS];
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        const int r = l16 + 16 * rt;
        const bool rok = r < a.R;
        const int h = hk * rep + (rok ? r / a.L : 0), lq = rok ? r % a.L : 0;
        const int64_t qbase = (((int64_t)b * a.H + h) * a.L + lq) * a.D;
#pragma unroll
        for (int k = 0; k < KSTEPS; k++) {
            const int d0 = 32 * k + 8 * jg;
            u32x4 v;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float x0 = rok ? load_any(a.q, qbase + d0 + 2 * e, a.qdt) * a.scale : 0.f;
                const float x1 = rok ? load_any(a.q, qbase + d0 + 2 * e + 1, a.qdt) * a.scale : 0.f;
                v[e] = pack_f16(x0, x1);
            }
            qop[rt][k] = v;
        }
    }

    float m[RT], lsum[RT];
    f32x4 O[DT][RT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        m[rt] = -INFINITY;
        lsum[rt] = 0.f;
#pragma unroll
        for (int dt = 0; dt < DT; dt++) O[dt][rt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    const int64_t kwb = b * a.st[0][0] + hk * a.st[0][1];
    const int64_t ksb = b * a.st[1][0] + hk * a.st[1][1];
    const int64_t kbb = b * a.st[2][0] + hk * a.st[2][1];
    const int64_t vwb = b * a.st[3][0] + hk * a.st[3][1];
    const int64_t vsb = b * a.st[4][0] + hk * a.st[4][1];
    const int64_t vbb = b * a.st[5][0] + hk * a.st[5][1];

    for (int s = 0; s < steps; s++) {
        const int n0 = wkey0 + s * KV_STEP;
        // ---- load + dequantize 32 keys of K and V into LDS -----------------
#pragma unroll
        for (int it = 0; it < LOADS; it++) {
            const int idx = lane + 64 * it;
            const int quad = idx / PIECES, piece = idx % PIECES;
            const int g = (16 * piece) / a.group;
            u32x4 kd[4], vd[4];
            float ksc[4], kbi[4], vsc[4], vbi[4];
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                const int n = n0 + 4 * quad + kk;
                const bool ok = n < a.N;
                const int nn = ok ? n : 0;
                kd[kk] = ok ? *(const u32x4*)(a.kw + kwb + nn * a.st[0][2] + 4 * piece) : u32x4{0u, 0u, 0u, 0u};
                vd[kk] = ok ? *(const u32x4*)(a.vw + vwb + nn * a.st[3][2] + 4 * piece) : u32x4{0u, 0u, 0u, 0u};
                ksc[kk] = ok ? load_any(a.ks, ksb + nn * a.st[1][2] + g, a.sdt) : 0.f;
                kbi[kk] = ok ? load_any(a.kb, kbb + nn * a.st[2][2] + g, a.sdt) : 0.f;
                vsc[kk] = ok ? load_any(a.vs, vsb + nn * a.st[4][2] + g, a.sdt) : 0.f;
                vbi[kk] = ok ? load_any(a.vb, vbb + nn * a.st[5][2] + g, a.sdt) : 0.f;
            }
            // K^[key][d]: 16 fp16 per key row piece
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                uint32_t o8[8];
#pragma unroll
                for (int w = 0; w < 4; w++) {
                    const uint32_t word = kd[kk][w];
                    const float q0 = (float)(word & 0xffu), q1 = (float)((word >> 8) & 0xffu);
                    const float q2 = (float)((word >> 16) & 0xffu), q3 = (float)(word >> 24);
                    o8[2 * w] = pack_f16(__builtin_fmaf(ksc[kk], q0, kbi[kk]), __builtin_fmaf(ksc[kk], q1, kbi[kk]));
                    o8[2 * w + 1] = pack_f16(__builtin_fmaf(ksc[kk], q2, kbi[kk]), __builtin_fmaf(ksc[kk], q3, kbi[kk]));
                }
                _Float16* dst = kh + (4 * quad + kk) * Lds::KSTR + 16 * piece;
                *(u32x4*)dst = u32x4{o8[0], o8[1], o8[2], o8[3]};
                *(u32x4*)(dst + 8) = u32x4{o8[4], o8[5], o8[6], o8[7]};
            }
            // V^T[d][key]: 4 keys of one d per 8-byte write
#pragma unroll
            for (int w = 0; w < 4; w++) {
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    float f[4];
#pragma unroll
                    for (int kk = 0; kk < 4; kk++)
                        f[kk] = __builtin_fmaf(vsc[kk], (float)((vd[kk][w] >> (8 * e)) & 0xffu), vbi[kk]);
                    const int d = 16 * piece + 4 * w + e;
                    *(u32x2*)(vt + d * Lds::VSTR + 4 * quad) = u32x2{pack_f16(f[0], f[1]), pack_f16(f[2], f[3])};
                }
            }
        }
        wave_lds_sync();

        // ---- S^T = K^ Q^T ------------------------------------------------------
        f32x4 S[2][RT];
#pragma unroll
        for (int nt = 0; nt < 2; nt++) {
#pragma unroll
            for (int rt = 0; rt < RT; rt++) S[nt][rt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int k = 0; k < KSTEPS; k++) {
                const u32x4 A = *(const u32x4*)(kh + (16 * nt + l16) * Lds::KSTR + 32 * k + 8 * jg);
#pragma unroll
                for (int rt = 0; rt < RT; rt++) S[nt][rt] = mfma_f16(A, qop[rt][k], S[nt][rt]);
            }
        }

        // ---- online softmax over this step's keys, per row r -----------------
        u32x4 P[RT];
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            const int r = l16 + 16 * rt;
            const int lq = r % a.L;
            float sv[8];
            float bm = -INFINITY;
#pragma unroll
            for (int nt = 0; nt < 2; nt++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int n = n0 + 16 * nt + 4 * jg + i;
                    bool ok = n < a.N && r < a.R;
                    if (a.causal) ok = ok && n <= a.N - a.L + lq;
                    if (a.mask) ok = ok && a.mask[((int64_t)b * a.L + lq) * a.N + (ok ? n : 0)] != 0;
                    const float v = ok ? S[nt][rt][i] : -INFINITY;
                    sv[4 * nt + i] = v;
                    bm = fmaxf(bm, v);
                }
            bm = fmaxf(bm, __shfl_xor(bm, 16, 64));
            bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
            const float mn = fmaxf(m[rt], bm);
            float corr = 1.f, ps = 0.f;
            float p[8];
            if (mn == -INFINITY) {
#pragma unroll
                for (int e = 0; e < 8; e++) p[e] = 0.f;
            } else {
                corr = __expf(m[rt] - mn);   // m = -inf -> 0
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    p[e] = __expf(sv[e] - mn);
                    ps += p[e];
                }
            }
            ps += __shfl_xor(ps, 16, 64);
            ps += __shfl_xor(ps, 32, 64);
            lsum[rt] = lsum[rt] * corr + ps;
            m[rt] = mn;
#pragma unroll
            for (int dt = 0; dt < DT; dt++) O[dt][rt] *= corr;
            P[rt] = u32x4{pack_f16(p[0], p[1]), pack_f16(p[2], p[3]), pack_f16(p[4], p[5]), pack_f16(p[6], p[7])};
        }

        // ---- O^T += V^T P^T  (key order: lane group j holds keys 4j..4j+3 and 16+4j..16+4j+3)
#pragma unroll
        for (int dt = 0; dt < DT; dt++) {
            const _Float16* row = vt + (16 * dt + l16) * Lds::VSTR;
            const u32x2 lo = *(const u32x2*)(row + 4 * jg);
            const u32x2 hi = *(const u32x2*)(row + 16 + 4 * jg);
            const u32x4 A = u32x4{lo.x, lo.y, hi.x, hi.y};
#pragma unroll
            for (int rt = 0; rt < RT; rt++) O[dt][rt] = mfma_f16(A, P[rt], O[dt][rt]);
        }
        wave_lds_sync();   // the next step overwrites K^ / V^T
    }

    // ---- merge the 4 waves (wave order), write this block's partial -------------
    __syncthreads();
    float* fs = (float*)smem;                       // reuses the K^/V^T area
    float* mw = fs;                                 // [4][R]
    float* lw = mw + KV_WAVES * 64;                 // [4][R]
    float* osum = lw + KV_WAVES * 64;               // [R][D]
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        const int r = l16 + 16 * rt;
        if (jg == 0 && r < a.R) {
            mw[wave * 64 + r] = m[rt];
            lw[wave * 64 + r] = lsum[rt];
        }
    }
    __syncthreads();
    float f[RT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        const int r = l16 + 16 * rt;
        float M = -INFINITY;
        if (r < a.R)
            for (int w = 0; w < KV_WAVES; w++) M = fmaxf(M, mw[w * 64 + r]);
        f[rt] = (M == -INFINITY || m[rt] == -INFINITY) ? 0.f : __expf(m[rt] - M);
    }
    for (int w = 0; w < KV_WAVES; w++) {
        if (wave == w) {
#pragma unroll
            for (int rt = 0; rt < RT; rt++) {
                const int r = l16 + 16 * rt;
                if (r >= a.R) continue;
#pragma unroll
                for (int dt = 0; dt < DT; dt++)
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int d = 16 * dt + 4 * jg + i;
                        const float v = O[dt][rt][i] * f[rt];
                        osum[r * D + d] = (w == 0) ? v : osum[r * D + d] + v;
                    }
            }
        }
        __syncthreads();
    }
    float* out = a.part + ((int64_t)bh * a.nblk + blk) * a.R * (D + 2);
    for (int i = tid; i < a.R * D; i += blockDim.x) out[(i / D) * (D + 2) + (i % D)] = osum[i];
    for (int r = tid; r < a.R; r += blockDim.x) {
        float M = -INFINITY;
        for (int w = 0; w < KV_WAVES; w++) M = fmaxf(M, mw[w * 64 + r]);
        float L = 0.f;
        if (M != -INFINITY)
            for (int w = 0; w < KV_WAVES; w++) {
                const float mwv = mw[w * 64 + r];
                if (mwv != -INFINITY) L += lw[w * 64 + r] * __expf(mwv - M);
            }
        out[r * (D + 2) + D] = M;
        out[r * (D + 2) + D + 1] = L;
    }
}

// out[b, h, l, d] = sum_blk w_blk o_blk[d] / sum_blk w_blk l_blk, w = exp(m_blk - max m);
// 0 when no block saw a key (the reference kernel's rule).
__global__ void kv8_combine(const float* __restrict__ part, int nblk, int R, int D, int H, int Hk,
                            int L, int qdt, void* __restrict__ out) {
    const int row = blockIdx.x;            // (b*Hk + hk) * R + r
    const int bh = row / R, r = row % R;
    const int b = bh / Hk, hk = bh % Hk;
    const int rep = H / Hk;
    const int h = hk * rep + r / L, lq = r % L;
    const float* p = part + ((int64_t)bh * nblk) * R * (D + 2) + (int64_t)r * (D + 2);
    const int64_t bstride = (int64_t)R * (D + 2);
    float M = -INFINITY;
    for (int i = 0; i < nblk; i++) M = fmaxf(M, p[i * bstride + D]);
    const int64_t oi = (((int64_t)b * H + h) * L + lq) * D;
    for (int d = threadIdx.x; d < D; d += blockDim.x) {
        float num = 0.f, den = 0.f;
        if (M != -INFINITY) {
            for (int i = 0; i < nblk; i++) {
                const float mi = p[i * bstride + D];
                if (mi == -INFINITY) continue;
                const float w = __expf(mi - M);
                den += w * p[i * bstride + D + 1];
                num += w * p[i * bstride + d];
            }
        }
        const float v = den > 0.f ? num / den : 0.f;
        if (qdt == BF16) ((uint16_t*)out)[oi + d] = f32_to_bf16(v);
        else if (qdt == F16) ((uint16_t*)out)[oi + d] = f32_to_f16(v);
        else ((float*)out)[oi + d] = v;
    }
}

__global__ void fill_zero_u32(uint32_t* __restrict__ p, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

struct Kv8Plan {
    int keys_per_wg, nblk, rt;
    size_t lds;
};

static Kv8Plan plan_kv8(int B, int Hk, int N, int D, int R) {
    Kv8Plan p;
    p.rt = (R + 15) / 16;
    // keys per workgroup: 4 waves x whole steps, ~1024 workgroups overall
    const int64_t pairs = (int64_t)B * Hk;
    int64_t want_blk = ceil_div(1024, pairs);
    int64_t kpw = ceil_div(N, want_blk);
    kpw = ceil_div(kpw, KV_WAVES * KV_STEP) * KV_WAVES * KV_STEP;
    if (kpw < KV_WAVES * KV_STEP) kpw = KV_WAVES * KV_STEP;
    p.keys_per_wg = (int)kpw;
    p.nblk = (int)ceil_div(N, kpw);
    const size_t waves = (size_t)KV_WAVES * (KV_STEP * (D + 8) + D * (KV_STEP + 8)) * 2;
    const size_t merge = (size_t)(2 * KV_WAVES * 64 + R * D) * 4;
    p.lds = waves > merge ? waves : merge;
    return p;
}

}  // namespace kmi

using namespace kmi;

extern "C" {

size_t kmi_kv8_workspace_bytes(int B, int H, int Hk, int L, int N, int D) {
    if (B <= 0 || H <= 0 || Hk <= 0 || L <= 0 || N <= 0 || D <= 0 || H % Hk) return 0;
    const int R = (H / Hk) * L;
    Kv8Plan p = plan_kv8(B, Hk, N, D, R);
    return (size_t)B * Hk * p.nblk * R * (D + 2) * sizeof(float);
}

int kmi_kv8_decode(const void* q, int q_dtype, int B, int H, int L, int D,
                   const uint32_t* kw, const void* ks, const void* kb,
                   const uint32_t* vw, const void* vs, const void* vb,
                   const int64_t* strides, int scale_dtype, int Hk, int N, int group,
                   float scale, const uint8_t* mask, int causal, void* out,
                   void* workspace, size_t workspace_bytes, void* stream) {
    clear_error();
    KMI_CHECK_ARG(q && kw && ks && kb && vw && vs && vb && out && strides, "kv8_decode: null pointer");
    KMI_CHECK_ARG(B > 0 && H > 0 && L > 0 && Hk > 0 && H % Hk == 0, "kv8_decode: bad head counts");
    KMI_CHECK_ARG(D == 128 || D == 256, "kv8_decode: head dim %d not in {128, 256}", D);
    KMI_CHECK_ARG(group >= 16 && D % group == 0, "kv8_decode: group %d must divide D=%d and be >= 16", group, D);
    KMI_CHECK_ARG(q_dtype >= BF16 && q_dtype <= F32 && scale_dtype >= BF16 && scale_dtype <= F32,
                  "kv8_decode: bad dtype");
    const int R = (H / Hk) * L;
    KMI_CHECK_ARG(R <= 64, "kv8_decode: %d query rows per KV head (at most 64)", R);
    KMI_CHECK_ARG(!(D == 256 && R > 32), "kv8_decode: head dim 256 takes at most 32 rows per KV head");
    KMI_CHECK_ARG(N >= 0, "kv8_decode: N=%d", N);
    hipStream_t st = (hipStream_t)stream;
    if (N == 0) {   // no key: every row returns 0 (a fill kernel: graph-capture safe)
        const int64_t words = (int64_t)B * H * L * D * (q_dtype == F32 ? 4 : 2) / 4;
        fill_zero_u32<<<(unsigned)ceil_div(words, 256), 256, 0, st>>>((uint32_t*)out, words);
        KMI_CHECK_LAUNCH("kv8_decode(empty)");
        return OK;
    }
    Kv8Plan p = plan_kv8(B, Hk, N, D, R);
    const size_t need = (size_t)B * Hk * p.nblk * R * (D + 2) * sizeof(float);
    if (!workspace || workspace_bytes < need) {
        set_error("kv8_decode: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
        return EWORKSPACE;
    }
    Kv8Args a = {};
    a.q = q; a.kw = kw; a.ks = ks; a.kb = kb; a.vw = vw; a.vs = vs; a.vb = vb;
    for (int i = 0; i < 6; i++)
        for (int j = 0; j < 3; j++) a.st[i][j] = strides[3 * i + j];
    a.mask = mask; a.part = (float*)workspace;
    a.qdt = q_dtype; a.sdt = scale_dtype;
    a.B = B; a.H = H; a.Hk = Hk; a.L = L; a.N = N; a.D = D; a.group = group; a.R = R;
    a.causal = causal && L > 1; a.keys_per_wg = p.keys_per_wg; a.nblk = p.nblk; a.scale = scale;
    dim3 grid((unsigned)p.nblk, (unsigned)(B * Hk));
#define KMI_KV(DD, RR)                                                                          \
    do {                                                                                        \
        static bool attr_set = false;                                                           \
        if (!attr_set) {                                                                        \
            (void)hipFuncSetAttribute((const void*)kv8_partial<DD, RR>,                             \
                                hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);        \
            attr_set = true;                                                                    \
        }                                                                                       \
        kv8_partial<DD, RR><<<grid, 256, p.lds, st>>>(a);                                       \
    } while (0)
    if (D == 128) {
        if (p.rt == 1) KMI_KV(128, 1);
        else if (p.rt == 2) KMI_KV(128, 2);
        else if (p.rt == 3) KMI_KV(128, 3);
        else KMI_KV(128, 4);
    } else {
        if (p.rt == 1) KMI_KV(256, 1);
        else KMI_KV(256, 2);
    }
#undef KMI_KV
    KMI_CHECK_LAUNCH("kv8_partial");
    kv8_combine<<<(unsigned)(B * Hk * R), D < 256 ? D : 256, 0, st>>>(a.part, p.nblk, R, D, H, Hk, L,
                                                                       q_dtype, out);
    KMI_CHECK_LAUNCH("kv8_combine");
    return OK;
}

}  // extern "C"
