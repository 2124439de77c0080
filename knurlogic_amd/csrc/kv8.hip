// 8-bit-KV decode attention for gfx950: the reference's kvattn.decode_sdpa
// semantics (q pre-scaled, softmax over the keys each row may see, a row
// that sees no key returns 0) read straight from the quantized cache.
//
// Work split: one workgroup = (batch b, KV head hk, a block of keys).  Its 4
// waves take interleaved 32-key steps of the block (wave w: keys
// 32*(4j + w) ..), each keeping an online-softmax state for all R = (H/Hk)*L
// query rows of the KV head, so every K/V byte is read from HBM once per
// call whatever R is.  Per step a wave
//   - has the step's packed K/V, scales and biases already in registers (the
//     raw buffer loads for step j+1 are issued before step j's math, and a
//     key past N reads 0 instead of branching);
//   - dequantizes K (scale*q + bias formed in fp32 by v_fma_mix from the
//     code as fp16 1024 + q, one fp16 rounding) straight into
//     v_mfma_f32_16x16x32_f16 A operands: lane (key l16, run jg) owns d in
//     [jg*D/4, (jg+1)*D/4), so its bytes are contiguous and no LDS is used;
//     the pre-scaled Q^T operands use the same d order, which leaves the dot
//     products unchanged;
//   - S^T[key, r] = K^ Q^T; online softmax per row (fp32, exp);
//   - dequantizes V into a wave-private V^T tile in LDS ([d][32 keys],
//     keys stored in the order the P^T operand holds them, so each MFMA A
//     operand is one 16-byte read) and accumulates O^T[d, r] += V^T P^T.
//     A lane dequantizes (4-key quad, 16-d piece) items; lanes 8 i .. 8 i + 7
//     take the 8 quads of one piece, so an 8-byte V^T write of 8 lanes fills
//     one 64-byte row (consecutive pieces, rows 16 d apart, share banks).
// The 4 waves' states merge in LDS (fixed order: deterministic) into one
// partial per workgroup: o / l in fp16 (a convex combination of dequantized
// V rows, so it is bounded like V) and (m, l) in fp32.  kv8_combine merges
// the blocks' partials (log-sum-exp) and writes q's dtype.
//
// kv8_partial keeps every row's state of the KV head in a wave's registers,
// which holds for D = 128 (up to 64 rows) and D = 256 (up to 32) with one
// group per D/4-wide lane run; the other shapes (D up to 512, 64 rows,
// groups of 16 and up) go to kv8_wide (up to 16 rows: one row tile per
// workgroup, its waves splitting the keys) or kv8_rows (17-64 rows: a row
// tile per wave over K/V steps the workgroup dequantizes once into LDS).
#include "common.hpp"
#include "../../include/knurlogic_amd.h"


namespace kmi {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

struct Kv8Args {
    const void* q;              // [B, H, L, D] contiguous, dtype qdt
    const void* base[6];        // kw, ks, kb, vw, vs, vb
    int64_t st[6][3];           // element strides (b, h, n) of the six
    int64_t ext[6];             // bytes from a (b, hk) origin through key N-1
    const uint8_t* mask;        // [B, L, N] (1 = key visible) or null
    _Float16* po;               // [B*Hk][nblk][R][D]  o / l of each block
    float2* pml;                // [B*Hk][nblk][R]     (m, l) of each block
    int qdt;
    int B, H, Hk, L, N, group, R, causal, keys_per_wg, nblk;
    float scale;
};

constexpr int KV_WAVES = 4;
constexpr int KV_STEP = 32;            // keys per wave step
constexpr int KV_WG_KEYS = KV_WAVES * KV_STEP;
// kv8_rows: how far a step's max may pass a row's reference max before the
// reference moves (p = exp(s - m) <= e^8 in fp16)
constexpr float KV_LAZY = 8.f;

__device__ __forceinline__ uint32_t pack_f16(float lo, float hi) {
    f16x2 v = {(_Float16)lo, (_Float16)hi};
    return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ f32x4 mfma_f16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// Orders this wave's LDS writes before its later LDS reads.
__device__ __forceinline__ void wave_lds_sync() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_wave_barrier();
}

template <class ST>
__device__ __forceinline__ uint32_t load_scale_raw(__amdgpu_buffer_rsrc_t r, uint32_t elem) {
    if constexpr (sizeof(typename ST::storage) == 4)
        return __builtin_amdgcn_raw_buffer_load_b32(r, (int)(elem * 4u), 0, 0);
    else
        return __builtin_amdgcn_raw_buffer_load_b16(r, (int)(elem * 2u), 0, 0);
}

// the same at a byte offset
template <class ST>
__device__ __forceinline__ uint32_t load_scale_at(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    if constexpr (sizeof(typename ST::storage) == 4)
        return __builtin_amdgcn_raw_buffer_load_b32(r, (int)byte_off, 0, 0);
    else
        return __builtin_amdgcn_raw_buffer_load_b16(r, (int)byte_off, 0, 0);
}

template <class ST>
__device__ __forceinline__ float scale_val(uint32_t raw) {
    if constexpr (sizeof(typename ST::storage) == 4) return __uint_as_float(raw);
    else return ST::load((uint16_t)raw);
}

// ---- byte codes -> fp16 -------------------------------------------------------
// A code byte c becomes the fp16 1024 + c (a v_perm puts the byte 0x64
// above it: exact), and a mixed-precision FMA (v_fma_mix) forms
// s * (1024 + c) + (b - 1024 s) in float32 and rounds it to fp16: s * c + b
// up to the float32 rounding of the offset b - 1024 s (at most 2^-14 |s|)
// and one fp16 rounding -- three instructions per two codes where the
// float32 form (convert, FMA, FMA, pack) takes five.
__device__ __forceinline__ float deq_off(float s, float b) { return __builtin_fmaf(-1024.f, s, b); }

// a code byte as float32 (the form kv8_rows keeps: its 256-register state
// leaves no room for the fp16 pairs)
__device__ __forceinline__ float byte_f(uint32_t w, int e) { return (float)((w >> (8 * e)) & 0xffu); }

// bytes 2 hf and 2 hf + 1 of w as the fp16 pair (1024 + c0, 1024 + c1)
template <int HF>
__device__ __forceinline__ f16x2 magic2(uint32_t w) {
    return __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, w, HF ? 0x04030402u : 0x04010400u));
}

__device__ __forceinline__ _Float16 deq1(float s, _Float16 m, float off) {
    return (_Float16)__builtin_fmaf(s, (float)m, off);
}

__device__ __forceinline__ uint32_t h2bits(_Float16 lo, _Float16 hi) {
    const f16x2 v = {lo, hi};
    return __builtin_bit_cast(uint32_t, v);
}

// the four codes of word w under one scale, as two fp16 pairs (codes 0, 1 and 2, 3)
__device__ __forceinline__ void deq4(uint32_t w, float s, float off, uint32_t& lo, uint32_t& hi) {
    const f16x2 a = magic2<0>(w), c = magic2<1>(w);
    lo = h2bits(deq1(s, a.x, off), deq1(s, a.y, off));
    hi = h2bits(deq1(s, c.x, off), deq1(s, c.y, off));
}

// V^T pieces of four keys: w[kk] is a word of key kk (d = 4i .. 4i + 3 for
// some i); out[e] = the keys' values at d = 4i + e as fp16 pairs (k0, k1), (k2, k3)
__device__ __forceinline__ void deq_vt4(const uint32_t (&w)[4], const float (&s)[4], const float (&off)[4],
                                        u32x2 (&out)[4]) {
    f16x2 m[4][2];
#pragma unroll
    for (int kk = 0; kk < 4; kk++) {
        m[kk][0] = magic2<0>(w[kk]);
        m[kk][1] = magic2<1>(w[kk]);
    }
#pragma unroll
    for (int e = 0; e < 4; e++) {
        _Float16 c[4];
#pragma unroll
        for (int kk = 0; kk < 4; kk++) c[kk] = (e & 1) ? m[kk][e >> 1].y : m[kk][e >> 1].x;
        out[e] = u32x2{h2bits(deq1(s[0], c[0], off[0]), deq1(s[1], c[1], off[1])),
                       h2bits(deq1(s[2], c[2], off[2]), deq1(s[3], c[3], off[3]))};
    }
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ float wave_add(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

template <int D, int RT>
struct KvShape {
    static constexpr int DL = D / 4;             // d per lane run in QK
    static constexpr int KC = DL / 16;           // 16-byte K chunks per lane and key
    static constexpr int KSTEPS = D / 32;        // MFMA k-steps over d
    static constexpr int DT = D / 16;            // PV d tiles
    static constexpr int VP = D / 16;            // 16-byte pieces per V row
    static constexpr int VIT = 8 * VP / 64;      // (key quad, piece) items per lane
    static constexpr int OP = D + 4;             // fp32 per row of a merge slot
    static constexpr size_t vt_bytes = (size_t)KV_WAVES * D * KV_STEP * 2;
    static constexpr size_t merge_bytes = (size_t)(2 * KV_WAVES * 64 + 2 * 16 * RT * OP) * 4;
    static constexpr size_t lds = vt_bytes > merge_bytes ? vt_bytes : merge_bytes;
};

// Q^T operands of v_mfma_f32_16x16x32_f16 for rows r = l16 + 16 rt: the 8 q
// values of d run (D/4)*jg + 8k, times `scale`, in fp16; rows past R are 0.
// All loads are issued before any is used.
template <class QT, int D, int RT>
__device__ __forceinline__ void load_q(u32x4 (&qop)[RT][D / 32], const Kv8Args& a, int b, int hk,
                                       int l16, int jg) {
    constexpr int KSTEPS = D / 32, DL = D / 4;
    constexpr int QES = (int)sizeof(typename QT::storage);
    constexpr int V16 = QES / 2;                  // 16-byte loads per 8 values
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(a.q, (int64_t)a.B * a.H * a.L * D * QES);
    const int rep = a.H / a.Hk;
    u32x4 raw[RT][KSTEPS][V16];
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        const int r = l16 + 16 * rt;
        const int rr = r < a.R ? r : 0;
        const int h = hk * rep + rr / a.L, lq = rr % a.L;
        const uint32_t e0 = (uint32_t)((((b * a.H + h) * a.L + lq) * D) + DL * jg);
#pragma unroll
        for (int k = 0; k < KSTEPS; k++)
#pragma unroll
            for (int v = 0; v < V16; v++)
                raw[rt][k][v] = __builtin_amdgcn_raw_buffer_load_b128(
                    rq, (int)((e0 + 8 * k) * (uint32_t)QES + 16u * v), 0, 0);
    }
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        const bool rok = l16 + 16 * rt < a.R;
#pragma unroll
        for (int k = 0; k < KSTEPS; k++) {
            float x[8];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                if constexpr (QES == 4) {
                    x[e] = __uint_as_float(raw[rt][k][e / 4][e % 4]);
                } else {
                    const uint32_t w = raw[rt][k][0][e / 2];
                    x[e] = QT::load((uint16_t)(e % 2 ? w >> 16 : w & 0xffffu));
                }
            }
            u32x4 o;
#pragma unroll
            for (int e = 0; e < 4; e++) o[e] = rok ? pack_f16(x[2 * e] * a.scale, x[2 * e + 1] * a.scale) : 0u;
            qop[rt][k] = o;
        }
    }
}

// Two workgroups per CU where the state fits 256 registers (D = 128, up to
// 32 rows); otherwise one, so the accumulators may also use AGPRs.
template <int D, int RT>
constexpr int kv8_min_blocks() { return (D == 128 && RT <= 2) ? 2 : 1; }

template <int D, int RT, class ST>
__global__ __launch_bounds__(256, (kv8_min_blocks<D, RT>())) void kv8_partial(Kv8Args a) {
    using S_ = KvShape<D, RT>;
    constexpr int DL = S_::DL, KC = S_::KC, KSTEPS = S_::KSTEPS, DT = S_::DT;
    constexpr int VP = S_::VP, VIT = S_::VIT;
    constexpr int ES = (int)sizeof(typename ST::storage);
    constexpr bool RESCALE_ALWAYS = D == 256 && RT == 2;
    extern __shared__ __align__(16) unsigned char smem[];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, jg = lane >> 4;
    const int bh = blockIdx.y, blk = blockIdx.x;
    const int b = bh / a.Hk, hk = bh % a.Hk;
    const int R = a.R, N = a.N, L = a.L;

    // buffer views of this (b, hk): a key past N reads 0
    const char* bp[6];
#pragma unroll
    for (int i = 0; i < 6; i++) {
        const int es = (i == 0 || i == 3) ? 4 : ES;
        bp[i] = (const char*)a.base[i] + (b * a.st[i][0] + hk * a.st[i][1]) * es;
    }
    const uint32_t kst = (uint32_t)a.st[0][2] * 4u, vst = (uint32_t)a.st[3][2] * 4u;
    const uint32_t kss = (uint32_t)a.st[1][2], kbs = (uint32_t)a.st[2][2];
    const uint32_t vss = (uint32_t)a.st[4][2], vbs = (uint32_t)a.st[5][2];
    const uint32_t kgi = (uint32_t)((DL * jg) / a.group);   // K group of this lane's d run

    const int steps = a.keys_per_wg / KV_WG_KEYS;
    const int kbase = blk * a.keys_per_wg + wave * KV_STEP;

    // ---- raw step data, in flight one step ahead -------------------------------
    u32x4 kr[2][KC];
    uint32_t ksr[2], kbr[2];
    u32x4 vr[VIT][4];
    uint32_t vsr[VIT][4], vbr[VIT][4];

    // Per-lane parts of every load's byte offset, formed once (the first key
    // of the lane's group of rows); a load adds the wave-uniform rest -- its
    // key's offset from there times the row stride, a scalar -- in one v_add.
    const uint32_t kssb = kss * ES, kbsb = kbs * ES, vssb = vss * ES, vbsb = vbs * ES;
    const uint32_t kwo = (uint32_t)l16 * kst + (uint32_t)(DL * jg);
    const uint32_t kso = (uint32_t)l16 * kssb + kgi * ES, kbo = (uint32_t)l16 * kbsb + kgi * ES;
    uint32_t vwo[VIT], vso[VIT], vbo[VIT];
#pragma unroll
    for (int it = 0; it < VIT; it++) {
        const int idx = lane + 64 * it;
        const int quad = idx % 8, piece = idx / 8;   // lanes 8 i .. 8 i + 7: the 8 quads of a piece
        const uint32_t g = (uint32_t)((16 * piece) / a.group);
        vwo[it] = 4u * quad * vst + 16u * piece;
        vso[it] = 4u * quad * vssb + g * ES;
        vbo[it] = 4u * quad * vbsb + g * ES;
    }

    // Loads of step j.  Issued unconditionally, so the loop carries no
    // "loaded or not" state: past the last step the views have extent 0 and
    // the loads return 0 without touching memory.
    auto issue = [&](int j) {
        const bool live = j < steps;
        __amdgpu_buffer_rsrc_t rs[6];
#pragma unroll
        for (int i = 0; i < 6; i++) rs[i] = make_rsrc(bp[i], live ? a.ext[i] : 0);
        const uint32_t n0 = (uint32_t)(kbase + (live ? j : 0) * KV_WG_KEYS);   // wave-uniform
#pragma unroll
        for (int nt = 0; nt < 2; nt++) {
            const uint32_t n = n0 + 16u * nt;
            const uint32_t wo = kwo + n * kst;
#pragma unroll
            for (int c = 0; c < KC; c++)
                kr[nt][c] = __builtin_amdgcn_raw_buffer_load_b128(rs[0], (int)(wo + 16u * c), 0, AUX_NT);
            ksr[nt] = load_scale_at<ST>(rs[1], kso + n * kssb);
            kbr[nt] = load_scale_at<ST>(rs[2], kbo + n * kbsb);
        }
#pragma unroll
        for (int it = 0; it < VIT; it++)
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                const uint32_t n = n0 + kk;
                vr[it][kk] = __builtin_amdgcn_raw_buffer_load_b128(rs[3], (int)(vwo[it] + n * vst), 0, AUX_NT);
                vsr[it][kk] = load_scale_at<ST>(rs[4], vso[it] + n * vssb);
                vbr[it][kk] = load_scale_at<ST>(rs[5], vbo[it] + n * vbsb);
            }
    };
    issue(0);

    // ---- Q^T operands (fp16, pre-scaled): lane column r, d run jg ---------------
    u32x4 qop[RT][KSTEPS];
    if (a.qdt == F32) load_q<TF32, D, RT>(qop, a, b, hk, l16, jg);
    else if (a.qdt == F16) load_q<TF16, D, RT>(qop, a, b, hk, l16, jg);
    else load_q<TBF16, D, RT>(qop, a, b, hk, l16, jg);

    float m[RT], lsum[RT];
    f32x4 O[DT][RT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        m[rt] = -INFINITY;
        lsum[rt] = 0.f;
#pragma unroll
        for (int dt = 0; dt < DT; dt++) O[dt][rt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    _Float16* vt = (_Float16*)smem + wave * D * KV_STEP;   // [D][32] V^T in P^T key order
    const bool has_mask = a.mask != nullptr;
    const __amdgpu_buffer_rsrc_t rm = make_rsrc(a.mask, (int64_t)a.B * L * N);

    for (int j = 0; j < steps; j++) {
        const int n0 = kbase + j * KV_WG_KEYS;
        // mask bytes of this lane's 8 keys per row, loaded first and used at the
        // softmax, so waiting on them does not wait on the next step's loads
        uint32_t mraw[RT][8];
        if (has_mask) {
#pragma unroll
            for (int rt = 0; rt < RT; rt++) {
                const int r = l16 + 16 * rt;
                const uint32_t row = (uint32_t)((b * L + (r < R ? r : 0) % L) * N);
#pragma unroll
                for (int e = 0; e < 8; e++)
                    mraw[rt][e] = __builtin_amdgcn_raw_buffer_load_b8(
                        rm, (int)(row + (uint32_t)(n0 + 16 * (e >> 2) + 4 * jg + (e & 3))), 0, 0);
            }
        } else {
#pragma unroll
            for (int rt = 0; rt < RT; rt++)
#pragma unroll
                for (int e = 0; e < 8; e++) mraw[rt][e] = 1u;
        }

        // ---- K^ -> MFMA A operands: kop[nt][2c + hh] = d run 16c + 8hh of the lane's DL
        u32x4 kop[2][KSTEPS];
#pragma unroll
        for (int nt = 0; nt < 2; nt++) {
            const float s = scale_val<ST>(ksr[nt]), off = deq_off(s, scale_val<ST>(kbr[nt]));
#pragma unroll
            for (int c = 0; c < KC; c++)
#pragma unroll
                for (int hh = 0; hh < 2; hh++) {
                    u32x4 o;
#pragma unroll
                    for (int w2 = 0; w2 < 2; w2++) {
                        uint32_t lo, hi;
                        deq4(kr[nt][c][2 * hh + w2], s, off, lo, hi);
                        o[2 * w2] = lo;
                        o[2 * w2 + 1] = hi;
                    }
                    kop[nt][2 * c + hh] = o;
                }
        }
        // ---- V^ -> V^T tile: quad q (keys 4q..4q+3) sits at fp16 offset 8(q&3) + 4(q>>2)
#pragma unroll
        for (int it = 0; it < VIT; it++) {
            const int idx = lane + 64 * it;
            const int quad = idx % 8, piece = idx / 8;
            const int slot = 8 * (quad & 3) + 4 * (quad >> 2);
            float s[4], off[4];
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                s[kk] = scale_val<ST>(vsr[it][kk]);
                off[kk] = deq_off(s[kk], scale_val<ST>(vbr[it][kk]));
            }
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const uint32_t wk[4] = {vr[it][0][w], vr[it][1][w], vr[it][2][w], vr[it][3][w]};
                u32x2 pr[4];
                deq_vt4(wk, s, off, pr);
#pragma unroll
                for (int e = 0; e < 4; e++) *(u32x2*)(vt + (16 * piece + 4 * w + e) * KV_STEP + slot) = pr[e];
            }
        }

        issue(j + 1);   // next step's bytes stream in during this step's math
        wave_lds_sync();

        // ---- S^T = K^ Q^T --------------------------------------------------------
        f32x4 S[2][RT];
#pragma unroll
        for (int nt = 0; nt < 2; nt++)
#pragma unroll
            for (int rt = 0; rt < RT; rt++) {
                f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int k = 0; k < KSTEPS; k++) acc = mfma_f16(kop[nt][k], qop[rt][k], acc);
                S[nt][rt] = acc;
            }

        // ---- online softmax over this step's keys, per row --------------------------
        // every key of the step visible to every row (no mask, inside N and,
        // causal, below every row's diagonal): no per-key test
        const bool plain = !has_mask && n0 + KV_STEP + (a.causal ? L - 1 : 0) <= N;
        u32x4 P[RT];
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            const int r = l16 + 16 * rt;
            const int lq = (r < R ? r : 0) % L;
            float sv[8];
            float bm = -INFINITY;
            if (plain) {
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const float v = r < R ? S[e >> 2][rt][e & 3] : -INFINITY;
                    sv[e] = v;
                    bm = fmaxf(bm, v);
                }
            } else {
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const int n = n0 + 16 * (e >> 2) + 4 * jg + (e & 3);
                    const bool ok = (n < N) & (r < R) & (!a.causal | (n <= N - L + lq)) & (mraw[rt][e] != 0);
                    const float v = ok ? S[e >> 2][rt][e & 3] : -INFINITY;
                    sv[e] = v;
                    bm = fmaxf(bm, v);
                }
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
            // wave-uniform skip while no row's max moved -- except with the
            // 256-wide 2-tile state, whose registers the branch would spill
            if (RESCALE_ALWAYS || __any(corr != 1.f)) {
#pragma unroll
                for (int dt = 0; dt < DT; dt++) O[dt][rt] *= corr;
            }
            P[rt] = u32x4{pack_f16(p[0], p[1]), pack_f16(p[2], p[3]), pack_f16(p[4], p[5]), pack_f16(p[6], p[7])};
        }

        // ---- O^T += V^T P^T: lane (d row l16, run jg) reads the 8 keys P^T holds
#pragma unroll
        for (int dt = 0; dt < DT; dt++) {
            const u32x4 A = *(const u32x4*)(vt + (16 * dt + l16) * KV_STEP + 8 * jg);
#pragma unroll
            for (int rt = 0; rt < RT; rt++) O[dt][rt] = mfma_f16(A, P[rt], O[dt][rt]);
        }
    }

    // ---- merge the 4 waves in a fixed order: (2 -> 0, 3 -> 1), then 1 -> 0 ------
    __syncthreads();                                   // V^T tiles are dead; reuse the LDS
    constexpr int OP = S_::OP, SLOT = 16 * RT * OP;
    float* mw = (float*)smem;                          // [4][64]
    float* lw = mw + KV_WAVES * 64;                    // [4][64]
    float* slot = lw + KV_WAVES * 64;                  // [2][16*RT][OP]
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        if (jg == 0) {
            mw[wave * 64 + l16 + 16 * rt] = m[rt];
            lw[wave * 64 + l16 + 16 * rt] = lsum[rt];
        }
    }
    __syncthreads();
    float Mr[RT], Lr[RT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        const int r = l16 + 16 * rt;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < KV_WAVES; w++) M = fmaxf(M, mw[w * 64 + r]);
        float Ls = 0.f;
        if (M != -INFINITY) {
#pragma unroll
            for (int w = 0; w < KV_WAVES; w++) {
                const float mv = mw[w * 64 + r];
                if (mv != -INFINITY) Ls += lw[w * 64 + r] * __expf(mv - M);
            }
        }
        Mr[rt] = M;
        Lr[rt] = Ls;
        const float f = m[rt] == -INFINITY ? 0.f : __expf(m[rt] - M);
#pragma unroll
        for (int dt = 0; dt < DT; dt++) O[dt][rt] *= f;
    }
    if (wave >= 2) {
        float* sl = slot + (wave - 2) * SLOT;
#pragma unroll
        for (int rt = 0; rt < RT; rt++)
#pragma unroll
            for (int dt = 0; dt < DT; dt++)
                *(f32x4*)(sl + (l16 + 16 * rt) * OP + 16 * dt + 4 * jg) = O[dt][rt];
    }
    __syncthreads();
    if (wave < 2) {
        float* sl = slot + wave * SLOT;
#pragma unroll
        for (int rt = 0; rt < RT; rt++)
#pragma unroll
            for (int dt = 0; dt < DT; dt++) {
                f32x4* p = (f32x4*)(sl + (l16 + 16 * rt) * OP + 16 * dt + 4 * jg);
                O[dt][rt] += *p;
                if (wave == 1) *p = O[dt][rt];   // same wave, same address: in order
            }
    }
    __syncthreads();
    if (wave == 0) {
        const float* sl = slot + SLOT;
        const int64_t pb = ((int64_t)bh * a.nblk + blk) * R;
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            const int r = l16 + 16 * rt;
            if (r >= R) continue;
            const float inv = Lr[rt] > 0.f ? 1.f / Lr[rt] : 0.f;
            _Float16* orow = a.po + (pb + r) * D;
#pragma unroll
            for (int dt = 0; dt < DT; dt++) {
                const f32x4 v = (O[dt][rt] + *(const f32x4*)(sl + r * OP + 16 * dt + 4 * jg)) * inv;
                *(u32x2*)(orow + 16 * dt + 4 * jg) = u32x2{pack_f16(v[0], v[1]), pack_f16(v[2], v[3])};
            }
            if (jg == 0) a.pml[pb + r] = make_float2(Mr[rt], Lr[rt]);
        }
    }
}

// =============================================================================
// kv8_wide: the shapes whose state kv8_partial's registers do not hold --
// head dims up to 512 (D = 128 DC), up to 64 query rows per KV head at any
// head dim, and groups down to 16 (the reference's rule, kvattn.py:221-228,
// for every group size that is a multiple of 16).
//
// One workgroup per (b, hk, key block, 16-row tile): its O accumulators are
// one row tile over all of D (D / 4 fp32 per lane), and R / 16 workgroups
// share a key block, their numbering keeping the row tiles of a block on one
// XCD so the block's K/V bytes come from HBM once and from L2 after.  The 4
// waves take interleaved 32-key steps as in kv8_partial, and a step walks D
// in chunks of 128: K^ chunk -> MFMA A operands (lane (key, run jg) owns
// d in [128 c + 32 jg, +32), a group per 16-d half), S^T += K^ Q^T over the
// chunk; the online softmax over the step's keys; then per chunk V^ into
// the wave's [128][32] V^T tile (P^T key order) and O^T += V^T P^T.  Every
// unit's raw loads (a K chunk, a V chunk) are issued one unit ahead, into
// the register set the previous unit has just freed.  The waves merge in
// LDS as in kv8_partial, and kv8_combine merges the blocks.
// =============================================================================
// Q^T operands of kv8_wide for row r (0 past R): the 8 q values of d run
// 128 c + 32 jg + 8 kk, times `scale`, in fp16.  All loads issue before any use.
template <class QT, int DC>
__device__ __forceinline__ void load_q_wide(u32x4 (&qop)[DC][4], const Kv8Args& a, int b, int hk,
                                            int r, int jg) {
    constexpr int D = 128 * DC;
    constexpr int QES = (int)sizeof(typename QT::storage);
    constexpr int V16 = QES / 2;
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(a.q, (int64_t)a.B * a.H * a.L * D * QES);
    const bool rok = r < a.R;
    const int rr = rok ? r : 0;
    const int h = hk * (a.H / a.Hk) + rr / a.L, lq = rr % a.L;
    const uint32_t e0 = (uint32_t)((((b * a.H + h) * a.L + lq) * D) + 32 * jg);
    u32x4 raw[DC][4][V16];
#pragma unroll
    for (int c = 0; c < DC; c++)
#pragma unroll
        for (int kk = 0; kk < 4; kk++)
#pragma unroll
            for (int v = 0; v < V16; v++)
                raw[c][kk][v] = __builtin_amdgcn_raw_buffer_load_b128(
                    rq, (int)((e0 + 128 * c + 8 * kk) * (uint32_t)QES + 16u * v), 0, 0);
#pragma unroll
    for (int c = 0; c < DC; c++)
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
            float x[8];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                if constexpr (QES == 4) {
                    x[e] = __uint_as_float(raw[c][kk][e / 4][e % 4]);
                } else {
                    const uint32_t w = raw[c][kk][0][e / 2];
                    x[e] = QT::load((uint16_t)(e % 2 ? w >> 16 : w & 0xffffu));
                }
            }
            u32x4 o;
#pragma unroll
            for (int e = 0; e < 4; e++) o[e] = rok ? pack_f16(x[2 * e] * a.scale, x[2 * e + 1] * a.scale) : 0u;
            qop[c][kk] = o;
        }
}

template <int DC, class ST>
__global__ __launch_bounds__(256, 1) void kv8_wide(Kv8Args a, int nrt) {
    constexpr int D = 128 * DC;
    constexpr int ES = (int)sizeof(typename ST::storage);
    extern __shared__ __align__(16) unsigned char smem[];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, jg = lane >> 4;
    // workgroup -> (key block, row tile): the row tiles of a block share an XCD
    const int xid = (int)blockIdx.x, xcd = xid & 7, rest = xid >> 3;
    const int rtile = rest % nrt, blk = (rest / nrt) * 8 + xcd;
    if (blk >= a.nblk) return;
    const int bh = blockIdx.y;
    const int b = bh / a.Hk, hk = bh % a.Hk;
    const int R = a.R, N = a.N, L = a.L;
    const int r = 16 * rtile + l16;                      // this lane's query row
    const bool rok = r < R;

    const char* bp[6];
#pragma unroll
    for (int i = 0; i < 6; i++) {
        const int es = (i == 0 || i == 3) ? 4 : ES;
        bp[i] = (const char*)a.base[i] + (b * a.st[i][0] + hk * a.st[i][1]) * es;
    }
    const uint32_t kst = (uint32_t)a.st[0][2] * 4u, vst = (uint32_t)a.st[3][2] * 4u;
    const uint32_t kss = (uint32_t)a.st[1][2], kbs = (uint32_t)a.st[2][2];
    const uint32_t vss = (uint32_t)a.st[4][2], vbs = (uint32_t)a.st[5][2];

    const int steps = a.keys_per_wg / KV_WG_KEYS;
    const int kbase = blk * a.keys_per_wg + wave * KV_STEP;

    // ---- raw data of one unit, issued a unit ahead --------------------------------
    u32x4 kr[2][2];                 // K chunk: key tile nt, 16-byte half of the lane's 32-d run
    uint32_t ksr[2][2], kbr[2][2];
    u32x4 vr[4];                    // V chunk: the lane's (key quad, 16-byte piece), 4 keys
    uint32_t vsr[4], vbr[4];
    const int vquad = lane & 7, vpiece = lane >> 3;     // 8 quads x 8 pieces of a 128-d chunk
    auto views = [&](bool live, __amdgpu_buffer_rsrc_t (&rs)[6]) {
#pragma unroll
        for (int i = 0; i < 6; i++) rs[i] = make_rsrc(bp[i], live ? a.ext[i] : 0);
    };
    auto issue_k = [&](int j, int c) {
        const bool live = j < steps;
        __amdgpu_buffer_rsrc_t rs[6];
        views(live, rs);
        const uint32_t n0 = (uint32_t)(kbase + (live ? j : 0) * KV_WG_KEYS);
        const uint32_t d0 = (uint32_t)(128 * c + 32 * jg);
#pragma unroll
        for (int nt = 0; nt < 2; nt++) {
            const uint32_t n = n0 + 16u * nt + l16;
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {
                const uint32_t g = (d0 + 16u * hh) / (uint32_t)a.group;
                kr[nt][hh] = __builtin_amdgcn_raw_buffer_load_b128(rs[0], (int)(n * kst + d0 + 16u * hh), 0, AUX_NT);
                ksr[nt][hh] = load_scale_raw<ST>(rs[1], n * kss + g);
                kbr[nt][hh] = load_scale_raw<ST>(rs[2], n * kbs + g);
            }
        }
    };
    auto issue_v = [&](int j, int c) {
        const bool live = j < steps;
        __amdgpu_buffer_rsrc_t rs[6];
        views(live, rs);
        const uint32_t n0 = (uint32_t)(kbase + (live ? j : 0) * KV_WG_KEYS);
        const uint32_t d0 = (uint32_t)(128 * c + 16 * vpiece);
        const uint32_t g = d0 / (uint32_t)a.group;
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
            const uint32_t n = n0 + 4u * vquad + kk;
            vr[kk] = __builtin_amdgcn_raw_buffer_load_b128(rs[3], (int)(n * vst + d0), 0, AUX_NT);
            vsr[kk] = load_scale_raw<ST>(rs[4], n * vss + g);
            vbr[kk] = load_scale_raw<ST>(rs[5], n * vbs + g);
        }
    };
    issue_k(0, 0);

    // ---- Q^T operands (fp16, pre-scaled): row r, d = 128 c + 32 jg + 8 kk .. +8 ---
    u32x4 qop[DC][4];
    if (a.qdt == F32) load_q_wide<TF32, DC>(qop, a, b, hk, r, jg);
    else if (a.qdt == F16) load_q_wide<TF16, DC>(qop, a, b, hk, r, jg);
    else load_q_wide<TBF16, DC>(qop, a, b, hk, r, jg);

    float m = -INFINITY, lsum = 0.f;
    f32x4 O[DC][8];
#pragma unroll
    for (int c = 0; c < DC; c++)
#pragma unroll
        for (int dt = 0; dt < 8; dt++) O[c][dt] = f32x4{0.f, 0.f, 0.f, 0.f};

    _Float16* vt = (_Float16*)smem + wave * 128 * KV_STEP;   // [128][32] V^T in P^T key order
    const bool has_mask = a.mask != nullptr;
    const __amdgpu_buffer_rsrc_t rm = make_rsrc(a.mask, (int64_t)a.B * L * N);
    const int lq = (rok ? r : 0) % L;

    for (int j = 0; j < steps; j++) {
        const int n0 = kbase + j * KV_WG_KEYS;
        uint32_t mraw[8];
        if (has_mask) {
            const uint32_t row = (uint32_t)((b * L + lq) * N);
#pragma unroll
            for (int e = 0; e < 8; e++)
                mraw[e] = __builtin_amdgcn_raw_buffer_load_b8(
                    rm, (int)(row + (uint32_t)(n0 + 16 * (e >> 2) + 4 * jg + (e & 3))), 0, 0);
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++) mraw[e] = 1u;
        }

        // ---- S^T = K^ Q^T, chunk by chunk -------------------------------------------
        f32x4 S[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (int c = 0; c < DC; c++) {
            u32x4 kop[2][4];
#pragma unroll
            for (int nt = 0; nt < 2; nt++) {
#pragma unroll
                for (int kk = 0; kk < 4; kk++) {
                    const float sc = scale_val<ST>(ksr[nt][kk >> 1]);
                    const float off = deq_off(sc, scale_val<ST>(kbr[nt][kk >> 1]));
                    u32x4 o;
#pragma unroll
                    for (int w2 = 0; w2 < 2; w2++) {
                        uint32_t lo, hi;
                        deq4(kr[nt][kk >> 1][2 * (kk & 1) + w2], sc, off, lo, hi);
                        o[2 * w2] = lo;
                        o[2 * w2 + 1] = hi;
                    }
                    kop[nt][kk] = o;
                }
            }
            if (c + 1 < DC) issue_k(j, c + 1);
            else issue_v(j, 0);
#pragma unroll
            for (int nt = 0; nt < 2; nt++)
#pragma unroll
                for (int kk = 0; kk < 4; kk++) S[nt] = mfma_f16(kop[nt][kk], qop[c][kk], S[nt]);
        }

        // ---- online softmax over the step's keys, row r -------------------------------
        u32x4 P;
        {
            float sv[8];
            float bm = -INFINITY;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int n = n0 + 16 * (e >> 2) + 4 * jg + (e & 3);
                const bool ok = (n < N) & rok & (!a.causal | (n <= N - L + lq)) & (mraw[e] != 0);
                const float v = ok ? S[e >> 2][e & 3] : -INFINITY;
                sv[e] = v;
                bm = fmaxf(bm, v);
            }
            bm = fmaxf(bm, __shfl_xor(bm, 16, 64));
            bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
            const float mn = fmaxf(m, bm);
            float corr = 1.f, ps = 0.f;
            float pv[8];
            if (mn == -INFINITY) {
#pragma unroll
                for (int e = 0; e < 8; e++) pv[e] = 0.f;
            } else {
                corr = __expf(m - mn);   // m = -inf -> 0
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    pv[e] = __expf(sv[e] - mn);
                    ps += pv[e];
                }
            }
            ps += __shfl_xor(ps, 16, 64);
            ps += __shfl_xor(ps, 32, 64);
            lsum = lsum * corr + ps;
            m = mn;
            if (__any(corr != 1.f)) {   // wave-uniform: skipped while no row's max moved
#pragma unroll
                for (int c = 0; c < DC; c++)
#pragma unroll
                    for (int dt = 0; dt < 8; dt++) O[c][dt] *= corr;
            }
            P = u32x4{pack_f16(pv[0], pv[1]), pack_f16(pv[2], pv[3]), pack_f16(pv[4], pv[5]), pack_f16(pv[6], pv[7])};
        }

        // ---- O^T += V^T P^T, chunk by chunk: quad q (keys 4q..4q+3) at fp16
        //      offset 8 (q & 3) + 4 (q >> 2) of a V^T row
#pragma unroll
        for (int c = 0; c < DC; c++) {
            {
                const int slot = 8 * (vquad & 3) + 4 * (vquad >> 2);
                float sc[4], off[4];
#pragma unroll
                for (int kk = 0; kk < 4; kk++) {
                    sc[kk] = scale_val<ST>(vsr[kk]);
                    off[kk] = deq_off(sc[kk], scale_val<ST>(vbr[kk]));
                }
#pragma unroll
                for (int w = 0; w < 4; w++) {
                    const uint32_t wk[4] = {vr[0][w], vr[1][w], vr[2][w], vr[3][w]};
                    u32x2 pr[4];
                    deq_vt4(wk, sc, off, pr);
#pragma unroll
                    for (int e = 0; e < 4; e++) *(u32x2*)(vt + (16 * vpiece + 4 * w + e) * KV_STEP + slot) = pr[e];
                }
            }
            if (c + 1 < DC) issue_v(j, c + 1);
            else issue_k(j + 1, 0);
            wave_lds_sync();
#pragma unroll
            for (int dt = 0; dt < 8; dt++) {
                const u32x4 A = *(const u32x4*)(vt + (16 * dt + l16) * KV_STEP + 8 * jg);
                O[c][dt] = mfma_f16(A, P, O[c][dt]);
            }
        }
    }

    // ---- merge the 4 waves in a fixed order: (2 -> 0, 3 -> 1), then 1 -> 0 ------
    __syncthreads();
    constexpr int OP = D + 4, SLOT = 16 * OP;
    float* mw = (float*)smem;                          // [4][16]
    float* lw = mw + KV_WAVES * 16;                    // [4][16]
    float* slot = lw + KV_WAVES * 16;                  // [2][16][OP]
    if (jg == 0) {
        mw[wave * 16 + l16] = m;
        lw[wave * 16 + l16] = lsum;
    }
    __syncthreads();
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < KV_WAVES; w++) M = fmaxf(M, mw[w * 16 + l16]);
    float Ls = 0.f;
    if (M != -INFINITY) {
#pragma unroll
        for (int w = 0; w < KV_WAVES; w++) {
            const float mv = mw[w * 16 + l16];
            if (mv != -INFINITY) Ls += lw[w * 16 + l16] * __expf(mv - M);
        }
    }
    {
        const float f = m == -INFINITY ? 0.f : __expf(m - M);
#pragma unroll
        for (int c = 0; c < DC; c++)
#pragma unroll
            for (int dt = 0; dt < 8; dt++) O[c][dt] *= f;
    }
    if (wave >= 2) {
        float* sl = slot + (wave - 2) * SLOT;
#pragma unroll
        for (int c = 0; c < DC; c++)
#pragma unroll
            for (int dt = 0; dt < 8; dt++)
                *(f32x4*)(sl + l16 * OP + 128 * c + 16 * dt + 4 * jg) = O[c][dt];
    }
    __syncthreads();
    if (wave < 2) {
        float* sl = slot + wave * SLOT;
#pragma unroll
        for (int c = 0; c < DC; c++)
#pragma unroll
            for (int dt = 0; dt < 8; dt++) {
                f32x4* pp = (f32x4*)(sl + l16 * OP + 128 * c + 16 * dt + 4 * jg);
                O[c][dt] += *pp;
                if (wave == 1) *pp = O[c][dt];   // same wave, same address: in order
            }
    }
    __syncthreads();
    if (wave == 0 && rok) {
        const float* sl = slot + SLOT;
        const int64_t pb = ((int64_t)bh * a.nblk + blk) * R;
        const float inv = Ls > 0.f ? 1.f / Ls : 0.f;
        _Float16* orow = a.po + (pb + r) * D;
#pragma unroll
        for (int c = 0; c < DC; c++)
#pragma unroll
            for (int dt = 0; dt < 8; dt++) {
                const f32x4 v = (O[c][dt] + *(const f32x4*)(sl + l16 * OP + 128 * c + 16 * dt + 4 * jg)) * inv;
                *(u32x2*)(orow + 128 * c + 16 * dt + 4 * jg) = u32x2{pack_f16(v[0], v[1]), pack_f16(v[2], v[3])};
            }
        if (jg == 0) a.pml[pb + r] = make_float2(M, Ls);
    }
}

template <int DC>
constexpr size_t kv8_wide_lds() {
    constexpr size_t vt = (size_t)KV_WAVES * 128 * KV_STEP * 2;
    constexpr size_t merge = (size_t)(2 * KV_WAVES * 16 + 2 * 16 * (128 * DC + 4)) * 4;
    return vt > merge ? vt : merge;
}

// =============================================================================
// kv8_rows: kv8_wide's shapes with 17 to 64 query rows per KV head.  One
// workgroup per (b, hk, key block) with all R rows: wave w owns row tile w
// (rows 16 w ..) over every key of the block, so no wave state is merged,
// and per 32-key step the whole workgroup dequantizes the step's K and V
// once into LDS -- K^ [32 keys][D] row-major, V^T [D][32 keys] in P^T key
// order -- which every row tile then reads as MFMA operands.  LDS holds two
// such steps: the step after the current one is dequantized (its raw loads
// issued a step earlier) while the row tiles compute on the current one.
// Row stride paddings of 16 bytes keep 8 consecutive rows' 16-byte reads on
// distinct banks.  Raw-load mapping: K as 16-byte pieces (key idx / (D/16),
// piece idx % (D/16)), DC per thread; V as (key quad, 16-byte piece) items,
// D / 2 of them, one per thread.
// =============================================================================
constexpr int KR_KP = 8;            // fp16 padding of a K^ row
constexpr int KR_VS = KV_STEP + 8;  // fp16 per V^T row (32 keys + padding)

template <int DC>
constexpr size_t kv8_rows_buf() {
    return (size_t)KV_STEP * (128 * DC + KR_KP) * 2 + (size_t)128 * DC * KR_VS * 2;
}

// Q^T operands for row r (0 past R) in natural d order: qop[ks] = the 8 q
// values of d = 32 ks + 8 jg .. +8, times `scale`, in fp16.
template <class QT, int DC>
__device__ __forceinline__ void load_q_rows(u32x4 (&qop)[4 * DC], const Kv8Args& a, int b, int hk, int r,
                                            int jg) {
    constexpr int D = 128 * DC;
    constexpr int QES = (int)sizeof(typename QT::storage);
    constexpr int V16 = QES / 2;
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(a.q, (int64_t)a.B * a.H * a.L * D * QES);
    const bool rok = r < a.R;
    const int rr = rok ? r : 0;
    const int h = hk * (a.H / a.Hk) + rr / a.L, lq = rr % a.L;
    const uint32_t e0 = (uint32_t)((((b * a.H + h) * a.L + lq) * D) + 8 * jg);
    u32x4 raw[4 * DC][V16];
#pragma unroll
    for (int ks = 0; ks < 4 * DC; ks++)
#pragma unroll
        for (int v = 0; v < V16; v++)
            raw[ks][v] = __builtin_amdgcn_raw_buffer_load_b128(rq, (int)((e0 + 32 * ks) * (uint32_t)QES + 16u * v),
                                                               0, 0);
#pragma unroll
    for (int ks = 0; ks < 4 * DC; ks++) {
        float x[8];
#pragma unroll
        for (int e = 0; e < 8; e++) {
            if constexpr (QES == 4) {
                x[e] = __uint_as_float(raw[ks][e / 4][e % 4]);
            } else {
                const uint32_t w = raw[ks][0][e / 2];
                x[e] = QT::load((uint16_t)(e % 2 ? w >> 16 : w & 0xffffu));
            }
        }
        u32x4 o;
#pragma unroll
        for (int e = 0; e < 4; e++) o[e] = rok ? pack_f16(x[2 * e] * a.scale, x[2 * e + 1] * a.scale) : 0u;
        qop[ks] = o;
    }
}

template <int DC, class ST>
__global__ __launch_bounds__(256, 1) void kv8_rows(Kv8Args a) {
    constexpr int D = 128 * DC;
    constexpr int ES = (int)sizeof(typename ST::storage);
    constexpr int KS = D + KR_KP;                   // fp16 per K^ row
    constexpr int PPR = D / 16;                     // 16-byte pieces per key row
    constexpr int KPT = DC;                         // K pieces per thread per step (2 D / 256)
    constexpr int NV = D / 2;                       // V items per step
    constexpr size_t BUF = kv8_rows_buf<DC>();
    extern __shared__ __align__(16) unsigned char smem[];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, jg = lane >> 4;
    const int bh = blockIdx.y, blk = blockIdx.x;
    const int b = bh / a.Hk, hk = bh % a.Hk;
    const int R = a.R, N = a.N, L = a.L;
    const int r = 16 * wave + l16;                  // this lane's query row
    const bool rok = r < R;
    const bool active = 16 * wave < R;              // wave-uniform: the wave has rows

    const char* bp[6];
#pragma unroll
    for (int i = 0; i < 6; i++) {
        const int es = (i == 0 || i == 3) ? 4 : ES;
        bp[i] = (const char*)a.base[i] + (b * a.st[i][0] + hk * a.st[i][1]) * es;
    }
    const uint32_t kst = (uint32_t)a.st[0][2] * 4u, vst = (uint32_t)a.st[3][2] * 4u;
    const uint32_t kssb = (uint32_t)a.st[1][2] * ES, kbsb = (uint32_t)a.st[2][2] * ES;
    const uint32_t vssb = (uint32_t)a.st[4][2] * ES, vbsb = (uint32_t)a.st[5][2] * ES;
    const int steps = a.keys_per_wg / KV_STEP;
    const int kbase = blk * a.keys_per_wg;

    // ---- raw loads of a step: K pieces and the V item, lane bases formed once ----
    int kkey[KPT], kpc[KPT];
    uint32_t kwo[KPT], kgo[KPT];
#pragma unroll
    for (int i = 0; i < KPT; i++) {
        const int idx = tid + 256 * i;
        kkey[i] = idx / PPR;
        kpc[i] = idx % PPR;
        kwo[i] = (uint32_t)kkey[i] * kst + 16u * kpc[i];
        kgo[i] = (uint32_t)((16 * kpc[i]) / a.group) * ES;
    }
    const bool vthr = tid < NV;
    const int vquad = vthr ? tid % 8 : 0, vpiece = vthr ? tid / 8 : 0;
    const uint32_t vwo = 4u * vquad * vst + 16u * vpiece;
    const uint32_t vgo = (uint32_t)((16 * vpiece) / a.group) * ES;
    const uint32_t vkey0 = 4u * vquad;

    u32x4 kr[KPT];
    uint32_t ksr[KPT], kbr[KPT];
    u32x4 vr[4];
    uint32_t vsr[4], vbr[4];
    auto issue = [&](int j) {
        const bool live = j < steps;
        __amdgpu_buffer_rsrc_t rs[6];
#pragma unroll
        for (int i = 0; i < 6; i++) rs[i] = make_rsrc(bp[i], live ? a.ext[i] : 0);
        const uint32_t n0 = (uint32_t)(kbase + (live ? j : 0) * KV_STEP);   // wave-uniform
#pragma unroll
        for (int i = 0; i < KPT; i++) {
            kr[i] = __builtin_amdgcn_raw_buffer_load_b128(rs[0], (int)(kwo[i] + n0 * kst), 0, AUX_NT);
            const uint32_t n = n0 + (uint32_t)kkey[i];
            ksr[i] = load_scale_at<ST>(rs[1], n * kssb + kgo[i]);
            kbr[i] = load_scale_at<ST>(rs[2], n * kbsb + kgo[i]);
        }
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
            const uint32_t n = n0 + vkey0 + kk;
            vr[kk] = __builtin_amdgcn_raw_buffer_load_b128(rs[3], (int)(vwo + (n0 + kk) * vst), 0, AUX_NT);
            vsr[kk] = load_scale_at<ST>(rs[4], n * vssb + vgo);
            vbr[kk] = load_scale_at<ST>(rs[5], n * vbsb + vgo);
        }
    };
    // the raw step -> K^ and V^T of LDS buffer `buf`
    auto dequant = [&](int buf) {
        _Float16* kd = (_Float16*)(smem + buf * BUF);
        _Float16* vt = kd + KV_STEP * KS;
#pragma unroll
        for (int i = 0; i < KPT; i++) {
            const float sc = scale_val<ST>(ksr[i]), bi = scale_val<ST>(kbr[i]);
            u32x4 o[2];
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const uint32_t wd = kr[i][w];
                o[w >> 1][2 * (w & 1)] = pack_f16(__builtin_fmaf(sc, byte_f(wd, 0), bi), __builtin_fmaf(sc, byte_f(wd, 1), bi));
                o[w >> 1][2 * (w & 1) + 1] = pack_f16(__builtin_fmaf(sc, byte_f(wd, 2), bi), __builtin_fmaf(sc, byte_f(wd, 3), bi));
            }
            u32x4* dst = (u32x4*)(kd + kkey[i] * KS + 16 * kpc[i]);
            dst[0] = o[0];
            dst[1] = o[1];
        }
        if (vthr) {
            const int slot = 8 * (vquad & 3) + 4 * (vquad >> 2);
            float sc[4], bi[4];
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                sc[kk] = scale_val<ST>(vsr[kk]);
                bi[kk] = scale_val<ST>(vbr[kk]);
            }
#pragma unroll
            for (int w = 0; w < 4; w++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    float f[4];
#pragma unroll
                    for (int kk = 0; kk < 4; kk++) f[kk] = __builtin_fmaf(sc[kk], byte_f(vr[kk][w], e), bi[kk]);
                    const int d = 16 * vpiece + 4 * w + e;
                    *(u32x2*)(vt + d * KR_VS + slot) = u32x2{pack_f16(f[0], f[1]), pack_f16(f[2], f[3])};
                }
        }
    };

    issue(0);
    u32x4 qop[4 * DC];
    if (a.qdt == F32) load_q_rows<TF32, DC>(qop, a, b, hk, r, jg);
    else if (a.qdt == F16) load_q_rows<TF16, DC>(qop, a, b, hk, r, jg);
    else load_q_rows<TBF16, DC>(qop, a, b, hk, r, jg);
    dequant(0);
    issue(1);
    __syncthreads();

    float m = -INFINITY, lsum = 0.f;
    f32x4 O[DC][8];
#pragma unroll
    for (int c = 0; c < DC; c++)
#pragma unroll
        for (int dt = 0; dt < 8; dt++) O[c][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    const bool has_mask = a.mask != nullptr;
    const __amdgpu_buffer_rsrc_t rm = make_rsrc(a.mask, (int64_t)a.B * L * N);
    const int lq = (rok ? r : 0) % L;

    for (int j = 0; j < steps; j++) {
        const int n0 = kbase + j * KV_STEP;
        const _Float16* kd = (const _Float16*)(smem + (j & 1) * BUF);
        const _Float16* vt = kd + KV_STEP * KS;
        if (active) {
            uint32_t mraw[8];
            if (has_mask) {
                const uint32_t row = (uint32_t)((b * L + lq) * N);
#pragma unroll
                for (int e = 0; e < 8; e++)
                    mraw[e] = __builtin_amdgcn_raw_buffer_load_b8(
                        rm, (int)(row + (uint32_t)(n0 + 16 * (e >> 2) + 4 * jg + (e & 3))), 0, 0);
            } else {
#pragma unroll
                for (int e = 0; e < 8; e++) mraw[e] = 1u;
            }
            // S^T = K^ Q^T: A = K^ rows 16 nt + l16, d 32 ks + 8 jg
            f32x4 S[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
            // 4 k-steps of both key tiles read ahead of their 8 MFMAs
#pragma unroll
            for (int kb = 0; kb < 4 * DC; kb += 4) {
                u32x4 A[2][4];
#pragma unroll
                for (int nt = 0; nt < 2; nt++)
#pragma unroll
                    for (int k4 = 0; k4 < 4; k4++)
                        A[nt][k4] = *(const u32x4*)(kd + (16 * nt + l16) * KS + 32 * (kb + k4) + 8 * jg);
#pragma unroll
                for (int k4 = 0; k4 < 4; k4++)
#pragma unroll
                    for (int nt = 0; nt < 2; nt++) S[nt] = mfma_f16(A[nt][k4], qop[kb + k4], S[nt]);
            }
            // online softmax over the step's keys, row r
            u32x4 P;
            {
                float sv[8];
                float bm = -INFINITY;
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const int n = n0 + 16 * (e >> 2) + 4 * jg + (e & 3);
                    const bool ok = (n < N) & rok & (!a.causal | (n <= N - L + lq)) & (mraw[e] != 0);
                    const float v = ok ? S[e >> 2][e & 3] : -INFINITY;
                    sv[e] = v;
                    bm = fmaxf(bm, v);
                }
                bm = fmaxf(bm, __shfl_xor(bm, 16, 64));
                bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
                // the reference max m moves only when a step's max passes it
                // by more than KV_LAZY (p = exp(s - m) then stays <= e^8 in
                // fp16), so O -- in AGPRs here, three instructions per value
                // to scale -- is rescaled rarely; o / l is unchanged by m
                const bool grow = bm > m + KV_LAZY;   // m = -inf: any key seen
                const float mn = grow ? bm : m;
                float corr = 1.f, ps = 0.f;
                float pv[8];
                if (mn == -INFINITY) {
#pragma unroll
                    for (int e = 0; e < 8; e++) pv[e] = 0.f;
                } else {
                    corr = grow ? __expf(m - mn) : 1.f;   // m = -inf -> 0
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        pv[e] = __expf(sv[e] - mn);
                        ps += pv[e];
                    }
                }
                ps += __shfl_xor(ps, 16, 64);
                ps += __shfl_xor(ps, 32, 64);
                lsum = lsum * corr + ps;
                m = mn;
                if (__any(grow)) {   // wave-uniform
#pragma unroll
                    for (int c = 0; c < DC; c++)
#pragma unroll
                        for (int dt = 0; dt < 8; dt++) O[c][dt] *= corr;
                }
                P = u32x4{pack_f16(pv[0], pv[1]), pack_f16(pv[2], pv[3]), pack_f16(pv[4], pv[5]),
                          pack_f16(pv[6], pv[7])};
            }
            // O^T += V^T P^T: A = V^T rows 128 c + 16 dt + l16, keys 8 jg ..
#pragma unroll
            for (int c = 0; c < DC; c++) {
                u32x4 A[8];   // the chunk's 8 d-tiles read ahead of their MFMAs
#pragma unroll
                for (int dt = 0; dt < 8; dt++)
                    A[dt] = *(const u32x4*)(vt + (128 * c + 16 * dt + l16) * KR_VS + 8 * jg);
#pragma unroll
                for (int dt = 0; dt < 8; dt++) O[c][dt] = mfma_f16(A[dt], P, O[c][dt]);
            }
        }
        if (j + 1 < steps) {      // workgroup-uniform
            dequant((j + 1) & 1);
            issue(j + 2);
        }
        __syncthreads();
    }

    // ---- this wave's rows: o / l and (m, l) of the block --------------------------
    if (rok) {
        const int64_t pb = ((int64_t)bh * a.nblk + blk) * R;
        const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
        _Float16* orow = a.po + (pb + r) * D;
#pragma unroll
        for (int c = 0; c < DC; c++)
#pragma unroll
            for (int dt = 0; dt < 8; dt++) {
                const f32x4 v = O[c][dt] * inv;
                *(u32x2*)(orow + 128 * c + 16 * dt + 4 * jg) = u32x2{pack_f16(v[0], v[1]), pack_f16(v[2], v[3])};
            }
        if (jg == 0) a.pml[pb + r] = make_float2(m, lsum);
    }
}

// out[b, h, l, :] = sum_blk w_blk o_blk / sum_blk w_blk, w_blk = l_blk exp(m_blk - max m),
// with o_blk stored as o / l; 0 when no block saw a key (the reference kernel's rule).
// One wave per (b, hk, row r); blocks merged 32 at a time with online rescaling,
// each chunk's loads issued together.
template <int D>
__global__ __launch_bounds__(64) void kv8_combine(const _Float16* __restrict__ po,
                                                  const float2* __restrict__ pml, int nblk, int R,
                                                  int H, int Hk, int L, int qdt, void* __restrict__ out,
                                                  int64_t po_bytes, int64_t pml_bytes) {
    constexpr int PER = D / 64;          // d per lane (2, 4, 6 or 8)
    constexpr int W = PER / 2;           // 32-bit words per lane and block
    constexpr int CH = 32;               // blocks per chunk
    const int row = blockIdx.x;          // (b*Hk + hk) * R + r
    const int bh = row / R, r = row % R;
    const int lane = threadIdx.x;
    const __amdgpu_buffer_rsrc_t rp = make_rsrc(po, po_bytes);
    const __amdgpu_buffer_rsrc_t rml = make_rsrc(pml, pml_bytes);

    float M = -INFINITY, den = 0.f, num[PER];
#pragma unroll
    for (int e = 0; e < PER; e++) num[e] = 0.f;
    for (int i0 = 0; i0 < nblk; i0 += CH) {
        uint32_t ov[CH][W];
#pragma unroll
        for (int t = 0; t < CH; t++) {
            const uint32_t off = (uint32_t)((((int64_t)bh * nblk + i0 + t) * R + r) * D + lane * PER) * 2u;
            if constexpr (W == 1) {
                ov[t][0] = __builtin_amdgcn_raw_buffer_load_b32(rp, (int)off, 0, 0);
            } else if constexpr (W == 2) {
                const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rp, (int)off, 0, 0);
                ov[t][0] = v.x;
                ov[t][1] = v.y;
            } else if constexpr (W == 3) {
                const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rp, (int)off, 0, 0);
                ov[t][0] = v.x;
                ov[t][1] = v.y;
                ov[t][2] = __builtin_amdgcn_raw_buffer_load_b32(rp, (int)(off + 8u), 0, 0);
            } else {
                const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rp, (int)off, 0, 0);
#pragma unroll
                for (int e = 0; e < 4; e++) ov[t][e] = v[e];
            }
        }
        const int i = i0 + lane;
        const bool valid = lane < CH && i < nblk;
        const u32x2 mlr = __builtin_amdgcn_raw_buffer_load_b64(
            rml, (int)((uint32_t)(((int64_t)bh * nblk + (valid ? i : 0)) * R + r) * 8u), 0, 0);
        const float mi = valid ? __uint_as_float(mlr.x) : -INFINITY;
        const float li = valid ? __uint_as_float(mlr.y) : 0.f;
        const float Mn = fmaxf(M, wave_max(mi));
        if (Mn == -INFINITY) continue;               // nothing visible yet
        const float alpha = M == -INFINITY ? 0.f : __expf(M - Mn);
        den *= alpha;
#pragma unroll
        for (int e = 0; e < PER; e++) num[e] *= alpha;
        const float w = mi == -INFINITY ? 0.f : li * __expf(mi - Mn);
        den += w;
#pragma unroll
        for (int t = 0; t < CH; t++) {
            const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), t));
#pragma unroll
            for (int e = 0; e < W; e++) {
                const f16x2 hv = __builtin_bit_cast(f16x2, ov[t][e]);
                num[2 * e] += c * (float)hv[0];
                num[2 * e + 1] += c * (float)hv[1];
            }
        }
        M = Mn;
    }
    den = wave_add(den);
    const int b = bh / Hk, hk = bh % Hk;
    const int h = hk * (H / Hk) + r / L, lq = r % L;
    const int64_t oi = (((int64_t)b * H + h) * L + lq) * D + lane * PER;
    const float inv = den > 0.f ? 1.f / den : 0.f;
#pragma unroll
    for (int e = 0; e < PER; e++) {
        const float v = num[e] * inv;
        if (qdt == BF16) ((uint16_t*)out)[oi + e] = f32_to_bf16(v);
        else if (qdt == F16) ((uint16_t*)out)[oi + e] = f32_to_f16(v);
        else ((float*)out)[oi + e] = v;
    }
}

__global__ void fill_zero_u32(uint32_t* __restrict__ p, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

struct Kv8Plan {
    int keys_per_wg, nblk, rt;
    size_t po_bytes, pml_off, pml_bytes, total;
};

// Workgroups per call the key blocks aim at: 512 for kv8_partial (256 / 512
// / 1024 measured alike at 8k keys); for kv8_wide and kv8_rows one round of
// the chip -- 256 CUs times the workgroups a CU holds (2 up to D = 128 for
// kv8_wide, up to D = 256 for kv8_rows, else 1) -- kv8_wide's over the key
// blocks times its row tiles (at D = 512: 166 us at 512, 155 at 256).
constexpr int KV8_TARGET_WGS = 512;

// The key blocks of a call, aiming at `target` workgroups of `tiles` row
// tiles per key block.  Every plan has at most as many blocks as
// kv8_partial's (target 512, one tile), so the workspace that
// kmi_kv8_workspace_bytes sizes by the latter holds any of them.
static Kv8Plan plan_kv8(int B, int Hk, int N, int D, int R, int target = KV8_TARGET_WGS, int tiles = 1) {
    Kv8Plan p;
    p.rt = (R + 15) / 16;
    const int64_t pairs = (int64_t)B * Hk;
    const int64_t want_blk = ceil_div(target / tiles > 0 ? target / tiles : 1, pairs);
    int64_t kpw = ceil_div(N > 0 ? N : 1, want_blk);
    kpw = ceil_div(kpw, KV_WG_KEYS) * KV_WG_KEYS;
    p.keys_per_wg = (int)kpw;
    p.nblk = (int)ceil_div(N > 0 ? N : 1, kpw);
    const size_t rows = (size_t)pairs * p.nblk * R;
    p.po_bytes = rows * D * 2;
    p.pml_off = (p.po_bytes + 255) & ~(size_t)255;
    p.pml_bytes = rows * sizeof(float2);
    p.total = p.pml_off + p.pml_bytes;
    return p;
}

template <int D, int RT, class ST>
static void launch_partial(const Kv8Args& a, dim3 grid, hipStream_t st) {
    constexpr size_t lds = KvShape<D, RT>::lds;
    allow_dynamic_lds_once((const void*)kv8_partial<D, RT, ST>);
    kv8_partial<D, RT, ST><<<grid, 256, lds, st>>>(a);
}

template <class ST>
static void launch_partial_st(const Kv8Args& a, int D, int rt, dim3 grid, hipStream_t st) {
    if (D == 128) {
        if (rt == 1) launch_partial<128, 1, ST>(a, grid, st);
        else if (rt == 2) launch_partial<128, 2, ST>(a, grid, st);
        else if (rt == 3) launch_partial<128, 3, ST>(a, grid, st);
        else launch_partial<128, 4, ST>(a, grid, st);
    } else {
        launch_partial<256, 2, ST>(a, grid, st);   // 17-32 rows (partial_covers)
    }
}

template <int DC, class ST>
static void launch_wide_dc(const Kv8Args& a, int nrt, hipStream_t st) {
    constexpr size_t lds = kv8_wide_lds<DC>();
    allow_dynamic_lds_once((const void*)kv8_wide<DC, ST>);
    const dim3 grid((unsigned)(8 * nrt * ceil_div(a.nblk, 8)), (unsigned)(a.B * a.Hk));
    kv8_wide<DC, ST><<<grid, 256, lds, st>>>(a, nrt);
}

template <class ST>
static void launch_wide(const Kv8Args& a, int D, hipStream_t st) {
    const int nrt = (a.R + 15) / 16;
    if (D == 128) launch_wide_dc<1, ST>(a, nrt, st);
    else if (D == 256) launch_wide_dc<2, ST>(a, nrt, st);
    else if (D == 384) launch_wide_dc<3, ST>(a, nrt, st);
    else launch_wide_dc<4, ST>(a, nrt, st);
}

template <int DC, class ST>
static void launch_rows_dc(const Kv8Args& a, hipStream_t st) {
    constexpr size_t lds = 2 * kv8_rows_buf<DC>();
    allow_dynamic_lds_once((const void*)kv8_rows<DC, ST>);
    kv8_rows<DC, ST><<<dim3((unsigned)a.nblk, (unsigned)(a.B * a.Hk)), 256, lds, st>>>(a);
}

template <class ST>
static void launch_rows(const Kv8Args& a, int D, hipStream_t st) {
    if (D == 128) launch_rows_dc<1, ST>(a, st);
    else if (D == 256) launch_rows_dc<2, ST>(a, st);
    else if (D == 384) launch_rows_dc<3, ST>(a, st);
    else launch_rows_dc<4, ST>(a, st);
}

// kv8_partial holds all R rows' state of a wave in registers: D = 128 up to
// 64 rows, D = 256 up to 32, one group per D/4-wide lane run.  At D = 256
// it takes 17-32 rows only: with one row tile kv8_wide is faster (4 x 16
// heads, 32k keys, 4 rows: 90 vs 100 us; at 32 rows 86 vs 73).
static bool partial_covers(int D, int group, int R) {
    return (D == 128 || (D == 256 && R > 16 && R <= 32)) && group >= D / 4;
}

template <int D>
static void launch_combine(const Kv8Args& a, const Kv8Plan& p, int q_dtype, void* out, hipStream_t st) {
    kv8_combine<D><<<(unsigned)(a.B * a.Hk * a.R), 64, 0, st>>>(a.po, a.pml, p.nblk, a.R, a.H, a.Hk, a.L,
                                                                q_dtype, out, (int64_t)p.po_bytes,
                                                                (int64_t)p.pml_bytes);
}

}  // namespace kmi

using namespace kmi;

extern "C" {

size_t kmi_kv8_workspace_bytes(int B, int H, int Hk, int L, int N, int D) {
    if (B <= 0 || H <= 0 || Hk <= 0 || L <= 0 || N <= 0 || D <= 0 || H % Hk) return 0;
    const int R = (H / Hk) * L;
    return plan_kv8(B, Hk, N, D, R).total;
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
    KMI_CHECK_ARG(D > 0 && D % 128 == 0 && D <= 512, "kv8_decode: head dim %d not in {128, 256, 384, 512}", D);
    KMI_CHECK_ARG(group > 0 && group % 16 == 0 && D % group == 0,
                  "kv8_decode: group %d must divide D=%d and be a multiple of 16", group, D);
    KMI_CHECK_ARG(q_dtype >= BF16 && q_dtype <= F32 && scale_dtype >= BF16 && scale_dtype <= F32,
                  "kv8_decode: bad dtype");
    const int R = (H / Hk) * L;
    KMI_CHECK_ARG(R <= 64, "kv8_decode: %d query rows per KV head (at most 64)", R);
    KMI_CHECK_ARG(N >= 0, "kv8_decode: N=%d", N);
    hipStream_t st = (hipStream_t)stream;
    const int qes = q_dtype == F32 ? 4 : 2;
    if (N == 0) {   // no key: every row returns 0 (a fill kernel: graph-capture safe)
        const int64_t words = (int64_t)B * H * L * D * qes / 4;
        fill_zero_u32<<<(unsigned)ceil_div(words, 256), 256, 0, st>>>((uint32_t*)out, words);
        KMI_CHECK_LAUNCH("kv8_decode(empty)");
        return OK;
    }
    // kv8_partial where its registers hold the rows; else one row tile:
    // kv8_wide, more: kv8_rows
    const bool wide = !partial_covers(D, group, R);
    const bool rows = wide && R > 16;
    Kv8Plan p = !wide ? plan_kv8(B, Hk, N, D, R)
                : rows ? plan_kv8(B, Hk, N, D, R, D <= 256 ? 512 : 256)
                       : plan_kv8(B, Hk, N, D, R, D == 128 ? 512 : 256, (R + 15) / 16);
    if (!workspace || workspace_bytes < p.total) {
        set_error("kv8_decode: workspace of %zu bytes needed, %zu given", p.total, workspace_bytes);
        return EWORKSPACE;
    }
    // 32-bit buffer offsets: every byte offset the kernels form stays below 2^31
    const int64_t lim = (int64_t)1 << 31;
    const int sdes = scale_dtype == F32 ? 4 : 2;
    const int64_t keys_formed = (int64_t)p.nblk * p.keys_per_wg;
    Kv8Args a = {};
    const void* bases[6] = {kw, ks, kb, vw, vs, vb};
    for (int i = 0; i < 6; i++) {
        const int es = (i == 0 || i == 3) ? 4 : sdes;
        const int64_t row = (i == 0 || i == 3) ? D / 4 : D / group;
        for (int j = 0; j < 3; j++) {
            KMI_CHECK_ARG(strides[3 * i + j] >= 0, "kv8_decode: negative stride");
            a.st[i][j] = strides[3 * i + j];
        }
        a.base[i] = bases[i];
        a.ext[i] = ((int64_t)(N - 1) * a.st[i][2] + row) * es;
        KMI_CHECK_ARG((keys_formed * a.st[i][2] + row) * es < lim,
                      "kv8_decode: K/V rows span more than 2 GiB per head");
    }
    KMI_CHECK_ARG((int64_t)B * H * L * D * qes < lim, "kv8_decode: q larger than 2 GiB");
    KMI_CHECK_ARG((int64_t)B * L * (keys_formed + 1) < lim, "kv8_decode: mask larger than 2 GiB");
    KMI_CHECK_ARG((int64_t)p.po_bytes + (int64_t)B * Hk * p.nblk * R * 8 < lim,
                  "kv8_decode: partials larger than 2 GiB");
    a.q = q; a.mask = mask;
    a.po = (_Float16*)workspace;
    a.pml = (float2*)((char*)workspace + p.pml_off);
    a.qdt = q_dtype;
    a.B = B; a.H = H; a.Hk = Hk; a.L = L; a.N = N; a.group = group; a.R = R;
    a.causal = causal && L > 1; a.keys_per_wg = p.keys_per_wg; a.nblk = p.nblk; a.scale = scale;
    if (!wide) {
        dim3 grid((unsigned)p.nblk, (unsigned)(B * Hk));
        if (scale_dtype == BF16) launch_partial_st<TBF16>(a, D, p.rt, grid, st);
        else if (scale_dtype == F16) launch_partial_st<TF16>(a, D, p.rt, grid, st);
        else launch_partial_st<TF32>(a, D, p.rt, grid, st);
        KMI_CHECK_LAUNCH("kv8_partial");
    } else if (rows) {
        if (scale_dtype == BF16) launch_rows<TBF16>(a, D, st);
        else if (scale_dtype == F16) launch_rows<TF16>(a, D, st);
        else launch_rows<TF32>(a, D, st);
        KMI_CHECK_LAUNCH("kv8_rows");
    } else {
        if (scale_dtype == BF16) launch_wide<TBF16>(a, D, st);
        else if (scale_dtype == F16) launch_wide<TF16>(a, D, st);
        else launch_wide<TF32>(a, D, st);
        KMI_CHECK_LAUNCH("kv8_wide");
    }
    if (D == 128) launch_combine<128>(a, p, q_dtype, out, st);
    else if (D == 256) launch_combine<256>(a, p, q_dtype, out, st);
    else if (D == 384) launch_combine<384>(a, p, q_dtype, out, st);
    else launch_combine<512>(a, p, q_dtype, out, st);
    KMI_CHECK_LAUNCH("kv8_combine");
    return OK;
}

}  // extern "C"
