// VQ expert matmul over the bit-packed on-disk code layout, for gfx950.
// The VQ artifacts' routed experts store, per output row, the codebook
// indices of the row's dim-element vectors as ceil(log2 K)-bit fields
// packed into uint32 words, ceil(in/dim/32) * bits words per row
// (src/knurlogic/engine/families/deepseek/heads/deepseek_v4.py:36-44,
// 95-129; the shipped geometry is K = 2048 entries of dim 2-4 at 11 bits,
// tests/engine/test_deepseek_v4_mtp.py:206-233), with fp16 scales per group
// of `group` inputs:
//   What[o, i] = scales[o, i / group] * codebook[code(o, i / dim)][i % dim]
//   y[r, o]    = x[rows[r]] . What_{experts[r]}[o]
// Field j of a row occupies bits [j*PB, j*PB + PB) of the row's words read
// as one little-endian bit stream (LSB first), so each run of 32 fields is
// exactly PB whole words.
//
// One lane decodes one 32-field block at a time: it loads the block's PB
// words, extracts the fields with funnel shifts at compile-time offsets,
// gathers each field's codebook vector from LDS (fp16, the whole codebook
// staged per workgroup) and dots it with the matching x values (staged in
// LDS as fp16, read by every row at the same address) by v_dot2_f32_f16.
// SEG lanes share a row and take its blocks round-robin; their partial
// sums meet by cross-lane shuffles.  Scale groups are summed in fp32 and
// scaled once per group.  With two row sets (gate and up) the epilogue is
// Qwen3.5's _SwiGLU with its roundings.
#include "common.hpp"
#include "qgemv.hpp"
#include "vq_packed_mfma.hpp"
#include "pair_tiles.hpp"
#include "route.hpp"
#include "../../include/knurlogic_amd.h"


namespace kmi {

typedef _Float16 vp_f16x2 __attribute__((ext_vector_type(2)));

struct VpArgs {
    const uint16_t* x;          // bf16 [X, K]
    int64_t X;
    const int32_t* rows;        // [R] x row of each output row set, or null: x row r / rows_div
    int64_t rows_div;
    const int32_t* experts;     // [R] expert of each
    int64_t R;
    const uint32_t* codes[2];   // [E, N, W] packed fields (set 1: the up rows, GLU only)
    const uint16_t* sc[2];      // [E, N, K / group] fp16
    const uint16_t* cb[2];      // [kc, dim] fp16
    int nset;
    int kc;
    int64_t E, N, K, W;         // W: words per row
    int group;
    uint16_t* y;                // [R, N] bf16
    // In-kernel routing (gate/up over one token's pairs, rows_div = k): each
    // workgroup routes its pair's token from logits [X, E] bf16 (route.hpp,
    // E <= 256) in place of reading experts; column block 0 writes the
    // pair's expert and score.
    const uint16_t* logits;
    int32_t* inds_out;
    uint16_t* scores_out;
    int k;
};

__device__ __forceinline__ float vp_dot2(uint32_t a, uint32_t b, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(vp_f16x2, a), __builtin_bit_cast(vp_f16x2, b), acc, false);
}

template <int DIM>
__device__ __forceinline__ float vp_dot(const uint16_t* cbe, const uint16_t* xe, float acc) {
    if constexpr (DIM == 2) {
        return vp_dot2(*(const uint32_t*)cbe, *(const uint32_t*)xe, acc);
    } else if constexpr (DIM == 4) {
        const u32x2 c = *(const u32x2*)cbe, v = *(const u32x2*)xe;
        return vp_dot2(c.y, v.y, vp_dot2(c.x, v.x, acc));
    } else {
        const u32x4 c = *(const u32x4*)cbe, v = *(const u32x4*)xe;
        acc = vp_dot2(c.x, v.x, acc);
        acc = vp_dot2(c.y, v.y, acc);
        acc = vp_dot2(c.z, v.z, acc);
        return vp_dot2(c.w, v.w, acc);
    }
}

// 1 KB LDS blocks holding a codebook of kc entries of DIM fp16
__host__ __device__ inline int vp_cb_blocks(int kc, int dim) { return (kc * dim * 2 + 1023) / 1024; }

// One direct-to-LDS load: lane i's 16 bytes at `voff` land at lds + 16 i
// (a device function: the builtin inside a kernel template's lambda stops
// hipcc emitting the host launch stubs).
__device__ __forceinline__ void vp_dma16(__amdgpu_buffer_rsrc_t r, unsigned char* lds, uint32_t voff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, 0, 0, 0);
}

// field j (0..31) of a block of PB words
template <int PB>
__device__ __forceinline__ uint32_t vp_field(const uint32_t* w, int j) {
    const int off = j * PB, q = off >> 5, sh = off & 31;
    uint32_t v;
    if (sh + PB <= 32) v = w[q] >> sh;
    else v = __builtin_amdgcn_alignbit(w[q + 1], w[q], (uint32_t)sh);
    return v & ((1u << PB) - 1u);
}

// A full 32-field block: fields decoded, codebook vectors and x read from
// LDS in batches of 8 -- the next batch's reads issued before the current
// batch's dot products (the scheduling barriers keep them there) -- and
// each group's sum formed in field order, as vp_dot field by field.
template <int DIM>
struct VpVec;
template <> struct VpVec<2> { typedef uint32_t T; };
template <> struct VpVec<4> { typedef u32x2 T; };
template <> struct VpVec<8> { typedef u32x4 T; };

template <int DIM>
__device__ __forceinline__ float vp_dotv(typename VpVec<DIM>::T c, typename VpVec<DIM>::T v, float acc) {
    if constexpr (DIM == 2) {
        return vp_dot2(c, v, acc);
    } else if constexpr (DIM == 4) {
        return vp_dot2(c.y, v.y, vp_dot2(c.x, v.x, acc));
    } else {
        acc = vp_dot2(c.x, v.x, acc);
        acc = vp_dot2(c.y, v.y, acc);
        acc = vp_dot2(c.z, v.z, acc);
        return vp_dot2(c.w, v.w, acc);
    }
}

template <int PB, int DIM, int GPB>
__device__ __forceinline__ void vp_block_full(const uint32_t (&w)[PB + 1], const uint16_t* cbl, const uint16_t* xb,
                                              uint32_t kcm1, float (&acc)[GPB]) {
    typedef typename VpVec<DIM>::T V;
    constexpr int FB = 8, FPG = 32 / GPB;
    V cv[2][FB], xv[2][FB];
    auto fetch = [&](int j0, int b) {
#pragma unroll
        for (int f = 0; f < FB; f++) {
            const int j = j0 + f;
            const uint32_t c = __builtin_elementwise_min(vp_field<PB>(w, j), kcm1);
            cv[b][f] = *(const V*)(cbl + c * DIM);
            xv[b][f] = *(const V*)(xb + j * DIM);
        }
    };
    fetch(0, 0);
#pragma unroll
    for (int j0 = 0; j0 < 32; j0 += FB) {
        const int b = (j0 / FB) & 1;
        if (j0 + FB < 32) fetch(j0 + FB, b ^ 1);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int f = 0; f < FB; f++) acc[(j0 + f) / FPG] = vp_dotv<DIM>(cv[b][f], xv[b][f], acc[(j0 + f) / FPG]);
        __builtin_amdgcn_sched_barrier(0);
    }
}

__device__ __forceinline__ float vp_bf16r(float v) { return bf16_to_f32(f32_to_bf16(v)); }

__device__ __forceinline__ float vp_f32_kept(double v) {
    float f = (float)v;
    asm volatile("" : "+v"(f));
    return f;
}

// PB bits per field, DIM elements per code vector, GPB scale groups per
// 32-field block (1: a block lies inside one group), SEG lanes per row.
template <int PB, int DIM, int GPB, int SEG>
__global__ __launch_bounds__(256) void vq_packed_gemv(VpArgs a) {
    constexpr int RPWG = 256 / SEG;
    constexpr int FPG = 32 / GPB;                    // fields per group within a block (GPB > 1)
    extern __shared__ __align__(16) unsigned char smem[];
    const int tid = threadIdx.x;
    const int64_t r = blockIdx.y;
    const bool route = a.logits != nullptr;
    int e = route ? 0 : a.experts[r];
    float rlog[1];
    if (route) route_load<TBF16, 1>(a.logits + (r / a.k) * a.E, (int)a.E, rlog);
    const int64_t xrow = a.rows ? (int64_t)a.rows[r] : r / a.rows_div;
    const bool ok_x = xrow >= 0 && xrow < a.X;
    const bool two_cb = a.nset == 2 && a.cb[1] != a.cb[0];
    const int64_t nsub = a.K / DIM;                  // fields per row
    const int64_t Kp = (nsub + 31) / 32 * 32 * DIM;  // x staged to whole blocks (zeros past K)
    // x in LDS: block b's 32 vectors at b * XBS elements, one vector of
    // padding per block, so the lanes of a row (one block each) read
    // different banks (a block is a multiple of 256 bytes otherwise)
    constexpr int XBS = 33 * DIM;
    const int cbytes = a.kc * DIM * 2;               // bytes of one codebook
    const int cbb = vp_cb_blocks(a.kc, DIM);         // its 1 KB LDS blocks
    uint16_t* cbl0 = (uint16_t*)smem;
    uint16_t* cbl1 = two_cb ? (uint16_t*)(smem + (size_t)cbb * 1024) : cbl0;
    uint16_t* xl = (uint16_t*)(smem + (size_t)cbb * 1024 * (two_cb ? 2 : 1));

    // codebook(s) and the x row (fp16) -> LDS, every load issued before any
    // wait: codebooks of whole 16-byte pieces by direct-to-LDS loads (1 KB per
    // wave instruction, nothing through registers), others by dword copies;
    // x in batches of 8 dwords per thread
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int ncb = two_cb ? 2 : 1;
    if (cbytes % 16 == 0) {
        for (int j = wave; j < cbb * ncb; j += 4) {
            const int s = j >= cbb, p = (j - s * cbb) * 64 + lane;
            vp_dma16(make_rsrc(a.cb[s], cbytes), smem + (size_t)j * 1024,
                     p * 16 < cbytes ? (uint32_t)p * 16u : 0x80000000u);
        }
    } else {
        for (int s = 0; s < ncb; s++) {
            uint16_t* dst = s ? cbl1 : cbl0;
            const __amdgpu_buffer_rsrc_t rcb = make_rsrc(a.cb[s], cbytes);
            for (int i = tid; i < cbytes / 4; i += 256)
                *(uint32_t*)(dst + 2 * i) = __builtin_amdgcn_raw_buffer_load_b32(rcb, i * 4, 0, 0);
        }
    }
    {
        const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x + (ok_x ? xrow : 0) * a.K, ok_x ? a.K * 2 : 0);
        const int nd = (int)(Kp / 2);
        for (int i0 = tid; i0 < nd; i0 += 256 * 8) {
            uint32_t v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int i = i0 + 256 * u;
                v[u] = __builtin_amdgcn_raw_buffer_load_b32(rx, i < nd ? i * 4 : (int)0x80000000u, 0, 0);
            }
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int i = i0 + 256 * u;
                if (i < nd) {
                    const vp_f16x2 h = {(_Float16)bf16_to_f32((uint16_t)(v[u] & 0xffffu)),
                                        (_Float16)bf16_to_f32((uint16_t)(v[u] >> 16))};
                    const int e = 2 * i, blk = e / (32 * DIM);
                    *(uint32_t*)(xl + blk * XBS + (e - blk * 32 * DIM)) = __builtin_bit_cast(uint32_t, h);
                }
            }
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the direct-to-LDS writes have landed
    __syncthreads();
    // past the codebooks and x (16-byte aligned): the router's state when
    // routing (the host sizes the LDS for it only then)
    unsigned char* extra = smem + (((size_t)cbb * 1024 * (two_cb ? 2 : 1) + (size_t)((nsub + 31) / 32) * XBS * 2 + 15) &
                                   ~(size_t)15);
    if (route) {     // once the codebook and x are staged (uniform branch: every thread routes)
        RouteLdsT<ROUTE_THREADS>& rsm = *(RouteLdsT<ROUTE_THREADS>*)extra;
        route_from<TBF16, 1>(rlog, (int)a.E, a.k, rsm);
        const int s = (int)(r % a.k);
        e = __builtin_amdgcn_readfirstlane(rsm.sel_e[s]);
        if (blockIdx.x == 0 && tid == 0) {
            a.inds_out[r] = e;
            a.scores_out[r] = f32_to_bf16(rsm.sel_p[s]);
        }
    }
    const bool ok_e = e >= 0 && e < a.E;

    const int64_t row = (int64_t)blockIdx.x * RPWG + tid / SEG;
    const int seg = tid % SEG;
    const int64_t nblk = (nsub + 31) / 32;
    const int64_t gpr = a.K / a.group;                // scale groups per row
    const int64_t fpg = a.group / DIM;                // fields per group
    // the expert's views are workgroup-uniform (a per-lane descriptor would
    // put every load in a loop over the wave's distinct rows); the row is in
    // the lane's offset, and a row past N reads 0
    const int64_t ebase = (int64_t)(ok_e ? e : 0) * a.N;
    const bool row_ok = ok_e && row < a.N;
    const uint32_t rowc = (uint32_t)(row < a.N ? row : 0);
    float res[2] = {0.f, 0.f};
    for (int s = 0; s < a.nset; s++) {
        const uint16_t* cbl = s ? cbl1 : cbl0;
        const __amdgpu_buffer_rsrc_t rc = make_rsrc(a.codes[s] + ebase * a.W, ok_e ? a.N * a.W * 4 : 0);
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.sc[s] + ebase * gpr, ok_e ? a.N * gpr * 2 : 0);
        const uint32_t cro = rowc * (uint32_t)a.W * 4u, sro = rowc * (uint32_t)gpr * 2u;
        float tot = 0.f;
        for (int b = seg; b < (int)nblk; b += SEG) {
            uint32_t w[PB + 1];
#pragma unroll
            for (int q = 0; q < PB; q++)
                w[q] = __builtin_amdgcn_raw_buffer_load_b32(
                    rc, row_ok ? (int)(cro + (uint32_t)(b * PB + q) * 4u) : (int)0x80000000u, 0, AUX_NT);
            w[PB] = 0;
            float sv[GPB];
#pragma unroll
            for (int g = 0; g < GPB; g++) {
                const int gi = (int)((b * 32 + g * FPG) / fpg);
                sv[g] = f16_to_f32(__builtin_amdgcn_raw_buffer_load_b16(
                    rs, row_ok ? (int)(sro + (uint32_t)gi * 2u) : (int)0x80000000u, 0, 0));
            }
            const int64_t f0 = b * 32;
            const int nvalid = (int)(nsub - f0 < 32 ? nsub - f0 : 32);
            const uint16_t* xb = xl + b * XBS;
            float acc[GPB];
#pragma unroll
            for (int g = 0; g < GPB; g++) acc[g] = 0.f;
            if (nvalid == 32) {
                vp_block_full<PB, DIM, GPB>(w, cbl, xb, (uint32_t)(a.kc - 1), acc);
            } else {                 // the last, partial block of a row
#pragma unroll
                for (int j = 0; j < 32; j++) {
                    uint32_t c = vp_field<PB>(w, j);
                    c = __builtin_elementwise_min(c, (uint32_t)(a.kc - 1));
                    const float d = vp_dot<DIM>(cbl + c * DIM, xb + j * DIM, 0.f);
                    acc[j / FPG] += j < nvalid ? d : 0.f;
                }
            }
#pragma unroll
            for (int g = 0; g < GPB; g++) tot = __builtin_fmaf(sv[g], acc[g], tot);
        }
#pragma unroll
        for (int o = SEG / 2; o >= 1; o >>= 1) tot += __shfl_xor(tot, o, 64);
        res[s] = vp_bf16r(tot);
    }
    if (seg == 0 && row < a.N) {
        float out = res[0];
        if (a.nset == 2) {           // round(round(silu_f32(gate)) * up)
            out = silu_bf16r(res[0]) * res[1];
        }
        a.y[r * a.N + row] = (ok_e && ok_x) ? f32_to_bf16(out) : (uint16_t)0;
    }
}

// Lanes per row: the blocks of a row rounded down to a power of two, at
// most 16 (fewer lanes per row, each with more blocks, measured slower: a
// lane's blocks are a serial chain of loads and codebook gathers).
static int vp_seg(int64_t nblk) {
    int s = 1;
    while (s < 16 && s * 2 <= nblk) s *= 2;
    return s;
}

template <int PB, int DIM, int GPB>
static int launch_vp3(const VpArgs& a, int seg, size_t lds, hipStream_t st) {
#define KMI_VP_SEG(S_)                                                                                  \
    if (seg == S_) {                                                                                    \
        allow_dynamic_lds_once((const void*)vq_packed_gemv<PB, DIM, GPB, S_>);                   \
        const dim3 grid((unsigned)ceil_div(a.N, 256 / S_), (unsigned)a.R);                              \
        vq_packed_gemv<PB, DIM, GPB, S_><<<grid, 256, lds, st>>>(a);                                    \
        return OK;                                                                                      \
    }
    KMI_VP_SEG(1) KMI_VP_SEG(2) KMI_VP_SEG(4) KMI_VP_SEG(8) KMI_VP_SEG(16)
#undef KMI_VP_SEG
    return EINVAL_ARG;
}

template <int PB>
static int launch_vp_pb(const VpArgs& a, int dim, int gpb, int seg, size_t lds, hipStream_t st) {
    if (dim == 2 && gpb == 1) return launch_vp3<PB, 2, 1>(a, seg, lds, st);
    if (dim == 2 && gpb == 2) return launch_vp3<PB, 2, 2>(a, seg, lds, st);
    if (dim == 4 && gpb == 1) return launch_vp3<PB, 4, 1>(a, seg, lds, st);
    if (dim == 4 && gpb == 2) return launch_vp3<PB, 4, 2>(a, seg, lds, st);
    if (dim == 4 && gpb == 4) return launch_vp3<PB, 4, 4>(a, seg, lds, st);
    if (dim == 8 && gpb == 2) return launch_vp3<PB, 8, 2>(a, seg, lds, st);
    if (dim == 8 && gpb == 4) return launch_vp3<PB, 8, 4>(a, seg, lds, st);
    if (dim == 8 && gpb == 8) return launch_vp3<PB, 8, 8>(a, seg, lds, st);
    if (dim == 8 && gpb == 1) return launch_vp3<PB, 8, 1>(a, seg, lds, st);
    return EINVAL_ARG;
}

// ---- down projection + weighted combine for a few tokens, token-major ----
// grid (ceil(N / rows per workgroup), T).  A workgroup owns a few output
// rows of one token; lane (slot s, row r, segment g), SEG lanes per (row,
// slot) as vq_packed_gemv puts them on a row (same blocks per lane, same
// sums, same shuffle tree), so y[t*k+s, n] is the per-pair kernel's value
// bit for bit; the token's k act rows are staged once.  Each slot's
// round(y * score) meets in LDS and lane r sums them in slot order in
// float64, rounded once: out[t, n], as moe_combine gives from those y.
struct VpdArgs {
    const uint16_t* act;        // [T*k, K] bf16 (pair-major)
    const int32_t* inds;        // [T*k] expert per pair
    const uint16_t* scores;     // [T*k] bf16
    const uint32_t* codes;      // [E, N, W]
    const uint16_t* sc;         // [E, N, K / group]
    const uint16_t* cb;         // [kc, dim]
    uint16_t* out;              // [T, N] bf16
    int64_t E, N, K, W, T;
    int k, kc, group, seg;
};

constexpr int VPD_SLOTS = 8;    // slots per token (k <= 8)

template <int PB, int DIM, int GPB>
__global__ __launch_bounds__(256) void vq_packed_down_tok(VpdArgs a) {
    constexpr int FPG = 32 / GPB;
    constexpr int XBS = 33 * DIM;                    // x block stride (elements), as vq_packed_gemv
    extern __shared__ __align__(16) unsigned char smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int SEG = a.seg, rpwg = 256 / (VPD_SLOTS * SEG);
    // rows fastest after the segments: a wave's lanes cover consecutive rows
    // of one or two slots' experts (their words lie together)
    const int g = tid % SEG, r = (tid / SEG) % rpwg, s = tid / (SEG * rpwg);
    const int64_t t = blockIdx.y;
    const int k = a.k;
    const int64_t nsub = a.K / DIM, nblk = (nsub + 31) / 32;
    const int64_t Kp = nblk * 32 * DIM;
    const int cbytes = a.kc * DIM * 2, cbb = vp_cb_blocks(a.kc, DIM);
    uint16_t* cbl = (uint16_t*)smem;
    uint16_t* xl = (uint16_t*)(smem + (size_t)cbb * 1024);                    // [k][nblk * XBS]
    float* prod = (float*)(smem + (size_t)cbb * 1024 + (size_t)k * nblk * XBS * 2);   // [rpwg][8]

    // codebook (direct-to-LDS when whole 16-byte pieces) and the k act rows (fp16)
    if (cbytes % 16 == 0) {
        for (int j = wave; j < cbb; j += 4) {
            const int p = j * 64 + lane;
            vp_dma16(make_rsrc(a.cb, cbytes), smem + (size_t)j * 1024, p * 16 < cbytes ? (uint32_t)p * 16u : 0x80000000u);
        }
    } else {
        const __amdgpu_buffer_rsrc_t rcb = make_rsrc(a.cb, cbytes);
        for (int i = tid; i < cbytes / 4; i += 256)
            *(uint32_t*)(cbl + 2 * i) = __builtin_amdgcn_raw_buffer_load_b32(rcb, i * 4, 0, 0);
    }
    {
        const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.act + t * k * a.K, (int64_t)k * a.K * 2);
        const int nd = (int)(Kp / 2);                 // dwords per staged row
        const int total = k * nd;
        for (int i0 = tid; i0 < total; i0 += 256 * 8) {
            uint32_t v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int i = i0 + 256 * u, j = i / nd, d = i - j * nd;
                v[u] = __builtin_amdgcn_raw_buffer_load_b32(
                    rx, i < total && 2 * d < a.K ? (int)((j * a.K + 2 * d) * 2) : (int)0x80000000u, 0, 0);
            }
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int i = i0 + 256 * u;
                if (i < total) {
                    const int j = i / nd, d = i - j * nd;
                    const vp_f16x2 h = {(_Float16)bf16_to_f32((uint16_t)(v[u] & 0xffffu)),
                                        (_Float16)bf16_to_f32((uint16_t)(v[u] >> 16))};
                    const int e = 2 * d, blk = e / (32 * DIM);
                    *(uint32_t*)(xl + (size_t)j * nblk * XBS + blk * XBS + (e - blk * 32 * DIM)) =
                        __builtin_bit_cast(uint32_t, h);
                }
            }
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the direct-to-LDS writes have landed
    __syncthreads();

    const int64_t row = (int64_t)blockIdx.x * rpwg + r;
    const bool slot_ok = s < k;
    const int e = slot_ok ? a.inds[t * k + s] : -1;
    const bool ok_e = e >= 0 && e < a.E;
    const int64_t gpr = a.K / a.group, fpg = a.group / DIM;
    const bool row_ok = ok_e && row < a.N;
    // one view of all experts (a wave's lanes hold several slots, and a
    // per-lane view would put every load in a loop over the wave's distinct
    // views): the expert and row in the lane's 32-bit offset (the host keeps
    // the codes under 2 GiB)
    const __amdgpu_buffer_rsrc_t rc = make_rsrc(a.codes, a.E * a.N * a.W * 4);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.sc, a.E * a.N * gpr * 2);
    const uint32_t erow = (uint32_t)((ok_e ? e : 0) * a.N + (row < a.N ? row : 0));
    const uint32_t cro = erow * (uint32_t)a.W * 4u, sro = erow * (uint32_t)gpr * 2u;
    const uint16_t* xs = xl + (size_t)(slot_ok ? s : 0) * nblk * XBS;
    float tot = 0.f;
    for (int b = g; b < (int)nblk; b += SEG) {
        uint32_t w[PB + 1];
#pragma unroll
        for (int q = 0; q < PB; q++)
            w[q] = __builtin_amdgcn_raw_buffer_load_b32(
                rc, row_ok ? (int)(cro + (uint32_t)(b * PB + q) * 4u) : (int)0x80000000u, 0, AUX_NT);
        w[PB] = 0;
        float sv[GPB];
#pragma unroll
        for (int gg = 0; gg < GPB; gg++) {
            const int gi = (int)((b * 32 + gg * FPG) / fpg);
            sv[gg] = f16_to_f32(__builtin_amdgcn_raw_buffer_load_b16(
                rs, row_ok ? (int)(sro + (uint32_t)gi * 2u) : (int)0x80000000u, 0, 0));
        }
        const int64_t f0 = b * 32;
        const int nvalid = (int)(nsub - f0 < 32 ? nsub - f0 : 32);
        const uint16_t* xb = xs + b * XBS;
        float acc[GPB];
#pragma unroll
        for (int gg = 0; gg < GPB; gg++) acc[gg] = 0.f;
        if (nvalid == 32) {
            vp_block_full<PB, DIM, GPB>(w, cbl, xb, (uint32_t)(a.kc - 1), acc);
        } else {
#pragma unroll
            for (int j = 0; j < 32; j++) {
                uint32_t c = vp_field<PB>(w, j);
                c = __builtin_elementwise_min(c, (uint32_t)(a.kc - 1));
                const float d = vp_dot<DIM>(cbl + c * DIM, xb + j * DIM, 0.f);
                acc[j / FPG] += j < nvalid ? d : 0.f;
            }
        }
#pragma unroll
        for (int gg = 0; gg < GPB; gg++) tot = __builtin_fmaf(sv[gg], acc[gg], tot);
    }
    for (int o = SEG / 2; o >= 1; o >>= 1) tot += __shfl_xor(tot, o, 64);
    const float y = ok_e ? vp_bf16r(tot) : 0.f;
    if (g == 0 && slot_ok) prod[r * VPD_SLOTS + s] = vp_bf16r(y * bf16_to_f32(a.scores[t * k + s]));
    __syncthreads();
    if (tid < rpwg) {
        const int64_t n = (int64_t)blockIdx.x * rpwg + tid;
        if (n < a.N) {
            double acc = 0.0;
            for (int j = 0; j < k; j++) acc += (double)prod[tid * VPD_SLOTS + j];
            a.out[t * a.N + n] = f32_to_bf16(vp_f32_kept(acc));
        }
    }
}

static size_t vpd_lds(int64_t K, int kc, int dim, int k) {
    const int64_t nblk = (K / dim + 31) / 32;
    return (size_t)vp_cb_blocks(kc, dim) * 1024 + (size_t)k * nblk * 33 * dim * 2 + 256 * sizeof(float);
}

template <int PB>
static int launch_vpd_pb(const VpdArgs& a, int dim, int gpb, size_t lds, hipStream_t st) {
    const int rpwg = 256 / (VPD_SLOTS * a.seg);
    const dim3 grid((unsigned)ceil_div(a.N, rpwg), (unsigned)a.T);
#define KMI_VPD(D_, G_)                                                         \
    if (dim == D_ && gpb == G_) {                                               \
        allow_dynamic_lds_once((const void*)vq_packed_down_tok<PB, D_, G_>);                     \
        vq_packed_down_tok<PB, D_, G_><<<grid, 256, lds, st>>>(a);              \
        return OK;                                                              \
    }
    KMI_VPD(2, 1) KMI_VPD(2, 2) KMI_VPD(4, 1) KMI_VPD(4, 2) KMI_VPD(4, 4)
    KMI_VPD(8, 1) KMI_VPD(8, 2) KMI_VPD(8, 4) KMI_VPD(8, 8)
#undef KMI_VPD
    return EINVAL_ARG;
}

// Token-major down + combine for a few tokens (k <= 8, the LDS holding the
// codebook and the token's k act rows): 0 launched, 1 not covered.
static int run_vpd(VpdArgs& a, int pack_bits, int dim, hipStream_t st) {
    const int64_t nsub = a.K / dim, nblk = (nsub + 31) / 32;
    const int fpg = a.group / dim;
    const int gpb = fpg >= 32 ? 1 : 32 / fpg;
    a.seg = vp_seg(nblk);                     // the per-pair kernel's lanes per row
    const size_t lds = vpd_lds(a.K, a.kc, dim, a.k);
    if (a.k < 1 || a.k > VPD_SLOTS || VPD_SLOTS * a.seg > 256 || lds > 160 * 1024) return 1;
    int rc;
    switch (pack_bits) {
        case 8: rc = launch_vpd_pb<8>(a, dim, gpb, lds, st); break;
        case 9: rc = launch_vpd_pb<9>(a, dim, gpb, lds, st); break;
        case 10: rc = launch_vpd_pb<10>(a, dim, gpb, lds, st); break;
        case 11: rc = launch_vpd_pb<11>(a, dim, gpb, lds, st); break;
        case 12: rc = launch_vpd_pb<12>(a, dim, gpb, lds, st); break;
        default: rc = launch_vpd_pb<16>(a, dim, gpb, lds, st); break;
    }
    return rc == OK ? 0 : 1;
}

static int vp_check(int dtype, int pack_bits, int kc, int dim, int group, int64_t K, int64_t N, int64_t E) {
    KMI_CHECK_ARG(dtype == BF16, "vq (packed): only bfloat16 activations are implemented");
    KMI_CHECK_ARG(pack_bits == 8 || pack_bits == 9 || pack_bits == 10 || pack_bits == 11 || pack_bits == 12 ||
                      pack_bits == 16,
                  "vq (packed): %d-bit fields (8-12 and 16 are implemented)", pack_bits);
    KMI_CHECK_ARG(dim == 2 || dim == 4 || dim == 8, "vq (packed): vector length %d (2, 4, 8)", dim);
    KMI_CHECK_ARG(kc >= 1 && kc <= (1 << pack_bits), "vq (packed): %d codebook entries for %d-bit fields", kc,
                  pack_bits);
    KMI_CHECK_ARG(K > 0 && N > 0 && E > 0 && K % dim == 0, "vq (packed): K=%lld is not a multiple of dim %d",
                  (long long)K, dim);
    KMI_CHECK_ARG(group > 0 && K % group == 0 && group % dim == 0,
                  "vq (packed): scale group %d must divide K=%lld and be a multiple of dim %d", group,
                  (long long)K, dim);
    const int fpg = group / dim;
    KMI_CHECK_ARG((fpg & (fpg - 1)) == 0 && group >= 32,
                  "vq (packed): scale group %d (at least 32 inputs, a power of two fields) is not implemented",
                  group);
    const int64_t W = (K / dim + 31) / 32 * pack_bits;
    KMI_CHECK_ARG(E * N * W * 4 < (1LL << 31) &&
                      (size_t)vp_cb_blocks(kc, dim) * 1024 * 2 + (size_t)(W / pack_bits) * 33 * dim * 2 <= 160 * 1024,
                  "vq (packed): codes past 2 GiB or codebook + x past the LDS");
    return OK;
}

// LDS of vq_packed_gemv: the codebook(s) and x, then (16-byte aligned) the
// router's state when it routes
static size_t vp_lds(int64_t K, int kc, int dim, bool two_cb, bool route) {
    const int64_t nblk = (K / dim + 31) / 32;
    size_t b = (size_t)vp_cb_blocks(kc, dim) * 1024 * (two_cb ? 2 : 1) + (size_t)nblk * 33 * dim * 2;
    if (route) b = ((b + 15) & ~(size_t)15) + sizeof(RouteLdsT<ROUTE_THREADS>);
    return b;
}

static int run_vp(VpArgs& a, int pack_bits, int dim, hipStream_t st) {
    const int64_t nsub = a.K / dim, nblk = (nsub + 31) / 32;
    const int fpg = a.group / dim;
    const int gpb = fpg >= 32 ? 1 : 32 / fpg;
    const int seg = vp_seg(nblk);
    const bool two_cb = a.nset == 2 && a.cb[1] != a.cb[0];
    const size_t lds = vp_lds(a.K, a.kc, dim, two_cb, a.logits != nullptr);
    if (lds > 160 * 1024) {
        set_error("vq (packed): %zu bytes of LDS", lds);
        return EINVAL_ARG;
    }
    int rc;
    switch (pack_bits) {
        case 8: rc = launch_vp_pb<8>(a, dim, gpb, seg, lds, st); break;
        case 9: rc = launch_vp_pb<9>(a, dim, gpb, seg, lds, st); break;
        case 10: rc = launch_vp_pb<10>(a, dim, gpb, seg, lds, st); break;
        case 11: rc = launch_vp_pb<11>(a, dim, gpb, seg, lds, st); break;
        case 12: rc = launch_vp_pb<12>(a, dim, gpb, seg, lds, st); break;
        default: rc = launch_vp_pb<16>(a, dim, gpb, seg, lds, st); break;
    }
    if (rc) {
        set_error("vq (packed): no kernel for %d-bit fields, dim %d, %d groups per block", pack_bits, dim, gpb);
        return rc;
    }
    KMI_CHECK_LAUNCH("vq_packed_gemv");
    return OK;
}

}  // namespace kmi

using namespace kmi;

extern "C" {

int kmi_vq_packed_gather_qmm(const void* x, int64_t X, int64_t K, const uint32_t* codes, int pack_bits,
                             const void* codebook, int kc, int dim, const void* scales, int group, int64_t E,
                             int64_t N, const int32_t* rows, int64_t rows_div, const int32_t* experts, int64_t R,
                             int dtype, void* y, void* stream) {
    clear_error();
    int rc = vp_check(dtype, pack_bits, kc, dim, group, K, N, E);
    if (rc) return rc;
    KMI_CHECK_ARG(R >= 0 && X >= 1 && R < 65536, "vq_packed_gather_qmm: %lld output rows (at most 65535)",
                  (long long)R);
    if (R == 0) return OK;
    KMI_CHECK_ARG(x && codes && codebook && scales && experts && y && (rows || rows_div >= 1),
                  "vq_packed_gather_qmm: null pointer");
    VpArgs a = {};
    a.x = (const uint16_t*)x; a.X = X; a.rows = rows; a.rows_div = rows_div; a.experts = experts; a.R = R;
    a.codes[0] = a.codes[1] = codes;
    a.sc[0] = a.sc[1] = (const uint16_t*)scales;
    a.cb[0] = a.cb[1] = (const uint16_t*)codebook;
    a.nset = 1; a.kc = kc; a.E = E; a.N = N; a.K = K; a.W = (K / dim + 31) / 32 * pack_bits; a.group = group;
    a.y = (uint16_t*)y;
    return run_vp(a, pack_bits, dim, (hipStream_t)stream);
}

int kmi_vq_packed_glu(const void* x, int64_t X, int64_t H, int64_t I, const uint32_t* codes_gate,
                      const void* scales_gate, const void* codebook_gate, const uint32_t* codes_up,
                      const void* scales_up, const void* codebook_up, int pack_bits, int kc, int dim, int group,
                      int64_t E, const int32_t* rows, int64_t rows_div, const int32_t* experts, int64_t R,
                      int dtype, void* act, void* stream) {
    clear_error();
    int rc = vp_check(dtype, pack_bits, kc, dim, group, H, I, E);
    if (rc) return rc;
    KMI_CHECK_ARG(R >= 0 && X >= 1 && R < 65536, "vq_packed_glu: %lld output rows (at most 65535)", (long long)R);
    if (R == 0) return OK;
    KMI_CHECK_ARG(x && codes_gate && scales_gate && codebook_gate && codes_up && scales_up && codebook_up &&
                      experts && act && (rows || rows_div >= 1),
                  "vq_packed_glu: null pointer");
    VpArgs a = {};
    a.x = (const uint16_t*)x; a.X = X; a.rows = rows; a.rows_div = rows_div; a.experts = experts; a.R = R;
    a.codes[0] = codes_gate; a.codes[1] = codes_up;
    a.sc[0] = (const uint16_t*)scales_gate; a.sc[1] = (const uint16_t*)scales_up;
    a.cb[0] = (const uint16_t*)codebook_gate; a.cb[1] = (const uint16_t*)codebook_up;
    a.nset = 2; a.kc = kc; a.E = E; a.N = I; a.K = H; a.W = (H / dim + 31) / 32 * pack_bits; a.group = group;
    a.y = (uint16_t*)act;
    return run_vp(a, pack_bits, dim, (hipStream_t)stream);
}

// SwitchGLU over packed VQ experts in one call.  Workspace: act [T*k, I],
// y [T*k, H] for the combine, then the expert sort (sized for up to 4096
// experts at any tile height).
static size_t vps_act_bytes(int64_t P, int64_t I) { return ((size_t)P * I * 2 + 255) & ~(size_t)255; }
static size_t vps_y_bytes(int64_t P, int64_t H) { return ((size_t)P * H * 2 + 255) & ~(size_t)255; }

size_t kmi_vq_packed_switch_glu_workspace_bytes(int64_t T, int64_t H, int64_t I, int k) {
    if (T <= 0 || H <= 0 || I <= 0 || k <= 0) return 0;
    const int64_t P = T * k;
    return vps_act_bytes(P, I) + vps_y_bytes(P, H) + sort_index_bytes(P, 4096, 1);
}

}  // extern "C"

// Below 17 (token, slot) pairs (or where the expert-tile kernel does not
// cover the shape) each pair runs on its own; beyond, rows are grouped by
// expert.
static bool vps_grouped(int64_t P, int64_t E, int pack_bits, int dim, int group, int64_t H, int64_t I, int kc,
                        bool two_cb) {
    return P > 16 && E <= 4096 && vpm_supported(pack_bits, dim, group, H, kc, two_cb) &&
           vpm_supported(pack_bits, dim, group, I, kc, false);
}

// In-kernel routing: the per-pair path, E <= 256, k <= 8, and the router's
// state beside the gate/up kernel's codebooks and x in the LDS.
static bool vps_route_fits(int64_t P, int64_t E, int k, int pack_bits, int dim, int group, int64_t H, int64_t I,
                           int kc, bool two_cb) {
    return E <= ROUTE_THREADS && k >= 1 && k <= 8 && !vps_grouped(P, E, pack_bits, dim, group, H, I, kc, two_cb) &&
           vp_lds(H, kc, dim, two_cb, true) <= 160 * 1024;
}

// The packed SwitchGLU.  With logits (per-pair path, E <= 256, k <= 8) the
// gate/up kernel routes each pair's token and writes inds / scores, which
// the down kernel and the combine read.
static int vps_switch_glu_impl(const void* x, int64_t T, int64_t H, int64_t I, int k, const int32_t* inds,
                               const void* scores, const uint32_t* codes_gate, const void* scales_gate,
                               const void* codebook_gate, const uint32_t* codes_up, const void* scales_up,
                               const void* codebook_up, const uint32_t* codes_down, const void* scales_down,
                               const void* codebook_down, int pack_bits, int kc, int dim, int group, int64_t E,
                               int dtype, void* out, void* workspace, size_t workspace_bytes, void* stream,
                               const void* logits, bool routed = false) {
    int rc = vp_check(dtype, pack_bits, kc, dim, group, H, I, E);
    if (rc) return rc;
    rc = vp_check(dtype, pack_bits, kc, dim, group, I, H, E);
    if (rc) return rc;
    KMI_CHECK_ARG(T >= 0 && k >= 1 && k <= 64, "vq_packed_switch_glu: bad sizes");
    if (T == 0) return OK;
    KMI_CHECK_ARG(x && inds && codes_gate && scales_gate && codebook_gate && codes_up && scales_up &&
                      codebook_up && codes_down && scales_down && codebook_down && out,
                  "vq_packed_switch_glu: null pointer");
    const int64_t P = T * k;
    KMI_CHECK_ARG(P < 65536 && T * H * 2 < (1LL << 31) && P * (H > I ? H : I) * 2 < (1LL << 31),
                  "vq_packed_switch_glu: %lld (token, slot) pairs (at most 65535)", (long long)P);
    const size_t need = kmi_vq_packed_switch_glu_workspace_bytes(T, H, I, k);
    if (!workspace || workspace_bytes < need) {
        set_error("vq_packed_switch_glu: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
        return EWORKSPACE;
    }
    hipStream_t st = (hipStream_t)stream;
    uint16_t* act = (uint16_t*)workspace;
    uint16_t* y = scores ? (uint16_t*)((char*)workspace + vps_act_bytes(P, I)) : (uint16_t*)out;
    const int64_t Wg = (H / dim + 31) / 32 * pack_bits, Wd = (I / dim + 31) / 32 * pack_bits;
    // Expert-major on MFMA beyond 16 pairs where the kernel covers the shape
    // (pairs that share an expert then share its decode); per pair below.
    const bool two_cb = codebook_up != codebook_gate;
    const bool grouped = vps_grouped(P, E, pack_bits, dim, group, H, I, kc, two_cb);
    if (logits && !vps_route_fits(P, E, k, pack_bits, dim, group, H, I, kc, two_cb)) {
        set_error("vq_packed_switch_glu: in-kernel routing is for the per-pair path, E <= %d, k <= 8", ROUTE_THREADS);
        return EINVAL_ARG;
    }
    if (grouped) {
        const int64_t avg = ceil_div(P, E < P ? E : P);
        // tiles sized to the rows an expert sees: the LDS holds a tile's x rows,
        // so small tiles fit more workgroups per CU (T = 16 of 128 experts,
        // top-8, 2048 x 4: 8-row tiles 146 us, 4-row 117 us)
        int tile_rows = (int)(avg <= 2 ? 4 : avg <= 4 ? 8 : VPM_TILE);
        if (tile_rows > P) tile_rows = (int)P;
        // inds from the router (every expert in range) and few pairs: the
        // kernels form their tiles themselves, no sort
        const bool formed = routed && pair_tiles_fit(P, E, tile_rows);
        SortedRows sr = {};
        int32_t* const list = (int32_t*)((char*)workspace + vps_act_bytes(P, I) + vps_y_bytes(P, H));
        if (!formed) {
            void* index_ws = list;
            // the sort zeroes y's rows of out-of-range experts (no tile holds them)
            rc = launch_sort_rows(inds, P, 1, (int)E, tile_rows, index_ws, y, H, st, &sr);
            if (rc) return rc;
        }
        const int64_t max_tiles = sort_max_tiles(P, E, tile_rows);
        VpmArgs g = {};
        g.x = (const uint16_t*)x; g.X = T; g.lhs_div = k; g.tiles = sr.tiles; g.sorted = sr.sorted; g.E = E;
        g.rhs = inds; g.pairs = (int)P;
        if (formed) {       // the gate/up kernel writes the sort's list for the down kernel
            g.sorted_out = list;
            g.tiles_out = list + P;
        }
        g.codes[0] = codes_gate; g.codes[1] = codes_up;
        g.sc[0] = (const uint16_t*)scales_gate; g.sc[1] = (const uint16_t*)scales_up;
        g.cb[0] = (const uint16_t*)codebook_gate; g.cb[1] = (const uint16_t*)codebook_up;
        g.kc = kc; g.N = I; g.K = H; g.W = Wg; g.y = act; g.tile_rows = tile_rows;
        rc = launch_vpm(g, pack_bits, dim, group, 2, max_tiles, st);
        if (rc) return rc;
        KMI_CHECK_LAUNCH("vq_packed_mfma(glu)");
        VpmArgs d = {};
        d.x = act; d.X = P; d.lhs_div = 1; d.tiles = sr.tiles; d.sorted = sr.sorted; d.E = E;
        if (formed) {       // the list the gate/up kernel wrote
            d.sorted = list;
            d.tiles = list + P;
        }
        d.codes[0] = d.codes[1] = codes_down;
        d.sc[0] = d.sc[1] = (const uint16_t*)scales_down;
        d.cb[0] = d.cb[1] = (const uint16_t*)codebook_down;
        d.kc = kc; d.N = H; d.K = I; d.W = Wd; d.y = y; d.tile_rows = tile_rows;
        rc = launch_vpm(d, pack_bits, dim, group, 1, max_tiles, st);
        if (rc) return rc;
        KMI_CHECK_LAUNCH("vq_packed_mfma(down)");
    } else {
        VpArgs g = {};
        g.x = (const uint16_t*)x; g.X = T; g.rows = nullptr; g.rows_div = k; g.experts = inds; g.R = P;
        g.codes[0] = codes_gate; g.codes[1] = codes_up;
        g.sc[0] = (const uint16_t*)scales_gate; g.sc[1] = (const uint16_t*)scales_up;
        g.cb[0] = (const uint16_t*)codebook_gate; g.cb[1] = (const uint16_t*)codebook_up;
        g.nset = 2; g.kc = kc; g.E = E; g.N = I; g.K = H; g.W = Wg; g.group = group; g.y = act;
        if (logits) {
            g.logits = (const uint16_t*)logits;
            g.inds_out = (int32_t*)inds;
            g.scores_out = (uint16_t*)scores;
            g.k = k;
        }
        rc = run_vp(g, pack_bits, dim, st);
        if (rc) return rc;
        VpArgs d = {};
        d.x = act; d.X = P; d.rows = nullptr; d.rows_div = 1; d.experts = inds; d.R = P;
        d.codes[0] = d.codes[1] = codes_down;
        d.sc[0] = d.sc[1] = (const uint16_t*)scales_down;
        d.cb[0] = d.cb[1] = (const uint16_t*)codebook_down;
        d.nset = 1; d.kc = kc; d.E = E; d.N = H; d.K = I; d.W = Wd; d.group = group; d.y = y;
        if (scores) {    // token-major down with the combine in its epilogue, where it fits
            VpdArgs td = {};
            td.act = act; td.inds = inds; td.scores = (const uint16_t*)scores; td.codes = codes_down;
            td.sc = (const uint16_t*)scales_down; td.cb = (const uint16_t*)codebook_down; td.out = (uint16_t*)out;
            td.E = E; td.N = H; td.K = I; td.W = Wd; td.T = T; td.k = k; td.kc = kc; td.group = group;
            if (run_vpd(td, pack_bits, dim, st) == 0) {
                KMI_CHECK_LAUNCH("vq_packed_down_tok");
                return OK;
            }
        }
        rc = run_vp(d, pack_bits, dim, st);
        if (rc) return rc;
    }
    if (scores) return kmi_moe_combine(y, scores, dtype, T, k, H, out, stream);
    return OK;
}

extern "C" {

int kmi_vq_packed_switch_glu(const void* x, int64_t T, int64_t H, int64_t I, int k, const int32_t* inds,
                             const void* scores, const uint32_t* codes_gate, const void* scales_gate,
                             const void* codebook_gate, const uint32_t* codes_up, const void* scales_up,
                             const void* codebook_up, const uint32_t* codes_down, const void* scales_down,
                             const void* codebook_down, int pack_bits, int kc, int dim, int group, int64_t E,
                             int dtype, void* out, void* workspace, size_t workspace_bytes, void* stream) {
    clear_error();
    return vps_switch_glu_impl(x, T, H, I, k, inds, scores, codes_gate, scales_gate, codebook_gate, codes_up,
                               scales_up, codebook_up, codes_down, scales_down, codebook_down, pack_bits, kc, dim,
                               group, E, dtype, out, workspace, workspace_bytes, stream, nullptr);
}

int kmi_vq_packed_experts(const void* x, const void* logits, int64_t T, int64_t H, int64_t I, int k,
                          const uint32_t* codes_gate, const void* scales_gate, const void* codebook_gate,
                          const uint32_t* codes_up, const void* scales_up, const void* codebook_up,
                          const uint32_t* codes_down, const void* scales_down, const void* codebook_down,
                          int pack_bits, int kc, int dim, int group, int64_t E, int dtype, void* out,
                          int32_t* inds, void* scores, void* workspace, size_t workspace_bytes, void* stream) {
    clear_error();
    KMI_CHECK_ARG(dtype == BF16, "vq_packed_experts: only bfloat16 activations and logits are implemented");
    KMI_CHECK_ARG(E >= 1 && E <= ROUTE_MAX_E && k >= 1 && k <= 8 && k <= E,
                  "vq_packed_experts: top-%d of %lld experts (k <= 8, E <= %d)", k, (long long)E, ROUTE_MAX_E);
    KMI_CHECK_ARG(T >= 0, "vq_packed_experts: T=%lld", (long long)T);
    if (T == 0) return OK;
    KMI_CHECK_ARG(logits && inds && scores, "vq_packed_experts: null pointer");
    const bool two_cb = codebook_up != codebook_gate;
    const bool in_kernel = vps_route_fits(T * k, E, k, pack_bits, dim, group, H, I, kc, two_cb);
    if (!in_kernel) {
        const int rc = kmi_moe_route(logits, dtype, T, (int)E, k, inds, scores, stream);
        if (rc) return rc;
    }
    return vps_switch_glu_impl(x, T, H, I, k, inds, scores, codes_gate, scales_gate, codebook_gate, codes_up,
                               scales_up, codebook_up, codes_down, scales_down, codebook_down, pack_bits, kc, dim,
                               group, E, dtype, out, workspace, workspace_bytes, stream,
                               in_kernel ? logits : nullptr, true);
}

}  // extern "C"
