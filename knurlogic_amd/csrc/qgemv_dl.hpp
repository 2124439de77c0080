// Direct-to-LDS staging shared by the skinny quantized matmul kernels
// (qgemv_dl.hip: dense 2..16 rows; qgemv_xs.hip: rows grouped by expert
// with the tile's x staged once): chunk shapes of 64 weight rows, the DMA
// load helpers (buffer_load ... lds), the vmcnt wait and the exact 4-bit
// decode in natural k order.
#pragma once

#include "qgemv.hpp"

#define KMI_LDSP(p) ((__attribute__((address_space(3))) void*)(p))

namespace kmi {

namespace {


constexpr int DL_KC = 256;                // codes per chunk (least)
constexpr int DL_ROWS = 64;               // weight rows per workgroup
constexpr int DL_WBLK_BYTES = 1024 + 16;  // one DMA block of weight rows, padded
constexpr uint32_t DL_NONE = 0x80000000u; // an offset past every buffer: reads 0

// 8 codes (code i at bits 4i) -> 8 exact bf16 in natural order: a byte q in
// 0..15 read as fp8 e4m3 is q * 2^-9, and the conversion's scale 2^9 is exact
__device__ __forceinline__ u32x4 nib8_natural(uint32_t w) {
    const uint32_t lo = w & 0x0F0F0F0Fu;            // codes 0, 2, 4, 6
    const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;     // codes 1, 3, 5, 7
    const uint32_t a = __builtin_amdgcn_perm(hi, lo, 0x05010400u);   // [c0, c1, c2, c3]
    const uint32_t b = __builtin_amdgcn_perm(hi, lo, 0x07030602u);   // [c4, c5, c6, c7]
    u32x4 r;
    r.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(a, 512.f, false));
    r.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(a, 512.f, true));
    r.z = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(b, 512.f, false));
    r.w = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(b, 512.f, true));
    return r;
}

// 8 codes (code i at bits 4i) -> 8 exact bf16 in the order [0,2,4,6,1,3,5,7]
// (the low nibbles of the four bytes, then the high ones): no byte shuffle,
// for x staged in the same order (x8_paired)
__device__ __forceinline__ u32x4 nib8_paired(uint32_t w) {
    const uint32_t lo = w & 0x0F0F0F0Fu;            // codes 0, 2, 4, 6
    const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;     // codes 1, 3, 5, 7
    u32x4 r;
    r.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 512.f, false));
    r.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 512.f, true));
    r.z = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 512.f, false));
    r.w = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 512.f, true));
    return r;
}

// 8 bf16 in natural k order -> the order [0,2,4,6,1,3,5,7]
__device__ __forceinline__ u32x4 x8_paired(u32x4 v) {
    return u32x4{__builtin_amdgcn_perm(v.y, v.x, 0x05040100u), __builtin_amdgcn_perm(v.w, v.z, 0x05040100u),
                 __builtin_amdgcn_perm(v.y, v.x, 0x07060302u), __builtin_amdgcn_perm(v.w, v.z, 0x07060302u)};
}

template <int N_>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N_ >= 0 && N_ < 64, "vmcnt");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N_) : "memory");
}

// One DMA load: lane i's `size` bytes at voff + soff land at lds + i * size.
// (Device functions, not the builtin itself inside the kernel template's
// lambda: there the builtin stops hipcc emitting the host launch stubs.)
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, unsigned char* lds, uint32_t voff, uint32_t soff,
                                      int aux) {
    if (aux) __builtin_amdgcn_raw_ptr_buffer_load_lds(r, KMI_LDSP(lds), 16, voff, soff, 0, AUX_NT);
    else __builtin_amdgcn_raw_ptr_buffer_load_lds(r, KMI_LDSP(lds), 16, voff, soff, 0, 0);
}

__device__ __forceinline__ void dma4(__amdgpu_buffer_rsrc_t r, unsigned char* lds, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, KMI_LDSP(lds), 4, voff, soff, 0, 0);
}

// A chunk is KS slices of 256 codes; the workgroup has 4 * KS waves, wave w
// owning weight rows 16 (w % 4) .. + 15 of slice w / 4 of every chunk, and
// the slices' partial sums are added in the epilogue (KS waves per SIMD,
// without a second kernel).
// MX: microscaled codes (E2M1 / E4M3, exact in bf16), one E8M0 byte scale
// per 32 inputs and no biases.  A row's scales of one chunk are GPC bytes:
// each wave moves 16 / KS rows' (32 lanes of 4 bytes, the other 32 lanes
// read zeros into padding: 256 bytes per wave).  The affine bf16 scales and
// biases move in 4-byte units, DPR blocks each.
template <int BITS, int GS, bool MX, int KS>
struct DlShape {
    static constexpr int KC = DL_KC * KS;               // codes per chunk
    static constexpr int NW = 4 * KS;                    // waves
    static constexpr int RB = KC * BITS / 8;             // weight bytes per row per chunk
    static constexpr int RPI = 1024 / RB;                // weight rows per DMA block
    static constexpr int WBLK = DL_ROWS / RPI;           // weight blocks per chunk
    static constexpr int PPR = RB / 16;                  // 16-byte pieces per weight row
    static constexpr int W_BYTES = WBLK * DL_WBLK_BYTES;
    static constexpr int XR = KC * 2;                    // x bytes per row per chunk
    static constexpr int XPB = XR <= 1024 ? 1024 / XR : 1;   // x rows per DMA block
    static constexpr int XBR = XR >= 1024 ? XR / 1024 : 1;   // DMA blocks per x row
    static constexpr int XI = 16 * XBR / XPB;            // x blocks per chunk
    static constexpr int X_BYTES = 16 * XR;
    static constexpr int GPC = KC / GS;                  // groups per chunk
    static constexpr int GPS = GPC / KS;                 // groups per slice
    static constexpr int SB = MX ? 1 : 2;                // bytes per scale
    static constexpr int DPR = MX ? 1 : GPC / 2;         // affine: 4-byte elements per row per chunk
    static constexpr int SBI = MX ? NW : 2 * DPR;        // scale (+ bias) blocks per chunk
    static constexpr int SB_BYTES = MX ? NW * 256 : 2 * DL_ROWS * GPC * 2;
    static constexpr int MXL = GPC / 4;                  // MX: lanes per row
    static constexpr int MXR = 32 / MXL;                 // MX: rows per block
    static constexpr int STAGE = W_BYTES + X_BYTES + SB_BYTES;
    static constexpr int PER_WAVE = (WBLK + XI + SBI) / NW;   // DMA loads per wave per chunk
    static constexpr int GB = GS * BITS / 8;             // bytes per row per group
    static constexpr int LB = GB / 4;                    // bytes of a group per lane (k run)
    static constexpr int NT = GS / 32;                   // MFMAs per group
    static_assert(WBLK % NW == 0 && XI % NW == 0 && SBI % NW == 0, "every wave issues the same loads");
    static_assert(LB == 4 || LB == 8 || LB == 16, "lane run of 4, 8 or 16 bytes");
    static_assert(!MX || MXR * NW == DL_ROWS, "MX: one scale block per wave");
    static_assert(XR == 512 || XR % 1024 == 0, "x rows of 512 bytes or whole 1 KB blocks");
    static_assert(GPS >= 1 && GPS % (GPS < 4 ? GPS : 4) == 0, "whole group batches per slice");
};

}  // namespace

}  // namespace kmi
