// Shared device/host helpers for the gfx950 quantized-weight kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stdio.h>
#include <stdarg.h>

#include <mutex>
#include <set>
#include <utility>

namespace kmi {

// dtype codes of the C ABI (include/knurlogic_amd.h)
enum Dtype : int { BF16 = 0, F16 = 1, F32 = 2 };

// ---- error reporting: thread-local message, negative return codes ---------
enum Err : int {
    OK = 0,
    EINVAL_ARG = -1,   // bad shape / unsupported combination
    EHIP = -2,         // a HIP runtime call failed
    EWORKSPACE = -3,   // workspace missing or too small
};

void set_error(const char* fmt, ...);
void clear_error();

#define KMI_CHECK_ARG(cond, ...)                 \
    do {                                         \
        if (!(cond)) {                           \
            ::kmi::set_error(__VA_ARGS__);       \
            return ::kmi::EINVAL_ARG;            \
        }                                        \
    } while (0)

#define KMI_CHECK_LAUNCH(what)                                               \
    do {                                                                     \
        hipError_t e_ = hipGetLastError();                                   \
        if (e_ != hipSuccess) {                                              \
            ::kmi::set_error("%s: launch failed: %s", what, hipGetErrorString(e_)); \
            return ::kmi::EHIP;                                              \
        }                                                                    \
    } while (0)

// ---- bf16 / fp16 <-> fp32 (bit exact, round to nearest even) ----------------

// E8M0 scale byte e -> 2^(e - 127) in fp32, without branches: e << 23 is
// that float for e in 1..254; e = 0 (2^-127, the subnormal 0x00400000) and
// e = 255 (NaN, 0x7fc00000) are e << 23 with bit 22 set, and exactly these
// two values have (e + 1) & 0xfe == 0.
// Lets kernel f take all the LDS its static allocation leaves (160 KB per
// workgroup on gfx950), and leaves no error behind for the launch check.
inline void allow_dynamic_lds(const void* f) {
    hipFuncAttributes fa = {};
    const size_t stat = hipFuncGetAttributes(&fa, f) == hipSuccess ? fa.sharedSizeBytes : 0;
    (void)hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)(160 * 1024 - stat));
    (void)hipGetLastError();
}

// allow_dynamic_lds for kernel f on the current device, once per (kernel,
// device): the attribute is a property of the function on each device.
inline void allow_dynamic_lds_once(const void* f) {
    static std::mutex mu;
    static std::set<std::pair<const void*, int>> done;
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess) {
        (void)hipGetLastError();
        dev = -1;
    }
    std::lock_guard<std::mutex> lock(mu);
    if (done.insert({f, dev}).second) allow_dynamic_lds(f);
}

__device__ __forceinline__ float e8m0_to_f32(uint32_t e) {
    e &= 0xffu;
    const uint32_t special = ((((e + 1u) & 0xfeu) - 1u) >> 31) << 22;
    return __uint_as_float((e << 23) | special);
}

__host__ __device__ __forceinline__ float bf16_to_f32(uint16_t h) {
    return __uint_as_float(((uint32_t)h) << 16);
}

__host__ __device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
    return __half2float(__ushort_as_half(h));
}

__device__ __forceinline__ uint16_t f32_to_f16(float f) {
    return __half_as_ushort(__float2half_rn(f));
}

// Storage type tags: the kernels are templated on how an element of the
// activation / scale dtype is stored and converted.
struct TBF16 {
    using storage = uint16_t;
    static __device__ __forceinline__ float load(storage v) { return bf16_to_f32(v); }
    static __device__ __forceinline__ storage store(float f) { return f32_to_bf16(f); }
    static __device__ __forceinline__ float round(float f) { return bf16_to_f32(f32_to_bf16(f)); }
};
struct TF16 {
    using storage = uint16_t;
    static __device__ __forceinline__ float load(storage v) { return f16_to_f32(v); }
    static __device__ __forceinline__ storage store(float f) { return f32_to_f16(f); }
    static __device__ __forceinline__ float round(float f) { return f16_to_f32(f32_to_f16(f)); }
};
struct TF32 {
    using storage = float;
    static __device__ __forceinline__ float load(storage v) { return v; }
    static __device__ __forceinline__ storage store(float f) { return f; }
    static __device__ __forceinline__ float round(float f) { return f; }
};

// silu(g) = g / (1 + e^-g) of a bf16 value g, rounded to float32 and then to
// bf16: the SwiGLU epilogues' round(silu_f32(g)), silu evaluated exactly
// and rounded once to float32.  Float32 arithmetic (an accurate expf and a
// reciprocal, a few float32 ulps from that rounding) gives the same bf16
// unless its low 16 bits lie within SILU_WINDOW of the bf16 rounding
// midpoint, or |g| > 64 (e^-g past float32's range): those lanes take the
// float64 evaluation.  Checked on every bf16 value of g (kmi_swiglu in
// bf16 runs it; its test covers all 65536 gate patterns).
constexpr int SILU_WINDOW = 16;
__device__ __forceinline__ float silu_bf16r(float g) {
    const float t = g * __builtin_amdgcn_rcpf(1.0f + expf(-g));
    const int lo = (int)(__float_as_uint(t) & 0xffffu) - 0x8000;
    if (__builtin_expect((lo >= -SILU_WINDOW && lo <= SILU_WINDOW) || !(__builtin_fabsf(g) <= 64.0f), 0)) {
        const double gd = (double)g;
        float f = (float)(gd / (1.0 + exp(-gd)));
        asm volatile("" : "+v"(f));      // keep the float32 rounding (no fused f64 -> bf16 rounding)
        return bf16_to_f32(f32_to_bf16(f));
    }
    return bf16_to_f32(f32_to_bf16(t));
}

// ---- MFMA operand vector types ------------------------------------------------
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Two floats -> two bf16 (round to nearest even) in one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t cvt_pk_bf16(float lo, float hi) {
    const f32x2_t v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// 16x16x32 bf16 MFMA, fp32 accumulate (gfx950).  Lane l holds A[m = l%16]
// [k-run l/16], B[k-run l/16][n = l%16]; D[m = 4*(l/16)+i][n = l%16] in
// item i.  A and B share the k-run mapping, so any permutation of k
// applied to both leaves the product unchanged.
__device__ __forceinline__ f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

// Two bytes of a word -> two bf16 (exact: integers 0..255 need 8 significant bits).
__device__ __forceinline__ uint32_t bytes_to_bf16x2(uint32_t w, int lo_byte) {
    // (float)(byte) selects v_cvt_f32_ubyteN
    const float a = (float)((w >> (8 * lo_byte)) & 0xffu);
    const float b = (float)((w >> (8 * lo_byte + 8)) & 0xffu);
    // high halves of the two floats: the bf16 bit patterns (truncation is exact)
    return __builtin_amdgcn_perm(__float_as_uint(b), __float_as_uint(a), 0x07060302u);
}

// 4-bit nibbles -> bf16 "128 + q" pairs.  Register r holds nibbles r (low
// half) and r+4 (high half) of the word: k order [0,4,1,5,2,6,3,7].
__device__ __forceinline__ u32x4 nibbles_to_bf16_magic(uint32_t w) {
    const uint32_t M = 0x000F000Fu, E = 0x43004300u;
    u32x4 r;
    r.x = (w & M) | E;
    r.y = ((w >> 4) & M) | E;
    r.z = ((w >> 8) & M) | E;
    r.w = ((w >> 12) & M) | E;
    return r;
}

// Workgroup barrier that orders LDS only.  __syncthreads() also waits for
// every outstanding global load of the wave (vmcnt(0)), which would drain a
// weight stream issued before the barrier; here only LDS traffic
// (lgkmcnt) is drained, so loads in flight stay in flight.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// ---- raw buffer resources --------------------------------------------------------
// A load at byte offset >= `bytes` returns 0 instead of touching memory, so
// tails need no branch.  Offsets are 32-bit: callers check that every offset
// they form stays below 2^31.
constexpr int RSRC_DWORD3 = 0x00020000;   // raw buffer, gfx9 family
constexpr int AUX_NT = 2;                 // non-temporal: data read once per call

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, int64_t bytes) {
    const int64_t cap = 0x7fffffff;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, (int)(bytes < cap ? bytes : cap),
                                             RSRC_DWORD3);
}

// ---- misc ---------------------------------------------------------------------
inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace kmi
