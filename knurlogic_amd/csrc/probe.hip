// Calibration kernels.
//   - read_probe: a plain read of a device buffer with the loads the
//     hot-path kernels use (16-byte nontemporal buffer loads, whole 64-byte
//     runs per 4 lanes), so a caller can measure the HBM read rate this GPU
//     reaches at a given size.  Nothing is computed; the XOR of the data is
//     written only when it equals a value no caller passes, which keeps the
//     loads from being dropped.
//   - mfma_probe: the prefill GEMM's matrix-core work alone -- 8 waves per
//     workgroup (two per SIMD), each 2 x 2 accumulators of
//     v_mfma_f32_32x32x16_bf16 fed from registers, 16 MFMAs per round -- so
//     a caller can measure the bf16 MFMA rate and, from the shader-clock and
//     100 MHz counters read around the first wave's loop, the clock the
//     matrix cores run at under that load.
#include "common.hpp"
#include "../../include/knurlogic_amd.h"

namespace kmi {

__global__ __launch_bounds__(256) void read_probe_kernel(const void* p, int64_t bytes, uint32_t never,
                                                         uint32_t* out) {
    const __amdgpu_buffer_rsrc_t r = make_rsrc(p, bytes);
    const int64_t pieces = bytes / 16;
    const int64_t stride = (int64_t)gridDim.x * 256;
    uint32_t acc = 0;
    int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    // four loads in flight per thread
    for (; i + 3 * stride < pieces; i += 4 * stride) {
        u32x4 v[4];
#pragma unroll
        for (int j = 0; j < 4; j++)
            v[j] = __builtin_amdgcn_raw_buffer_load_b128(r, (int)((i + j * stride) * 16), 0, AUX_NT);
#pragma unroll
        for (int j = 0; j < 4; j++) acc ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
    }
    for (; i < pieces; i += stride) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)(i * 16), 0, AUX_NT);
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == never) out[0] = acc;
}

__global__ __launch_bounds__(512, 1) void mfma_probe_kernel(const uint32_t* __restrict__ seed, int iters,
                                                           uint32_t never, uint32_t* out, uint64_t* stamps) {
    // 96 KB of LDS that no other workgroup fits beside: one workgroup per CU
    __shared__ uint32_t hold[24576];
    const int lane = threadIdx.x & 63;
    hold[threadIdx.x] = never ^ lane;
    u32x4 a[2], b[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        a[i] = u32x4{seed[(lane + 4 * i) & 63], seed[(lane + 4 * i + 1) & 63], seed[(lane + 4 * i + 2) & 63],
                     seed[(lane + 4 * i + 3) & 63]};
        b[i] = u32x4{seed[(lane + 8 + 4 * i) & 63], seed[(lane + 9 + 4 * i) & 63], seed[(lane + 10 + 4 * i) & 63],
                     seed[(lane + 11 + 4 * i) & 63]};
    }
    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;
    const uint64_t c0 = __builtin_readcyclecounter(), r0 = __builtin_amdgcn_s_memrealtime();
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int s = 0; s < 4; s++)
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a[i]), as_bf16x8(b[j]),
                                                                          acc[i][j], 0, 0, 0);
    }
    const uint64_t c1 = __builtin_readcyclecounter(), r1 = __builtin_amdgcn_s_memrealtime();
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) t += acc[i][j][r];
    if (__float_as_uint(t) == never) out[0] = hold[threadIdx.x] ^ __float_as_uint(t);
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        stamps[0] = c1 - c0;
        stamps[1] = r1 - r0;
    }
}

}  // namespace kmi

using namespace kmi;

extern "C" int kmi_read_probe(const void* p, int64_t bytes, int workgroups, uint32_t* out, void* stream) {
    clear_error();
    KMI_CHECK_ARG(p && out, "read_probe: null pointer");
    KMI_CHECK_ARG(bytes > 0 && bytes % 16 == 0 && bytes < (1LL << 31),
                  "read_probe: %lld bytes (a positive multiple of 16 under 2 GiB)", (long long)bytes);
    KMI_CHECK_ARG(workgroups > 0 && workgroups <= 65536, "read_probe: %d workgroups", workgroups);
    read_probe_kernel<<<workgroups, 256, 0, (hipStream_t)stream>>>(p, bytes, 0x9E3779B9u, out);
    KMI_CHECK_LAUNCH("read_probe");
    return OK;
}

extern "C" int kmi_mfma_probe(const uint32_t* seed, int workgroups, int iters, uint32_t* out, uint64_t* stamps,
                              void* stream) {
    clear_error();
    KMI_CHECK_ARG(seed && out && stamps, "mfma_probe: null pointer");
    KMI_CHECK_ARG(workgroups > 0 && workgroups <= 65536, "mfma_probe: %d workgroups", workgroups);
    KMI_CHECK_ARG(iters > 0 && iters <= (1 << 24), "mfma_probe: %d rounds", iters);
    mfma_probe_kernel<<<workgroups, 512, 0, (hipStream_t)stream>>>(seed, iters, 0x7fc00001u, out, stamps);
    KMI_CHECK_LAUNCH("mfma_probe");
    return OK;
}
