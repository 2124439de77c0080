// Calibration kernel: a plain read of a device buffer with the loads the
// hot-path kernels use (16-byte nontemporal buffer loads, whole 64-byte
// runs per 4 lanes), so a caller can measure the HBM read rate this GPU
// reaches at a given size.  Nothing is computed; the XOR of the data is
// written only when it equals a value no caller passes, which keeps the
// loads from being dropped.
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
