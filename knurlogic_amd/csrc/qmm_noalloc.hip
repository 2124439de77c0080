// kmi_qmm_noalloc: mx.quantized_matmul (the kmi_qmm kernels, unchanged) for
// callers that cannot allocate device memory -- code under HIP graph
// capture, serving loops that forbid allocation.  kmi_qmm takes its split-K
// partials in a caller-allocated workspace; here they live in `scratch`, a
// file-scope device array of KMI_QMM_SCRATCH_BYTES that every GPU the
// library runs on holds until the process ends.
//
// `scratch` names the array only in device code.  In host code the name is
// a host-side stand-in, not a device address, so the host side resolves the
// array's address once per device with hipGetSymbolAddress (with that device
// current) and passes that pointer to the kernels, never the name.
//
// Every call on a GPU shares that GPU's array: calls that overlap on one GPU
// (two streams, two threads) race on it.  The kernels write every partial
// they later read (split s writes all of its [M, N] slice before the
// in-order reduce reads it), so nothing in the array has to start at zero
// and the previous call's contents are never read.
#include "common.hpp"
#include "../../include/knurlogic_amd.h"

#include <mutex>

namespace kmi {

static __device__ __align__(256) unsigned char scratch[KMI_QMM_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;

// Device address of `scratch` on the current device, resolved on the first
// call per device.
static int scratch_on_current_device(void** out) {
    static std::mutex mu;
    static void* addr[MAX_DEVICES] = {};
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        set_error("quantized_matmul (no-alloc): hipGetDevice failed: %s", hipGetErrorString(e));
        return EHIP;
    }
    KMI_CHECK_ARG(dev >= 0 && dev < MAX_DEVICES, "quantized_matmul (no-alloc): device %d out of range", dev);
    std::lock_guard<std::mutex> lock(mu);
    if (addr[dev] == nullptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            set_error("quantized_matmul (no-alloc): hipGetSymbolAddress(scratch) on device %d failed: %s", dev,
                      hipGetErrorString(e));
            return EHIP;
        }
        addr[dev] = p;
    }
    *out = addr[dev];
    return OK;
}

}  // namespace kmi

using namespace kmi;

extern "C" {

size_t kmi_qmm_noalloc_scratch_bytes(void) { return KMI_QMM_SCRATCH_BYTES; }

int kmi_qmm_noalloc(const void* x, int64_t M, int64_t K, int64_t N, const uint32_t* w, const void* scales,
                    const void* biases, int dtype, int group_size, int bits, void* y, void* stream) {
    clear_error();
    const size_t need = kmi_qmm_workspace_bytes(M, K, N, group_size, bits);
    if (need > KMI_QMM_SCRATCH_BYTES) {
        set_error("quantized_matmul (no-alloc): M=%lld K=%lld N=%lld needs %zu bytes of split-K partials, "
                  "more than the %zu-byte scratch array; use kmi_qmm with a workspace",
                  (long long)M, (long long)K, (long long)N, need, (size_t)KMI_QMM_SCRATCH_BYTES);
        return EINVAL_ARG;
    }
    void* ws = nullptr;
    const int rc = scratch_on_current_device(&ws);
    if (rc) return rc;
    return kmi_qmm(x, M, K, N, w, scales, biases, dtype, group_size, bits, y, need ? ws : nullptr, need,
                   stream);
}

}  // extern "C"
