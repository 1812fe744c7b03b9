// Measurement floor of the streaming kernels: a kernel that only reads.
//
// bz_stream_read reads `bytes` from `p` once, 16 bytes per load with
// non-temporal loads, four loads in flight per thread, and writes nothing
// unless a thread's XOR of what it read equals a key the caller passes (so
// the loads cannot be dropped; with data that never matches, nothing is
// written).  Its time over bytes is the best any kernel of this library that
// streams its weights once can do on the device; bytes = 0 launches one
// empty workgroup, the fixed cost of a launch.
#include <hip/hip_runtime.h>

#include "bz_device.h"
#include "bz_gemv.h"

namespace bz {

constexpr int kProbeThreads = 256;
constexpr int kProbeLoads = 4;
constexpr size_t kProbeBlockBytes = (size_t)kProbeThreads * kProbeLoads * 16;

__global__ void __launch_bounds__(kProbeThreads) stream_read_kernel(const u32x4* src, uint32_t key, uint32_t* sink) {
    const size_t base = (size_t)blockIdx.x * (kProbeThreads * kProbeLoads) + threadIdx.x;
    u32x4 v[kProbeLoads];
#pragma unroll
    for (int i = 0; i < kProbeLoads; ++i) v[i] = __builtin_nontemporal_load(src + base + (size_t)i * kProbeThreads);
    uint32_t a = 0;
#pragma unroll
    for (int i = 0; i < kProbeLoads; ++i) a ^= v[i][0] ^ v[i][1] ^ v[i][2] ^ v[i][3];
    if (a == key) sink[0] = a;
}

__global__ void empty_kernel(uint32_t key, uint32_t* sink) {
    if (threadIdx.x == key) sink[0] = key;
}

}  // namespace bz

extern "C" int bz_stream_read(const void* p, size_t bytes, uint32_t key, uint32_t* sink, void* stream) {
    using namespace bz;
    if (!sink || (bytes && !p)) return BZ_ERR_INVALID_ARG;
    if (bytes % kProbeBlockBytes) return BZ_ERR_SHAPE;
    if (reinterpret_cast<uintptr_t>(p) & 15) return BZ_ERR_ALIGNMENT;
    const size_t blocks = bytes / kProbeBlockBytes;
    if (blocks > 0x7FFFFFFFu) return BZ_ERR_UNSUPPORTED;
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (blocks == 0)
        hipLaunchKernelGGL(empty_kernel, dim3(1), dim3(64), 0, st, 0xFFFFFFFFu, sink);
    else
        hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)blocks), dim3(kProbeThreads), 0, st,
                           static_cast<const u32x4*>(p), key, sink);
    return hipGetLastError() == hipSuccess ? BZ_OK : BZ_ERR_LAUNCH;
}
