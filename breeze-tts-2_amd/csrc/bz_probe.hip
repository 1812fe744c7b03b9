// Measurement floor of the streaming kernels: a kernel that only reads.
//
// bz_stream_read reads `bytes` from `p` once: workgroup b reads the
// contiguous chunk [b * chunk, (b + 1) * chunk) the way the streaming GEMV
// reads a 16-row block of a tiled weight -- wave w takes L consecutive 1 KiB
// tiles and issues all of its 16-byte non-temporal loads at once -- through a
// range-checked buffer resource (a load past the chunk reads zeros without a
// memory request).  It writes nothing unless a thread's XOR of what it read
// equals a key the caller passes (so the loads cannot be dropped).  Its time
// over bytes is the best a kernel of this library that streams its weights
// once, `chunk` bytes per workgroup, can do on the device; bytes = 0
// launches one empty workgroup, the fixed cost of a launch.
#include <hip/hip_runtime.h>

#include "bz_device.h"
#include "bz_gemv.h"

namespace bz {

template <int L>
__global__ void __launch_bounds__(1024) stream_read_kernel(const uint8_t* src, uint32_t chunk, uint32_t key,
                                                           uint32_t* sink) {
    const __amdgpu_buffer_rsrc_t r = buffer_rsrc(src + (size_t)blockIdx.x * chunk, chunk);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    u32x4 v[L];
#pragma unroll
    for (int i = 0; i < L; ++i) v[i] = buffer_ld16_nt(r, (uint32_t)(wave * L + i) * 1024u + lane * 16);
    uint32_t a = 0;
#pragma unroll
    for (int i = 0; i < L; ++i) a ^= v[i][0] ^ v[i][1] ^ v[i][2] ^ v[i][3];
    if (a == key) sink[0] = a;
}

__global__ void empty_kernel(uint32_t key, uint32_t* sink) {
    if (threadIdx.x == key) sink[0] = key;
}

}  // namespace bz

extern "C" int bz_stream_read(const void* p, size_t bytes, size_t chunk, uint32_t key, uint32_t* sink, void* stream) {
    using namespace bz;
    if (!sink || (bytes && (!p || !chunk))) return BZ_ERR_INVALID_ARG;
    if (bytes && (bytes % chunk || chunk % 16 || chunk > 0x7FFFFFF0u)) return BZ_ERR_SHAPE;
    if (reinterpret_cast<uintptr_t>(p) & 15) return BZ_ERR_ALIGNMENT;
    const size_t blocks = bytes ? bytes / chunk : 0;
    if (blocks > 0x7FFFFFFFu) return BZ_ERR_UNSUPPORTED;
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (blocks == 0) {
        hipLaunchKernelGGL(empty_kernel, dim3(1), dim3(64), 0, st, 0xFFFFFFFFu, sink);
    } else {
        // 1 KiB tiles per chunk, about 4 per wave, at most 16 waves
        const size_t tiles = (chunk + 1023) / 1024;
        int L = 4;
        while (L < 16 && (tiles + L - 1) / L > 16) L *= 2;
        if ((tiles + L - 1) / L > 16) return BZ_ERR_UNSUPPORTED;  // chunk above 256 KiB
        const dim3 grid((unsigned)blocks), block((unsigned)(64 * ((tiles + L - 1) / L)));
        const uint8_t* src = static_cast<const uint8_t*>(p);
        switch (L) {
            case 4: hipLaunchKernelGGL(stream_read_kernel<4>, grid, block, 0, st, src, (uint32_t)chunk, key, sink); break;
            case 8: hipLaunchKernelGGL(stream_read_kernel<8>, grid, block, 0, st, src, (uint32_t)chunk, key, sink); break;
            default: hipLaunchKernelGGL(stream_read_kernel<16>, grid, block, 0, st, src, (uint32_t)chunk, key, sink); break;
        }
    }
    return hipGetLastError() == hipSuccess ? BZ_OK : BZ_ERR_LAUNCH;
}
