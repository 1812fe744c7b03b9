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
//
// bz_shared_read is the floor of a several-row GEMV that gives every
// workgroup the whole K: each of `workgroups` workgroups reads all `xbytes`
// of x (the same bytes for all, so L2 serves them after the first touch)
// and its own `wchunk` bytes of w.
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

// Every workgroup reads all of x (L2-resident after the first touch) and its
// own chunk of w.  Vector loads retire in order, so a wave that mixed the two
// would make every x load wait behind the slower HBM loads of w: waves
// 0..kSharedWWaves-1 stream the chunk of w, the others stream x, each wave U
// 16-byte loads per lane in flight.
constexpr int kSharedWWaves = 4;

template <int U>
__global__ void __launch_bounds__(1024) shared_read_kernel(const uint8_t* x, uint32_t xbytes, const uint8_t* w,
                                                           uint32_t wchunk, uint32_t key, uint32_t* sink) {
    const int wave = threadIdx.x >> 6;
    const bool wrole = wave < kSharedWWaves;
    const int nroles = wrole ? kSharedWWaves : (int)(blockDim.x >> 6) - kSharedWWaves;
    const uint32_t step = (uint32_t)nroles * 1024u;  // bytes per round of the role's waves
    const uint32_t bytes = wrole ? wchunk : xbytes;
    const __amdgpu_buffer_rsrc_t r =
        wrole ? buffer_rsrc(w + (size_t)blockIdx.x * wchunk, wchunk) : buffer_rsrc(x, xbytes);
    const uint32_t lane_off = (uint32_t)((wrole ? wave : wave - kSharedWWaves) * 64 + (threadIdx.x & 63)) * 16u;
    const uint32_t rounds = (bytes + step - 1) / step;
    uint32_t a = 0;
    for (uint32_t r0 = 0; r0 < rounds; r0 += U) {
        u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t off = (r0 + u) * step + lane_off;
            v[u] = wrole ? buffer_ld16_nt(r, off) : buffer_ld16(r, off);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) a ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
    }
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

extern "C" int bz_shared_read(const void* x, size_t xbytes, const void* w, size_t wchunk, int workgroups,
                              uint32_t key, uint32_t* sink, void* stream) {
    using namespace bz;
    if (!sink || !x || (wchunk && !w) || workgroups < 1) return BZ_ERR_INVALID_ARG;
    if (!xbytes || xbytes % 16 || wchunk % 16 || xbytes > ((size_t)64 << 20) || wchunk > ((size_t)16 << 20))
        return BZ_ERR_SHAPE;
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w)) & 15) return BZ_ERR_ALIGNMENT;
    if (workgroups > 65536) return BZ_ERR_UNSUPPORTED;
    hipLaunchKernelGGL(shared_read_kernel<8>, dim3((unsigned)workgroups), dim3(1024), 0,
                       static_cast<hipStream_t>(stream), static_cast<const uint8_t*>(x), (uint32_t)xbytes,
                       static_cast<const uint8_t*>(w), (uint32_t)wchunk, key, sink);
    return hipGetLastError() == hipSuccess ? BZ_OK : BZ_ERR_LAUNCH;
}
