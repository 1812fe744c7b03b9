// bz_gemv_noalloc: bz_gemv for callers that cannot allocate device memory.
//
// bz_gemv's several-row tile path needs a workspace (split-K partials and the
// arrival counters of its last-arrival sum) that the caller passes in the
// descriptor.  This entry point brings its own: a file-scope device array of
// BZ_GEMV_SCRATCH_BYTES, one copy per GPU the library runs on, held until the
// process ends.  It allocates nothing, so it can be called where hipMalloc is
// not allowed (code under graph capture, serving loops that forbid it).
//
// The array's name is a host-side stand-in, never a device address: each
// device's address comes from hipGetSymbolAddress on the first call made with
// that device current, and only that address is handed to kernels.  The
// counters at the start of the array must be zero when a call begins; the
// first call on a device clears them with a fill kernel on the caller's
// stream (a kernel rather than hipMemsetAsync so that a first call under
// capture records an ordinary kernel node), and every tile-path call leaves
// them zero again when it ends.  All calls on one GPU share its array: calls
// that overlap in time on one GPU race on it.
#include <hip/hip_runtime.h>

#include <mutex>

#include "bz_gemv.h"
#include "bz_gemv_tile.h"

namespace bz {
namespace {

static __device__ __align__(256) uint8_t scratch[BZ_GEMV_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;

struct DeviceScratch {
    uint8_t* ptr = nullptr;  // this device's address of `scratch`
};

std::mutex g_mu;
DeviceScratch g_dev[kMaxDevices];

__global__ void clear_words(uint32_t* p, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

static_assert(kTilePartOffset <= BZ_GEMV_SCRATCH_BYTES, "tile counters must fit the scratch array");

// This device's scratch address, set up (address looked up, counters
// cleared on `st`) by the first call on the device.  BZ_OK or an error.
int device_scratch(hipStream_t st, uint8_t** out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return BZ_ERR_LAUNCH;
    std::lock_guard<std::mutex> lock(g_mu);
    DeviceScratch& ds = g_dev[dev];
    if (!ds.ptr) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return BZ_ERR_LAUNCH;
        const uint32_t words = (uint32_t)(kTilePartOffset / 4);
        hipLaunchKernelGGL(clear_words, dim3((words + 255) / 256), dim3(256), 0, st, static_cast<uint32_t*>(p),
                           words);
        if (hipGetLastError() != hipSuccess) return BZ_ERR_LAUNCH;
        ds.ptr = static_cast<uint8_t*>(p);
    }
    *out = ds.ptr;
    return BZ_OK;
}

}  // namespace
}  // namespace bz

extern "C" int bz_gemv_noalloc(const bz_gemv_desc* d, void* stream) {
    // a malformed descriptor is refused before the first call on a device
    // sets up (and clears) its scratch
    const int rc0 = bz::gemv_check_desc(d);
    if (rc0 != BZ_OK) return rc0;
    if (bz_gemv_workspace(d) > BZ_GEMV_SCRATCH_BYTES) return BZ_ERR_SCRATCH;
    uint8_t* ws = nullptr;
    const int rc = bz::device_scratch(static_cast<hipStream_t>(stream), &ws);
    if (rc != BZ_OK) return rc;
    bz_gemv_desc c = *d;
    c.workspace = ws;
    c.workspace_bytes = BZ_GEMV_SCRATCH_BYTES;
    return bz_gemv(&c, stream);
}
