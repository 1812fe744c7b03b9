// fp32 output heads (gfx950): out[m][n] = sum_k x[m][k] * W[n][k], all fp32,
// for the per-frame heads the reference keeps unquantized and casts to fp32
// (backbone lm_head, models/cudagraph/backbone_graph.py:69-70,273; depth
// BreezeCodebooksHead, models/breeze.py:590-614 with
// models/cudagraph/depth_decoder_graph.py:159-161).
//
// W is one of `nmat` matrices [N][K] (K contiguous) spaced `mat_stride`
// floats apart; the matrix is w + sel * mat_stride with
// sel = *index + index_offset read on the device (index NULL: sel =
// index_offset), so a codebook chosen by a device cache position needs no
// host round trip and can sit in a captured graph.  A selection outside
// [0, nmat) writes zeros.
//
// Layout of the work: x rows (up to kHeadMaxRows per launch) in LDS as fp32,
// loaded into registers before the first weights are requested (vector loads
// retire in order, so staging x then waits for x alone); each wave owns
// kHeadRowsPerWave output rows n and streams them with 16-byte loads (64
// lanes cover 256 k per load), up to 8 such loads per row issued together
// so a 2048-k row takes one memory round trip; fp32 products are summed per
// lane in k order, then across the wave (DPP row sums, rows 0..3 in order).
#include "bz_device.h"
#include "bz_gemv.h"

namespace bz {

constexpr int kHeadThreads = 256;
constexpr int kHeadWaves = kHeadThreads / 64;
constexpr int kHeadRowsPerWave = 2;
constexpr int kHeadMaxRows = 4;                  // x rows per launch
constexpr int kHeadMaxK = 4096;                  // LDS: kHeadMaxRows * K floats <= 64 KB

__device__ __forceinline__ float head_row_sum(float v) {
    v += dpp_f32<kDppXor1>(v);
    v += dpp_f32<kDppXor2>(v);
    v += dpp_f32<0x124>(v);  // row_ror:4
    v += dpp_f32<0x128>(v);  // row_ror:8
    const int b = __float_as_int(v);
    return ((__int_as_float(__builtin_amdgcn_readlane(b, 0)) + __int_as_float(__builtin_amdgcn_readlane(b, 16))) +
            __int_as_float(__builtin_amdgcn_readlane(b, 32))) +
           __int_as_float(__builtin_amdgcn_readlane(b, 48));
}

// S = 256-k loads per row issued together (min(8, K / 256), so no load is
// issued past a row for K a multiple of 256 S; the last chunk of other K
// clamps its indices into the row).
template <int M, int S>
__global__ void __launch_bounds__(kHeadThreads) head_f32_kernel(const float* x, int64_t ldx, int K, const float* w,
                                                               int64_t mat_stride, int nmat, const int64_t* index,
                                                               int64_t index_offset, int N, float* out, int64_t ldo) {
    extern __shared__ float xs[];  // [M][K]
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t sel = (index ? *index : 0) + index_offset;
    const bool ok = sel >= 0 && sel < nmat;
    const float* wm = w + (ok ? sel : 0) * mat_stride;
    const int n0 = (blockIdx.x * kHeadWaves + wave) * kHeadRowsPerWave;  // rows past N load row N - 1

    // 1. x into registers first (float4 e = tid + 256 i: row 4e / K), so
    //    waiting for it does not wait for the weights issued after it
    constexpr int XV = M * kHeadMaxK / (4 * kHeadThreads);
    const int nx = M * (K >> 2);
    float4 xr[XV];
#pragma unroll
    for (int i = 0; i < XV; ++i) {
        const int e = min(tid + i * kHeadThreads, nx - 1);
        const int m = (4 * e) / K;
        xr[i] = *reinterpret_cast<const float4*>(x + m * ldx + (4 * e - m * K));
    }
    // 2. the first chunk of weights (S loads of 256 k per row)
    const float* wrow[kHeadRowsPerWave];
    for (int r = 0; r < kHeadRowsPerWave; ++r) wrow[r] = wm + (int64_t)min(n0 + r, N - 1) * K;
    float4 wv[S][kHeadRowsPerWave];
    auto load_chunk = [&](int k0) {
#pragma unroll
        for (int u = 0; u < S; ++u) {
            const int k = min(k0 + 256 * u + 4 * lane, K - 4);
#pragma unroll
            for (int r = 0; r < kHeadRowsPerWave; ++r) wv[u][r] = *reinterpret_cast<const float4*>(wrow[r] + k);
        }
    };
    load_chunk(0);  // (no scheduling barrier here: one made the compiler spill xr)
    // 3. stage x (clamped entries hold element nx - 1 and store it again:
    //    unconditional stores keep xr in registers)
#pragma unroll
    for (int i = 0; i < XV; ++i) {
        const int e = min(tid + i * kHeadThreads, nx - 1);
        *reinterpret_cast<float4*>(xs + 4 * e) = xr[i];
    }
    __syncthreads();
    if (n0 >= N) return;

    float acc[kHeadRowsPerWave][M];
    for (int r = 0; r < kHeadRowsPerWave; ++r)
        for (int m = 0; m < M; ++m) acc[r][m] = 0.0f;
    for (int k0 = 0; k0 < K; k0 += 256 * S) {
#pragma unroll
        for (int u = 0; u < S; ++u) {
            const int k = k0 + 256 * u + 4 * lane;
            if (k < K) {  // lane-uniform except in a row's last chunk
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    const float4 xv = *reinterpret_cast<const float4*>(xs + m * K + k);
#pragma unroll
                    for (int r = 0; r < kHeadRowsPerWave; ++r)
                        acc[r][m] += wv[u][r].x * xv.x + wv[u][r].y * xv.y + wv[u][r].z * xv.z + wv[u][r].w * xv.w;
                }
            }
        }
        if (k0 + 256 * S < K) {
            load_chunk(k0 + 256 * S);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    for (int r = 0; r < kHeadRowsPerWave; ++r) {
        for (int m = 0; m < M; ++m) {
            const float s = head_row_sum(acc[r][m]);
            if (lane == 0 && n0 + r < N) out[m * ldo + n0 + r] = ok ? s : 0.0f;
        }
    }
}

template <int M>
static void launch_head_m(int steps, dim3 grid, size_t lds, hipStream_t st, const float* x, int64_t ldx, int K,
                          const float* w, int64_t mat_stride, int nmat, const int64_t* index, int64_t index_offset,
                          int N, float* out, int64_t ldo) {
    switch (steps) {
        case 8: hipLaunchKernelGGL((head_f32_kernel<M, 8>), grid, dim3(kHeadThreads), lds, st, x, ldx, K, w, mat_stride, nmat, index, index_offset, N, out, ldo); break;
        case 4: hipLaunchKernelGGL((head_f32_kernel<M, 4>), grid, dim3(kHeadThreads), lds, st, x, ldx, K, w, mat_stride, nmat, index, index_offset, N, out, ldo); break;
        case 2: hipLaunchKernelGGL((head_f32_kernel<M, 2>), grid, dim3(kHeadThreads), lds, st, x, ldx, K, w, mat_stride, nmat, index, index_offset, N, out, ldo); break;
        default: hipLaunchKernelGGL((head_f32_kernel<M, 1>), grid, dim3(kHeadThreads), lds, st, x, ldx, K, w, mat_stride, nmat, index, index_offset, N, out, ldo); break;
    }
}

static void launch_head(int rows, int steps, dim3 grid, size_t lds, hipStream_t st, const float* x, int64_t ldx,
                        int K, const float* w, int64_t mat_stride, int nmat, const int64_t* index,
                        int64_t index_offset, int N, float* out, int64_t ldo) {
    switch (rows) {
        case 1: launch_head_m<1>(steps, grid, lds, st, x, ldx, K, w, mat_stride, nmat, index, index_offset, N, out, ldo); break;
        case 2: launch_head_m<2>(steps, grid, lds, st, x, ldx, K, w, mat_stride, nmat, index, index_offset, N, out, ldo); break;
        case 3: launch_head_m<3>(steps, grid, lds, st, x, ldx, K, w, mat_stride, nmat, index, index_offset, N, out, ldo); break;
        default: launch_head_m<4>(steps, grid, lds, st, x, ldx, K, w, mat_stride, nmat, index, index_offset, N, out, ldo); break;
    }
}

}  // namespace bz

using namespace bz;

extern "C" int bz_head_f32(const float* x, int64_t ldx, int32_t M, int32_t K, const float* w, int32_t N,
                           int64_t mat_stride, int32_t nmat, const int64_t* index, int64_t index_offset, float* out,
                           int64_t ldo, void* stream) {
    if (!x || !w || !out) return BZ_ERR_INVALID_ARG;
    if (M < 1 || N < 1 || K < 1 || nmat < 1 || mat_stride < 0) return BZ_ERR_INVALID_ARG;
    if (nmat > 1 && mat_stride < (int64_t)N * K) return BZ_ERR_SHAPE;
    if (K % 4 || K > kHeadMaxK || ldx < K || ldo < N || ldx % 4 || mat_stride % 4) return BZ_ERR_SHAPE;
    const uintptr_t a = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w);
    if (a & 15) return BZ_ERR_ALIGNMENT;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int per_block = kHeadWaves * kHeadRowsPerWave;
    const dim3 grid((N + per_block - 1) / per_block);
    for (int m0 = 0; m0 < M; m0 += kHeadMaxRows) {
        const int rows = M - m0 < kHeadMaxRows ? M - m0 : kHeadMaxRows;
        const float* xm = x + (int64_t)m0 * ldx;
        float* om = out + (int64_t)m0 * ldo;
        const size_t lds = (size_t)rows * K * sizeof(float);
        const int steps = K >= 2048 ? 8 : (K >= 1024 ? 4 : (K >= 512 ? 2 : 1));
        launch_head(rows, steps, grid, lds, st, xm, ldx, K, w, mat_stride, nmat, index, index_offset, N, om, ldo);
        if (hipGetLastError() != hipSuccess) return BZ_ERR_LAUNCH;
    }
    return BZ_OK;
}
