// The tiled weight formats of the streaming GEMV path (bz_gemv_stream.h):
// sizes, packing from the row-major formats, and dequantization.
//
//   bz_tiled_bytes   chunk size x row blocks
//   bz_pack_tiled    row-major int4 (scales_zeros) / fp8 (row scales) -> tiles;
//                    the load-time counterpart of the reference's repack into
//                    tinygemm's layout (models/int4_linear.py:59), with this
//                    build's own layout
//   dequant_tiled    w_eff (bench_gemv.py:47-52) in logical row order, decoded
//                    with the same arithmetic as the row-major bz_dequant
#include <algorithm>

#include "bz_gemv_stream.h"

namespace bz {

bool is_tiled(int wf) { return wf == WF_I4T || wf == WF_I4TP || wf == WF_F8T || wf == WF_F8TP; }

// Units per row of a tiled weight, or 0 when K cannot be tiled.
int tiled_units(int wf, int K) {
    const int uk = tiled_unit_k(wf);
    return (K > 0 && K % uk == 0) ? K / uk : 0;
}

// Row block and row within it of logical row r of an N-row tiled weight.
__host__ __device__ inline void tiled_row_pos(bool paired, int N, int r, int& blk, int& tr) {
    if (paired) {
        const int h = N >> 1;
        const int rr = r < h ? r : r - h;
        blk = rr >> 3;
        tr = (rr & 7) + (r < h ? 0 : 8);
    } else {
        blk = r >> 4;
        tr = r & 15;
    }
}

// One thread per (source row, unit): 64 bytes of weights and the unit's scale
// pair (int4) or, for unit 0, the row scale (fp8).  The source is row-major
// (BZ_W_INT4_ZP / BZ_W_FP8: n rows) or an unpaired tiled weight of n rows.
__global__ void pack_tiled_kernel(int src_wf, const uint8_t* src, const void* sc0, int n, int K, int dst_wf,
                                  uint8_t* dst, int N, int row0, int NU, int64_t chunk, int64_t src_chunk) {
    const bool i4 = tiled_i4(dst_wf), paired = tiled_paired(dst_wf);
    const bool src_tiled = src_wf == WF_I4T || src_wf == WF_F8T;
    const int64_t row_bytes = i4 ? K / 2 : K;
    const int64_t total = (int64_t)n * NU;
    for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int rs = (int)(idx / NU), u = (int)(idx % NU);
        int blk, tr;
        tiled_row_pos(paired, N, row0 + rs, blk, tr);
        const uint8_t* sb = src_tiled ? src + (rs >> 4) * src_chunk : nullptr;  // source chunk
        const u32x4* s = reinterpret_cast<const u32x4*>(
            src_tiled ? sb + (int64_t)u * 1024 + (rs & 15) * 64 : src + rs * row_bytes + (int64_t)u * 64);
        uint8_t* cb = dst + blk * chunk;
        u32x4* d = reinterpret_cast<u32x4*>(cb + (int64_t)u * 1024 + tr * 64);
#pragma unroll
        for (int q = 0; q < 4; ++q) d[q] = s[q];
        if (i4) {
            *reinterpret_cast<uint32_t*>(cb + (int64_t)NU * 1024 + u * 64 + tr * 4) =
                src_tiled ? *reinterpret_cast<const uint32_t*>(sb + (int64_t)NU * 1024 + u * 64 + (rs & 15) * 4)
                          : reinterpret_cast<const uint32_t*>(sc0)[(int64_t)u * n + rs];
        } else if (u == 0) {
            reinterpret_cast<float*>(cb + (int64_t)NU * 1024)[tr] =
                src_tiled ? reinterpret_cast<const float*>(sb + (int64_t)NU * 1024)[rs & 15]
                          : reinterpret_cast<const float*>(sc0)[rs];
        }
    }
}

// One thread per (logical row, unit, 16-byte piece of the unit).
__global__ void dequant_tiled_kernel(int wf, const uint8_t* w, int N, int K, int NU, int64_t chunk, float* out) {
    const bool i4 = tiled_i4(wf), paired = tiled_paired(wf);
    const int64_t total = (int64_t)N * NU * 4;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const int r = (int)(idx / (NU * 4));
    const int u = (int)((idx / 4) % NU), kq = (int)(idx % 4);
    int blk, tr;
    tiled_row_pos(paired, N, r, blk, tr);
    const uint8_t* cb = w + blk * chunk;
    const u32x4 q = ldg16(cb + (int64_t)u * 1024 + tr * 64 + kq * 16);
    float* o = out + (int64_t)r * K;
    if (i4) {
        const int k0 = u * 128 + kq * 32;
        const uint32_t sz = *reinterpret_cast<const uint32_t*>(cb + (int64_t)NU * 1024 + u * 64 + tr * 4);
        const float s = bf16_lo(sz), zp = bf16_hi(sz);
#pragma unroll
        for (int d = 0; d < 4; ++d) {
#pragma unroll
            for (int sh = 0; sh < 4; ++sh) {
                const uint32_t b = nib2_bf16(q[d] >> (4 * sh));  // 128+q pairs (p, p+4)
                o[k0 + 8 * d + sh] = (bf16_lo(b) - 136.0f) * s + zp;
                o[k0 + 8 * d + sh + 4] = (bf16_hi(b) - 136.0f) * s + zp;
            }
        }
    } else {
        const int k0 = u * 64 + kq * 16;
        const float s = reinterpret_cast<const float*>(cb + (int64_t)NU * 1024)[tr];
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const uint32_t lo = fp8x2_bf16<false>(q[d]), hi = fp8x2_bf16<true>(q[d]);
            o[k0 + 4 * d + 0] = bf16_lo(lo) * s;
            o[k0 + 4 * d + 1] = bf16_hi(lo) * s;
            o[k0 + 4 * d + 2] = bf16_lo(hi) * s;
            o[k0 + 4 * d + 3] = bf16_hi(hi) * s;
        }
    }
}

int dequant_tiled(int wf, const void* w, int N, int K, int group, float* out, hipStream_t st) {
    if (!w || !out || N < 1 || K < 1) return BZ_ERR_INVALID_ARG;
    const int NU = tiled_units(wf, K);
    if (!NU || N % 16 || (tiled_i4(wf) && group != 128)) return BZ_ERR_SHAPE;
    if (reinterpret_cast<uintptr_t>(w) & 15) return BZ_ERR_ALIGNMENT;
    const int64_t total = (int64_t)N * NU * 4;
    hipLaunchKernelGGL(dequant_tiled_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, wf,
                       static_cast<const uint8_t*>(w), N, K, NU, tiled_chunk_bytes(wf, NU), out);
    return hipGetLastError() == hipSuccess ? BZ_OK : BZ_ERR_LAUNCH;
}

}  // namespace bz

using namespace bz;

extern "C" size_t bz_tiled_bytes(int32_t wfmt, int32_t N, int32_t K) {
    if (!is_tiled(wfmt) || N < 16 || N % 16) return 0;
    const int NU = tiled_units(wfmt, K);
    if (!NU) return 0;
    return (size_t)(N / 16) * (size_t)tiled_chunk_bytes(wfmt, NU);
}

extern "C" int bz_pack_tiled(int32_t src_wfmt, const void* src_w, const void* src_sc0, int32_t n, int32_t K,
                             int32_t group, int32_t dst_wfmt, void* dst, int32_t N, int32_t row0, void* stream) {
    if (!src_w || !dst || n < 1 || K < 1 || N < 1 || row0 < 0) return BZ_ERR_INVALID_ARG;
    if (!is_tiled(dst_wfmt)) return BZ_ERR_INVALID_ARG;
    const bool i4 = tiled_i4(dst_wfmt);
    const bool src_tiled = src_wfmt == (i4 ? BZ_W_INT4_TILED : BZ_W_FP8_TILED);
    if (src_wfmt != (i4 ? BZ_W_INT4_ZP : BZ_W_FP8) && !src_tiled) return BZ_ERR_INVALID_ARG;
    if (!src_tiled && !src_sc0) return BZ_ERR_INVALID_ARG;
    if ((int64_t)row0 + n > N) return BZ_ERR_INVALID_ARG;
    const int NU = tiled_units(dst_wfmt, K);
    if (!NU || N % 16 || (src_tiled && n % 16) || (i4 && group != 128)) return BZ_ERR_SHAPE;
    if ((reinterpret_cast<uintptr_t>(src_w) & 15) || (reinterpret_cast<uintptr_t>(dst) & 15) ||
        (!src_tiled && (reinterpret_cast<uintptr_t>(src_sc0) & 3)))
        return BZ_ERR_ALIGNMENT;
    const int64_t total = (int64_t)n * NU;
    const unsigned grid = (unsigned)std::min<int64_t>((total + 255) / 256, 65535);
    hipLaunchKernelGGL(pack_tiled_kernel, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream), src_wfmt,
                       static_cast<const uint8_t*>(src_w), src_sc0, n, K, dst_wfmt, static_cast<uint8_t*>(dst), N,
                       row0, NU, tiled_chunk_bytes(dst_wfmt, NU), tiled_chunk_bytes(src_wfmt, NU));
    return hipGetLastError() == hipSuccess ? BZ_OK : BZ_ERR_LAUNCH;
}
