// Load-time quantizers, dequantization and the two glue kernels of the
// reference's fused path, for gfx950.
//
//   bz_quantize_int4  quantize_int4 (models/int4_linear.py:47-64) and
//                     pack_int4 (models/fused/kernels.py:141-150)
//   bz_quantize_fp8   Fp8Linear.__init__ (models/fp8_linear.py:56-66) and
//                     pack_fp8 (models/fused/kernels.py:153-158)
//   bz_dequant        w_eff of bench_gemv.py:47-52, decoded with the same
//                     helpers the GEMV uses
//   bz_rmsnorm        rmsnorm_kernel (models/fused/kernels.py:541-557)
//   bz_silu_mul       silu_mul_kernel (models/fused/kernels.py:560-575)
//
// The quantizers reproduce the reference's float32 steps one for one
// (IEEE divide, round-half-even), so their outputs are bit-identical to the
// torch formulas they restate.
#include "bz_device.h"
#include "bz_gemv.h"

namespace bz {

// the tiled formats' dequantization (bz_tiled.hip)
bool is_tiled(int wf);
int dequant_tiled(int wf, const void* w, int N, int K, int group, float* out, hipStream_t st);

__device__ __forceinline__ float load_w(const void* w, int dtype, int64_t i) {
    return dtype == BZ_DT_F32 ? reinterpret_cast<const float*>(w)[i]
                              : bf16_to_f32(reinterpret_cast<const uint16_t*>(w)[i]);
}

// float -> OCP e4m3 code, round to nearest, ties to even.  |v| <= 448 or NaN.
// Normal range: round the float32 mantissa to 3 bits in the integer domain
// (adding 0x7FFFF plus the kept LSB gives ties-to-even), then rebias the
// exponent from 127 to 7.  Below 2^-6 the code is rne(|v| * 2^9) (exact
// scaling), which also rounds up into the smallest normal (code 8).
__device__ __forceinline__ uint8_t e4m3_encode(float v) {
    const uint32_t u = __float_as_uint(v);
    const uint32_t sign = (u >> 24) & 0x80u;
    const uint32_t a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return (uint8_t)(sign | 0x7Fu);
    if (a < 0x3C800000u) {  // 2^-6
        const float t = __uint_as_float(a) * 512.0f;
        return (uint8_t)(sign | (uint32_t)rintf(t));
    }
    const uint32_t r = (a + 0x7FFFFu + ((a >> 20) & 1u)) >> 20;
    return (uint8_t)(sign | (r - (120u << 3)));
}

// One thread per (row n, group g).
__global__ void quantize_int4_kernel(const void* w, int dtype, int N, int K, int group, int symmetric, int layout,
                                     uint8_t* packed, void* sc0, void* sc1) {
    const int G = K / group;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)N * G) return;
    const int n = (int)(idx / G), g = (int)(idx % G);
    const int64_t base = (int64_t)n * K + (int64_t)g * group;
    float s, zq, lo = 0.0f;
    if (!symmetric) {
        float mn = load_w(w, dtype, base), mx = mn;
        for (int i = 1; i < group; ++i) {
            const float v = load_w(w, dtype, base + i);
            mn = fminf(mn, v);
            mx = fmaxf(mx, v);
        }
        lo = mn;
        s = fmaxf((mx - mn) / 15.0f, 1e-8f);
        zq = mn + 8.0f * s;  // 8*s is exact: one rounding, as torch
    } else {
        float am = 0.0f;
        for (int i = 0; i < group; ++i) am = fmaxf(am, fabsf(load_w(w, dtype, base + i)));
        s = fmaxf(am / 7.0f, 1e-8f);
        zq = 0.0f;
        lo = -8.0f * s;
    }
    uint8_t* dst = packed + (int64_t)n * (K / 2) + (int64_t)g * (group / 2);
    for (int i = 0; i < group; i += 2) {
        uint32_t q2[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const float v = load_w(w, dtype, base + i + e);
            float qf = symmetric ? rintf(v / s) + 8.0f : rintf((v - lo) / s);
            qf = fminf(fmaxf(qf, 0.0f), 15.0f);
            q2[e] = (uint32_t)qf;
        }
        dst[i / 2] = (uint8_t)(q2[0] | (q2[1] << 4));
    }
    if (layout == BZ_W_INT4_ZP) {
        uint16_t* sz = reinterpret_cast<uint16_t*>(sc0);
        const int64_t o = ((int64_t)g * N + n) * 2;
        sz[o] = f32_to_bf16(s);
        sz[o + 1] = f32_to_bf16(zq);
    } else {
        reinterpret_cast<uint16_t*>(sc0)[(int64_t)n * G + g] = f32_to_bf16(s);
        reinterpret_cast<uint16_t*>(sc1)[(int64_t)n * G + g] = f32_to_bf16(lo);
    }
}

// One 256-thread workgroup per row.
__global__ void __launch_bounds__(256) quantize_fp8_kernel(const void* w, int dtype, int K, float floor_,
                                                           uint8_t* codes, float* scale) {
    __shared__ float part[4];
    const int n = blockIdx.x, tid = threadIdx.x;
    const int64_t base = (int64_t)n * K;
    float am = 0.0f;
    for (int k = tid; k < K; k += 256) am = fmaxf(am, fabsf(load_w(w, dtype, base + k)));
    am = wave_max(am);
    if ((tid & 63) == 0) part[tid >> 6] = am;
    __syncthreads();
    am = fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3]));
    const float sc = fmaxf(am, floor_) / 448.0f;
    if (tid == 0) scale[n] = sc;
    for (int k = tid; k < K; k += 256) {
        const float v = fminf(fmaxf(load_w(w, dtype, base + k) / sc, -448.0f), 448.0f);
        codes[base + k] = e4m3_encode(v);
    }
}

// One thread per 16-byte chunk of a weight row, using the GEMV's decoders.
__global__ void dequant_kernel(int wf, const uint8_t* w, const void* sc0, const void* sc1, int N, int K, int group,
                               float* out) {
    const bool i4 = (wf == BZ_W_INT4_ZP || wf == BZ_W_INT4_MIN);
    const int64_t row_bytes = i4 ? K / 2 : (wf == BZ_W_FP8 ? K : (int64_t)K * 2);
    const int64_t per_row = row_bytes / 16;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)N * per_row) return;
    const int64_t n = idx / per_row, c = idx % per_row;
    const u32x4 q = ldg16(w + n * row_bytes + c * 16);
    float* o = out + n * K;
    if (i4) {
        const int k0 = (int)(c * 32);
        const int g = k0 / group, G = K / group;
        float s, zp;
        if (wf == BZ_W_INT4_ZP) {
            const uint32_t sz = reinterpret_cast<const uint32_t*>(sc0)[(int64_t)g * N + n];
            s = bf16_lo(sz);
            zp = bf16_hi(sz);
        } else {
            s = bf16_to_f32(reinterpret_cast<const uint16_t*>(sc0)[n * G + g]);
            zp = bf16_to_f32(reinterpret_cast<const uint16_t*>(sc1)[n * G + g]);
        }
        const float off = wf == BZ_W_INT4_ZP ? 136.0f : 128.0f;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
#pragma unroll
            for (int sh = 0; sh < 4; ++sh) {
                const uint32_t b = nib2_bf16(q[d] >> (4 * sh));  // 128+q pairs (p, p+4)
                o[k0 + 8 * d + sh] = (bf16_lo(b) - off) * s + zp;
                o[k0 + 8 * d + sh + 4] = (bf16_hi(b) - off) * s + zp;
            }
        }
    } else if (wf == BZ_W_FP8) {
        const int k0 = (int)(c * 16);
        const float s = reinterpret_cast<const float*>(sc0)[n];
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const uint32_t lo = fp8x2_bf16<false>(q[d]), hi = fp8x2_bf16<true>(q[d]);
            o[k0 + 4 * d + 0] = bf16_lo(lo) * s;
            o[k0 + 4 * d + 1] = bf16_hi(lo) * s;
            o[k0 + 4 * d + 2] = bf16_lo(hi) * s;
            o[k0 + 4 * d + 3] = bf16_hi(hi) * s;
        }
    } else {
        const int k0 = (int)(c * 8);
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            o[k0 + 2 * d] = bf16_lo(q[d]);
            o[k0 + 2 * d + 1] = bf16_hi(q[d]);
        }
    }
}

// One 256-thread workgroup per row.
__global__ void __launch_bounds__(256) rmsnorm_kernel(const uint16_t* x, int64_t ldx, const uint16_t* gamma, float eps,
                                                      uint16_t* out, int64_t ldo, int K) {
    __shared__ float part[4];
    const int m = blockIdx.x, tid = threadIdx.x;
    const uint16_t* xr = x + m * ldx;
    float ss = 0.0f;
    for (int k = tid; k < K; k += 256) {
        const float v = bf16_to_f32(xr[k]);
        ss += v * v;
    }
    ss = wave_sum(ss);
    if ((tid & 63) == 0) part[tid >> 6] = ss;
    __syncthreads();
    const float inv = rsqrtf(((part[0] + part[1]) + (part[2] + part[3])) / (float)K + eps);
    for (int k = tid; k < K; k += 256)
        out[m * ldo + k] = f32_to_bf16(bf16_to_f32(xr[k]) * inv * bf16_to_f32(gamma[k]));
}

__global__ void silu_mul_kernel(const uint16_t* g, int64_t ldg, const uint16_t* u, int64_t ldu, uint16_t* out,
                                int64_t ldo, int N) {
    const int m = blockIdx.y;
    const int n = blockIdx.x * blockDim.x + threadIdx.x;
    if (n >= N) return;
    const float gv = bf16_to_f32(g[m * ldg + n]);
    out[m * ldo + n] = f32_to_bf16(silu(gv) * bf16_to_f32(u[m * ldu + n]));
}

static int launched() { return hipGetLastError() == hipSuccess ? BZ_OK : BZ_ERR_LAUNCH; }

}  // namespace bz

using namespace bz;

extern "C" int bz_abi_version(void) { return BZ_ABI_VERSION; }

extern "C" const char* bz_strerror(int status) {
    switch (status) {
        case BZ_OK: return "ok";
        case BZ_ERR_INVALID_ARG: return "invalid argument";
        case BZ_ERR_SHAPE: return "unsupported shape (K not divisible by group / format step)";
        case BZ_ERR_ALIGNMENT: return "pointer or leading dimension not aligned";
        case BZ_ERR_UNSUPPORTED: return "request exceeds what this build supports";
        case BZ_ERR_LAUNCH: return "kernel launch failed";
        case BZ_ERR_ABI: return "descriptor abi_version mismatch";
        case BZ_ERR_SCRATCH: return "call needs more workspace than the static scratch (BZ_GEMV_SCRATCH_BYTES)";
        default: return "unknown status";
    }
}

extern "C" int bz_stream_capture(void* stream, int32_t* active, uint64_t* id) {
    if (!active || !id) return BZ_ERR_INVALID_ARG;
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    unsigned long long cid = 0;
    if (hipStreamGetCaptureInfo(static_cast<hipStream_t>(stream), &status, &cid) != hipSuccess) return BZ_ERR_LAUNCH;
    *active = status == hipStreamCaptureStatusActive ? 1 : 0;
    *id = *active ? (uint64_t)cid : 0;
    return BZ_OK;
}

extern "C" int bz_rmsnorm(const void* x, int64_t ldx, const void* gamma, float eps, void* out, int64_t ldo, int32_t M,
                          int32_t K, void* stream) {
    if (!x || !gamma || !out || M < 1 || K < 1 || ldx < K || ldo < K) return BZ_ERR_INVALID_ARG;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(M), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint16_t*>(x), ldx, static_cast<const uint16_t*>(gamma), eps,
                       static_cast<uint16_t*>(out), ldo, K);
    return launched();
}

extern "C" int bz_silu_mul(const void* g, int64_t ldg, const void* u, int64_t ldu, void* out, int64_t ldo, int32_t M,
                           int32_t N, void* stream) {
    if (!g || !u || !out || M < 1 || N < 1 || ldg < N || ldu < N || ldo < N) return BZ_ERR_INVALID_ARG;
    hipLaunchKernelGGL(silu_mul_kernel, dim3((N + 255) / 256, M), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint16_t*>(g), ldg, static_cast<const uint16_t*>(u), ldu,
                       static_cast<uint16_t*>(out), ldo, N);
    return launched();
}

extern "C" int bz_quantize_int4(const void* w, int32_t w_dtype, int32_t N, int32_t K, int32_t group, int32_t symmetric,
                                int32_t layout, void* packed, void* sc0, void* sc1, void* stream) {
    if (!w || !packed || !sc0 || N < 1 || K < 1) return BZ_ERR_INVALID_ARG;
    if (w_dtype != BZ_DT_F32 && w_dtype != BZ_DT_BF16) return BZ_ERR_INVALID_ARG;
    if (layout != BZ_W_INT4_ZP && layout != BZ_W_INT4_MIN) return BZ_ERR_INVALID_ARG;
    if (layout == BZ_W_INT4_MIN && !sc1) return BZ_ERR_INVALID_ARG;
    if (group < 2 || (group % 2) || K % group) return BZ_ERR_SHAPE;
    const int64_t total = (int64_t)N * (K / group);
    hipLaunchKernelGGL(quantize_int4_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), w, w_dtype, N, K, group, symmetric, layout,
                       static_cast<uint8_t*>(packed), sc0, sc1);
    return launched();
}

extern "C" int bz_quantize_fp8(const void* w, int32_t w_dtype, int32_t N, int32_t K, float amax_floor, void* codes,
                               void* scale, void* stream) {
    if (!w || !codes || !scale || N < 1 || K < 1) return BZ_ERR_INVALID_ARG;
    if (w_dtype != BZ_DT_F32 && w_dtype != BZ_DT_BF16) return BZ_ERR_INVALID_ARG;
    hipLaunchKernelGGL(quantize_fp8_kernel, dim3(N), dim3(256), 0, static_cast<hipStream_t>(stream), w, w_dtype, K,
                       amax_floor, static_cast<uint8_t*>(codes), static_cast<float*>(scale));
    return launched();
}

extern "C" int bz_dequant(int32_t wfmt, const void* w, const void* sc0, const void* sc1, int32_t N, int32_t K,
                          int32_t group, void* out, void* stream) {
    if (!w || !out || N < 1 || K < 1) return BZ_ERR_INVALID_ARG;
    if (is_tiled(wfmt))
        return dequant_tiled(wfmt, w, N, K, group, static_cast<float*>(out), static_cast<hipStream_t>(stream));
    if (wfmt < BZ_W_INT4_ZP || wfmt > BZ_W_BF16) return BZ_ERR_INVALID_ARG;
    const bool i4 = (wfmt == BZ_W_INT4_ZP || wfmt == BZ_W_INT4_MIN);
    if ((i4 || wfmt == BZ_W_FP8) && !sc0) return BZ_ERR_INVALID_ARG;
    if (wfmt == BZ_W_INT4_MIN && !sc1) return BZ_ERR_INVALID_ARG;
    if (i4 && (group < 32 || (group & (group - 1)) || K % group)) return BZ_ERR_SHAPE;
    if (wfmt == BZ_W_FP8 && K % 16) return BZ_ERR_SHAPE;
    if (wfmt == BZ_W_BF16 && K % 8) return BZ_ERR_SHAPE;
    if ((reinterpret_cast<uintptr_t>(w) & 15)) return BZ_ERR_ALIGNMENT;
    const int64_t row_bytes = i4 ? K / 2 : (wfmt == BZ_W_FP8 ? K : (int64_t)K * 2);
    const int64_t total = (int64_t)N * (row_bytes / 16);
    hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), wfmt, static_cast<const uint8_t*>(w), sc0, sc1, N, K, group,
                       static_cast<float*>(out));
    return launched();
}
