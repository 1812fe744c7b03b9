// Streaming decode GEMV for gfx950 (MI355X): RMSNorm prologue + int4 / fp8 /
// bf16 weight dequant-dot + SiLU-gate / residual epilogue in ONE launch.
//
// Reference behaviour replaced (models/fused/kernels.py):
//   rms_gemv_kernel      :41-104  partial sums over K slices, norm recomputed
//                                 in every program from the full row of x
//   gemv_epilogue_kernel :107-138 split-K sum, fp8 row scale, SiLU-gate /
//                                 residual epilogue, cast
//   _launch / rms_gemv   :201-219, 334-351
// and the tinygemm / _scaled_mm GEMVs behind Int4Linear / Fp8Linear
// (models/int4_linear.py:99-109, models/fp8_linear.py:68-83).
//
// Work decomposition (one workgroup = one output tile of 8 columns):
//   * Weights are row-major.  A "chunk" is 128 contiguous bytes of one weight
//     row (one cache line).  Lane l of a wave loads 16 bytes (dwordx4) at
//     offset 16*(l%8) of chunk ch of row 8*tile + l/8, so one wave load
//     instruction covers 8 rows x 128 B = 8 full lines.
//   * The chunks of a row are dealt to the NW waves of the workgroup
//     round-robin (chunk ch goes to wave ch % NW); each wave issues all of its
//     NCH (x T) loads before it touches any of them, so ~NCH*T*1 KB per wave
//     is in flight while x is staged.
//   * SiLU-gate tiles own two weight tiles (gate rows j and up rows j + N/2,
//     the [gate; up] concatenation of models/fused/layer.py:60), so the
//     epilogue silu(g)*u needs no second pass.
//   * x (optionally RMS-normalized, rounded to bf16) is staged once per
//     workgroup in LDS; lanes read it back with ds_read_b128.
//   * Per-lane fp32 partials are reduced over the 8 lanes of a row with DPP,
//     then over waves through LDS, in a fixed order (deterministic).
//
// int4 arithmetic: a nibble q becomes the bf16 value 128+q with one
// and-or (exponent 2^7, nibble in the low mantissa bits).  For a lane's 32
// consecutive k (all inside one quantization group, since groups are >= 32
// and aligned), D = sum x_k (128+q_k) comes from 16 v_dot2c_f32_bf16, and
//     sum x_k w_k = s*D + (z - 136 s) * X          ((q-8)*s + z form)
//     sum x_k w_k = s*D + (m - 128 s) * X          (q*s + min form)
// with X = sum x_k over the same 32 k, precomputed per 32-k block while x is
// staged.  The x block is stored permuted [x0 x4 x1 x5 x2 x6 x3 x7] so that
// the (nibble p, nibble p+4) pairs produced by one and-or line up with bf16x2
// pairs of x.
#include <atomic>

#include "bz_device.h"
#include "bz_gemv.h"

namespace bz {

enum { WF_I4ZP = BZ_W_INT4_ZP, WF_I4MIN = BZ_W_INT4_MIN, WF_FP8 = BZ_W_FP8, WF_BF16 = BZ_W_BF16 };

struct GemvParams {
    const uint16_t* x;
    int64_t ldx;
    const uint8_t* w;
    int64_t row_bytes;
    const void* sc0;
    const void* sc1;
    const uint16_t* gamma;
    const void* res;
    int64_t ldr;
    void* out;
    int64_t ldo;
    float eps;
    int N, K, G, glog2, n_out, nchunks;
    int epi, out_f32, res_f32, norm;
};

__host__ __device__ constexpr int align16(int v) { return (v + 15) & ~15; }

// LDS carve-up, shared by the kernel and the host launcher.
struct LdsLayout {
    int xs, xsum, red, nrm, total;
};
__host__ __device__ inline LdsLayout lds_layout(int M, int T, int NW, int K, bool i4) {
    LdsLayout L;
    L.xs = 0;
    L.xsum = align16(M * K * 2);
    L.red = L.xsum + (i4 ? align16(M * (K / 32) * 4) : 0);
    L.nrm = L.red + align16(NW * T * M * 8 * 4);
    L.total = L.nrm + align16(NW * M * 4);
    return L;
}

// Stage x (and the RMSNorm of it) into LDS.  All threads take part.
template <int WF, int M>
__device__ __forceinline__ void stage_x(const GemvParams& p, uint16_t* xs, float* xsum, float* nrm,
                                        int tid, int nthr, int NW, int wave, int lane) {
    constexpr bool I4 = (WF == WF_I4ZP || WF == WF_I4MIN);
    const int nblk = p.K >> 3;  // 8-element (16-byte) blocks per row
    float inv[M];
#pragma unroll
    for (int m = 0; m < M; ++m) inv[m] = 1.0f;
    if (p.norm) {
        float ss[M];
#pragma unroll
        for (int m = 0; m < M; ++m) {
            ss[m] = 0.0f;
            for (int kb = tid; kb < nblk; kb += nthr) {
                const u32x4 v = ldg16(p.x + (int64_t)m * p.ldx + kb * 8);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float a = bf16_lo(v[i]), b = bf16_hi(v[i]);
                    ss[m] += a * a + b * b;
                }
            }
            ss[m] = wave_sum(ss[m]);
            if (lane == 0) nrm[wave * M + m] = ss[m];
        }
        __syncthreads();
#pragma unroll
        for (int m = 0; m < M; ++m) {
            float s = 0.0f;
            for (int w = 0; w < NW; ++w) s += nrm[w * M + m];
            inv[m] = rsqrtf(s / (float)p.K + p.eps);
        }
    }
#pragma unroll
    for (int m = 0; m < M; ++m) {
        for (int kb = tid; kb < nblk; kb += nthr) {
            const u32x4 v = ldg16(p.x + (int64_t)m * p.ldx + kb * 8);
            float f[8];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                f[2 * i] = bf16_lo(v[i]);
                f[2 * i + 1] = bf16_hi(v[i]);
            }
            if (p.norm) {
                const u32x4 g = ldg16(p.gamma + kb * 8);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    f[2 * i] = bf16_to_f32(f32_to_bf16(f[2 * i] * inv[m] * bf16_lo(g[i])));
                    f[2 * i + 1] = bf16_to_f32(f32_to_bf16(f[2 * i + 1] * inv[m] * bf16_hi(g[i])));
                }
            }
            u32x4 o;
            if (I4) {
                o[0] = pack_bf16x2(f[0], f[4]);
                o[1] = pack_bf16x2(f[1], f[5]);
                o[2] = pack_bf16x2(f[2], f[6]);
                o[3] = pack_bf16x2(f[3], f[7]);
                float cs = ((f[0] + f[1]) + (f[2] + f[3])) + ((f[4] + f[5]) + (f[6] + f[7]));
                cs = sum4(cs);  // 4 consecutive blocks = one 32-k block
                if ((kb & 3) == 0) xsum[m * (p.K >> 5) + (kb >> 2)] = cs;
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) o[i] = pack_bf16x2(f[2 * i], f[2 * i + 1]);
            }
            *reinterpret_cast<u32x4*>(xs + m * p.K + kb * 8) = o;
        }
    }
}

template <int M>
__device__ __forceinline__ void unit_int4(const u32x4 q, float s, float zp, const uint16_t* xs, const float* xsum,
                                          int K, int k0, float (&acc)[M]) {
    uint32_t b[4][4];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
#pragma unroll
        for (int sh = 0; sh < 4; ++sh) b[d][sh] = nib2_bf16(q[d] >> (4 * sh));
    }
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const u32x4* xp = reinterpret_cast<const u32x4*>(xs + m * K + k0);
        float d0 = 0.0f, d1 = 0.0f;
#pragma unroll
        for (int d = 0; d < 4; d += 2) {
            const u32x4 xa = xp[d], xb = xp[d + 1];
#pragma unroll
            for (int sh = 0; sh < 4; ++sh) {
                d0 = dot2(b[d][sh], xa[sh], d0);
                d1 = dot2(b[d + 1][sh], xb[sh], d1);
            }
        }
        acc[m] += s * (d0 + d1) + zp * xsum[m * (K >> 5) + (k0 >> 5)];
    }
}

template <int M>
__device__ __forceinline__ void unit_fp8(const u32x4 q, const uint16_t* xs, int K, int k0, float (&acc)[M]) {
    uint32_t b[8];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        b[2 * d] = fp8x2_bf16<false>(q[d]);
        b[2 * d + 1] = fp8x2_bf16<true>(q[d]);
    }
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const u32x4* xp = reinterpret_cast<const u32x4*>(xs + m * K + k0);
        const u32x4 xa = xp[0], xb = xp[1];
        float d0 = 0.0f, d1 = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            d0 = dot2(b[i], xa[i], d0);
            d1 = dot2(b[4 + i], xb[i], d1);
        }
        acc[m] += d0 + d1;
    }
}

template <int M>
__device__ __forceinline__ void unit_bf16(const u32x4 q, const uint16_t* xs, int K, int k0, float (&acc)[M]) {
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const u32x4 xa = *reinterpret_cast<const u32x4*>(xs + m * K + k0);
        float d0 = dot2(q[0], xa[0], 0.0f);
        float d1 = dot2(q[1], xa[1], 0.0f);
        d0 = dot2(q[2], xa[2], d0);
        d1 = dot2(q[3], xa[3], d1);
        acc[m] += d0 + d1;
    }
}

template <int WF, int M, int T, int NCH>
__global__ void __launch_bounds__(1024) gemv_stream(GemvParams p) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    constexpr bool I4 = (WF == WF_I4ZP || WF == WF_I4MIN);
    const int nthr = blockDim.x;
    const int NW = nthr >> 6;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c8 = lane & 7, r = lane >> 3;
    const int col = blockIdx.x * 8 + r;
    const bool rowok = col < p.n_out;

    const LdsLayout L = lds_layout(M, T, NW, p.K, I4);
    uint16_t* xs = reinterpret_cast<uint16_t*>(smem + L.xs);
    float* xsum = reinterpret_cast<float*>(smem + L.xsum);
    float* red = reinterpret_cast<float*>(smem + L.red);
    float* nrm = reinterpret_cast<float*>(smem + L.nrm);

    float acc[T][M];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[t][m] = 0.0f;

    const int step = NW * NCH;
    for (int base = 0; base < p.nchunks; base += step) {
        u32x4 wv[T][NCH];
        uint32_t sa[T][NCH], sb[T][NCH];
        bool ok[NCH];
        // 1. issue every weight (and group scale) load of this pass
#pragma unroll
        for (int j = 0; j < NCH; ++j) {
            const int ch = base + wave + j * NW;
            const int boff = ch * 128 + c8 * 16;
            ok[j] = rowok && ch < p.nchunks && boff < p.row_bytes;
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const int64_t row = col + t * p.n_out;
                sa[t][j] = 0;
                sb[t][j] = 0;
                if (ok[j]) {
                    wv[t][j] = ldg16(p.w + row * p.row_bytes + boff);
                    if (I4) {
                        const int g = (boff * 2) >> p.glog2;
                        if (WF == WF_I4ZP) {
                            sa[t][j] = reinterpret_cast<const uint32_t*>(p.sc0)[(int64_t)g * p.N + row];
                        } else {
                            sa[t][j] = reinterpret_cast<const uint16_t*>(p.sc0)[row * p.G + g];
                            sb[t][j] = reinterpret_cast<const uint16_t*>(p.sc1)[row * p.G + g];
                        }
                    }
                } else {
                    wv[t][j] = u32x4{0u, 0u, 0u, 0u};
                }
            }
        }
        // 2. stage x while the weights are in flight
        if (base == 0) {
            stage_x<WF, M>(p, xs, xsum, nrm, tid, nthr, NW, wave, lane);
            __syncthreads();
        }
        // 3. consume in issue order
#pragma unroll
        for (int j = 0; j < NCH; ++j) {
            if (!ok[j]) continue;
            const int ch = base + wave + j * NW;
            const int boff = ch * 128 + c8 * 16;
#pragma unroll
            for (int t = 0; t < T; ++t) {
                if (I4) {
                    float s, zp;
                    if (WF == WF_I4ZP) {
                        s = bf16_lo(sa[t][j]);
                        zp = bf16_hi(sa[t][j]) - 136.0f * s;
                    } else {
                        s = bf16_lo(sa[t][j]);
                        zp = bf16_lo(sb[t][j]) - 128.0f * s;
                    }
                    unit_int4<M>(wv[t][j], s, zp, xs, xsum, p.K, boff * 2, acc[t]);
                } else if (WF == WF_FP8) {
                    unit_fp8<M>(wv[t][j], xs, p.K, boff, acc[t]);
                } else {
                    unit_bf16<M>(wv[t][j], xs, p.K, boff >> 1, acc[t]);
                }
            }
        }
    }

    // 4. reduce: 8 lanes of a row (DPP), then waves (LDS, fixed order)
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const float v = sum8(acc[t][m]);
            if (c8 == 0) red[((wave * T + t) * M + m) * 8 + r] = v;
        }
    __syncthreads();
    if (tid < M * 8) {
        const int m = tid >> 3, rr = tid & 7;
        const int c = blockIdx.x * 8 + rr;
        if (c < p.n_out) {
            float a[T];
#pragma unroll
            for (int t = 0; t < T; ++t) {
                float s = 0.0f;
                for (int w = 0; w < NW; ++w) s += red[((w * T + t) * M + m) * 8 + rr];
                if (WF == WF_FP8) s *= reinterpret_cast<const float*>(p.sc0)[c + t * p.n_out];
                a[t] = s;
            }
            float o = a[0];
            if (T == 2) o = silu(a[0]) * a[1];
            if (p.epi == BZ_EPI_RESIDUAL) {
                o += p.res_f32 ? reinterpret_cast<const float*>(p.res)[m * p.ldr + c]
                               : bf16_to_f32(reinterpret_cast<const uint16_t*>(p.res)[m * p.ldr + c]);
            }
            if (p.out_f32)
                reinterpret_cast<float*>(p.out)[m * p.ldo + c] = o;
            else
                reinterpret_cast<uint16_t*>(p.out)[m * p.ldo + c] = f32_to_bf16(o);
        }
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

static int device_lds_limit() {
    static std::atomic<int> cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 65536;
    int v = cached[dev].load(std::memory_order_relaxed);
    if (v > 0) return v;
    int lim = 0;
    if (hipDeviceGetAttribute(&lim, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || lim <= 0)
        lim = 65536;
    cached[dev].store(lim, std::memory_order_relaxed);
    return lim;
}

template <int WF, int M, int T, int NCH>
static int launch_stream(const GemvParams& p, int nw, size_t lds, hipStream_t st) {
    auto kern = gemv_stream<WF, M, T, NCH>;
    if (lds > 65536) {
        static std::atomic<bool> raised{false};
        if (!raised.load(std::memory_order_relaxed)) {
            if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                    device_lds_limit()) != hipSuccess)
                return BZ_ERR_LAUNCH;
            raised.store(true, std::memory_order_relaxed);
        }
    }
    dim3 grid((p.n_out + 7) / 8), block(nw * 64);
    hipLaunchKernelGGL(kern, grid, block, lds, st, p);
    return hipGetLastError() == hipSuccess ? BZ_OK : BZ_ERR_LAUNCH;
}

template <int WF, int M, int T>
static int launch_nch(const GemvParams& p, int nch, int nw, size_t lds, hipStream_t st) {
    switch (nch) {
        case 2: return launch_stream<WF, M, T, 2>(p, nw, lds, st);
        case 4: return launch_stream<WF, M, T, 4>(p, nw, lds, st);
        case 8: return launch_stream<WF, M, T, 8>(p, nw, lds, st);
        default: return BZ_ERR_INVALID_ARG;
    }
}

template <int WF, int M>
static int launch_t(const GemvParams& p, int T, int nch, int nw, size_t lds, hipStream_t st) {
    return T == 2 ? launch_nch<WF, M, 2>(p, nch, nw, lds, st) : launch_nch<WF, M, 1>(p, nch, nw, lds, st);
}

template <int WF>
static int launch_m(const GemvParams& p, int M, int T, int nch, int nw, size_t lds, hipStream_t st) {
    switch (M) {
        case 1: return launch_t<WF, 1>(p, T, nch, nw, lds, st);
        case 2: return launch_t<WF, 2>(p, T, nch, nw, lds, st);
        case 3: return launch_t<WF, 3>(p, T, nch, nw, lds, st);
        case 4: return launch_t<WF, 4>(p, T, nch, nw, lds, st);
        default: return BZ_ERR_INVALID_ARG;
    }
}

static int launch_wf(int wf, const GemvParams& p, int M, int T, int nch, int nw, size_t lds, hipStream_t st) {
    switch (wf) {
        case WF_I4ZP: return launch_m<WF_I4ZP>(p, M, T, nch, nw, lds, st);
        case WF_I4MIN: return launch_m<WF_I4MIN>(p, M, T, nch, nw, lds, st);
        case WF_FP8: return launch_m<WF_FP8>(p, M, T, nch, nw, lds, st);
        case WF_BF16: return launch_m<WF_BF16>(p, M, T, nch, nw, lds, st);
        default: return BZ_ERR_INVALID_ARG;
    }
}

static bool aligned(const void* ptr, uintptr_t a) { return (reinterpret_cast<uintptr_t>(ptr) & (a - 1)) == 0; }

// Rows of x handled by one streaming launch (larger M is processed in
// slices of this many rows, each re-streaming the weights).
constexpr int kMaxRowsPerLaunch = 4;

}  // namespace bz

using namespace bz;

extern "C" size_t bz_gemv_workspace(const bz_gemv_desc* d) {
    (void)d;
    return 0;
}

extern "C" int bz_gemv(const bz_gemv_desc* d, void* stream) {
    if (!d) return BZ_ERR_INVALID_ARG;
    if (d->abi_version != BZ_ABI_VERSION) return BZ_ERR_ABI;
    const int M = d->M, N = d->N, K = d->K, wf = d->wfmt, epi = d->epilogue;
    if (M < 1 || N < 1 || K < 1) return BZ_ERR_INVALID_ARG;
    if (wf < BZ_W_INT4_ZP || wf > BZ_W_BF16) return BZ_ERR_INVALID_ARG;
    if (epi < BZ_EPI_NONE || epi > BZ_EPI_RESIDUAL) return BZ_ERR_INVALID_ARG;
    if (d->out_dtype != BZ_DT_BF16 && d->out_dtype != BZ_DT_F32) return BZ_ERR_INVALID_ARG;
    if (!d->x || !d->w || !d->out) return BZ_ERR_INVALID_ARG;
    const bool i4 = (wf == BZ_W_INT4_ZP || wf == BZ_W_INT4_MIN);
    if ((i4 || wf == BZ_W_FP8) && !d->sc0) return BZ_ERR_INVALID_ARG;
    if (wf == BZ_W_INT4_MIN && !d->sc1) return BZ_ERR_INVALID_ARG;
    if (epi == BZ_EPI_RESIDUAL) {
        if (!d->residual) return BZ_ERR_INVALID_ARG;
        if (d->residual_dtype != BZ_DT_BF16 && d->residual_dtype != BZ_DT_F32) return BZ_ERR_INVALID_ARG;
    }
    if (epi == BZ_EPI_SILU_GATE && (N % 2)) return BZ_ERR_SHAPE;
    const int n_out = epi == BZ_EPI_SILU_GATE ? N / 2 : N;
    int glog2 = 0;
    int64_t row_bytes;
    if (i4) {
        const int g = d->group;
        if (g < 32 || (g & (g - 1))) return BZ_ERR_SHAPE;
        if (K % g) return BZ_ERR_SHAPE;
        while ((1 << glog2) < g) ++glog2;
        row_bytes = K / 2;
    } else if (wf == BZ_W_FP8) {
        if (K % 16) return BZ_ERR_SHAPE;
        row_bytes = K;
    } else {
        if (K % 8) return BZ_ERR_SHAPE;
        row_bytes = (int64_t)K * 2;
    }
    if (d->ldx < K || d->ldo < n_out) return BZ_ERR_INVALID_ARG;
    if (epi == BZ_EPI_RESIDUAL && d->ldr < n_out) return BZ_ERR_INVALID_ARG;
    if (!aligned(d->x, 16) || (d->ldx % 8) || !aligned(d->w, 16)) return BZ_ERR_ALIGNMENT;
    if (d->gamma && !aligned(d->gamma, 16)) return BZ_ERR_ALIGNMENT;
    if (wf == BZ_W_INT4_ZP || wf == BZ_W_FP8) {
        if (!aligned(d->sc0, 4)) return BZ_ERR_ALIGNMENT;
    } else if (wf == BZ_W_INT4_MIN) {
        if (!aligned(d->sc0, 2) || !aligned(d->sc1, 2)) return BZ_ERR_ALIGNMENT;
    }
    if (!aligned(d->out, d->out_dtype == BZ_DT_F32 ? 4 : 2)) return BZ_ERR_ALIGNMENT;

    const int T = epi == BZ_EPI_SILU_GATE ? 2 : 1;
    const int nchunks = (int)((row_bytes + 127) / 128);
    int nch = d->cfg_nch, nw = d->cfg_nw;
    if (nch == 0) nch = T == 2 ? 4 : 8;
    if (nch != 2 && nch != 4 && nch != 8) return BZ_ERR_INVALID_ARG;
    if (nw == 0) {
        nw = (nchunks + nch - 1) / nch;
        nw = nw < 1 ? 1 : (nw > 16 ? 16 : nw);
    }
    if (nw < 1 || nw > 16) return BZ_ERR_INVALID_ARG;

    const int mrows = M < kMaxRowsPerLaunch ? M : kMaxRowsPerLaunch;
    const LdsLayout L = lds_layout(mrows, T, nw, K, i4);
    if (L.total > device_lds_limit()) return BZ_ERR_UNSUPPORTED;

    GemvParams p;
    p.w = static_cast<const uint8_t*>(d->w);
    p.row_bytes = row_bytes;
    p.sc0 = d->sc0;
    p.sc1 = d->sc1;
    p.gamma = static_cast<const uint16_t*>(d->gamma);
    p.eps = d->eps;
    p.ldx = d->ldx;
    p.ldr = d->ldr;
    p.ldo = d->ldo;
    p.N = N;
    p.K = K;
    p.G = i4 ? K / d->group : 0;
    p.glog2 = glog2;
    p.n_out = n_out;
    p.nchunks = nchunks;
    p.epi = epi;
    p.out_f32 = d->out_dtype == BZ_DT_F32;
    p.res_f32 = d->residual_dtype == BZ_DT_F32;
    p.norm = d->gamma != nullptr;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const size_t osz = p.out_f32 ? 4 : 2, rsz = p.res_f32 ? 4 : 2;
    for (int m0 = 0; m0 < M; m0 += kMaxRowsPerLaunch) {
        const int mc = (M - m0) < kMaxRowsPerLaunch ? (M - m0) : kMaxRowsPerLaunch;
        p.x = static_cast<const uint16_t*>(d->x) + (int64_t)m0 * d->ldx;
        p.out = static_cast<uint8_t*>(d->out) + (int64_t)m0 * d->ldo * osz;
        p.res = d->residual ? static_cast<const uint8_t*>(d->residual) + (int64_t)m0 * d->ldr * rsz : nullptr;
        const LdsLayout Lc = lds_layout(mc, T, nw, K, i4);
        const int rc = launch_wf(wf, p, mc, T, nch, nw, (size_t)Lc.total, st);
        if (rc != BZ_OK) return rc;
    }
    return BZ_OK;
}
