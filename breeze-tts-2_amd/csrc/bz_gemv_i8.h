// Integer matrix-core variant of the streaming decode GEMV for int4 weights
// (gfx950 v_mfma_i32_16x16x64_i8).
//
// Same contract, work decomposition and register pipeline as gemv_mfma
// (bz_gemv_mfma.h): 16-column tiles, 64-byte units of each row (128 k, one
// quantization group for group >= 128), lane l loading 16 bytes of row l%16
// at offset 16*(l/16) of the unit.  What changes is the arithmetic, which is
// the cost that bounds the bf16 paths at M = 1:
//   * weights: the lane's 32 nibbles become two int8 B operands with three
//     VALU ops per 8 nibbles:  even k = w & 0x0F0F0F0F,
//     odd k = (w >> 4) & 0x0F0F0F0F  (q in 0..15, no bias, no float);
//   * x: each 128-k unit of each row is scaled by its own s_x = absmax/127
//     and split into two int8 planes, u = s_x * (hi + lo/254) (|error| <=
//     s_x/508: about 16 significant bits relative to the unit's largest
//     value, so an outlier channel costs precision only within its own
//     unit), staged in LDS in the even/odd k order of the B operands;
//   * per unit and tile: D_hi = A_hi . B (2 MFMAs, even and odd k), D_lo
//     likewise; sum u*w = s * s_x * (D_hi + D_lo/254) + zp * X, with
//     zp = z - 8s ((q-8)*s + z form) or min (q*s + min form) and X = sum of
//     u over the unit (fp32).
// MFMA operand layout (verified on gfx950): A[i][k] in lane i + 16*(k/16),
// byte k%16; B[k][j] in lane j + 16*(k/16), byte k%16; D[i][j] in lane
// j + 16*(i/4), element i%4.  MFMA k index kk of a unit maps to unit-local
// k = 2*kk (even plane) or 2*kk + 1 (odd plane).
//
// x rows: up to 16 per launch (the A operand's 16 rows); M is a runtime value
// and MQ = min(M, 4) (the rows one lane's accumulator can hold) a template
// parameter.
#pragma once
#include "bz_gemv_mfma.h"

namespace bz {

typedef int32_t i32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ i32x4_t mfma_i8(const u32x4 a, const u32x4 b, i32x4_t c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4_t, a), __builtin_bit_cast(i32x4_t, b), c,
                                                 0, 0, 0);
}

// LDS of the int8 kernel.  x8: per unit u, per kb (32-k quarter of the unit),
// per plane (0: hi even k, 1: hi odd k, 2: lo even k, 3: lo odd k), per row m:
// 16 bytes, so the 16 lanes of one kb read 16 consecutive 16-byte rows (no
// bank conflict).  xsx: per (row, unit) (s_x, sum of u, sum of x^2, -).
// inv: per row 1/rms (epilogue).
struct I8Lds {
    int x8, xsx, red, inv, total;
};
__host__ __device__ inline I8Lds i8_lds_layout(int M, int T, int NW, int K, int tpw) {
    const int units = K / 128;
    I8Lds L;
    L.x8 = 0;
    L.xsx = align16(units * 4 * 4 * M * 16);
    L.red = L.xsx + M * units * 16;
    L.inv = L.red + align16(tpw * NW * T * M * 16 * 4);
    L.total = L.inv + align16(M * 4);
    return L;
}

// Rows of x one launch of the int8 kernel may take for K (its LDS holds 2
// bytes of x per element next to the partial sums).
__host__ __device__ inline int i8_max_rows(int K, int lds_limit, int T, int NW, int tpw) {
    for (int m = 16; m >= 1; --m)
        if (i8_lds_layout(m, T, NW, K, tpw).total <= lds_limit) return m;
    return 0;
}

// Max over each aligned group of 16 lanes; every lane of the group gets it.
__device__ __forceinline__ float max16(float v) {
    v = fmaxf(v, __shfl_xor(v, 1, 64));
    v = fmaxf(v, __shfl_xor(v, 2, 64));
    v = fmaxf(v, __shfl_xor(v, 4, 64));
    return fmaxf(v, __shfl_xor(v, 8, 64));
}

// Quantize block b (8 consecutive k: unit b/16, quarter kb = (b/4)%4, eighth
// s = b%4 of the quarter) of row m.  The unit's 16 blocks sit in 16
// consecutive lanes, which agree on the unit's scale with a 16-lane max; each
// block stores 4 bytes in each of the four planes.  Lane 0 of the 16 stores
// the unit's (s_x, sum of u, sum of x^2).
__device__ __forceinline__ void i8_stage_block(const float (&f)[8], float x2, int m, int M, int b, uint8_t* x8,
                                               float* xsx, int units) {
    const int unit = b >> 4, kb = (b >> 2) & 3, s = b & 3;
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) mx = fmaxf(mx, fabsf(f[i]));
    mx = max16(mx);
    const float sx = mx > 0.0f ? mx * (1.0f / 127.0f) : 1.0f;
    const float isx = 1.0f / sx;
    uint32_t hi_e = 0, hi_o = 0, lo_e = 0, lo_o = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float t = f[i] * isx;
        const float h = rintf(t);
        const float l = rintf((t - h) * 254.0f);
        const uint32_t hb = (uint32_t)(int)h & 0xFFu, lb = (uint32_t)(int)l & 0xFFu;
        const int sh = 8 * (i >> 1);
        if (i & 1) {
            hi_o |= hb << sh;
            lo_o |= lb << sh;
        } else {
            hi_e |= hb << sh;
            lo_e |= lb << sh;
        }
    }
    uint8_t* dst = x8 + ((unit * 4 + kb) * 4 * M + m) * 16 + 4 * s;
    *reinterpret_cast<uint32_t*>(dst) = hi_e;
    *reinterpret_cast<uint32_t*>(dst + 1 * M * 16) = hi_o;
    *reinterpret_cast<uint32_t*>(dst + 2 * M * 16) = lo_e;
    *reinterpret_cast<uint32_t*>(dst + 3 * M * 16) = lo_o;
    float cs = ((f[0] + f[1]) + (f[2] + f[3])) + ((f[4] + f[5]) + (f[6] + f[7]));
    cs = sum16(cs);
    x2 = sum16(x2);
    if ((b & 15) == 0) *reinterpret_cast<float4*>(xsx + (m * units + unit) * 4) = make_float4(sx, cs, x2, 0.0f);
}

// x prologue: u = bf16(gamma * x) (or x) per block, quantized into the
// planes with its unit's statistics.  Blocks beyond the kXB per thread kept
// in registers are reloaded (L2 hits).  Rows: runtime M <= 16.
__device__ __forceinline__ void i8_finish_x(const GemvParams& p, int M, const u32x4 (&xr)[kXB],
                                            const u32x4 (&gr)[kXB], uint8_t* x8, float* xsx, int tid, int nthr) {
    const int nblk = p.K >> 3, total = M * nblk, units = p.K >> 7;
    auto stage = [&](u32x4 v, u32x4 g, int b) {
        const int m = b / nblk;
        float f[8];
        block_values(p, v, g, f);
        float x2 = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float a = bf16_lo(v[i]), c = bf16_hi(v[i]);
            x2 += a * a + c * c;
        }
        i8_stage_block(f, x2, m, M, b - m * nblk, x8, xsx, units);
    };
#pragma unroll
    for (int i = 0; i < kXB; ++i) {
        const int b = tid + i * nthr;
        if (b < total) stage(xr[i], gr[i], b);
    }
    for (int b = tid + kXB * nthr; b < total; b += nthr) {
        const int m = b / nblk;
        const int kb = b - m * nblk;
        const u32x4 v = ldg16(p.x + (int64_t)m * p.ldx + kb * 8);
        const u32x4 g = p.norm ? ldg16(p.gamma + kb * 8) : v;
        stage(v, g, b);
    }
}

// Issue x loads for up to M rows (runtime M).
__device__ __forceinline__ void i8_issue_x(const GemvParams& p, int M, int tid, int nthr, u32x4 (&xr)[kXB],
                                           u32x4 (&gr)[kXB]) {
    const int nblk = p.K >> 3, total = M * nblk;
#pragma unroll
    for (int i = 0; i < kXB; ++i) {
        const int b = min(tid + i * nthr, total - 1);
        const int m = b / nblk;
        const int kb = b - m * nblk;
        xr[i] = ldg16(p.x + (int64_t)m * p.ldx + kb * 8);
        gr[i] = p.norm ? ldg16(p.gamma + kb * 8) : u32x4{0u, 0u, 0u, 0u};
    }
}

// One unit: 4 ds_read_b128 of the A planes (shared by the T tiles), then per
// tile the nibble split and 4 MFMAs, and the group scaling into fp32.
template <int WF, int MQ, int T>
__device__ __forceinline__ void i8_consume_unit(const GemvParams& p, StepCursor c, int M, int j, int kb,
                                                const uint8_t* x8, const float* xsx, const u32x4 (&buf)[T],
                                                const uint32_t (&scv)[T], f32x4_t (&acc)[T]) {
    const int u = c.ch;
    const int units = p.K >> 7;
    const int am = min(j, M - 1);  // x row this lane supplies to the A operand
    const uint8_t* xa = x8 + ((u * 4 + kb) * 4 * M + am) * 16;
    const u32x4 a_he = *reinterpret_cast<const u32x4*>(xa);
    const u32x4 a_ho = *reinterpret_cast<const u32x4*>(xa + 1 * M * 16);
    const u32x4 a_le = *reinterpret_cast<const u32x4*>(xa + 2 * M * 16);
    const u32x4 a_lo = *reinterpret_cast<const u32x4*>(xa + 3 * M * 16);
    float X[MQ], SX[MQ];
#pragma unroll
    for (int q = 0; q < MQ; ++q) {
        const float2 e = *reinterpret_cast<const float2*>(xsx + (min(4 * kb + q, M - 1) * units + u) * 4);
        SX[q] = e.x;
        X[q] = e.y;
    }
#pragma unroll
    for (int t = 0; t < T; ++t) {
        u32x4 be, bo;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            be[i] = buf[t][i] & 0x0F0F0F0Fu;
            bo[i] = (buf[t][i] >> 4) & 0x0F0F0F0Fu;
        }
        i32x4_t dh = {0, 0, 0, 0}, dl = {0, 0, 0, 0};
        dh = mfma_i8(a_he, be, dh);
        dh = mfma_i8(a_ho, bo, dh);
        dl = mfma_i8(a_le, be, dl);
        dl = mfma_i8(a_lo, bo, dl);
        const uint32_t e = scv[t];
        const float s = bf16_lo(e);
        const float zp = WF == WF_I4ZP ? bf16_hi(e) - 8.0f * s : bf16_hi(e);
#pragma unroll
        for (int q = 0; q < MQ; ++q) {
            const float dq = (float)dh[q] + (float)dl[q] * (1.0f / 254.0f);
            acc[t][q] += (s * SX[q]) * dq + zp * X[q];
        }
    }
}

template <int WF, int MQ, int T, int D, bool SILU>
__global__ void __launch_bounds__(kMaxThreads) gemv_i8mma(BZ_GEMV_HOT_PARAMS, GemvParams p, int M) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    gemv_hot(p, hx, hw, hsc0, hgamma, hldx, hrow_bytes, hK, hN, hntiles, htpw);
    const int nthr = blockDim.x;
    const int NW = nthr >> 6;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 15, kb = lane >> 4;
    const int nunits = (int)(p.row_bytes / 64);  // K % 128 == 0 on this path
    const TileRange tr(p.ntiles);
    const int tile0 = tr.tile0, ntl = tr.ntl;
    const int S = wave_steps(ntl, nunits, NW, wave);  // host ensures NW <= nunits

    const I8Lds L = i8_lds_layout(M, T, NW, p.K, p.tpw);
    uint8_t* x8 = smem + L.x8;
    float* xsx = reinterpret_cast<float*>(smem + L.xsx);
    float* red = reinterpret_cast<float*>(smem + L.red);
    float* invs = reinterpret_cast<float*>(smem + L.inv);

    u32x4 buf[D][T];
    uint32_t scb[D][T];
    auto issue = [&](int d, StepCursor c) { issue_unit<WF, T, SILU>(p, c, tile0, j, kb, buf[d], scb[d]); };

    // 0. x (and gamma) loads first, then the first D units of weights
    u32x4 xr[kXB], gr[kXB];
    i8_issue_x(p, M, tid, nthr, xr, gr);
    __builtin_amdgcn_sched_barrier(0);
    StepCursor ic{0, wave};
    pipeline_prime<0, D>(S, NW, nunits, wave, ic, issue);
    __builtin_amdgcn_sched_barrier(0);
    // 1. x in int8 planes (with per-unit scales) while the weights are in
    //    flight
    i8_finish_x(p, M, xr, gr, x8, xsx, tid, nthr);
    __syncthreads();
    // 1/rms per row from the units' sums of x^2, in unit order, while the
    // first weights are in flight (read after the epilogue's barrier)
    if (tid < M) {
        float inv = 1.0f;
        if (p.norm) {
            const int units = p.K >> 7;
            const float* sq = xsx + tid * units * 4 + 2;
            float ss = 0.0f;
            for (int u0 = 0; u0 < units; u0 += 8)  // 8 reads in flight, one running sum in unit order
                ss = sum_strided<8>(sq + u0 * 4, 4, min(8, units - u0), ss);
            inv = rsqrtf(ss / (float)p.K + p.eps);
        }
        invs[tid] = inv;
    }

    // 2. every unit once
    f32x4_t acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    pipeline_run<D>(S, NW, nunits, wave, ic, issue, [&](int d, StepCursor c) {
        i8_consume_unit<WF, MQ, T>(p, c, M, j, kb, x8, xsx, buf[d], scb[d], acc);
        if (c.last_in_tile(NW, nunits)) {
#pragma unroll
            for (int t = 0; t < T; ++t) {
#pragma unroll
                for (int q = 0; q < MQ; ++q) {
                    const int m = 4 * kb + q;
                    if (m < M) red[(((c.tl * NW + wave) * T + t) * M + m) * 16 + j] = acc[t][q];
                }
                acc[t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
            }
        }
    });
    __syncthreads();

    // 3. epilogue (runtime M): fixed-order sum of the waves' partials, 1/rms,
    //    SiLU-gate or residual, store
    for (int i = tid; i < ntl * M * 16; i += nthr) {
        const int tl = i / (M * 16);
        const int m = (i >> 4) % M, q = i & 15;
        const int col = (tile0 + tl) * 16 + q;
        if (col >= p.n_out) continue;
        const float inv = invs[m];
        float a[T];
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const float v = sum_strided<kMaxWaves>(red + ((tl * NW * T + t) * M + m) * 16 + q, T * M * 16, NW);
            a[t] = v * inv;
        }
        float o = SILU ? silu(a[0]) * a[T - 1] : a[0];
        const int64_t ri = (int64_t)m * p.ldr + col;
        if (p.epi == BZ_EPI_RESIDUAL)
            o += p.res_f32 ? reinterpret_cast<const float*>(p.res)[ri]
                           : bf16_to_f32(reinterpret_cast<const uint16_t*>(p.res)[ri]);
        const int64_t oi = (int64_t)m * p.ldo + col;
        if (p.out_f32)
            reinterpret_cast<float*>(p.out)[oi] = o;
        else
            reinterpret_cast<uint16_t*>(p.out)[oi] = f32_to_bf16(o);
    }
}

template <int WF, int MQ, int T, int D, bool SILU>
int launch_i8_kernel(const GemvParams& p, const Launch& l, hipStream_t st) {
    auto kern = gemv_i8mma<WF, MQ, T, D, SILU>;
    if (l.lds > 65536 && raise_lds_limit(reinterpret_cast<const void*>(kern)) != BZ_OK) return BZ_ERR_LAUNCH;
    if (!gemv_hot_ok(p)) return BZ_ERR_UNSUPPORTED;
    hipLaunchKernelGGL(kern, dim3(l.grid), dim3(l.nw * 64), l.lds, st, BZ_GEMV_HOT_ARGS(p), p, l.M);
    return hipGetLastError() == hipSuccess ? BZ_OK : BZ_ERR_LAUNCH;
}

template <int WF, int MQ, bool SILU>
int launch_i8_depth(const GemvParams& p, const Launch& l, hipStream_t st) {
    constexpr int T = SILU ? 2 : 1;
    switch (l.depth) {
        case 2: return launch_i8_kernel<WF, MQ, T, 2, SILU>(p, l, st);
        case 4: return launch_i8_kernel<WF, MQ, T, 4, SILU>(p, l, st);
        case 8: return launch_i8_kernel<WF, MQ, T, 8, SILU>(p, l, st);
        default: return BZ_ERR_INVALID_ARG;
    }
}

template <int WF>
int launch_i8_m(const GemvParams& p, const Launch& l, hipStream_t st) {
    switch (l.M < 4 ? l.M : 4) {
        case 1: return l.silu ? launch_i8_depth<WF, 1, true>(p, l, st) : launch_i8_depth<WF, 1, false>(p, l, st);
        case 2: return l.silu ? launch_i8_depth<WF, 2, true>(p, l, st) : launch_i8_depth<WF, 2, false>(p, l, st);
        case 3: return l.silu ? launch_i8_depth<WF, 3, true>(p, l, st) : launch_i8_depth<WF, 3, false>(p, l, st);
        case 4: return l.silu ? launch_i8_depth<WF, 4, true>(p, l, st) : launch_i8_depth<WF, 4, false>(p, l, st);
        default: return BZ_ERR_INVALID_ARG;
    }
}

int launch_i8_i4zp(const GemvParams& p, const Launch& l, hipStream_t st);
int launch_i8_i4min(const GemvParams& p, const Launch& l, hipStream_t st);

}  // namespace bz
