// Matrix-core variant of the streaming decode GEMV (gfx950 MFMA).
//
// Same contract, prologue and pipeline as gemv_persist (bz_gemv_kernel.h);
// the arithmetic of a step moves from v_dot2 to v_mfma_f32_16x16x32_bf16,
// which takes the unpacked weights as the B operand directly and leaves the
// VALU only the nibble/fp8 unpacking:
//   * a tile is 16 output columns; a "unit" is 64 contiguous bytes of each of
//     the tile's 16 weight rows (int4: 128 k = one quantization group for
//     group >= 128; fp8: 64 k; bf16: 32 k);
//   * lane l loads 16 bytes of row l%16 at offset 16*(l/16) of the unit, which
//     is exactly the B-operand placement of the instruction
//     (B[k][j] in lane j + 16*(k/8), element k%8), so no shuffles are needed;
//   * the A operand is x: lane l supplies row m = min(l%16, M-1) of x; the
//     output rows m >= M it produces are never stored, so M = 1..4 wastes
//     matrix-core cycles, never memory or VALU;
//   * D[i][j] lands in lane j + 16*(i/4), element i%4: lane l holds output
//     column l%16 for x rows 4*(l/16) + q.
// int4 units are scaled per group after their 4 MFMAs:
//   y += s * D + (z - 136 s) * X     (X = sum of x over the unit's 128 k)
// with the unit's (s, z) pair loaded next to its weights (lane l: row l%16).
// fp8 and bf16 units accumulate in the MFMA accumulator itself (the fp8
// per-row scale is applied in the epilogue).
#pragma once
#include "bz_gemv_kernel.h"

namespace bz {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4_t mfma_bf16(const u32x4 a, const u32x4 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
}

// k covered by one 64-byte unit of a weight row.
__host__ __device__ constexpr int mfma_unit_k(int wf) { return is_int4(wf) ? 128 : (wf == WF_FP8 ? 64 : 32); }

// Elements of one LDS x row: K rounded up to whole units (zero padded).
__host__ __device__ inline int mfma_x_row_elems(int K, int wf) {
    const int u = mfma_unit_k(wf);
    return (K + u - 1) / u * u;
}

struct MfmaLds {
    int xs, x128, red, nrm, total;
};
__host__ __device__ inline MfmaLds mfma_lds_layout(int M, int T, int NW, int K, int wf, int tpw) {
    const bool i4 = is_int4(wf);
    const int xe = mfma_x_row_elems(K, wf);
    MfmaLds L;
    L.xs = 0;
    L.x128 = L.xs + align16(M * xe * 2);
    L.red = L.x128 + (i4 ? align16(M * (xe / 128) * 4) : 0);
    L.nrm = L.red + align16(tpw * NW * T * M * 16 * 4);
    L.total = L.nrm + align16(NW * M * 4);
    return L;
}

// Sum over each aligned group of 16 lanes (one DPP row); every lane of the
// group gets it.  row_ror:8 pairs lane i with lane i ^ 8 of the same row.
__device__ __forceinline__ float sum16(float v) {
    v = sum8(v);
    return v + dpp_f32<0x128>(v);
}

// Stage one 8-element block of x (natural block order; int4 blocks are
// permuted [x0 x4 x1 x5 x2 x6 x3 x7] inside, to pair with nibble pairs).
template <int WF>
__device__ __forceinline__ void stage_block_mfma(const GemvParams& p, u32x4 v, u32x4 g, int m, int kb, uint16_t* xs,
                                                 float* x128, int xe) {
    float f[8];
    block_values(p, v, g, f);
    u32x4 o;
    if (is_int4(WF)) {
        o[0] = pack_bf16x2(f[0], f[4]);
        o[1] = pack_bf16x2(f[1], f[5]);
        o[2] = pack_bf16x2(f[2], f[6]);
        o[3] = pack_bf16x2(f[3], f[7]);
        float cs = ((f[0] + f[1]) + (f[2] + f[3])) + ((f[4] + f[5]) + (f[6] + f[7]));
        cs = sum16(cs);  // 16 consecutive blocks (16 consecutive lanes) = one 128-k unit
        if ((kb & 15) == 0) x128[m * (xe >> 7) + (kb >> 4)] = cs;
    } else if (p.norm) {
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = pack_bf16x2(f[2 * i], f[2 * i + 1]);
    } else {
        o = v;
    }
    *reinterpret_cast<u32x4*>(xs + m * xe + kb * 8) = o;
}

template <int WF, int M>
__device__ __forceinline__ void finish_x_mfma(const GemvParams& p, const u32x4 (&xr)[kXB], const u32x4 (&gr)[kXB],
                                              uint16_t* xs, float* x128, float* nrm, int tid, int nthr, int wave,
                                              int lane) {
    const int xe = mfma_x_row_elems(p.K, WF);
    finish_x_generic<WF, M>(p, xr, gr, nrm, tid, nthr, wave, lane, [&](u32x4 v, u32x4 g, int m, int kb) {
        stage_block_mfma<WF>(p, v, g, m, kb, xs, x128, xe);
    });
    // zero the padding past K (fp8 / bf16 units may overhang K)
    const int pad = (xe - p.K) >> 3;
    for (int b = tid; b < M * pad; b += nthr) {
        const int m = b / pad;
        *reinterpret_cast<u32x4*>(xs + m * xe + p.K + (b - m * pad) * 8) = u32x4{0u, 0u, 0u, 0u};
    }
}

// Issue the T weight loads of the unit at cursor c, and for int4 the (s, z) /
// (s, min) pair of the unit's group for row j.
template <int WF, int T, bool SILU>
__device__ __forceinline__ void issue_unit(const GemvParams& p, StepCursor c, int tile0, int j, int kb,
                                           u32x4 (&buf)[T], uint32_t (&sc)[T]) {
    const int u = c.ch;
    const int colbase = (tile0 + c.tl) * 16;
    const uint8_t* base = p.w + (int64_t)colbase * p.row_bytes + u * 64;  // uniform
    const int lr = min(j, p.n_out - 1 - colbase);                          // partial last tile
    const int lk = min(kb * 16, (int)p.row_bytes - 16 - u * 64);            // K tail (fp8 / bf16)
    const uint32_t off = __umul24((uint32_t)lr, (uint32_t)p.row_bytes) + (uint32_t)lk;  // lr < 16
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const uint8_t* bt = SILU && t ? base + (int64_t)p.n_out * p.row_bytes : base;
        buf[t] = ldg16(bt + off);
    }
    const int g = (u * 128) >> p.glog2;  // one group per unit (group >= 128)
    if (WF == WF_I4ZP) {
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int row = colbase + lr + (SILU && t ? p.n_out : 0);
            sc[t] = reinterpret_cast<const uint32_t*>(p.sc0)[(int64_t)g * p.N + row];
        }
    } else if (WF == WF_I4MIN) {
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int row = colbase + lr + (SILU && t ? p.n_out : 0);
            sc[t] = (uint32_t)reinterpret_cast<const uint16_t*>(p.sc0)[(int64_t)row * p.G + g] |
                    ((uint32_t)reinterpret_cast<const uint16_t*>(p.sc1)[(int64_t)row * p.G + g] << 16);
        }
    }
}

template <int M>
constexpr int kQM = M < 4 ? M : 4;  // x rows a lane's accumulator holds that can be < M

template <int WF, int M, int T>
__device__ __forceinline__ void consume_unit(const GemvParams& p, StepCursor c, int j, int kb, int xe,
                                             const uint16_t* xs, const float* x128, const NibbleConsts& nc,
                                             const u32x4 (&buf)[T], const uint32_t (&scv)[T], f32x4_t (&acc)[T]) {
    const int u = c.ch;
    const int am = min(j, M - 1);  // x row this lane supplies to the A operand
    if (is_int4(WF)) {
        u32x4 a[4];
        const uint16_t* xa = xs + am * xe + u * 128 + kb * 32;
#pragma unroll
        for (int d = 0; d < 4; ++d) a[d] = *reinterpret_cast<const u32x4*>(xa + d * 8);
        float X[kQM<M>];
#pragma unroll
        for (int q = 0; q < kQM<M>; ++q) X[q] = x128[min(4 * kb + q, M - 1) * (xe >> 7) + u];
#pragma unroll
        for (int t = 0; t < T; ++t) {
            f32x4_t dacc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                u32x4 bv;
#pragma unroll
                for (int sh = 0; sh < 4; ++sh) bv[sh] = nib2_bf16(buf[t][d] >> (4 * sh), nc.mask, nc.magic);
                dacc = mfma_bf16(a[d], bv, dacc);
            }
            const uint32_t e = scv[t];
            const float s = bf16_lo(e);
            const float zp = bf16_hi(e) - (WF == WF_I4ZP ? 136.0f : 128.0f) * s;
#pragma unroll
            for (int q = 0; q < kQM<M>; ++q) acc[t][q] += s * dacc[q] + zp * X[q];
        }
    } else if (WF == WF_FP8) {
        const bool kok = u * 64 + kb * 16 < p.row_bytes;
        const uint16_t* xa = xs + am * xe + u * 64 + kb * 16;
        const u32x4 a0 = *reinterpret_cast<const u32x4*>(xa);
        const u32x4 a1 = *reinterpret_cast<const u32x4*>(xa + 8);
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const u32x4 w = kok ? buf[t] : u32x4{0u, 0u, 0u, 0u};
            const u32x4 b0 = {fp8x2_bf16<false>(w[0]), fp8x2_bf16<true>(w[0]), fp8x2_bf16<false>(w[1]),
                              fp8x2_bf16<true>(w[1])};
            const u32x4 b1 = {fp8x2_bf16<false>(w[2]), fp8x2_bf16<true>(w[2]), fp8x2_bf16<false>(w[3]),
                              fp8x2_bf16<true>(w[3])};
            acc[t] = mfma_bf16(a0, b0, acc[t]);
            acc[t] = mfma_bf16(a1, b1, acc[t]);
        }
    } else {
        const bool kok = u * 64 + kb * 16 < p.row_bytes;
        const u32x4 a0 = *reinterpret_cast<const u32x4*>(xs + am * xe + u * 32 + kb * 8);
#pragma unroll
        for (int t = 0; t < T; ++t) acc[t] = mfma_bf16(a0, kok ? buf[t] : u32x4{0u, 0u, 0u, 0u}, acc[t]);
    }
}

// T = 2 for the SiLU-gate pair, else 1.  D = units of loads in flight per wave.
template <int WF, int M, int T, int D, bool SILU>
__global__ void __launch_bounds__(kMaxThreads) gemv_mfma(BZ_GEMV_HOT_PARAMS, GemvParams p) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    gemv_hot(p, hx, hw, hsc0, hgamma, hldx, hrow_bytes, hK, hN, hntiles, htpw);
    const int nthr = blockDim.x;
    const int NW = nthr >> 6;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 15, kb = lane >> 4;
    const int xe = mfma_x_row_elems(p.K, WF);
    const int nunits = (int)((p.row_bytes + 63) / 64);
    const TileRange tr(p.ntiles);
    const int tile0 = tr.tile0, ntl = tr.ntl;
    const int S = wave_steps(ntl, nunits, NW, wave);  // host ensures NW <= nunits

    const MfmaLds L = mfma_lds_layout(M, T, NW, p.K, WF, p.tpw);
    uint16_t* xs = reinterpret_cast<uint16_t*>(smem + L.xs);
    float* x128 = reinterpret_cast<float*>(smem + L.x128);
    float* red = reinterpret_cast<float*>(smem + L.red);
    float* nrm = reinterpret_cast<float*>(smem + L.nrm);

    u32x4 buf[D][T];
    uint32_t scb[D][T];
    auto issue = [&](int d, StepCursor c) { issue_unit<WF, T, SILU>(p, c, tile0, j, kb, buf[d], scb[d]); };

    // 0. x and gamma first, then the first D units of weights (+ scales)
    u32x4 xr[kXB], gr[kXB];
    issue_x<WF, M>(p, tid, nthr, xr, gr);
    const EpiPrefetch<T> pre = epi_prefetch<WF, M, T, SILU, 16>(p, tile0, ntl, tid);
    __builtin_amdgcn_sched_barrier(0);
    StepCursor ic{0, wave};
    pipeline_prime<0, D>(S, NW, nunits, wave, ic, issue);
    __builtin_amdgcn_sched_barrier(0);
    // 1. staging completes while the weights are in flight
    finish_x_mfma<WF, M>(p, xr, gr, xs, x128, nrm, tid, nthr, wave, lane);
    __syncthreads();
    float inv[M];
    row_inv_all<M>(p, nrm, NW, inv);

    // 2. every unit once; a wave's partial sums of a tile go to LDS after its
    //    last unit in that tile
    const NibbleConsts nc;
    f32x4_t acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    pipeline_run<D>(S, NW, nunits, wave, ic, issue, [&](int d, StepCursor c) {
        consume_unit<WF, M, T>(p, c, j, kb, xe, xs, x128, nc, buf[d], scb[d], acc);
        if (c.last_in_tile(NW, nunits)) {
#pragma unroll
            for (int t = 0; t < T; ++t) {
#pragma unroll
                for (int q = 0; q < kQM<M>; ++q) {
                    const int m = 4 * kb + q;
                    if (m < M) red[(((c.tl * NW + wave) * T + t) * M + m) * 16 + j] = acc[t][q];
                }
                acc[t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
            }
        }
    });
    __syncthreads();

    // 3. epilogue
    epilogue<WF, M, T, SILU, 16>(p, tile0, ntl, tid, nthr, NW, red, nrm, inv, pre);
}

template <int WF, int M, int T, int D, bool SILU>
int launch_mfma_kernel(const GemvParams& p, const Launch& l, hipStream_t st) {
    auto kern = gemv_mfma<WF, M, T, D, SILU>;
    if (l.lds > 65536 && raise_lds_limit(reinterpret_cast<const void*>(kern)) != BZ_OK) return BZ_ERR_LAUNCH;
    if (!gemv_hot_ok(p)) return BZ_ERR_UNSUPPORTED;
    hipLaunchKernelGGL(kern, dim3(l.grid), dim3(l.nw * 64), l.lds, st, BZ_GEMV_HOT_ARGS(p), p);
    return hipGetLastError() == hipSuccess ? BZ_OK : BZ_ERR_LAUNCH;
}

template <int WF, int M, bool SILU>
int launch_mfma_depth(const GemvParams& p, const Launch& l, hipStream_t st) {
    constexpr int T = SILU ? 2 : 1;
    switch (l.depth) {
        case 2: return launch_mfma_kernel<WF, M, T, 2, SILU>(p, l, st);
        case 4: return launch_mfma_kernel<WF, M, T, 4, SILU>(p, l, st);
        case 8: return launch_mfma_kernel<WF, M, T, 8, SILU>(p, l, st);
        case 16:
            if constexpr (T == 1) return launch_mfma_kernel<WF, M, T, 16, SILU>(p, l, st);
            return BZ_ERR_INVALID_ARG;
        default: return BZ_ERR_INVALID_ARG;
    }
}

template <int WF>
int launch_mfma_m(const GemvParams& p, const Launch& l, hipStream_t st) {
    switch (l.M) {
        case 1: return l.silu ? launch_mfma_depth<WF, 1, true>(p, l, st) : launch_mfma_depth<WF, 1, false>(p, l, st);
        case 2: return l.silu ? launch_mfma_depth<WF, 2, true>(p, l, st) : launch_mfma_depth<WF, 2, false>(p, l, st);
        case 3: return l.silu ? launch_mfma_depth<WF, 3, true>(p, l, st) : launch_mfma_depth<WF, 3, false>(p, l, st);
        case 4: return l.silu ? launch_mfma_depth<WF, 4, true>(p, l, st) : launch_mfma_depth<WF, 4, false>(p, l, st);
        default: return BZ_ERR_INVALID_ARG;
    }
}

int launch_mfma_i4zp(const GemvParams& p, const Launch& l, hipStream_t st);
int launch_mfma_i4min(const GemvParams& p, const Launch& l, hipStream_t st);
int launch_mfma_fp8(const GemvParams& p, const Launch& l, hipStream_t st);
int launch_mfma_bf16(const GemvParams& p, const Launch& l, hipStream_t st);

}  // namespace bz
