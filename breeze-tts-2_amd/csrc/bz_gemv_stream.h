// Streaming decode GEMV over row-block-tiled weights (GEMV path 5).
//
// Replaces, as one launch (like the row-major paths of bz_gemv_kernel.h):
//   rms_gemv_kernel + gemv_epilogue_kernel   models/fused/kernels.py:41-138
//   torch._weight_int4pack_mm (Int4Linear)   models/int4_linear.py:103-108
//   torch._scaled_mm (Fp8Linear, weight-only form)  models/fp8_linear.py:76-82
//
// Tiled weight formats (include/bz_gemv.h, BZ_W_*_TILED / *_TILED_PAIRED)
//   * A row block is 16 weight rows: rows 16b..16b+15 (plain), or for the
//     paired formats of a SiLU-gate weight [gate; up] (models/fused/layer.py:60)
//     gate rows 8b..8b+7 followed by up rows 8b..8b+7, so one block yields 8
//     finished outputs silu(g) * u with no second pass.
//   * A unit is 64 bytes of each row: 128 k of int4 (one quantization group of
//     128) or 64 k of fp8.
//   * The chunk of block b is contiguous: NU tiles of 1024 bytes (tile u holds
//     unit u of the 16 rows, row r at byte 64 r), then the block's scales:
//       int4: NU x 16 (s, z) bf16 pairs, unit u row r at byte 64 u + 4 r,
//             w = (q - 8) s + z  (the scales_zeros pair of
//             models/int4_linear.py:61-63);
//       fp8:  16 fp32 row scales (applied to the finished dot products).
//     Chunks are padded to 128 bytes, so every tile is a full cache line run.
//
// Why tiles: one wave instruction (64 lanes x 16 bytes) reads exactly one
// contiguous 1 KiB tile, and a workgroup streams one contiguous chunk
// including its scales.  Measured on MI355X against the row-major layout
// (16 rows x 64 bytes per wave instruction, scales [G][N] 64 bytes apart per
// unit): the same kernel streams int4 gate|up (K2560 N20480) 0.6 us faster
// and down (K10240 N2560) 0.7 us faster.
//
// Work decomposition
//   * One workgroup per row block; its NW waves split the NU units, UPW
//     consecutive units each (split-K inside the workgroup, summed in a fixed
//     order: deterministic).
//   * A wave stages into LDS only the slice of x its own units multiply, so
//     no wave waits for another before its main loop; the workgroup's one
//     barrier precedes the epilogue.  (Staging all of x in every workgroup,
//     behind a barrier, put 2.7 us of latency and redundant VALU work in front
//     of every workgroup's first tile at M = 1 and 4.8 us at M = 2.)
//   * Each wave keeps D tiles in flight in a rolling register pipeline; its x
//     loads go out first and are range-checked buffer loads, so the staging
//     waits exactly for them and not for the tiles behind them.
//   * Weight loads are non-temporal (they are read once; x, the scales and the
//     next kernel's inputs keep the L2).
//
// Arithmetic: v_mfma_f32_16x16x32_bf16 for both formats (A = up to 16 rows
// of x, B = 16 weight rows; with one x row the MFMA wastes 15/16 of its work,
// but the matrix cores are otherwise idle and the VALU work per weight byte is
// what has to stay off the critical path).  Operand layouts (gfx950):
// A[i][k] in lane i + 16 (k/8), elements k%8; B[k][j] in lane j + 16 (k/8);
// D[i][j] in lane j + 16 (i/4), element i%4.  Lane l of a wave holds 16 bytes
// of tile row l%16 at byte 16 (l/16) of the unit.
//   * int4: the lane's 32 nibbles are k = 32 (l/16) + 8 d + e (dword d, nibble
//     e).  Dword d becomes the B operand of MFMA d: four bf16 pairs
//     (128 + q_e, 128 + q_{e+4}), one v_and_or_b32 each (exponent 2^7, nibble in
//     the mantissa).  x is staged in the same order ([x0 x4 x1 x5 x2 x6 x3 x7]
//     per 8 values), so MFMA d's A operand is one 16-byte LDS read.  Per unit:
//       sum_k u_k w_k = s D + (z - 136 s) X,   D = sum_k u_k (128 + q_k),
//     X = sum of u over the unit's 128 k (fp32, from the staging).
//   * fp8: gfx950's OCP e4m3 -> bf16 conversion (exact) of codes 0-7 and 8-15
//     gives the B operands of two MFMAs; x is staged in natural order.  The
//     accumulator runs over all units; the row scale is applied at the end.
//   * RMSNorm is folded as in the row-major paths: LDS holds u = bf16(gamma x)
//     and the per-row 1/rms multiplies the finished dot products.
#pragma once

#include "bz_gemv_i8.h"

namespace bz {

enum {
    WF_I4T = BZ_W_INT4_TILED,
    WF_I4TP = BZ_W_INT4_TILED_PAIRED,
    WF_F8T = BZ_W_FP8_TILED,
    WF_F8TP = BZ_W_FP8_TILED_PAIRED
};

__host__ __device__ constexpr bool tiled_i4(int wf) { return wf == WF_I4T || wf == WF_I4TP; }
__host__ __device__ constexpr bool tiled_paired(int wf) { return wf == WF_I4TP || wf == WF_F8TP; }

// k per 64-byte unit, and bytes of one row block's chunk.
__host__ __device__ constexpr int tiled_unit_k(int wf) { return tiled_i4(wf) ? 128 : 64; }
__host__ __device__ inline int64_t tiled_chunk_bytes(int wf, int NU) {
    const int64_t raw = (int64_t)NU * 1024 + (tiled_i4(wf) ? (int64_t)NU * 64 : 64);
    return (raw + 127) / 128 * 128;
}

struct StreamParams {
    const uint16_t* x;
    int64_t ldx;
    const uint8_t* w;
    int64_t chunk;  // bytes per row block
    const uint16_t* gamma;
    const void* res;
    int64_t ldr;
    void* out;
    int64_t ldo;
    void* out2;     // columns [0, n_out2) stored here as well (n_out2 = 0: none)
    int64_t ldo2;
    int n_out2;
    float eps;
    int M, K, NU, n_out;
    int epi, out_f32, res_f32, norm;
    int x_lead;     // 1: the x loads get a head start before the first tiles (long rows)
};

// LDS carve-up (bytes), shared with the host launcher: x rows as bf16 (row
// stride 2K + 16 bytes), the int4 per-unit sums X [row][unit], the sums of x^2
// of each wave's four 16-lane rows [wave][row][4] and the partial dot
// products [row][column][wave].
struct StreamLds {
    int xs, xst, sq, red, total;
};
__host__ __device__ inline int stream_x_row_bytes(int K) { return 2 * K + 16; }
__host__ __device__ inline StreamLds stream_lds(int wf, int M, int K, int NW) {
    StreamLds L;
    L.xs = 0;
    L.xst = align16(M * stream_x_row_bytes(K));
    L.sq = L.xst + align16(tiled_i4(wf) ? M * (K / 128) * 4 : 0);
    L.red = L.sq + align16(NW * M * 16);
    L.total = L.red + align16(M * 16 * 16 * 4);  // 16 wave slots
    return L;
}

// Units per wave the kernels are instantiated for, the most rows of x one
// launch takes and the most waves of a workgroup.
constexpr int kStreamUpw[] = {1, 2, 3, 4, 5, 6, 8, 10};
constexpr int kStreamMaxRows = 8;
constexpr int kStreamMaxWaves = 16;

// Pipeline depth for UPW units per wave (measured on MI355X: 2 for 2-4
// units, 3 for 5 or more; all of them when a wave has at most 2).
__host__ __device__ constexpr int stream_depth(int upw) { return upw <= 2 ? upw : (upw >= 5 ? 3 : 2); }

// Kernel arguments that the hardware preloads into SGPRs when a wave
// launches (gfx950 kernarg preloading: the first 14 dwords of the kernarg
// segment, enabled by -mllvm -amdgpu-kernarg-preload-count=16 in the build;
// an aggregate is never preloaded).  The streaming kernels take the fields
// their first x and weight loads need as these leading scalars, ahead of the
// parameter struct, so those loads do not wait at every workgroup's start
// for the struct's scalar loads from memory.  Measured on MI355X (the
// several-block kernel at M = 1): int4 gate|up 7.05 -> 6.86 us, qkv 4.12 ->
// 4.02, down 5.69 -> 5.29, o_proj 3.78 -> 3.62.  The host passes the same
// values in the struct; the kernel takes them from the scalars.
__device__ __forceinline__ void stream_hot(StreamParams& p, const uint8_t* w, const uint16_t* x, const uint16_t* gamma,
                                           int chunk, int ldx, int K, int NU, int M, int norm) {
    p.w = w;
    p.x = x;
    p.gamma = gamma;
    p.chunk = chunk;
    p.ldx = ldx;
    p.K = K;
    p.NU = NU;
    p.M = M;
    p.norm = norm;
}

// Host side: whether a StreamParams fits the 32-bit leading scalars.
inline bool stream_hot_ok(const StreamParams& p) { return p.chunk <= 0x7FFFFFFF && p.ldx <= 0x7FFFFFFF; }

// ---- the kernel --------------------------------------------------------------

template <int WF, int MM, int UPW>
__global__ void __launch_bounds__(1024) gemv_stream(const uint8_t* hw, const uint16_t* hx, const uint16_t* hg, int hchunk,
                                                    int hldx, int hK, int hNU, int hM, int hnorm, int hlead,
                                                    StreamParams p) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    stream_hot(p, hw, hx, hg, hchunk, hldx, hK, hNU, hM, hnorm);
    p.x_lead = hlead;
    constexpr bool I4 = tiled_i4(WF);
    constexpr bool PAIR = tiled_paired(WF);
    constexpr int D = stream_depth(UPW);
    constexpr int BPU = tiled_unit_k(WF) / 8;   // blocks of 8 x values per unit
    constexpr int RK = (UPW * BPU + 63) / 64;   // rounds of blocks per lane over a wave's slice
    constexpr int NXL = RK * (1 + MM) <= 12 ? RK * (1 + MM) : 12;  // x / gamma loads held in registers
    const int nthr = blockDim.x, NW = nthr >> 6;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 15, kq = lane >> 4;
    const int M = p.M, K = p.K, NU = p.NU;
    const int b = blockIdx.x;
    const uint8_t* chunk = p.w + (int64_t)b * p.chunk;

    const StreamLds L = stream_lds(WF, M, K, NW);
    uint8_t* xs = smem + L.xs;
    float* xst = reinterpret_cast<float*>(smem + L.xst);
    float* sq = reinterpret_cast<float*>(smem + L.sq);
    float* red = reinterpret_cast<float*>(smem + L.red);
    const int xrow = stream_x_row_bytes(K);

    // this wave's units [u0, u0 + nu) and blocks of x [kb0, kb0 + nkb)
    const int u0 = wave * UPW;
    const int nu = max(0, min(UPW, NU - u0));
    const int kb0 = u0 * BPU, nkb = nu * BPU;

    // 0. the slice's x and gamma, first: load t = r (1 + MM) + s is gamma
    //    (s = 0) or x row s - 1 at block kb0 + lane + 64 r.  Range-checked
    //    buffer loads, issued unconditionally (exact wait counts); one that
    //    does not exist sends no request.
    const __amdgpu_buffer_rsrc_t xrs = buffer_rsrc(p.x, (uint32_t)(((int64_t)(M - 1) * p.ldx + K) * 2));
    const __amdgpu_buffer_rsrc_t grs = buffer_rsrc(p.gamma, p.norm ? (uint32_t)K * 2 : 0u);
    auto xoff = [&](int r, int s2) -> uint32_t {
        const int kl = lane + 64 * r;
        if (kl >= nkb) return kBufferOob;
        if (s2 == 0) return p.norm ? (uint32_t)(kb0 + kl) * 16 : kBufferOob;
        if (s2 - 1 >= M) return kBufferOob;
        return (uint32_t)(((int64_t)(s2 - 1) * p.ldx + (kb0 + kl) * 8) * 2);
    };
    u32x4 xl[NXL];
#pragma unroll
    for (int t = 0; t < NXL; ++t) {
        const int r = t / (1 + MM), s2 = t % (1 + MM);
        xl[t] = buffer_ld16(s2 == 0 ? grs : xrs, xoff(r, s2));
    }
    // The epilogue reduces each output's per-wave partials in a group of 16
    // lanes (lane w reads wave w's partial); group g = (row, column) for
    // g = tid/16, tid/16 + nthr/16, ...  What it reads from memory for its
    // first group -- the residual and the fp8 row scale(s) -- is loaded now.
    const int ocols = PAIR ? 8 : 16;
    const int ngrp = M * ocols, gstep = nthr >> 4;
    const int g0 = tid >> 4, gw = tid & 15;
    auto load_res = [&](int g) -> uint32_t {
        const int m = g / ocols, c = g - m * ocols;
        const int64_t ri = (int64_t)m * p.ldr + b * ocols + c;
        return p.res_f32 ? reinterpret_cast<const uint32_t*>(p.res)[ri]
                         : (uint32_t)reinterpret_cast<const uint16_t*>(p.res)[ri];
    };
    uint32_t resv = 0u;
    if (p.epi == BZ_EPI_RESIDUAL && g0 < ngrp && gw == 0) resv = load_res(g0);
    const float* rsc = reinterpret_cast<const float*>(chunk + (int64_t)NU * 1024);  // fp8 row scales
    float rs0 = 1.0f, rs1 = 1.0f;
    if (!I4 && g0 < ngrp) {
        const int c = g0 % ocols;
        rs0 = rsc[c];
        if (PAIR) rs1 = rsc[c + 8];
    }
    // The wave's UPW tiles and, for int4, the (s, z) pairs of this lane's row,
    // through range-checked buffer loads over the block's tiles and scales:
    // a unit past the block (the last wave may own fewer than UPW) reads as
    // zeros without a memory request and adds exactly 0 (zero codes, s = z =
    // 0), so every wave runs the same branch-free loop with exact wait counts
    const __amdgpu_buffer_rsrc_t wrs = buffer_rsrc(chunk, (uint32_t)NU * 1024u);
    uint32_t sc[UPW];
    if (I4) {
        const __amdgpu_buffer_rsrc_t srs = buffer_rsrc(chunk + (int64_t)NU * 1024, (uint32_t)NU * 64u);
#pragma unroll
        for (int q = 0; q < UPW; ++q) sc[q] = buffer_ld4(srs, (uint32_t)(u0 + q) * 64u + j * 4);
    }
    u32x4 wv[UPW];
    auto issue = [&](int q) { wv[q] = buffer_ld16_nt(wrs, (uint32_t)(u0 + q) * 1024u + j * 64 + kq * 16); };
    // Long rows (80 units or more) over at most 256 row blocks (at most one
    // workgroup per CU): the x loads get about 270 ns before the first tiles
    // go out, so they do not queue behind the tiles of every wave of the CU.
    // Measured on MI355X: int4 K10240 N2560 5.60 -> 5.32 us, fp8 K10240
    // N2560 7.53 -> 7.40 us; shorter rows are slower with it (fp8 K4096
    // N2560, 64 units, 3.96 -> 4.17 us; K2560 N20480 7.30 -> 7.55 us).
    __builtin_amdgcn_sched_barrier(0);
    if (p.x_lead) __builtin_amdgcn_s_sleep(10);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < D; ++q) issue(q);
    __builtin_amdgcn_sched_barrier(0);

    // 1. stage the slice while the first tiles are in flight: u = bf16(gamma x)
    //    (or x) per block; int4 blocks are stored [x0 x4 x1 x5 x2 x6 x3 x7] and
    //    their unit's sum X is reduced over the unit's 16 consecutive lanes
    //    (kb0 is a multiple of 16, so a unit is an aligned 16-lane group).
    //    The sums of x^2 and X come from v_dot2_f32_bf16 on the packed
    //    values (the products of bf16 values are exact in fp32).
    float ss[MM];
#pragma unroll
    for (int m = 0; m < MM; ++m) ss[m] = 0.0f;
    constexpr uint32_t kOnes = 0x3F803F80u;  // bf16 (1.0, 1.0)
    auto stage = [&](u32x4 v, u32x4 g, int m, int kl, bool norm) {
        u32x4 u = v;
        if (norm) {
            float s2 = 0.0f;
#pragma unroll
            for (int q = 0; q < 4; ++q) s2 = dot2(v[q], v[q], s2);
#pragma unroll
            for (int mm = 0; mm < MM; ++mm)
                if (mm == m) ss[mm] += s2;
#pragma unroll
            for (int q = 0; q < 4; ++q) u[q] = pack_bf16x2(bf16_lo(v[q]) * bf16_lo(g[q]), bf16_hi(v[q]) * bf16_hi(g[q]));
        }
        u32x4 o = u;
        if (I4) {
            // (x_q, x_{q+4}) pairs: the low halves of u[0], u[2], the high halves, then u[1], u[3]
            o[0] = __builtin_amdgcn_perm(u[2], u[0], 0x05040100u);
            o[1] = __builtin_amdgcn_perm(u[2], u[0], 0x07060302u);
            o[2] = __builtin_amdgcn_perm(u[3], u[1], 0x05040100u);
            o[3] = __builtin_amdgcn_perm(u[3], u[1], 0x07060302u);
        }
        if (kl < nkb) *reinterpret_cast<u32x4*>(xs + m * xrow + (kb0 + kl) * 16) = o;
        if (I4) {
            float cs = 0.0f;
#pragma unroll
            for (int q = 0; q < 4; ++q) cs = dot2(u[q], kOnes, cs);
            cs = sum16_dpp(cs);
            if (kl < nkb && (kl & 15) == 0) xst[m * NU + (kb0 + kl) / 16] = cs;
        }
    };
    // blocks held in registers (lanes past the slice hold zeros: they still
    // join the 16-lane sums, which their whole group skips storing)
#pragma unroll
    for (int r = 0; r < RK; ++r) {
        if (r * 64 < nkb) {
            const int t0 = r * (1 + MM);
            const u32x4 g = t0 < NXL ? xl[t0] : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
            for (int m = 0; m < MM; ++m) {
                if (m < M) {
                    const int t = t0 + 1 + m;
                    // beyond the register budget: a load now (L2), range-checked
                    // like the ones above, so a lane past the slice reads zeros
                    // and adds nothing to the row's sum of squares
                    const u32x4 v = t < NXL ? xl[t] : buffer_ld16(xrs, xoff(r, m + 1));
                    u32x4 gg = g;
                    if (t0 >= NXL && p.norm) gg = buffer_ld16(grs, xoff(r, 0));
                    if (p.norm)  // uniform
                        stage(v, gg, m, lane + 64 * r, true);
                    else
                        stage(v, gg, m, lane + 64 * r, false);
                }
            }
        }
    }
    if (p.norm) {  // per 16-lane row; the epilogue adds the four rows of each wave
#pragma unroll
        for (int m = 0; m < MM; ++m) {
            const float t = sum16_dpp(ss[m]);
            if (j == 0 && m < M) sq[(wave * M + m) * 4 + kq] = t;
        }
    }
    // the wave reads back only what it wrote: LDS operations of one wave
    // complete in order, so no workgroup barrier is needed here
    __builtin_amdgcn_wave_barrier();

    // 2. the wave's units: consume tile q, issue tile q + D, without run-time
    //    conditions, so each wait counts exactly the loads in flight.  A unit
    //    past the block reads x and X at the block's last unit, which the
    //    same wave staged (every wave owns at least one unit), so it
    //    multiplies finite values by its zero weights.
    float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    f32x4_t facc = {0.0f, 0.0f, 0.0f, 0.0f};
    const uint8_t* xa = xs + min(j, M - 1) * xrow;  // the x row this lane supplies to A
    const NibbleConsts nc;
    auto consume = [&](int q, bool next) {
        const int u = min(u0 + q, NU - 1);
        if (I4) {
            u32x4 bq[4];
#pragma unroll
            for (int d = 0; d < 4; ++d)
#pragma unroll
                for (int e = 0; e < 4; ++e) bq[d][e] = nib2_bf16(wv[q][d] >> (4 * e), nc.mask, nc.magic);
            if (next) issue(q + D);
            const uint8_t* xu = xa + (u * 128 + kq * 32) * 2;
            f32x4_t dv = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int d = 0; d < 4; ++d) dv = mfma_bf16(*reinterpret_cast<const u32x4*>(xu + d * 16), bq[d], dv);
            const float s = bf16_lo(sc[q]);
            const float zp = fmaf(-136.0f, s, bf16_hi(sc[q]));
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if (r < MM) {
                    const float X = xst[min(4 * kq + r, M - 1) * NU + u];
                    y[r] = fmaf(s, dv[r], fmaf(zp, X, y[r]));
                }
            }
        } else {
            u32x4 b0, b1;
            b0[0] = fp8x2_bf16<false>(wv[q][0]);
            b0[1] = fp8x2_bf16<true>(wv[q][0]);
            b0[2] = fp8x2_bf16<false>(wv[q][1]);
            b0[3] = fp8x2_bf16<true>(wv[q][1]);
            b1[0] = fp8x2_bf16<false>(wv[q][2]);
            b1[1] = fp8x2_bf16<true>(wv[q][2]);
            b1[2] = fp8x2_bf16<false>(wv[q][3]);
            b1[3] = fp8x2_bf16<true>(wv[q][3]);
            if (next) issue(q + D);
            const uint8_t* xu = xa + (u * 64 + kq * 16) * 2;
            facc = mfma_bf16(*reinterpret_cast<const u32x4*>(xu), b0, facc);
            facc = mfma_bf16(*reinterpret_cast<const u32x4*>(xu + 16), b1, facc);
        }
    };
#pragma unroll
    for (int q = 0; q < UPW; ++q) consume(q, q + D < UPW);
    if (!I4) {
#pragma unroll
        for (int r = 0; r < 4; ++r) y[r] = facc[r];
    }
    // 3. park the wave's partials: red[(row * 16 + column) * 16 + wave]
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int m = 4 * kq + r;
        if (r < MM && m < M) red[(m * 16 + j) * 16 + wave] = y[r];
    }
    __syncthreads();
    // 4. per output: 16-lane DPP sums over the waves of its partials and of
    //    its row's sums of x^2 (lane w reads wave w's; lanes w >= NW add 0; a
    //    fixed tree, so the result does not depend on timing; one LDS round
    //    trip -- a loop over the waves' partials in one lane measured 0.5-0.8
    //    us slower per launch), then 1/rms, the fp8 row scale, SiLU-gate or
    //    residual, and the store
    for (int g = g0; g < ngrp; g += gstep) {
        const bool first = g == g0;
        const int m = g / ocols, c = g - m * ocols;
        const float* rg = red + (m * 16 + c) * 16;
        const bool live = gw < NW;
        float a = live ? rg[gw] : 0.0f;
        float a2 = PAIR && live ? rg[8 * 16 + gw] : 0.0f;
        float s2 = 0.0f;
        if (p.norm && live) {
            const float4 q4 = *reinterpret_cast<const float4*>(sq + (gw * M + m) * 4);
            s2 = (q4.x + q4.y) + (q4.z + q4.w);
        }
        a = sum16_dpp(a);
        if (PAIR) a2 = sum16_dpp(a2);
        if (p.norm) s2 = sum16_dpp(s2);
        if (gw == 0) {
            const float inv = p.norm ? rsqrtf(s2 / (float)K + p.eps) : 1.0f;
            const float s0 = I4 ? 1.0f : (first ? rs0 : rsc[c]);
            float o;
            if (PAIR) {
                const float s1 = I4 ? 1.0f : (first ? rs1 : rsc[c + 8]);
                o = silu(a * inv * s0) * (a2 * inv * s1);
            } else {
                o = a * inv * s0;
                if (p.epi == BZ_EPI_RESIDUAL) {
                    const uint32_t rv = first ? resv : load_res(g);
                    o += __uint_as_float(p.res_f32 ? rv : rv << 16);
                }
            }
            const int col = b * ocols + c;
            const int64_t oi = (int64_t)m * p.ldo + col;
            if (p.out_f32)
                reinterpret_cast<float*>(p.out)[oi] = o;
            else
                reinterpret_cast<uint16_t*>(p.out)[oi] = f32_to_bf16(o);
            if (col < p.n_out2) {
                const int64_t oi2 = (int64_t)m * p.ldo2 + col;
                if (p.out_f32)
                    reinterpret_cast<float*>(p.out2)[oi2] = o;
                else
                    reinterpret_cast<uint16_t*>(p.out2)[oi2] = f32_to_bf16(o);
            }
        }
    }
}

// ---- host side -----------------------------------------------------------------


struct StreamLaunch {
    int nw, upw, mm;
    unsigned grid;
    size_t lds;
};

template <int WF, int MM, int UPW>
int launch_stream_kernel(const StreamParams& p, const StreamLaunch& l, hipStream_t st) {
    auto kern = gemv_stream<WF, MM, UPW>;
    if (l.lds > 65536 && raise_lds_limit(reinterpret_cast<const void*>(kern)) != BZ_OK) return BZ_ERR_LAUNCH;
    if (!stream_hot_ok(p)) return BZ_ERR_UNSUPPORTED;
    hipLaunchKernelGGL(kern, dim3(l.grid), dim3(l.nw * 64), l.lds, st, p.w, p.x, p.gamma, (int)p.chunk, (int)p.ldx, p.K,
                       p.NU, p.M, p.norm, p.x_lead, p);
    return hipGetLastError() == hipSuccess ? BZ_OK : BZ_ERR_LAUNCH;
}

template <int WF, int MM>
int launch_stream_upw(const StreamParams& p, const StreamLaunch& l, hipStream_t st) {
    switch (l.upw) {
        case 1: return launch_stream_kernel<WF, MM, 1>(p, l, st);
        case 2: return launch_stream_kernel<WF, MM, 2>(p, l, st);
        case 3: return launch_stream_kernel<WF, MM, 3>(p, l, st);
        case 4: return launch_stream_kernel<WF, MM, 4>(p, l, st);
        case 5: return launch_stream_kernel<WF, MM, 5>(p, l, st);
        case 6: return launch_stream_kernel<WF, MM, 6>(p, l, st);
        case 8: return launch_stream_kernel<WF, MM, 8>(p, l, st);
        case 10: return launch_stream_kernel<WF, MM, 10>(p, l, st);
        default: return BZ_ERR_INVALID_ARG;
    }
}

template <int WF>
int launch_stream_wf(const StreamParams& p, const StreamLaunch& l, hipStream_t st) {
    switch (l.mm) {
        case 1: return launch_stream_upw<WF, 1>(p, l, st);
        case 2: return launch_stream_upw<WF, 2>(p, l, st);
        case 4: return launch_stream_upw<WF, 4>(p, l, st);
        case 8: return launch_stream_upw<WF, 8>(p, l, st);
        default: return BZ_ERR_INVALID_ARG;
    }
}

// Tiled-format helpers (bz_tiled.hip).
bool is_tiled(int wf);
int tiled_units(int wf, int K);  // K / unit k, 0 when K cannot be tiled
int dequant_tiled(int wf, const void* w, int N, int K, int group, float* out, hipStream_t st);

// One explicit instantiation set per tiled format, each in its own
// translation unit (bz_gemv_stream_<fmt>.hip).
int launch_stream_i4t(const StreamParams& p, const StreamLaunch& l, hipStream_t st);
int launch_stream_i4tp(const StreamParams& p, const StreamLaunch& l, hipStream_t st);
int launch_stream_f8t(const StreamParams& p, const StreamLaunch& l, hipStream_t st);
int launch_stream_f8tp(const StreamParams& p, const StreamLaunch& l, hipStream_t st);

}  // namespace bz
