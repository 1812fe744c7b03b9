// Several-row tile kernel of the decode GEMV (gfx950 MFMA): M = 1..32 rows
// of x against int4 / fp8 / bf16 weights, every weight byte streamed from HBM
// once per launch.
//
// The row-sliced streaming kernels (bz_gemv_mfma.h, bz_gemv_i8.h) hold at
// most 4 rows of x per launch (16 on the int8 path for rows of <= 4096 k), so
// 16 or 32 rows re-stream the weights 2-8 times.  Here a workgroup owns a
// column block (NW = 4 or 8 waves x T tiles of 16 output columns) and one K
// slice:
//   * grid = column blocks x K slices; block b takes column block b / nsl and
//     slice b % nsl, so the slices of one column block run back to back and
//     its last arrival finds the partials recently written;
//   * the slice of x for all M rows (bf16) is staged in LDS, rows padded by
//     16 bytes so the 16 rows read by one quarter-wave hit distinct banks; the
//     first loads of x are issued before the first weights, so waiting for x
//     does not wait behind the weights (vector loads retire in order);
//   * a wave streams its T tiles over the slice's 64-byte units with the
//     operand placement of the bf16 MFMA kernel: lane l loads 16 bytes of
//     weight row l%16 at offset 16*(l/16) (the B operand of
//     v_mfma_f32_16x16x32_bf16), and MB = 1 or 2 A operands of 16 x rows
//     (rows 0-15, 16-31) come from LDS, so each unpacked weight feeds 16 or
//     32 rows;
//   * int4 units are scaled per group as in the bf16 MFMA kernel,
//     y += s * D + (z - 136 s) * X with X the unit's sum of x per row, kept
//     in LDS as [unit][row] so the 4 rows of a lane come in one 16-byte read;
//   * one slice: the epilogue (fp8 row scale, residual) is applied straight
//     from the accumulators.  Several slices: fp32 partials go to the
//     workspace with 16-byte agent-scope stores (they reach the point of
//     coherence without an L2 write-back), each workgroup waits for its
//     stores, counts its arrival on the column block's counter, and the last
//     one sums the slices in slice order (the result does not depend on
//     arrival order) with all its 16-byte loads of a batch of slices in
//     flight, applies the epilogue and resets the counter to zero for the
//     next call.  (Measured on MI355X, int4 K10240 N2560 M = 32: 4-byte
//     partial stores and loads in batches of 8 outputs x 4 slices made the
//     last arrival's sum a tail of several memory round trips.)
//
// Workspace: kTileCounters uint32 counters (zero before the first call; every
// call leaves them zero), then fp32 partials [nsl][N_out][MP], MP = M rounded
// up to a multiple of 4 (tile_part_rows).
#pragma once
#include "bz_gemv_mfma.h"

namespace bz {

constexpr int kTileMaxThreads = 512;  // 8 waves
constexpr int kTileXB = 8;            // 16-byte blocks of x per thread loaded ahead of the weights
constexpr int kTileCounters = 4096;   // column blocks per launch (counters at the workspace start)
constexpr size_t kTilePartOffset = (size_t)kTileCounters * 4;
constexpr int kTileMaxRows = 32;

struct TileParams {
    GemvParams p;
    int M;      // rows of x (<= 16 * MB)
    int ks;     // k per slice (a multiple of the format's unit)
    int nsl;    // K slices
    uint32_t* cnt;
    float* part;
    int64_t chunk;  // tiled formats: bytes per 16-row block
    int NU;         // tiled formats: units per row (K / unit k)
};

// Formats the tile kernel reads: the row-major ones (WF_I4ZP, WF_I4MIN,
// WF_FP8, WF_BF16) and the unpaired tiled formats (include/bz_gemv.h), whose
// 1 KiB tiles are exactly this kernel's per-wave unit loads (16 rows x 64
// bytes) made contiguous, with the int4 (s, z) pairs and fp8 row scales at
// the end of each 16-row block.
__host__ __device__ constexpr bool tile_tiled(int wf) { return wf == BZ_W_INT4_TILED || wf == BZ_W_FP8_TILED; }
__host__ __device__ constexpr bool tile_i4(int wf) { return is_int4(wf) || wf == BZ_W_INT4_TILED; }
__host__ __device__ constexpr bool tile_f8(int wf) { return wf == WF_FP8 || wf == BZ_W_FP8_TILED; }
__host__ __device__ constexpr bool tile_zp(int wf) { return wf == WF_I4ZP || wf == BZ_W_INT4_TILED; }
__host__ __device__ constexpr int tile_unit_k(int wf) { return tile_i4(wf) ? 128 : (tile_f8(wf) ? 64 : 32); }

struct TileLaunch {
    int MB, T, D, nw;
    size_t lds;
    unsigned grid;
};

// LDS row of x in elements: the slice plus 16 bytes of padding.
__host__ __device__ inline int tile_xrow(int ks) { return ks + 8; }

// LDS: x rows, the int4 unit sums, the last-arrival flag.  All of it is
// dynamic (no static __shared__), so a launch may raise the dynamic limit to
// the whole LDS.
struct TileLds {
    int xs, x128, flag, total;
};
__host__ __device__ inline TileLds tile_lds_layout(int M, int MB, int ks, int wf) {
    TileLds L;
    L.xs = 0;
    L.x128 = align16(M * tile_xrow(ks) * 2);
    L.flag = L.x128 + (tile_i4(wf) ? align16((ks / 128) * 16 * MB * 4) : 0);
    L.total = L.flag + 16;
    return L;
}

// Stage one 8-element block of x row m at slice element 8*kq.  int4 blocks
// are permuted [x0 x4 x1 x5 x2 x6 x3 x7] to pair with the nibble pairs, and
// 16 consecutive lanes (one 128-k unit of one row) sum their blocks into
// x128[unit][row].
template <int WF>
__device__ __forceinline__ void tile_stage(u32x4 v, int m, int kq, uint16_t* xs, float* x128, int xrow, int rstride) {
    u32x4 o = v;
    if (tile_i4(WF)) {
        // (x_q, x_{q+4}) pairs by byte permutes; the block's sum by v_dot2 with (1, 1)
        o[0] = __builtin_amdgcn_perm(v[2], v[0], 0x05040100u);
        o[1] = __builtin_amdgcn_perm(v[2], v[0], 0x07060302u);
        o[2] = __builtin_amdgcn_perm(v[3], v[1], 0x05040100u);
        o[3] = __builtin_amdgcn_perm(v[3], v[1], 0x07060302u);
        float cs = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q) cs = dot2(v[q], 0x3F803F80u, cs);
        cs = sum16(cs);
        if ((kq & 15) == 0) x128[(kq >> 4) * rstride + m] = cs;
    }
    *reinterpret_cast<u32x4*>(xs + m * xrow + kq * 8) = o;
}

// Epilogue of one output: fp8 row scale, residual, store.
template <int WF>
__device__ __forceinline__ void tile_store(const TileParams& tp, float v, int r, int c) {
    const GemvParams& p = tp.p;
    if (WF == WF_FP8) v *= reinterpret_cast<const float*>(p.sc0)[c];
    if (WF == BZ_W_FP8_TILED)
        v *= reinterpret_cast<const float*>(p.w + (int64_t)(c >> 4) * tp.chunk + (int64_t)tp.NU * 1024)[c & 15];
    if (p.epi == BZ_EPI_RESIDUAL) {
        const int64_t idx = (int64_t)r * p.ldr + c;
        v += p.res_f32 ? reinterpret_cast<const float*>(p.res)[idx]
                       : bf16_to_f32(reinterpret_cast<const uint16_t*>(p.res)[idx]);
    }
    const int64_t oi = (int64_t)r * p.ldo + c;
    if (p.out_f32)
        reinterpret_cast<float*>(p.out)[oi] = v;
    else
        reinterpret_cast<uint16_t*>(p.out)[oi] = f32_to_bf16(v);
}

// Partials of one slice, column-major: the MP = M rounded up to 4 rows of
// column c at [c * MP, c * MP + MP), so the four consecutive rows an MFMA lane
// holds (rows 4 kb .. 4 kb + 3 of column j) are one 16-byte store and the last
// arrival reads them back as one 16-byte load per slice.  Rows M..MP-1 hold
// sums of clamped x rows and are never stored as outputs.
__host__ __device__ inline int tile_part_rows(int M) { return (M + 3) & ~3; }

// The last arrival's sum of a column block's partials over the slices, in
// slice order, and the epilogue: each thread takes G groups of four rows of
// one column per pass and has G x RS 16-byte loads of partials in flight per
// batch of RS slices (slice and group indices clamped into range, so the
// loads stay straight-line).  Loads and stores of partials carry the
// agent-scope cache policy (sc1): they reach the point of coherence, not a
// non-coherent L2 line of another XCD.
template <int WF, int G, int RS>
__device__ __forceinline__ void tile_sum_slices(const TileParams& tp, int cb, int CBW, int64_t sstride, int tid,
                                                int nthr) {
    const GemvParams& p = tp.p;
    const int nsl = tp.nsl, M = tp.M, MP = tile_part_rows(M);
    const int rq = MP >> 2;             // groups of four rows per column
    const int ngrp = CBW * rq;          // groups of the column block
    const int c0 = cb * CBW;
    for (int i0 = 0; i0 < ngrp; i0 += G * nthr) {
        f32x4_t sum[G];
        uint32_t off[G];
#pragma unroll
        for (int q = 0; q < G; ++q) {
            sum[q] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
            const int i = min(i0 + tid + q * nthr, ngrp - 1);
            const int cl = i / rq, g = i - cl * rq;
            off[q] = (uint32_t)((min(c0 + cl, p.n_out - 1) * MP + 4 * g) * 4);
        }
        for (int s0 = 0; s0 < nsl; s0 += RS) {
            u32x4 v[G][RS];
#pragma unroll
            for (int u = 0; u < RS; ++u) {
                const __amdgpu_buffer_rsrc_t r =
                    buffer_rsrc(tp.part + min(s0 + u, nsl - 1) * sstride, (uint32_t)(sstride * 4));  // uniform
#pragma unroll
                for (int q = 0; q < G; ++q) v[q][u] = __builtin_amdgcn_raw_buffer_load_b128(r, off[q], 0, kCpolAgent);
            }
#pragma unroll
            for (int q = 0; q < G; ++q)
#pragma unroll
                for (int u = 0; u < RS; ++u)
                    if (s0 + u < nsl)
#pragma unroll
                        for (int e = 0; e < 4; ++e) sum[q][e] += __uint_as_float(v[q][u][e]);
        }
#pragma unroll
        for (int q = 0; q < G; ++q) {
            const int i = i0 + tid + q * nthr;
            if (i >= ngrp) continue;
            const int cl = i / rq, g = i - cl * rq;
            const int c = c0 + cl;
            if (c >= p.n_out) continue;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (4 * g + e < M) tile_store<WF>(tp, sum[q][e], 4 * g + e, c);
        }
    }
}

// The fields the first loads need come as leading scalar arguments, which
// the hardware preloads into SGPRs at wave launch (kernarg preloading, as
// for the other GEMV kernels); the host passes the same values in the struct.
template <int WF, int MB, int T, int D>
__global__ void __launch_bounds__(kTileMaxThreads) gemv_tile(const uint16_t* hx, const uint8_t* hw, const void* hsc0,
                                                             int hldx, int hrow_bytes, int hK, int hM, int hks, int hnsl,
                                                             int hchunk, int hNU, TileParams tp) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    tp.p.x = hx;
    tp.p.w = hw;
    tp.p.sc0 = hsc0;
    tp.p.ldx = hldx;
    tp.p.row_bytes = hrow_bytes;
    tp.p.K = hK;
    tp.M = hM;
    tp.ks = hks;
    tp.nsl = hnsl;
    tp.chunk = hchunk;
    tp.NU = hNU;
    const GemvParams& p = tp.p;
    constexpr int UK = tile_unit_k(WF);
    constexpr int RS = 16 * MB;  // x128 row stride (rows per unit)
    const int nthr = blockDim.x, NW = nthr >> 6;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 15, kb = lane >> 4;
    const int M = tp.M, nsl = tp.nsl;
    const int cb = (int)blockIdx.x / nsl, sl = (int)blockIdx.x - cb * nsl;
    const int k0 = sl * tp.ks;
    const int kl = min(tp.ks, p.K - k0);  // host: a multiple of UK, > 0
    const int nu = kl / UK;
    const int xrow = tile_xrow(tp.ks);
    const int col0 = (cb * NW + wave) * 16 * T;  // wave-uniform
    const bool active = col0 < p.n_out;

    const TileLds L = tile_lds_layout(M, MB, tp.ks, WF);
    uint16_t* xs = reinterpret_cast<uint16_t*>(smem + L.xs);
    float* x128 = reinterpret_cast<float*>(smem + L.x128);
    int& last_arrival = *reinterpret_cast<int*>(smem + L.flag);

    // 0. the first blocks of the x slice.  Block tid + nthr i is row m, block
    //    kq of that row; (m, kq) advance by a uniform step, so there is one
    //    division per thread.  Rows past the end load row M-1 (never staged):
    //    the loads stay straight-line.
    const int nblk = kl >> 3;
    const int dm = nthr / nblk, dk = nthr - dm * nblk;
    const int m_first = tid / nblk, kq_first = tid - m_first * nblk;
    const uint16_t* xb = p.x + k0;
    const int ldx = (int)p.ldx;  // host: M * ldx < 2^31
    auto advance = [&](int& m, int& kq) {
        kq += dk;
        m += dm;
        if (kq >= nblk) {
            kq -= nblk;
            ++m;
        }
    };
    u32x4 xr[kTileXB];
    {
        int m = m_first, kq = kq_first;
#pragma unroll
        for (int i = 0; i < kTileXB; ++i) {
            xr[i] = ldg16(xb + min(m, M - 1) * ldx + kq * 8);
            advance(m, kq);
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // 1. the first D units of weights (+ int4 group scales)
    u32x4 buf[D][T];
    uint32_t scb[D][T];
    const int ub0 = k0 / UK;
    uint32_t loff[T];  // lane offset inside the tile: row (clamped to the last column) and 16-byte slot
    uint32_t soff[T];  // int4: the lane's row in the scale arrays ([G][N] pairs, or [N][G])
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const int lr = min(j, max(p.n_out - 1 - (col0 + 16 * t), 0));
        loff[t] = tile_tiled(WF) ? (uint32_t)(j * 64 + kb * 16)
                                 : __umul24((uint32_t)lr, (uint32_t)p.row_bytes) + (uint32_t)(kb * 16);
        const int row = min(col0 + 16 * t + j, p.n_out - 1);
        soff[t] = WF == WF_I4ZP ? (uint32_t)row : (uint32_t)row * (uint32_t)p.G;
    }
    auto issue = [&](int d, StepCursor c) {
        const int u = ub0 + c.ch;
        const int g = (u * 128) >> p.glog2;  // one group per unit (group >= 128)
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int ct = min(col0 + 16 * t, p.n_out - 1);
            if (tile_tiled(WF)) {
                // the tile of unit u in the 16-row block of column ct (uniform), its scales after the tiles
                const uint8_t* blk = p.w + (int64_t)(ct >> 4) * tp.chunk;
                buf[d][t] = ldg16_nt(blk + (int64_t)u * 1024 + loff[t]);
                if (tile_i4(WF))
                    scb[d][t] = *reinterpret_cast<const uint32_t*>(blk + (int64_t)tp.NU * 1024 + u * 64 + j * 4);
                continue;
            }
            // row-major rows: plain loads (each wave instruction reads 64 bytes of
            // 16 rows, and a row's next 64 bytes share the cache line; the
            // non-temporal hint measured up to 4 us slower at fp8 K2560 N20480)
            const uint8_t* base = p.w + (int64_t)ct * p.row_bytes + (int64_t)u * 64;  // uniform
            buf[d][t] = ldg16(base + loff[t]);
            if (WF == WF_I4ZP) {
                scb[d][t] = (reinterpret_cast<const uint32_t*>(p.sc0) + (int64_t)g * p.N)[soff[t]];
            } else if (WF == WF_I4MIN) {
                scb[d][t] = (uint32_t)(reinterpret_cast<const uint16_t*>(p.sc0) + g)[soff[t]] |
                            ((uint32_t)(reinterpret_cast<const uint16_t*>(p.sc1) + g)[soff[t]] << 16);
            }
        }
    };
    StepCursor ic{0, 0};
    if (active) pipeline_prime<0, D>(nu, 1, nu, 0, ic, issue);
    __builtin_amdgcn_sched_barrier(0);

    // 2. stage x (the rest of the slice is loaded here, behind the weights,
    //    kTileXB blocks per thread in flight).  m < M is uniform over each
    //    aligned 16-lane group for int4 (nblk is a multiple of 16), as the
    //    unit sums need.
    {
        int m = m_first, kq = kq_first;
#pragma unroll
        for (int i = 0; i < kTileXB; ++i) {
            if (m < M) tile_stage<WF>(xr[i], m, kq, xs, x128, xrow, RS);
            advance(m, kq);
        }
        while (m < M) {
            int mi[kTileXB], ki[kTileXB];
#pragma unroll
            for (int i = 0; i < kTileXB; ++i) {
                mi[i] = m;
                ki[i] = kq;
                xr[i] = ldg16(xb + min(m, M - 1) * ldx + kq * 8);
                advance(m, kq);
            }
#pragma unroll
            for (int i = 0; i < kTileXB; ++i)
                if (mi[i] < M) tile_stage<WF>(xr[i], mi[i], ki[i], xs, x128, xrow, RS);
        }
    }
    __syncthreads();

    // 3. every unit of the slice
    f32x4_t acc[T][MB];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[t][mb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    const uint16_t* xa[MB];  // this lane's A row (clamped to the last row of x) at its 16-byte slot
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
        xa[mb] = xs + min(16 * mb + j, M - 1) * xrow + kb * (tile_i4(WF) ? 32 : (tile_f8(WF) ? 16 : 8));
    const NibbleConsts nc;
    auto consume = [&](int d, StepCursor c) {
        const int u = c.ch;
        if (tile_i4(WF)) {
            u32x4 a[MB][4];
            f32x4_t X[MB];
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
                for (int dd = 0; dd < 4; ++dd) a[mb][dd] = *reinterpret_cast<const u32x4*>(xa[mb] + u * 128 + dd * 8);
                X[mb] = *reinterpret_cast<const f32x4_t*>(x128 + u * RS + 16 * mb + 4 * kb);
            }
#pragma unroll
            for (int t = 0; t < T; ++t) {
                f32x4_t dacc[MB];
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) dacc[mb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int dd = 0; dd < 4; ++dd) {
                    u32x4 bv;
#pragma unroll
                    for (int sh = 0; sh < 4; ++sh) bv[sh] = nib2_bf16(buf[d][t][dd] >> (4 * sh), nc.mask, nc.magic);
#pragma unroll
                    for (int mb = 0; mb < MB; ++mb) dacc[mb] = mfma_bf16(a[mb][dd], bv, dacc[mb]);
                }
                const uint32_t e = scb[d][t];
                const float s = bf16_lo(e);
                const float zp = fmaf(tile_zp(WF) ? -136.0f : -128.0f, s, bf16_hi(e));
#pragma unroll
                for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                    for (int q = 0; q < 4; ++q) acc[t][mb][q] = fmaf(s, dacc[mb][q], fmaf(zp, X[mb][q], acc[t][mb][q]));
            }
        } else if (tile_f8(WF)) {
            u32x4 a0[MB], a1[MB];
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                a0[mb] = *reinterpret_cast<const u32x4*>(xa[mb] + u * 64);
                a1[mb] = *reinterpret_cast<const u32x4*>(xa[mb] + u * 64 + 8);
            }
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const u32x4 w = buf[d][t];
                const u32x4 b0 = {fp8x2_bf16<false>(w[0]), fp8x2_bf16<true>(w[0]), fp8x2_bf16<false>(w[1]),
                                  fp8x2_bf16<true>(w[1])};
                const u32x4 b1 = {fp8x2_bf16<false>(w[2]), fp8x2_bf16<true>(w[2]), fp8x2_bf16<false>(w[3]),
                                  fp8x2_bf16<true>(w[3])};
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) {
                    acc[t][mb] = mfma_bf16(a0[mb], b0, acc[t][mb]);
                    acc[t][mb] = mfma_bf16(a1[mb], b1, acc[t][mb]);
                }
            }
        } else {
            u32x4 a0[MB];
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) a0[mb] = *reinterpret_cast<const u32x4*>(xa[mb] + u * 32);
#pragma unroll
            for (int t = 0; t < T; ++t)
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) acc[t][mb] = mfma_bf16(a0[mb], buf[d][t], acc[t][mb]);
        }
    };
    if (active) pipeline_run<D>(nu, 1, nu, 0, ic, issue, consume);

    // 4a. one slice: epilogue from the accumulators (lane: column j of each
    //     tile, rows 16 mb + 4 kb + q)
    if (nsl == 1) {
        if (!active) return;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int c = col0 + 16 * t + j;
            if (c >= p.n_out) continue;
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int r = 16 * mb + 4 * kb + q;
                    if (r < M) tile_store<WF>(tp, acc[t][mb][q], r, c);
                }
        }
        return;
    }

    // 4b. several slices: partials (column-major, 16-byte agent-scope
    //    stores), arrival, and the last arrival's sum.  Partial offsets inside
    //    a slice are 32-bit (host: MP * N_out * 4 < 2^31).
    const int MP = tile_part_rows(M);
    const int64_t sstride = (int64_t)MP * p.n_out;
    if (active) {
        const __amdgpu_buffer_rsrc_t prs = buffer_rsrc(tp.part + sl * sstride, (uint32_t)(sstride * 4));  // uniform
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int c = col0 + 16 * t + j;
            if (c >= p.n_out) continue;
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                const int r0 = 16 * mb + 4 * kb;
                if (r0 < M)
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[t][mb]), prs,
                                                           (uint32_t)((c * MP + r0) * 4), 0, kCpolAgent);
            }
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) {
        const unsigned prev = __hip_atomic_fetch_add(&tp.cnt[cb], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last_arrival = prev == (unsigned)nsl - 1u;
    }
    __syncthreads();
    if (!last_arrival) return;
    // The sum over slices, in slice order: two groups of four outputs per
    // thread and eight slices of each in flight per batch (M = 32 of a
    // 128-column block over 512 threads: one pass, batches of 16 loads).
    const int CBW = NW * 16 * T;  // columns of a block
    tile_sum_slices<WF, 2, 8>(tp, cb, CBW, sstride, tid, nthr);
    if (tid == 0) __hip_atomic_store(&tp.cnt[cb], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int WF, int MB, int T, int D>
int launch_tile_kernel(const TileParams& tp, const TileLaunch& l, hipStream_t st) {
    auto kern = gemv_tile<WF, MB, T, D>;
    if (l.lds > 65536 && raise_lds_limit(reinterpret_cast<const void*>(kern)) != BZ_OK) return BZ_ERR_LAUNCH;
    if (tp.p.ldx > 0x7FFFFFFF || tp.p.row_bytes > 0x7FFFFFFF || tp.chunk > 0x7FFFFFFF) return BZ_ERR_UNSUPPORTED;
    hipLaunchKernelGGL(kern, dim3(l.grid), dim3(l.nw * 64), l.lds, st, tp.p.x, tp.p.w, tp.p.sc0, (int)tp.p.ldx,
                       (int)tp.p.row_bytes, tp.p.K, tp.M, tp.ks, tp.nsl, (int)tp.chunk, tp.NU, tp);
    return hipGetLastError() == hipSuccess ? BZ_OK : BZ_ERR_LAUNCH;
}

template <int WF, int MB, int T>
int launch_tile_depth(const TileParams& tp, const TileLaunch& l, hipStream_t st) {
    switch (l.D) {
        case 2: return launch_tile_kernel<WF, MB, T, 2>(tp, l, st);
        case 4: return launch_tile_kernel<WF, MB, T, 4>(tp, l, st);
        case 8: return launch_tile_kernel<WF, MB, T, 8>(tp, l, st);
        default: return BZ_ERR_INVALID_ARG;
    }
}

template <int WF>
int launch_tile_wf(const TileParams& tp, const TileLaunch& l, hipStream_t st) {
    if (l.MB == 1) return l.T == 1 ? launch_tile_depth<WF, 1, 1>(tp, l, st) : launch_tile_depth<WF, 1, 2>(tp, l, st);
    if (l.MB == 2) return l.T == 1 ? launch_tile_depth<WF, 2, 1>(tp, l, st) : launch_tile_depth<WF, 2, 2>(tp, l, st);
    return BZ_ERR_INVALID_ARG;
}

int launch_tile_i4zp(const TileParams& tp, const TileLaunch& l, hipStream_t st);
int launch_tile_i4min(const TileParams& tp, const TileLaunch& l, hipStream_t st);
int launch_tile_fp8(const TileParams& tp, const TileLaunch& l, hipStream_t st);
int launch_tile_bf16(const TileParams& tp, const TileLaunch& l, hipStream_t st);
int launch_tile_i4t(const TileParams& tp, const TileLaunch& l, hipStream_t st);
int launch_tile_f8t(const TileParams& tp, const TileLaunch& l, hipStream_t st);

// The descriptor checks of bz_gemv (bz_gemv.hip), without launching: BZ_OK or
// the status bz_gemv would return for a malformed descriptor.
int gemv_check_desc(const bz_gemv_desc* d);

}  // namespace bz
