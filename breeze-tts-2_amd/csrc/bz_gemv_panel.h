// Several-row GEMV over the tiled weight formats (GEMV path 6, the "panel"
// kernel): up to 32 rows of x against an unpaired int4 or fp8 tiled weight,
// every weight byte streamed once.  A workgroup covers its row blocks over
// the whole K, or over one of nsl K slices when the x of a launch is large
// (every workgroup reads all of its K range of x from L2: 655 KB at M = 32,
// K = 10240 is about 6.5 us of one CU's L2 bandwidth, measured on MI355X).
//
// Replaces, for M > 2 (MTP draft verification plus CFG):
//   torch._weight_int4pack_mm (Int4Linear)          models/int4_linear.py:103-108
//   torch._scaled_mm (Fp8Linear, weight-only form)  models/fp8_linear.py:76-82
//
// Tiled formats: see bz_gemv_stream.h (16-row blocks; 64-byte units of 128
// int4 k or 64 fp8 k; a block's NU tiles of 1 KiB, then its scales).
//
// Work decomposition
//   * A workgroup owns T consecutive row blocks; its NW waves split the NU
//     units, UPW consecutive units each, and every wave runs its units over
//     all T blocks (split-K inside the workgroup, summed in a fixed order:
//     deterministic).
//   * x never goes through LDS memory: each wave loads the 16-byte pieces
//     of x its MFMAs multiply from global memory (L2) straight into
//     registers, once per unit for all T blocks, with range-checked buffer
//     loads (rows >= M and units past the block read as zeros and send no
//     request).  A load instruction reads 16 rows x 64 bytes; the four
//     lanes of a quad read one row's 64-byte run (lane 4 a + b: row a, piece
//     b), and ds_bpermute moves each piece to its MFMA lane a + 16 b (with
//     the MFMA lane order, a quad would touch four rows: measured 1.5x
//     slower at M = 32, K = 10240).
//   * Each wave keeps D units in flight (x pieces, T tiles and, for int4,
//     T scale quads per unit) in a rolling register pipeline.
//   * One workgroup barrier: the waves' partials go to LDS, then each thread
//     sums its outputs' partials over the waves in wave order.
//   * K slices (nsl > 1): the grid is (row-block groups) x nsl, the slices of
//     one group consecutive.  Each workgroup stores its fp32 sums to the
//     workspace ([nsl][M][N] after kTileCounters counters, 16-byte agent-scope
//     stores that reach the point of coherence), waits for its stores and
//     counts its arrival on the group's counter; the last arrival sums the
//     slices in slice order (independent of the arrival order), applies the
//     epilogue and resets the counter to zero for the next call.
//
// Arithmetic: v_mfma_f32_16x16x32_bf16 with A = 16 weight rows (lane l holds
// 16 bytes of tile row l % 16 at byte 16 (l / 16) of the unit, which is the
// A placement A[n][k] in lane n + 16 (k / 8)) and B = 16 rows of x (B[k][m]
// in lane m + 16 (k / 8)); one or two MFMAs per operand for rows 0-15 and
// 16-31.  D[n][m] lands in lane m + 16 (n / 4), element n % 4: each lane
// finishes 4 weight rows of one x row.
//   * int4: the lane's dword d gives MFMA d its four bf16 pairs
//     (128 + q_e, 128 + q_{e+4}) with one v_and_or_b32 each, so the x piece
//     of MFMA d is permuted to [x0 x4 x1 x5 x2 x6 x3 x7] (four v_perm_b32).
//     Per unit and weight row n:
//       sum_k x_k w_k = s_n D + (z_n - 136 s_n) X,   D = sum_k x_k (128 + q_k),
//     with X = sum of x over the unit's 128 k, from an MFMA with A = ones
//     (the same D placement: every element of a lane holds its row's X).
//   * fp8: gfx950's exact OCP e4m3 -> bf16 conversion of codes 0-7 and 8-15
//     gives the A operands of two MFMAs; the accumulator runs over all units
//     and the row scale multiplies the finished sum.
#pragma once

#include "bz_gemv_stream.h"

namespace bz {

struct PanelParams {
    const uint16_t* x;
    int64_t ldx;
    const uint8_t* w;
    int64_t chunk;  // bytes per row block
    const void* res;
    int64_t ldr;
    void* out;
    int64_t ldo;
    int M, K, NU, nblk;
    int epi, out_f32, res_f32;
    int nsl, ups;    // K slices and units per slice (nsl = 1: ups = NU)
    uint32_t* cnt;   // nsl > 1: per-group arrival counters (zero between calls)
    float* part;     // nsl > 1: fp32 sums [nsl][M][nblk * 16]
};

// Rows of x one launch takes, and the most waves of a workgroup.
constexpr int kPanelMaxRows = 32;
constexpr int kPanelMaxWaves = 16;
// Units per wave and row blocks per workgroup the kernel is instantiated for.
constexpr int kPanelUpw[] = {1, 2, 3, 4, 5, 6, 8, 10};
constexpr int kPanelBlocks[] = {1, 2, 3, 4, 5};

// Units in flight per wave: two, or one where a unit's registers are many
// (int4 with two row halves: 32 VGPRs of x pieces plus their permuted copy)
// or where a second unit measured slower (several blocks per workgroup with
// one row half).  fp8 with two row halves and several blocks keeps two:
// measured on MI355X, K2560 N20480 M = 32 14.1 -> 13.4 us (184 VGPRs, no
// spills), while two units made int4 K2560 N20480 at M = 8 / 16 and fp8 at
// M = 16 0.1-1.3 us slower, and int4 K10240 N2560 M = 32 over 2 blocks and 3
// K slices 12.7 -> 13.6 us.
__host__ __device__ constexpr int panel_depth(bool i4, int mt, int t, int upw) {
    return (i4 ? (t > 1 || mt == 2) : (t > 1 && mt == 1)) ? 1 : (upw <= 2 ? upw : 2);
}

// LDS: the waves' partials [wave][block][row half][x row % 16][weight row],
// fp32, then the last-arrival flag.
__host__ __device__ inline int panel_lds(int NW, int T, int MT) { return NW * T * MT * 256 * 4 + 16; }

// Lane g = l / 16 of a wave's 16-lane rows holds 16-byte piece g of its
// weight row (dwords M[g][0..3]).  An MFMA whose four lane rows hold one
// aligned 32-element run of k reads that run of x as one 64-byte piece per
// x row, so the pieces are redistributed across the rows:
//   int4: lane row g gets dword g of every piece, v[d] = M[d][g] (a 4 x 4
//   transpose: v_permlane32_swap exchanges the upper 32 lanes of its first
//   operand with the lower 32 of its second, v_permlane16_swap the odd
//   16-lane rows of its first with the even rows of its second);
//   fp8: rows 0, 1 keep their first 8 codes and receive the first 8 of rows
//   2, 3, which receive the last 8 of rows 0, 1: v[0..1] hold codes
//   k = 16 (g & 1) + 8 (g >> 1) + 0..7 of the unit, v[2..3] the same + 32.
__device__ __forceinline__ u32x4 transpose_pieces(u32x4 w) {
    const auto a02 = __builtin_amdgcn_permlane32_swap(w[0], w[2], false, false);
    const auto a13 = __builtin_amdgcn_permlane32_swap(w[1], w[3], false, false);
    const auto v01 = __builtin_amdgcn_permlane16_swap(a02[0], a13[0], false, false);
    const auto v23 = __builtin_amdgcn_permlane16_swap(a02[1], a13[1], false, false);
    return u32x4{v01[0], v01[1], v23[0], v23[1]};
}
__device__ __forceinline__ u32x4 swap_halves(u32x4 w) {
    const auto a02 = __builtin_amdgcn_permlane32_swap(w[0], w[2], false, false);
    const auto a13 = __builtin_amdgcn_permlane32_swap(w[1], w[3], false, false);
    return u32x4{a02[0], a13[0], a02[1], a13[1]};
}

// The fields the first loads need come as leading scalar arguments, which
// the hardware preloads into SGPRs at wave launch (kernarg preloading, as
// for the streaming kernels in bz_gemv_stream.h); the host passes the same
// values in the struct.
template <int WF, int MT, int T, int UPW>
__global__ void __launch_bounds__(T == 1 ? 1024 : 512) gemv_panel(const uint8_t* hw, const uint16_t* hx, int hchunk, int hldx,
                                                                  int hM, int hK, int hNU, int hnblk, int hnsl, int hups,
                                                                  PanelParams p) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    p.w = hw;
    p.x = hx;
    p.chunk = hchunk;
    p.ldx = hldx;
    p.M = hM;
    p.K = hK;
    p.NU = hNU;
    p.nblk = hnblk;
    p.nsl = hnsl;
    p.ups = hups;
    constexpr bool I4 = tiled_i4(WF);
    constexpr int D = panel_depth(I4, MT, T, UPW);
    constexpr int NX = I4 ? 4 : 2;     // x pieces (16 bytes) per unit and row half
    constexpr int UK = tiled_unit_k(WF);
    const int nthr = blockDim.x, NW = nthr >> 6;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 15, kq = lane >> 4;
    const int M = p.M;
    const int grp = (int)blockIdx.x / p.nsl, sl = (int)blockIdx.x - grp * p.nsl;
    const int blk0 = grp * T;
    const int ub = sl * p.ups, ue = min(p.NU, ub + p.ups);  // the slice's units
    const int NU = p.NU;
    const int u0 = ub + wave * UPW;

    // x pieces: MFMA lane j + 16 kq multiplies row m = 16 mt + j at
    // k = u UK + 32 d + (int4: 8 kq; fp8: 16 (kq & 1) + 8 (kq >> 1)), so the
    // four pieces of a row in one instruction are one aligned 64-byte run.
    // They are loaded by quads (lane 4 a + b reads row a's piece b: one
    // quad, one run) and moved to the MFMA lane a + 16 b with ds_bpermute.
    // Each unit's loads go through a buffer resource starting at the unit
    // (uniform: scalar registers), so a lane keeps one offset per row half;
    // rows >= M take an offset past every range (reads as zeros, no
    // request), as does every lane of a unit past the row (empty range).
    const int qa = lane >> 2, qb = lane & 3;
    // int4 with two row halves loads each quad's four pieces 64 bytes apart
    // (x in the tile's own piece order: lane a + 16 g of register d holds
    // k = 32 g + 8 d of row a), so the weight pieces need no transpose; it
    // saves 4 permlane swaps per tile and was measured faster only there
    // (int4 K2560 N20480 M = 32 14.5 -> 14.2 us; with one row half, M = 8 /
    // 16, about 1 us slower, where each quad reads four 16-byte pieces over
    // two lines of its row instead of one 64-byte run).
    constexpr bool XT = I4 && MT == 2;
    const int kx = I4 ? (XT ? 32 * qb : 8 * qb) : 16 * (qb & 1) + 8 * (qb >> 1);
    constexpr uint32_t kXStep = XT ? 16u : 64u;  // bytes between a lane's pieces d
    const uint32_t xbytes = (uint32_t)(((int64_t)(M - 1) * p.ldx + p.K) * 2);
    constexpr uint32_t kXOob = 0x80000000u;
    uint32_t xlo[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int m = 16 * mt + qa;
        xlo[mt] = m < M ? (uint32_t)(((int64_t)m * p.ldx + kx) * 2) : kXOob;
    }
    const int xsrc = quad_source(lane);
    auto xmove = [&](u32x4 v) -> u32x4 { return quad_to_mfma(v, xsrc); };
    // the workgroup's blocks: tiles and (int4) scale quads up to the end of
    // the slice; a block past the weight has empty ranges (zeros, no
    // requests) and is never stored, and a unit past the slice is past the
    // ranges
    __amdgpu_buffer_rsrc_t wrs[T], srs[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const bool live = blk0 + t < p.nblk;
        const uint8_t* chunk = p.w + (int64_t)(live ? blk0 + t : 0) * p.chunk;
        wrs[t] = buffer_rsrc(chunk, live ? (uint32_t)ue * 1024u : 0u);
        srs[t] = buffer_rsrc(chunk + (int64_t)NU * 1024, live && I4 ? (uint32_t)ue * 64u : 0u);
    }
    const uint32_t wlane = j * 64 + kq * 16, slane = kq * 16;

    u32x4 xv[UPW][MT][NX];
    u32x4 wv[UPW][T];
    u32x4 sv[UPW][T];
    auto issue = [&](int q) {
        const int u = u0 + q;
        const uint32_t ux = (uint32_t)u * UK * 2;
        const __amdgpu_buffer_rsrc_t xrs =
            buffer_rsrc(reinterpret_cast<const uint8_t*>(p.x) + ux, u < ue ? xbytes - ux : 0u);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int d = 0; d < NX; ++d) xv[q][mt][d] = buffer_ld16(xrs, xlo[mt] + kXStep * d);
#pragma unroll
        for (int t = 0; t < T; ++t) wv[q][t] = buffer_ld16_nt(wrs[t], (uint32_t)u * 1024u + wlane);
        if (I4) {
#pragma unroll
            for (int t = 0; t < T; ++t) sv[q][t] = buffer_ld16(srs[t], (uint32_t)u * 64u + slane);
        }
    };
#pragma unroll
    for (int q = 0; q < D; ++q) issue(q);
    __builtin_amdgcn_sched_barrier(0);

    f32x4_t acc[T][MT];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[t][mt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    const NibbleConsts nc;
    const u32x4 ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};  // bf16 1.0

    auto consume = [&](int q, bool next) {
        if (I4) {
            // the x pieces in the pair order of the unpacked nibbles, and X
            // (a plain sum: it takes them in that order too)
            u32x4 xp[MT][4];
            f32x4_t xs[MT];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                xs[mt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    const u32x4 v = xmove(xv[q][mt][d]);
                    xp[mt][d][0] = __builtin_amdgcn_perm(v[2], v[0], 0x05040100u);
                    xp[mt][d][1] = __builtin_amdgcn_perm(v[2], v[0], 0x07060302u);
                    xp[mt][d][2] = __builtin_amdgcn_perm(v[3], v[1], 0x05040100u);
                    xp[mt][d][3] = __builtin_amdgcn_perm(v[3], v[1], 0x07060302u);
                    xs[mt] = mfma_bf16(ones, xp[mt][d], xs[mt]);
                }
            }
            u32x4 wr[T], s4[T];
#pragma unroll
            for (int t = 0; t < T; ++t) {
                wr[t] = wv[q][t];
                s4[t] = sv[q][t];
            }
            // the next unit's loads go out here, once this unit's x pieces
            // are consumed: the scheduler may not hoist them (holding two
            // units' x pieces at once would spill)
            __builtin_amdgcn_sched_barrier(0);
            if (next) issue(q + D);
            __builtin_amdgcn_sched_barrier(0);
            // block by block: unpack its tile, 4 MFMAs per row half, scale
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const u32x4 v = XT ? wr[t] : transpose_pieces(wr[t]);
                u32x4 bq[4];
#pragma unroll
                for (int d = 0; d < 4; ++d)
#pragma unroll
                    for (int e = 0; e < 4; ++e) bq[d][e] = nib2_bf16(v[d] >> (4 * e), nc.mask, nc.magic);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    f32x4_t dv = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int d = 0; d < 4; ++d) dv = mfma_bf16(bq[d], xp[mt][d], dv);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float sc = bf16_lo(s4[t][r]);
                        const float zp = fmaf(-136.0f, sc, bf16_hi(s4[t][r]));
                        acc[t][mt][r] = fmaf(sc, dv[r], fmaf(zp, xs[mt][r], acc[t][mt][r]));
                    }
                }
            }
        } else {
            u32x4 b0[T], b1[T];
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const u32x4 v = swap_halves(wv[q][t]);
                b0[t][0] = fp8x2_bf16<false>(v[0]);
                b0[t][1] = fp8x2_bf16<true>(v[0]);
                b0[t][2] = fp8x2_bf16<false>(v[1]);
                b0[t][3] = fp8x2_bf16<true>(v[1]);
                b1[t][0] = fp8x2_bf16<false>(v[2]);
                b1[t][1] = fp8x2_bf16<true>(v[2]);
                b1[t][2] = fp8x2_bf16<false>(v[3]);
                b1[t][3] = fp8x2_bf16<true>(v[3]);
            }
            u32x4 x0[MT], x1[MT];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                x0[mt] = xmove(xv[q][mt][0]);
                x1[mt] = xmove(xv[q][mt][1]);
            }
            // the next unit's loads go out here, after this unit's registers
            // are consumed: the scheduler may not hoist them (holding two
            // units' x pieces at once would spill)
            __builtin_amdgcn_sched_barrier(0);
            if (next) issue(q + D);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int t = 0; t < T; ++t)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    acc[t][mt] = mfma_bf16(b0[t], x0[mt], acc[t][mt]);
                    acc[t][mt] = mfma_bf16(b1[t], x1[mt], acc[t][mt]);
                }
        }
    };
#pragma unroll
    for (int q = 0; q < UPW; ++q) consume(q, q + D < UPW);

    // park the wave's partials: red[((wave T + t) MT + mt) 256 + j 16 + n],
    // n = 4 kq + r (one 16-byte store per block and row half)
    float* red = reinterpret_cast<float*>(smem);
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
            *reinterpret_cast<f32x4_t*>(red + ((wave * T + t) * MT + mt) * 256 + j * 16 + 4 * kq) = acc[t][mt];
    __syncthreads();

    // each item, x row m and columns c..c+3 of the workgroup's 16 T: the sum
    // over the waves in wave order (one 16-byte LDS read per wave, all issued
    // before the first add: a wave slot the workgroup does not have is read
    // at the last present wave and added as zero, which leaves every sum
    // bit-identical to the plain loop over the present waves); then (one
    // slice) the epilogue, or (several slices) the partial.  The epilogue's
    // own inputs (residual, fp8 row scales) are loaded first, so their round
    // trip overlaps the LDS sums or the partials' loads.
    const int nq = 4 * T;  // 4-column groups of a row
    const int nitem = M * nq;
    const int wstride = T * MT * 256;
    const int n_out = p.nblk * 16;
    struct EpIn {
        float r[4];   // residual
        f32x4_t sc;   // fp8 row scales
    };
    auto ep_load = [&](int m, int c) {
        EpIn e;
        const int t = c >> 4, n = c & 15;
        const int col = blk0 * 16 + c;
#pragma unroll
        for (int q = 0; q < 4; ++q) e.r[q] = 0.0f;
        if (p.epi == BZ_EPI_RESIDUAL) {
            const int64_t ri = (int64_t)m * p.ldr + col;
#pragma unroll
            for (int q = 0; q < 4; ++q)
                e.r[q] = p.res_f32 ? reinterpret_cast<const float*>(p.res)[ri + q]
                                   : bf16_to_f32(reinterpret_cast<const uint16_t*>(p.res)[ri + q]);
        }
        e.sc = f32x4_t{1.0f, 1.0f, 1.0f, 1.0f};
        if (!I4)
            e.sc = *reinterpret_cast<const f32x4_t*>(p.w + (int64_t)(blk0 + t) * p.chunk + (int64_t)NU * 1024 + n * 4);
        return e;
    };
    auto ep_store = [&](f32x4_t a, const EpIn& e, int m, int c) {
        const int64_t oi = (int64_t)m * p.ldo + blk0 * 16 + c;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float v = a[q];
            if (!I4) v *= e.sc[q];
            if (p.epi == BZ_EPI_RESIDUAL) v += e.r[q];
            if (p.out_f32)
                reinterpret_cast<float*>(p.out)[oi + q] = v;
            else
                reinterpret_cast<uint16_t*>(p.out)[oi + q] = f32_to_bf16(v);
        }
    };
    // the partials of all slices through one buffer resource (host: nsl M N
    // fp32 < 2^31 bytes), 16-byte agent-scope accesses
    const __amdgpu_buffer_rsrc_t prs =
        buffer_rsrc(p.part, p.nsl > 1 ? (uint32_t)((int64_t)p.nsl * M * n_out * 4) : 0u);
    for (int it = tid; it < nitem; it += nthr) {
        const int m = it / nq, c = (it - m * nq) * 4;
        const int t = c >> 4, n = c & 15;
        if (blk0 + t >= p.nblk) continue;
        EpIn e;
        if (p.nsl == 1) e = ep_load(m, c);
        const float* rp = red + (t * MT + (m >> 4)) * 256 + (m & 15) * 16 + n;
        f32x4_t v[kPanelMaxWaves];
#pragma unroll
        for (int w = 0; w < kPanelMaxWaves; ++w) v[w] = *reinterpret_cast<const f32x4_t*>(rp + min(w, NW - 1) * wstride);
        f32x4_t a = {0.0f, 0.0f, 0.0f, 0.0f};
        const f32x4_t zero = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int w = 0; w < kPanelMaxWaves; ++w) a += w < NW ? v[w] : zero;
        if (p.nsl == 1)
            ep_store(a, e, m, c);
        else
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, a), prs,
                                                   (uint32_t)((((int64_t)sl * M + m) * n_out + blk0 * 16 + c) * 4), 0,
                                                   kCpolAgent);
    }
    if (p.nsl == 1) return;
    int& last_arrival = *reinterpret_cast<int*>(smem + panel_lds(NW, T, MT) - 16);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) {
        const unsigned prev = __hip_atomic_fetch_add(&p.cnt[grp], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last_arrival = prev == (unsigned)p.nsl - 1u;
    }
    __syncthreads();
    if (!last_arrival) return;
    // the last arrival: each item's slices in slice order, kPanelSumBatch
    // 16-byte loads in flight per batch (slice indices clamped into range)
    constexpr int kPanelSumBatch = 8;
    for (int it = tid; it < nitem; it += nthr) {
        const int m = it / nq, c = (it - m * nq) * 4;
        if (blk0 + (c >> 4) >= p.nblk) continue;
        const EpIn e = ep_load(m, c);
        const uint32_t off0 = (uint32_t)(((int64_t)m * n_out + blk0 * 16 + c) * 4);
        const uint32_t sstride = (uint32_t)((int64_t)M * n_out * 4);
        f32x4_t a = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int s0 = 0; s0 < p.nsl; s0 += kPanelSumBatch) {
            u32x4 v[kPanelSumBatch];
#pragma unroll
            for (int u = 0; u < kPanelSumBatch; ++u)
                v[u] = __builtin_amdgcn_raw_buffer_load_b128(prs, off0 + (uint32_t)min(s0 + u, p.nsl - 1) * sstride, 0,
                                                             kCpolAgent);
#pragma unroll
            for (int u = 0; u < kPanelSumBatch; ++u)
                if (s0 + u < p.nsl) a += __builtin_bit_cast(f32x4_t, v[u]);
        }
        ep_store(a, e, m, c);
    }
    if (tid == 0) __hip_atomic_store(&p.cnt[grp], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- host side -----------------------------------------------------------------

struct PanelLaunch {
    int nw, upw, mt, T;
    int nsl, ups;    // K slices and units per slice
    unsigned grid;   // row-block groups x nsl
    size_t lds;
    size_t ws;       // workspace bytes (nsl > 1)
};

template <int WF, int MT, int T, int UPW>
int launch_panel_kernel(const PanelParams& p, const PanelLaunch& l, hipStream_t st) {
    auto kern = gemv_panel<WF, MT, T, UPW>;
    if (l.lds > 65536 && raise_lds_limit(reinterpret_cast<const void*>(kern)) != BZ_OK) return BZ_ERR_LAUNCH;
    if (p.chunk > 0x7FFFFFFF || p.ldx > 0x7FFFFFFF) return BZ_ERR_UNSUPPORTED;
    hipLaunchKernelGGL(kern, dim3(l.grid), dim3(l.nw * 64), l.lds, st, p.w, p.x, (int)p.chunk, (int)p.ldx, p.M, p.K, p.NU,
                       p.nblk, p.nsl, p.ups, p);
    return hipGetLastError() == hipSuccess ? BZ_OK : BZ_ERR_LAUNCH;
}

template <int WF, int MT, int T>
int launch_panel_upw(const PanelParams& p, const PanelLaunch& l, hipStream_t st) {
    switch (l.upw) {
        case 1: return launch_panel_kernel<WF, MT, T, 1>(p, l, st);
        case 2: return launch_panel_kernel<WF, MT, T, 2>(p, l, st);
        case 3: return launch_panel_kernel<WF, MT, T, 3>(p, l, st);
        case 4: return launch_panel_kernel<WF, MT, T, 4>(p, l, st);
        case 5: return launch_panel_kernel<WF, MT, T, 5>(p, l, st);
        case 6: return launch_panel_kernel<WF, MT, T, 6>(p, l, st);
        case 8: return launch_panel_kernel<WF, MT, T, 8>(p, l, st);
        case 10: return launch_panel_kernel<WF, MT, T, 10>(p, l, st);
        default: return BZ_ERR_INVALID_ARG;
    }
}

template <int WF, int MT>
int launch_panel_t(const PanelParams& p, const PanelLaunch& l, hipStream_t st) {
    switch (l.T) {
        case 1: return launch_panel_upw<WF, MT, 1>(p, l, st);
        case 2: return launch_panel_upw<WF, MT, 2>(p, l, st);
        case 3: return launch_panel_upw<WF, MT, 3>(p, l, st);
        case 4: return launch_panel_upw<WF, MT, 4>(p, l, st);
        case 5: return launch_panel_upw<WF, MT, 5>(p, l, st);
        default: return BZ_ERR_INVALID_ARG;
    }
}

template <int WF>
int launch_panel_wf(const PanelParams& p, const PanelLaunch& l, hipStream_t st) {
    switch (l.mt) {
        case 1: return launch_panel_t<WF, 1>(p, l, st);
        case 2: return launch_panel_t<WF, 2>(p, l, st);
        default: return BZ_ERR_INVALID_ARG;
    }
}

// One instantiation set per unpaired tiled format (bz_gemv_panel_<fmt>.hip).
int launch_panel_i4t(const PanelParams& p, const PanelLaunch& l, hipStream_t st);
int launch_panel_f8t(const PanelParams& p, const PanelLaunch& l, hipStream_t st);

}  // namespace bz
