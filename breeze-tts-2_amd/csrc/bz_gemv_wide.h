// Streaming decode GEMV over several row blocks per workgroup (GEMV path 5
// for the tiled formats when the rule or cfg_tiles asks for it).
//
// Same weight layout, arithmetic and per-unit sums as the one-block kernel
// of bz_gemv_stream.h (and so the same reference functions replaced:
// rms_gemv_kernel + gemv_epilogue_kernel, models/fused/kernels.py:41-138;
// torch._weight_int4pack_mm, models/int4_linear.py:103-108; torch._scaled_mm
// in its weight-only form, models/fp8_linear.py:76-82).  What changes is the
// work decomposition, for weights with more 16-row blocks than the GPU has
// CUs (gate|up N = 20480: 1280 blocks):
//   * workgroup g covers T consecutive row blocks [g T, g T + T); its NW
//     waves own the same UPW units of every block, so each wave stages the x
//     of its units once and then streams T x UPW tiles.  With one workgroup
//     per CU, every wave of the CU issues its x loads before any weight load
//     (an s_barrier after the x issue, not a wait for the data), so x does
//     not queue behind weight tiles.  Measured on MI355X against one block
//     per workgroup (1280 workgroups, 5 per CU): the x of the last workgroups
//     placed on a CU arrived up to 5 us after their start, behind the tiles
//     of the four before them, and those workgroups ended 2 us after the
//     median one;
//   * a rolling pipeline of UPW register slots across the blocks: slot q
//     holds unit q of the current block and is refilled with unit q of the
//     next block as soon as its tile is unpacked, so UPW tiles stay in flight
//     through the block boundaries (two register sets, for even and odd
//     blocks; a unit past the row, or a block past the workgroup's last,
//     reads as zeros without a memory request, so every wait counts a fixed
//     number of loads);
//   * each block's per-wave partials are parked in LDS when its last unit is
//     done (and zeros in the slots of waves the workgroup does not have);
//     after one workgroup barrier each output is finished by one lane: its
//     16 wave slots read as float4 runs and added in wave order (fixed,
//     timing-independent), 1/rms, the fp8 row scale, SiLU-gate or residual.
//     The fp8 row scales and the residual of a lane's first output are
//     loaded before the main loop.
#pragma once

#include "bz_gemv_stream.h"

namespace bz {

// LDS carve-up (bytes): x rows as bf16 (row stride 2K + 16), the int4
// per-unit sums X [row][unit], each wave's sum of x^2 per row [row][16 wave
// slots] and the partial dot products [block][row][column][16 wave slots].
struct WideLds {
    int xs, xst, sq, red, total;
};
__host__ __device__ inline WideLds wide_lds(int wf, int M, int K, int T) {
    WideLds L;
    L.xs = 0;
    L.xst = align16(M * stream_x_row_bytes(K));
    L.sq = L.xst + align16(tiled_i4(wf) ? M * (K / 128) * 4 : 0);
    L.red = L.sq + align16(M * 16 * 4);
    L.total = L.red + align16(T * M * 16 * 16 * 4);
    return L;
}

// Units per wave the wide kernel is instantiated for (int4 up to 5 over one
// or two rows of x and up to 4 over more: beyond that the two tile sets and
// the accumulators do not fit the 128 registers of a 16-wave workgroup
// without spilling), and the most row blocks of one workgroup.
constexpr int kWideUpw[] = {2, 3, 4, 5, 6, 8, 10};
__host__ __device__ constexpr int wide_max_upw(int wf, int mm) { return tiled_i4(wf) ? (mm <= 2 ? 5 : 4) : 10; }
constexpr int kWideMaxBlocks = 8;

// TC > 0: the row blocks per workgroup fixed at compile time (every
// workgroup takes exactly TC, the host checks that TC divides the blocks), so
// the block loop unrolls completely; TC = 0 takes T at run time.
template <int WF, int MM, int UPW, int TC = 0>
__global__ void __launch_bounds__(1024) gemv_wide(const uint8_t* hw, const uint16_t* hx, const uint16_t* hg, int hchunk,
                                                  int hldx, int hK, int hNU, int hM, int hnorm, int T, int nblk,
                                                  StreamParams p) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    stream_hot(p, hw, hx, hg, hchunk, hldx, hK, hNU, hM, hnorm);  // the preloaded arguments (bz_gemv_stream.h)
    constexpr bool I4 = tiled_i4(WF);
    constexpr bool PAIR = tiled_paired(WF);
    constexpr int BPU = tiled_unit_k(WF) / 8;   // blocks of 8 x values per unit
    constexpr int RK = (UPW * BPU + 63) / 64;   // rounds of blocks per lane over a wave's slice
    constexpr int NXL = RK * (1 + MM) <= 12 ? RK * (1 + MM) : 12;
    const int nthr = blockDim.x, NW = nthr >> 6;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 15, kq = lane >> 4;
    const int M = p.M, K = p.K, NU = p.NU;
    if constexpr (TC > 0) T = TC;
    const int b0 = blockIdx.x * T;
    const int nb = TC > 0 ? TC : min(T, nblk - b0);
    const int ocols = PAIR ? 8 : 16;

    const WideLds L = wide_lds(WF, M, K, T);
    uint8_t* xs = smem + L.xs;
    float* xst = reinterpret_cast<float*>(smem + L.xst);
    float* sq = reinterpret_cast<float*>(smem + L.sq);
    float* red = reinterpret_cast<float*>(smem + L.red);
    const int xrow = stream_x_row_bytes(K);

    const int u0 = wave * UPW;
    const int nu = max(0, min(UPW, NU - u0));
    const int kb0 = u0 * BPU, nkb = nu * BPU;

    // 0. the slice's x and gamma: load t = r (1 + MM) + s is gamma (s = 0) or
    //    x row s - 1 at block kb0 + lane + 64 r; range-checked, so a lane past
    //    the slice reads zeros and sends no request
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
    // the first output this lane finishes in the epilogue (block, row,
    // column): its fp8 row scale(s) and residual, loaded now
    const int g0 = tid;
    const int nout = nb * M * ocols;
    auto out_coords = [&](int g, int& jb, int& m, int& c) {
        c = g & (ocols - 1);
        const int jm = PAIR ? g >> 3 : g >> 4;
        jb = jm / M;
        m = jm - jb * M;
    };
    auto load_res = [&](int jb, int m, int c) -> uint32_t {
        const int64_t ri = (int64_t)m * p.ldr + (b0 + jb) * ocols + c;
        return p.res_f32 ? reinterpret_cast<const uint32_t*>(p.res)[ri]
                         : (uint32_t)reinterpret_cast<const uint16_t*>(p.res)[ri];
    };
    auto row_scale = [&](int jb, int c) -> const float* {
        return reinterpret_cast<const float*>(p.w + (int64_t)(b0 + jb) * p.chunk + (int64_t)NU * 1024) + c;
    };
    float rs0 = 1.0f, rs1 = 1.0f;
    uint32_t resv = 0u;
    if (g0 < nout) {
        int jb, m, c;
        out_coords(g0, jb, m, c);
        if (!I4) {
            rs0 = row_scale(jb, c)[0];
            if (PAIR) rs1 = row_scale(jb, c)[8];
        }
        if (p.epi == BZ_EPI_RESIDUAL) resv = load_res(jb, m, c);
    }
    // tiles of the workgroup's blocks through one buffer resource: tile q of
    // block jb is unit u0 + q of row block b0 + jb; with int4 the lane's
    // (s, z) pair of that unit comes with it
    const __amdgpu_buffer_rsrc_t wrs = buffer_rsrc(p.w + (int64_t)b0 * p.chunk, (uint32_t)((int64_t)nb * p.chunk));
    // two register sets with fixed roles (a: even blocks, b: odd blocks), so
    // no tile register is carried around the block loop (a carried one made
    // the compiler wait for every load in flight at each block)
    u32x4 wa[UPW], wb[UPW];
    uint32_t sa[UPW], sb[UPW];
    auto issue = [&](int jb, int q, u32x4* wv, uint32_t* sc) {  // unit q of block jb into slot q
        const bool ok = jb < nb && u0 + q < NU;
        const uint32_t base = (uint32_t)(jb * p.chunk);
        wv[q] = buffer_ld16_nt(wrs, ok ? base + (uint32_t)(u0 + q) * 1024u + j * 64 + kq * 16 : kBufferOob);
        if (I4) sc[q] = buffer_ld4(wrs, ok ? base + (uint32_t)NU * 1024u + (uint32_t)(u0 + q) * 64u + j * 4 : kBufferOob);
    };
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();  // every wave's x loads are issued before any weight load
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < UPW; ++q) issue(0, q, wa, sa);
    __builtin_amdgcn_sched_barrier(0);

    // 1. stage the slice while the first tiles are in flight (as the
    //    one-block kernel: u = bf16(gamma x) or x; int4 blocks stored
    //    [x0 x4 x1 x5 x2 x6 x3 x7] with their unit's sum X)
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
#pragma unroll
    for (int r = 0; r < RK; ++r) {
        if (r * 64 < nkb) {
            const int t0 = r * (1 + MM);
            const u32x4 g = t0 < NXL ? xl[t0] : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
            for (int m = 0; m < MM; ++m) {
                if (m < M) {
                    const int t = t0 + 1 + m;
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
    if (p.norm) {  // the wave's sum of x^2 per row: its four 16-lane rows added, one slot per wave
#pragma unroll
        for (int m = 0; m < MM; ++m) {
            const float w4 = rows4_sum_lane63(sum16_dpp(ss[m]));
            if (lane == 63 && m < M) {
                sq[m * 16 + wave] = w4;
                for (int s2 = NW + wave; s2 < 16; s2 += NW) sq[m * 16 + s2] = 0.0f;  // slots of absent waves
            }
        }
    }
    // the wave reads back only what it wrote (LDS operations of one wave
    // complete in order): no workgroup barrier here
    __builtin_amdgcn_wave_barrier();

    // 2. the blocks in order; slot q's tile is unpacked, refilled with unit q
    //    of the next block, then multiplied.  A unit past the row reads x and
    //    X at the row's last unit (staged by this wave) and multiplies them by
    //    zero weights.
    const uint8_t* xa = xs + min(j, M - 1) * xrow;  // the x row this lane supplies to A
    const NibbleConsts nc;
    // block jb from set (cw, cs); slot q refilled with unit q of block jb + 1
    // into set (nw2, ns2) as soon as its tile is unpacked
    auto run_block = [&](int jb, const u32x4* cw, const uint32_t* cs, u32x4* nw2, uint32_t* ns2) {
        float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        f32x4_t facc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int q = 0; q < UPW; ++q) {
            const int u = min(u0 + q, NU - 1);
            if (I4) {
                u32x4 bq[4];
#pragma unroll
                for (int d = 0; d < 4; ++d)
#pragma unroll
                    for (int e = 0; e < 4; ++e) bq[d][e] = nib2_bf16(cw[q][d] >> (4 * e), nc.mask, nc.magic);
                issue(jb + 1, q, nw2, ns2);
                const uint8_t* xu = xa + (u * 128 + kq * 32) * 2;
                f32x4_t dv = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int d = 0; d < 4; ++d) dv = mfma_bf16(*reinterpret_cast<const u32x4*>(xu + d * 16), bq[d], dv);
                const float s = bf16_lo(cs[q]);
                const float zp = fmaf(-136.0f, s, bf16_hi(cs[q]));
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if (r < MM) {
                        const float X = xst[min(4 * kq + r, M - 1) * NU + u];
                        y[r] = fmaf(s, dv[r], fmaf(zp, X, y[r]));
                    }
                }
            } else {
                u32x4 c0, c1;
                c0[0] = fp8x2_bf16<false>(cw[q][0]);
                c0[1] = fp8x2_bf16<true>(cw[q][0]);
                c0[2] = fp8x2_bf16<false>(cw[q][1]);
                c0[3] = fp8x2_bf16<true>(cw[q][1]);
                c1[0] = fp8x2_bf16<false>(cw[q][2]);
                c1[1] = fp8x2_bf16<true>(cw[q][2]);
                c1[2] = fp8x2_bf16<false>(cw[q][3]);
                c1[3] = fp8x2_bf16<true>(cw[q][3]);
                issue(jb + 1, q, nw2, ns2);
                const uint8_t* xu = xa + (u * 64 + kq * 16) * 2;
                facc = mfma_bf16(*reinterpret_cast<const u32x4*>(xu), c0, facc);
                facc = mfma_bf16(*reinterpret_cast<const u32x4*>(xu + 16), c1, facc);
            }
        }
        // park: red[((jb * M + row) * 16 + column) * 16 + wave slot]
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = 4 * kq + r;
            if (r < MM && m < M) {
                float* slots = red + ((jb * M + m) * 16 + j) * 16;
                slots[wave] = I4 ? y[r] : facc[r];
                for (int s2 = NW + wave; s2 < 16; s2 += NW) slots[s2] = 0.0f;  // slots of absent waves
            }
        }
    };
    // pairs of blocks without a branch inside (a conditional second half made
    // the loop's two paths leave different registers with loads in flight,
    // and the compiler then waited for all of them), then an odd last block
    if constexpr (TC > 0) {
#pragma unroll
        for (int jb = 0; jb + 1 < TC; jb += 2) {
            run_block(jb, wa, sa, wb, sb);
            run_block(jb + 1, wb, sb, wa, sa);
        }
        if constexpr ((TC & 1) != 0) run_block(TC - 1, wa, sa, wb, sb);
    } else {
        int jb = 0;
        for (; jb + 1 < nb; jb += 2) {
            run_block(jb, wa, sa, wb, sb);
            run_block(jb + 1, wb, sb, wa, sa);
        }
        if (jb < nb) run_block(jb, wa, sa, wb, sb);
    }
    __syncthreads();

    // 3. one lane per output: its 16 wave slots added in wave order, then the
    //    epilogue
    auto wave_sum = [&](const float* slots) {  // slots of absent waves hold zeros
        float4 v[4];
#pragma unroll
        for (int w4 = 0; w4 < 4; ++w4) v[w4] = *reinterpret_cast<const float4*>(slots + 4 * w4);
        float s = 0.0f;
#pragma unroll
        for (int w4 = 0; w4 < 4; ++w4) s = (((s + v[w4].x) + v[w4].y) + v[w4].z) + v[w4].w;
        return s;
    };
    for (int g = g0; g < nout; g += nthr) {
        const bool first = g == g0;
        int jb, m, c;
        out_coords(g, jb, m, c);
        const float* rg = red + ((jb * M + m) * 16 + c) * 16;
        const float a = wave_sum(rg);
        const float inv = p.norm ? rsqrtf(wave_sum(sq + m * 16) / (float)K + p.eps) : 1.0f;
        const float s0 = I4 ? 1.0f : (first ? rs0 : row_scale(jb, c)[0]);
        float o;
        if (PAIR) {
            const float a2 = wave_sum(rg + 8 * 16);
            const float s1 = I4 ? 1.0f : (first ? rs1 : row_scale(jb, c)[8]);
            o = silu(a * inv * s0) * (a2 * inv * s1);
        } else {
            o = a * inv * s0;
            if (p.epi == BZ_EPI_RESIDUAL) {
                const uint32_t rv = first ? resv : load_res(jb, m, c);
                o += __uint_as_float(p.res_f32 ? rv : rv << 16);
            }
        }
        const int col = (b0 + jb) * ocols + c;
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

// ---- host side -----------------------------------------------------------------

struct WideLaunch {
    int nw, upw, mm, T;
    unsigned grid;
    size_t lds;
};

template <int WF, int MM, int UPW, int TC = 0>
int launch_wide_kernel(const StreamParams& p, const WideLaunch& l, int nblk, hipStream_t st) {
    auto kern = gemv_wide<WF, MM, UPW, TC>;
    if (l.lds > 65536 && raise_lds_limit(reinterpret_cast<const void*>(kern)) != BZ_OK) return BZ_ERR_LAUNCH;
    if (!stream_hot_ok(p)) return BZ_ERR_UNSUPPORTED;
    hipLaunchKernelGGL(kern, dim3(l.grid), dim3(l.nw * 64), l.lds, st, p.w, p.x, p.gamma, (int)p.chunk, (int)p.ldx, p.K,
                       p.NU, p.M, p.norm, l.T, nblk, p);
    return hipGetLastError() == hipSuccess ? BZ_OK : BZ_ERR_LAUNCH;
}

template <int WF, int MM>
int launch_wide_upw(const StreamParams& p, const WideLaunch& l, int nblk, hipStream_t st) {
    // the int4 decode shapes with the block count fixed at compile time: 2
    // units per wave over 5 blocks (gate|up N20480), and over 2 blocks (qkv
    // N6144) at 2 rows (at one row measured 0.02-0.03 us slower)
    if constexpr (MM <= 2 && tiled_i4(WF)) {
        if (l.upw == 2 && l.T == 5 && nblk % 5 == 0) return launch_wide_kernel<WF, MM, 2, 5>(p, l, nblk, st);
        if constexpr (MM == 2)
            if (l.upw == 2 && l.T == 2 && nblk % 2 == 0) return launch_wide_kernel<WF, MM, 2, 2>(p, l, nblk, st);
    }
    switch (l.upw) {
        case 2: return launch_wide_kernel<WF, MM, 2>(p, l, nblk, st);
        case 3: return launch_wide_kernel<WF, MM, 3>(p, l, nblk, st);
        case 4: return launch_wide_kernel<WF, MM, 4>(p, l, nblk, st);
        default: break;
    }
    if constexpr (wide_max_upw(WF, MM) >= 5)
        if (l.upw == 5) return launch_wide_kernel<WF, MM, 5>(p, l, nblk, st);
    if constexpr (wide_max_upw(WF, MM) >= 10) {
        switch (l.upw) {
            case 6: return launch_wide_kernel<WF, MM, 6>(p, l, nblk, st);
            case 8: return launch_wide_kernel<WF, MM, 8>(p, l, nblk, st);
            case 10: return launch_wide_kernel<WF, MM, 10>(p, l, nblk, st);
            default: break;
        }
    }
    return BZ_ERR_INVALID_ARG;
}

template <int WF>
int launch_wide_wf(const StreamParams& p, const WideLaunch& l, int nblk, hipStream_t st) {
    switch (l.mm) {
        case 1: return launch_wide_upw<WF, 1>(p, l, nblk, st);
        case 2: return launch_wide_upw<WF, 2>(p, l, nblk, st);
        case 4: return launch_wide_upw<WF, 4>(p, l, nblk, st);
        case 8: return launch_wide_upw<WF, 8>(p, l, nblk, st);
        default: return BZ_ERR_INVALID_ARG;
    }
}

// One explicit instantiation set per tiled format, each in its own
// translation unit (bz_gemv_wide_<fmt>.hip).
int launch_wide_i4t(const StreamParams& p, const WideLaunch& l, int nblk, hipStream_t st);
int launch_wide_i4tp(const StreamParams& p, const WideLaunch& l, int nblk, hipStream_t st);
int launch_wide_f8t(const StreamParams& p, const WideLaunch& l, int nblk, hipStream_t st);
int launch_wide_f8tp(const StreamParams& p, const WideLaunch& l, int nblk, hipStream_t st);

}  // namespace bz
