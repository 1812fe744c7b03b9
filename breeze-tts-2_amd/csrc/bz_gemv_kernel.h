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
// Work decomposition
//   * Weights are row-major.  A "chunk" is 128 contiguous bytes of one weight
//     row (one cache line).  Lane l of a wave loads 16 bytes (dwordx4) at
//     offset 16*(l%8) of a chunk of row 8*tile + l/8: one wave load
//     instruction covers 8 rows x 128 B = 8 full lines.
//   * A "tile" is 8 output columns: 8 weight rows, or for the SiLU-gate
//     epilogue 8 gate rows j and the 8 up rows j + N/2 of the [gate; up]
//     concatenation (models/fused/layer.py:60), so silu(g)*u needs no second
//     pass.
//   * The grid is persistent-sized (about one workgroup per CU).  Each
//     workgroup owns `tpw` consecutive tiles, i.e. tpw * nchunks "steps"
//     (one chunk of the T weight tiles each) in tile-major order; wave w
//     takes steps w, w + NW, w + 2 NW, ... so every wave gets the same number
//     of steps (+-1) whatever nchunks % NW is, and walks them through a
//     rolling register pipeline that keeps D steps of loads in flight across
//     tile boundaries.  Nothing is loaded past a wave's last step.
//   * x is staged once per workgroup into LDS.  Its loads are issued BEFORE
//     the first weight loads: vector loads retire in issue order, so waiting
//     for x does not wait for the (HBM-latency) weights.  The RMSNorm is
//     folded: LDS holds u = bf16(gamma * x) and the per-row 1/rms is applied
//     to the finished dot products in the epilogue, so the sum of squares is
//     off the path to the first weight.
//   * int4 group scales travel with the weights: each step also loads the
//     (s, z) pair of its group, one dword per lane.
//   * LDS holds x chunk-interleaved: the 16-byte x block a lane needs for its
//     weight bytes sits next to the blocks of the other 7 lanes of its row,
//     so each ds_read_b128 of 8 lanes reads 128 contiguous bytes (no bank
//     conflict), and one read serves both tiles of a SiLU pair.
//   * A finished tile's per-lane fp32 partials are reduced over the 8 lanes of
//     a row with DPP and parked in LDS; after the last step one barrier, then
//     the waves' partials are summed in a fixed order (deterministic) and the
//     epilogue writes the outputs.
//
// int4 arithmetic: a nibble q becomes the bf16 value 128+q with one
// v_and_or_b32 (exponent 2^7, nibble in the low mantissa bits).  For a lane's
// 32 consecutive k (all inside one quantization group, since groups are >= 32
// and aligned), D = sum u_k (128+q_k) comes from 16 v_dot2c_f32_bf16, and
//     sum u_k w_k = s*D + (z - 136 s) * X          ((q-8)*s + z form)
//     sum u_k w_k = s*D + (m - 128 s) * X          (q*s + min form)
// with X = sum u_k over the same 32 k, precomputed per 32-k block while x is
// staged.  Inside each 8-element x block the order is [x0 x4 x1 x5 x2 x6 x3
// x7], so the (nibble p, nibble p+4) pairs of one and-or line up with bf16x2
// pairs of x.
#pragma once
#include <atomic>
#include <mutex>
#include <set>
#include <utility>

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
    int ntiles, tpw;  // tiles of 8 (dot2) or 16 (MFMA) output columns; most tiles a workgroup owns
    int epi, out_f32, res_f32, norm;
};

__host__ __device__ constexpr int align16(int v) { return (v + 15) & ~15; }

// The fields the first loads of the row-major kernels need, passed as
// leading scalar kernel arguments so the hardware preloads them into SGPRs
// at wave launch (kernarg preloading, -mllvm -amdgpu-kernarg-preload-count=16
// in the build: 14 dwords; an aggregate is never preloaded).  The host
// passes the same values in the struct.
#define BZ_GEMV_HOT_PARAMS \
    const uint16_t *hx, const uint8_t *hw, const void *hsc0, const uint16_t *hgamma, int hldx, int hrow_bytes, int hK, \
        int hN, int hntiles, int htpw
#define BZ_GEMV_HOT_ARGS(p) \
    (p).x, (p).w, (p).sc0, (p).gamma, (int)(p).ldx, (int)(p).row_bytes, (p).K, (p).N, (p).ntiles, (p).tpw
__device__ __forceinline__ void gemv_hot(GemvParams& p, const uint16_t* x, const uint8_t* w, const void* sc0,
                                         const uint16_t* gamma, int ldx, int row_bytes, int K, int N, int ntiles,
                                         int tpw) {
    p.x = x;
    p.w = w;
    p.sc0 = sc0;
    p.gamma = gamma;
    p.ldx = ldx;
    p.row_bytes = row_bytes;
    p.K = K;
    p.N = N;
    p.ntiles = ntiles;
    p.tpw = tpw;
}
// Host side: whether a GemvParams fits the 32-bit leading scalars.
inline bool gemv_hot_ok(const GemvParams& p) { return p.ldx <= 0x7FFFFFFF && p.row_bytes <= 0x7FFFFFFF; }

__host__ __device__ constexpr bool is_int4(int wf) { return wf == WF_I4ZP || wf == WF_I4MIN; }

// Elements of one LDS x row: K rounded up to whole chunks.
__host__ __device__ inline int x_row_elems(int K, int wf) {
    const int per_chunk = is_int4(wf) ? 256 : (wf == WF_FP8 ? 128 : 64);
    return (K + per_chunk - 1) / per_chunk * per_chunk;
}

// LDS carve-up, shared by the kernel and the host launcher.
// Largest workgroup: 8 waves.
constexpr int kMaxThreads = 512;
constexpr int kMaxWaves = kMaxThreads / 64;

struct LdsLayout {
    int xs, xsum, red, nrm, total;
};
// LDS: x, the int4 32-k sums of x, the parked partial sums, the norm.
__host__ __device__ inline LdsLayout lds_layout(int M, int T, int NW, int K, int wf, int tpw) {
    const bool i4 = is_int4(wf);
    const int xe = x_row_elems(K, wf);
    LdsLayout L;
    L.xs = 0;
    L.xsum = L.xs + align16(M * xe * 2);
    L.red = L.xsum + (i4 ? align16(M * (xe / 32) * 4) : 0);
    L.nrm = L.red + align16(tpw * NW * T * M * 8 * 4);
    L.total = L.nrm + align16(NW * M * 4);
    return L;
}

// LDS element offset (within an x row) of the 8-element block kb = k/8.
template <int WF>
__device__ __forceinline__ int x_block_addr(int kb) {
    if (is_int4(WF)) {
        // k = 256 ch + 32 c8 + 8 dd + e  ->  [ch][dd][c8][e]
        return ((kb >> 5) << 8) + ((kb & 3) << 6) + (((kb >> 2) & 7) << 3);
    } else if (WF == WF_FP8) {
        // k = 128 ch + 16 c8 + 8 h + e   ->  [ch][h][c8][e]
        return ((kb >> 4) << 7) + ((kb & 1) << 6) + (((kb >> 1) & 7) << 3);
    }
    return kb << 3;
}

// ---------------------------------------------------------------------------
// prologue: x (+ RMSNorm) into LDS
// ---------------------------------------------------------------------------

// Blocks of x each thread keeps in registers during the prologue.
constexpr int kXB = 4;



// Loads are unconditional (indices clamped into range) so the code stays
// straight-line and the wait-count pass can wait for exactly the loads it
// needs; blocks past the end are simply never used.
template <int WF, int M>
__device__ __forceinline__ void issue_x(const GemvParams& p, int tid, int nthr, u32x4 (&xr)[kXB], u32x4 (&gr)[kXB]) {
    const int nblk = p.K >> 3, total = M * nblk;
#pragma unroll
    for (int i = 0; i < kXB; ++i) {
        const int b = min(tid + i * nthr, total - 1);
        const int m = M == 1 ? 0 : b / nblk;
        const int kb = b - m * nblk;
        xr[i] = ldg16(p.x + (int64_t)m * p.ldx + kb * 8);
        gr[i] = p.norm ? ldg16(p.gamma + kb * 8) : u32x4{0u, 0u, 0u, 0u};
    }
}

template <int M>
__device__ __forceinline__ void acc_sq(const u32x4 v, int m, float (&ss)[M]) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float a = bf16_lo(v[i]), b = bf16_hi(v[i]);
        s += a * a + b * b;
    }
#pragma unroll
    for (int mm = 0; mm < M; ++mm)
        if (mm == m) ss[mm] += s;
}

// The 8 staged values of a block: u = bf16(gamma * x) with the RMSNorm, else
// x itself.
__device__ __forceinline__ void block_values(const GemvParams& p, u32x4 v, u32x4 g, float (&f)[8]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[2 * i] = bf16_lo(v[i]);
        f[2 * i + 1] = bf16_hi(v[i]);
    }
    if (p.norm) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f[2 * i] = bf16_to_f32(f32_to_bf16(f[2 * i] * bf16_lo(g[i])));
            f[2 * i + 1] = bf16_to_f32(f32_to_bf16(f[2 * i + 1] * bf16_hi(g[i])));
        }
    }
}

template <int WF>
__device__ __forceinline__ void stage_block(const GemvParams& p, u32x4 v, u32x4 g, int m, int kb, uint16_t* xs,
                                            float* xsum, int xe) {
    float f[8];
    block_values(p, v, g, f);
    u32x4 o;
    if (is_int4(WF)) {
        o[0] = pack_bf16x2(f[0], f[4]);
        o[1] = pack_bf16x2(f[1], f[5]);
        o[2] = pack_bf16x2(f[2], f[6]);
        o[3] = pack_bf16x2(f[3], f[7]);
        float cs = ((f[0] + f[1]) + (f[2] + f[3])) + ((f[4] + f[5]) + (f[6] + f[7]));
        cs = sum4(cs);  // 4 consecutive blocks (4 consecutive lanes) = one 32-k block
        if ((kb & 3) == 0) xsum[m * (xe >> 5) + (kb >> 2)] = cs;
    } else if (p.norm) {
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = pack_bf16x2(f[2 * i], f[2 * i + 1]);
    } else {
        o = v;
    }
    *reinterpret_cast<u32x4*>(xs + m * xe + x_block_addr<WF>(kb)) = o;
}

// Finish the x prologue from the registers filled by issue_x (plus reloads
// when x does not fit in kXB blocks per thread).  With the RMSNorm, each
// wave also parks its partial sums of x^2 in nrm[wave][m]; the caller's
// barrier publishes them and the epilogue turns them into 1/rms.
template <int WF, int M, typename StageFn>
__device__ __forceinline__ void finish_x_generic(const GemvParams& p, const u32x4 (&xr)[kXB],
                                                 const u32x4 (&gr)[kXB], float* nrm, int tid, int nthr, int wave,
                                                 int lane, StageFn stage) {
    const int nblk = p.K >> 3, total = M * nblk;
    float ss[M];
#pragma unroll
    for (int m = 0; m < M; ++m) ss[m] = 0.0f;
#pragma unroll
    for (int i = 0; i < kXB; ++i) {
        const int b = tid + i * nthr;
        if (b < total) {
            const int m = M == 1 ? 0 : b / nblk;
            if (p.norm) acc_sq<M>(xr[i], m, ss);
            stage(xr[i], gr[i], m, b - m * nblk);
        }
    }
    for (int b = tid + kXB * nthr; b < total; b += nthr) {
        const int m = M == 1 ? 0 : b / nblk;
        const int kb = b - m * nblk;
        const u32x4 v = ldg16(p.x + (int64_t)m * p.ldx + kb * 8);
        const u32x4 g = p.norm ? ldg16(p.gamma + kb * 8) : v;
        if (p.norm) acc_sq<M>(v, m, ss);
        stage(v, g, m, kb);
    }
    if (p.norm) {
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const float t = wave_sum(ss[m]);
            if (lane == 0) nrm[wave * M + m] = t;
        }
    }
}

template <int WF, int M>
__device__ __forceinline__ void finish_x(const GemvParams& p, const u32x4 (&xr)[kXB], const u32x4 (&gr)[kXB],
                                         uint16_t* xs, float* xsum, float* nrm, int tid, int nthr, int wave,
                                         int lane) {
    const int xe = x_row_elems(p.K, WF);
    finish_x_generic<WF, M>(p, xr, gr, nrm, tid, nthr, wave, lane, [&](u32x4 v, u32x4 g, int m, int kb) {
        stage_block<WF>(p, v, g, m, kb, xs, xsum, xe);
    });
}

// s + v[0] + v[stride] + ... + v[(n - 1) stride] (1 <= n <= N), added in
// that order.  The wave count n is a run-time value: a plain loop over it
// stays rolled and waits for each LDS read before issuing the next (one LDS
// round trip per term, ~0.8 us per GEMV epilogue).  Here all N reads go out
// first (indices clamped into range) and a select drops the terms past n, so
// the sum is bit-identical to the plain loop's.
template <int N>
__device__ __forceinline__ float sum_strided(const float* v, int stride, int n, float s = 0.0f) {
    float t[N];
#pragma unroll
    for (int w = 0; w < N; ++w) t[w] = v[min(w, n - 1) * stride];
#pragma unroll
    for (int w = 0; w < N; ++w) s = w < n ? s + t[w] : s;
    return s;
}

// 1/rms of row m from the waves' partial sums of squares (1 without norm).
__device__ __forceinline__ float row_inv_rms(const GemvParams& p, const float* nrm, int NW, int M, int m) {
    if (!p.norm) return 1.0f;
    const float s = sum_strided<kMaxWaves>(nrm + m, M, NW);
    return rsqrtf(s / (float)p.K + p.eps);
}

// For M <= 2 every row's 1/rms is computed right after the x-staging
// barrier: its LDS reads, divide and rsqrt then run while the first weight
// loads are in flight instead of lengthening the epilogue.  For more rows
// the epilogue computes it: a register array kept across the main loop and
// selected by the output's row is turned into a scratch array.
template <int M>
constexpr bool kEarlyInv = M <= 2;

template <int M>
__device__ __forceinline__ void row_inv_all(const GemvParams& p, const float* nrm, int NW, float (&inv)[M]) {
#pragma unroll
    for (int m = 0; m < M; ++m) inv[m] = kEarlyInv<M> ? row_inv_rms(p, nrm, NW, M, m) : 1.0f;
}

// ---------------------------------------------------------------------------
// epilogue (shared by the dot2 and MFMA kernels; COLS = output columns per
// tile, which is also the row stride of the parked partial sums)
// ---------------------------------------------------------------------------

// Output i of a workgroup: local tile i / (M*COLS), x row (i / COLS) % M,
// column i % COLS of the tile.
template <int M, int COLS>
struct OutIndex {
    int tl, m, c;
    __device__ __forceinline__ OutIndex(int i, int tile0) {
        tl = i / (M * COLS);
        m = (i / COLS) % M;
        c = (tile0 + tl) * COLS + (i % COLS);
    }
};

// What the epilogue reads from global memory (fp8 row scales, the residual)
// for the first output a thread owns, loaded during the prologue so the
// epilogue does not start with a memory round trip.
template <int T>
struct EpiPrefetch {
    float sc[T];
    uint32_t res;  // raw bits (f32, or bf16 zero-extended): converted in the epilogue, so
                   // the prologue never waits for this load
};

template <int WF, int M, int T, bool SILU, int COLS>
__device__ __forceinline__ EpiPrefetch<T> epi_prefetch(const GemvParams& p, int tile0, int ntl, int tid) {
    const OutIndex<M, COLS> o(min(tid, ntl * M * COLS - 1), tile0);
    const int c = min(o.c, p.n_out - 1);
    EpiPrefetch<T> e;
#pragma unroll
    for (int t = 0; t < T; ++t)
        e.sc[t] = WF == WF_FP8 ? reinterpret_cast<const float*>(p.sc0)[SILU ? c + t * p.n_out : c] : 1.0f;
    e.res = 0u;
    if (p.epi == BZ_EPI_RESIDUAL) {
        const int64_t idx = (int64_t)o.m * p.ldr + c;
        e.res = p.res_f32 ? reinterpret_cast<const uint32_t*>(p.res)[idx]
                          : (uint32_t)reinterpret_cast<const uint16_t*>(p.res)[idx];
    }
    return e;
}

// Sum the waves' parked partials of each output in a fixed order
// (deterministic), apply 1/rms, the fp8 row scale, SiLU-gate or residual,
// and store.  red[((tl*NW + w)*T + t)*M + m][COLS].
template <int WF, int M, int T, bool SILU, int COLS>
__device__ __forceinline__ void epilogue(const GemvParams& p, int tile0, int ntl, int tid, int nthr, int NW,
                                         const float* red, const float* nrm, const float (&early)[M],
                                         const EpiPrefetch<T>& pre) {
    float inv[M];
#pragma unroll
    for (int m = 0; m < M; ++m) inv[m] = kEarlyInv<M> ? early[m] : row_inv_rms(p, nrm, NW, M, m);
    for (int i = tid; i < ntl * M * COLS; i += nthr) {
        const OutIndex<M, COLS> o(i, tile0);
        if (o.c >= p.n_out) continue;
        const bool first = i == tid;
        float iv = inv[0];
#pragma unroll
        for (int m = 1; m < M; ++m)
            if (o.m == m) iv = inv[m];
        float a[T];
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const float* rp = red + (((o.tl * NW) * T + t) * M + o.m) * COLS + (i % COLS);
            float v = sum_strided<kMaxWaves>(rp, T * M * COLS, NW);
            v *= iv;
            if (WF == WF_FP8)
                v *= first ? pre.sc[t] : reinterpret_cast<const float*>(p.sc0)[SILU ? o.c + t * p.n_out : o.c];
            a[t] = v;
        }
        float out = SILU ? silu(a[0]) * a[T - 1] : a[0];
        if (p.epi == BZ_EPI_RESIDUAL) {
            const int64_t idx = (int64_t)o.m * p.ldr + o.c;
            out += first ? __uint_as_float(p.res_f32 ? pre.res : pre.res << 16)
                         : (p.res_f32 ? reinterpret_cast<const float*>(p.res)[idx]
                                      : bf16_to_f32(reinterpret_cast<const uint16_t*>(p.res)[idx]));
        }
        const int64_t oi = (int64_t)o.m * p.ldo + o.c;
        if (p.out_f32)
            reinterpret_cast<float*>(p.out)[oi] = out;
        else
            reinterpret_cast<uint16_t*>(p.out)[oi] = f32_to_bf16(out);
    }
}

// ---------------------------------------------------------------------------
// the streaming pipeline
// ---------------------------------------------------------------------------

// Position of a wave in the workgroup's tile-major step list: local tile tl
// and chunk ch.  A wave advances by NW steps; NW <= nchunks (host-checked),
// so a wave visits every tile, and its last step in a tile is the one with
// ch + NW >= nchunks.  Both fields are wave-uniform.
struct StepCursor {
    int tl, ch;
    __device__ __forceinline__ void advance(int NW, int nch) {
        ch += NW;
        if (ch >= nch) {
            ch -= nch;
            ++tl;
        }
    }
    __device__ __forceinline__ bool last_in_tile(int NW, int nch) const { return ch + NW >= nch; }
};

// Steps of wave `wave` among ntl * nch, and the cursor of its last one.
__device__ __forceinline__ int wave_steps(int ntl, int nch, int NW, int wave) {
    return (ntl * nch - 1 - wave) / NW + 1;
}
__device__ __forceinline__ StepCursor step_cursor(int s, int NW, int nch, int wave) {
    const int flat = wave + s * NW;
    const int tl = flat / nch;
    return StepCursor{tl, flat - tl * nch};
}

// The rolling pipeline shared by both kernels.  issue(d, c) loads step c
// into register slot d; consume(d, c) uses slot d.  pipeline_prime issues the
// first D steps (past the last step it re-issues the last one, so the
// prologue stays branch-free); pipeline_run then consumes every step exactly
// once and issues nothing past a wave's last step.  The steady loop issues
// unconditionally, which keeps the compiler's vector-memory wait counts
// exact (each consume waits only for its own slot); the tail issues behind a
// wave-uniform branch.
// Slots [B, E) of the prime (the kernels issue all D before staging x:
// issuing one step first and the rest after staging measured slower).
template <int B, int E, typename IssueFn>
__device__ __forceinline__ void pipeline_prime(int S, int NW, int nch, int wave, StepCursor& ic, IssueFn issue) {
    const StepCursor last = step_cursor(S - 1, NW, nch, wave);
#pragma unroll
    for (int d = B; d < E; ++d) {
        issue(d, d < S ? ic : last);
        ic.advance(NW, nch);
    }
}

// This workgroup's tiles: a balanced share (counts differ by at most one).
struct TileRange {
    int tile0, ntl;
    __device__ __forceinline__ TileRange(int ntiles) {
        tile0 = (int)(((int64_t)blockIdx.x * ntiles) / gridDim.x);
        ntl = (int)(((int64_t)(blockIdx.x + 1) * ntiles) / gridDim.x) - tile0;
    }
};

template <int D, typename IssueFn, typename ConsumeFn>
__device__ __forceinline__ void pipeline_run(int S, int NW, int nch, int wave, StepCursor ic, IssueFn issue,
                                             ConsumeFn consume) {
    StepCursor cc{0, wave};
    int s0 = 0;
    for (; s0 + 2 * D <= S; s0 += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            consume(d, cc);
            cc.advance(NW, nch);
            issue(d, ic);
            ic.advance(NW, nch);
        }
    }
#pragma unroll
    for (int d = 0; d < D; ++d) {
        const int s = s0 + d;
        if (s < S) {
            consume(d, cc);
            cc.advance(NW, nch);
        }
        if (s + D < S) {
            issue(d, ic);
            ic.advance(NW, nch);
        }
    }
#pragma unroll
    for (int d = 0; d < D; ++d) {
        const int s = s0 + D + d;
        if (s < S) {
            consume(d, cc);
            cc.advance(NW, nch);
        }
    }
}

// Issue the T weight loads of the step at cursor c, and for int4 the
// (s, z) / (s, min) pair of each lane's group.
template <int WF, int T, bool SILU>
__device__ __forceinline__ void issue_step(const GemvParams& p, StepCursor c, int tile0, int c8, int r,
                                           u32x4 (&buf)[T], uint32_t (&sc)[T]) {
    const int ch = c.ch;
    const int colbase = (tile0 + c.tl) * 8;
    const uint8_t* base = p.w + (int64_t)colbase * p.row_bytes + ch * 128;  // uniform
    const int lr = min(r, p.n_out - 1 - colbase);                            // partial last tile
    const int lk = min(c8 * 16, (int)p.row_bytes - 16 - ch * 128);            // K tail
    // 24-bit multiply (lr < 8, row_bytes < 2^24): a 64-bit mad here would
    // read an unrelated register and force a wait on every load in flight
    const uint32_t off = __umul24((uint32_t)lr, (uint32_t)p.row_bytes) + (uint32_t)lk;
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const uint8_t* bt = SILU && t ? base + (int64_t)p.n_out * p.row_bytes : base;
        buf[t] = ldg16(bt + off);
    }
    if (WF == WF_I4ZP) {
        const int g = ((ch * 128 + lk) * 2) >> p.glog2;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int row = colbase + lr + (SILU && t ? p.n_out : 0);
            sc[t] = reinterpret_cast<const uint32_t*>(p.sc0)[(int64_t)g * p.N + row];
        }
    } else if (WF == WF_I4MIN) {
        const int g = ((ch * 128 + lk) * 2) >> p.glog2;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int row = colbase + lr + (SILU && t ? p.n_out : 0);
            sc[t] = (uint32_t)reinterpret_cast<const uint16_t*>(p.sc0)[(int64_t)row * p.G + g] |
                    ((uint32_t)reinterpret_cast<const uint16_t*>(p.sc1)[(int64_t)row * p.G + g] << 16);
        }
    }
}

template <int WF, int M, int T>
__device__ __forceinline__ void consume_step(const GemvParams& p, StepCursor c, int tile0, int c8, int r, int xe,
                                             const uint16_t* xs, const float* xsum, const NibbleConsts& nc,
                                             const u32x4 (&buf)[T], const uint32_t (&scv)[T], float (&acc)[T][M]) {
    const int ch = c.ch;
    const int boff = ch * 128 + c8 * 16;
    if (!((tile0 + c.tl) * 8 + r < p.n_out && boff < p.row_bytes)) return;
    if (is_int4(WF)) {
        uint32_t b[T][4][4];
        float sc[T], zp[T];
#pragma unroll
        for (int t = 0; t < T; ++t) {
#pragma unroll
            for (int d = 0; d < 4; ++d)
#pragma unroll
                for (int sh = 0; sh < 4; ++sh) b[t][d][sh] = nib2_bf16(buf[t][d] >> (4 * sh), nc.mask, nc.magic);
            const uint32_t e = scv[t];
            sc[t] = bf16_lo(e);
            zp[t] = bf16_hi(e) - (WF == WF_I4ZP ? 136.0f : 128.0f) * sc[t];
        }
        const uint16_t* xc = xs + (ch << 8) + (c8 << 3);
        const float* xsc = xsum + (ch << 3) + c8;
#pragma unroll
        for (int m = 0; m < M; ++m) {
            u32x4 xv[4];
#pragma unroll
            for (int d = 0; d < 4; ++d) xv[d] = *reinterpret_cast<const u32x4*>(xc + m * xe + d * 64);
            const float X = xsc[m * (xe >> 5)];
#pragma unroll
            for (int t = 0; t < T; ++t) {
                float d0 = 0.0f, d1 = 0.0f;
#pragma unroll
                for (int sh = 0; sh < 4; ++sh) {
                    d0 = dot2(b[t][0][sh], xv[0][sh], d0);
                    d1 = dot2(b[t][1][sh], xv[1][sh], d1);
                }
#pragma unroll
                for (int sh = 0; sh < 4; ++sh) {
                    d0 = dot2(b[t][2][sh], xv[2][sh], d0);
                    d1 = dot2(b[t][3][sh], xv[3][sh], d1);
                }
                acc[t][m] += sc[t] * (d0 + d1) + zp[t] * X;
            }
        }
    } else if (WF == WF_FP8) {
        uint32_t b[T][8];
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                b[t][2 * d] = fp8x2_bf16<false>(buf[t][d]);
                b[t][2 * d + 1] = fp8x2_bf16<true>(buf[t][d]);
            }
        const uint16_t* xc = xs + (ch << 7) + (c8 << 3);
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const u32x4 x0 = *reinterpret_cast<const u32x4*>(xc + m * xe);
            const u32x4 x1 = *reinterpret_cast<const u32x4*>(xc + m * xe + 64);
#pragma unroll
            for (int t = 0; t < T; ++t) {
                float d0 = 0.0f, d1 = 0.0f;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    d0 = dot2(b[t][i], x0[i], d0);
                    d1 = dot2(b[t][4 + i], x1[i], d1);
                }
                acc[t][m] += d0 + d1;
            }
        }
    } else {
        const uint16_t* xc = xs + (ch << 6) + (c8 << 3);
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const u32x4 x0 = *reinterpret_cast<const u32x4*>(xc + m * xe);
#pragma unroll
            for (int t = 0; t < T; ++t) {
                float d0 = dot2(buf[t][0], x0[0], 0.0f);
                float d1 = dot2(buf[t][1], x0[1], 0.0f);
                d0 = dot2(buf[t][2], x0[2], d0);
                d1 = dot2(buf[t][3], x0[3], d1);
                acc[t][m] += d0 + d1;
            }
        }
    }
}

// T = 2 for the SiLU-gate pair, else 1.  D = steps of loads in flight per wave.
template <int WF, int M, int T, int D, bool SILU>
__global__ void __launch_bounds__(kMaxThreads) gemv_persist(BZ_GEMV_HOT_PARAMS, GemvParams p) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    gemv_hot(p, hx, hw, hsc0, hgamma, hldx, hrow_bytes, hK, hN, hntiles, htpw);
    const int nthr = blockDim.x;
    const int NW = nthr >> 6;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c8 = lane & 7, r = lane >> 3;
    const int xe = x_row_elems(p.K, WF);
    const TileRange tr(p.ntiles);
    const int tile0 = tr.tile0, ntl = tr.ntl;
    const int nch = p.nchunks;
    const int S = wave_steps(ntl, nch, NW, wave);  // this wave's steps (host ensures NW <= nchunks)

    const LdsLayout L = lds_layout(M, T, NW, p.K, WF, p.tpw);
    uint16_t* xs = reinterpret_cast<uint16_t*>(smem + L.xs);
    float* xsum = reinterpret_cast<float*>(smem + L.xsum);
    float* red = reinterpret_cast<float*>(smem + L.red);
    float* nrm = reinterpret_cast<float*>(smem + L.nrm);

    u32x4 buf[D][T];
    uint32_t scb[D][T];
    auto issue = [&](int d, StepCursor c) { issue_step<WF, T, SILU>(p, c, tile0, c8, r, buf[d], scb[d]); };

    // 0. x (and gamma) loads first, then the first D steps of weights.  The
    //    first scheduling barrier keeps the x loads ahead of the weight loads
    //    (vector loads retire in order, so x is then waited for without
    //    waiting for the weights); the second keeps every consumer of x below
    //    the weight loads.
    u32x4 xr[kXB], gr[kXB];
    issue_x<WF, M>(p, tid, nthr, xr, gr);
    const EpiPrefetch<T> pre = epi_prefetch<WF, M, T, SILU, 8>(p, tile0, ntl, tid);
    __builtin_amdgcn_sched_barrier(0);
    StepCursor ic{0, wave};
    pipeline_prime<0, D>(S, NW, nch, wave, ic, issue);
    __builtin_amdgcn_sched_barrier(0);
    // 1. x staging completes while the weights are in flight
    finish_x<WF, M>(p, xr, gr, xs, xsum, nrm, tid, nthr, wave, lane);
    __syncthreads();
    float inv[M];
    row_inv_all<M>(p, nrm, NW, inv);

    // 2. every step once; a wave's partial sums of a tile go to LDS after its
    //    last step in that tile, reduced over the 8 lanes of each row
    const NibbleConsts nc;
    float acc[T][M];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[t][m] = 0.0f;
    pipeline_run<D>(S, NW, nch, wave, ic, issue, [&](int d, StepCursor c) {
        consume_step<WF, M, T>(p, c, tile0, c8, r, xe, xs, xsum, nc, buf[d], scb[d], acc);
        if (c.last_in_tile(NW, nch)) {
#pragma unroll
            for (int t = 0; t < T; ++t)
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    const float v = sum8(acc[t][m]);
                    if (c8 == 0) red[(((c.tl * NW + wave) * T + t) * M + m) * 8 + r] = v;
                    acc[t][m] = 0.0f;
                }
        }
    });
    __syncthreads();

    // 3. epilogue
    epilogue<WF, M, T, SILU, 8>(p, tile0, ntl, tid, nthr, NW, red, nrm, inv, pre);
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

inline int device_lds_limit() {
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

// Raise a kernel's dynamic-LDS limit to the device's maximum, once per
// (device, kernel): hipFuncSetAttribute acts on the current device only, so
// a kernel first launched on one GPU still needs it on the next.
inline int raise_lds_limit(const void* kern) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return BZ_ERR_LAUNCH;
    static std::mutex mu;
    static std::set<std::pair<int, const void*>> done;
    {
        std::lock_guard<std::mutex> lock(mu);
        if (done.count({dev, kern})) return BZ_OK;
    }
    if (hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, device_lds_limit()) != hipSuccess)
        return BZ_ERR_LAUNCH;
    std::lock_guard<std::mutex> lock(mu);
    done.insert({dev, kern});
    return BZ_OK;
}

struct Launch {
    int M, depth, nw;
    bool silu;
    size_t lds;
    unsigned grid;
};

// T * D <= 16 loads of 16 bytes per lane in flight.
constexpr int kMaxLoadsInFlight = 16;

template <int WF, int M, int T, int D, bool SILU>
int launch_persist(const GemvParams& p, const Launch& l, hipStream_t st) {
    auto kern = gemv_persist<WF, M, T, D, SILU>;
    if (l.lds > 65536 && raise_lds_limit(reinterpret_cast<const void*>(kern)) != BZ_OK) return BZ_ERR_LAUNCH;
    if (!gemv_hot_ok(p)) return BZ_ERR_UNSUPPORTED;
    hipLaunchKernelGGL(kern, dim3(l.grid), dim3(l.nw * 64), l.lds, st, BZ_GEMV_HOT_ARGS(p), p);
    return hipGetLastError() == hipSuccess ? BZ_OK : BZ_ERR_LAUNCH;
}

template <int WF, int M, bool SILU>
int launch_depth(const GemvParams& p, const Launch& l, hipStream_t st) {
    constexpr int T = SILU ? 2 : 1;
    switch (l.depth) {
        case 2: return launch_persist<WF, M, T, 2, SILU>(p, l, st);
        case 4: return launch_persist<WF, M, T, 4, SILU>(p, l, st);
        case 8: return launch_persist<WF, M, T, 8, SILU>(p, l, st);
        case 16:
            if constexpr (T == 1) return launch_persist<WF, M, T, 16, SILU>(p, l, st);
            return BZ_ERR_INVALID_ARG;
        default: return BZ_ERR_INVALID_ARG;
    }
}

template <int WF, int M>
int launch_t(const GemvParams& p, const Launch& l, hipStream_t st) {
    return l.silu ? launch_depth<WF, M, true>(p, l, st) : launch_depth<WF, M, false>(p, l, st);
}

template <int WF>
int launch_m(const GemvParams& p, const Launch& l, hipStream_t st) {
    switch (l.M) {
        case 1: return launch_t<WF, 1>(p, l, st);
        case 2: return launch_t<WF, 2>(p, l, st);
        case 3: return launch_t<WF, 3>(p, l, st);
        case 4: return launch_t<WF, 4>(p, l, st);
        default: return BZ_ERR_INVALID_ARG;
    }
}

// One explicit instantiation per weight format, each in its own
// translation unit (bz_gemv_<fmt>.hip) so the build compiles them in parallel.
int launch_i4zp(const GemvParams& p, const Launch& l, hipStream_t st);
int launch_i4min(const GemvParams& p, const Launch& l, hipStream_t st);
int launch_fp8(const GemvParams& p, const Launch& l, hipStream_t st);
int launch_bf16(const GemvParams& p, const Launch& l, hipStream_t st);

}  // namespace bz
