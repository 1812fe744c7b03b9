// Decode-step attention of the fused decoder layer (gfx950): one new token
// per batch row against a static KV cache.
//
// Reference behaviour replaced (models/fused/kernels.py):
//   _rms_head, _rope, qkv_rope_cache_kernel :356-401  per-head q/k RMSNorm,
//       rotate-half RoPE, q to fp32, new k and v into the cache at pos
//   attn_decode_kernel                       :404-453  softmax(q k^T scale +
//       mask) v over the cache positions [0, pos], split over positions
//   attn_combine_kernel, attention_step      :456-536
//
// Layouts: qkv bf16 [B][ld_qkv] = [q heads | k heads | v heads] x D; caches
// [B][HKV][S][D] (bf16 or fp32); cos/sin [B or 1][D] (bf16 or fp32, batch
// stride ld_cs, 0 to broadcast one row); mask [B][ld_mask] additive bf16 or
// fp32, or bool (ld_mask 0: one row for all);
// q_out fp32 [B][HQ][D]; out bf16 [B][ld_out] with q head h at columns
// h*D..h*D+D-1.  Partials (split > 1) fp32 [B][HQ][split][D + 4] = (acc, m, l).
//
// attn_decode runs one workgroup per (batch row, kv head, split), so the G =
// HQ/HKV query heads sharing a kv head read its keys and values once.  Its
// four waves take 16-position blocks of the split in turn:
//   scores   v_mfma_f32_16x16x32_bf16 with A = the G query rows (padded to
//            16) and B = 16 key rows; q is carried as bf16 hi + lo parts
//            (two MFMAs, ~16 significant bits; an fp32 cache also splits k)
//   softmax  online (running max m, sum l) per head, exp2-based
//   p v      bf16 cache, D <= 256: v_mfma_f32_16x16x16_bf16 per 16-column
//            tile, A = p (through LDS, as bf16 hi + lo), B = 4 value rows
//            of one column, which lane (col, grp) loads directly (4 rows x
//            D/16 contiguous columns) so no cross-lane transpose is needed;
//            fp32 cache or D = 512: VALU, lane l owns D/64 consecutive
//            columns of every head and reads each value row with one
//            coalesced load
// The waves' (m, l, acc) are merged through LDS in a fixed order.
#include "bz_attn.h"
#include "bz_device.h"

namespace bz {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// D = A B + C, 16x16x32: A[i][k] in lane i + 16 (k/8) element k%8, B[k][j]
// in lane j + 16 (k/8) element k%8, D[i][j] in lane j + 16 (i/4) element i%4.
__device__ __forceinline__ f32x4_t mfma16(const u32x4 a, const u32x4 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                  c, 0, 0, 0);
}

typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// D = A B + C, 16x16x16: A[i][k] in lane i + 16 (k/4) element k%4, B[k][j]
// in lane j + 16 (k/4) element k%4, D[i][j] in lane j + 16 (i/4) element i%4
// (checked on the hardware).
__device__ __forceinline__ f32x4_t mfma16k16(const u32x2 a, const u32x2 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(bf16x4_t, a), __builtin_bit_cast(bf16x4_t, b),
                                                    c, 0, 0, 0);
}

__device__ __forceinline__ float ld_any(const void* p, bool f32, int64_t i) {
    return f32 ? reinterpret_cast<const float*>(p)[i] : bf16_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
}

// Raw bits of element i of a bf16 (BZ_DT_BF16), fp32 (BZ_DT_F32) or bool
// (BZ_MASK_BOOL) array, widened later by raw_f32: keeping the conversion
// away from the load lets the loads issued before and after it stay in
// flight.
__device__ __forceinline__ uint32_t ld_raw(const void* p, int kind, int64_t i) {
    if (kind == BZ_DT_F32) return reinterpret_cast<const uint32_t*>(p)[i];
    if (kind == BZ_MASK_BOOL) return reinterpret_cast<const uint8_t*>(p)[i];
    return reinterpret_cast<const uint16_t*>(p)[i];
}

// bf16 / fp32 as a value; a bool mask entry as additive (nonzero = attend
// -> 0, zero -> -1e30, the reference's conversion).
__device__ __forceinline__ float raw_f32(uint32_t v, int kind) {
    if (kind == BZ_DT_F32) return __uint_as_float(v);
    if (kind == BZ_MASK_BOOL) return v ? 0.0f : -1e30f;
    return __uint_as_float(v << 16);
}

__device__ __forceinline__ void st_any(void* p, bool f32, int64_t i, float v) {
    if (f32)
        reinterpret_cast<float*>(p)[i] = v;
    else
        reinterpret_cast<uint16_t*>(p)[i] = f32_to_bf16(v);
}

// Eight floats as bf16 hi + lo parts (x = hi + lo to ~16 significant bits).
__device__ __forceinline__ void split8(const float (&v)[8], u32x4& hi, u32x4& lo) {
    uint32_t h[4], l[4];
    for (int i = 0; i < 4; ++i) {
        const uint16_t h0 = f32_to_bf16(v[2 * i]), h1 = f32_to_bf16(v[2 * i + 1]);
        h[i] = (uint32_t)h0 | ((uint32_t)h1 << 16);
        l[i] = pack_bf16x2(v[2 * i] - bf16_to_f32(h0), v[2 * i + 1] - bf16_to_f32(h1));
    }
    hi = u32x4{h[0], h[1], h[2], h[3]};
    lo = u32x4{l[0], l[1], l[2], l[3]};
}

// Sum over the 64 lanes, every lane gets it: each 16-lane row by DPP, then
// rows 0..3 in order (the same order in every kernel of this file).
__device__ __forceinline__ float row_sum16(float v) {
    v += dpp_f32<kDppXor1>(v);
    v += dpp_f32<kDppXor2>(v);
    v += dpp_f32<0x124>(v);  // row_ror:4
    return v + dpp_f32<0x128>(v);  // row_ror:8
}

__device__ __forceinline__ float wave_sum64(float v) {
    v = row_sum16(v);
    const int bits = __float_as_int(v);
    return ((__int_as_float(__builtin_amdgcn_readlane(bits, 0)) + __int_as_float(__builtin_amdgcn_readlane(bits, 16))) +
            __int_as_float(__builtin_amdgcn_readlane(bits, 32))) +
           __int_as_float(__builtin_amdgcn_readlane(bits, 48));
}

// ---------------------------------------------------------------------------
// q/k RMSNorm + RoPE + cache write.  One workgroup per (batch row b, head h);
// heads [0, HQ) are queries, [HQ, HQ + HKV) key/value pairs.
// ---------------------------------------------------------------------------
constexpr int kRopeThreads = 256;
constexpr int kMaxRopeDim = 1024;

__global__ void __launch_bounds__(kRopeThreads) qkv_rope_cache_kernel(
    const uint16_t* qkv, int64_t ld_qkv, int HQ, int HKV, int D, const uint16_t* qn, const uint16_t* kn, float eps,
    const void* cosp, const void* sinp, bool cs_f32, int64_t ld_cs, const int64_t* pos_p, float* q_out, void* kc,
    void* vc, int S, bool cache_f32, int64_t* seq_len) {
    __shared__ float vals[kMaxRopeDim];
    __shared__ float part[kRopeThreads / 64];
    const int b = blockIdx.x, h = blockIdx.y;
    const bool is_q = h < HQ;
    const uint16_t* src = qkv + (int64_t)b * ld_qkv + (int64_t)h * D;
    const uint16_t* nw = is_q ? qn : kn;
    float ss = 0.0f;
    for (int d = threadIdx.x; d < D; d += kRopeThreads) {
        const float v = bf16_to_f32(src[d]);
        vals[d] = v;
        ss += v * v;
    }
    ss = wave_sum64(ss);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
    __syncthreads();
    float inv = 1.0f;
    if (nw) {
        float t = 0.0f;
        for (int w = 0; w < kRopeThreads / 64; ++w) t += part[w];
        inv = 1.0f / sqrtf(t / (float)D + eps);
    }
    const int half = D >> 1;
    const int64_t cs = (int64_t)b * ld_cs;
    const int64_t pos = *pos_p;
    if (seq_len && b == 0 && h == 0 && threadIdx.x == 0) *seq_len = pos + 1;
    // a position outside the cache writes no cache entry
    if (!is_q && (pos < 0 || pos >= S)) return;
    for (int d = threadIdx.x; d < D; d += kRopeThreads) {
        // rotate_half(v) = [-v2, v1]
        const int dp = d < half ? d + half : d - half;
        float v = vals[d], r = vals[dp];
        if (nw) {
            v = v * inv * bf16_to_f32(nw[d]);
            r = r * inv * bf16_to_f32(nw[dp]);
        }
        if (d < half) r = -r;
        const float o = v * ld_any(cosp, cs_f32, cs + d) + r * ld_any(sinp, cs_f32, cs + d);
        if (is_q) {
            q_out[((int64_t)b * HQ + h) * D + d] = o;
        } else {
            const int64_t base = (((int64_t)b * HKV + (h - HQ)) * S + pos) * D;
            st_any(kc, cache_f32, base + d, o);
            st_any(vc, cache_f32, base + d, bf16_to_f32(src[(int64_t)HKV * D + d]));
        }
    }
}

// ---------------------------------------------------------------------------
// Decode attention: one workgroup per (batch row b, kv head j, split sp).
// ---------------------------------------------------------------------------
constexpr int kBlk = 16;           // positions per block (the MFMA's 16 columns)
constexpr int kUnsplitMax = 160;   // attended positions up to which a call runs unsplit
constexpr float kNegBig = -1e30f;  // initial running max, as the reference
constexpr float kLog2e = 1.4426950408889634f;

// 2^x with the hardware instruction alone (results below 2^-126 flush to
// zero, which a softmax weight can afford).
__device__ __forceinline__ float fexp2(float x) { return __builtin_amdgcn_exp2f(x); }

struct AttnParams {
    // fused step: the token's qkv row and the q/k norm + RoPE inputs
    const uint16_t* qkv;
    int64_t ld_qkv;
    const uint16_t* qn;
    const uint16_t* kn;
    float eps;
    const void* cosp;
    const void* sinp;
    int cs_f32;
    int64_t ld_cs;
    int64_t* seq_len;
    // attention only: q already normed and rotated, fp32 [B][HQ][D]
    const float* q;
    void* kc;
    void* vc;
    const void* mask;
    int64_t ld_mask;
    int mask_dtype;
    const int64_t* pos;
    float scale;
    int HQ, HKV, G, S, split;
    float* part;         // [B][HQ][split][D + 4] (acc, m, l, 2 pad)
    unsigned* counters;  // [B][HKV] arrivals, zero between calls
    uint16_t* out;
    int64_t ld_out;
};

// The registers of one 16-position block: key operands and raw value words.
// MV (bf16 cache, D <= 256): p v on the matrix cores, and lane (col, grp)
// holds value rows 4 grp .. 4 grp + 3 of the block at columns D/16 col ..
// D/16 col + D/16 - 1 -- column D/16 col + c of those 4 rows is exactly the
// B operand of the 16x16x16 MFMA of column tile c.  Otherwise (VALU p v)
// lane l holds columns DL l .. DL l + DL - 1 of all 16 rows.
template <int DL, bool F32C>
struct KvBlock {
    static constexpr int T = 2 * DL;  // MFMA k-steps per key row
    static constexpr bool MV = !F32C && DL <= 4;
    static constexpr int VW = MV ? 2 * DL : (F32C ? DL : (DL >= 2 ? DL / 2 : 1));  // value words per row
    static constexpr int VR = MV ? 4 : kBlk;                                     // value rows per lane
    u32x4 kh[T], kl[T];
    uint32_t v[VR][VW];
    uint32_t mraw;  // raw mask entry at this lane's key position
};

// 8 cache elements of one key row as an MFMA operand; an fp32 cache gives
// hi + lo bf16 parts.
template <bool F32C>
__device__ __forceinline__ void load_k8(const void* kc, int64_t off, u32x4& hi, u32x4& lo) {
    if constexpr (F32C) {
        const float* p = reinterpret_cast<const float*>(kc) + off;
        const float4 x0 = *reinterpret_cast<const float4*>(p);
        const float4 x1 = *reinterpret_cast<const float4*>(p + 4);
        const float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        split8(v, hi, lo);
    } else {
        hi = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(kc) + off);
        lo = u32x4{0u, 0u, 0u, 0u};
    }
}

// DL consecutive value elements of one row, as raw words.
template <int DL, bool F32C>
__device__ __forceinline__ void load_vraw(const void* vc, int64_t off, uint32_t (&w)[KvBlock<DL, F32C>::VW]) {
    if constexpr (F32C) {
        const uint32_t* p = reinterpret_cast<const uint32_t*>(vc) + off;
        if constexpr (DL >= 4) {
            for (int i = 0; i < DL; i += 4) {
                const u32x4 t = *reinterpret_cast<const u32x4*>(p + i);
                w[i] = t[0];
                w[i + 1] = t[1];
                w[i + 2] = t[2];
                w[i + 3] = t[3];
            }
        } else {
            for (int i = 0; i < DL; ++i) w[i] = p[i];
        }
    } else {
        const uint16_t* p = reinterpret_cast<const uint16_t*>(vc) + off;
        if constexpr (DL == 8) {
            const u32x4 t = *reinterpret_cast<const u32x4*>(p);
            for (int i = 0; i < 4; ++i) w[i] = t[i];
        } else if constexpr (DL == 4) {
            const uint2 t = *reinterpret_cast<const uint2*>(p);
            w[0] = t.x;
            w[1] = t.y;
        } else if constexpr (DL == 2) {
            w[0] = *reinterpret_cast<const uint32_t*>(p);
        } else {
            w[0] = p[0];
        }
    }
}

template <int DL, bool F32C>
__device__ __forceinline__ float vword(const uint32_t (&w)[KvBlock<DL, F32C>::VW], int e) {
    if constexpr (F32C) return __uint_as_float(w[e]);
    if constexpr (DL == 1) return bf16_lo(w[0]);
    return (e & 1) ? bf16_hi(w[e >> 1]) : bf16_lo(w[e >> 1]);
}

// bf16 caches with D = 128 or 256 (the matrix-core p v path) load a block
// through range-checked buffer loads over the (row, kv head)'s cache, so a
// wave can issue a block's loads that send no request (an empty range).
__host__ __device__ constexpr bool kv_buffered(int DL, bool F32C) { return !F32C && DL >= 2 && DL <= 4; }

// One block's loads: key rows s0 + col (lane col), value rows s0 .. s0 + 15
// and the mask entries, rows past the split's last one clamped to it.  s0
// and s_hi are wave-uniform, so the value rows' addresses are scalar and
// each load carries only the lane's column offset.  On the buffered path a
// block that is not `live` reads zeros without memory requests (its mask
// entry still loads, at a clamped position); the other paths always load.
template <int DL, bool F32C>
__device__ __forceinline__ void load_block(const AttnParams& a, int64_t kv_base, int s0, int s_hi, int64_t mrow,
                                           int lane, KvBlock<DL, F32C>& blk, bool live = true) {
    constexpr int D = 64 * DL;
    constexpr int ES = F32C ? 4 : 2;  // element bytes
    const int last = max(s_hi - 1, 0);  // an empty range reads row 0 (every cache has one), unused
    const int col = lane & 15, grp = lane >> 4;
    const int kpos = min(s0 + col, last);
    blk.mraw = ld_raw(a.mask, a.mask_dtype, mrow + kpos);  // first: its load depends on the dtype
    if constexpr (kv_buffered(DL, F32C)) {
        const uint32_t bytes = live ? (uint32_t)a.S * (D * 2) : 0u;  // S D 2 < 2^32 (checked at set-up)
        const __amdgpu_buffer_rsrc_t kr = buffer_rsrc(static_cast<const char*>(a.kc) + kv_base * 2, bytes);
        const __amdgpu_buffer_rsrc_t vr = buffer_rsrc(static_cast<const char*>(a.vc) + kv_base * 2, bytes);
        const uint32_t ko = (uint32_t)kpos * (D * 2) + 16 * grp;
        for (int t = 0; t < KvBlock<DL, F32C>::T; ++t) {
            blk.kh[t] = buffer_ld16(kr, ko + 64 * t);
            blk.kl[t] = u32x4{0u, 0u, 0u, 0u};
        }
        for (int r = 0; r < 4; ++r) {
            const uint32_t vo = (uint32_t)min(s0 + 4 * grp + r, last) * (D * 2) + 8 * DL * col;
            for (int i = 0; i < DL / 2; ++i) {
                const u32x4 t = buffer_ld16(vr, vo + 16 * i);
                for (int e = 0; e < 4; ++e) blk.v[r][4 * i + e] = t[e];
            }
        }
        return;
    }
    const char* kc = static_cast<const char*>(a.kc) + kv_base * ES;
    const char* krow = kc + (int64_t)kpos * (D * ES) + 8 * grp * ES;
    for (int t = 0; t < KvBlock<DL, F32C>::T; ++t) load_k8<F32C>(krow, 32 * t, blk.kh[t], blk.kl[t]);
    const char* vc = static_cast<const char*>(a.vc) + kv_base * ES;
    if constexpr (KvBlock<DL, F32C>::MV) {
        for (int r = 0; r < 4; ++r) {
            const int row = min(s0 + 4 * grp + r, last);
            const uint16_t* vp = reinterpret_cast<const uint16_t*>(vc + (int64_t)row * (D * ES)) + 4 * DL * col;
            if constexpr (DL == 1) {
                const u32x2 t = *reinterpret_cast<const u32x2*>(vp);
                blk.v[r][0] = t[0];
                blk.v[r][1] = t[1];
            } else {
                for (int i = 0; i < DL / 2; ++i) {
                    const u32x4 t = ldg16(vp + 8 * i);
                    for (int e = 0; e < 4; ++e) blk.v[r][4 * i + e] = t[e];
                }
            }
        }
    } else {
        for (int p = 0; p < kBlk; ++p) {
            const int row = min(s0 + p, last);
            load_vraw<DL, F32C>(vc + (int64_t)row * (D * ES), DL * lane, blk.v[p]);
        }
    }
}

// Max / sum over each aligned group of 16 lanes (one DPP row; every lane
// gets it): swap within pairs, within quads, then rotate the row by 4 and 8.
constexpr int kDppRowRor4 = 0x124, kDppRowRor8 = 0x128;

__device__ __forceinline__ float max16(float v) {
    v = fmaxf(v, dpp_f32<kDppXor1>(v));
    v = fmaxf(v, dpp_f32<kDppXor2>(v));
    v = fmaxf(v, dpp_f32<kDppRowRor4>(v));
    return fmaxf(v, dpp_f32<kDppRowRor8>(v));
}

__device__ __forceinline__ float sum16(float v) {
    v += dpp_f32<kDppXor1>(v);
    v += dpp_f32<kDppXor2>(v);
    v += dpp_f32<kDppRowRor4>(v);
    return v + dpp_f32<kDppRowRor8>(v);
}

__device__ __forceinline__ float bcast(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// DL = D / 64 columns per lane; GM = 4 or 16 heads of register state (G <=
// GM); F32C: fp32 cache; FUSED: q (and the new k, v) computed from qkv.
template <int DL, int GM, bool F32C, bool FUSED, int NWV>
__global__ void __launch_bounds__(64 * NWV) attn_kernel(const void* hrows, const void* hcos, const void* hsin,
                                                        const int64_t* hpos, void* hkc, void* hvc, int hld_qkv, int hG,
                                                        AttnParams a) {
    // the fields of the first loads, preloaded into SGPRs at wave launch
    // (kernarg preloading, as for the GEMV kernels); the host passes the same
    // values in the struct
    if constexpr (FUSED)
        a.qkv = static_cast<const uint16_t*>(hrows);
    else
        a.q = static_cast<const float*>(hrows);
    a.cosp = hcos;
    a.sinp = hsin;
    a.pos = hpos;
    a.kc = hkc;
    a.vc = hvc;
    a.ld_qkv = hld_qkv;
    a.G = hG;
    constexpr int kAttnWaves = NWV;
    constexpr int kAttnThreads = 64 * NWV;
    constexpr int D = 64 * DL;
    constexpr int T = D / 32;
    constexpr bool PF = !F32C && DL <= 4 && NWV == 4;  // prefetch the next block (registers allow it)
    using Blk = KvBlock<DL, F32C>;
    constexpr bool MV = Blk::MV;          // p v on the matrix cores
    constexpr int NT = D / 16;            // its column tiles
    __shared__ float qf[GM][D];
    __shared__ float css[(GM + 2) * DL];
    __shared__ float rinv[GM + 1];
    __shared__ u32x4 qop[T][2][64];  // the A operand (q hi, lo) of every lane
    __shared__ float p_lds[kAttnWaves][kBlk * GM];  // MV: [head][position], else [position][head]
    __shared__ float st_m[kAttnWaves][GM], st_l[kAttnWaves][GM];
    __shared__ float st_acc[kAttnWaves][GM][D];  // also the raw qkv rows of the prologue
    __shared__ int last;

    const int b = blockIdx.x, j = blockIdx.y, sp = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: block starts are scalar
    const int G = a.G;
    const int col = lane & 15, grp = lane >> 4;

    // The query rows (FUSED: the token's q heads j*G.., its key head j and
    // value head j) go out first, as raw words, one element per thread and
    // row chunk; nothing here waits on the cache position.
    constexpr int NR = FUSED ? GM + 2 : GM;                            // rows at most
    constexpr int NI = (NR * D + kAttnThreads - 1) / kAttnThreads;     // elements per thread
    const int nrows = FUSED ? G + 2 : G;
    uint32_t pre[NI];
    // (every thread issues all NI loads, rows past the last clamped to it,
    // so the number of loads in flight never depends on a branch)
    for (int i = 0; i < NI; ++i) {
        const int e = tid + i * kAttnThreads;
        const int r = min(e / D, nrows - 1), d = e % D;
        if constexpr (FUSED) {
            const int head = r < G ? j * G + r : (r == G ? a.HQ + j : a.HQ + a.HKV + j);
            pre[i] = a.qkv[(int64_t)b * a.ld_qkv + (int64_t)head * D + d];
        } else {
            pre[i] = __float_as_uint(a.q[((int64_t)b * a.HQ + (int64_t)j * G + r) * D + d]);
        }
    }

    // RoPE and norm operands of this thread's columns: element e = tid +
    // 256 i of a row sits in column (tid + 256 i) % D, i.e. column tid % D
    // for D <= 256 and tid or tid + 256 (i even / odd) for D = 512.
    constexpr int NC = D > kAttnThreads ? 2 : 1;
    const int cs_kind = a.cs_f32 ? BZ_DT_F32 : BZ_DT_BF16;
    uint32_t cs_r[NC], sn_r[NC], nw_r[NC][4];  // cos, sin, q/k norm weights at d and its partner
    if constexpr (FUSED) {
        const int64_t cs = (int64_t)b * a.ld_cs;
        for (int c = 0; c < NC; ++c) {
            const int d = (tid + c * kAttnThreads) % D;
            const int dp = d < D / 2 ? d + D / 2 : d - D / 2;
            cs_r[c] = ld_raw(a.cosp, cs_kind, cs + d);
            sn_r[c] = ld_raw(a.sinp, cs_kind, cs + d);
            // without norm weights, in-bounds loads of cos stand in (unused)
            const uint16_t* qn = a.qn ? a.qn : static_cast<const uint16_t*>(a.cosp);
            const uint16_t* kn = a.qn ? a.kn : static_cast<const uint16_t*>(a.cosp);
            nw_r[c][0] = qn[d];
            nw_r[c][1] = qn[dp];
            nw_r[c][2] = kn[d];
            nw_r[c][3] = kn[dp];
        }
    }

    // cache positions [0, min(pos, S - 1)]; none for pos < 0 (output 0)
    const int64_t pos = *a.pos;
    const int kv_len = pos < 0 ? 0 : (pos >= a.S ? a.S : (int)pos + 1);
    // Short contexts run unsplit: the workgroup of split 0 takes every
    // position and writes the output itself; the others leave before any
    // barrier.  Up to about 160 positions that beats a split plus the
    // cross-workgroup combine (measured on MI355X, 16 q / 4 kv heads of 256:
    // unsplit 8.5 against 9.7 us at 128 positions, even at 160, split 9.9
    // against 10.2 us at 192).  The choice follows the device position, so a
    // captured graph adapts to it.
    const int nsp = kv_len <= kUnsplitMax ? 1 : a.split;
    if (sp >= nsp) return;
    const int per = (kv_len + nsp - 1) / nsp;
    const int s_lo = sp * per, s_hi = min(s_lo + per, kv_len);
    const bool has_new = FUSED && pos >= s_lo && pos < s_hi;  // this split holds the new token
    const int64_t kv_base = ((int64_t)b * a.HKV + j) * a.S * D;
    const int64_t mrow = (int64_t)b * a.ld_mask;

    // The wave's first block goes out before the prologue's arithmetic --
    // except the block that holds the new token, which its wave loads after
    // the workgroup has written that token's key and value (the barrier at
    // the end of the prologue orders the workgroup's own stores before its
    // loads).  Later blocks load after that barrier anyway.  On the buffered
    // path every wave issues the block's loads, empty (no requests) where the
    // wave has no block or holds the new token: with the same loads on every
    // path, the waits for the query rows below count exactly instead of also
    // waiting for the cache rows behind a branch.  Measured on MI355X (16 q /
    // 4 kv heads of 256, bf16 cache of 1024, one row): 9.5 -> 8.6 us at 128
    // positions, 13.6 -> 12.7 us at 1024 over 8 splits; 0.2-0.3 us slower at
    // 256-512 positions over 8 splits, where most waves issue empty loads.
    Blk cur;
    int s0 = s_lo + wave * kBlk;
    const bool first_new = has_new && pos >= s0 && pos < s0 + kBlk;
    const bool first_live = !first_new && s0 < s_hi;
    if (kv_buffered(DL, F32C) || first_live) load_block<DL, F32C>(a, kv_base, s0, s_hi, mrow, lane, cur, first_live);

    if constexpr (FUSED) {
        // raw rows: [0, G) query heads, G: key head j, G + 1: value head j;
        // each wave's 64 elements of one i share a row
        float* raw = &st_acc[0][0][0];
        for (int i = 0; i < NI; ++i) {
            const int e = tid + i * kAttnThreads;
            if (e / D < nrows) {
                const float v = bf16_to_f32((uint16_t)pre[i]);
                raw[e] = v;
                const float ss = wave_sum64(v * v);
                if (lane == 0) css[e >> 6] = ss;
            }
        }
        __syncthreads();
        // inverse RMS of each normed row (q heads and the key head), chunk
        // partials summed in column order
        if (tid <= G) {
            float ss = 0.0f;
            for (int q = 0; q < DL; ++q) ss += css[tid * DL + q];
            rinv[tid] = a.qn ? 1.0f / sqrtf(ss / (float)D + a.eps) : 1.0f;
        }
        __syncthreads();
        const int nout = G + (has_new ? 1 : 0);
        for (int i = 0; i < NI; ++i) {
            const int e = tid + i * kAttnThreads;
            const int r = e / D, d = e - r * D;
            if (r >= nout) continue;
            const int c = NC == 2 ? (i & 1) : 0;
            const int dp = d < D / 2 ? d + D / 2 : d - D / 2;
            float v = raw[r * D + d], rr = raw[r * D + dp];
            if (a.qn) {
                const float inv = rinv[r];
                const bool isq = r < G;  // selects, not a run-time index into a register array
                v = v * inv * bf16_to_f32((uint16_t)(isq ? nw_r[c][0] : nw_r[c][2]));
                rr = rr * inv * bf16_to_f32((uint16_t)(isq ? nw_r[c][1] : nw_r[c][3]));
            }
            if (d < D / 2) rr = -rr;
            const float o = v * raw_f32(cs_r[c], cs_kind) + rr * raw_f32(sn_r[c], cs_kind);
            if (r < G) {
                qf[r][d] = o;
            } else {  // the new key into the cache
                st_any(a.kc, F32C, kv_base + pos * D + d, o);
            }
        }
        if (has_new) {
            for (int d = tid; d < D; d += kAttnThreads) st_any(a.vc, F32C, kv_base + pos * D + d, raw[(G + 1) * D + d]);
        }
        if (a.seq_len && b == 0 && j == 0 && sp == 0 && tid == 0) *a.seq_len = pos + 1;
    } else {
        float* qflat = &qf[0][0];
        for (int i = 0; i < NI; ++i) {
            const int e = tid + i * kAttnThreads;
            if (e < G * D) qflat[e] = __uint_as_float(pre[i]);
        }
    }
    __syncthreads();

    if (first_new && s0 < s_hi) load_block<DL, F32C>(a, kv_base, s0, s_hi, mrow, lane, cur);

    // A operand: row `col` = query head j*G + col (zero rows from G on);
    // element e of step t is scale * q[32t + 8 grp + e], as bf16 hi + lo.
    // The operands are the same for every wave: built once into LDS (wave w
    // builds steps w, w + 4, ...) and read back per block.
    {
        const bool qv = col < G;
        const float sc = qv ? a.scale : 0.0f;
        const float* qrow = qf[qv ? col : 0];
        for (int t = wave; t < T; t += kAttnWaves) {
            float v[8];
            for (int e = 0; e < 8; ++e) v[e] = qrow[32 * t + 8 * grp + e] * sc;
            split8(v, qop[t][0][lane], qop[t][1][lane]);
        }
    }
    __syncthreads();

    // Score state: lane holds heads 4 grp + r (r < 4) at position col; m is
    // uniform over the 16 lanes of a group, l is this lane's share.
    float m[4], l[4];
    for (int r = 0; r < 4; ++r) {
        m[r] = kNegBig;
        l[r] = 0.0f;
    }
    float acc[GM][DL];  // VALU p v: head h, this lane's DL columns
    for (int h = 0; h < GM; ++h)
        for (int e = 0; e < DL; ++e) acc[h][e] = 0.0f;
    f32x4_t accm[MV ? NT : 1];  // MV: tile c, lane (col, grp): heads 4 grp + r at column NT col + c
    for (int c = 0; c < (MV ? NT : 1); ++c) accm[c] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

    // One block: scores on the matrix cores, online softmax, p v on the
    // matrix cores (MV) or the VALU.
    auto process = [&](Blk& blk, const int s0) __attribute__((always_inline)) {
        const int kpos = s0 + col;
        const bool valid = kpos < s_hi;
        f32x4_t sc = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int t = 0; t < T; ++t) {
            const u32x4 qh = qop[t][0][lane], ql = qop[t][1][lane];
            sc = mfma16(qh, blk.kh[t], sc);
            sc = mfma16(ql, blk.kh[t], sc);
            if constexpr (F32C) sc = mfma16(qh, blk.kl[t], sc);
        }
        float alpha[4];
        const float mk = valid ? raw_f32(blk.mraw, a.mask_dtype) : 0.0f;
        for (int r = 0; r < 4; ++r) {
            const float s = valid ? sc[r] + mk : kNegBig;
            const float mn = fmaxf(m[r], max16(s));
            alpha[r] = fexp2((m[r] - mn) * kLog2e);
            const float pr = valid ? fexp2((s - mn) * kLog2e) : 0.0f;
            l[r] = l[r] * alpha[r] + pr;
            m[r] = mn;
            // every head slot of the block is written (rows past G hold
            // finite values of zero query rows and are never output)
            if (4 * grp + r < GM) {
                if constexpr (MV)
                    p_lds[wave][(4 * grp + r) * kBlk + col] = pr;
                else
                    p_lds[wave][col * GM + 4 * grp + r] = pr;
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if constexpr (MV) {
            // A: head col's p at positions 4 grp .. 4 grp + 3 (rows from G
            // on repeat head GM - 1 and are never output), as bf16 hi + lo
            const float4 pq = *reinterpret_cast<const float4*>(&p_lds[wave][min(col, GM - 1) * kBlk + 4 * grp]);
            const uint16_t h0 = f32_to_bf16(pq.x), h1 = f32_to_bf16(pq.y), h2 = f32_to_bf16(pq.z),
                           h3 = f32_to_bf16(pq.w);
            const u32x2 ah = {(uint32_t)h0 | ((uint32_t)h1 << 16), (uint32_t)h2 | ((uint32_t)h3 << 16)};
            const u32x2 al = {pack_bf16x2(pq.x - bf16_to_f32(h0), pq.y - bf16_to_f32(h1)),
                              pack_bf16x2(pq.z - bf16_to_f32(h2), pq.w - bf16_to_f32(h3))};
            // the accumulator lane (col, grp) holds heads 4 grp + r: its own alphas
            for (int c = 0; c < NT; ++c)
                for (int r = 0; r < 4; ++r) accm[c][r] *= alpha[r];
            for (int c = 0; c < NT; ++c) {
                // B: column NT col + c of value rows 4 grp .. 4 grp + 3
                const uint32_t w0 = blk.v[0][c >> 1], w1 = blk.v[1][c >> 1], w2 = blk.v[2][c >> 1],
                               w3 = blk.v[3][c >> 1];
                u32x2 bv;
                if (c & 1) {
                    bv[0] = (w0 >> 16) | (w1 & 0xFFFF0000u);
                    bv[1] = (w2 >> 16) | (w3 & 0xFFFF0000u);
                } else {
                    bv[0] = (w0 & 0xFFFFu) | (w1 << 16);
                    bv[1] = (w2 & 0xFFFFu) | (w3 << 16);
                }
                accm[c] = mfma16k16(ah, bv, accm[c]);
                accm[c] = mfma16k16(al, bv, accm[c]);
            }
        } else {
        // rescale by head h's alpha (lane 16 (h / 4), element h % 4)
        for (int h = 0; h < GM; ++h) {
            const float al = bcast(alpha[h & 3], 16 * (h >> 2));
            for (int e = 0; e < DL; ++e) acc[h][e] *= al;
        }
        for (int p = 0; p < kBlk; ++p) {
            float vv[DL];
            for (int e = 0; e < DL; ++e) vv[e] = vword<DL, F32C>(blk.v[p], e);
            float pw[GM];
            for (int h = 0; h < GM; h += 4) {
                const float4 t = *reinterpret_cast<const float4*>(&p_lds[wave][p * GM + h]);
                pw[h] = t.x;
                pw[h + 1] = t.y;
                pw[h + 2] = t.z;
                pw[h + 3] = t.w;
            }
            for (int h = 0; h < GM; ++h)
                for (int e = 0; e < DL; ++e) acc[h][e] += pw[h] * vv[e];
        }
        }
        // p_lds is rewritten by this wave's next block
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
    };
    constexpr int kStride = kAttnWaves * kBlk;
    if constexpr (PF) {
        // two register blocks in turn: the next one loads while this one computes
        Blk other;
        for (; s0 < s_hi; s0 += 2 * kStride) {
            const int s1 = s0 + kStride;
            if (s1 < s_hi) load_block<DL, F32C>(a, kv_base, s1, s_hi, mrow, lane, other);
            process(cur, s0);
            if (s1 >= s_hi) break;
            if (s1 + kStride < s_hi) load_block<DL, F32C>(a, kv_base, s1 + kStride, s_hi, mrow, lane, cur);
            process(other, s1);
        }
    } else {
        for (; s0 < s_hi; s0 += kStride) {
            process(cur, s0);
            if (s0 + kStride < s_hi) load_block<DL, F32C>(a, kv_base, s0 + kStride, s_hi, mrow, lane, cur);
        }
    }

    // Per-wave state to LDS: head 4 grp + r's m and l (l summed over the
    // group's 16 positions).
    __syncthreads();  // the prologue's raw rows share st_acc
    for (int r = 0; r < 4; ++r) {
        const float ls = sum16(l[r]);
        const int h = 4 * grp + r;
        if (col == 0 && h < G) {
            st_m[wave][h] = m[r];
            st_l[wave][h] = ls;
        }
    }
    if constexpr (MV) {
        for (int r = 0; r < 4; ++r) {
            const int h = 4 * grp + r;
            if (h < G)
                for (int c = 0; c < NT; c += 4)
                    *reinterpret_cast<float4*>(&st_acc[wave][h][NT * col + c]) =
                        make_float4(accm[c][r], accm[c + 1][r], accm[c + 2][r], accm[c + 3][r]);
        }
    } else {
        for (int h = 0; h < GM; ++h)
            if (h < G)
                for (int e = 0; e < DL; ++e) st_acc[wave][h][DL * lane + e] = acc[h][e];
    }
    __syncthreads();

    // Merge the waves in a fixed order; write the output or the partial.
    // Each thread forms its head's wave weights itself (8 values from LDS):
    // no serial step and no barrier between the state and the merge.
    const int64_t hq0 = (int64_t)b * a.HQ + (int64_t)j * G;
    for (int i = tid; i < G * D; i += kAttnThreads) {
        const int h = i / D, d = i - h * D;
        float mt = kNegBig;
        for (int w = 0; w < kAttnWaves; ++w) mt = fmaxf(mt, st_m[w][h]);
        float lt = 0.0f, at = 0.0f;
        for (int w = 0; w < kAttnWaves; ++w) {
            const float f = fexp2((st_m[w][h] - mt) * kLog2e);
            lt += st_l[w][h] * f;
            at += st_acc[w][h][d] * f;
        }
        if (nsp == 1) {
            a.out[(int64_t)b * a.ld_out + (int64_t)(j * G + h) * D + d] = f32_to_bf16(lt > 0.0f ? at / lt : 0.0f);
        } else {  // agent-scope stores: coherent across XCDs without an L2 write-back
            float* pp = a.part + ((hq0 + h) * a.split + sp) * (D + 4);
            __hip_atomic_store(&pp[d], at, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (d == 0) {
                __hip_atomic_store(&pp[D], mt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(&pp[D + 1], lt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
    if (nsp == 1) return;

    // The last workgroup of (b, j) to finish combines the splits.  Every
    // thread waits until its partial stores have completed (agent-scope
    // stores complete at the point of coherence) before the workgroup counts
    // its arrival; the last one reads the partials with agent-scope loads.
    // No L2 write-back or invalidate is needed for that.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) {
        const unsigned prev =
            __hip_atomic_fetch_add(&a.counters[b * a.HKV + j], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = prev == (unsigned)a.split - 1u;
    }
    __syncthreads();
    if (!last) return;
    // Element i = (h, d): each thread loads, for its NE elements, every
    // split's partial and its head's (m, l) in batches of SB splits (all in
    // flight at once; SB NE <= 16 keeps them in registers), and merges them
    // in split order, online: with M the running max, acc and L are rescaled
    // by exp(M_old - M) and gain w_s acc_s and w_s l_s, w_s = exp(m_s - M).
    // One memory round trip per batch and no barrier (the weights were first
    // formed per head in LDS: a second round trip and a barrier).
    constexpr int NE = (GM * D + kAttnThreads - 1) / kAttnThreads;
    constexpr int SB = NE <= 2 ? 8 : (NE <= 4 ? 4 : (NE <= 8 ? 2 : 1));
    float acc0[NE], lsum[NE], mrun[NE];
    for (int q = 0; q < NE; ++q) {
        acc0[q] = 0.0f;
        lsum[q] = 0.0f;
        mrun[q] = kNegBig;
    }
    for (int s0 = 0; s0 < a.split; s0 += SB) {
        float v[NE][SB], ms[NE][SB], ls[NE][SB];
        for (int q = 0; q < NE; ++q) {
            const int i = min(tid + q * kAttnThreads, G * D - 1);
            const int h = i / D, d = i - h * D;
            const float* ph = a.part + (hq0 + h) * a.split * (D + 4);
            for (int u = 0; u < SB; ++u) {
                const float* pp = ph + min(s0 + u, a.split - 1) * (D + 4);
                v[q][u] = __hip_atomic_load(pp + d, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                ms[q][u] = __hip_atomic_load(pp + D, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                ls[q][u] = __hip_atomic_load(pp + D + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        for (int q = 0; q < NE; ++q) {
            float mb = mrun[q];
            for (int u = 0; u < SB; ++u)
                if (s0 + u < a.split) mb = fmaxf(mb, ms[q][u]);
            const float rs = fexp2((mrun[q] - mb) * kLog2e);
            acc0[q] *= rs;
            lsum[q] *= rs;
            mrun[q] = mb;
            for (int u = 0; u < SB; ++u)
                if (s0 + u < a.split) {
                    const float w = fexp2((ms[q][u] - mb) * kLog2e);
                    acc0[q] += v[q][u] * w;
                    lsum[q] += ls[q][u] * w;
                }
        }
    }
    for (int q = 0; q < NE; ++q) {
        const int i = tid + q * kAttnThreads;
        if (i < G * D) {
            const int h = i / D, d = i - h * D;
            const float lt = lsum[q];
            a.out[(int64_t)b * a.ld_out + (int64_t)(j * G + h) * D + d] =
                f32_to_bf16(lt > 0.0f ? acc0[q] / lt : 0.0f);
        }
    }
    if (tid == 0) __hip_atomic_store(&a.counters[b * a.HKV + j], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Waves per workgroup: 8 for a bf16 cache with D <= 256 and up to 4 query
// heads per kv head (one 16-position block per wave at a time, no double
// buffer, so the blocks of a short context run side by side), else 4 (two
// blocks in turn per wave on the double-buffered path, or the VALU path).
template <int DL, int GM, bool FUSED>
static void launch_attn(const AttnParams& a, bool f32c, dim3 grid, hipStream_t st) {
    const void* rows = FUSED ? static_cast<const void*>(a.qkv) : static_cast<const void*>(a.q);
    const int ld = (int)a.ld_qkv;  // bz_attn_step: checked to fit 32 bits
    if (f32c)
        hipLaunchKernelGGL((attn_kernel<DL, GM, true, FUSED, 4>), grid, dim3(64 * 4), 0, st, rows, a.cosp, a.sinp, a.pos,
                           a.kc, a.vc, ld, a.G, a);
    else if constexpr (DL <= 4 && GM == 4)
        hipLaunchKernelGGL((attn_kernel<DL, GM, false, FUSED, 8>), grid, dim3(64 * 8), 0, st, rows, a.cosp, a.sinp, a.pos,
                           a.kc, a.vc, ld, a.G, a);
    else
        hipLaunchKernelGGL((attn_kernel<DL, GM, false, FUSED, 4>), grid, dim3(64 * 4), 0, st, rows, a.cosp, a.sinp, a.pos,
                           a.kc, a.vc, ld, a.G, a);
}

template <bool FUSED>
static int launch_attn_any(const AttnParams& a, int D, bool f32c, dim3 grid, hipStream_t st) {
    const bool g4 = a.G <= 4;
    switch (D) {
        case 64: g4 ? launch_attn<1, 4, FUSED>(a, f32c, grid, st) : launch_attn<1, 16, FUSED>(a, f32c, grid, st); break;
        case 128: g4 ? launch_attn<2, 4, FUSED>(a, f32c, grid, st) : launch_attn<2, 16, FUSED>(a, f32c, grid, st); break;
        case 256: g4 ? launch_attn<4, 4, FUSED>(a, f32c, grid, st) : launch_attn<4, 16, FUSED>(a, f32c, grid, st); break;
        default: launch_attn<8, 4, FUSED>(a, f32c, grid, st); break;
    }
    return hipGetLastError() == hipSuccess ? BZ_OK : BZ_ERR_LAUNCH;
}

static bool aligned(const void* p, uintptr_t n) { return (reinterpret_cast<uintptr_t>(p) & (n - 1)) == 0; }

static size_t partial_floats(int B, int HQ, int D, int split) { return (size_t)B * HQ * split * (D + 4); }

// Checks shared by bz_attn_decode and bz_attn_step; fills the attention part
// of the parameters.
static int attn_setup(AttnParams& a, const void* k_cache, const void* v_cache, int cache_dtype, int B, int HQ, int HKV,
                      int D, int S, const void* mask, int mask_dtype, int64_t ld_mask, const int64_t* pos, float scale,
                      int split, void* workspace, void* out, int64_t ld_out) {
    if (!k_cache || !v_cache || !mask || !pos || !out) return BZ_ERR_INVALID_ARG;
    if (B < 1 || HQ < 1 || HKV < 1 || S < 1 || HQ % HKV) return BZ_ERR_INVALID_ARG;
    if (cache_dtype != BZ_DT_BF16 && cache_dtype != BZ_DT_F32) return BZ_ERR_INVALID_ARG;
    if (mask_dtype != BZ_DT_BF16 && mask_dtype != BZ_DT_F32 && mask_dtype != BZ_MASK_BOOL) return BZ_ERR_INVALID_ARG;
    if (split < 1 || split > BZ_ATTN_MAX_SPLIT || (split > 1 && !workspace)) return BZ_ERR_INVALID_ARG;
    if ((ld_mask != 0 && ld_mask < S) || ld_mask < 0 || ld_out < (int64_t)HQ * D) return BZ_ERR_SHAPE;
    const int G = HQ / HKV;
    if (D != 64 && D != 128 && D != 256 && D != 512) return BZ_ERR_UNSUPPORTED;
    if ((int64_t)S * D * 4 >= (int64_t(1) << 32)) return BZ_ERR_UNSUPPORTED;  // 32-bit offsets in one head's cache
    if (G > 16 || (G > 4 && D == 512)) return BZ_ERR_UNSUPPORTED;
    if (!aligned(k_cache, 16) || !aligned(v_cache, 16) || !aligned(out, 2) || !aligned(workspace, 4))
        return BZ_ERR_ALIGNMENT;
    a.kc = const_cast<void*>(k_cache);
    a.vc = const_cast<void*>(v_cache);
    a.mask = mask;
    a.ld_mask = ld_mask;
    a.mask_dtype = mask_dtype;
    a.pos = pos;
    a.scale = scale;
    a.HQ = HQ;
    a.HKV = HKV;
    a.G = G;
    a.S = S;
    a.split = split;
    a.part = static_cast<float*>(workspace);
    a.counters = split > 1 ? reinterpret_cast<unsigned*>(a.part + partial_floats(B, HQ, D, split)) : nullptr;
    a.out = static_cast<uint16_t*>(out);
    a.ld_out = ld_out;
    return BZ_OK;
}

}  // namespace bz

using namespace bz;

extern "C" int bz_qkv_rope_cache(const void* qkv, int64_t ld_qkv, int32_t B, int32_t HQ, int32_t HKV, int32_t D,
                                 const void* q_norm, const void* k_norm, float eps, const void* cos, const void* sin,
                                 int32_t cs_dtype, int64_t ld_cs, const int64_t* pos, float* q_out, void* k_cache,
                                 void* v_cache, int32_t S, int32_t cache_dtype, int64_t* seq_len, void* stream) {
    if (!qkv || !cos || !sin || !pos || !q_out || !k_cache || !v_cache) return BZ_ERR_INVALID_ARG;
    if (B < 1 || HQ < 1 || HKV < 1 || S < 1 || (q_norm == nullptr) != (k_norm == nullptr)) return BZ_ERR_INVALID_ARG;
    if ((cs_dtype != BZ_DT_BF16 && cs_dtype != BZ_DT_F32) || (cache_dtype != BZ_DT_BF16 && cache_dtype != BZ_DT_F32))
        return BZ_ERR_INVALID_ARG;
    if (D < 2 || D % 2 || D > kMaxRopeDim || ld_qkv < (int64_t)(HQ + 2 * HKV) * D || ld_cs < 0) return BZ_ERR_SHAPE;
    hipLaunchKernelGGL(qkv_rope_cache_kernel, dim3(B, HQ + HKV), dim3(kRopeThreads), 0,
                       static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(qkv), ld_qkv, HQ, HKV, D,
                       static_cast<const uint16_t*>(q_norm), static_cast<const uint16_t*>(k_norm), eps, cos, sin,
                       cs_dtype == BZ_DT_F32, ld_cs, pos, q_out, k_cache, v_cache, S, cache_dtype == BZ_DT_F32,
                       seq_len);
    return hipGetLastError() == hipSuccess ? BZ_OK : BZ_ERR_LAUNCH;
}

extern "C" int32_t bz_attn_default_split(int32_t S) {
    const int32_t s = (S + 127) / 128;  // about 128 positions per workgroup at a full cache
    return s < 1 ? 1 : (s > 32 ? 32 : s);
}

extern "C" size_t bz_attn_workspace(int32_t B, int32_t HQ, int32_t HKV, int32_t D, int32_t split) {
    if (B < 1 || HQ < 1 || HKV < 1 || D < 1 || split <= 1) return 0;
    return partial_floats(B, HQ, D, split) * sizeof(float) + (size_t)B * HKV * sizeof(unsigned);
}

extern "C" int bz_attn_decode(const float* q, const void* k_cache, const void* v_cache, int32_t cache_dtype, int32_t B,
                              int32_t HQ, int32_t HKV, int32_t D, int32_t S, const void* mask, int32_t mask_dtype,
                              int64_t ld_mask, const int64_t* pos, float scale, int32_t split, void* workspace,
                              void* out, int64_t ld_out, void* stream) {
    if (!q) return BZ_ERR_INVALID_ARG;
    AttnParams a = {};
    int rc = attn_setup(a, k_cache, v_cache, cache_dtype, B, HQ, HKV, D, S, mask, mask_dtype, ld_mask, pos, scale,
                        split, workspace, out, ld_out);
    if (rc != BZ_OK) return rc;
    if (!aligned(q, 16)) return BZ_ERR_ALIGNMENT;
    a.q = q;
    return launch_attn_any<false>(a, D, cache_dtype == BZ_DT_F32, dim3(B, HKV, split),
                                  static_cast<hipStream_t>(stream));
}

extern "C" int bz_attn_step(const void* qkv, int64_t ld_qkv, int32_t B, int32_t HQ, int32_t HKV, int32_t D,
                            const void* q_norm, const void* k_norm, float eps, const void* cos, const void* sin,
                            int32_t cs_dtype, int64_t ld_cs, const int64_t* pos, void* k_cache, void* v_cache,
                            int32_t S, int32_t cache_dtype, int64_t* seq_len, const void* mask, int32_t mask_dtype,
                            int64_t ld_mask, float scale, int32_t split, void* workspace, void* out, int64_t ld_out,
                            void* stream) {
    if (!qkv || !cos || !sin || (q_norm == nullptr) != (k_norm == nullptr)) return BZ_ERR_INVALID_ARG;
    if (cs_dtype != BZ_DT_BF16 && cs_dtype != BZ_DT_F32) return BZ_ERR_INVALID_ARG;
    AttnParams a = {};
    int rc = attn_setup(a, k_cache, v_cache, cache_dtype, B, HQ, HKV, D, S, mask, mask_dtype, ld_mask, pos, scale,
                        split, workspace, out, ld_out);
    if (rc != BZ_OK) return rc;
    if (ld_qkv < (int64_t)(HQ + 2 * HKV) * D || ld_cs < 0) return BZ_ERR_SHAPE;
    if (ld_qkv > 0x7FFFFFFF) return BZ_ERR_UNSUPPORTED;  // a preloaded 32-bit kernel argument
    a.qkv = static_cast<const uint16_t*>(qkv);
    a.ld_qkv = ld_qkv;
    a.qn = static_cast<const uint16_t*>(q_norm);
    a.kn = static_cast<const uint16_t*>(k_norm);
    a.eps = eps;
    a.cosp = cos;
    a.sinp = sin;
    a.cs_f32 = cs_dtype == BZ_DT_F32;
    a.ld_cs = ld_cs;
    a.seq_len = seq_len;
    return launch_attn_any<true>(a, D, cache_dtype == BZ_DT_F32, dim3(B, HKV, split),
                                 static_cast<hipStream_t>(stream));
}
