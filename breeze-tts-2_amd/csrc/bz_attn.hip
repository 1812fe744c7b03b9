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
// h*D..h*D+D-1.  Partials (split > 1) fp32 [B][HQ][split][D + 2] = (acc, m, l).
//
// attn_decode runs one workgroup per (batch row, kv head, split), so the G =
// HQ/HKV query heads sharing a kv head read its keys and values once.  Its
// four waves take 16-position blocks of the split in turn:
//   scores   v_mfma_f32_16x16x32_bf16 with A = the G query rows (padded to
//            16) and B = 16 key rows; q is carried as bf16 hi + lo parts
//            (two MFMAs, ~16 significant bits; an fp32 cache also splits k)
//   softmax  online (running max m, sum l) per head, exp2-based
//   p v      VALU: lane l owns D/64 consecutive columns of every head and
//            reads each value row with one coalesced load
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

__device__ __forceinline__ float ld_any(const void* p, bool f32, int64_t i) {
    return f32 ? reinterpret_cast<const float*>(p)[i] : bf16_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
}

// Additive mask value: bf16, fp32, or a bool mask (nonzero = attend -> 0,
// zero -> -1e30, the reference's conversion).
__device__ __forceinline__ float ld_mask(const void* p, int dtype, int64_t i) {
    if (dtype == BZ_MASK_BOOL) return reinterpret_cast<const uint8_t*>(p)[i] ? 0.0f : -1e30f;
    return ld_any(p, dtype == BZ_DT_F32, i);
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
    ss = wave_sum(ss);
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
// Decode attention.
// ---------------------------------------------------------------------------
constexpr int kAttnWaves = 4;
constexpr int kBlk = 16;           // positions per block (the MFMA's 16 columns)
constexpr float kNegBig = -1e30f;  // initial running max, as the reference
constexpr float kLog2e = 1.4426950408889634f;

struct AttnParams {
    const float* q;
    const void* kc;
    const void* vc;
    const void* mask;
    int64_t ld_mask;
    int mask_dtype;
    const int64_t* pos;
    float scale;
    int HQ, HKV, G, S, split;
    float* part;
    uint16_t* out;
    int64_t ld_out;
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

// DL consecutive value elements of one row, widened to fp32.
template <int DL, bool F32C>
__device__ __forceinline__ void load_v(const void* vc, int64_t off, float (&v)[DL]) {
    if constexpr (F32C) {
        const float* p = reinterpret_cast<const float*>(vc) + off;
        if constexpr (DL >= 4) {
            for (int i = 0; i < DL; i += 4) {
                const float4 t = *reinterpret_cast<const float4*>(p + i);
                v[i] = t.x;
                v[i + 1] = t.y;
                v[i + 2] = t.z;
                v[i + 3] = t.w;
            }
        } else {
            for (int i = 0; i < DL; ++i) v[i] = p[i];
        }
    } else {
        const uint16_t* p = reinterpret_cast<const uint16_t*>(vc) + off;
        if constexpr (DL == 8) {
            const u32x4 t = *reinterpret_cast<const u32x4*>(p);
            for (int i = 0; i < 4; ++i) {
                v[2 * i] = bf16_lo(t[i]);
                v[2 * i + 1] = bf16_hi(t[i]);
            }
        } else if constexpr (DL == 4) {
            const uint2 t = *reinterpret_cast<const uint2*>(p);
            v[0] = bf16_lo(t.x);
            v[1] = bf16_hi(t.x);
            v[2] = bf16_lo(t.y);
            v[3] = bf16_hi(t.y);
        } else if constexpr (DL == 2) {
            const uint32_t t = *reinterpret_cast<const uint32_t*>(p);
            v[0] = bf16_lo(t);
            v[1] = bf16_hi(t);
        } else {
            v[0] = bf16_to_f32(p[0]);
        }
    }
}

// Max / sum over each aligned group of 16 lanes (every lane gets it).
__device__ __forceinline__ float max16(float v) {
    for (int o = 1; o < 16; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

__device__ __forceinline__ float sum16(float v) {
    for (int o = 1; o < 16; o <<= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ float bcast(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// DL = D / 64 columns per lane; GM = 4 or 16 heads of register state (G <= GM).
template <int DL, int GM, bool F32C>
__global__ void __launch_bounds__(64 * kAttnWaves) attn_decode_kernel(AttnParams a) {
    constexpr int D = 64 * DL;
    constexpr int T = D / 32;  // MFMA k-steps per key row
    __shared__ float p_lds[kAttnWaves][kBlk][GM];
    __shared__ float st_m[kAttnWaves][GM], st_l[kAttnWaves][GM];
    __shared__ float st_acc[kAttnWaves][GM][D];

    const int b = blockIdx.x, j = blockIdx.y, sp = blockIdx.z;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int G = a.G;
    const int col = lane & 15, grp = lane >> 4;
    // cache positions [0, min(pos, S - 1)]; none for pos < 0 (output 0)
    const int64_t pos = *a.pos;
    const int kv_len = pos < 0 ? 0 : (pos >= a.S ? a.S : (int)pos + 1);
    const int per = (kv_len + a.split - 1) / a.split;
    const int s_lo = sp * per, s_hi = min(s_lo + per, kv_len);
    const int64_t kv_base = ((int64_t)b * a.HKV + j) * a.S * D;

    // A operand: row `col` = query head j*G + col (zero rows from G on);
    // element e of step t is scale * q[32t + 8 grp + e].
    u32x4 qh[T], ql[T];
    {
        const bool qv = col < G;
        const float* qrow = a.q + ((int64_t)b * a.HQ + (int64_t)j * G + (qv ? col : 0)) * D;
        const float sc = qv ? a.scale : 0.0f;
        for (int t = 0; t < T; ++t) {
            const float4 x0 = *reinterpret_cast<const float4*>(qrow + 32 * t + 8 * grp);
            const float4 x1 = *reinterpret_cast<const float4*>(qrow + 32 * t + 8 * grp + 4);
            const float v[8] = {x0.x * sc, x0.y * sc, x0.z * sc, x0.w * sc,
                                x1.x * sc, x1.y * sc, x1.z * sc, x1.w * sc};
            split8(v, qh[t], ql[t]);
        }
    }

    // Score state: lane holds heads 4 grp + r (r < 4) at position col; m is
    // uniform over the 16 lanes of a group, l is this lane's share.
    float m[4], l[4];
    for (int r = 0; r < 4; ++r) {
        m[r] = kNegBig;
        l[r] = 0.0f;
    }
    float acc[GM][DL];
    for (int h = 0; h < GM; ++h)
        for (int e = 0; e < DL; ++e) acc[h][e] = 0.0f;
    const int64_t mrow = (int64_t)b * a.ld_mask;

    for (int s0 = s_lo + wave * kBlk; s0 < s_hi; s0 += kAttnWaves * kBlk) {
        const int kpos = s0 + col;
        const bool valid = kpos < s_hi;
        const int64_t krow = kv_base + (int64_t)(valid ? kpos : s_lo) * D;
        u32x4 kh[T], kl[T];
        for (int t = 0; t < T; ++t) load_k8<F32C>(a.kc, krow + 32 * t + 8 * grp, kh[t], kl[t]);
        float vv[kBlk][DL];
        for (int p = 0; p < kBlk; ++p) {
            const int vp = s0 + p < s_hi ? s0 + p : s_lo;
            load_v<DL, F32C>(a.vc, kv_base + (int64_t)vp * D + DL * lane, vv[p]);
        }
        const float mk = valid ? ld_mask(a.mask, a.mask_dtype, mrow + kpos) : 0.0f;

        f32x4_t sc = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int t = 0; t < T; ++t) {
            sc = mfma16(qh[t], kh[t], sc);
            sc = mfma16(ql[t], kh[t], sc);
            if constexpr (F32C) sc = mfma16(qh[t], kl[t], sc);
        }
        float alpha[4];
        for (int r = 0; r < 4; ++r) {
            const float s = valid ? sc[r] + mk : kNegBig;
            const float mn = fmaxf(m[r], max16(s));
            alpha[r] = exp2f((m[r] - mn) * kLog2e);
            const float pr = valid ? exp2f((s - mn) * kLog2e) : 0.0f;
            l[r] = l[r] * alpha[r] + pr;
            m[r] = mn;
            const int h = 4 * grp + r;
            if (h < G) p_lds[wave][col][h] = pr;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // rescale by head h's alpha (lane 16 (h / 4), element h % 4)
        for (int h = 0; h < GM; ++h) {
            if (h < G) {
                const float al = bcast(alpha[h & 3], 16 * (h >> 2));
                for (int e = 0; e < DL; ++e) acc[h][e] *= al;
            }
        }
        for (int p = 0; p < kBlk; ++p) {
            for (int h = 0; h < GM; ++h) {
                if (h < G) {
                    const float pw = p_lds[wave][p][h];
                    for (int e = 0; e < DL; ++e) acc[h][e] += pw * vv[p][e];
                }
            }
        }
        // p_lds is rewritten by this wave's next block
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
    }

    // Per-wave state to LDS: head 4 grp + r's m and l (l summed over the
    // group's 16 positions).
    for (int r = 0; r < 4; ++r) {
        const float ls = sum16(l[r]);
        const int h = 4 * grp + r;
        if (col == 0 && h < G) {
            st_m[wave][h] = m[r];
            st_l[wave][h] = ls;
        }
    }
    for (int h = 0; h < GM; ++h)
        if (h < G)
            for (int e = 0; e < DL; ++e) st_acc[wave][h][DL * lane + e] = acc[h][e];
    __syncthreads();

    // Merge the waves in a fixed order; write the output or the partial.
    for (int i = threadIdx.x; i < G * D; i += 64 * kAttnWaves) {
        const int h = i / D, d = i - h * D;
        float mt = kNegBig;
        for (int w = 0; w < kAttnWaves; ++w) mt = fmaxf(mt, st_m[w][h]);
        float lt = 0.0f, at = 0.0f;
        for (int w = 0; w < kAttnWaves; ++w) {
            const float f = exp2f((st_m[w][h] - mt) * kLog2e);
            lt += st_l[w][h] * f;
            at += st_acc[w][h][d] * f;
        }
        const int hq = j * G + h;
        if (a.split == 1) {
            a.out[(int64_t)b * a.ld_out + (int64_t)hq * D + d] = f32_to_bf16(lt > 0.0f ? at / lt : 0.0f);
        } else {
            float* pp = a.part + (((int64_t)b * a.HQ + hq) * a.split + sp) * (D + 2);
            pp[d] = at;
            if (d == 0) {
                pp[D] = mt;
                pp[D + 1] = lt;
            }
        }
    }
}

// One workgroup of 64 lanes per (batch row, q head): merge the splits in
// split order.
__global__ void __launch_bounds__(64) attn_combine_kernel(const float* part, uint16_t* out, int64_t ld_out, int HQ,
                                                          int D, int split) {
    const int b = blockIdx.x, h = blockIdx.y;
    const float* base = part + ((int64_t)b * HQ + h) * split * (D + 2);
    float m = kNegBig;
    for (int s = 0; s < split; ++s) m = fmaxf(m, base[s * (D + 2) + D]);
    float l = 0.0f;
    for (int s = 0; s < split; ++s) l += base[s * (D + 2) + D + 1] * exp2f((base[s * (D + 2) + D] - m) * kLog2e);
    for (int d = threadIdx.x; d < D; d += 64) {
        float acc = 0.0f;
        for (int s = 0; s < split; ++s) acc += base[s * (D + 2) + d] * exp2f((base[s * (D + 2) + D] - m) * kLog2e);
        out[(int64_t)b * ld_out + (int64_t)h * D + d] = f32_to_bf16(l > 0.0f ? acc / l : 0.0f);
    }
}

template <int DL, int GM>
static void launch_attn(const AttnParams& a, bool f32c, dim3 grid, hipStream_t st) {
    if (f32c)
        hipLaunchKernelGGL((attn_decode_kernel<DL, GM, true>), grid, dim3(64 * kAttnWaves), 0, st, a);
    else
        hipLaunchKernelGGL((attn_decode_kernel<DL, GM, false>), grid, dim3(64 * kAttnWaves), 0, st, a);
}

static int launched() { return hipGetLastError() == hipSuccess ? BZ_OK : BZ_ERR_LAUNCH; }

static bool aligned(const void* p, uintptr_t n) { return (reinterpret_cast<uintptr_t>(p) & (n - 1)) == 0; }

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
    return launched();
}

extern "C" int32_t bz_attn_default_split(int32_t S) {
    const int32_t s = (S + 127) / 128;  // about 128 positions per workgroup at a full cache
    return s < 1 ? 1 : (s > 32 ? 32 : s);
}

extern "C" size_t bz_attn_workspace(int32_t B, int32_t HQ, int32_t D, int32_t split) {
    if (B < 1 || HQ < 1 || D < 1 || split <= 1) return 0;
    return (size_t)B * HQ * split * (D + 2) * sizeof(float);
}

extern "C" int bz_attn_decode(const float* q, const void* k_cache, const void* v_cache, int32_t cache_dtype, int32_t B,
                              int32_t HQ, int32_t HKV, int32_t D, int32_t S, const void* mask, int32_t mask_dtype,
                              int64_t ld_mask, const int64_t* pos, float scale, int32_t split, float* part, void* out, int64_t ld_out,
                              void* stream) {
    if (!q || !k_cache || !v_cache || !mask || !pos || !out) return BZ_ERR_INVALID_ARG;
    if (B < 1 || HQ < 1 || HKV < 1 || S < 1 || HQ % HKV) return BZ_ERR_INVALID_ARG;
    if (cache_dtype != BZ_DT_BF16 && cache_dtype != BZ_DT_F32) return BZ_ERR_INVALID_ARG;
    if (split < 1 || split > BZ_ATTN_MAX_SPLIT || (split > 1 && !part)) return BZ_ERR_INVALID_ARG;
    if (mask_dtype != BZ_DT_BF16 && mask_dtype != BZ_DT_F32 && mask_dtype != BZ_MASK_BOOL) return BZ_ERR_INVALID_ARG;
    if ((ld_mask != 0 && ld_mask < S) || ld_mask < 0 || ld_out < (int64_t)HQ * D) return BZ_ERR_SHAPE;
    const int G = HQ / HKV;
    if (D != 64 && D != 128 && D != 256 && D != 512) return BZ_ERR_UNSUPPORTED;
    if (G > 16 || (G > 4 && D == 512)) return BZ_ERR_UNSUPPORTED;
    if (!aligned(q, 16) || !aligned(k_cache, 16) || !aligned(v_cache, 16) || !aligned(out, 2)) return BZ_ERR_ALIGNMENT;
    AttnParams a;
    a.q = q;
    a.kc = k_cache;
    a.vc = v_cache;
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
    a.part = part;
    a.out = static_cast<uint16_t*>(out);
    a.ld_out = ld_out;
    const bool f32c = cache_dtype == BZ_DT_F32;
    const dim3 grid(B, HKV, split);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const bool g4 = G <= 4;
    switch (D) {
        case 64: g4 ? launch_attn<1, 4>(a, f32c, grid, st) : launch_attn<1, 16>(a, f32c, grid, st); break;
        case 128: g4 ? launch_attn<2, 4>(a, f32c, grid, st) : launch_attn<2, 16>(a, f32c, grid, st); break;
        case 256: g4 ? launch_attn<4, 4>(a, f32c, grid, st) : launch_attn<4, 16>(a, f32c, grid, st); break;
        default: launch_attn<8, 4>(a, f32c, grid, st); break;
    }
    const int rc = launched();
    if (rc != BZ_OK || split == 1) return rc;
    hipLaunchKernelGGL(attn_combine_kernel, dim3(B, HQ), dim3(64), 0, st, part, static_cast<uint16_t*>(out), ld_out, HQ,
                       D, split);
    return launched();
}
